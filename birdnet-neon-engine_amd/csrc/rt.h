// libbnneon_hip package runtime: the .bnpk reader, the batched executor and its kernel registry.
//
// The package format and the op-record contract are libbnneon's (src/rt.h, python/bnneon/compiler/pkgfmt.py), so
// a package compiled by bnc for the reference runs here unchanged. What differs is where the buffers live and how
// many windows one run covers: every buffer of a path is allocated in HBM for B windows (window w of buffer i at
// base_i + w * ws_i elements, ws_i = its memory slot's size), and every op's kernels process all B windows in one
// launch on the context's stream.
#ifndef BNH_RT_H
#define BNH_RT_H
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#define RT_FORMAT_VERSION 1
#define RT_READER_VERSION 1
enum { RT_F32 = 0, RT_F16 = 1, RT_I8 = 2, RT_I32 = 3 };
enum { RT_HW_FP16 = 1, RT_HW_DOTPROD = 2 };  // path requirements (the reference's hwcap bits)

#pragma pack(push, 1)
typedef struct {
  char name[48];
  uint32_t dtype, ndim, dims[4];
  uint64_t offset, nbytes, reserved;
} rt_tensor;  // 96 bytes in the file
typedef struct {
  uint32_t dtype, H, W, C, ld, halo, slot, reserved;
  uint64_t elems;
} rt_bufdesc;  // 40 bytes in the file
typedef struct {
  char name[24];
  uint32_t hwcap, n_buf, n_ops, ops_bytes, in_buf, out_buf, emb_buf, reserved;
  uint64_t buf_off, ops_off;
} rt_pathdesc;  // 72 bytes in the file
#pragma pack(pop)

struct rt_pkg;
struct rt_ctx;
#define RT_MAXSUB 4  // sub-batches of a run

typedef struct rt_op {
  uint16_t code, nb, nt, ni;
  const int32_t *b, *t, *p;  // into the mapped file
  void *state;               // device weights and launch plan built by init
  const struct rt_kernel *k;
  // fusion (set after every op's init): an int8 expansion whose only reader is the next op, a fp32 depthwise conv,
  // only quantizes its rows (quant_only), and the depthwise op recomputes the expansion from them (pw)
  struct rt_op *pw;
  int quant_only;
  // and an fp16 SE whose scaled buffer only the next op, an fp16 PW, reads computes the gates only (gate_only), which
  // that PW applies as it loads its rows (se)
  struct rt_op *se;
  int gate_only;
} rt_op;

typedef struct rt_kernel {
  int (*init)(rt_ctx *c, rt_op *op);  // 0, RT_E_PARAM or RT_E_OOM (every failure recorded with rt_bad / rt_oom)
  int (*run)(rt_ctx *c, rt_op *op);   // 0; an op that can fail a window flags it in c->win_fail (device)
  void (*fini)(rt_op *op);
  const char *name;
  uint32_t outmask, optmask;
} rt_kernel;

enum { RT_E_PARAM = -1, RT_E_OOM = -2 };

// op state of the ops whose tensors live on the device: up to 4 uploaded tensors, plus an op-private per-window
// scratch buffer grown with the arena's window capacity
typedef struct {
  void *t[4];
  void *scratch;
  size_t scratch_cap;  // bytes
} rt_dev_state;
int rt_dev_tensors(rt_ctx *c, rt_op *op, int n);
void rt_dev_fini(rt_op *op);
// the op's scratch, at least c->bcap windows of `per_window` bytes each (NULL after rt_oom when it cannot grow)
void *rt_dev_scratch(rt_ctx *c, rt_op *op, size_t per_window);

struct rt_ctx {
  rt_pkg *pkg;
  const rt_pathdesc *path;
  rt_bufdesc *bufd;
  int n_buf;
  rt_op *ops;
  int n_ops;
  // device memory: per buffer, window 0's address and the per-window stride in elements
  int bcap;              // windows the arena holds
  int nwin;              // windows of the current run (<= bcap): ops launch for this many
  int w0;                // the first of them (a sub-batch of the run starts past window 0)
  size_t *wsb;           // per buffer: bytes between windows
  // sub-batches 1 .. RT_MAXSUB - 1: their streams (created on first use; default priority) and the events that start
  // them (fork) and that the context's stream waits for (join); sub-batch 0 runs on `stream`
  hipStream_t sub_stream[RT_MAXSUB];
  hipEvent_t sub_fork[RT_MAXSUB], sub_join[RT_MAXSUB];
  int n_sub;             // sub-batch streams created, including the context's own
  int one_stream;        // never split a batch over two streams
  // Whether batches run as two sub-batches or on the context's stream alone is measured on the context's first
  // batches of one size (64 windows or more): split_choice -1 while undecided, then 0 (two) or 1 (one stream)
  int split_choice;
  int tune_seen;         // batches of tune_B windows finished while undecided
  int tune_B;
  double tune_best[2];   // per mode (0 two sub-batches, 1 one stream): the least wall seconds per window measured
  int tune_n[2];
  int batch_open;        // a batch's first range has been launched and the batch has not finished
  int batch_mode;        // the mode that batch runs in
  double batch_t0;
  int f16_mfma;          // fp16 PW ops on fp16 MFMA (fp32 accumulation) instead of the reference's exact fp16 chains
  size_t *slot_bytes;    // per slot: bytes of one window's copy (64-aligned, >= 64 bytes of zero slack)
  int *slot_users;       // per slot: the number of buffers placed in it
  size_t arena_bytes;
  char *arena;           // device
  void **buf;            // device address of window 0 of each buffer
  long long *ws;         // per buffer: elements between windows
  int *win_fail;         // device [bcap]: op index + 1 of the first op that failed the window, 0 = scored
  hipStream_t stream;
  int own_stream;
  // loader errors
  char *err;
  size_t errlen;
  int err_kind;
  char err_params[160];
  const char *src;       // the package's source-node lines of this path (one per op), or NULL
  size_t src_len;
  size_t *src_line_at;   // byte offset of each line in src
  int n_src_lines;
  int fail_op;
  int prof;
  double *t_op;
  int nprof;
};

// ---- package
rt_pkg *rt_pkg_open(const char *path, char *err, size_t errlen);
void rt_pkg_close(rt_pkg *p);
int rt_meta_str(const rt_pkg *p, const char *key, char *buf, size_t n);
int rt_meta_i64(const rt_pkg *p, const char *key, int64_t *v);
int rt_meta_f64(const rt_pkg *p, const char *key, double *v);
int rt_n_paths(const rt_pkg *p);
int rt_path_served(const rt_pkg *p, int i);  // 1 when every op of path i has a kernel here
int rt_n_tensors(const rt_pkg *p);
int rt_format_version(const rt_pkg *p);
const uint8_t *rt_pkg_bytes(const rt_pkg *p);  // the mapped file
// a metadata record's value (NULL when the key is absent), its type (0 text, 1 i64, 2 f64, 3 bytes) and size
const uint8_t *rt_meta_raw(const rt_pkg *p, const char *key, uint16_t *type, uint32_t *bytes);
const rt_pathdesc *rt_path(const rt_pkg *p, int i);
const rt_tensor *rt_tensor_at(const rt_pkg *p, int i, const void **data);

// ---- context
rt_ctx *rt_ctx_new(rt_pkg *p, int path_index, char *err, size_t errlen, int *kind);
void rt_ctx_free(rt_ctx *c);
// ensure the arena holds `windows` windows (grows it; contents of earlier windows are not kept)
int rt_reserve(rt_ctx *c, int windows, char *err, size_t errlen);
// run every op over windows [0, B) whose input already sits in buffer in_buf; fills status[B] (0 = scored, else
// 1 + the failing op index) and returns the number of failed windows, or -1 on a device error (err set)
int rt_run_batch(rt_ctx *c, int B, int *status, char *err, size_t errlen);
// the same in two halves, for windows [W0, W0 + B) of the arena: the launches on the context's stream (after whatever
// it holds), then the wait and the windows' status (the number of failed windows, or -1)
int rt_launch_range(rt_ctx *c, int W0, int B, char *err, size_t errlen);
int rt_finish_range(rt_ctx *c, int W0, int B, int *status, char *err, size_t errlen);
int rt_op_src(const rt_ctx *c, int i, char *buf, size_t n);
const char *rt_op_name(const rt_ctx *c, int i);
const char *rt_dtype_name(uint32_t dt);
size_t rt_dsize(uint32_t dt);

// ---- fusion
struct bnh_s8w;
// PW_S8 (ops_s8n.cpp): its weights when the op is an expansion a reader may recompute (no gate, no residual, a
// zero-haloed output), else NULL
const struct bnh_s8w *rt_pw8_plain(const rt_op *op);
// fp32 DW3 / DWK (ops_f32.cpp): fuse expansion pw into depthwise op dw when bnh_pwdw_f32 takes the pair; 1 if fused
int rt_fuse_pwdw(rt_ctx *c, rt_op *pw, rt_op *dw);
// fp16 SE + PW (ops_f16.cpp): fuse when the PW reads the SE's buffer as its rows; 1 if fused
int rt_fuse_se16(rt_ctx *c, rt_op *se, rt_op *pw);

// ---- helpers for kernel init / run (the reference's contract helpers, src/rt.h:133-167)
const void *rt_t(const rt_ctx *c, const rt_op *op, int i, size_t *nbytes);
const rt_bufdesc *rt_bd(const rt_ctx *c, const rt_op *op, int i);
int rt_bad(const rt_ctx *c, const rt_op *op, const char *fmt, ...) __attribute__((format(printf, 3, 4)));
int rt_oom(const rt_ctx *c, const rt_op *op, size_t bytes);
int rt_need(const rt_ctx *c, const rt_op *op, int i, int dt, size_t elems);
int rt_need_haloed(const rt_ctx *c, const rt_op *op, int i, int dt, int H, int W, int ld, int h);
int rt_need_rows(const rt_ctx *c, const rt_op *op, int i, int dt, size_t rows, int ld);
int rt_need_nohalo(const rt_ctx *c, const rt_op *op, int i, int dt, size_t elems);
int rt_need_t(const rt_ctx *c, const rt_op *op, int i, size_t nbytes, int atleast);
int rt_need_args(const rt_ctx *c, const rt_op *op, int nb, int nt, int ni);
#define RT_REQ(c, op, cond) \
  do { if (!(cond)) return rt_bad(c, op, "parameter check failed: %s", #cond); } while (0)
// device address of buffer argument i for window w0, the current sub-batch's first (NULL when absent), and its
// per-window stride (elements)
static inline void *rt_b(const rt_ctx *c, const rt_op *op, int i) {
  return i >= op->nb || op->b[i] < 0 ? nullptr : (char *)c->buf[op->b[i]] + (size_t)c->w0 * c->wsb[op->b[i]];
}
static inline long long rt_ws(const rt_ctx *c, const rt_op *op, int i) {
  return i >= op->nb || op->b[i] < 0 ? 0 : c->ws[op->b[i]];
}
void rt_free_state(rt_op *op);
// 1 when buffer argument i has a halo that stays zero between runs: its memory slot holds no other buffer and it is
// not the path's input (the arena is zeroed when allocated and no kernel writes a halo), so its producer need not
// zero the halo again; 0 otherwise
int rt_halo_kept(const rt_ctx *c, const rt_op *op, int i);

// opcodes (the reference's numbering, src/rt.h:170-208; append only)
enum {
  RT_OP_FE_STFT2 = 1, RT_OP_C0POOL = 2, RT_OP_PW = 3, RT_OP_DW3 = 4, RT_OP_SE = 5, RT_OP_POSTPC = 6, RT_OP_DENSE = 7,
  RT_OP_FE_LOGMEL = 8, RT_OP_STEM = 9, RT_OP_DWK = 10, RT_OP_PAD = 11, RT_OP_MEAN = 12, RT_OP_PROTO = 13,
  RT_OP_PROTO_F32H = 14, RT_OP_GEMV = 15, RT_OP_FE_DBIMG = 16, RT_OP_CONVK = 17, RT_OP_GEM = 18, RT_OP_SED = 19,
  RT_OP_VADD = 20, RT_OP_CONVW = 21, RT_OP_PW_S8 = 22, RT_OP_GEMV_S8 = 23, RT_OP_SED_S8 = 24, RT_OP_SE_GATE = 25,
  RT_OP_STEM3 = 26, RT_OP_CONV3C24 = 27, RT_OP_UNPAD = 28, RT_OP_WINO_S8 = 29, RT_OP_QCONV3 = 30, RT_OP_QPW = 31,
  RT_OP_SE_GATE16 = 32, RT_OP_GEM_A = 33, RT_OP_HEADS_S8 = 34, RT_OP_PROTO_S8 = 35, RT_OP_N
};
enum { RT_ACT_NONE = 0, RT_ACT_SILU = 1, RT_ACT_RELU = 2 };

// kernel tables (indexed by base opcode; an entry without run = not in the table), by variant
extern const rt_kernel *rt_k_var0(int base);  // fp32 arithmetic and the int8 no-dotprod GEMMs
extern const rt_kernel *rt_k_var1(int base);  // fp16 arithmetic
extern const rt_kernel *rt_k_var2(int base);  // the dotprod + fp16 family
const rt_kernel *rt_kernel_for(int code);
#endif
