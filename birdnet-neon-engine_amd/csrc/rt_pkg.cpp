// The batched executor: a context's device arena (every buffer of a path for B windows), its op list built from a
// package path (stages below), runtime op fusion, and the run of an op list over a batch in sub-batches on streams.
#include <stdarg.h>
#include <stddef.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include "bnneon_hip.h"
#include "rt.h"

// ------------------------------------------------------------------ device arena
// Per window, every memory slot gets its largest buffer's bytes + 64 zero bytes, rounded to 64 (the reference's
// arena rule, src/rt_pkg.c:379-391); the arena holds `bcap` copies of each slot back to back.
static int arena_alloc(rt_ctx *c, int windows, char *err, size_t errlen) {
  size_t per = 0;
  for (int s = 0; s < c->n_buf; s++) per += c->slot_bytes[s];
  size_t total = per * (size_t)windows;
  char *a = nullptr;
  int *wf = nullptr;
  hipError_t e = hipMalloc(&a, total ? total : 64);
  if (e != hipSuccess) {
    snprintf(err, errlen, "out of device memory: %zu bytes (%.1f MB) for %d windows of activation buffers; hint: use fewer "
             "windows per batch", total, total / 1e6, windows);
    return RT_E_OOM;
  }
  e = hipMalloc(&wf, sizeof(int) * (size_t)windows);
  if (e != hipSuccess) {
    hipFree(a);
    snprintf(err, errlen, "out of device memory for %d window flags", windows);
    return RT_E_OOM;
  }
  if (hipMemsetAsync(a, 0, total ? total : 64, c->stream) != hipSuccess || hipStreamSynchronize(c->stream) != hipSuccess) {
    hipFree(a); hipFree(wf);
    snprintf(err, errlen, "device error while zeroing the activation arena");
    return RT_E_OOM;
  }
  if (c->arena) hipFree(c->arena);
  if (c->win_fail) hipFree(c->win_fail);
  c->arena = a;
  c->win_fail = wf;
  c->arena_bytes = total;
  c->bcap = windows;
  // slot s of window w at arena + slot_off[s] * windows + w * slot_bytes[s]
  size_t off = 0;
  size_t *slot_off = (size_t *)calloc(c->n_buf, sizeof(size_t));
  if (!slot_off) { snprintf(err, errlen, "out of memory"); return RT_E_OOM; }
  for (int s = 0; s < c->n_buf; s++) { slot_off[s] = off; off += c->slot_bytes[s] * (size_t)windows; }
  for (int i = 0; i < c->n_buf; i++) {
    const rt_bufdesc *d = &c->bufd[i];
    c->buf[i] = a + slot_off[d->slot];
    c->ws[i] = (long long)(c->slot_bytes[d->slot] / rt_dsize(d->dtype));
    c->wsb[i] = c->slot_bytes[d->slot];
  }
  free(slot_off);
  return 0;
}

int rt_reserve(rt_ctx *c, int windows, char *err, size_t errlen) {
  if (windows <= c->bcap) return 0;
  return arena_alloc(c, windows, err, errlen);
}

// An int8 expansion (PW_S8) followed by the fp32 depthwise conv that is the only reader of its output runs as one
// kernel (bnh_pwdw_f32): the expansion op then only quantizes its rows. Its output buffer is then never written, so
// no other op and no path output may read it.
static void fuse_ops(rt_ctx *c) {
  for (int i = 0; i + 1 < c->n_ops; i++) {
    rt_op *pw = &c->ops[i], *dw = &c->ops[i + 1];
    if (pw->nb < 2 || pw->b[1] < 0) continue;
    const int32_t buf = pw->b[1];
    bool other = buf == (int32_t)c->path->in_buf || buf == (int32_t)c->path->out_buf || buf == (int32_t)c->path->emb_buf;
    for (int j = 0; j < c->n_ops && !other; j++)
      for (int a = 0; a < c->ops[j].nb && !other; a++)
        if (c->ops[j].b[a] == buf && !(j == i && a == 1) && !(j == i + 1 && a == 0)) other = true;
    // the fused kernel reads the quantized rows (PW_S8 buffers 3..5, dead after the expansion in the package's slot
    // plan) while it writes the depthwise outputs (buffers 1, 2): they must not share a memory slot
    for (int a = 3; a <= 5 && !other; a++)
      for (int o = 1; o <= 2 && !other; o++)
        if (a < pw->nb && o < dw->nb && pw->b[a] >= 0 && dw->b[o] >= 0 &&
            c->bufd[pw->b[a]].slot == c->bufd[dw->b[o]].slot)
          other = true;
    if (!other) rt_fuse_pwdw(c, pw, dw);
  }
  // An fp16 SE (which scales its buffer D in place) followed by an fp16 PW whose rows are D: the SE computes its gates
  // only and the PW applies them as it loads D, so D is never rewritten. No other op may read D.
  for (int i = 0; i + 1 < c->n_ops; i++) {
    rt_op *se = &c->ops[i], *pw = &c->ops[i + 1];
    if (se->nb < 1 || se->b[0] < 0 || pw->quant_only || pw->pw || se->quant_only) continue;
    const int32_t buf = se->b[0];
    bool other = buf == (int32_t)c->path->in_buf || buf == (int32_t)c->path->out_buf || buf == (int32_t)c->path->emb_buf;
    for (int j = 0; j < c->n_ops && !other; j++) {
      if (j == i || j == i + 1) continue;
      const rt_op *o = &c->ops[j];
      for (int a = 0; a < o->nb && !other; a++)  // a reader (the op that writes D is no obstacle)
        if (o->b[a] == buf && !(a < 32 && (o->k->outmask >> a & 1))) other = true;
    }
    if (!other) rt_fuse_se16(c, se, pw);
  }
}

// ------------------------------------------------------------------ context creation
// A context is built in stages: the path's buffer descriptors and their memory slots, the device arena, then every
// op record (decoded, its arguments checked against the path and the package, its kernel chosen by opcode and
// variant, the kernel's argument masks checked, and the kernel's own init run). The stages refuse a package for the
// same reasons, in the same order and with the same words as the reference loader (src/rt_pkg.c:349-509).
namespace {

constexpr const char *kHintRecompile =
    "hint: package/library mismatch or a lowering bug: recompile with bnc; if it reproduces, report this message";
constexpr uint32_t kNoBuffer = 0xffffffffu;
constexpr size_t kMaxWindowBytes = (size_t)1 << 30;  // activation memory one window may need
constexpr uint64_t kMaxBufElems = (uint64_t)1 << 30;

// an op record's fixed 12-byte head: opcode, record bytes, argument counts
struct OpHead {
  uint16_t code, bytes, n_buf, n_ten, n_int, zero;
};
static_assert(sizeof(OpHead) == 12, "op record head");

class ContextBuilder {
 public:
  ContextBuilder(rt_pkg *p, int pi, char *err, size_t errlen) : p_(p), pi_(pi), err_(err), errlen_(errlen) {}
  int kind = RT_E_PARAM;

  rt_ctx *build() {
    if (!(d_ = rt_path(p_, pi_))) {
      snprintf(err_, errlen_, "no path %d in the package (%d paths)", pi_, rt_n_paths(p_));
      return nullptr;
    }
    c_ = (rt_ctx *)calloc(1, sizeof *c_);
    if (!c_) {
      kind = RT_E_OOM;
      snprintf(err_, errlen_, "out of memory (%zu bytes for the context)", sizeof *c_);
      return nullptr;
    }
    c_->pkg = p_;
    c_->path = d_;
    c_->fail_op = -1;
    c_->err = err_;
    c_->errlen = errlen_;
    c_->n_buf = (int)d_->n_buf;
    const bool ok = index_sources() && open_stream() && read_buffers() && plan_slots() && alloc_arena() && read_ops();
    c_->err = nullptr;
    if (!ok) {
      rt_ctx_free(c_);
      return nullptr;
    }
    return c_;
  }

 private:
  bool refuse(int k, const char *fmt, ...) __attribute__((format(printf, 3, 4))) {
    kind = k;
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(err_, errlen_, fmt, ap);
    va_end(ap);
    return false;
  }

  // "src_nodes/<path name>": the ONNX node each op came from, one line per op, for messages
  bool index_sources() {
    char key[64];
    snprintf(key, sizeof key, "src_nodes/%.24s", d_->name);
    uint16_t type = 0;
    uint32_t bytes = 0;
    const uint8_t *v = rt_meta_raw(p_, key, &type, &bytes);
    if (!v || (type != 0 && type != 3)) return true;
    c_->src = (const char *)v;
    c_->src_len = bytes;
    int lines = 0;
    for (size_t at = 0; at < bytes; lines++) {
      const void *nl = memchr(c_->src + at, '\n', bytes - at);
      at = nl ? (size_t)((const char *)nl - c_->src) + 1 : bytes;
    }
    c_->src_line_at = (size_t *)calloc(lines ? lines : 1, sizeof(size_t));
    if (!c_->src_line_at) return refuse(RT_E_OOM, "out of memory (%d source lines)", lines);
    size_t at = 0;
    for (int i = 0; i < lines; i++) {
      c_->src_line_at[i] = at;
      const void *nl = memchr(c_->src + at, '\n', bytes - at);
      at = nl ? (size_t)((const char *)nl - c_->src) + 1 : bytes;
    }
    c_->n_src_lines = lines;
    return true;
  }

  bool open_stream() {
    if (hipStreamCreateWithFlags(&c_->stream, hipStreamNonBlocking) != hipSuccess) {
      c_->stream = nullptr;
      return refuse(RT_E_OOM, "cannot create a HIP stream (no usable GPU?); hint: check that an MI355X is visible "
                              "(rocm-smi)");
    }
    c_->own_stream = 1;
    return true;
  }

  bool read_buffers() {
    const uint32_t n = d_->n_buf;
    c_->bufd = (rt_bufdesc *)malloc(sizeof(rt_bufdesc) * n);
    c_->buf = (void **)calloc(n, sizeof(void *));
    c_->ws = (long long *)calloc(n, sizeof(long long));
    c_->wsb = (size_t *)calloc(n, sizeof(size_t));
    c_->slot_bytes = (size_t *)calloc(n, sizeof(size_t));
    c_->slot_users = (int *)calloc(n, sizeof(int));
    if (!c_->bufd || !c_->buf || !c_->ws || !c_->wsb || !c_->slot_bytes || !c_->slot_users)
      return refuse(RT_E_OOM, "out of memory (%u buffer descriptors)", n);
    memcpy(c_->bufd, rt_pkg_bytes(p_) + d_->buf_off, sizeof(rt_bufdesc) * n);
    return true;
  }

  // every buffer's descriptor sane, the input alone in its slot; each slot sized for its largest buffer plus the
  // 64 zero bytes the reference's arena keeps after every buffer (src/rt_pkg.c:379-391), rounded to 64
  bool plan_slots() {
    const uint32_t n = d_->n_buf;
    const uint32_t in_slot = c_->bufd[d_->in_buf].slot;
    for (uint32_t i = 0; i < n; i++) {
      const rt_bufdesc &b = c_->bufd[i];
      if (b.dtype > RT_I32 || b.elems > kMaxBufElems || b.slot >= n)
        return refuse(RT_E_PARAM, "path %.24s buffer #%u: bad descriptor (dtype %u, %llu elements, slot %u of %u); %s",
                      d_->name, i, b.dtype, (unsigned long long)b.elems, b.slot, n, kHintRecompile);
      if ((i == d_->in_buf) != (b.slot == in_slot))
        return refuse(RT_E_PARAM, "path %.24s buffer #%u shares the input window's memory slot %u; %s", d_->name, i,
                      b.slot, kHintRecompile);
      const size_t need = ((size_t)b.elems * rt_dsize(b.dtype) + 64 + 63) / 64 * 64;
      c_->slot_bytes[b.slot] = need > c_->slot_bytes[b.slot] ? need : c_->slot_bytes[b.slot];
      c_->slot_users[b.slot]++;
    }
    size_t window = 0;
    for (uint32_t s = 0; s < n; s++)
      if ((window += c_->slot_bytes[s]) > kMaxWindowBytes)
        return refuse(RT_E_PARAM, "path %.24s needs more than 1 GB of activation buffers per window; hint: the package "
                      "is corrupt or the model is far larger than this runtime is built for", d_->name);
    const uint32_t out_slot = c_->bufd[d_->out_buf].slot;
    const bool has_emb = d_->emb_buf != kNoBuffer;
    const uint32_t emb_slot = has_emb ? c_->bufd[d_->emb_buf].slot : kNoBuffer;
    for (uint32_t i = 0; i < n; i++) {
      if (i == d_->out_buf) continue;
      const uint32_t s = c_->bufd[i].slot;
      if (s == out_slot || (has_emb && i != d_->emb_buf && s == emb_slot))
        return refuse(RT_E_PARAM, "path %.24s buffer #%u shares memory slot %u with the output buffer (#%u / #%u); %s",
                      d_->name, i, s, d_->out_buf, d_->emb_buf, kHintRecompile);
    }
    return true;
  }

  bool alloc_arena() {
    const int k = arena_alloc(c_, 1, err_, errlen_);
    if (k) kind = k;
    return !k;
  }

  // "op i kernel (ONNX node ...)" for messages about op i
  const char *who(int i, const char *kname) {
    char src[160];
    if (rt_op_src(c_, i, src, sizeof src) == 0 && src[0]) {
      if (strlen(src) > 96) memcpy(src + 93, "...'", 5);
      snprintf(who_, sizeof who_, "op %d %s (ONNX node %s)", i, kname ? kname : "?", src);
    } else {
      snprintf(who_, sizeof who_, "op %d %s (no source node names in the package: compile with bnc 2 or newer)", i,
               kname ? kname : "?");
    }
    return who_;
  }

  bool read_ops() {
    c_->ops = (rt_op *)calloc(d_->n_ops, sizeof(rt_op));
    if (!c_->ops) return refuse(RT_E_OOM, "out of memory (%u op records)", d_->n_ops);
    const uint8_t *file = rt_pkg_bytes(p_);
    const uint8_t *at = file + d_->ops_off, *end = at + d_->ops_bytes;
    for (uint32_t i = 0; i < d_->n_ops; i++) {
      if (end - at < (ptrdiff_t)sizeof(OpHead))
        return refuse(RT_E_PARAM, "op %u: truncated op list (%u ops declared, %u bytes); %s", i, d_->n_ops,
                      d_->ops_bytes, kHintRecompile);
      OpHead h;
      memcpy(&h, at, sizeof h);
      const size_t args = 4 * ((size_t)h.n_buf + h.n_ten + h.n_int);
      if (h.bytes < sizeof h + args || end - at < (ptrdiff_t)h.bytes || (size_t)(at - file) % 4)
        return refuse(RT_E_PARAM, "op %u: bad op record (%u bytes for %u buffer, %u tensor, %u int arguments); %s", i,
                      h.bytes, h.n_buf, h.n_ten, h.n_int, kHintRecompile);
      rt_op &op = c_->ops[i];
      op.code = h.code;
      op.nb = h.n_buf;
      op.nt = h.n_ten;
      op.ni = h.n_int;
      op.b = (const int32_t *)(at + sizeof h);
      op.t = op.b + op.nb;
      op.p = op.t + op.nt;
      if (!check_references(i, op) || !bind_kernel(i, op) || !check_masks(i, op)) return false;
      c_->n_ops = (int)i + 1;
      if (!run_init(i, op)) return false;
      at += h.bytes;
    }
    return true;
  }

  // buffer and tensor indices name buffers of the path and tensors of the package; the variant matches the path
  bool check_references(uint32_t i, const rt_op &op) {
    for (int a = 0; a < op.nb; a++)
      if (op.b[a] < -1 || op.b[a] >= (int32_t)d_->n_buf)
        return refuse(RT_E_PARAM, "%s: buffer argument %d names buffer #%d but the path has %u buffers; %s",
                      who((int)i, nullptr), a, op.b[a], d_->n_buf, kHintRecompile);
    const int n_ten = rt_n_tensors(p_);
    for (int a = 0; a < op.nt; a++)
      if (op.t[a] >= n_ten)
        return refuse(RT_E_PARAM, "%s: tensor argument %d names tensor #%d but the package has %d tensors; %s",
                      who((int)i, nullptr), a, op.t[a], n_ten, kHintRecompile);
    const int variant = op.code >> 8;
    if (variant && !(d_->hwcap & RT_HW_FP16))
      return refuse(RT_E_PARAM, "%s: fp16 kernel (opcode 0x%x) in path %.24s, which does not declare the fp16 "
                    "requirement; %s", who((int)i, nullptr), op.code, d_->name, kHintRecompile);
    if (variant == 2 && !(d_->hwcap & RT_HW_DOTPROD))
      return refuse(RT_E_PARAM, "%s: dotprod kernel (opcode 0x%x) in path %.24s, which does not declare the dotprod "
                    "requirement; %s", who((int)i, nullptr), op.code, d_->name, kHintRecompile);
    return true;
  }

  bool bind_kernel(uint32_t i, rt_op &op) {
    if ((op.k = rt_kernel_for(op.code))) return true;
    char compiler[48];
    if (rt_meta_str(p_, "compiler", compiler, sizeof compiler) < 0) snprintf(compiler, sizeof compiler, "unknown");
    return refuse(RT_E_PARAM, "%s: unknown opcode 0x%x (base %d variant %d); this library runs opcodes 1..%d of "
                  "variants 0, 1 and 2 on the GPU, not every opcode of each (reader version %d), the package was written by compiler '%s'; hint: "
                  "pick a path of the package this library runs (mode 0), or update libbnneon_hip", who((int)i, nullptr),
                  op.code, op.code & 0xff, op.code >> 8, RT_OP_N - 1, RT_READER_VERSION, compiler);
  }

  // required buffers present, the input never written, a written buffer sharing memory with no other argument
  bool check_masks(uint32_t i, const rt_op &op) {
    const rt_kernel &k = *op.k;
    auto writes = [&](int a) { return a < 32 && (k.outmask >> a & 1); };
    auto optional = [&](int a) { return a < 32 && (k.optmask >> a & 1); };
    for (int a = 0; a < op.nb; a++) {
      if (op.b[a] < 0 && !optional(a))
        return refuse(RT_E_PARAM, "%s: buffer argument %d is required by the kernel but absent (-1) in the op record; %s",
                      who((int)i, k.name), a, kHintRecompile);
      if (op.b[a] == (int32_t)d_->in_buf && writes(a))
        return refuse(RT_E_PARAM, "%s: buffer argument %d is the input window (#%u) but the kernel writes it; %s",
                      who((int)i, k.name), a, d_->in_buf, kHintRecompile);
    }
    for (int a = 0; a < op.nb; a++) {
      if (!writes(a) || op.b[a] < 0) continue;
      for (int o = 0; o < op.nb; o++) {
        if (o == a || op.b[o] < 0) continue;
        const uint32_t sa = c_->bufd[op.b[a]].slot, so = c_->bufd[op.b[o]].slot;
        if (op.b[a] == op.b[o] || sa == so)
          return refuse(RT_E_PARAM, "%s: buffer arguments %d (#%d, written) and %d (#%d) share memory slot %u; %s",
                        who((int)i, k.name), a, op.b[a], o, op.b[o], sa, kHintRecompile);
      }
    }
    return true;
  }

  bool run_init(uint32_t i, rt_op &op) {
    if (!op.k->init) return true;
    c_->err_kind = 0;
    c_->err_params[0] = 0;
    if (!op.k->init(c_, &op)) return true;
    char detail[400];
    snprintf(detail, sizeof detail, "%s", c_->err_kind ? err_ : "init failed without a message (kernel bug)");
    const char *w = who((int)i, op.k->name);
    if (c_->err_kind == RT_E_OOM) {
      kind = RT_E_OOM;
      snprintf(err_, errlen_, "%s: %s; hint: free device memory or use a smaller model", w, detail);
      return false;
    }
    kind = RT_E_PARAM;
    const int n = snprintf(err_, errlen_, "%s: %s; %s", w, detail, kHintRecompile);
    if (n > 0 && (size_t)n + 24 < errlen_ && c_->err_params[0])
      snprintf(err_ + n, errlen_ - (size_t)n, " (int params: [%s])", c_->err_params);
    return false;
  }

  rt_pkg *p_;
  int pi_;
  char *err_;
  size_t errlen_;
  const rt_pathdesc *d_ = nullptr;
  rt_ctx *c_ = nullptr;
  char who_[256];
};

}  // namespace

// 1 when this library has a kernel for every op record of path `pi` (a list it cannot walk counts as served, so
// that bnn_init names the defect), else 0
int rt_path_served(const rt_pkg *p, int pi) {
  const rt_pathdesc *d = rt_path(p, pi);
  if (!d) return 0;
  const uint8_t *at = rt_pkg_bytes(p) + d->ops_off, *end = at + d->ops_bytes;
  for (uint32_t i = 0; i < d->n_ops; i++) {
    OpHead h;
    if (end - at < (ptrdiff_t)sizeof h) return 1;
    memcpy(&h, at, sizeof h);
    if (h.bytes < sizeof h || end - at < (ptrdiff_t)h.bytes) return 1;
    if (!rt_kernel_for(h.code)) return 0;
    at += h.bytes;
  }
  return 1;
}

rt_ctx *rt_ctx_new(rt_pkg *p, int pi, char *err, size_t errlen, int *kind) {
  ContextBuilder b(p, pi, err, errlen);
  rt_ctx *c = b.build();
  if (!c) {
    if (kind) *kind = b.kind;
    return nullptr;
  }
  const char *fe = getenv("BNH_FUSE");  // BNH_FUSE=0 runs every op as the package lists it
  if (!fe || atoi(fe) != 0) fuse_ops(c);
  // BNH_SPLIT=0 runs every batch on one stream, BNH_SPLIT=1 splits every batch of 64 windows or more; unset, the
  // context measures both on its first batches and keeps the faster
  const char *se = getenv("BNH_SPLIT");
  c->one_stream = se && atoi(se) == 0;
  c->split_choice = se ? (atoi(se) == 0 ? 1 : 0) : -1;
  const char *fm = getenv("BNH_F16_MFMA");  // BNH_F16_MFMA=1: fp16 PW ops accumulate in fp32 on the matrix cores
  c->f16_mfma = fm && atoi(fm) == 1;
  const char *pe = getenv("BNN_PROF");
  c->prof = pe ? atoi(pe) : 0;
  if (c->prof) c->t_op = (double *)calloc(c->n_ops, sizeof(double));
  if (kind) *kind = 0;
  return c;
}

static double now_s(void) {
  struct timespec t;
  clock_gettime(CLOCK_MONOTONIC, &t);
  return t.tv_sec + t.tv_nsec * 1e-9;
}

// Two sub-batches on two streams run 8 % faster than one stream on the Perch-shaped net when the HIP runtime maps
// the two streams to different hardware queues; when it maps them to the same queue (it multiplexes a process's
// streams over a few queues, and which ones share depends on what the process created and destroyed before),
// measured on the MI355X: 1.4x slower than one stream. The library cannot see the mapping, so each context times
// its first batches of one size (64 windows or more): one untimed, two split, two on one stream, and keeps one
// stream only when it was at least 10 % faster.
static int tune_mode(const rt_ctx *c) {
  return c->tune_seen >= 3 ? 1 : 0;  // batches 0 (untimed), 1, 2 split; 3, 4 one stream
}

static void tune_note(rt_ctx *c, int B, double secs) {
  if (B < 64) return;
  if (c->tune_seen == 0) c->tune_B = B;
  if (B != c->tune_B) return;
  const int mode = c->batch_mode;
  if (c->tune_seen > 0) {
    const double per = secs / B;
    if (!c->tune_n[mode] || per < c->tune_best[mode]) c->tune_best[mode] = per;
    c->tune_n[mode]++;
  }
  c->tune_seen++;
  if (c->tune_n[0] >= 2 && c->tune_n[1] >= 2) c->split_choice = c->tune_best[1] < 0.9 * c->tune_best[0] ? 1 : 0;
}

// the streams and fork / join events of sub-batches 1 .. n - 1, created once (fewer when the runtime refuses them)
static int ensure_subs(rt_ctx *c, int n) {
  if (c->n_sub == 0) c->n_sub = 1;
  while (c->n_sub < n) {
    const int h = c->n_sub;
    hipStream_t s = nullptr;
    hipEvent_t a = nullptr, b = nullptr;
    if (hipStreamCreateWithFlags(&s, hipStreamNonBlocking) != hipSuccess) break;
    if (hipEventCreateWithFlags(&a, hipEventDisableTiming) != hipSuccess ||
        hipEventCreateWithFlags(&b, hipEventDisableTiming) != hipSuccess) {
      if (a) hipEventDestroy(a);
      hipStreamDestroy(s);
      break;
    }
    c->sub_stream[h] = s;
    c->sub_fork[h] = a;
    c->sub_join[h] = b;
    c->n_sub = h + 1;
  }
  return c->n_sub < n ? c->n_sub : n;
}

int rt_run_batch(rt_ctx *c, int B, int *status, char *err, size_t errlen) {
  if (rt_launch_range(c, 0, B, err, errlen)) return -1;
  return rt_finish_range(c, 0, B, status, err, errlen);
}

int rt_launch_range(rt_ctx *c, int W0, int B, char *err, size_t errlen) {
  if (W0 < 0 || B < 1 || W0 + B > c->bcap) {
    snprintf(err, errlen, "rt_run_batch: windows %d..%d but the arena holds %d", W0, W0 + B - 1, c->bcap);
    return c->batch_open = 0, -1;
  }
  if (hipMemsetAsync(c->win_fail + W0, 0, sizeof(int) * (size_t)B, c->stream) != hipSuccess) {
    snprintf(err, errlen, "device error clearing the window flags");
    return c->batch_open = 0, -1;
  }
  // Sub-batches on their own streams, their launches interleaved op by op: the windows are independent, so the GPU
  // may run one sub-batch's kernel beside another's (a VALU-bound kernel beside a memory-bound one). Sub-batch h
  // runs one op behind sub-batch h - 1 (it starts after that one's first op, and so after everything the context's
  // stream held), so that kernels of different kinds meet more often than copies of the same kernel; the context's
  // stream waits for every sub-batch at the end.
  // two sub-batches (measured: three or four, on as many streams, are 15-25 % slower on both nets; one op of skew is
  // 1.5-1.7 % faster than none, four or more slower)
  if (!c->batch_open) {
    c->batch_open = 1;
    c->batch_t0 = now_s();
    c->batch_mode = c->split_choice >= 0 ? c->split_choice : tune_mode(c);
  }
  int ns = 2;
  if (c->prof || c->one_stream || B < 64 || c->batch_mode == 1) ns = 1;
  if (ns > RT_MAXSUB) ns = RT_MAXSUB;
  while (ns > 1 && B / ns < 32) ns--;  // sub-batches of at least 32 windows
  if (ns > 1) ns = ensure_subs(c, ns);
  hipStream_t s1 = c->stream;
  const int skew = 1;
  auto first = [&](int h) { return (int)((long long)B * h / ns); };
  auto strm = [&](int h) { return h ? c->sub_stream[h] : s1; };
  auto drain = [&]() {
    for (int h = 1; h < ns; h++) hipStreamSynchronize(c->sub_stream[h]);
  };
  double t0 = c->prof ? now_s() : 0;
  // step t runs sub-batch h's op t - h skew
  for (int t = 0; t < c->n_ops + (ns - 1) * skew; t++) {
    for (int h = 0; h < ns; h++) {
      const int i = t - h * skew;
      if (i < 0 || i >= c->n_ops) continue;
      rt_op *op = &c->ops[i];
      if (h && i == 0 && hipStreamWaitEvent(c->sub_stream[h], c->sub_fork[h], 0) != hipSuccess) {
        drain();
        snprintf(err, errlen, "device error starting sub-batch %d", h);
        return c->batch_open = 0, -1;
      }
      c->fail_op = i;  // ops read it to tag the windows they fail
      c->w0 = W0 + first(h);
      c->nwin = first(h + 1) - first(h);
      c->stream = strm(h);
      int r = op->k->run(c, op);
      c->w0 = 0;
      c->nwin = B;
      c->stream = s1;
      if (!r && h + 1 < ns && i == skew - 1 && hipEventRecord(c->sub_fork[h + 1], strm(h)) != hipSuccess) r = -1;
      if (r) {
        drain();  // leave no launch of this batch in flight
        char src[160];
        rt_op_src(c, i, src, sizeof src);
        const char *why = bnh_last_error();
        snprintf(err, errlen, "op %d %s%s%s%s: launch failed (%s)", i, op->k->name, src[0] ? " (ONNX node " : "", src,
                 src[0] ? ")" : "", why && why[0] ? why : hipGetErrorString(hipGetLastError()));
        return c->batch_open = 0, -1;
      }
      if (c->prof) {
        hipStreamSynchronize(c->stream);
        double tn = now_s();
        c->t_op[i] += tn - t0;
        t0 = tn;
      }
    }
  }
  for (int h = 1; h < ns; h++)
    if (hipEventRecord(c->sub_join[h], c->sub_stream[h]) != hipSuccess ||
        hipStreamWaitEvent(s1, c->sub_join[h], 0) != hipSuccess) {
      drain();
      snprintf(err, errlen, "device error joining sub-batch %d", h);
      return c->batch_open = 0, -1;
    }
  c->fail_op = -1;
  return 0;
}

int rt_finish_range(rt_ctx *c, int W0, int B, int *status, char *err, size_t errlen) {
  hipError_t e = hipMemcpyAsync(status, c->win_fail + W0, sizeof(int) * (size_t)B, hipMemcpyDeviceToHost, c->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
  const bool opened = c->batch_open;
  c->batch_open = 0;
  if (e != hipSuccess) { snprintf(err, errlen, "device error after the op list: %s", hipGetErrorString(e)); return -1; }
  if (opened && c->split_choice < 0) tune_note(c, B, now_s() - c->batch_t0);
  c->nprof += B;
  int nf = 0;
  for (int w = 0; w < B; w++) nf += status[w] != 0;
  return nf;
}

int rt_halo_kept(const rt_ctx *c, const rt_op *op, int i) {
  if (i >= op->nb || op->b[i] < 0 || (uint32_t)op->b[i] == c->path->in_buf) return 0;
  const rt_bufdesc *d = &c->bufd[op->b[i]];
  return d->halo > 0 && d->slot < (uint32_t)c->n_buf && c->slot_users[d->slot] == 1;
}

void rt_ctx_free(rt_ctx *c) {
  if (!c) return;
  if (c->stream) hipStreamSynchronize(c->stream);
  if (c->prof && c->nprof && c->t_op) {
    double tot = 0;
    fprintf(stderr, "profile over %d windows (ms per window, batched), path %s:\n", c->nprof, c->path->name);
    for (int i = 0; i < c->n_ops; i++) {
      tot += c->t_op[i];
      char src[120];
      rt_op_src(c, i, src, sizeof src);
      const rt_op *op = &c->ops[i];
      char fz[48] = "";
      if (op->pw) snprintf(fz, sizeof fz, " [fused: computes op %d's expansion]", (int)(op->pw - c->ops));
      else if (op->quant_only) snprintf(fz, sizeof fz, " [quantizes only]");
      else if (op->se) snprintf(fz, sizeof fz, " [fused: applies op %d's gates]", (int)(op->se - c->ops));
      else if (op->gate_only) snprintf(fz, sizeof fz, " [gates only]");
      if (c->prof > 1)
        fprintf(stderr, "  %3d %-14s %10.5f  %s%s\n", i, op->k->name, 1e3 * c->t_op[i] / c->nprof, src, fz);
    }
    fprintf(stderr, "  %-14s      %10.5f\n", "total", 1e3 * tot / c->nprof);
  }
  for (int i = 0; i < c->n_ops; i++) {
    rt_op *op = &c->ops[i];
    if (op->k && op->k->fini) op->k->fini(op);
  }
  free(c->ops);
  free(c->t_op);
  if (c->arena) hipFree(c->arena);
  if (c->win_fail) hipFree(c->win_fail);
  free(c->buf);
  free(c->ws);
  free(c->wsb);
  free(c->slot_bytes);
  free(c->slot_users);
  free(c->bufd);
  free(c->src_line_at);
  if (c->stream && c->own_stream) hipStreamDestroy(c->stream);
  for (int h = 1; h < c->n_sub; h++) {
    hipStreamSynchronize(c->sub_stream[h]);
    hipStreamDestroy(c->sub_stream[h]);
    hipEventDestroy(c->sub_fork[h]);
    hipEventDestroy(c->sub_join[h]);
  }
  free(c);
}
