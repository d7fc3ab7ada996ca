// .bnpk reader (mmap, bounds-checked tables, metadata) and the batched executor (device arena, op list).
// Package checks and error texts follow the reference loader's contract (src/rt_pkg.c:30-102, 349-509): a package
// the reference refuses is refused here with the same kind of message, and a package it accepts runs here.
#include <errno.h>
#include <fcntl.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <time.h>
#include <unistd.h>

#include "bnneon_hip.h"
#include "rt.h"

struct rt_pkg {
  void *map;
  size_t size;
  uint32_t n_meta, n_tensors, n_paths;
  int version;
  const uint8_t *meta;
  size_t meta_bytes;
  rt_tensor *tensors;
  rt_pathdesc *paths;
};

#define FAIL(...) do { snprintf(err, errlen, __VA_ARGS__); goto fail; } while (0)

rt_pkg *rt_pkg_open(const char *path, char *err, size_t errlen) {
  rt_pkg *p = (rt_pkg *)calloc(1, sizeof *p);
  const uint8_t *m;
  uint32_t bom, cnt[4];
  uint16_t ver[2];
  uint64_t off[4];
  if (!p) { snprintf(err, errlen, "out of memory"); return nullptr; }
  int fd = open(path, O_RDONLY);
  if (fd < 0) { snprintf(err, errlen, "cannot open %s (%s)", path, strerror(errno)); free(p); return nullptr; }
  struct stat sb;
  int no_stat = fstat(fd, &sb) != 0;
  if (no_stat || sb.st_size < 64) {
    close(fd);
    snprintf(err, errlen, "%s: %lld bytes, smaller than a package header (64); hint: incomplete download or the wrong file",
             path, no_stat ? -1LL : (long long)sb.st_size);
    free(p);
    return nullptr;
  }
  p->size = (size_t)sb.st_size;
  p->map = mmap(nullptr, p->size, PROT_READ, MAP_PRIVATE, fd, 0);
  close(fd);
  if (p->map == MAP_FAILED) {
    p->map = nullptr;
    snprintf(err, errlen, "%s: mmap of %zu bytes failed (%s); hint: memory or a filesystem that cannot map files", path,
             p->size, strerror(errno));
    free(p);
    return nullptr;
  }
  m = (const uint8_t *)p->map;
  if (memcmp(m, "BNNPKG01", 8))
    FAIL("%s: not a .bnpk package (magic '%.8s', expected BNNPKG01); hint: the file is not a compiled model package: "
         "compile the model with bnc, or check the download (sha256)", path, (const char *)m);
  memcpy(&bom, m + 8, 4);
  memcpy(ver, m + 12, 4);
  if (bom != 0x01020304u) FAIL("%s: byte-order mark 0x%08x, expected 0x01020304 (little endian); hint: corrupt file", path, bom);
  p->version = ver[0];
  if (ver[1] > RT_READER_VERSION)
    FAIL("%s: the package needs reader version %u, this library reads format version %u; hint: update libbnneon_hip, or "
         "recompile the model with the compiler that matches this library", path, ver[1], RT_READER_VERSION);
  memcpy(cnt, m + 16, 16);
  memcpy(off, m + 32, 32);
  p->n_meta = cnt[0]; p->n_tensors = cnt[1]; p->n_paths = cnt[2];
  if (off[3] != p->size)
    FAIL("%s: package truncated (size %zu, header says %llu); hint: incomplete download or copy; compare the sha256", path,
         p->size, (unsigned long long)off[3]);
  if (p->n_tensors > 65536 || p->n_paths < 1 || p->n_paths > 8 || p->n_meta > 4096)
    FAIL("%s: corrupt header (%u metadata records, %u tensors, %u paths; limits 4096 / 65536 / 1..8); hint: corrupt file or "
         "not a package", path, p->n_meta, p->n_tensors, p->n_paths);
  if (off[0] > p->size || off[1] > p->size || off[2] > p->size || off[1] < off[0] ||
      off[1] + (uint64_t)p->n_tensors * sizeof(rt_tensor) > p->size ||
      off[2] + (uint64_t)p->n_paths * sizeof(rt_pathdesc) > p->size)
    FAIL("%s: table offsets outside the file (meta %llu, tensors %llu, paths %llu, size %zu); hint: corrupt file", path,
         (unsigned long long)off[0], (unsigned long long)off[1], (unsigned long long)off[2], p->size);
  p->meta = m + off[0];
  p->meta_bytes = off[1] - off[0];
  p->tensors = (rt_tensor *)malloc(sizeof(rt_tensor) * (p->n_tensors ? p->n_tensors : 1));
  p->paths = (rt_pathdesc *)malloc(sizeof(rt_pathdesc) * p->n_paths);
  if (!p->tensors || !p->paths) FAIL("out of memory");
  memcpy(p->tensors, m + off[1], sizeof(rt_tensor) * p->n_tensors);
  memcpy(p->paths, m + off[2], sizeof(rt_pathdesc) * p->n_paths);
  for (uint32_t i = 0; i < p->n_tensors; i++) {
    const rt_tensor *t = &p->tensors[i];
    if (t->offset % 64 || t->offset > p->size || t->nbytes > p->size - t->offset || t->offset + t->nbytes + 64 > p->size)
      FAIL("%s: tensor %u (%.48s) lies outside the file (offset %llu, %llu bytes, file %zu); hint: truncated or corrupt file",
           path, i, t->name, (unsigned long long)t->offset, (unsigned long long)t->nbytes, p->size);
  }
  for (uint32_t i = 0; i < p->n_paths; i++) {
    const rt_pathdesc *d = &p->paths[i];
    if (d->n_buf == 0 || d->n_buf > 4096 || d->n_ops == 0 || d->n_ops > 4096 || d->buf_off % 8 || d->ops_off % 8 ||
        d->buf_off + (uint64_t)d->n_buf * sizeof(rt_bufdesc) > p->size || d->ops_off + d->ops_bytes > p->size ||
        d->in_buf >= d->n_buf || d->out_buf >= d->n_buf || (d->emb_buf != 0xffffffffu && d->emb_buf >= d->n_buf))
      FAIL("%s: path %u (%.24s) has corrupt tables (%u buffers, %u ops, in %u out %u emb %u); hint: corrupt file", path, i,
           d->name, d->n_buf, d->n_ops, d->in_buf, d->out_buf, d->emb_buf);
  }
  return p;
fail:
  rt_pkg_close(p);
  return nullptr;
}

void rt_pkg_close(rt_pkg *p) {
  if (!p) return;
  if (p->map) munmap(p->map, p->size);
  free(p->tensors);
  free(p->paths);
  free(p);
}

// metadata records: u16 key_len, u16 type (0 str, 1 i64, 2 f64, 3 bytes), u32 val_len, key, value, padded to 8
static const uint8_t *meta_find(const rt_pkg *p, const char *key, uint16_t *type, uint32_t *vlen) {
  const uint8_t *q = p->meta, *end = p->meta + p->meta_bytes;
  size_t kl = strlen(key);
  for (uint32_t i = 0; i < p->n_meta && q + 8 <= end; i++) {
    uint16_t h[2];
    uint32_t vl;
    memcpy(h, q, 4);
    memcpy(&vl, q + 4, 4);
    size_t rec = (8 + (size_t)h[0] + vl + 7) & ~(size_t)7;
    if ((size_t)(end - q) < rec) return nullptr;
    if (h[0] == kl && !memcmp(q + 8, key, kl)) { *type = h[1]; *vlen = vl; return q + 8 + h[0]; }
    q += rec;
  }
  return nullptr;
}

int rt_meta_str(const rt_pkg *p, const char *key, char *buf, size_t n) {
  uint16_t ty;
  uint32_t vl;
  const uint8_t *v = meta_find(p, key, &ty, &vl);
  if (!v) return -1;
  char tmp[64];
  if (ty == 1 || ty == 2) {  // numbers as decimal text
    if (ty == 1) { int64_t x; memcpy(&x, v, 8); snprintf(tmp, sizeof tmp, "%lld", (long long)x); }
    else { double x; memcpy(&x, v, 8); snprintf(tmp, sizeof tmp, "%.17g", x); }
    v = (const uint8_t *)tmp;
    vl = (uint32_t)strlen(tmp);
  }
  if (buf && n) {
    size_t k = vl < n - 1 ? vl : n - 1;
    memcpy(buf, v, k);
    buf[k] = 0;
  }
  return (int)vl;
}
static int meta_num(const rt_pkg *p, const char *key, uint16_t type, void *x) {
  uint16_t ty;
  uint32_t vl;
  const uint8_t *v = meta_find(p, key, &ty, &vl);
  if (!v || ty != type || vl != 8) return -1;
  memcpy(x, v, 8);
  return 0;
}
int rt_meta_i64(const rt_pkg *p, const char *key, int64_t *x) { return meta_num(p, key, 1, x); }
int rt_meta_f64(const rt_pkg *p, const char *key, double *x) { return meta_num(p, key, 2, x); }
int rt_n_paths(const rt_pkg *p) { return (int)p->n_paths; }
int rt_format_version(const rt_pkg *p) { return p->version; }
const rt_pathdesc *rt_path(const rt_pkg *p, int i) { return i >= 0 && i < (int)p->n_paths ? &p->paths[i] : nullptr; }
const rt_tensor *rt_tensor_at(const rt_pkg *p, int i, const void **data) {
  if (i < 0 || i >= (int)p->n_tensors) return nullptr;
  if (data) *data = (const uint8_t *)p->map + p->tensors[i].offset;
  return &p->tensors[i];
}

// ------------------------------------------------------------------ contract helpers
size_t rt_dsize(uint32_t dt) { return dt == RT_F16 ? 2 : dt == RT_I8 ? 1 : 4; }
const char *rt_dtype_name(uint32_t dt) {
  static const char *nm[] = {"f32", "f16", "i8", "i32"};
  return dt < 4 ? nm[dt] : "?";
}
const void *rt_t(const rt_ctx *c, const rt_op *op, int i, size_t *nbytes) {
  if (i >= op->nt || op->t[i] < 0) return nullptr;
  const void *d;
  const rt_tensor *t = rt_tensor_at(c->pkg, op->t[i], &d);
  if (!t) return nullptr;
  if (nbytes) *nbytes = t->nbytes;
  return d;
}
const rt_bufdesc *rt_bd(const rt_ctx *c, const rt_op *op, int i) {
  return i >= op->nb || op->b[i] < 0 ? nullptr : &c->bufd[op->b[i]];
}
void rt_free_state(rt_op *op) { free(op->state); }

static void err_set(const rt_ctx *c, int kind, const char *msg) {
  rt_ctx *w = (rt_ctx *)c;
  if (!w->err || w->err_kind) return;
  w->err_kind = kind;
  snprintf(w->err, w->errlen, "%s", msg);
}
static void int_params(const rt_op *op, char *buf, size_t n) {
  size_t k = 0;
  buf[0] = 0;
  for (int i = 0; i < op->ni && k + 16 < n; i++) k += (size_t)snprintf(buf + k, n - k, "%s%d", i ? " " : "", op->p[i]);
  if (op->ni && k + 16 >= n) snprintf(buf + k, n - k, " ...");
}
int rt_bad(const rt_ctx *c, const rt_op *op, const char *fmt, ...) {
  char msg[320];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(msg, sizeof msg, fmt, ap);
  va_end(ap);
  if (c->err && !c->err_kind) int_params(op, ((rt_ctx *)c)->err_params, sizeof c->err_params);
  err_set(c, RT_E_PARAM, msg);
  return RT_E_PARAM;
}
int rt_oom(const rt_ctx *c, const rt_op *op, size_t bytes) {
  (void)op;
  char msg[128];
  snprintf(msg, sizeof msg, "out of memory allocating %zu bytes of kernel state", bytes);
  err_set(c, RT_E_OOM, msg);
  return RT_E_OOM;
}
int rt_need(const rt_ctx *c, const rt_op *op, int i, int dt, size_t elems) {
  const rt_bufdesc *d = rt_bd(c, op, i);
  if (!d) return rt_bad(c, op, "buffer argument %d is absent (the op record has %d buffer arguments)", i, op->nb);
  if ((int)d->dtype == dt && d->elems >= elems) return 0;
  return rt_bad(c, op, "buffer argument %d (buffer #%d): expected dtype %s with >= %zu elements, found dtype %s "
                "[%ux%ux%u ld %u halo %u] with %llu elements", i, op->b[i], rt_dtype_name((uint32_t)dt), elems,
                rt_dtype_name(d->dtype), d->H, d->W, d->C, d->ld, d->halo, (unsigned long long)d->elems);
}
int rt_need_haloed(const rt_ctx *c, const rt_op *op, int i, int dt, int H, int W, int ld, int h) {
  if (rt_need(c, op, i, dt, ((size_t)H + 2 * (size_t)h) * ((size_t)W + 2 * (size_t)h) * (size_t)ld)) return RT_E_PARAM;
  const rt_bufdesc *d = rt_bd(c, op, i);
  if ((int)d->halo != h || (int)d->ld != ld)
    return rt_bad(c, op, "buffer argument %d (buffer #%d): expected halo %d and channel stride %d, found halo %u and stride %u",
                  i, op->b[i], h, ld, d->halo, d->ld);
  return 0;
}
int rt_need_rows(const rt_ctx *c, const rt_op *op, int i, int dt, size_t rows, int ld) {
  if (rt_need(c, op, i, dt, rows * (size_t)ld)) return RT_E_PARAM;
  const rt_bufdesc *d = rt_bd(c, op, i);
  if (d->halo || (int)d->ld != ld)
    return rt_bad(c, op, "buffer argument %d (buffer #%d): expected unpadded rows of channel stride %d, found halo %u and "
                  "stride %u", i, op->b[i], ld, d->halo, d->ld);
  return 0;
}
int rt_need_nohalo(const rt_ctx *c, const rt_op *op, int i, int dt, size_t elems) {
  if (rt_need(c, op, i, dt, elems)) return RT_E_PARAM;
  const rt_bufdesc *d = rt_bd(c, op, i);
  if (d->halo) return rt_bad(c, op, "buffer argument %d (buffer #%d, input): expected no halo, found halo %u", i, op->b[i], d->halo);
  return 0;
}
int rt_need_t(const rt_ctx *c, const rt_op *op, int i, size_t nbytes, int atleast) {
  size_t nb = 0;
  if (!rt_t(c, op, i, &nb))
    return rt_bad(c, op, "tensor argument %d is absent (the op record has %d tensor arguments)", i, op->nt);
  if (atleast ? nb >= nbytes : nb == nbytes) return 0;
  const rt_tensor *t = rt_tensor_at(c->pkg, op->t[i], nullptr);
  return rt_bad(c, op, "tensor argument %d (tensor #%d '%.48s' %s [%u %u %u %u]): expected %s%zu bytes, found %llu bytes",
                i, op->t[i], t->name, rt_dtype_name(t->dtype), t->dims[0], t->dims[1], t->dims[2], t->dims[3],
                atleast ? ">= " : "", nbytes, (unsigned long long)t->nbytes);
}
int rt_need_args(const rt_ctx *c, const rt_op *op, int nb, int nt, int ni) {
  if ((nb < 0 || op->nb == nb) && (nt < 0 || op->nt == nt) && (ni < 0 || op->ni == ni)) return 0;
  return rt_bad(c, op, "op record shape: expected %d buffer, %d tensor and %d int arguments, found %d, %d and %d", nb, nt,
                ni, op->nb, op->nt, op->ni);
}

int rt_op_src(const rt_ctx *c, int i, char *buf, size_t n) {
  if (n) buf[0] = 0;
  if (!c->src) return -1;
  const char *p = c->src, *end = c->src + c->src_len;
  for (int k = 0; k < i && p < end; k++) {
    const char *nl = (const char *)memchr(p, '\n', (size_t)(end - p));
    if (!nl) return -1;
    p = nl + 1;
  }
  if (p >= end) return -1;
  const char *nl = (const char *)memchr(p, '\n', (size_t)(end - p));
  size_t l = (size_t)((nl ? nl : end) - p);
  if (n) { if (l > n - 1) l = n - 1; memcpy(buf, p, l); buf[l] = 0; }
  return 0;
}
const char *rt_op_name(const rt_ctx *c, int i) { return i >= 0 && i < c->n_ops && c->ops[i].k ? c->ops[i].k->name : "?"; }

const rt_kernel *rt_kernel_for(int code) {
  int base = code & 0xff, var = code >> 8;
  if (base <= 0 || base >= RT_OP_N) return nullptr;
  const rt_kernel *k = var == 0 ? rt_k_var0(base) : var == 1 ? rt_k_var1(base) : nullptr;
  return k && k->run ? k : nullptr;
}

static const char *op_prefix(const rt_ctx *c, int i, const char *kname, char *buf, size_t n) {
  char src[160];
  if (rt_op_src(c, i, src, sizeof src) == 0 && src[0]) {
    if (strlen(src) > 96) strcpy(src + 93, "...'");
    snprintf(buf, n, "op %d %s (ONNX node %s)", i, kname ? kname : "?", src);
  } else
    snprintf(buf, n, "op %d %s (no source node names in the package: compile with bnc 2 or newer)", i, kname ? kname : "?");
  return buf;
}
#define HINT_PKG "hint: package/library mismatch or a lowering bug: recompile with bnc; if it reproduces, report this message"
#define KIND(k) do { if (kind) *kind = (k); } while (0)
#define PFX(kname) op_prefix(c, (int)i, kname, pfx, sizeof pfx)

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

rt_ctx *rt_ctx_new(rt_pkg *p, int pi, char *err, size_t errlen, int *kind) {
  KIND(RT_E_PARAM);
  const rt_pathdesc *d = rt_path(p, pi);
  const uint8_t *m, *q, *end;
  char pfx[256];
  size_t total = 0;
  if (!d) { snprintf(err, errlen, "no path %d in the package (%d paths)", pi, rt_n_paths(p)); return nullptr; }
  rt_ctx *c = (rt_ctx *)calloc(1, sizeof *c);
  if (!c) { KIND(RT_E_OOM); snprintf(err, errlen, "out of memory (%zu bytes for the context)", sizeof *c); return nullptr; }
  c->pkg = p;
  c->path = d;
  c->fail_op = -1;
  c->err = err;
  c->errlen = errlen;
  c->n_buf = (int)d->n_buf;
  {
    char key[64];
    uint16_t ty;
    uint32_t vl;
    snprintf(key, sizeof key, "src_nodes/%.24s", d->name);
    const uint8_t *v = meta_find(p, key, &ty, &vl);
    if (v && (ty == 0 || ty == 3)) { c->src = (const char *)v; c->src_len = vl; }
  }
  m = (const uint8_t *)p->map;
  if (hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking) != hipSuccess) {
    c->stream = nullptr;
    KIND(RT_E_OOM);
    FAIL("cannot create a HIP stream (no usable GPU?); hint: check that an MI355X is visible (rocm-smi)");
  }
  c->own_stream = 1;
  c->bufd = (rt_bufdesc *)malloc(sizeof(rt_bufdesc) * d->n_buf);
  c->buf = (void **)calloc(d->n_buf, sizeof(void *));
  c->ws = (long long *)calloc(d->n_buf, sizeof(long long));
  c->wsb = (size_t *)calloc(d->n_buf, sizeof(size_t));
  c->slot_bytes = (size_t *)calloc(d->n_buf, sizeof(size_t));
  c->slot_users = (int *)calloc(d->n_buf, sizeof(int));
  if (!c->bufd || !c->buf || !c->ws || !c->wsb || !c->slot_bytes || !c->slot_users) { KIND(RT_E_OOM); FAIL("out of memory (%u buffer descriptors)", d->n_buf); }
  memcpy(c->bufd, m + d->buf_off, sizeof(rt_bufdesc) * d->n_buf);
  for (uint32_t i = 0; i < d->n_buf; i++) {
    const rt_bufdesc *b = &c->bufd[i];
    if (b->dtype > RT_I32 || b->elems > ((uint64_t)1 << 30) || b->slot >= d->n_buf)
      FAIL("path %.24s buffer #%u: bad descriptor (dtype %u, %llu elements, slot %u of %u); " HINT_PKG, d->name, i, b->dtype,
           (unsigned long long)b->elems, b->slot, d->n_buf);
    if ((i == d->in_buf) != (b->slot == c->bufd[d->in_buf].slot))
      FAIL("path %.24s buffer #%u shares the input window's memory slot %u; " HINT_PKG, d->name, i, b->slot);
    size_t bytes = ((size_t)b->elems * rt_dsize(b->dtype) + 64 + 63) & ~(size_t)63;
    if (bytes > c->slot_bytes[b->slot]) c->slot_bytes[b->slot] = bytes;
    c->slot_users[b->slot]++;
  }
  for (uint32_t s = 0; s < d->n_buf; s++) {
    total += c->slot_bytes[s];
    if (total > ((size_t)1 << 30))
      FAIL("path %.24s needs more than 1 GB of activation buffers per window; hint: the package is corrupt or the model is "
           "far larger than this runtime is built for", d->name);
  }
  for (uint32_t i = 0; i < d->n_buf; i++)
    if (i != d->out_buf && (c->bufd[i].slot == c->bufd[d->out_buf].slot ||
                            (d->emb_buf != 0xffffffffu && i != d->emb_buf && c->bufd[i].slot == c->bufd[d->emb_buf].slot)))
      FAIL("path %.24s buffer #%u shares memory slot %u with the output buffer (#%u / #%u); " HINT_PKG, d->name, i,
           c->bufd[i].slot, d->out_buf, d->emb_buf);
  {
    int k2 = arena_alloc(c, 1, err, errlen);
    if (k2) { KIND(k2); goto fail; }
  }
  c->ops = (rt_op *)calloc(d->n_ops, sizeof(rt_op));
  if (!c->ops) { KIND(RT_E_OOM); FAIL("out of memory (%u op records)", d->n_ops); }
  q = m + d->ops_off;
  end = q + d->ops_bytes;
  for (uint32_t i = 0; i < d->n_ops; i++) {
    uint16_t h[6];
    if (q + 12 > end) FAIL("op %u: truncated op list (%u ops declared, %u bytes); " HINT_PKG, i, d->n_ops, d->ops_bytes);
    memcpy(h, q, 12);
    size_t need = 12 + 4 * ((size_t)h[2] + h[3] + h[4]);
    if (h[1] < need || q + h[1] > end || ((uintptr_t)(q - m) % 4))
      FAIL("op %u: bad op record (%u bytes for %u buffer, %u tensor, %u int arguments); " HINT_PKG, i, h[1], h[2], h[3], h[4]);
    rt_op *op = &c->ops[i];
    op->code = h[0]; op->nb = h[2]; op->nt = h[3]; op->ni = h[4];
    op->b = (const int32_t *)(q + 12);
    op->t = op->b + op->nb;
    op->p = op->t + op->nt;
    for (int k = 0; k < op->nb; k++)
      if (op->b[k] >= (int32_t)d->n_buf || op->b[k] < -1)
        FAIL("%s: buffer argument %d names buffer #%d but the path has %u buffers; " HINT_PKG, PFX(nullptr), k, op->b[k],
             d->n_buf);
    for (int k = 0; k < op->nt; k++)
      if (op->t[k] >= (int32_t)p->n_tensors)
        FAIL("%s: tensor argument %d names tensor #%d but the package has %u tensors; " HINT_PKG, PFX(nullptr), k, op->t[k],
             p->n_tensors);
    int var = op->code >> 8;
    if (var && !(d->hwcap & RT_HW_FP16))
      FAIL("%s: fp16 kernel (opcode 0x%x) in path %.24s, which does not declare the fp16 requirement; " HINT_PKG,
           PFX(nullptr), op->code, d->name);
    if (var == 2 && !(d->hwcap & RT_HW_DOTPROD))
      FAIL("%s: dotprod kernel (opcode 0x%x) in path %.24s, which does not declare the dotprod requirement; " HINT_PKG,
           PFX(nullptr), op->code, d->name);
    const rt_kernel *k = op->k = rt_kernel_for(op->code);
    if (!k) {
      char comp[48];
      if (rt_meta_str(p, "compiler", comp, sizeof comp) < 0) snprintf(comp, sizeof comp, "unknown");
      FAIL("%s: unknown opcode 0x%x (base %d variant %d); this library runs opcodes 1..%d of variants 0 and 1 on the GPU "
           "(reader version %d), the package was written by compiler '%s'; hint: pick a path of the package this library "
           "runs (mode 0), or update libbnneon_hip", PFX(nullptr), op->code, op->code & 0xff, var, RT_OP_N - 1,
           RT_READER_VERSION, comp);
    }
    PFX(k->name);
    for (int a = 0; a < op->nb; a++) {
      if (op->b[a] < 0 && !(a < 32 && (k->optmask >> a & 1)))
        FAIL("%s: buffer argument %d is required by the kernel but absent (-1) in the op record; " HINT_PKG, pfx, a);
      if (op->b[a] == (int32_t)d->in_buf && a < 32 && (k->outmask >> a & 1))
        FAIL("%s: buffer argument %d is the input window (#%u) but the kernel writes it; " HINT_PKG, pfx, a, d->in_buf);
    }
    for (int a = 0; a < op->nb; a++)
      for (int b2 = 0; b2 < op->nb; b2++)
        if (a != b2 && op->b[a] >= 0 && op->b[b2] >= 0 && a < 32 && (k->outmask >> a & 1) &&
            (op->b[a] == op->b[b2] || c->bufd[op->b[a]].slot == c->bufd[op->b[b2]].slot))
          FAIL("%s: buffer arguments %d (#%d, written) and %d (#%d) share memory slot %u; " HINT_PKG, pfx, a, op->b[a], b2,
               op->b[b2], c->bufd[op->b[a]].slot);
    c->n_ops = (int)i + 1;
    c->err_kind = 0;
    c->err_params[0] = 0;
    if (k->init && k->init(c, op)) {
      char detail[400];
      snprintf(detail, sizeof detail, "%s", c->err_kind ? err : "init failed without a message (kernel bug)");
      if (c->err_kind == RT_E_OOM) {
        KIND(RT_E_OOM);
        snprintf(err, errlen, "%s: %s; hint: free device memory or use a smaller model", pfx, detail);
      } else {
        int n = snprintf(err, errlen, "%s: %s; " HINT_PKG, pfx, detail);
        if (n > 0 && (size_t)n + 24 < errlen && c->err_params[0])
          snprintf(err + n, errlen - (size_t)n, " (int params: [%s])", c->err_params);
      }
      goto fail;
    }
    q += h[1];
  }
  c->err = nullptr;
  {
    const char *fe = getenv("BNH_FUSE");  // BNH_FUSE=0 runs every op as the package lists it
    if (!fe || atoi(fe) != 0) fuse_ops(c);
    const char *se = getenv("BNH_SPLIT");  // BNH_SPLIT=0 runs every batch on one stream
    c->one_stream = se && atoi(se) == 0;
  }
  {
    const char *pe = getenv("BNN_PROF");
    c->prof = pe ? atoi(pe) : 0;
    if (c->prof) c->t_op = (double *)calloc(d->n_ops, sizeof(double));
  }
  return c;
fail:
  c->err = nullptr;
  rt_ctx_free(c);
  return nullptr;
}
#undef PFX

static double now_s(void) {
  struct timespec t;
  clock_gettime(CLOCK_MONOTONIC, &t);
  return t.tv_sec + t.tv_nsec * 1e-9;
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
  if (B > c->bcap) { snprintf(err, errlen, "rt_run_batch: %d windows but the arena holds %d", B, c->bcap); return -1; }
  if (hipMemsetAsync(c->win_fail, 0, sizeof(int) * (size_t)B, c->stream) != hipSuccess) {
    snprintf(err, errlen, "device error clearing the window flags");
    return -1;
  }
  // Sub-batches on their own streams, their launches interleaved op by op: the windows are independent, so the GPU
  // may run one sub-batch's kernel beside another's (a VALU-bound kernel beside a memory-bound one). Sub-batch h
  // runs one op behind sub-batch h - 1 (it starts after that one's first op, and so after everything the context's
  // stream held), so that kernels of different kinds meet more often than copies of the same kernel; the context's
  // stream waits for every sub-batch at the end.
  // two sub-batches (measured: three or four, on as many streams, are 15-25 % slower on both nets; one op of skew is
  // 1.5-1.7 % faster than none, four or more slower)
  int ns = 2;
  if (c->prof || c->one_stream || B < 64) ns = 1;
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
        return -1;
      }
      c->fail_op = i;  // ops read it to tag the windows they fail
      c->w0 = first(h);
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
        return -1;
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
      return -1;
    }
  c->fail_op = -1;
  hipError_t e = hipMemcpyAsync(status, c->win_fail, sizeof(int) * (size_t)B, hipMemcpyDeviceToHost, c->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
  if (e != hipSuccess) { snprintf(err, errlen, "device error after the op list: %s", hipGetErrorString(e)); return -1; }
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
  if (c->stream && c->own_stream) hipStreamDestroy(c->stream);
  for (int h = 1; h < c->n_sub; h++) {
    hipStreamSynchronize(c->sub_stream[h]);
    hipStreamDestroy(c->sub_stream[h]);
    hipEventDestroy(c->sub_fork[h]);
    hipEventDestroy(c->sub_join[h]);
  }
  free(c);
}
