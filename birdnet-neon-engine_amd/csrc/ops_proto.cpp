// PROTO_S8: the int8 prototype head's op contract (src/rt_ops_s8n.c:212-253 with rt_proto_geom / rt_proto_io,
// src/rt_ops_f32.c:525-546), run on the GPU for a batch of windows.
//   b = [x f32 [P][ld], logits f32 [nc], qa i8 [P][Kp], colmax f32 [Np]];
//   t = [qw i8 [Np/4][Kp/16][4][16], sw f32 [Np], n4 i8 [Np/4], cls w [nc][ppc], cls b [nc], eps [1]];
//   p = [N K Kp Np, P C ld nc ppc]
#include <stdlib.h>
#include <string.h>

#include "bnh_internal.h"
#include "rt.h"



typedef struct {
  bnh_s8p *W;
  float *clsw, *clsb;  // device copies of the class tensors
  float eps;
  float *sx;           // device [bcap][P] cell scales (op-private scratch)
  int sx_cap;
} proto_state;

// the geometry of a prototype head (rt_proto_geom): P cells of C channels (row stride ld), N = nc * ppc prototypes
// of length K = C
static int proto_geom(rt_ctx *c, rt_op *op, int nt, int ni, int kmax) {
  if (rt_need_args(c, op, 4, nt, ni)) return RT_E_PARAM;
  const int *p = op->p, *q = p + ni - 5;
  int N = p[0], K = p[1], P = q[0], C = q[1], ld = q[2], nc = q[3], ppc = q[4];
  RT_REQ(c, op, P > 0 && P <= 65536 && nc > 0 && ppc >= 1);
  RT_REQ(c, op, N > 0 && N <= (1 << 26) && K > 0 && K <= kmax);
  RT_REQ(c, op, K == C);
  RT_REQ(c, op, ld >= C);
  RT_REQ(c, op, (size_t)nc * ppc == (size_t)N);
  return 0;
}

// the n4 loader check (pc_proto_n4_check, src/proto_s8n.c:115-132): flagged panels must keep every lane of 4
// weights (bytes l, l + 8 of two consecutive 16-byte steps of a prototype) at sum |w| <= 258. The GPU kernels sum in
// int32 and never need the flags, but a package that forges them is refused here as by the reference.
static int n4_check(const int8_t *qw, int Kp, const uint8_t *n4, int npanels) {
  if (Kp % 32) return -1;
  for (int pn = 0; pn < npanels; pn++) {
    if (!n4[pn]) continue;
    const int8_t *w = qw + (size_t)pn * Kp * 4;
    for (int k = 0; k < Kp; k += 32, w += 128)
      for (int ch = 0; ch < 4; ch++)
        for (int l = 0; l < 8; l++) {
          int s = abs(w[16 * ch + l]) + abs(w[16 * ch + l + 8]) + abs(w[64 + 16 * ch + l]) + abs(w[64 + 16 * ch + l + 8]);
          if (s > 258) return pn;
        }
  }
  return -1;
}

static float *upload_f32(const void *h, size_t n) {
  float *d = (float *)bnh_malloc(n * 4 ? n * 4 : 4);
  if (d && bnh_memcpy_h2d(d, h, n * 4)) { hipFree(d); return nullptr; }
  return d;
}

int bnh_proto_s8_init(rt_ctx *c, rt_op *op) {
  proto_state *s = (proto_state *)calloc(1, sizeof *s);
  op->state = s;
  if (!s) return rt_oom(c, op, sizeof *s);
  if (proto_geom(c, op, 6, 9, 1 << 17)) return RT_E_PARAM;
  const int *p = op->p;
  int N = p[0], K = p[1], Kp = p[2], Np = p[3], P = p[4], C = p[5], ld = p[6], nc = p[7];
  RT_REQ(c, op, C % 8 == 0 && Kp == ((K + 15) & ~15));
  RT_REQ(c, op, P % 4 == 0 && Np == ((N + 3) & ~3));
  if (rt_need_t(c, op, 0, (size_t)Np * Kp, 0) || rt_need_t(c, op, 1, (size_t)Np * 4, 1) ||
      rt_need_t(c, op, 2, (size_t)Np / 4, 1))
    return RT_E_PARAM;
  if (rt_need_t(c, op, 3, (size_t)N * 4, 0) || rt_need_t(c, op, 4, (size_t)nc * 4, 0) || rt_need_t(c, op, 5, 4, 0))
    return RT_E_PARAM;
  if (rt_need_nohalo(c, op, 0, RT_F32, (size_t)P * ld) || rt_need(c, op, 1, RT_F32, (size_t)nc)) return RT_E_PARAM;
  if (rt_need(c, op, 2, RT_I8, (size_t)P * Kp) || rt_need(c, op, 3, RT_F32, (size_t)Np)) return RT_E_PARAM;
  const int8_t *qw = (const int8_t *)rt_t(c, op, 0, nullptr);
  int bad = n4_check(qw, Kp, (const uint8_t *)rt_t(c, op, 2, nullptr), Np / 4);
  if (bad >= 0)
    return rt_bad(c, op, "prototype panel %d is flagged for 4 products per int16 lane, but a lane's 4 weights sum to more "
                  "than 258 (the sums could wrap)", bad);
  memcpy(&s->eps, rt_t(c, op, 5, nullptr), 4);
  s->W = bnh_s8p_new(Np, Kp, qw, (const float *)rt_t(c, op, 1, nullptr));
  s->clsw = upload_f32(rt_t(c, op, 3, nullptr), (size_t)N);
  s->clsb = upload_f32(rt_t(c, op, 4, nullptr), (size_t)nc);
  if (!s->W || !s->clsw || !s->clsb) return rt_oom(c, op, (size_t)Np * Kp);
  return 0;
}

int bnh_proto_s8_run(rt_ctx *c, rt_op *op) {
  proto_state *s = (proto_state *)op->state;
  const int *p = op->p;
  const int N = p[0], Kp = p[2], P = p[4], C = p[5], ld = p[6], nc = p[7], ppc = p[8], B = c->nwin;
  (void)N;
  if (s->sx_cap < c->bcap) {  // per-window cell scales: op-private, grown with the arena
    if (s->sx) hipFree(s->sx);
    s->sx = (float *)bnh_malloc(sizeof(float) * (size_t)P * c->bcap);
    if (!s->sx) { s->sx_cap = 0; return -1; }
    s->sx_cap = c->bcap;
  }
  int8_t *qa = (int8_t *)rt_b(c, op, 2);
  float *cm = (float *)rt_b(c, op, 3);
  float *sx = s->sx + (size_t)P * c->w0;  // this sub-batch's windows
  if (bnh_quant_cells((const float *)rt_b(c, op, 0), rt_ws(c, op, 0), P, C, ld, s->eps, qa, rt_ws(c, op, 2), Kp, sx, P,
                      B, c->stream))
    return -1;
  if (bnh_proto_colmax(qa, rt_ws(c, op, 2), sx, P, P, s->W, cm, rt_ws(c, op, 3), B, c->stream)) return -1;
  return bnh_proto_logits(cm, rt_ws(c, op, 3), s->clsw, s->clsb, nc, ppc, (float *)rt_b(c, op, 1), rt_ws(c, op, 1), B,
                          c->win_fail + c->w0, c->fail_op + 1, c->stream);
}

void bnh_proto_s8_fini(rt_op *op) {
  proto_state *s = (proto_state *)op->state;
  if (s) {
    bnh_s8p_free(s->W);
    if (s->clsw) hipFree(s->clsw);
    if (s->clsb) hipFree(s->clsb);
    if (s->sx) hipFree(s->sx);
  }
  free(s);
}

// -------- PROTO variant 2 (proto8_init / proto8_run, src/rt_ops_f16.c:252-281): the dotprod prototype head on fp16
//   cells. b = [x f16 [P][ld], logits f32 [nc], qa int8 [P][K], colmax f32 [Np]];
//   t = [qw int8 [Np/12][K/4][12][4], sw f32 [Np], cls w, cls b, eps]; p = [N K Np, P C ld nc ppc]
// The cells' int8 rows are padded to Kp = K rounded up to 16, so they live in op-private scratch rather than in qa.
typedef struct {
  bnh_s8p *W;
  float *clsw, *clsb;
  float eps;
  void *work;  // per window: sx [P] floats, then the rows [P][Kp]
  size_t cap, ws;
} proto8_state;

int bnh_proto8_dot_init(rt_ctx *c, rt_op *op) {
  proto8_state *s = (proto8_state *)calloc(1, sizeof *s);
  op->state = s;
  if (!s) return rt_oom(c, op, sizeof *s);
  /* K <= 2^17: an int32 sum of K products of at most 128 x 127 cannot overflow */
  if (proto_geom(c, op, 5, 8, 1 << 17)) return RT_E_PARAM;
  const int *p = op->p;
  int N = p[0], K = p[1], Np = p[2], P = p[3], ld = p[5], nc = p[6];
  RT_REQ(c, op, K % 8 == 0);
  RT_REQ(c, op, P % 8 == 0 && Np % 12 == 0 && Np >= N);
  if (rt_need_t(c, op, 0, (size_t)Np * K, 1) || rt_need_t(c, op, 1, (size_t)Np * 4, 1)) return RT_E_PARAM;
  if (rt_need_t(c, op, 2, (size_t)N * 4, 0) || rt_need_t(c, op, 3, (size_t)nc * 4, 0) || rt_need_t(c, op, 4, 4, 0))
    return RT_E_PARAM;
  if (rt_need_nohalo(c, op, 0, RT_F16, (size_t)P * ld) || rt_need(c, op, 1, RT_F32, (size_t)nc)) return RT_E_PARAM;
  if (rt_need(c, op, 2, RT_I8, (size_t)P * K) || rt_need(c, op, 3, RT_F32, (size_t)Np)) return RT_E_PARAM;
  memcpy(&s->eps, rt_t(c, op, 4, nullptr), 4);
  s->W = bnh_s8p_new_c12(Np, K, (const int8_t *)rt_t(c, op, 0, nullptr), (const float *)rt_t(c, op, 1, nullptr));
  s->clsw = upload_f32(rt_t(c, op, 2, nullptr), (size_t)N);
  s->clsb = upload_f32(rt_t(c, op, 3, nullptr), (size_t)nc);
  const size_t Kp = (size_t)((K + 15) & ~15);
  s->ws = ((size_t)P * 4 + (size_t)P * Kp + 255) / 256 * 256;
  if (!s->W || !s->clsw || !s->clsb) return rt_oom(c, op, (size_t)Np * Kp);
  return 0;
}

int bnh_proto8_dot_run(rt_ctx *c, rt_op *op) {
  proto8_state *s = (proto8_state *)op->state;
  const int *p = op->p;
  const int K = p[1], P = p[3], C = p[4], ld = p[5], nc = p[6], ppc = p[7], B = c->nwin, Kp = (K + 15) & ~15;
  const size_t need = s->ws * (size_t)c->bcap;
  if (s->cap < need) {
    if (s->work) hipFree(s->work);
    s->cap = 0;
    if (!(s->work = bnh_malloc(need))) {
      rt_oom(c, op, need);
      return -1;
    }
    s->cap = need;
  }
  char *base = (char *)s->work + s->ws * c->w0;  // this sub-batch's window slots
  float *sx = (float *)base;
  int8_t *qa = (int8_t *)(base + (size_t)P * 4);
  const long long ws = (long long)s->ws;
  float *cm = (float *)rt_b(c, op, 3);
  if (bnh_quant_cells_f16((const uint16_t *)rt_b(c, op, 0), rt_ws(c, op, 0), P, C, ld, s->eps, qa, ws, Kp, sx, ws / 4,
                          B, c->stream))
    return -1;
  if (bnh_proto_colmax(qa, ws, sx, ws / 4, P, s->W, cm, rt_ws(c, op, 3), B, c->stream)) return -1;
  return bnh_proto_logits(cm, rt_ws(c, op, 3), s->clsw, s->clsb, nc, ppc, (float *)rt_b(c, op, 1), rt_ws(c, op, 1), B,
                          c->win_fail + c->w0, c->fail_op + 1, c->stream);
}

void bnh_proto8_dot_fini(rt_op *op) {
  proto8_state *s = (proto8_state *)op->state;
  if (s) {
    bnh_s8p_free(s->W);
    if (s->clsw) hipFree(s->clsw);
    if (s->clsb) hipFree(s->clsb);
    if (s->work) hipFree(s->work);
  }
  free(s);
}

// -------- PROTO variant 0 (proto_init / proto_run, src/rt_ops_f32.c:548-570), PROTO_F32H (proto_h_init /
// proto_h_run, :572-591) and PROTO variant 1 (src/rt_ops_f16.c:227-250): the fp32 / fp16 prototype heads.
//   b = [x [P][ld], logits f32 [nc], a [P][C] scratch, colmax f32 [Np]];
//   PROTO f32: t = [w fp32 panels, b, cls w, cls b, eps], p = [N K Kp Np, P C ld nc ppc];
//   PROTO f16: t = [w hpack panels, b32, b16, cls w, cls b, eps], p = [N K Kp Np, P C ld nc ppc];
//   PROTO_F32H: t = [w16 [Np/8][K][8], cls w, cls b, eps], p = [N K Np, P C ld nc ppc]
typedef struct {
  bnh_fproto *W;
  float *clsw, *clsb;
  float eps;
  int f16;
} fproto_state;

// the class tensors at ct, ct + 1, ct + 2, the unpadded cells (buffer 0, dtype dt) and the logits (rt_proto_io,
// src/rt_ops_f32.c:537-546)
static int proto_io(rt_ctx *c, rt_op *op, int ct, int dt) {
  const int *p = op->p, *q = p + op->ni - 5;
  const int N = p[0], P = q[0], ld = q[2], nc = q[3];
  if (rt_need_t(c, op, ct, (size_t)N * 4, 0) || rt_need_t(c, op, ct + 1, (size_t)nc * 4, 0) ||
      rt_need_t(c, op, ct + 2, 4, 0))
    return RT_E_PARAM;
  if (rt_need_nohalo(c, op, 0, dt, (size_t)P * ld)) return RT_E_PARAM;
  return rt_need(c, op, 1, RT_F32, (size_t)nc);
}

// after the geometry and the pack view: Kp = K, 8-cell / 8-channel tiles, then tensors and buffers (rt_proto_check,
// src/rt_ops_f32.c:547-556); nw = the pack's tensor count (2 fp32, 3 fp16)
static int proto_check(rt_ctx *c, rt_op *op, int nw) {
  const int *p = op->p;
  const int K = p[1], P = p[4], C = p[5], dt = nw == 3 ? RT_F16 : RT_F32;
  RT_REQ(c, op, p[2] == K);
  RT_REQ(c, op, C % 8 == 0 && P % 8 == 0);
  if (proto_io(c, op, nw, dt)) return RT_E_PARAM;
  return rt_need(c, op, 2, dt, (size_t)P * C) || rt_need(c, op, 3, RT_F32, (size_t)p[3]) ? RT_E_PARAM : 0;
}

static int fproto_finish(rt_ctx *c, rt_op *op, fproto_state *s, int kind, int Np, int K, const void *w, int ct) {
  const int N = op->p[0], nc = op->p[op->ni - 2];
  memcpy(&s->eps, rt_t(c, op, ct + 2, nullptr), 4);
  s->f16 = kind == 2;
  s->W = bnh_fproto_new(kind, Np, K, w);
  s->clsw = upload_f32(rt_t(c, op, ct, nullptr), (size_t)N);
  s->clsb = upload_f32(rt_t(c, op, ct + 1, nullptr), (size_t)nc);
  if (!s->W || !s->clsw || !s->clsb) return rt_oom(c, op, (size_t)Np * K * (kind ? 2 : 4));
  return 0;
}

// PROTO variant 0 and variant 1: the GEMM pack view (rt_fpack_view / hpack_view) then rt_proto_check
static int proto_fp_init(rt_ctx *c, rt_op *op, bool f16) {
  fproto_state *s = (fproto_state *)calloc(1, sizeof *s);
  op->state = s;
  if (!s) return rt_oom(c, op, sizeof *s);
  if (proto_geom(c, op, f16 ? 6 : 5, 9, 1 << 20)) return RT_E_PARAM;
  const int *p = op->p;
  const int N = p[0], K = p[1], Kp = p[2], Np = p[3];
  if (f16) {
    if (Np != ((N + 7) & ~7) || Kp < K || Kp % 8)
      return rt_bad(c, op, "GEMM shape N %d K %d Kp %d Np %d: expected Np = N rounded up to 8, Kp >= K, Kp %% 8 == 0",
                    N, K, Kp, Np);
    if (rt_need_t(c, op, 0, (size_t)Np * Kp * 2, 1) || rt_need_t(c, op, 1, (size_t)(Np + 16) * 4, 1) ||
        rt_need_t(c, op, 2, (size_t)(Np + 16) * 2, 1))
      return RT_E_PARAM;
  } else {
    if (N <= 0 || K <= 0 || Np != ((N + 7) & ~7) || Kp < K || Kp % 4)
      return rt_bad(c, op, "GEMM shape N %d K %d Kp %d Np %d: expected Np = N rounded up to 8, Kp >= K, Kp %% 4 == 0",
                    N, K, Kp, Np);
    if (rt_need_t(c, op, 0, (size_t)Np * Kp * 4, 1) || rt_need_t(c, op, 1, (size_t)Np * 4, 1)) return RT_E_PARAM;
  }
  if (proto_check(c, op, f16 ? 3 : 2)) return RT_E_PARAM;
  return fproto_finish(c, op, s, f16 ? 2 : 0, Np, K, rt_t(c, op, 0, nullptr), f16 ? 3 : 2);
}
int bnh_proto_f32_init(rt_ctx *c, rt_op *op) { return proto_fp_init(c, op, false); }
int bnh_proto_f16_init(rt_ctx *c, rt_op *op) { return proto_fp_init(c, op, true); }

int bnh_proto_f32h_init(rt_ctx *c, rt_op *op) {
  fproto_state *s = (fproto_state *)calloc(1, sizeof *s);
  op->state = s;
  if (!s) return rt_oom(c, op, sizeof *s);
  if (proto_geom(c, op, 4, 8, 1 << 20)) return RT_E_PARAM;
  const int *p = op->p;
  const int N = p[0], K = p[1], Np = p[2], P = p[3], C = p[4];
  RT_REQ(c, op, K % 4 == 0);
  RT_REQ(c, op, P % 8 == 0 && Np % 8 == 0 && Np >= N);
  if (rt_need_t(c, op, 0, (size_t)Np * K * 2, 1) || proto_io(c, op, 1, RT_F32)) return RT_E_PARAM;
  if (rt_need(c, op, 2, RT_F32, (size_t)P * C) || rt_need(c, op, 3, RT_F32, (size_t)Np)) return RT_E_PARAM;
  // the GPU's repack and chains take K in steps of 8 (every package's cells are 8-channel rows: C % 8 == 0)
  if (K % 8) return rt_bad(c, op, "K %d: this library's fp32 prototype head takes K %% 8 == 0", K);
  return fproto_finish(c, op, s, 1, Np, K, rt_t(c, op, 0, nullptr), 1);
}

int bnh_proto_fp_run(rt_ctx *c, rt_op *op) {
  fproto_state *s = (fproto_state *)op->state;
  const int *q = op->p + op->ni - 5;
  const int P = q[0], C = q[1], ld = q[2], nc = q[3], ppc = q[4], B = c->nwin;
  float *cm = (float *)rt_b(c, op, 3);
  void *a = rt_b(c, op, 2);
  if (bnh_l2norm_cells(rt_b(c, op, 0), rt_ws(c, op, 0), P, C, ld, s->eps, s->f16, a, rt_ws(c, op, 2), B, c->stream))
    return -1;
  if (bnh_fproto_colmax(a, rt_ws(c, op, 2), P, s->W, cm, rt_ws(c, op, 3), B, c->stream)) return -1;
  return bnh_proto_logits(cm, rt_ws(c, op, 3), s->clsw, s->clsb, nc, ppc, (float *)rt_b(c, op, 1), rt_ws(c, op, 1), B,
                          c->win_fail + c->w0, c->fail_op + 1, c->stream);
}

void bnh_proto_fp_fini(rt_op *op) {
  fproto_state *s = (fproto_state *)op->state;
  if (s) {
    bnh_fproto_free(s->W);
    if (s->clsw) hipFree(s->clsw);
    if (s->clsb) hipFree(s->clsb);
  }
  free(s);
}
