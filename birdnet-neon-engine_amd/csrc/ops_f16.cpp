// Registry kernels with fp16 arithmetic (variant 1, the reference's rt_ops_f16.c family) on the GPU.
#include <stdlib.h>

#include "bnh_internal.h"
#include "rt.h"

int rt_dwk_check(rt_ctx *c, rt_op *op, size_t esz);             // ops_f32.cpp
int rt_dw3_check(rt_ctx *c, rt_op *op, int dt, int pt, int pl);  // ops_f32.cpp
static inline const uint16_t *dev_h(const rt_op *op, int i) {
  return (const uint16_t *)((const rt_dev_state *)op->state)->t[i];
}
int rt_pw_out_check(rt_ctx *c, rt_op *op, int dt);             // ops_s8n.cpp
int rt_stem_check(rt_ctx *c, rt_op *op);                       // ops_f32.cpp
int rt_mean_check(rt_ctx *c, rt_op *op);
int rt_pad_check(rt_ctx *c, rt_op *op);
int rt_pad_run(rt_ctx *c, rt_op *op, int esz);
int rt_gemv_check(rt_ctx *c, rt_op *op, size_t esz);
int rt_gemv_run(rt_ctx *c, rt_op *op, int w16);
void *rt_dev_t(const rt_op *op, int i);

// -------- PW f16: b = [in f16 [M][lda], out, res | -1]; t = [w (hpack panels), b32, b16];
//          p = [N K Kp Np, M, lda, act, ldo, ow, opad, ldr]   (src/rt_ops_f16.c:14-27, 53-81; rt_pw_check,
//          src/rt_ops_f32.c:129-152)
typedef struct {
  bnh_h16w *W;
  void *ws;       // the split form's workspace (device), grown with the arena
  size_t ws_cap;  // bytes
} pw16_state;
static void pw16_fini(rt_op *op) {
  pw16_state *s = (pw16_state *)op->state;
  if (s) {
    bnh_h16w_free(s->W);
    if (s->ws) bnh_free(s->ws);
  }
  free(s);
}
static int pw16_init(rt_ctx *c, rt_op *op) {
  pw16_state *s = (pw16_state *)calloc(1, sizeof *s);
  op->state = s;
  if (!s) return rt_oom(c, op, sizeof *s);
  if (rt_need_args(c, op, 3, 3, 11)) return RT_E_PARAM;
  const int *p = op->p;
  const int N = p[0], K = p[1], Kp = p[2], Np = p[3];
  if (N <= 0 || K <= 0 || Np != ((N + 7) & ~7) || Kp < K || Kp % 8)
    return rt_bad(c, op, "GEMM shape N %d K %d Kp %d Np %d: expected Np = N rounded up to 8, Kp >= K, Kp %% 8 == 0", N,
                  K, Kp, Np);
  if (rt_need_t(c, op, 0, (size_t)Np * Kp * 2, 1) || rt_need_t(c, op, 1, (size_t)(Np + 16) * 4, 1) ||
      rt_need_t(c, op, 2, (size_t)(Np + 16) * 2, 1))
    return RT_E_PARAM;
  const int M = p[4], lda = p[5], act = p[6], ldo = p[7], opad = p[9], ldr = p[10];
  const size_t Mr = ((size_t)M + 7) & ~(size_t)7;
  RT_REQ(c, op, M > 0);
  RT_REQ(c, op, lda >= Kp);
  RT_REQ(c, op, ldo >= Np);
  RT_REQ(c, op, act >= 0 && act <= 2);
  RT_REQ(c, op, opad >= 0 && opad <= 3);
  if (rt_need(c, op, 0, RT_F16, Mr * lda) || rt_pw_out_check(c, op, RT_F16)) return RT_E_PARAM;
  if (op->b[2] >= 0) {
    RT_REQ(c, op, ldr >= Np);
    const rt_bufdesc *r = rt_bd(c, op, 2);
    if (r->halo)
      return rt_bad(c, op, "buffer argument 2 (buffer #%d, residual): halo %u needs an fp32 buffer with ld %d and H x W = "
                    "%d rows, found %s ld %u %ux%u", op->b[2], r->halo, ldr, M, rt_dtype_name(r->dtype), r->ld, r->H, r->W);
    if (rt_need(c, op, 2, RT_F16, (size_t)M * ldr)) return RT_E_PARAM;
  }
  RT_REQ(c, op, lda % 8 == 0);  // 16-byte operand loads (every package pads rows to 8 channels)
  s->W = bnh_h16w_new(N, K, Kp, Np, (const uint16_t *)rt_t(c, op, 0, nullptr), (const float *)rt_t(c, op, 1, nullptr),
                      (const uint16_t *)rt_t(c, op, 2, nullptr));
  if (!s->W) return rt_oom(c, op, (size_t)Np * Kp * 2);
  return 0;
}
// the fp16 gates of a gates-only SE, window 0: op scratch [bcap][C] fp32 gates, [bcap][rd] first-FC outputs, then
// [bcap][C] fp16 gates from the next 16-byte boundary (C % 8 == 0: every window's row stays 16-byte aligned)
static uint16_t *se_gh(const rt_ctx *c, const rt_op *se) {
  float *g = (float *)((const rt_dev_state *)se->state)->scratch;
  return (uint16_t *)(g + (((size_t)(se->p[0] + se->p[1]) * c->bcap + 3) & ~(size_t)3));
}

static int pw16_run(rt_ctx *c, rt_op *op) {
  pw16_state *s = (pw16_state *)op->state;
  const int *p = op->p;
  bnh_epi16 e = {p[6], (uint16_t *)rt_b(c, op, 1), rt_ws(c, op, 1), p[7], p[8], p[9], (const uint16_t *)rt_b(c, op, 2),
                 rt_ws(c, op, 2), p[10]};
  if (e.opad && !rt_halo_kept(c, op, 1)) {
    const int H = p[4] / p[8];
    if (bnh_zero_halo(e.out, e.out_ws, H, p[8], p[7], p[9], 2, c->nwin, c->stream)) return -1;
  }
  if (c->f16_mfma) {  // fp32 accumulation on the matrix cores: within the fp16 accumulation bound, not bit-exact
    const uint16_t *gh = op->se ? se_gh(c, op->se) + (size_t)op->se->p[0] * c->w0 : nullptr;
    return bnh_gemm_f16_mfma_body((const uint16_t *)rt_b(c, op, 0), rt_ws(c, op, 0), p[5], p[4], c->nwin, s->W, &e,
                                  gh, op->se ? op->se->p[0] : 0, c->stream);
  }
  // the split form's workspace: op-private, grown with the arena (the fp16 results of every K block of each window)
  void *ws = nullptr;
  size_t wsb = bnh_gemm_f16_ws_bytes(p[4], c->bcap, s->W);
  if (wsb) {
    if (s->ws_cap < wsb) {
      if (s->ws) bnh_free(s->ws);
      s->ws_cap = 0;
      if (!(s->ws = bnh_malloc(wsb))) {
        rt_oom(c, op, wsb);
        return -1;
      }
      s->ws_cap = wsb;
    }
    ws = (char *)s->ws + bnh_gemm_f16_ws_bytes(p[4], 1, s->W) * c->w0;  // this sub-batch's windows
  }
  if (op->se)  // the SE that precedes it left its rows unscaled: the gates apply as the rows are loaded
    return bnh_gemm_f16_gated_ws((const uint16_t *)rt_b(c, op, 0), rt_ws(c, op, 0), p[5], p[4], c->nwin, s->W, &e,
                                 se_gh(c, op->se) + (size_t)op->se->p[0] * c->w0, op->se->p[0], ws,
                                 bnh_gemm_f16_ws_bytes(p[4], c->nwin, s->W), c->stream);
  return bnh_gemm_f16_ws((const uint16_t *)rt_b(c, op, 0), rt_ws(c, op, 0), p[5], p[4], c->nwin, s->W, &e, ws,
                         bnh_gemm_f16_ws_bytes(p[4], c->nwin, s->W), c->stream);
}

// -------- DWK f16: as the fp32 op, fp16 buffers and tensors (src/rt_ops_f16.c:192-203)
static int dwk_init(rt_ctx *c, rt_op *op) {
  if (rt_dwk_check(c, op, 2)) return RT_E_PARAM;
  return rt_dev_tensors(c, op, 2);
}
static int dwk_run(rt_ctx *c, rt_op *op) {
  const int *p = op->p;
  return bnh_dwk_f16((const uint16_t *)rt_b(c, op, 0), rt_ws(c, op, 0), p[0], p[1], p[2], p[3], p[4], p[5], p[6],
                     dev_h(op, 0), dev_h(op, 1), p[9], (uint16_t *)rt_b(c, op, 1), rt_ws(c, op, 1), p[7], p[8],
                     (float *)rt_b(c, op, 2), rt_ws(c, op, 2), c->nwin, c->stream);
}

// -------- DW3 f16: b = [xp (halo 1), out, chsum f32]; t = [w f16 [9][C], b f16 [C]]; p = [H W C s Ho Wo pt pl]
//          (src/rt_ops_f16.c:83-122)
static int dw3_init(rt_ctx *c, rt_op *op) {
  if (rt_need_args(c, op, 3, 2, 8)) return RT_E_PARAM;
  RT_REQ(c, op, op->p[2] <= 2048);
  if (rt_dw3_check(c, op, RT_F16, op->p[6], op->p[7])) return RT_E_PARAM;
  return rt_dev_tensors(c, op, 2);
}
static int dw3_run(rt_ctx *c, rt_op *op) {
  const int *p = op->p;
  return bnh_dw3_f16((const uint16_t *)rt_b(c, op, 0), rt_ws(c, op, 0), p[0], p[1], p[2], p[3], p[6], p[7],
                     dev_h(op, 0), dev_h(op, 1), (uint16_t *)rt_b(c, op, 1), rt_ws(c, op, 1), p[4], p[5],
                     (float *)rt_b(c, op, 2), rt_ws(c, op, 2), c->nwin, c->stream);
}

// -------- STEM, fp32 math, fp16 padded output: b = [img, out f16, col f32, tmp f32 [M][Np]]
//          (src/rt_ops_f16.c:167-180); the kernel converts as it stores (no tmp pass)
static int stem_init(rt_ctx *c, rt_op *op) {
  if (rt_need_args(c, op, 4, -1, -1) || rt_stem_check(c, op) || rt_need(c, op, 1, RT_F16, 1)) return RT_E_PARAM;
  return rt_need(c, op, 3, RT_F32, (size_t)op->p[6] * op->p[7] * op->p[3]) ? RT_E_PARAM : 0;
}
static int stem_run(rt_ctx *c, rt_op *op) {
  const int *p = op->p;
  if (p[12] && !rt_halo_kept(c, op, 1) &&
      bnh_zero_halo(rt_b(c, op, 1), rt_ws(c, op, 1), p[6], p[7], p[11], p[12], 2, c->nwin, c->stream))
    return -1;
  return bnh_stem_f32to16_body((const float *)rt_b(c, op, 0), rt_ws(c, op, 0), p[4], p[5], p[8], p[9], p[6], p[7],
                               (const float *)rt_dev_t(op, 0), (const float *)rt_dev_t(op, 1), p[2], p[0], p[3], p[10],
                               (uint16_t *)rt_b(c, op, 1), rt_ws(c, op, 1), p[11], p[12], c->nwin, c->stream);
}

// -------- SE f16: b = [D f16 (in place), chsum]; t = [se1_w, se1_b, se2t, se2_b] (fp32); p = [C rd P]
//          (src/rt_ops_f16.c:124-137, rt_se_check src/rt_ops_f32.c:256-266)
static int se_init(rt_ctx *c, rt_op *op) {
  if (rt_need_args(c, op, 2, 4, 3)) return RT_E_PARAM;
  const int C = op->p[0], rd = op->p[1], P = op->p[2];
  RT_REQ(c, op, C > 0 && C % 8 == 0 && C <= 4096);
  RT_REQ(c, op, rd > 0 && rd <= 512);
  RT_REQ(c, op, P > 0);
  const size_t want[4] = {(size_t)rd * C, (size_t)rd, (size_t)rd * C, (size_t)C};
  for (int i = 0; i < 4; i++)
    if (rt_need_t(c, op, i, want[i] * 4, 0)) return RT_E_PARAM;
  if (rt_need(c, op, 0, RT_F16, (size_t)P * C) || rt_need(c, op, 1, RT_F32, (size_t)C)) return RT_E_PARAM;
  return rt_dev_tensors(c, op, 4);
}
static int se_run(rt_ctx *c, rt_op *op) {
  const int *p = op->p;
  // op scratch per window: the gates (C % 8 == 0: 16-byte aligned rows), then the first FC's outputs
  const long long g_ws = p[0];
  float *g = (float *)rt_dev_scratch(c, op, sizeof(float) * (size_t)(g_ws + p[1]) +
                                                (op->gate_only ? 2 * (size_t)p[0] + 16 : 0));
  if (!g) return -1;
  if (op->gate_only)  // the next op applies the gates as it loads the rows
    return bnh_se_gate_f16((const float *)rt_b(c, op, 1), rt_ws(c, op, 1), p[0], p[1], p[2], (const float *)dev_h(op, 0),
                           (const float *)dev_h(op, 1), (const float *)dev_h(op, 2), (const float *)dev_h(op, 3),
                           g + g_ws * c->w0, g_ws, g + g_ws * c->bcap + (long long)p[1] * c->w0,
                           se_gh(c, op) + (size_t)p[0] * c->w0, p[0], c->nwin, c->stream);
  return bnh_se_f16((const float *)rt_b(c, op, 1), rt_ws(c, op, 1), p[0], p[1], p[2], (const float *)dev_h(op, 0),
                    (const float *)dev_h(op, 1), (const float *)dev_h(op, 2), (const float *)dev_h(op, 3),
                    g + g_ws * c->w0, g_ws, g + g_ws * c->bcap + (long long)p[1] * c->w0, (uint16_t *)rt_b(c, op, 0),
                    rt_ws(c, op, 0), c->nwin, c->stream);
}

// -------- MEAN f16, PAD f16 (src/rt_ops_f16.c:204-214)
static int mean_init(rt_ctx *c, rt_op *op) {
  return rt_mean_check(c, op) || rt_need(c, op, 0, RT_F16, 1) ? RT_E_PARAM : 0;
}
static int mean_run(rt_ctx *c, rt_op *op) {
  return bnh_mean_f16((const uint16_t *)rt_b(c, op, 0), rt_ws(c, op, 0), op->p[0], op->p[1], op->p[2],
                      (float *)rt_b(c, op, 1), rt_ws(c, op, 1), c->nwin, c->stream);
}
static int pad_init(rt_ctx *c, rt_op *op) {
  return rt_pad_check(c, op) || rt_need(c, op, 0, RT_F16, 1) ? RT_E_PARAM : 0;
}
static int pad_run(rt_ctx *c, rt_op *op) { return rt_pad_run(c, op, 2); }

// -------- GEMV with fp16 weights, fp32 math (src/rt_ops_f16.c:160-166)
static int gemv_init(rt_ctx *c, rt_op *op) { return rt_gemv_check(c, op, 2); }
static int gemv_run(rt_ctx *c, rt_op *op) { return rt_gemv_run(c, op, 1); }

static const rt_kernel K_PW = {pw16_init, pw16_run, pw16_fini, "pw_f16", 0x2, 0x4};
static const rt_kernel K_STEM = {stem_init, stem_run, rt_dev_fini, "stem_f32to16", 0xe, 0};
static const rt_kernel K_SE = {se_init, se_run, rt_dev_fini, "se_f16", 0x1, 0};
static const rt_kernel K_MEAN = {mean_init, mean_run, nullptr, "mean_f16", 0x2, 0};
static const rt_kernel K_PAD = {pad_init, pad_run, nullptr, "pad_f16", 0x2, 0};
static const rt_kernel K_GEMV = {gemv_init, gemv_run, rt_dev_fini, "gemv_h16", 0x2, 0};
static const rt_kernel K_DW3 = {dw3_init, dw3_run, rt_dev_fini, "dw3_f16", 0x6, 0};
static const rt_kernel K_DWK = {dwk_init, dwk_run, rt_dev_fini, "dwk_f16", 0x6, 0};

int rt_fuse_se16(rt_ctx *c, rt_op *se, rt_op *pw) {
  (void)c;
  if (se->k != &K_SE || pw->k != &K_PW || pw->b[0] != se->b[0]) return 0;
  const int C = se->p[0], P = se->p[2];
  const int *p = pw->p;
  // the PW's rows are the SE's buffer as it stands: P rows of C channels, K = Kp = lda = C
  if (p[1] != C || p[2] != C || p[4] != P || p[5] != C) return 0;
  se->gate_only = 1;
  pw->se = se;
  return 1;
}

// the fp16 prototype head (ops_proto.cpp)
int bnh_proto_f16_init(rt_ctx *c, rt_op *op);
int bnh_proto_fp_run(rt_ctx *c, rt_op *op);
void bnh_proto_fp_fini(rt_op *op);
static const rt_kernel K_PROTO = {bnh_proto_f16_init, bnh_proto_fp_run, bnh_proto_fp_fini, "proto_f16", 0xe, 0};

const rt_kernel *rt_k_f16(int base) {
  switch (base) {
    case RT_OP_PROTO: return &K_PROTO;
    case RT_OP_PW: return &K_PW;
    case RT_OP_DW3: return &K_DW3;
    case RT_OP_DWK: return &K_DWK;
    case RT_OP_STEM: return &K_STEM;
    case RT_OP_SE: return &K_SE;
    case RT_OP_MEAN: return &K_MEAN;
    case RT_OP_PAD: return &K_PAD;
    case RT_OP_GEMV: return &K_GEMV;
    default: return nullptr;
  }
}
