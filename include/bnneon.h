/* libbnneon_hip: the libbnneon host API (cdw9bf/birdnet-neon-engine, src/bnneon.h:59-99) on an MI355X.
 *
 * Drop-in: the same 13 functions, the same bnn_info layout (struct_size handshake: fields only appended, the library
 * copies min(sizes)), the same .bnpk packages and modes, the same error texts and kinds. A context runs the package's
 * op list on the GPU, with every int8 op bit-identical to the reference's NEON kernels. What is added is batching:
 * bnn_infer_batch scores many windows per call (one kernel launch per op for all of them), discoverable with dlsym
 * the way bnn_set_threads is (src/bnneon.h:94-97). Legacy .bn24 / .bnv3 files are refused with BNN_ERR_PACKAGE (their
 * hand-written engines are not part of this library).
 *
 * Thread safety: one context per thread; contexts share nothing (each owns its HIP stream and device arena).
 */
#ifndef BNNEON_H
#define BNNEON_H
#include <stddef.h>
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

#define BNN_API_VERSION 2

enum { BNN_MODEL_V24 = 24, BNN_MODEL_V30 = 30, BNN_MODEL_PERCH_V2 = 120, BNN_MODEL_BAT_V24 = 224 };
enum { BNN_OUT_LOGITS = 0, BNN_OUT_SIGMOID = 1 };
enum { BNN_POST_NONE = 0, BNN_POST_SIGMOID = 1, BNN_POST_SOFTMAX = 2 };
/* 0: the first path of the package this library runs; 1: refused for packages; 2/3/4: the package's
 * "neon-fp32" / "neon-fp16" / "neon-int8" path (run on the GPU with the reference's arithmetic) */
enum { BNN_MODE_DEFAULT = 0, BNN_MODE_REFERENCE = 1, BNN_MODE_FP32 = 2, BNN_MODE_FP16 = 3, BNN_MODE_INT8 = 4 };

typedef struct {
  uint32_t struct_size;
  int model;
  int format_version;
  int sample_rate;
  int n_samples;
  int hop_samples;
  int n_classes;
  int output_kind;
  int post;
  float logit_scale;
  int emb_dim;
  int has_labels_sha;
  unsigned char labels_sha256[32];
  char model_id[64];
  char path[32];
  const char *precision;
} bnn_info; /* src/bnneon.h:36-55 */

typedef struct bnn_ctx bnn_ctx;

int bnn_api_version(void);                                                   /* src/bnneon.h:59 */
/* 1 for a known model family code when a GPU this library runs on is visible, else 0 (src/bnneon.h:60-66). As in the
 * reference this says nothing about a given package: whether this library runs one of its paths is bnn_probe's
 * info.path ("" = none). Mode 0 passes over paths with ops this library does not serve (the hand-written v2.4 front
 * end and head FE_STFT2, C0POOL, POSTPC, DENSE; the v3.0 front end FE_DBIMG), so such a package may be refused. */
int bnn_cpu_supported(int model);
int bnn_probe(const char *weights_path, bnn_info *info);                     /* src/bnneon.h:68 */
int bnn_probe_meta(const char *weights_path, const char *key, char *buf, size_t n); /* src/bnneon.h:74 */
int bnn_meta(const bnn_ctx *ctx, const char *key, char *buf, size_t n);       /* src/bnneon.h:75 */
bnn_ctx *bnn_init(const char *weights_path, int mode);                        /* src/bnneon.h:76 */
int bnn_get_info(const bnn_ctx *ctx, bnn_info *info);                         /* src/bnneon.h:77 */
/* one window (src/bnneon.h:80): info.n_samples floats -> info.n_classes logits (+ embedding); nonzero with
 * BNN_ERR_WINDOW when an op could not score it */
int bnn_infer(bnn_ctx *ctx, const float *pcm, float *out, float *emb);
int bnn_verify_labels(const char *weights_path, const char *labels_path);     /* src/bnneon.h:84 */
const char *bnn_last_error(void);                                             /* src/bnneon.h:88 */
enum { BNN_ERR_NONE = 0, BNN_ERR_PACKAGE = 1, BNN_ERR_OOM = 2, BNN_ERR_CPU = 3, BNN_ERR_WINDOW = 4, BNN_ERR_LABELS = 5,
       BNN_ERR_USAGE = 6 };
int bnn_last_error_kind(void);                                                /* src/bnneon.h:93 */
/* accepted for 1..64 as the reference (src/bnneon.h:98); the GPU path's parallelism is the batch, so the count
 * changes nothing and results are identical for every value */
int bnn_set_threads(bnn_ctx *ctx, int threads);
void bnn_free(bnn_ctx *ctx);                                                  /* src/bnneon.h:99 */

/* ---- batching (no counterpart in the reference, whose bnn_infer scores one window per call; added the way
 * bnn_set_threads was: look the symbols up with dlsym to support older libraries) */
/* n windows of info.n_samples floats each, back to back in host memory -> out [n][n_classes] (+ emb [n][emb_dim] when
 * emb != NULL and the model has one). status (or NULL): per window 0 = scored, else 1 + the index of the op that
 * could not score it. Returns 0 when every window was scored; the number of failed windows (> 0, BNN_ERR_WINDOW
 * naming the first) when some were not (their rows of out are what the ops left); -1 on other errors. */
int bnn_infer_batch(bnn_ctx *ctx, const float *pcm, int n, float *out, float *emb, int *status);
/* the same with DEVICE pointers (HBM) and the caller's HIP stream (NULL = the context's): pcm [n][n_samples],
 * out [n][n_classes], emb [n][emb_dim] or NULL; no host copies of the windows or the results */
int bnn_infer_batch_device(bnn_ctx *ctx, const float *pcm, int n, float *out, float *emb, int *status, void *stream);

#ifdef __cplusplus
}
#endif
#endif
