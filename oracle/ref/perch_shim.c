/* Test infrastructure, not product code: a C entry point over the reference's own scalar Perch v2 oracle
 * (src/perch_ref.c with its .bnp2 loader src/perch_model.c), compiled from the reference checkout by oracle/Makefile's
 * `ref` target into oracle/_ref/libperchref.so. Only tests/ and bench.py's CPU-baseline leg load it, as a checker and
 * as the reference code's own CPU timing.
 *   prs_load     pc_model_load (src/perch_model.c:43) into a heap model; NULL and the loader's message on failure
 *   prs_infer    pc_ref_infer (src/perch_ref.c:382) with a context of its own: pcm [160000] -> logits [n_classes]
 *                and the embedding [1536]
 */
#include <stdlib.h>

#include "perch_internal.h"

void *prs_load(const char *path, char *err, int errlen) {
  pc_model *m = (pc_model *)calloc(1, sizeof *m);
  if (!m) return NULL;
  if (pc_model_load(m, path, err, (size_t)errlen)) {
    free(m);
    return NULL;
  }
  return m;
}

int prs_n_classes(const void *h) { return ((const pc_model *)h)->n_classes; }

int prs_infer(const void *h, const float *pcm, float *logits, float *emb) {
  pc_ref *r = pc_ref_new((const pc_model *)h);
  if (!r) return -1;
  const int rc = pc_ref_infer(r, pcm, logits, emb);
  pc_ref_free(r);
  return rc;
}

void prs_free(void *h) {
  if (!h) return;
  pc_model_unload((pc_model *)h);
  free(h);
}
