/* ref_glue.c -- TEST INFRASTRUCTURE ONLY. Flat-pointer entry points around
 * the reference's own CPU kernels (hanw/amd.c src/cpu.c, src/model.c),
 * compiled from the reference sources where they lie (oracle/Makefile) into
 * oracle/_ref/libref_cpu.so. Used to pin the restatement in amdc_oracle.c
 * and, when present, as the CPU baseline of bench.py. */
#include <stdlib.h>
#include <string.h>

#include "backend.h"
#include "common.h"
#include "model.h"

/* src/cpu.c:36 */
void ref_quant_q8(const float *x, uint8_t *q, uint32_t nb) { cpu_quant_q8(x, q, nb); }

/* model_mat_from_gguf (src/model.c:479-485): the reference's load-time
 * repack of GGUF bytes of type ttype (GGML_Q4_0 = 2, GGML_Q8_0 = 8,
 * GGML_Q4_K = 12, GGML_Q6_K = 14). Returns a heap mat (free with
 * ref_mat_free), NULL if it is not MAT_Q4 / MAT_Q8 / MAT_Q4K / MAT_Q6K. */
void *ref_mat_new(int ttype, const uint8_t *src, uint32_t rows, uint32_t cols) {
  mat *w = calloc(1, sizeof *w);
  model_mat_from_gguf(w, (uint32_t)ttype, src, rows, cols);
  if (w->kind != MAT_Q4 && w->kind != MAT_Q4K && w->kind != MAT_Q8 && w->kind != MAT_Q6K) {
    free(w->qw), free(w->qs), free(w->f), free(w);
    return NULL;
  }
  return w;
}

int ref_mat_kind(const void *h) { return ((const mat *)h)->kind; }

/* The repacked arrays: qw (rows*nb*4 words; *8 for MAT_Q8, *6 for MAT_Q6K)
 * and qs (rows*nb u16, plus rows*nb/4 for MAT_Q4K, rows*nb/8 for MAT_Q6K). */
void ref_mat_copy(const void *h, uint32_t *qw, uint16_t *qs) {
  const mat *w = h;
  const size_t rn = (size_t)w->rows * w->nb;
  const size_t nw = rn * (w->kind == MAT_Q8 ? 8u : w->kind == MAT_Q6K ? 6u : 4u);
  const size_t ns = rn + (w->kind == MAT_Q4K ? (size_t)w->rows * (w->nb / 8u) * 2u : w->kind == MAT_Q6K ? (size_t)w->rows * (w->nb / 8u) : 0u);
  memcpy(qw, w->qw, nw * 4u);
  memcpy(qs, w->qs, ns * 2u);
}

/* cpu_gemv_q4 / cpu_gemv_q4k / cpu_gemv_q6k / cpu_gemv_q8 (src/cpu.c:64, 93, 123, 154) */
void ref_mat_gemv(const void *h, const uint8_t *xq, float *y) {
  const mat *w = h;
  switch (w->kind) {
    case MAT_Q4: cpu_gemv_q4(w, xq, y); break;
    case MAT_Q4K: cpu_gemv_q4k(w, xq, y); break;
    case MAT_Q6K: cpu_gemv_q6k(w, xq, y); break;
    default: cpu_gemv_q8(w, xq, y);
  }
}

void ref_mat_free(void *h) {
  mat *w = h;
  if (!w) return;
  free(w->qw), free(w->qs), free(w);
}
