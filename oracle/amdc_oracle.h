/* amdc_oracle.h -- TEST INFRASTRUCTURE ONLY.
 *
 * A CPU restatement of the reference's quantized GEMV path (hanw/amd.c,
 * src/cpu.c and the integer spec core/ie_core.h), used as the checker for the
 * HIP product path. Only tests/, __graft_entry__.smoke() and bench.py's CPU
 * baseline may call it; the product library never links or loads it.
 *
 * Layouts are the reference's own:
 *  - Q8 activation buffer of nb blocks (src/common.h:25-29):
 *      [int8 q[32 nb] | float d[nb] | u32 asum[nb]]  (40 nb bytes)
 *  - MAT_Q4  (src/model.h:17-21, core/ie_core.h:72-77): qw u32[rows*nb*4]
 *      (byte j of a block: weight j in the low nibble, j+16 in the high),
 *      qs f16[rows*nb]
 *  - MAT_Q4K (src/model.h:25-29, core/ie_core.h:247-263): qw as MAT_Q4 (the
 *      nibbles of each 32-weight sub-block in Q4_0 order), qs u16: (sc|mn<<8)
 *      per sub-block, then (f16 d, f16 dmin) per 256-weight super-block.
 *  - MAT_Q8  (src/model.h:23-24, core/ie_core.h:187-198): qw u32[rows*nb*8]
 *      (the 32 int8 weights of a block, 4 per word), qs f16[rows*nb]
 *  - MAT_Q6K (src/model.h:30-33, core/ie_core.h:306-349): qw = the low 4 bits
 *      as MAT_Q4 words (rows*nb*4), then 2 high-bit words per sub-block
 *      (rows*nb*2); qs u16: (sc0 | sc1 << 8) per sub-block (int8 scales of its
 *      two halves), then f16 d per 256-weight super-block.
 */
#ifndef AMDC_ORACLE_H
#define AMDC_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

float or_f16_to_f32(uint16_t h);
uint16_t or_f32_to_f16(float f);

/* Q8 activation quantization (src/cpu.c:36-53). q gets 40*nb bytes. */
void or_quant_q8(const float *x, uint8_t *q, uint32_t nb);

/* The producers of Q8 vectors in a decode step (the float part; the Q8 copy
 * is or_quant_q8 of the result, as src/cpu.c:501-504, 579-581 do):
 * RMSNorm y = x s w, s = 1 / sqrtf(sum x^2 / n + eps) (src/cpu.c:276-281);
 * SwiGLU a = a / (1 + expf(-a)) b in place (src/cpu.c:580). */
void or_rmsnorm(const float *x, const float *w, float *y, uint32_t n, float eps);
void or_swiglu(float *a, const float *b, uint32_t n);

/* GGUF -> the reference's MAT_Q4 / MAT_Q4K layouts (src/model.c:205-219,
 * 246-267). qw: rows*nb*4 words; qs: rows*nb (Q4) or rows*nb + rows*nb/4
 * (Q4K) u16 entries. */
void or_repack_q4(const uint8_t *src, uint32_t rows, uint32_t nb, uint32_t *qw, uint16_t *qs);
void or_repack_q4k(const uint8_t *src, uint32_t rows, uint32_t nb, uint32_t *qw, uint16_t *qs);
size_t or_q4k_qs_n(uint32_t rows, uint32_t nb);

/* GGUF -> the reference's MAT_Q8 / MAT_Q6K layouts (src/model.c:221-237,
 * 269-292). Q8: qw rows*nb*8 words, qs rows*nb. Q6K: qw rows*nb*6 words, qs
 * rows*nb + rows*nb/8 (or_q6k_qs_n). */
void or_repack_q8(const uint8_t *src, uint32_t rows, uint32_t nb, uint32_t *qw, uint16_t *qs);
void or_repack_q6k(const uint8_t *src, uint32_t rows, uint32_t nb, uint32_t *qw, uint16_t *qs);
size_t or_q6k_qs_n(uint32_t rows, uint32_t nb);

/* y = W x in the reference's order (src/cpu.c:64-87, 93-118): lane l of a
 * 32-lane wave adds the blocks l, l+32, ... of a row, then the lane sums are
 * added by the tree 16, 8, 4, 2, 1. Bitwise equal to the reference. */
void or_gemv_q4(const uint32_t *qw, const uint16_t *qs, uint32_t rows, uint32_t nb, const uint8_t *xq, float *y);
void or_gemv_q4k(const uint32_t *qw, const uint16_t *qs, uint32_t rows, uint32_t nb, const uint8_t *xq, float *y);
/* The same lanes and tree for MAT_Q8 (src/cpu.c:152-175: acc += (dw da) dot)
 * and MAT_Q6K (src/cpu.c:120-150: acc = fma(fma(d sc1, d1, (d sc0) d0), da, acc)). */
void or_gemv_q8(const uint32_t *qw, const uint16_t *qs, uint32_t rows, uint32_t nb, const uint8_t *xq, float *y);
void or_gemv_q6k(const uint32_t *qw, const uint16_t *qs, uint32_t rows, uint32_t nb, const uint8_t *xq, float *y);

/* The fused epilogue of a GEMV row (src/cpu.c:513-520): y = y (+ bias[r])
 * then (res[r] +) y. bias/res may be NULL. */
void or_epilogue(float *y, uint32_t rows, const float *bias, const float *res);

/* The integer block dots: out[r*nb + b] = ie_q4q8_block (Q4_0: sum (q-8) a,
 * core/ie_core.h:161-167) or ie_q4k_dot (Q4_K: sum q a, :281-286), as int32. */
void or_block_dots_q4(const uint32_t *qw, uint32_t rows, uint32_t nb, const uint8_t *xq, int32_t *out);
void or_block_dots_q4k(const uint32_t *qw, uint32_t rows, uint32_t nb, const uint8_t *xq, int32_t *out);
/* Q8_0: out[r*nb + b] = ie_q8q8_block (core/ie_core.h:222-233). Q6_K: the two
 * half dots sum (q - 32) a of sub-block b at out[(r*nb + b)*2 + h]
 * (ie_q6k_dots, core/ie_core.h:384-389). */
void or_block_dots_q8(const uint32_t *qw, uint32_t rows, uint32_t nb, const uint8_t *xq, int32_t *out);
void or_block_dots_q6k(const uint32_t *qw, uint32_t rows, uint32_t nb, const uint8_t *xq, int32_t *out);

/* The same integer dots by brute force over the GGUF bytes (int64 element
 * loop): an independent check of the functions above. kind: the GGML id
 * (2 Q4_0, 8 Q8_0, 12 Q4_K, 14 Q6_K; Q6_K gives two half dots per block). */
void or_block_dots_gguf(int kind, const uint8_t *src, uint32_t rows, uint32_t nb, const uint8_t *xq, int32_t *out);

/* GGUF dequantization of n weights from element `first` (src/model.c:89-97
 * for Q8_0, :98-107 for Q4_0, :108-140 for Q6_K, :142-171 for Q4_K). kind:
 * the GGML id (2, 8, 12, 14). */
void or_dequant(int kind, const uint8_t *src, uint64_t first, uint64_t n, float *out);
/* the same for weights 0 .. n - 1 on nthreads threads */
void or_dequant_mt(int kind, const uint8_t *src, uint64_t n, float *out, int nthreads);

/* A double-precision reference of y = W x straight from the GGUF bytes, and
 * the sum of |terms| of each row (tests/kernel_test.c:59-80): y_ref, mag. */
void or_gemv_f64(int kind, const uint8_t *src, uint32_t rows, uint32_t nb, const uint8_t *xq, double *y_ref, double *mag);

/* Row-parallel runs of or_gemv_q4 / or_gemv_q4k over nthreads threads: the
 * same per-row arithmetic, so the same bits. For the CPU baseline. */
void or_gemv_q4_mt(const uint32_t *qw, const uint16_t *qs, uint32_t rows, uint32_t nb, const uint8_t *xq, float *y, int nthreads);
void or_gemv_q4k_mt(const uint32_t *qw, const uint16_t *qs, uint32_t rows, uint32_t nb, const uint8_t *xq, float *y, int nthreads);
void or_gemv_q8_mt(const uint32_t *qw, const uint16_t *qs, uint32_t rows, uint32_t nb, const uint8_t *xq, float *y, int nthreads);
void or_gemv_q6k_mt(const uint32_t *qw, const uint16_t *qs, uint32_t rows, uint32_t nb, const uint8_t *xq, float *y, int nthreads);

#ifdef __cplusplus
}
#endif
#endif
