/* amdc_q4.h -- the C ABI of the MI355X (gfx950) quantized GEMV/GEMM path:
 * libamdc_q4.so. Plain pointers and sizes; no HIP or ROCm header needed to
 * use it (the library dlopens the HIP runtime, as the reference's host does,
 * hanw/amd.c src/hip.c:1-4, 59-99).
 *
 * It replaces, for MAT_Q4 / MAT_Q4K matrices, the reference's
 *  - load-time repack   repack_q4 / repack_q4k      (src/model.c:205, 246)
 *  - GPU dispatch       OP_QUANT, OP_GEMV_Q4, OP_GEMV_Q4K in launch_op
 *                                                    (src/hip.c:922-1026)
 *  - device kernels     ie_quant_q8, ie_gemv_q4q8, ie_gemv_q4kq8(_tr, _tr8,
 *                       _ts2), ie_gemm_q4kr          (kernels/ie_kernels.c)
 * with the same argument meaning (rows, nb = cols / 32, bias, res, T, and
 * the strides xs in bytes, ys / rs in floats) and the same Q8 activation
 * buffer: [int8 q[32 nb] | float d[nb] | u32 asum[nb]] (src/common.h:25-29).
 *
 * Device pointers (w, xq, y, bias, res, x, q) are HIP device addresses, the
 * stream a hipStream_t (NULL: the default stream). Launches are asynchronous.
 * Every function returns 0 on success, else an AMDC_E* code; amdc_last_error()
 * then says why (the reference instead prints and exit(1)s: src/common.c:6-14;
 * a host that wants that calls ie_die(amdc_last_error())).
 * Not re-entrant: one thread drives the library (as src/hip.c). The operators
 * that use the library's device workspace (the GEMMs, the split-K multi-vector
 * GEMV and its per-tile arrival counters, amdc_gemv_*_x with q8 NULL above the fused size) share it: work of
 * theirs queued on different streams, or in graphs replayed on them, must be
 * ordered (one stream, or an event between), or their results race. The same
 * holds for amdc_op_gemv_noalloc and its fixed workspace. */
#ifndef AMDC_Q4_H
#define AMDC_Q4_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { AMDC_OK = 0, AMDC_EINVAL = 1, AMDC_ENOHIP = 2, AMDC_EHIP = 3, AMDC_ENOTOPEN = 4 };

/* Matrix kinds: the reference's MAT_Q4, MAT_Q8, MAT_Q4K and MAT_Q6K
 * (src/model.h:15). */
enum { AMDC_KIND_Q4_0 = 0, AMDC_KIND_Q8_0 = 2, AMDC_KIND_Q4_K = 3, AMDC_KIND_Q6_K = 4 };

const char *amdc_last_error(void);
/* The name of the kernel the library launched last ("" before any launch):
 * for profilers and benchmarks that label their timings (no reference
 * counterpart). */
const char *amdc_last_kernel(void);

/* ---------------------------------------------------------------- load time (host only) */

/* Bytes of a repacked rows x cols matrix (cols % 32 == 0; Q4_K and Q6_K:
 * cols % 256 == 0) per row: Q4_0, Q4_K 144 * ceil(cols / 256), Q8_0 272 *
 * ceil(cols / 256) (the GGUF sizes when cols % 256 == 0), Q6_K 210 cols / 256
 * plus under 16 bytes of padding. 0 for an unknown kind or shape. */
size_t amdc_mat_bytes(int kind, uint32_t rows, uint32_t cols);

/* GGUF Q4_0 (18-byte blocks) / Q4_K (144-byte super-blocks) bytes of a
 * rows x cols matrix -> the CDNA4 layout in dst (amdc_mat_bytes bytes).
 * Replace repack_q4 (src/model.c:205-219) and repack_q4k (src/model.c:
 * 246-267); the nibble bytes are kept bit for bit, the scales are regrouped
 * (6-bit Q4_K scales and mins unpacked as ggml's get_scale_min_k4,
 * src/model.c:24-31, then repacked 8 per 6 bytes). Host memory only. */
int amdc_repack_q4(const uint8_t *gguf, uint32_t rows, uint32_t cols, uint8_t *dst);
int amdc_repack_q4k(const uint8_t *gguf, uint32_t rows, uint32_t cols, uint8_t *dst);
/* GGUF Q8_0 (34-byte blocks) / Q6_K (210-byte super-blocks) -> the CDNA4
 * layout. Replace repack_q8 (src/model.c:221-237) and repack_q6k
 * (src/model.c:269-292): the int8 weights, the Q6_K scales and d are kept bit
 * for bit; the 6-bit Q6_K weights are split into Q4_0-order nibbles and the
 * reference's high-bit words (core/ie_core.h:314-349). */
int amdc_repack_q8(const uint8_t *gguf, uint32_t rows, uint32_t cols, uint8_t *dst);
int amdc_repack_q6k(const uint8_t *gguf, uint32_t rows, uint32_t cols, uint8_t *dst);

/* ---------------------------------------------------------------- runtime */

/* Load the HIP runtime (dlopen), select device 0 and load the kernel code
 * object (NULL: amdc_kernels.hsaco next to this library). Replaces the
 * hsaco load of gpu_open (src/hip.c:568-598). Fails cleanly (AMDC_ENOHIP)
 * when there is no runtime or no device, like src/hip.c's "no GPU" path. */
int amdc_open(const char *hsaco);
void amdc_close(void);
/* Number of compute units of the device (0 before amdc_open). */
int amdc_cu_count(void);

/* Plumbing for hosts without their own allocator (tests, bench). */
int amdc_malloc(void **p, size_t n);
int amdc_free(void *p);
int amdc_memcpy_h2d(void *dst, const void *src, size_t n);
int amdc_memcpy_d2h(void *dst, const void *src, size_t n);
int amdc_memcpy_d2d(void *dst, const void *src, size_t n);
int amdc_memset(void *p, int v, size_t n);
int amdc_sync(void);
/* HIP events, for timing on a stream. */
int amdc_event_create(void **ev);
int amdc_event_destroy(void *ev);
int amdc_event_record(void *ev, void *stream);
int amdc_event_elapsed_ms(float *ms, void *start, void *stop);
/* Streams (default priority) and HIP graphs: operators launched on a stream
 * between amdc_graph_begin and amdc_graph_end are captured (kernel nodes
 * only: the operators record no memset) and replayed by amdc_graph_launch
 * with one host call. The device pointers of a graph are fixed at capture. */
int amdc_stream_create(void **stream);
int amdc_stream_destroy(void *stream);
int amdc_stream_sync(void *stream);
/* Later work on stream waits for event ev (recorded on another stream): the
 * fork/join of independent operators, also inside a graph capture. */
int amdc_stream_wait_event(void *stream, void *ev);
int amdc_graph_begin(void *stream);
/* *exec: an opaque handle (the executable graph and its template, both kept
 * until amdc_graph_destroy). */
int amdc_graph_end(void *stream, void **exec);
int amdc_graph_launch(void *exec, void *stream);
/* Waits for the device, then frees the graph (NULL: nothing). Not inside a
 * capture. */
int amdc_graph_destroy(void *exec);

/* ---------------------------------------------------------------- operators */

/* Q8 quantization of T rows of 32 nb floats: x of token t at x + t * xs
 * bytes, its Q8 buffer at q + t * qs bytes (xs, qs multiples of 16).
 * Replaces OP_QUANT / ie_quant_q8(x, q, nb, xs, qs) (src/hip.c:922-927,
 * kernels/ie_kernels.c:216-222); bitwise equal to cpu_quant_q8
 * (src/cpu.c:36-53). */
int amdc_quant_q8(const float *x, uint8_t *q, uint32_t nb, uint32_t T, uint32_t xs, uint32_t qs, void *stream);

/* y = W x for one Q8 vector (decode), then y (+ bias[r]) then (res[r] +) y.
 * Replace OP_GEMV_Q4 / ie_gemv_q4q8 and OP_GEMV_Q4K / ie_gemv_q4kq8
 * (src/hip.c:928-933, 1023-1024; kernels/ie_kernels.c:310-347, 401-406)
 * without the fused-RMSNorm tail (nw, ny, nq, eps, count). w: the repacked
 * matrix (amdc_repack_q4 / _q4k), 16-byte aligned; xq 16-byte aligned. */
int amdc_gemv_q4(const void *w, const uint8_t *xq, float *y, uint32_t rows, uint32_t nb, const float *bias, const float *res,
                 void *stream);
int amdc_gemv_q4k(const void *w, const uint8_t *xq, float *y, uint32_t rows, uint32_t nb, const float *bias, const float *res,
                  void *stream);
/* The same for Q8_0 and Q6_K matrices (amdc_repack_q8 / _q6k; Q6_K: nb %
 * 8 == 0; the matrix under 4 GiB): replace OP_GEMV_Q8 / ie_gemv_q8q8
 * (src/hip.c:1027-1089, kernels/ie_kernels.c:837) and OP_GEMV_Q6K /
 * ie_gemv_q6kq8 (src/hip.c:934-962, kernels/ie_kernels.c:675). Per block, the
 * reference's integer dot (ie_q8q8_block; the two half dots sum (q - 32) a
 * of ie_q6k_dots) and float step (src/cpu.c:168, 142). */
int amdc_gemv_q8(const void *w, const uint8_t *xq, float *y, uint32_t rows, uint32_t nb, const float *bias, const float *res,
                 void *stream);
int amdc_gemv_q6k(const void *w, const uint8_t *xq, float *y, uint32_t rows, uint32_t nb, const float *bias, const float *res,
                  void *stream);

/* The fused Q8 producers (the float op and the Q8 copy of its result, bit
 * for bit amdc_quant_q8 of that result, in one launch), as the reference's
 * OP_RMSNORM / OP_SWIGLU with a Q8 output (src/hip.c:915-921, 1266-1271;
 * kernels/ie_kernels.c:240-265 ie_rmsnorm, :2458 ie_swiglu):
 *   rmsnorm: y = x s w, s = 1 / sqrt(sum x^2 / n + eps) (src/cpu.c:276-281)
 *   swiglu:  a = a / (1 + exp(-a)) b, in place (src/cpu.c:580)
 * q may be NULL (no Q8 copy). n is a multiple of 32; T tokens at byte
 * strides xs / ys / as (floats) and qs (Q8). The float results differ from
 * the CPU's in summation order (rmsnorm) and exp rounding (swiglu) only. */
int amdc_rmsnorm_q8(const float *x, const float *w, float *y, uint32_t n, float eps, uint8_t *q, uint32_t T, uint32_t xs, uint32_t ys,
                    uint32_t qs, void *stream);
int amdc_swiglu_q8(float *a, const float *b, uint32_t n, uint8_t *q, uint32_t T, uint32_t as, uint32_t qs, void *stream);

/* The decode GEMV (T = 1, any kind) with the fused RMSNorm of its result:
 * the reference's GEMV launch with NW / NY / NQ / eps (IE_NORM_FUSE,
 * src/hip.c:928-931; the tail gemv_norm_tail, kernels/ie_kernels.c:267-283).
 * y as amdc_gemv_q4 / _q4k / _q8 / _q6k; then the GEMV's last workgroup
 * writes ny = rmsnorm(y) nw (rows floats) and, when nq is not NULL, its Q8
 * copy: the bits of amdc_rmsnorm_q8(y, nw, ny, rows, eps, nq). rows is a
 * multiple of 32, at most 8192. The workgroups count themselves on a library counter that
 * each launch leaves at 0: two of these GEMVs must not run concurrently. */
int amdc_gemv_norm(int kind, const void *w, const uint8_t *xq, float *y, uint32_t rows, uint32_t nb, const float *bias, const float *res,
                   const float *nw, float *ny, uint8_t *nq, float eps, void *stream);

/* The decode GEMV of an f32 input x (32 nb floats, 16-byte aligned): the
 * pair OP_QUANT + OP_GEMV_Q4 / OP_GEMV_Q4K (src/hip.c:922-933, 1023-1024).
 * For nb <= 128 (AMDC_GEMVX_FUSE_NB) one launch: every workgroup quantizes x
 * in its prologue, bit for bit as amdc_quant_q8, and when q8 is not NULL one
 * of them also writes the Q8 buffer there (for other GEMVs of the same
 * input). For larger nb, amdc_quant_q8 into q8 and the GEMV (two launches);
 * with q8 NULL the Q8 vector goes to the library's workspace, which grows on
 * first use (make one call before a graph capture). y is the same either way.
 * No reference counterpart as one kernel (the reference fuses the
 * quantization into the producer instead, kernels/ie_kernels.c:203-265). */
int amdc_gemv_q4_x(const void *w, const float *x, float *y, uint32_t rows, uint32_t nb, const float *bias, const float *res, uint8_t *q8,
                   void *stream);
int amdc_gemv_q4k_x(const void *w, const float *x, float *y, uint32_t rows, uint32_t nb, const float *bias, const float *res, uint8_t *q8,
                    void *stream);
/* Q8_0 / Q6_K: always amdc_quant_q8 and the GEMV (two launches). */
int amdc_gemv_q8_x(const void *w, const float *x, float *y, uint32_t rows, uint32_t nb, const float *bias, const float *res, uint8_t *q8,
                   void *stream);
int amdc_gemv_q6k_x(const void *w, const float *x, float *y, uint32_t rows, uint32_t nb, const float *bias, const float *res, uint8_t *q8,
                    void *stream);

/* y_t = W x_t for T Q8 vectors (MTP verify, any T >= 1; the weights are
 * read once per 16 vectors, on int8 MFMA, the exact integer dots of
 * ie_q4q8_block / ie_q4k_dot): x_t at xq + t * xs bytes, y_t at y + t * ys
 * floats, res_t at res + t * rs floats. A library workspace holds split-K
 * partial sums (allocated on the first call of a size: call once outside
 * graph capture before capturing). Replaces the multi-token branch of
 * OP_GEMV_Q4K (ie_gemv_q4kq8_ts2 / _tr8 / _tr, src/hip.c:1004-1020); the
 * Q4_0 form has no reference kernel (the reference runs OP_GEMV_Q4 per
 * token, src/hip.c:1583-1588). Every vector's y equals the decode GEMV of that
 * vector (amdc_gemv_q4 / _q4k / _q8) bit for bit, at every K split, as the
 * reference's multi-token kernels equal its single-token one
 * (kernels/ie_kernels.c:481-482); Q6_K's agrees within the 1e-5 bound. */
int amdc_gemv_q4_t(const void *w, const uint8_t *xq, float *y, uint32_t rows, uint32_t nb, const float *bias, const float *res,
                   uint32_t T, uint32_t xs, uint32_t ys, uint32_t rs, void *stream);
int amdc_gemv_q4k_t(const void *w, const uint8_t *xq, float *y, uint32_t rows, uint32_t nb, const float *bias, const float *res,
                    uint32_t T, uint32_t xs, uint32_t ys, uint32_t rs, void *stream);
/* Q8_0 / Q6_K over T vectors: the same int8-MFMA verify kernels (the
 * multi-token branches of OP_GEMV_Q8 and OP_GEMV_Q6K, ie_gemv_q8q8_t / _tr
 * and ie_gemv_q6kq8_tr / _tr8 / _ts2, src/hip.c:934-962, 1027-1089). */
int amdc_gemv_q8_t(const void *w, const uint8_t *xq, float *y, uint32_t rows, uint32_t nb, const float *bias, const float *res,
                   uint32_t T, uint32_t xs, uint32_t ys, uint32_t rs, void *stream);
int amdc_gemv_q6k_t(const void *w, const uint8_t *xq, float *y, uint32_t rows, uint32_t nb, const float *bias, const float *res,
                    uint32_t T, uint32_t xs, uint32_t ys, uint32_t rs, void *stream);

/* The prefill chunk GEMM for Q4_K weights (nb % 8 == 0): the arguments of
 * ie_gemm_q4kr (kernels/ie_kernels.c:1289, src/hip.c:998-1001). The integer
 * sums of the sub-blocks are exact: by default on the f16 MFMA with the 6-bit
 * scale folded into the weights (q sc <= 945 and the int8 activations are f16
 * integers; every partial sum is an integer below 2^24), or on the int8 MFMA
 * (tuning); f32 outputs within 1e-5 of cpu_gemv_q4k per token row. Uses a
 * device workspace that the library allocates on the first call of a size
 * (call once outside graph capture before capturing). */
int amdc_gemm_q4k(const void *w, const uint8_t *xq, float *y, uint32_t rows, uint32_t nb, const float *bias, const float *res,
                  uint32_t T, uint32_t xs, uint32_t ys, uint32_t rs, void *stream);
/* The same for Q8_0 and Q6_K matrices: replace ie_gemm_q8r / ie_gemm_q8
 * (kernels/ie_kernels.c:1018, 1166; src/hip.c:1040-1056) and ie_gemm_q6kr
 * (kernels/ie_kernels.c:2015; src/hip.c:938-944). Q8_0: the integer block
 * sums exact on the f16 MFMA (int8 weights are f16 integers), then
 * (d_w d_a) sum per block as src/cpu.c:168. Q6_K: (q - 32) sc split into two
 * exact f16 operands (16 (sc >> 4) and sc & 15 parts), so that the sums
 * (q - 32) sc a of a sub-block are exact, then d d_a per sub-block. f32 outputs
 * within 1e-5 of cpu_gemv_q8 / cpu_gemv_q6k per token row. The same
 * workspace as amdc_gemm_q4k. */
int amdc_gemm_q8(const void *w, const uint8_t *xq, float *y, uint32_t rows, uint32_t nb, const float *bias, const float *res,
                 uint32_t T, uint32_t xs, uint32_t ys, uint32_t rs, void *stream);
/* Q4_0 (any nb): the block's q - 8 as f16 on the f16 MFMA, then (d_w d_a) sum
 * per block as src/cpu.c:81. No reference counterpart (the reference runs
 * OP_GEMV_Q4 per token, src/hip.c:1583-1588); y within 1e-5 of cpu_gemv_q4
 * per token row. */
int amdc_gemm_q4(const void *w, const uint8_t *xq, float *y, uint32_t rows, uint32_t nb, const float *bias, const float *res,
                 uint32_t T, uint32_t xs, uint32_t ys, uint32_t rs, void *stream);
int amdc_gemm_q6k(const void *w, const uint8_t *xq, float *y, uint32_t rows, uint32_t nb, const float *bias, const float *res,
                  uint32_t T, uint32_t xs, uint32_t ys, uint32_t rs, void *stream);

/* The dispatch of launch_op for OP_GEMV_Q4 / OP_GEMV_Q8 / OP_GEMV_Q4K /
 * OP_GEMV_Q6K over T tokens (src/hip.c:928-1089): T == 1 -> the decode GEMV;
 * T >= IE_GEMM_MIN (env) -> the GEMM (Q4_0 included, where the reference
 * runs one GEMV per token); else the multi-vector GEMV. Without IE_GEMM_MIN
 * (the reference's default is 17) the MI355X rule: the GEMM for T >= 33, and
 * for T >= 20 on matrices of at most 2^24 weights. kind: any AMDC_KIND_*. */
int amdc_op_gemv(int kind, const void *w, const uint8_t *xq, float *y, uint32_t rows, uint32_t nb, const float *bias,
                 const float *res, uint32_t T, uint32_t xs, uint32_t ys, uint32_t rs, void *stream);

/* amdc_op_gemv without any device allocation, for callers that cannot allocate (code under
 * HIP graph capture on a workspace size not seen before, tight serving loops, hosts that
 * forbid hipMalloc). No reference counterpart. The same kernels and launch choices as
 * amdc_op_gemv, so the same bits; the workspace (split-K partial sums, the GEMM's prepared
 * activations) is a fixed device array of AMDC_SCRATCH_BYTES in the code object, held by the
 * device from amdc_open until amdc_close. A call whose workspace would exceed it fails with
 * AMDC_EINVAL before any launch (e.g. T = 256 prefill chunks fit up to about 17408 x 5120
 * and 5120 x 17408 matrices). All calls share the one array: calls that overlap on the
 * device (other streams, graphs replayed concurrently) race; order them. Its contents are
 * whatever the last call left; no kernel needs it cleared. */
#define AMDC_SCRATCH_BYTES ((size_t)64 << 20)
int amdc_op_gemv_noalloc(int kind, const void *w, const uint8_t *xq, float *y, uint32_t rows, uint32_t nb, const float *bias,
                         const float *res, uint32_t T, uint32_t xs, uint32_t ys, uint32_t rs, void *stream);

/* Parity probe: out[r * nb + b] = the int32 dot product of block b of row r
 * with Q8 block b, as the GEMV kernels compute it: sum (q - 8) a for Q4_0
 * (core/ie_core.h:161 ie_q4q8_block), sum q a for Q4_K (ie_q4k_dot, :281)
 * and Q8_0 (ie_q8q8_block, :222). Q6_K: two per block, out[(r * nb + b) * 2
 * + h] = sum (q - 32) a over half h (ie_q6k_dots, :384). */
int amdc_block_dots(int kind, const void *w, const uint8_t *xq, int32_t *out, uint32_t rows, uint32_t nb, void *stream);

/* Tuning knobs (0 = automatic): lanes per row of the GEMV (4..64, power of
 * two); the decode kernel (0: the pipelined one; 1 or 2: the multi-vector
 * kernel with 1 or 2 super-groups of loads per step); workgroups of a GEMV
 * launch; the GEMM kernel (1, 2: int8 MFMA with 64 or 128 tokens per
 * workgroup; 3, 4, 5: f16 MFMA, rows x tokens 64x128, 64x64, 128x128 (Q4_K));
 * the GEMM's K split (1..16); the decode kernel's form when gemv_unroll is 0
 * (1: the persistent pipelined form, 2: the buffer-load form that keeps the
 * next super-group in flight, 3: the single-shot form, one row group per
 * workgroup with all its loads issued at once, 4: the K-split form, ranges of
 * gemv_lanes super-groups (8 when 0) over the workgroups, the ranges' sums
 * added by the last to arrive, Q4_0 / Q4_K; 0: form 3 up to 256
 * super-groups per row, else form 2). Also read once from the environment: AMDC_GEMV_L,
 * AMDC_GEMV_U, AMDC_GEMV_WG, AMDC_GEMM_KERNEL, AMDC_GEMM_KSPLIT,
 * AMDC_GEMV_FORM. */
int amdc_set_tuning(int gemv_lanes, int gemv_unroll, int gemv_wgs, int gemm_kernel, int gemm_ksplit, int gemv_form);

/* A GEMV chain: a list of quantize, decode-GEMV and Q8-producer operations run by ONE
 * persistent launch, a grid barrier after every operation marked sync (the
 * reference's megakernel command list, kernels/ie_mk.c with mk_put in
 * src/hip.c:530, and its GEMV chain probe ie_mk_gemv_chain,
 * kernels/ie_kernels.c:464-478). While a workgroup waits at a barrier the
 * weight loads of the next GEMV are already in flight. Results equal the
 * separate launches bit for bit (amdc_quant_q8; amdc_gemv_q4 / _q4k with
 * the same lane split).
 *   AMDC_CHAIN_QUANT: x (32 nb floats) -> q (Q8 buffer, 40 nb bytes)
 *   AMDC_CHAIN_GEMV:  kind (any), w (rows x nb), xq (Q8) -> y (rows
 *                     floats), optional bias / res (rows floats) as
 *                     amdc_gemv_q4; Q8_0 / Q6_K as amdc_gemv_q8 / _q6k
 *                     (bit-equal to them)
 *   AMDC_CHAIN_GEMV_X: Q4_0 / Q4_K on x (32 nb floats): every workgroup
 *                     quantizes x into its LDS (as amdc_gemv_q4_x, no Q8
 *                     buffer, no barrier between quantization and GEMV)
 *   AMDC_CHAIN_RMSNORM_Q8: y = RMSNorm of x (32 nb floats) with the weights
 *                     w (32 nb floats) and eps, its Q8 copy -> q when q is
 *                     not NULL (amdc_rmsnorm_q8 of one token, bit-equal)
 *   AMDC_CHAIN_SWIGLU_Q8: y = silu(y) x in place (32 nb floats each), its
 *                     Q8 copy -> q when q is not NULL (amdc_swiglu_q8 of one
 *                     token with a = y, b = x, bit-equal)
 * Lists with the producer operations run in the persistent form.
 * Operations between two syncs run concurrently: when one writes bytes that
 * another reads or writes, the later one must come after a sync (the check
 * compares the byte ranges of every operand). All workgroups must be resident at
 * once: the grid is what the device holds (at most 2 per CU, 1 per CU for the
 * streaming form); nothing else
 * should run on the device meanwhile. A barrier that waits longer than 200 ms
 * aborts the launch (every workgroup leaves); amdc_chain_check reports it. */
enum { AMDC_CHAIN_QUANT = 0, AMDC_CHAIN_GEMV = 1, AMDC_CHAIN_GEMV_X = 2, AMDC_CHAIN_RMSNORM_Q8 = 3, AMDC_CHAIN_SWIGLU_Q8 = 4 };
typedef struct {
  int type, kind, sync;
  uint32_t rows, nb;
  const void *w;
  const float *x;
  uint8_t *q;
  const uint8_t *xq;
  float *y;
  const float *bias, *res;
  float eps; /* AMDC_CHAIN_RMSNORM_Q8 */
} amdc_chain_op;
/* Validate the list, upload it and the barrier counters (allocates: call
 * before any graph capture); *chain receives the handle. */
int amdc_chain_create(const amdc_chain_op *ops, uint32_t n, void **chain);
/* The same with the kernel chosen (no reference counterpart: the reference's
 * megakernel has one form):
 *   AMDC_CHAIN_PERSISTENT: 2 workgroups of 256 threads per CU, any kinds;
 *   AMDC_CHAIN_STREAMING: one workgroup of 768 threads per CU, every GEMV of
 *     the list Q4_0 or every one Q4_K (else AMDC_EINVAL); work is dealt per
 *     wave, each wave loads the weights of its next two items while it
 *     computes, across operations and barriers (a wave waiting at a barrier
 *     has the next operation's weights in flight), the barriers are split
 *     (arrive when done, wait before staging the next vector), and an f32
 *     input is quantized once per CU;
 *   AMDC_CHAIN_AUTO (amdc_chain_create): the streaming form where it applies.
 * Both give the same bits as the separate launches. */
enum { AMDC_CHAIN_AUTO = 0, AMDC_CHAIN_PERSISTENT = 1, AMDC_CHAIN_STREAMING = 2 };
int amdc_chain_create_form(const amdc_chain_op *ops, uint32_t n, int form, void **chain);
/* The timeline of the streaming form (the reference's megakernel profiler,
 * IE_MK_TRACE and IE_MK_PROF, kernels/ie_mk.c:16-19): with buf (device
 * memory, amdc_chain_trace_words(chain) words; NULL: off) every later launch
 * records, per workgroup p, at buf + p (2 + 4 n + 64), the 100 MHz clock at:
 * its start; the first operation's vector staged; for each operation k
 * (words 2 + 4 k ..) its results in the LDS, their stores complete, the grid
 * barrier passed, the next vector staged; then (words 2 + 4 n ..) each of
 * the first 64 items of its first compute wave computed. */
int amdc_chain_trace(void *chain, uint64_t *buf);
uint32_t amdc_chain_trace_words(void *chain);
/* One launch of the whole list on stream (no allocation: can be captured). */
int amdc_chain_launch(void *chain, void *stream);
/* Synchronizes the device; AMDC_EHIP if a launch of this chain aborted at a
 * barrier (the counters are then reset). */
int amdc_chain_check(void *chain);
int amdc_chain_destroy(void *chain);
/* The recorder (the reference's mk_put / mk_flush, src/hip.c:475-567, which
 * append the kernels of launch_op to the megakernel's command list instead of
 * launching them): after amdc_chain_record_begin(stream), these calls on that
 * stream launch nothing and append chain operations: amdc_quant_q8,
 * amdc_rmsnorm_q8, amdc_swiglu_q8 (T = 1), amdc_gemv_q4 / _q4k / _q8 / _q6k,
 * amdc_op_gemv with T = 1, and amdc_gemv_*_x (with q8: a quantize into q8
 * and the GEMV on it; without, Q4_0 / Q4_K only: AMDC_CHAIN_GEMV_X). Any
 * other launch on that stream fails (and so does the recording). A grid
 * barrier goes between two operations exactly where the later one shares
 * bytes that one of them writes with an operation since the last barrier.
 * amdc_chain_record_end(stream, form, &chain) ends the recording and creates
 * the chain (amdc_chain_create_form: allocates, not inside a graph capture);
 * launching it computes what the calls would have, bit for bit. One recording
 * at a time. */
int amdc_chain_record_begin(void *stream);
int amdc_chain_record_end(void *stream, int form, void **chain);

/* Bandwidth yardsticks (no reference counterpart): stream nbytes (a multiple
 * of 16) through a plain read kernel (one u32 per workgroup may be written to
 * scratch) or a copy kernel, grid workgroups of 256 threads. They give the
 * achievable HBM rate and calibrate the FETCH_SIZE / WRITE_SIZE counters. */
int amdc_probe_read(const void *src, size_t nbytes, void *scratch, uint32_t grid, void *stream);
int amdc_probe_copy(void *dst, const void *src, size_t nbytes, uint32_t grid, void *stream);

#ifdef __cplusplus
}
#endif
#endif
