// amdc_kernels.hip -- the HIP kernels of the quantized GEMV/GEMM path for
// MI355X (gfx950, CDNA4, wave64). Built into a code object
// (amdc_kernels.hsaco) that the C host (amdc_host.c) loads with
// hipModuleLoad and launches by name, as the reference's host loads its
// kernels (hanw/amd.c src/hip.c:102-107, 568-598).
//
// Kernels (grid x = workgroups, 256 threads each):
//   amdc_quant_q8      Q8 activation quantization (src/cpu.c:36-53)
//   amdc_rmsnorm_q8, amdc_swiglu_q8
//                      the Q8 producers (the float op and its Q8 copy)
//   amdc_gemv_{q4_0,q4_k}_p1, _x1, {q4_0,q4_k,q8_0,q6_k}_p2
//                      the decode GEMV (T = 1): short rows (_p1; _x1 with the
//                      quantization fused), long rows and the Q8_0 / Q6_K kinds
//                      (_p2) (ie_gemv_q4q8, ie_gemv_q4kq8, ie_gemv_q8q8,
//                      ie_gemv_q6kq8)
//   amdc_gemv_{q4_0,q4_k,q8_0,q6_k}_v8, amdc_gemv_{q4_0,q4_k,q8_0,q6_k}_v16,
//   amdc_gemm_reduce   the verify GEMV, T <= 8 (_v8) or 16 (_v16) vectors on
//                      int8 MFMA, weights staged through LDS, K split over
//                      workgroups over aligned ranges of tiles and reduced by a
//                      pairwise tree over the ranges
//                      (ie_gemv_q4kq8_tr8 / _tr / _ts2, ie_gemv_q6kq8_tr8, ...)
//   amdc_q8_prep, amdc_gemmh_m64_n{64,128}, amdc_gemmh_{q4_0,q8_0,q6_k}_m64_n{64,128}
//                      the prefill chunk GEMM on the f16 MFMA with exact
//                      integer block sums (ie_gemm_q4kr, ie_gemm_q8r, ie_gemm_q6kr)
//   amdc_gemm_q4_k_n{64,128}
//                      the same on int8 MFMA (a tuning alternative)
//   amdc_chain         a list of quantize / decode-GEMV / RMSNorm+Q8 / SwiGLU+Q8
//                      operations in one persistent launch (the megakernel's
//                      command list for these operations)
//   amdc_dots_{q4_0,q4_k,q8_0,q6_k}
//                      the per-block int32 dot products (parity check)
//   amdc_probe_read, amdc_probe_copy
//                      plain streams (bandwidth and counter calibration)
// The weight layout is amdc_layout.h. The Q8 buffer is the reference's:
// [int8 q[32 nb] | f32 d[nb] | u32 asum[nb]] (src/common.h:25-29).
#include <hip/hip_runtime.h>

#include <type_traits>

#include "amdc_layout.h"

// The fixed workspace of amdc_op_gemv_noalloc (AMDC_SCRATCH_BYTES): split-K partial sums and
// the GEMM's prepared activations, for callers that cannot allocate device memory. Every
// device that loads this code object holds one copy until the module is unloaded. No kernel
// names it: the host looks its address up once (hipModuleGetGlobal, with the device current)
// and passes that address as the workspace argument, as it passes an allocated workspace.
// Not static, so that the code object exports the symbol for that lookup.
__device__ __align__(256) unsigned char scratch[AMDC_SCRATCH_BYTES];

typedef uint32_t u32;
typedef uint64_t u64;
typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef u32 u32x4 __attribute__((ext_vector_type(4)));
typedef u32 u32x2 __attribute__((ext_vector_type(2)));

// A buffer resource over n bytes from p (raw, no stride): loads through it take
// a 32-bit lane offset and a 32-bit scalar offset.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void *p, u32 n) { return __builtin_amdgcn_make_buffer_rsrc((void *)p, (short)0, (int)n, 0x00020000); }

#define NT 256u
#define SCH 3u  // Q8 blocks per thread whose staging loads are in flight together (decode GEMV)
#define QCH 4u // passes of 32 blocks whose activation loads are in flight together (fused quantization: 128 blocks)

// ------------------------------------------------------------------ helpers

__device__ __forceinline__ float h2f(u32 h) { return (float)__builtin_bit_cast(_Float16, (unsigned short)(h & 0xFFFFu)); }

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// The sum of v over aligned segments of L lanes (L = 4, 8, 16, 32 or 64);
// every lane of a segment gets the sum. DPP inside rows of 16 lanes
// (quad_perm xor 1, xor 2, row_half_mirror, row_mirror), then ds_swizzle
// (xor 16) and ds_bpermute (xor 32).
__device__ __forceinline__ float seg_sum(float v, u32 L) {
  v += dpp<0xB1>(v); // quad_perm [1,0,3,2]
  v += dpp<0x4E>(v); // quad_perm [2,3,0,1]
  if (L >= 8u) v += dpp<0x141>(v);
  if (L >= 16u) v += dpp<0x140>(v);
  if (L >= 32u) v += __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x401F));
  if (L >= 64u) v += __shfl_xor(v, 32);
  return v;
}

// The summation order of a row (every GEMV form, decode and verify, follows
// it, so that their results are equal bit for bit): the leaf of super-group g
// is its 8 block terms added in block order from +0.0; the row sum is the
// pairwise tree over the leaves g = 0, 1, ..., ng - 1 (adjacent pairs first),
// padded with +0.0 leaves to a power of two. A leaf is never -0.0 (every
// chain starts at +0.0), so x + 0.0 = x and the padding width does not
// matter. seg_sum over L lanes holding leaves l (lane l) is that tree.
//
// A lane that holds the super-groups g = l + L i of its row (items i = 0 ..
// ni - 1, L lanes per row) gives each item's leaf to seg_sum and then adds
// the sums of the items in a pairwise tree over i: ItemTree, ni <= 4.
struct ItemTree {
  float a = 0.0f, b = 0.0f;
  __device__ __forceinline__ void add(float v, u32 i) {
    if (i == 0u) a = v;
    else if (i == 1u) a = a + v;
    else if (i == 2u) b = v;
    else b = b + v;
  }
  __device__ __forceinline__ float sum(u32 ni) const { return ni > 2u ? a + b : a; }
};

__device__ __forceinline__ int sdot4(u32 a, u32 b, int c) { return __builtin_amdgcn_sdot4((int)a, (int)b, c, false); }

// Sum over j < 32 of nibble_j * a_j: the 16 nibble bytes w (byte j: weight j
// low, weight j + 16 high) against the 32 activation bytes alo (0..15), ahi
// (16..31). The nibble bytes are 0..15, so the signed dot4 gives the same
// integer as the reference's unsigned-by-signed one (core/ie_core.h:113-139,
// 281-286).
__device__ __forceinline__ int nib_dot(u32x4 w, u32x4 alo, u32x4 ahi) {
  const u32 M = 0x0F0F0F0Fu;
  int s = 0;
  s = sdot4(w.x & M, alo.x, s);
  s = sdot4((w.x >> 4) & M, ahi.x, s);
  s = sdot4(w.y & M, alo.y, s);
  s = sdot4((w.y >> 4) & M, ahi.y, s);
  s = sdot4(w.z & M, alo.z, s);
  s = sdot4((w.z >> 4) & M, ahi.z, s);
  s = sdot4(w.w & M, alo.w, s);
  s = sdot4((w.w >> 4) & M, ahi.w, s);
  return s;
}

// Sum over j < 32 of w_j a_j for the 32 int8 weights of a Q8_0 block (w0:
// bytes 0..15, w1: 16..31) and activations alo, ahi (ie_q8q8_block,
// core/ie_core.h:222-233).
__device__ __forceinline__ int q8_dot(u32x4 w0, u32x4 w1, u32x4 alo, u32x4 ahi) {
  int s = sdot4(w0.x, alo.x, 0);
  s = sdot4(w0.y, alo.y, s), s = sdot4(w0.z, alo.z, s), s = sdot4(w0.w, alo.w, s);
  s = sdot4(w1.x, ahi.x, s), s = sdot4(w1.y, ahi.y, s), s = sdot4(w1.z, ahi.z, s), s = sdot4(w1.w, ahi.w, s);
  return s;
}

// Sum over each half h of a Q6_K sub-block of q a (q = 0..63: the nibble of
// word nw plus the high bits of word hh << 4; weight 16h + 4i + e at bits
// 8e + 2i of hh, so word i of the half takes (hh >> 2i) & 0x03030303, here
// as a shift and a mask of 0x30303030). The q - 32 of the reference
// (ie_q6k_dots, core/ie_core.h:355-389) is sum q a - 32 (sum a), subtracted
// by the caller.
__device__ __forceinline__ void q6k_dots(u32x4 nw, u32 h0, u32 h1, u32x4 alo, u32x4 ahi, int &d0, int &d1) {
  const u32 M = 0x0F0F0F0Fu, M2 = 0x30303030u;
  d0 = sdot4((nw.x & M) | ((h0 << 4) & M2), alo.x, 0);
  d0 = sdot4((nw.y & M) | ((h0 << 2) & M2), alo.y, d0);
  d0 = sdot4((nw.z & M) | (h0 & M2), alo.z, d0);
  d0 = sdot4((nw.w & M) | ((h0 >> 2) & M2), alo.w, d0);
  d1 = sdot4(((nw.x >> 4) & M) | ((h1 << 4) & M2), ahi.x, 0);
  d1 = sdot4(((nw.y >> 4) & M) | ((h1 << 2) & M2), ahi.y, d1);
  d1 = sdot4(((nw.z >> 4) & M) | (h1 & M2), ahi.z, d1);
  d1 = sdot4(((nw.w >> 4) & M) | ((h1 >> 2) & M2), ahi.w, d1);
}

// The sum of the 16 int8 activations of a word quad.
__device__ __forceinline__ int hsum16(u32x4 a) {
  const u32 one = 0x01010101u;
  return sdot4(a.w, one, sdot4(a.z, one, sdot4(a.y, one, sdot4(a.x, one, 0))));
}

// The 6-bit scale and min of sub-block k of a Q4_K header (amdc_layout.h).
__device__ __forceinline__ u32 q4k_sc(u32x4 h, u32 k) { return (u32)((((u64)h.z << 32) | h.y) >> (6u * k)) & 63u; }
__device__ __forceinline__ u32 q4k_mn(u32x4 h, u32 k) { return (u32)((((u64)h.w << 32) | h.z) >> (16u + 6u * k)) & 63u; }
__device__ __forceinline__ u32 hword(u32x4 h, u32 i) { return i == 0 ? h.x : i == 1 ? h.y : i == 2 ? h.z : h.w; }

// q = roundf(x / d) for the 4 values of a lane (IEEE division, rounded half
// away from zero; 0 for d = 0). A division-free form (the reciprocal, and the
// division only for quotients within 2^-15 of a half-integer) measured slower
// on MI355X (the c1 step 49.8 against 48.6 us).
__device__ __forceinline__ void q8_round4(const v4f &x, float d, int (&qi)[4]) {
#pragma unroll
  for (int m = 0; m < 4; m++) qi[m] = d != 0.0f ? (int)__builtin_roundf(x[m] / d) : 0;
}

// ------------------------------------------------------------------ Q8 quantization

// One 32-lane half of a wave per block of 32: amax by xor shuffles inside
// the half, d = amax / 127 (IEEE division), q = roundf(x / d) (half away from
// zero), 0 when d == 0; asum = the u32 sum of the 32 q. Grid: (ceil(nb / 8),
// T); x and q of token t start t * xs and t * qs bytes in.
extern "C" __global__ __launch_bounds__(256) void amdc_quant_q8(const float *__restrict__ x, uint8_t *__restrict__ q, u32 nb, u32 xs,
                                                                u32 qs) {
  x = (const float *)((const uint8_t *)x + (u64)blockIdx.y * xs);
  q += (u64)blockIdx.y * qs;
  const u32 b = blockIdx.x * 8u + (threadIdx.x >> 5), j = threadIdx.x & 31u;
  if (b >= nb) return; // whole 32-lane halves leave together
  const float v = x[32u * b + j];
  float a = __builtin_fabsf(v);
#pragma unroll
  for (u32 o = 1; o < 32u; o <<= 1) a = __builtin_fmaxf(a, __shfl_xor(a, (int)o));
  const float d = a / 127.0f;
  const int qi = d != 0.0f ? (int)__builtin_roundf(v / d) : 0;
  ((int8_t *)q)[32u * b + j] = (int8_t)qi;
  u32 s = (u32)qi;
#pragma unroll
  for (u32 o = 1; o < 32u; o <<= 1) s += (u32)__shfl_xor((int)s, (int)o);
  if (j == 0) {
    ((float *)(q + 32u * nb))[b] = d;
    ((u32 *)(q + 36u * nb))[b] = s;
  }
}

// The Q8 producers of a decode step, fused as the reference fuses them
// (kernels/ie_kernels.c:240-265 ie_rmsnorm, :2458 ie_swiglu): the float result
// and its Q8 copy (the arithmetic of amdc_quant_q8 on that result) in one
// launch. Grid (ceil(n / 256), T); token t at byte offsets t xs, t ys, t qs.

#define CPOL_SC1 16 // cache policy of agent-coherent buffer accesses (gfx94x / gfx950 SC1)

// half a wave quantizes the block of 32 values v (one per lane) into q; COH: agent-coherent stores
// (the chain kernel's operations, read by other workgroups of the launch)
template <bool COH = false>
__device__ __forceinline__ void quant_half(float v, u32 b, uint8_t *__restrict__ q, u32 nb) {
  const u32 j = threadIdx.x & 31u;
  float a = __builtin_fabsf(v);
#pragma unroll
  for (u32 o = 1; o < 32u; o <<= 1) a = __builtin_fmaxf(a, __shfl_xor(a, (int)o));
  const float d = a / 127.0f;
  const int qi = d != 0.0f ? (int)__builtin_roundf(v / d) : 0;
  u32 s = (u32)qi;
#pragma unroll
  for (u32 o = 1; o < 32u; o <<= 1) s += (u32)__shfl_xor((int)s, (int)o);
  if constexpr (COH) {
    const __amdgpu_buffer_rsrc_t rq = rsrc(q, 40u * nb);
    __builtin_amdgcn_raw_buffer_store_b8((uint8_t)qi, rq, 32u * b + j, 0, CPOL_SC1);
    if (j == 0u) {
      __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(u32, d), rq, 32u * nb + 4u * b, 0, CPOL_SC1);
      __builtin_amdgcn_raw_buffer_store_b32(s, rq, 36u * nb + 4u * b, 0, CPOL_SC1);
    }
  } else {
    ((int8_t *)q)[32u * b + j] = (int8_t)qi;
    if (j == 0u) {
      ((float *)(q + 32u * nb))[b] = d;
      ((u32 *)(q + 36u * nb))[b] = s;
    }
  }
}

// quant_half of N blocks at once (block b[k] of the 32 values v[k], one per lane; skipped where
// on[k] is false, uniform over the half-wave): the same values per block, the N independent
// reductions interleaved instead of one after the other
template <u32 N>
__device__ __forceinline__ void quant_halves(const float (&v)[N], const u32 (&b)[N], const bool (&on)[N], uint8_t *__restrict__ q, u32 nb) {
  const u32 j = threadIdx.x & 31u;
  float a[N];
#pragma unroll
  for (u32 k = 0; k < N; k++) a[k] = __builtin_fabsf(v[k]);
  // max and the integer sum are exact in any order: DPP inside rows of 16 and a swizzle across the
  // two rows of the half (as seg_sum) give the values quant_half's xor shuffles give
#pragma unroll
  for (u32 k = 0; k < N; k++) a[k] = __builtin_fmaxf(a[k], dpp<0xB1>(a[k]));
#pragma unroll
  for (u32 k = 0; k < N; k++) a[k] = __builtin_fmaxf(a[k], dpp<0x4E>(a[k]));
#pragma unroll
  for (u32 k = 0; k < N; k++) a[k] = __builtin_fmaxf(a[k], dpp<0x141>(a[k]));
#pragma unroll
  for (u32 k = 0; k < N; k++) a[k] = __builtin_fmaxf(a[k], dpp<0x140>(a[k]));
#pragma unroll
  for (u32 k = 0; k < N; k++) a[k] = __builtin_fmaxf(a[k], __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, a[k]), 0x401F)));
  int qi[N];
  u32 sm[N];
  float d[N];
#pragma unroll
  for (u32 k = 0; k < N; k++) {
    d[k] = a[k] / 127.0f;
    qi[k] = d[k] != 0.0f ? (int)__builtin_roundf(v[k] / d[k]) : 0;
    sm[k] = (u32)qi[k];
  }
#pragma unroll
  for (u32 k = 0; k < N; k++) sm[k] += (u32)__builtin_amdgcn_update_dpp(0, (int)sm[k], 0xB1, 0xF, 0xF, false);
#pragma unroll
  for (u32 k = 0; k < N; k++) sm[k] += (u32)__builtin_amdgcn_update_dpp(0, (int)sm[k], 0x4E, 0xF, 0xF, false);
#pragma unroll
  for (u32 k = 0; k < N; k++) sm[k] += (u32)__builtin_amdgcn_update_dpp(0, (int)sm[k], 0x141, 0xF, 0xF, false);
#pragma unroll
  for (u32 k = 0; k < N; k++) sm[k] += (u32)__builtin_amdgcn_update_dpp(0, (int)sm[k], 0x140, 0xF, 0xF, false);
#pragma unroll
  for (u32 k = 0; k < N; k++) sm[k] += (u32)__builtin_amdgcn_ds_swizzle((int)sm[k], 0x401F);
#pragma unroll
  for (u32 k = 0; k < N; k++) {
    if (!on[k]) continue;
    ((int8_t *)q)[32u * b[k] + j] = (int8_t)qi[k];
    if (j == 0u) {
      ((float *)(q + 32u * nb))[b[k]] = d[k];
      ((u32 *)(q + 36u * nb))[b[k]] = sm[k];
    }
  }
}

// a float of x[i]: a plain load, or (COH) an agent-coherent one through the resource r
template <bool COH>
__device__ __forceinline__ float ldf(const float *__restrict__ x, __amdgpu_buffer_rsrc_t r, u32 i) {
  if constexpr (COH) return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, 4u * i, 0, CPOL_SC1));
  else return x[i];
}

// The RMS scale s = 1 / sqrt(sum x^2 / n + eps) of n floats by the 256 threads of a workgroup: each
// thread adds the squares of its elements tid, tid + 256, ... in that order (NL loads in flight, which
// does not change the order), then the wave and workgroup reductions. The same code, so the same bits
// of s, in amdc_rmsnorm_q8 (NL = 8) and in the chain's RMSNorm operation (NL = 2: the chain kernel keeps
// the next GEMV's weight loads in registers meanwhile).
__device__ __forceinline__ float rms_reduce(float ss, u32 n, float eps, float *s_ss);
template <bool COH, u32 NL>
__device__ __forceinline__ float rms_scale(const float *__restrict__ x, u32 n, float eps, float *s_ss) {
  const __amdgpu_buffer_rsrc_t rx = rsrc(x, 4u * n);
  const u32 tid = threadIdx.x;
  float ss = 0.0f;
  u32 i0 = tid;
  for (; i0 + (NL - 1u) * NT < n; i0 += NL * NT) {
    float v[NL];
#pragma unroll
    for (u32 k = 0; k < NL; k++) v[k] = ldf<COH>(x, rx, i0 + k * NT);
#pragma unroll
    for (u32 k = 0; k < NL; k++) ss += v[k] * v[k];
  }
  for (; i0 < n; i0 += NT) {
    const float v = ldf<COH>(x, rx, i0);
    ss += v * v;
  }
  return rms_reduce(ss, n, eps, s_ss);
}

// s from each thread's sum of squares: the wave and workgroup reductions of rms_scale
__device__ __forceinline__ float rms_reduce(float ss, u32 n, float eps, float *s_ss) {
  const u32 tid = threadIdx.x;
  ss += dpp<0xB1>(ss);
  ss += dpp<0x4E>(ss);
  ss += dpp<0x141>(ss);
  ss += dpp<0x140>(ss);
  ss += __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, ss), 0x401F));
  ss += __shfl_xor(ss, 32);
  if ((tid & 63u) == 0u) s_ss[tid >> 6] = ss;
  __syncthreads();
  ss = (s_ss[0] + s_ss[1]) + (s_ss[2] + s_ss[3]);
  __syncthreads(); // s_ss is free again
  return 1.0f / __builtin_sqrtf(ss / (float)n + eps);
}

// SwiGLU of one element, src/cpu.c:580
__device__ __forceinline__ float swiglu1(float g, float b) { return g / (1.0f + __builtin_expf(-g)) * b; }

// y = x s w, s = 1 / sqrt(sum x^2 / n + eps) (src/cpu.c:276-281), and its Q8
// copy when q is not NULL. Every workgroup computes the whole sum of squares
// with the same code (so the same s), 8 loads in flight per thread, then
// normalizes its 8 blocks. n is a multiple of 32.
extern "C" __global__ __launch_bounds__(256) void amdc_rmsnorm_q8(const float *__restrict__ x, const float *__restrict__ w, float *__restrict__ y,
                                                                 u32 n, float eps, uint8_t *__restrict__ q, u32 xs, u32 ys, u32 qs) {
  __shared__ float s_ss[4];
  x = (const float *)((const uint8_t *)x + (u64)blockIdx.y * xs);
  y = (float *)((uint8_t *)y + (u64)blockIdx.y * ys);
  if (q) q += (u64)blockIdx.y * qs;
  const u32 tid = threadIdx.x;
  const float s = rms_scale<false, 8u>(x, n, eps, s_ss);
  const u32 nb = n >> 5, b = blockIdx.x * 8u + (tid >> 5);
  if (b >= nb) return; // whole 32-lane halves leave together
  const u32 i = 32u * b + (tid & 31u);
  const float v = x[i] * s * w[i];
  y[i] = v;
  if (q) quant_half(v, b, q, nb);
}

// a = a / (1 + exp(-a)) b in place (src/cpu.c:580), and its Q8 copy when q
// is not NULL. n is a multiple of 32.
extern "C" __global__ __launch_bounds__(256) void amdc_swiglu_q8(float *__restrict__ a, const float *__restrict__ b, u32 n,
                                                                uint8_t *__restrict__ q, u32 as, u32 qs) {
  a = (float *)((uint8_t *)a + (u64)blockIdx.y * as);
  b = (const float *)((const uint8_t *)b + (u64)blockIdx.y * as);
  if (q) q += (u64)blockIdx.y * qs;
  const u32 i = blockIdx.x * NT + threadIdx.x;
  if (i >= n) return; // whole 32-lane halves leave together
  const float v = swiglu1(a[i], b[i]);
  a[i] = v;
  if (q) quant_half(v, i >> 5, q, n >> 5);
}

// ------------------------------------------------------------------ GEMV

// The decode GEMV: y[r] = sum over blocks of W[r] . x, then the reference's
// epilogue (src/cpu.c:513-520): y (+ bias[r]) then (res[r] +) y.
//
// Work split: a wave holds 64 / L rows, L lanes per row (L = 4..64, a power
// of two); lane l of a row owns the super-groups g = l + L i (its items) and
// for each reads its 16-byte header and its 8 nibble blocks (9 loads of 128
// bits). A workgroup (4 waves) takes 4 * 64 / L rows per pass and loops over
// row groups (blockIdx.x, + gridDim.x). The row sum follows the super-group
// tree order (ItemTree above).
//
// The Q8 vector sits in LDS, permuted as the weights (block 8g + k at
// k ng + g), so that the lanes of a row read consecutive 16-byte words: q low
// half, q high half, d, asum (320 ng bytes).
//
// Per block: Q4_0: dot = sum (q - 8) a = nib_dot - 8 asum (u32 wrap as the
//   reference), acc += (d_w d_a) dot;
// Q4_K: dq = nib_dot; acc = fma(-(dmin mn), d_a asum, fma((d sc) dq, d_a,
//   acc)), the operations of src/cpu.c:111-112.
//
// First form (amdc_gemv_*_p1, _x1), software-pipelined: each lane walks its
// (row group, super-group) items in order and issues the 9 loads of the next
// item before it computes the current one, across row groups too; the first
// item's loads are issued before the activations are staged.
struct Item {
  u32x4 h, n[8];
};
// The weights of one super-group of the other kinds (amdc_layout.h).
struct ItemQ8 {
  u32x4 h, n[16];
};
struct ItemQ6 {
  u32x4 h, n[8], x[4];
  u32 d;
};
template <int KIND> struct ItemOf { using type = Item; };
template <> struct ItemOf<AMDC_Q8_0> { using type = ItemQ8; };
template <> struct ItemOf<AMDC_Q6_K> { using type = ItemQ6; };

// The loads are unconditional (a lane past the last super-group reads the
// row's first one again, inside the same wave's lines, and ignores it): no
// branch joins them, so that a wait for an earlier load does not become a
// wait for these.
template <int KIND>
__device__ __forceinline__ void load_item(Item &it, const uint8_t *wr, u32 ng, u32 g, bool ok) {
  g = ok ? g : 0u;
  it.h = __builtin_nontemporal_load((const u32x4 *)(wr + amdc_header_off(g)));
#pragma unroll
  for (u32 k = 0; k < 8u; k++) it.n[k] = __builtin_nontemporal_load((const u32x4 *)(wr + amdc_nib_off(ng, g, k)));
}

// One super-group's contribution to a row: for each of its 8 blocks k (LDS
// slot p = k GC + gl of the staged vector), the integer block dot and the
// reference's per-block float step (src/cpu.c:81, 112, 142, 168).
// LEAN: a scheduling barrier after every block, so that the LDS words of at
// most two blocks are live at once (for kernels that hold two items).
template <int KIND, bool LEAN = false>
__device__ __forceinline__ float item_dot(const typename ItemOf<KIND>::type &it, u32 gl, u32 GC, const u32x4 *s_lo, const u32x4 *s_hi,
                                          const float *s_d, const u32 *s_as, float acc) {
  float dsc = 0.0f, dmn = 0.0f;
  if constexpr (KIND == AMDC_Q4_K) dsc = h2f(it.h.x), dmn = h2f(it.h.x >> 16);
  if constexpr (KIND == AMDC_Q6_K) dsc = h2f(it.d);
#pragma unroll
  for (u32 k = 0; k < 8u; k++) {
    const u32 p = k * GC + gl;
    const float da = s_d[p];
    if constexpr (KIND == AMDC_Q8_0) {
      const int dq = q8_dot(it.n[2u * k], it.n[2u * k + 1u], s_lo[p], s_hi[p]);
      const float sw = h2f(hword(it.h, k >> 1) >> (16u * (k & 1u)));
      acc += (sw * da) * (float)dq;
    } else if constexpr (KIND == AMDC_Q6_K) {
      // half h of sub-block k: sum (q - 32) a = sum q a - 32 (sum a); the
      // staged vector holds 32 (sum a) of each half (two u32 per block)
      int d0, d1;
      q6k_dots(it.n[k], hword(it.x[k >> 1], 2u * (k & 1u)), hword(it.x[k >> 1], 2u * (k & 1u) + 1u), s_lo[p], s_hi[p], d0, d1);
      const u32x2 hs = ((const u32x2 *)s_as)[p];
      d0 = (int)((u32)d0 - hs.x), d1 = (int)((u32)d1 - hs.y);
      const u32 sw = hword(it.h, k >> 1) >> (16u * (k & 1u));
      const float s0 = dsc * (float)(int)(int8_t)(sw & 255u), s1 = dsc * (float)(int)(int8_t)((sw >> 8) & 255u);
      acc = __builtin_fmaf(__builtin_fmaf(s1, (float)d1, s0 * (float)d0), da, acc);
    } else {
      const int dq = nib_dot(it.n[k], s_lo[p], s_hi[p]);
      const u32 as = s_as[p];
      if constexpr (KIND == AMDC_Q4_0) {
        const float sw = h2f(hword(it.h, k >> 1) >> (16u * (k & 1u)));
        acc += (sw * da) * (float)(int)((u32)dq - 8u * as);
      } else {
        const float sw = dsc * (float)q4k_sc(it.h, k), mm = dmn * (float)q4k_mn(it.h, k);
        acc = __builtin_fmaf(-mm, da * (float)(int)as, __builtin_fmaf(sw * (float)dq, da, acc));
      }
    }
    if (LEAN && (k & 1u)) __builtin_amdgcn_sched_barrier(0);
  }
  return acc;
}

// Fused quantization into the staged vector (the arithmetic of
// amdc_quant_q8): 8 lanes per block, 4 values per lane, 32 blocks per pass of
// the workgroup; each block goes to the LDS slot of the staged layout
// (permuted as the weights, p = (b % 8) ng + b / 8) as lo/hi words, d and
// asum, and, when q8out is given, workgroup 0 also writes the Q8 buffer. The
// activation loads of NC passes are issued at once (load), so that a
// kernel can put them ahead of its first weight loads and quantize (quant)
// while the weights are in flight (loads count down in issue order); they are
// unconditional (a block past nb reads the last block again and takes zeros),
// so that no branch joins them. The max and the sum of a block's 8 lanes go
// by DPP (xor 1, xor 2, then the half-row mirror).
template <u32 NC, u32 NTH = NT> struct FusedQ8T {
  static constexpr u32 BP = NTH / 8u; // blocks per pass
  u32 bp = BP;                         // ... at run time (a workgroup of blockDim.x < NTH threads: blockDim.x / 8)
  // a K range of the vector (the split-K kernels): super-groups sgb .. of the row go to LDS columns
  // 0 .., with column stride gc (0: the whole row, stride ng)
  u32 sgb = 0u, gc = 0u;
  v4f xv[NC];
  __device__ __forceinline__ void load(const float *__restrict__ xf, u32 nb, u32 b0) {
    const u32 tid = threadIdx.x, e = tid & 7u;
#pragma unroll
    for (u32 c = 0; c < NC; c++) {
      const u32 b = b0 + bp * c + (tid >> 3);
      const v4f v = *(const v4f *)(xf + 32u * (b < nb ? b : nb - 1u) + 4u * e);
      xv[c] = b < nb ? v : (v4f){0.0f, 0.0f, 0.0f, 0.0f};
    }
  }
  __device__ __forceinline__ void quant(u32 b0, u32 nb, u32 ng, u32x4 *s_lo, u32x4 *s_hi, float *s_d, u32 *s_as, uint8_t *__restrict__ q8out) {
    const u32 tid = threadIdx.x, e = tid & 7u, nblk = 8u * (sgb + (gc ? gc : ng)), st = gc ? gc : ng;
#pragma unroll
    for (u32 c = 0; c < NC; c++) {
      if (b0 + bp * c >= nblk) break;
      const u32 b = b0 + bp * c + (tid >> 3);
      float a = __builtin_fmaxf(__builtin_fmaxf(__builtin_fabsf(xv[c].x), __builtin_fabsf(xv[c].y)),
                                __builtin_fmaxf(__builtin_fabsf(xv[c].z), __builtin_fabsf(xv[c].w)));
      a = __builtin_fmaxf(a, dpp<0xB1>(a));
      a = __builtin_fmaxf(a, dpp<0x4E>(a));
      a = __builtin_fmaxf(a, dpp<0x141>(a));
      const float d = a / 127.0f;
      int qi[4];
      q8_round4(xv[c], d, qi);
      const u32 word = (u32)(qi[0] & 255) | (u32)(qi[1] & 255) << 8 | (u32)(qi[2] & 255) << 16 | (u32)qi[3] << 24;
      u32 sum = (u32)qi[0] + (u32)qi[1] + (u32)qi[2] + (u32)qi[3];
      sum += (u32)__builtin_amdgcn_update_dpp(0, (int)sum, 0xB1, 0xF, 0xF, false);
      sum += (u32)__builtin_amdgcn_update_dpp(0, (int)sum, 0x4E, 0xF, 0xF, false);
      sum += (u32)__builtin_amdgcn_update_dpp(0, (int)sum, 0x141, 0xF, 0xF, false);
      if (b < nblk) {
        const u32 p = (b & 7u) * st + (b >> 3) - sgb;
        ((u32 *)(e < 4u ? &s_lo[p] : &s_hi[p]))[e & 3u] = word;
        if (e == 0u) s_d[p] = d, s_as[p] = sum;
      }
      if (q8out && blockIdx.x == 0u && b < nb) { // the Q8 buffer, for other consumers
        ((u32 *)(q8out + 32u * b))[e] = word;
        if (e == 0u) ((float *)(q8out + 32u * nb))[b] = d, ((u32 *)(q8out + 36u * nb))[b] = sum;
      }
    }
  }
};
typedef FusedQ8T<QCH> FusedQ8;

template <int KIND, bool FQ>
__device__ __forceinline__ void gemv1_body(const uint8_t *__restrict__ W, const uint8_t *__restrict__ xq, float *__restrict__ y, u32 rows,
                                           u32 nb, const float *__restrict__ bias, const float *__restrict__ res, u32 L,
                                           const float *__restrict__ xf = nullptr, uint8_t *__restrict__ q8out = nullptr) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const u32 ng = amdc_ngroups(nb), tid = threadIdx.x, lane = tid & 63u, wv = tid >> 6;
  const u32 l = lane & (L - 1u), q = lane / L, rpw = 64u / L, rpg = 4u * rpw;
  const u32 nrg = (rows + rpg - 1u) / rpg, ni = (ng + L - 1u) / L;
  const u64 RB = amdc_row_bytes(nb);
  const u32 nblk = 8u * ng;
  u32x4 *s_lo = (u32x4 *)smem;
  u32x4 *s_hi = s_lo + nblk;
  float *s_d = (float *)(s_hi + nblk);
  u32 *s_as = (u32 *)(s_d + nblk);
  u32 rg = blockIdx.x, i = 0;
  if (rg >= nrg) return; // the whole workgroup
  auto rowp = [&](u32 g_) {
    const u32 r_ = g_ * rpg + wv * rpw + q;
    return W + (u64)(r_ < rows ? r_ : rows - 1u) * RB;
  };
  FusedQ8 fq;
  Item cur, nxt;
  if (FQ) {
    fq.load(xf, nb, 0);
    __asm__ volatile("" ::: "memory"); // keep the activation loads ahead of the weight loads
  }
  load_item<KIND>(cur, rowp(rg), ng, l, l < ng);
  if (FQ) {
    fq.quant(0, nb, ng, s_lo, s_hi, s_d, s_as, q8out);
    for (u32 b0 = 32u * QCH; b0 < nblk; b0 += 32u * QCH) {
      fq.load(xf, nb, b0);
      fq.quant(b0, nb, ng, s_lo, s_hi, s_d, s_as, q8out);
    }
  } else {
    for (u32 j = tid; j < nblk; j += NT) { // stage the whole Q8 vector (permuted)
      const u32 p = (j & 7u) * ng + (j >> 3);
      u32x4 lo = (u32x4)(0u), hi = (u32x4)(0u);
      float d = 0.0f;
      u32 as = 0;
      if (j < nb) {
        lo = *(const u32x4 *)(xq + 32u * j);
        hi = *(const u32x4 *)(xq + 32u * j + 16u);
        d = ((const float *)(xq + 32u * nb))[j];
        as = ((const u32 *)(xq + 36u * nb))[j];
      }
      s_lo[p] = lo, s_hi[p] = hi, s_d[p] = d, s_as[p] = as;
    }
  }
  __syncthreads();
  ItemTree tr;
  for (;;) {
    u32 rg2 = rg, i2 = i + 1u;
    if (i2 == ni) i2 = 0, rg2 += gridDim.x;
    const bool more = rg2 < nrg;
    if (more) load_item<KIND>(nxt, rowp(rg2), ng, l + L * i2, l + L * i2 < ng);
    const u32 g = l + L * i;
    const float leaf = item_dot<KIND>(cur, g < ng ? g : 0u, ng, s_lo, s_hi, s_d, s_as, 0.0f);
    tr.add(seg_sum(g < ng ? leaf : 0.0f, L), i);
    if (i2 == 0u) { // the row group is done
      const float v = tr.sum(ni);
      const u32 r = rg * rpg + wv * rpw + q;
      if (l == 0u && r < rows) {
        float o = v;
        if (bias) o = o + bias[r];
        if (res) o = res[r] + o;
        y[r] = o;
      }
    }
    if (!more) break;
    cur = nxt, rg = rg2, i = i2;
  }
}

extern "C" __global__ __launch_bounds__(256) void amdc_gemv_q4_0_p1(const uint8_t *W, const uint8_t *xq, float *y, u32 rows, u32 nb,
                                                                   const float *bias, const float *res, u32 L) {
  gemv1_body<AMDC_Q4_0, false>(W, xq, y, rows, nb, bias, res, L);
}
extern "C" __global__ __launch_bounds__(256) void amdc_gemv_q4_k_p1(const uint8_t *W, const uint8_t *xq, float *y, u32 rows, u32 nb,
                                                                   const float *bias, const float *res, u32 L) {
  gemv1_body<AMDC_Q4_K, false>(W, xq, y, rows, nb, bias, res, L);
}
// The same, quantizing the f32 vector x in the prologue (fused OP_QUANT);
// workgroup 0 writes the Q8 buffer to q8 when q8 is not NULL.
extern "C" __global__ __launch_bounds__(256) void amdc_gemv_q4_0_x1(const uint8_t *W, const float *x, float *y, u32 rows, u32 nb,
                                                                   const float *bias, const float *res, u32 L, uint8_t *q8) {
  gemv1_body<AMDC_Q4_0, true>(W, nullptr, y, rows, nb, bias, res, L, x, q8);
}
extern "C" __global__ __launch_bounds__(256) void amdc_gemv_q4_k_x1(const uint8_t *W, const float *x, float *y, u32 rows, u32 nb,
                                                                   const float *bias, const float *res, u32 L, uint8_t *q8) {
  gemv1_body<AMDC_Q4_K, true>(W, nullptr, y, rows, nb, bias, res, L, x, q8);
}

// The decode GEMV, single-shot form (amdc_gemv_*_s{1,2,3,4}, _xs{1,2,3,4}):
// one row group per workgroup (grid = the row groups), and each lane issues
// the loads of all NI = ceil(ng / L) of its super-groups at once, before the
// activations are staged (or quantized: _xs), so that no load waits for
// another's arithmetic and no register carries an item across a loop. Without
// the second item buffer and the loop the kernel needs far fewer registers
// (64 to 80 VGPRs at NI = 1: 6 to 8 waves per SIMD), so that the workgroups
// of a whole matrix are resident at once and the arithmetic of one overlaps
// the loads of the others. Lane split, LDS layout, block arithmetic and
// summation order are those of gemv1_body (bit-equal results).
// QCN > 0 (the xw kernels): QCN passes of quantization loads in flight, and
// the workgroup's size taken at run time (blockDim.x <= NTH threads).
// The fused RMSNorm of a decode GEMV's result (the reference's gemv_norm_tail, kernels/ie_kernels.c:
// 267-283, IE_NORM_FUSE): the GEMV's workgroups store y agent-coherently; after its stores each
// workgroup counts itself on cnt; the last of the gridDim.x computes ny = rmsnorm(y) nw (rows <= 8192 floats)
// and, when nq is not NULL, its Q8 copy, with the device code of amdc_rmsnorm_q8 (256 threads: the
// same bits), and sets cnt back to 0. Every thread of every workgroup calls it.
struct NormTail {
  const float *nw;
  float *ny;
  uint8_t *nq;
  float eps;
  u32 *cnt;
};
__device__ __forceinline__ void put_y(float *y, float v, bool coh) {
  if (coh) __hip_atomic_store(y, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  else *y = v;
}
__device__ __forceinline__ void norm_tail(const float *__restrict__ y, u32 rows, const NormTail &nt) {
  __shared__ u32 s_last;
  __shared__ float s_ss[4];
  __builtin_amdgcn_s_waitcnt(0x0F70); // vmcnt(0): this thread's stores of y are complete
  __syncthreads();
  if (threadIdx.x == 0u) {
    const bool last = __hip_atomic_fetch_add(nt.cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u == gridDim.x;
    if (last) __hip_atomic_store(nt.cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = last ? 1u : 0u;
  }
  __syncthreads();
  if (!s_last) return;
  // every element of y once, coherently, all in flight: thread tid holds y[tid + 256 k] (k < rows / 256,
  // rows <= 8192), which is both rms_scale's order for the sum of squares and the element (block 8 k +
  // tid / 32, lane tid % 32) it normalizes
  const u32 nb = rows >> 5, tid = threadIdx.x;
  const __amdgpu_buffer_rsrc_t ry = rsrc(y, 4u * rows);
  const __amdgpu_buffer_rsrc_t rw = rsrc(nt.nw, 4u * rows);
  float yv[32], wv[32]; // with the norm weights, all loads in flight together
#pragma unroll
  for (u32 k = 0; k < 32u; k++) {
    const u32 i = tid + NT * k < rows ? 4u * (tid + NT * k) : 0xFFFFFFF0u;
    yv[k] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(ry, i, 0, CPOL_SC1));
    wv[k] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rw, i, 0, 0));
  }
  float ss = 0.0f;
#pragma unroll
  for (u32 k = 0; k < 32u; k++)
    if (tid + NT * k < rows) ss += yv[k] * yv[k];
  const float s = rms_reduce(ss, rows, nt.eps, s_ss);
  // 8 blocks per half-wave at a time, their quantizations interleaved
#pragma unroll
  for (u32 k0 = 0; k0 < 32u; k0 += 8u) {
    if (8u * k0 >= nb) break; // no half-wave has blocks from here on (uniform)
    float v[8];
    u32 b[8];
    bool on[8];
#pragma unroll
    for (u32 k = 0; k < 8u; k++) {
      b[k] = (tid >> 5) + 8u * (k0 + k), on[k] = b[k] < nb; // whole 32-lane halves
      v[k] = yv[k0 + k] * s * wv[k0 + k];
      if (on[k]) nt.ny[tid + NT * (k0 + k)] = v[k];
    }
    if (nt.nq) quant_halves<8>(v, b, on, nt.nq, nb);
  }
}

template <int KIND, u32 NI, bool FQ, u32 NTH, u32 QCN = 0u, bool TAIL = false>
__device__ __forceinline__ void gemvs_body(const uint8_t *__restrict__ W, const uint8_t *__restrict__ xq, float *__restrict__ y, u32 rows,
                                           u32 nb, const float *__restrict__ bias, const float *__restrict__ res, u32 L,
                                           const float *__restrict__ xf = nullptr, uint8_t *__restrict__ q8out = nullptr,
                                           const NormTail &ntl = NormTail{}) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const u32 nth = QCN ? blockDim.x : NTH;
  const u32 ng = amdc_ngroups(nb), tid = threadIdx.x, lane = tid & 63u, wv = tid >> 6;
  const u32 l = lane & (L - 1u), q = lane / L, rpw = 64u / L, rpg = (nth / 64u) * rpw;
  const u64 RB = amdc_row_bytes(nb);
  const u32 nblk = 8u * ng;
  u32x4 *s_lo = (u32x4 *)smem;
  u32x4 *s_hi = s_lo + nblk;
  float *s_d = (float *)(s_hi + nblk);
  u32 *s_as = (u32 *)(s_d + nblk);
  const u32 r = blockIdx.x * rpg + wv * rpw + q;
  const uint8_t *wr = W + (u64)(r < rows ? r : rows - 1u) * RB;
  constexpr u32 QC = QCN ? QCN : (QCH * NT) / NTH; // passes in flight: 128 blocks (QCN: QCN passes of nth / 8 blocks)
  FusedQ8T<QC, NTH> fq;
  fq.bp = nth / 8u;
  if (FQ) {
    fq.load(xf, nb, 0);
    __asm__ volatile("" ::: "memory"); // the activation loads ahead of the weight loads
  }
  // the Q8 vector's first NSV chunks of the staging loop loaded ahead of the weights: loads complete in
  // issue order, so staged after them the vector waited for every weight load (MI355X: 5120 x 17408
  // Q4_K 19.7-20.1 -> 18.6-19.3 us; with 3 chunks, all of its 544 blocks, 14.8-15.2 -> 14.5 us)
  constexpr u32 NSV = NI >= 2u ? 3u : 2u;
  u32x4 vlo[NSV], vhi[NSV];
  float vd[NSV];
  u32 vas[NSV];
  if (!FQ) {
#pragma unroll
    for (u32 c = 0; c < NSV; c++) {
      const u32 j = tid + c * NTH, jj = j < nb ? j : 0u;
      vlo[c] = *(const u32x4 *)(xq + 32u * jj);
      vhi[c] = *(const u32x4 *)(xq + 32u * jj + 16u);
      vd[c] = ((const float *)(xq + 32u * nb))[jj];
      vas[c] = ((const u32 *)(xq + 36u * nb))[jj];
    }
    __asm__ volatile("" ::: "memory");
  }
  // with the quantization fused, part of the weight loads go out after the quantization: issuing a
  // load stalls while the memory pipeline is full, and with every item in flight the quantization
  // started microseconds late (a wall-clock timeline of 22016 x 4096: 4.2 us to issue the loads); the
  // loads issued first by all workgroups keep the memory busy meanwhile, and the items issued later
  // are not live during the quantization (the two-item Q4_0 kernel: 157 -> 126 VGPRs, 4 workgroups
  // per CU)
  Item it[NI];
  constexpr u32 NI0 = FQ && NI >= 2u ? 1u : NI; // items issued before the quantization
  // Of the first item, only the header and PB nibble planes go out before the quantization (the rest
  // after it): the workgroup-per-CU kernels with one item per lane and the single-shot kernels with
  // two or more. Swept on MI355X (c1 Q4_0, us): wqkv 12288 x 4096 7.5 / 6.8 / 7.5 with 4 / 2 / 0
  // planes of the workgroup-per-CU kernel, down 4096 x 11008 8.96 / 8.5; wgu 22016 x 4096 and lm_head
  // 32000 x 4096 on the two-item kernel 11.9 + 14.3 with all 8 planes of item 0, 11.0 + 13.9 with 2,
  // 10.4 + 15.0 with 4. The 16-row one-item single-shot kernel keeps its whole item before (4.9 against
  // 5.5 us with 4 planes).
  constexpr bool SPL = FQ && (KIND == AMDC_Q4_0 || KIND == AMDC_Q4_K) && ((QCN > 0u && NI == 1u) || (QCN == 0u && NI >= 2u));
  constexpr u32 PB = 2u;
  if constexpr (SPL) {
    const u32 g = l < ng ? l : 0u;
    it[0].h = __builtin_nontemporal_load((const u32x4 *)(wr + amdc_header_off(g)));
#pragma unroll
    for (u32 k = 0; k < PB; k++) it[0].n[k] = __builtin_nontemporal_load((const u32x4 *)(wr + amdc_nib_off(ng, g, k)));
  } else {
#pragma unroll
    for (u32 i = 0; i < NI0; i++) load_item<KIND>(it[i], wr, ng, l + L * i, l + L * i < ng);
  }
  if (FQ) {
    fq.quant(0, nb, ng, s_lo, s_hi, s_d, s_as, q8out);
    for (u32 b0 = fq.bp * QC; b0 < nblk; b0 += fq.bp * QC) {
      fq.load(xf, nb, b0);
      fq.quant(b0, nb, ng, s_lo, s_hi, s_d, s_as, q8out);
    }
    if constexpr (SPL) {
      const u32 g = l < ng ? l : 0u;
#pragma unroll
      for (u32 k = PB; k < 8u; k++) it[0].n[k] = __builtin_nontemporal_load((const u32x4 *)(wr + amdc_nib_off(ng, g, k)));
    }
#pragma unroll
    for (u32 i = NI0; i < NI; i++) load_item<KIND>(it[i], wr, ng, l + L * i, l + L * i < ng);
  } else {
#pragma unroll
    for (u32 c = 0; c < NSV; c++) {
      const u32 j = tid + c * NTH;
      if (j < nblk) {
        const u32 p = (j & 7u) * ng + (j >> 3);
        const bool in = j < nb;
        s_lo[p] = in ? vlo[c] : (u32x4)(0u), s_hi[p] = in ? vhi[c] : (u32x4)(0u), s_d[p] = in ? vd[c] : 0.0f, s_as[p] = in ? vas[c] : 0u;
      }
    }
    for (u32 j = tid + NSV * NTH; j < nblk; j += NTH) { // stage the rest of the Q8 vector (permuted)
      const u32 p = (j & 7u) * ng + (j >> 3);
      u32x4 lo = (u32x4)(0u), hi = (u32x4)(0u);
      float d = 0.0f;
      u32 as = 0;
      if (j < nb) {
        lo = *(const u32x4 *)(xq + 32u * j);
        hi = *(const u32x4 *)(xq + 32u * j + 16u);
        d = ((const float *)(xq + 32u * nb))[j];
        as = ((const u32 *)(xq + 36u * nb))[j];
      }
      s_lo[p] = lo, s_hi[p] = hi, s_d[p] = d, s_as[p] = as;
    }
  }
  __syncthreads();
  ItemTree tr;
#pragma unroll
  for (u32 i = 0; i < NI; i++) {
    const u32 g = l + L * i;
    const float leaf = item_dot<KIND>(it[i], g < ng ? g : 0u, ng, s_lo, s_hi, s_d, s_as, 0.0f);
    tr.add(seg_sum(g < ng ? leaf : 0.0f, L), i);
  }
  const float v = tr.sum(NI);
  if (l == 0u && r < rows) {
    float o = v;
    if (bias) o = o + bias[r];
    if (res) o = res[r] + o;
    put_y(&y[r], o, TAIL);
  }
  if constexpr (TAIL) norm_tail(y, rows, ntl);
}

#define GEMVS_KERNELS(KN, KIND, NI, TAG, NTH)                                                                                            \
  extern "C" __global__ __launch_bounds__(NTH) void amdc_gemv_##KN##_##TAG##NI(const uint8_t *W, const uint8_t *xq, float *y, u32 rows, \
                                                                               u32 nb, const float *bias, const float *res, u32 L) {  \
    gemvs_body<KIND, NI, false, NTH>(W, xq, y, rows, nb, bias, res, L);                                                                 \
  }                                                                                                                                      \
  extern "C" __global__ __launch_bounds__(NTH) void amdc_gemv_##KN##_x##TAG##NI(const uint8_t *W, const float *x, float *y, u32 rows,  \
                                                                                u32 nb, const float *bias, const float *res, u32 L,   \
                                                                                uint8_t *q8) {                                        \
    gemvs_body<KIND, NI, true, NTH>(W, nullptr, y, rows, nb, bias, res, L, x, q8);                                                      \
  }
GEMVS_KERNELS(q4_0, AMDC_Q4_0, 1, s, 256)
GEMVS_KERNELS(q4_0, AMDC_Q4_0, 2, s, 256)
GEMVS_KERNELS(q4_0, AMDC_Q4_0, 3, s, 256)
GEMVS_KERNELS(q4_0, AMDC_Q4_0, 4, s, 256)
GEMVS_KERNELS(q4_k, AMDC_Q4_K, 1, s, 256)
GEMVS_KERNELS(q4_k, AMDC_Q4_K, 2, s, 256)
GEMVS_KERNELS(q4_k, AMDC_Q4_K, 3, s, 256)
GEMVS_KERNELS(q4_k, AMDC_Q4_K, 4, s, 256)
// The one-item single-shot kernels on 512-thread workgroups (amdc_gemv_{q4_0,q4_k}_s1w): the Q8 vector
// staged once per 8 waves instead of 4, for matrices of many rows (the host takes them from 16384
// rows; MI355X, us, 256 / 512 threads: 152064 x 5120 Q4_K 74.2 / 69.9, 34816 x 5120 20.3 / 19.6,
// 32000 x 4096 Q4_0 13.9 / 13.8; 6144 x 5120 Q4_K 6.9 / 7.1, 4096 x 4096 Q4_0 4.4 / 4.8). Same lanes per
// row and summation order: the same bits.
#define GEMVS_KERNEL_512(KN, KIND)                                                                                                  \
  extern "C" __global__ __launch_bounds__(512) void amdc_gemv_##KN##_s1w(const uint8_t *W, const uint8_t *xq, float *y, u32 rows,  \
                                                                         u32 nb, const float *bias, const float *res, u32 L) {     \
    gemvs_body<KIND, 1, false, 512u>(W, xq, y, rows, nb, bias, res, L);                                                           \
  }
GEMVS_KERNEL_512(q4_0, AMDC_Q4_0)
GEMVS_KERNEL_512(q4_k, AMDC_Q4_K)

// The single-shot kernels with the fused RMSNorm tail (amdc_gemv_norm)
#define GEMVSN_KERNEL(KN, KIND, NI)                                                                                                  \
  extern "C" __global__ __launch_bounds__(256) void amdc_gemv_##KN##_n##NI(const uint8_t *W, const uint8_t *xq, float *y, u32 rows, \
                                                                           u32 nb, const float *bias, const float *res, u32 L,      \
                                                                           const float *nw, float *ny, uint8_t *nq, float eps,      \
                                                                           u32 *cnt) {                                              \
    gemvs_body<KIND, NI, false, 256u, 0u, true>(W, xq, y, rows, nb, bias, res, L, nullptr, nullptr, NormTail{nw, ny, nq, eps, cnt}); \
  }
GEMVSN_KERNEL(q4_0, AMDC_Q4_0, 1)
GEMVSN_KERNEL(q4_0, AMDC_Q4_0, 2)
GEMVSN_KERNEL(q4_0, AMDC_Q4_0, 3)
GEMVSN_KERNEL(q4_0, AMDC_Q4_0, 4)
GEMVSN_KERNEL(q4_k, AMDC_Q4_K, 1)
GEMVSN_KERNEL(q4_k, AMDC_Q4_K, 2)
GEMVSN_KERNEL(q4_k, AMDC_Q4_K, 3)
GEMVSN_KERNEL(q4_k, AMDC_Q4_K, 4)

// The single-shot form with the quantization fused, sized to one workgroup per
// CU (amdc_gemv_q4_0_xw1, amdc_gemv_q4_k_xw1 / _xw2: blockDim.x threads, up
// to 1024; the host picks the size so that the grid is about one workgroup
// per CU; a Q4_0 two-item form measured slower than 256-thread workgroups on
// 22016 x 4096 and is not built): the vector
// is quantized once per CU instead of once per 16 or 32 rows, by every
// thread, with up to 4 passes of blockDim.x / 8 blocks loaded at once (ahead
// of the weight loads). Same lane split and arithmetic: bit-equal results.
#define GEMVXW_KERNEL(KN, KIND, NI, NTH)                                                                                             \
  extern "C" __global__ __launch_bounds__(NTH) void amdc_gemv_##KN##_xw##NI(const uint8_t *W, const float *x, float *y, u32 rows,  \
                                                                            u32 nb, const float *bias, const float *res, u32 L,   \
                                                                            uint8_t *q8) {                                        \
    gemvs_body<KIND, NI, true, NTH, 4u>(W, nullptr, y, rows, nb, bias, res, L, x, q8);                                             \
  }
GEMVXW_KERNEL(q4_0, AMDC_Q4_0, 1, 1024)
GEMVXW_KERNEL(q4_k, AMDC_Q4_K, 1, 1024)
GEMVXW_KERNEL(q4_k, AMDC_Q4_K, 2, 1024)

// The multi-vector GEMV of a few vectors (T <= 8: the MTP verify step) on
// the decode kernel's integer dots (amdc_gemv_*_m<NI>): the single-shot split
// (one row group per workgroup, each lane's NI super-groups loaded at once),
// with the Q8 vectors of all T tokens staged in LDS (320 ng bytes per token,
// permuted as the weights), and each lane's super-groups dotted with every
// token: the weights are read once for all T vectors and the arithmetic of
// each token is the decode GEMV's (the same block steps, leaves and tree, so
// each y_t equals the decode GEMV of vector t bit for bit). No K split and no
// reduction launch. Vector t at xq + t xs bytes, y_t at y + t ys floats,
// res_t at res + t rs floats. The VALU work grows with T (8 dot4 per block and
// vector), so the host takes it for few vectors on small matrices, where the
// int8-MFMA kernels' fixed costs (K split, reduction launch) dominate.
template <int KIND, u32 NI>
__device__ __forceinline__ void gemvm_body(const uint8_t *__restrict__ W, const uint8_t *__restrict__ xq, float *__restrict__ y, u32 rows,
                                           u32 nb, const float *__restrict__ bias, const float *__restrict__ res, u32 L, u32 T, u32 xs,
                                           u32 ys, u32 rs) {
  constexpr u32 TM = 8u; // the most vectors per launch
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const u32 ng = amdc_ngroups(nb), tid = threadIdx.x, lane = tid & 63u, wv = tid >> 6;
  const u32 l = lane & (L - 1u), q = lane / L, rpw = 64u / L, rpg = 4u * rpw;
  const u64 RB = amdc_row_bytes(nb);
  const u32 nblk = 8u * ng, tb = 320u * ng; // LDS bytes per token
  const u32 r = blockIdx.x * rpg + wv * rpw + q;
  const uint8_t *wr = W + (u64)(r < rows ? r : rows - 1u) * RB;
  Item it[NI];
#pragma unroll
  for (u32 i = 0; i < NI; i++) load_item<KIND>(it[i], wr, ng, l + L * i, l + L * i < ng);
  // stage (token, block) pairs, 4 per thread in flight at a time
  for (u32 j0 = tid; j0 < T * nblk; j0 += 4u * NT) {
    u32x4 lo[4], hi[4];
    float d[4];
    u32 as[4];
#pragma unroll
    for (u32 c = 0; c < 4u; c++) {
      const u32 j = j0 + c * NT, t = j / nblk, jb = j - t * nblk;
      const bool in = j < T * nblk && jb < nb;
      const uint8_t *xt = xq + (u64)(in ? t : 0u) * xs;
      const u32 jj = in ? jb : 0u;
      lo[c] = *(const u32x4 *)(xt + 32u * jj);
      hi[c] = *(const u32x4 *)(xt + 32u * jj + 16u);
      d[c] = ((const float *)(xt + 32u * nb))[jj];
      as[c] = ((const u32 *)(xt + 36u * nb))[jj];
      if (!in) lo[c] = (u32x4)(0u), hi[c] = (u32x4)(0u), d[c] = 0.0f, as[c] = 0u;
    }
#pragma unroll
    for (u32 c = 0; c < 4u; c++) {
      const u32 j = j0 + c * NT;
      if (j < T * nblk) {
        const u32 t = j / nblk, jb = j - t * nblk, p = (jb & 7u) * ng + (jb >> 3);
        uint8_t *base = smem + t * tb;
        ((u32x4 *)base)[p] = lo[c];
        ((u32x4 *)base + nblk)[p] = hi[c];
        ((float *)(base + 32u * nblk))[p] = d[c];
        ((u32 *)(base + 36u * nblk))[p] = as[c];
      }
    }
  }
  __syncthreads();
  ItemTree tr[TM];
#pragma unroll
  for (u32 i = 0; i < NI; i++) {
    const u32 g = l + L * i;
#pragma unroll
    for (u32 t = 0; t < TM; t++) {
      if (t < T) {
        const uint8_t *base = smem + t * tb;
        const float leaf = item_dot<KIND>(it[i], g < ng ? g : 0u, ng, (const u32x4 *)base, (const u32x4 *)base + nblk,
                                          (const float *)(base + 32u * nblk), (const u32 *)(base + 36u * nblk), 0.0f);
        tr[t].add(seg_sum(g < ng ? leaf : 0.0f, L), i);
      }
    }
  }
  if (l == 0u && r < rows) {
    const float b = bias ? bias[r] : 0.0f;
#pragma unroll
    for (u32 t = 0; t < TM; t++) {
      if (t < T) {
        float o = tr[t].sum(NI);
        if (bias) o = o + b;
        if (res) o = res[(u64)t * rs + r] + o;
        y[(u64)t * ys + r] = o;
      }
    }
  }
}

#define GEMVM_KERNEL(KN, KIND, NI)                                                                                                         \
  extern "C" __global__ __launch_bounds__(256) void amdc_gemv_##KN##_m##NI(const uint8_t *W, const uint8_t *xq, float *y, u32 rows,    \
                                                                           u32 nb, const float *bias, const float *res, u32 L, u32 T,  \
                                                                           u32 xs, u32 ys, u32 rs) {                                   \
    gemvm_body<KIND, NI>(W, xq, y, rows, nb, bias, res, L, T, xs, ys, rs);                                                               \
  }
GEMVM_KERNEL(q4_0, AMDC_Q4_0, 1)
GEMVM_KERNEL(q4_k, AMDC_Q4_K, 1)

// The decode GEMV, second form: the same lane split, LDS layout and
// per-block arithmetic as gemv1_body, with the weights read through a buffer
// resource (32-bit offsets; the host checks rows * row bytes + row bytes <
// 2^32) so that an item past the end -- a lane past the last super-group, a
// row past the last, the prefetch after the workgroup's last item -- is a
// load out of range, which returns zeros and touches no memory. No load is
// then under a branch, and the loop over a workgroup's items (row groups
// blockIdx.x, + gridDim.x, ...; ceil(ng / L) items per lane each) keeps one
// item in flight while it computes the previous one: two item buffers
// alternate (a 2-way unrolled loop: no register copy, which would wait for
// the loads). The bias and residual values of an item's row come with it
// (loads out of range when absent).
template <int KIND>
struct Item2 {
  typename ItemOf<KIND>::type w;
  float b, r;
};

// The loads of super-group g of the row at byte base of resource rw (base past
// the resource: every load returns zeros), cache policy COH.
template <int KIND, int COH>
__device__ __forceinline__ void item_load(typename ItemOf<KIND>::type &w, __amdgpu_buffer_rsrc_t rw, u32 base, u32 g, u32 ng) {
  const u32 t = g >> 3, gt = ng - 8u * t < 8u ? ng - 8u * t : 8u;
  w.h = __builtin_amdgcn_raw_buffer_load_b128(rw, base + 16u * g, 0, COH);
  if constexpr (KIND == AMDC_Q8_0) {
    const u32 o0 = base + 16u * ng + 2048u * t + 16u * (g & 7u);
#pragma unroll
    for (u32 k = 0; k < 16u; k++) w.n[k] = __builtin_amdgcn_raw_buffer_load_b128(rw, o0 + 16u * gt * k, 0, COH);
  } else if constexpr (KIND == AMDC_Q6_K) {
    const u32 D = amdc_q6k_dpad(ng), o0 = base + 16u * ng + D + 1024u * t + 16u * (g & 7u);
    const u32 o1 = base + 144u * ng + D + 512u * t + 16u * (g & 7u);
#pragma unroll
    for (u32 k = 0; k < 8u; k++) w.n[k] = __builtin_amdgcn_raw_buffer_load_b128(rw, o0 + 16u * gt * k, 0, COH);
#pragma unroll
    for (u32 k = 0; k < 4u; k++) w.x[k] = __builtin_amdgcn_raw_buffer_load_b128(rw, o1 + 16u * gt * k, 0, COH);
    w.d = __builtin_amdgcn_raw_buffer_load_b16(rw, base + 16u * ng + 2u * g, 0, COH);
  } else {
    const u32 o0 = base + 16u * ng + 1024u * t + 16u * (g & 7u);
#pragma unroll
    for (u32 k = 0; k < 8u; k++) w.n[k] = __builtin_amdgcn_raw_buffer_load_b128(rw, o0 + 16u * gt * k, 0, COH);
  }
}

template <int KIND, bool TAIL = false>
__device__ __forceinline__ void gemv2_body(const uint8_t *__restrict__ W, const uint8_t *__restrict__ xq, float *__restrict__ y, u32 rows,
                                           u32 nb, const float *__restrict__ bias, const float *__restrict__ res, u32 L,
                                           const NormTail &ntl = NormTail{}) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const u32 ng = amdc_ngroups(nb), tid = threadIdx.x, lane = tid & 63u, wv = tid >> 6;
  const u32 l = lane & (L - 1u), q = lane / L, rpw = 64u / L, rpg = 4u * rpw;
  const u32 nrg = (rows + rpg - 1u) / rpg, ni = (ng + L - 1u) / L;
  if (blockIdx.x >= nrg) { // the whole workgroup (with the tail it still counts itself)
    if constexpr (TAIL) norm_tail(y, rows, ntl);
    return;
  }
  const u32 RB = (u32)amdc_row_bytes_k(KIND, nb), NR = rows * RB; // the host checks NR + RB < 2^32
  const u32 nblk = 8u * ng;
  u32x4 *s_lo = (u32x4 *)smem;
  u32x4 *s_hi = s_lo + nblk;
  float *s_d = (float *)(s_hi + nblk);
  u32 *s_as = (u32 *)(s_d + nblk);
  const __amdgpu_buffer_rsrc_t rw = rsrc(W, NR), rb = rsrc(bias, bias ? 4u * rows : 0u), rr = rsrc(res, res ? 4u * rows : 0u);
  const u32 n = ((nrg - blockIdx.x + gridDim.x - 1u) / gridDim.x) * ni; // items per lane
  const u32 rbase = wv * rpw + q;

  // an item's loads: position (j, i) = row group blockIdx.x + j gridDim.x, super-group l + L i
  auto load = [&](Item2<KIND> &it, u32 f, u32 j, u32 i) {
    const u32 r = (blockIdx.x + j * gridDim.x) * rpg + rbase, g = l + L * i;
    const bool ok = f < n && g < ng && r < rows;
    item_load<KIND, 0>(it.w, rw, ok ? r * RB : NR, g, ng);
    const u32 ro = f < n && r < rows ? 4u * r : 0xFFFFFFF0u;
    it.b = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rb, ro, 0, 0));
    it.r = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rr, ro, 0, 0));
  };

  // stage the Q8 vector: the loads of the first SCH blocks per thread go out
  // ahead of the first item's
  u32x4 slo[SCH], shi[SCH];
  float sd[SCH];
  u32 sa[SCH];
  auto sload = [&](u32 i, u32 c) { // slot i <- block tid + NT c
    const u32 jb = tid + NT * c, jj = jb < nb ? jb : nb - 1u;
    slo[i] = *(const u32x4 *)(xq + 32u * jj);
    shi[i] = *(const u32x4 *)(xq + 32u * jj + 16u);
    sd[i] = ((const float *)(xq + 32u * nb))[jj];
    sa[i] = ((const u32 *)(xq + 36u * nb))[jj];
  };
  auto sstore = [&](u32 i, u32 c) {
    const u32 jb = tid + NT * c;
    if (jb < nblk) {
      const u32 p = (jb & 7u) * ng + (jb >> 3);
      const bool in = jb < nb;
      s_lo[p] = in ? slo[i] : (u32x4)(0u), s_hi[p] = in ? shi[i] : (u32x4)(0u);
      s_d[p] = in ? sd[i] : 0.0f;
      if constexpr (KIND == AMDC_Q6_K) { // 32 x the sum of each half of the block
        const int h0 = hsum16(slo[i]), h1 = hsum16(shi[i]);
        ((u32x2 *)s_as)[p] = in ? (u32x2){32u * (u32)h0, 32u * (u32)h1} : (u32x2)(0u);
      } else if constexpr (KIND != AMDC_Q8_0) {
        s_as[p] = in ? sa[i] : 0u;
      }
    }
  };
  for (u32 c = SCH; NT * c < nblk; c++) { // past SCH blocks per thread (more than 24576 columns)
    sload(0, c);
    sstore(0, c);
  }
#pragma unroll
  for (u32 c = 0; c < SCH; c++) sload(c, c);
  __asm__ volatile("" ::: "memory"); // the activation loads ahead of the weight loads
  Item2<KIND> A, B;
  load(A, 0u, 0u, 0u);
#pragma unroll
  for (u32 c = 0; c < SCH; c++) sstore(c, c);
  __syncthreads();

  // the results of the workgroup's rows collect in LDS (after the staged
  // vector) and go out after the loop: a store inside the loop would make the
  // reuse of its registers wait for every load in flight
  float *s_y = (float *)(s_as + (KIND == AMDC_Q6_K ? 2u : 1u) * nblk);
  ItemTree tr;
  auto comp = [&](const Item2<KIND> &it, u32 j, u32 i) {
    const u32 g = l + L * i;
    const float leaf = item_dot<KIND>(it.w, g < ng ? g : 0u, ng, s_lo, s_hi, s_d, s_as, 0.0f);
    tr.add(seg_sum(g < ng ? leaf : 0.0f, L), i);
    if (i == ni - 1u) { // the row group is done
      const float v = tr.sum(ni);
      float o = bias ? v + it.b : v;
      o = res ? it.r + o : o;
      if (l == 0u) s_y[j * rpg + rbase] = o;
    }
  };
  u32 cj = 0, ci = 0, lj = 0, li = 0; // compute / load positions
  auto adv = [&](u32 &j, u32 &i) {
    if (++i == ni) i = 0, j++;
  };
  adv(lj, li);
  for (u32 f = 0; f < n; f += 2u) {
    load(B, f + 1u, lj, li);
    adv(lj, li);
    __asm__ volatile("" ::: "memory"); // the next item's loads go out before this item's arithmetic
    comp(A, cj, ci);
    adv(cj, ci);
    if (f + 1u >= n) break;
    load(A, f + 2u, lj, li);
    adv(lj, li);
    __asm__ volatile("" ::: "memory");
    comp(B, cj, ci);
    adv(cj, ci);
  }
  __syncthreads();
  const u32 ny = (n / ni) * rpg;
  for (u32 k = tid; k < ny; k += NT) {
    const u32 r = (blockIdx.x + (k / rpg) * gridDim.x) * rpg + k % rpg;
    if (r < rows) put_y(&y[r], s_y[k], TAIL);
  }
  if constexpr (TAIL) norm_tail(y, rows, ntl);
}

extern "C" __global__ __launch_bounds__(256) void amdc_gemv_q4_0_p2(const uint8_t *W, const uint8_t *xq, float *y, u32 rows, u32 nb,
                                                                   const float *bias, const float *res, u32 L) {
  gemv2_body<AMDC_Q4_0>(W, xq, y, rows, nb, bias, res, L);
}
extern "C" __global__ __launch_bounds__(256) void amdc_gemv_q4_k_p2(const uint8_t *W, const uint8_t *xq, float *y, u32 rows, u32 nb,
                                                                   const float *bias, const float *res, u32 L) {
  gemv2_body<AMDC_Q4_K>(W, xq, y, rows, nb, bias, res, L);
}
extern "C" __global__ __launch_bounds__(256) void amdc_gemv_q8_0_p2(const uint8_t *W, const uint8_t *xq, float *y, u32 rows, u32 nb,
                                                                   const float *bias, const float *res, u32 L) {
  gemv2_body<AMDC_Q8_0>(W, xq, y, rows, nb, bias, res, L);
}
extern "C" __global__ __launch_bounds__(256) void amdc_gemv_q6_k_p2(const uint8_t *W, const uint8_t *xq, float *y, u32 rows, u32 nb,
                                                                   const float *bias, const float *res, u32 L) {
  gemv2_body<AMDC_Q6_K>(W, xq, y, rows, nb, bias, res, L);
}
// the Q8_0 / Q6_K decode form with the fused RMSNorm tail (amdc_gemv_norm)
#define GEMV2N_KERNEL(KN, KIND)                                                                                                      \
  extern "C" __global__ __launch_bounds__(256) void amdc_gemv_##KN##_pn(const uint8_t *W, const uint8_t *xq, float *y, u32 rows,    \
                                                                        u32 nb, const float *bias, const float *res, u32 L,         \
                                                                        const float *nw, float *ny, uint8_t *nq, float eps,         \
                                                                        u32 *cnt) {                                                 \
    gemv2_body<KIND, true>(W, xq, y, rows, nb, bias, res, L, NormTail{nw, ny, nq, eps, cnt});                                       \
  }
GEMV2N_KERNEL(q8_0, AMDC_Q8_0)
GEMV2N_KERNEL(q6_k, AMDC_Q6_K)

// A few vectors (T <= 8) on a small Q8_0 / Q6_K matrix (amdc_gemv_{q8_0,q6_k}_m1): the decode GEMV's
// items and block arithmetic (gemv2_body's, one row group per workgroup, NI super-groups per lane) with
// the Q8 vectors of all T tokens staged in the LDS; each lane dots its items with every token (the
// decode arithmetic per token: bit-equal to T decode GEMVs), weights read once, no K split.
template <int KIND, u32 NI>
__device__ __forceinline__ void gemvm8_body(const uint8_t *__restrict__ W, const uint8_t *__restrict__ xq, float *__restrict__ y, u32 rows,
                                            u32 nb, const float *__restrict__ bias, const float *__restrict__ res, u32 L, u32 T, u32 xs,
                                            u32 ys, u32 rs) {
  constexpr u32 TM = 8u, BPB = KIND == AMDC_Q6_K ? 44u : 40u; // vectors per launch; LDS bytes per block
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const u32 ng = amdc_ngroups(nb), tid = threadIdx.x, lane = tid & 63u, wv = tid >> 6;
  const u32 l = lane & (L - 1u), q = lane / L, rpw = 64u / L, rpg = 4u * rpw;
  const u32 RB = (u32)amdc_row_bytes_k(KIND, nb), NR = rows * RB; // the host checks NR + RB < 2^32
  const u32 nblk = 8u * ng, tb = BPB * nblk; // LDS bytes per token
  const u32 r = blockIdx.x * rpg + wv * rpw + q;
  const __amdgpu_buffer_rsrc_t rw = rsrc(W, NR);
  typename ItemOf<KIND>::type it[NI];
#pragma unroll
  for (u32 i = 0; i < NI; i++) {
    const u32 g = l + L * i;
    item_load<KIND, 0>(it[i], rw, g < ng && r < rows ? r * RB : NR, g, ng);
  }
  __asm__ volatile("" ::: "memory"); // the weight loads ahead of the vectors'
  // stage (token, block) pairs, 4 per thread in flight at a time, permuted as gemv2_body stages them
  for (u32 j0 = tid; j0 < T * nblk; j0 += 4u * NT) {
    u32x4 lo[4], hi[4];
    float d[4];
#pragma unroll
    for (u32 c = 0; c < 4u; c++) {
      const u32 j = j0 + c * NT, t = j / nblk, jb = j - t * nblk;
      const bool in = j < T * nblk && jb < nb;
      const uint8_t *xt = xq + (u64)(in ? t : 0u) * xs;
      const u32 jj = in ? jb : 0u;
      lo[c] = *(const u32x4 *)(xt + 32u * jj);
      hi[c] = *(const u32x4 *)(xt + 32u * jj + 16u);
      d[c] = ((const float *)(xt + 32u * nb))[jj];
      if (!in) lo[c] = (u32x4)(0u), hi[c] = (u32x4)(0u), d[c] = 0.0f;
    }
#pragma unroll
    for (u32 c = 0; c < 4u; c++) {
      const u32 j = j0 + c * NT;
      if (j < T * nblk) {
        const u32 t = j / nblk, jb = j - t * nblk, p = (jb & 7u) * ng + (jb >> 3);
        uint8_t *base = smem + t * tb;
        ((u32x4 *)base)[p] = lo[c];
        ((u32x4 *)base + nblk)[p] = hi[c];
        ((float *)(base + 32u * nblk))[p] = d[c];
        if constexpr (KIND == AMDC_Q6_K) // 32 x the sum of each half of the block, as gemv2_body stages it
          ((u32x2 *)(base + 36u * nblk))[p] = (u32x2){32u * (u32)hsum16(lo[c]), 32u * (u32)hsum16(hi[c])};
      }
    }
  }
  __syncthreads();
  ItemTree tr[TM];
#pragma unroll
  for (u32 i = 0; i < NI; i++) {
    const u32 g = l + L * i;
#pragma unroll
    for (u32 t = 0; t < TM; t++) {
      if (t < T) {
        const uint8_t *base = smem + t * tb;
        const float leaf = item_dot<KIND>(it[i], g < ng ? g : 0u, ng, (const u32x4 *)base, (const u32x4 *)base + nblk,
                                          (const float *)(base + 32u * nblk), (const u32 *)(base + 36u * nblk), 0.0f);
        tr[t].add(seg_sum(g < ng ? leaf : 0.0f, L), i);
      }
    }
  }
  if (l == 0u && r < rows) {
    const float b = bias ? bias[r] : 0.0f;
#pragma unroll
    for (u32 t = 0; t < TM; t++) {
      if (t < T) {
        float o = tr[t].sum(NI);
        if (bias) o = o + b;
        if (res) o = res[(u64)t * rs + r] + o;
        y[(u64)t * ys + r] = o;
      }
    }
  }
}
#define GEMVM8_KERNEL(KN, KIND, NI)                                                                                                        \
  extern "C" __global__ __launch_bounds__(256) void amdc_gemv_##KN##_m##NI(const uint8_t *W, const uint8_t *xq, float *y, u32 rows,    \
                                                                           u32 nb, const float *bias, const float *res, u32 L, u32 T,  \
                                                                           u32 xs, u32 ys, u32 rs) {                                   \
    gemvm8_body<KIND, NI>(W, xq, y, rows, nb, bias, res, L, T, xs, ys, rs);                                                              \
  }
GEMVM8_KERNEL(q8_0, AMDC_Q8_0, 1)
GEMVM8_KERNEL(q6_k, AMDC_Q6_K, 1)

// ------------------------------------------------------------------ GEMV chain (one launch)

// A list of quantize and decode-GEMV operations run by one persistent launch
// (the reference's megakernel command list, kernels/ie_mk.c, and its GEMV
// chain probe ie_mk_gemv_chain, kernels/ie_kernels.c:464-478): every
// workgroup walks the list; an operation's work is split over the grid
// (row groups blockIdx.x, + gridDim.x, ... of a GEMV; blocks of a
// quantization), and a grid barrier follows an operation marked `sync`.
// While a workgroup waits at a barrier, the weight loads of its first item of
// the next GEMV are already in flight (weights do not depend on earlier
// operations), so the HBM stream does not stop at operation boundaries.
//
// Data passed between workgroups (the Q8 vectors, the GEMV outputs) is
// written and read with agent-scope coherent accesses (sc1: the L2 of each
// XCD is not coherent with the others'), so no L2 flush is needed; a barrier
// first waits for the wave's own stores (vmcnt 0), then counts the
// workgroup's arrival with an agent-scope atomic add. The wait is bounded
// (spin_ns of the 100 MHz real-time counter): past it, the workgroup raises
// the abort flag, every workgroup leaves, and the host reports the error.
// The last workgroup to finish sets the counters back to zero.
struct ChainOp { // the host's amdc_chain_op, resolved (amdc_host.c): 64 bytes
  u32 type;      // 0: quantize a -> b (nb blocks); 1, 2: GEMV Q4_0 / Q4_K, W a, Q8 vector b -> y;
                 // 3, 4: the same with the f32 vector b, quantized by every workgroup into its LDS;
                 // 5, 6: GEMV Q8_0 / Q6_K, W a, Q8 vector b -> y;
                 // 7: RMSNorm of a (32 nb floats) with the weights bias -> y, its Q8 copy -> b (if not NULL),
                 //    eps the float bits of pad; 8: SwiGLU y = silu(y) up a in place, its Q8 copy -> b (if not NULL)
  u32 sync;      // grid barrier after this operation
  u32 rows, nb, L, pad;
  const void *a;
  void *b;
  float *y;
  const float *bias, *res;
};
// The grid barrier. Arrivals are counted per group of workgroups
// (blockIdx.x mod NGRP, one counter per 128-byte line: few atomics on any one
// address); the last arrival of a group counts the group, the last group
// publishes the barrier's number on a line of its own, which the waiting
// workgroups poll (with a short sleep). The end of the launch is one more
// arrival, without the wait: the last one sets the counters back to zero.
// Layout of sync (u32, 128-byte lines): line g < NGRP: group g's arrivals;
// line NGRP: groups arrived; NGRP + 1: released barrier number; NGRP + 2:
// abort flag.
#define SYNC_LINE 32u
#define NGRP 32u
__device__ __forceinline__ bool chain_arrive(u32 *sync, u32 nbar) {
  const u32 grp = blockIdx.x % NGRP, gs = (gridDim.x - grp + NGRP - 1u) / NGRP, ngrp = gridDim.x < NGRP ? gridDim.x : NGRP;
  return __hip_atomic_fetch_add(sync + SYNC_LINE * grp, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == nbar * gs - 1u &&
         __hip_atomic_fetch_add(sync + SYNC_LINE * NGRP, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == nbar * ngrp - 1u;
}

__device__ __forceinline__ bool chain_barrier(u32 *sync, u32 nbar, u32 spin_ns) {
  __shared__ u32 s_ok;
  __builtin_amdgcn_s_waitcnt(0); // this wave's coherent stores are complete
  __syncthreads();
  if (threadIdx.x == 0u) {
    if (chain_arrive(sync, nbar)) __hip_atomic_store(sync + SYNC_LINE * (NGRP + 1u), nbar, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const u64 t0 = __builtin_amdgcn_s_memrealtime(), lim = spin_ns / 10u;
    u32 ok = 0;
    for (u32 it = 0;; it++) {
      if ((int)(__hip_atomic_load(sync + SYNC_LINE * (NGRP + 1u), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) - nbar) >= 0) {
        ok = 1;
        break;
      }
      if ((it & 15u) == 15u) {
        if (__hip_atomic_load(sync + SYNC_LINE * (NGRP + 2u), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) break;
        if (__builtin_amdgcn_s_memrealtime() - t0 > lim) {
          __hip_atomic_store(sync + SYNC_LINE * (NGRP + 2u), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          break;
        }
      }
      __builtin_amdgcn_s_sleep(2);
    }
    s_ok = ok;
  }
  __syncthreads();
  return s_ok != 0u;
}

// One decode GEMV of the chain: the same lane split, LDS layout and block
// arithmetic as amdc_gemv_*_p1 (bit-equal results). A workgroup's items
// (row groups blockIdx.x, + gridDim.x, ..., ceil(ng / L) super-groups per
// lane each) go in batches of CHI: all loads of a batch first (a slot past
// the last item reads row 0's first super-group again and is not used), then
// the arithmetic; it[0] of the first batch may already be loaded (pre).
#define CHI 2u
template <int KIND, bool FQ>
__device__ __forceinline__ void chain_gemv(const ChainOp &op, Item (&it)[CHI], bool pre, uint8_t *smem) {
  const uint8_t *W = (const uint8_t *)op.a, *xq = (const uint8_t *)op.b;
  const u32 rows = op.rows, nb = op.nb, L = op.L, ng = amdc_ngroups(nb), tid = threadIdx.x, lane = tid & 63u, wv = tid >> 6;
  const u32 l = lane & (L - 1u), q = lane / L, rpw = 64u / L, rpg = 4u * rpw;
  const u32 nrg = (rows + rpg - 1u) / rpg, ni = (ng + L - 1u) / L, nblk = 8u * ng;
  const u32 mine = blockIdx.x < nrg ? (nrg - blockIdx.x + gridDim.x - 1u) / gridDim.x : 0u, nit = mine * ni;
  const u64 RB = amdc_row_bytes(nb);
  u32x4 *s_lo = (u32x4 *)smem;
  u32x4 *s_hi = s_lo + nblk;
  float *s_d = (float *)(s_hi + nblk);
  u32 *s_as = (u32 *)(s_d + nblk);
  auto rowp = [&](u32 g_) {
    const u32 r_ = g_ * rpg + wv * rpw + q;
    return W + (u64)(r_ < rows ? r_ : rows - 1u) * RB;
  };
  auto load_batch = [&](u32 f0, u32 u0) {
#pragma unroll
    for (u32 u = 0; u < CHI; u++) {
      if (u < u0) continue;
      const u32 f = f0 + u, j = f / ni, i = f - j * ni;
      const bool ok = f < nit;
      load_item<KIND>(it[u], ok ? rowp(blockIdx.x + j * gridDim.x) : W, ng, l + L * i, ok && l + L * i < ng);
    }
  };
  if (nit) load_batch(0u, pre ? 1u : 0u);
  __asm__ volatile("" ::: "memory"); // the weight loads ahead of the activation loads
  if (FQ) { // the f32 vector (written by other workgroups: coherent loads), quantized as amdc_quant_q8
    const __amdgpu_buffer_rsrc_t rx = rsrc(xq, 128u * nb);
    const u32 e = tid & 7u;
    FusedQ8T<2> fq; // 2 passes of 32 blocks in flight: the chain kernel keeps 2 workgroups per CU and
                    // the next GEMV's first weights in registers
    for (u32 b0 = 0; b0 < nblk; b0 += 32u * 2u) {
#pragma unroll
      for (u32 c = 0; c < 2u; c++) {
        const u32 b = b0 + 32u * c + (tid >> 3);
        fq.xv[c] = __builtin_bit_cast(v4f, __builtin_amdgcn_raw_buffer_load_b128(rx, b < nb ? 128u * b + 16u * e : 0xFFFFFFF0u, 0, CPOL_SC1));
      }
      fq.quant(b0, nb, ng, s_lo, s_hi, s_d, s_as, nullptr);
    }
  }
  const __amdgpu_buffer_rsrc_t rq = rsrc(xq, 40u * nb);
  for (u32 j = tid; !FQ && j < nblk; j += NT) { // the Q8 vector, written by other workgroups: coherent loads
    const u32 p = (j & 7u) * ng + (j >> 3);
    u32x4 lo = (u32x4)(0u), hi = (u32x4)(0u);
    float d = 0.0f;
    u32 as = 0;
    if (j < nb) {
      lo = __builtin_amdgcn_raw_buffer_load_b128(rq, 32u * j, 0, CPOL_SC1);
      hi = __builtin_amdgcn_raw_buffer_load_b128(rq, 32u * j + 16u, 0, CPOL_SC1);
      d = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rq, 32u * nb + 4u * j, 0, CPOL_SC1));
      as = __builtin_amdgcn_raw_buffer_load_b32(rq, 36u * nb + 4u * j, 0, CPOL_SC1);
    }
    s_lo[p] = lo, s_hi[p] = hi, s_d[p] = d, s_as[p] = as;
  }
  __syncthreads();
  const __amdgpu_buffer_rsrc_t ry = rsrc(op.y, 4u * rows), rb = rsrc(op.bias, 4u * rows), rr = rsrc(op.res, 4u * rows);
  ItemTree tr;
  for (u32 f0 = 0; f0 < nit; f0 += CHI) {
    if (f0) load_batch(f0, 0u);
#pragma unroll
    for (u32 u = 0; u < CHI; u++) {
      const u32 f = f0 + u, j = f / ni, i = f - j * ni, g = l + L * i;
      if (f >= nit) break;
      const float leaf = item_dot<KIND>(it[u], g < ng ? g : 0u, ng, s_lo, s_hi, s_d, s_as, 0.0f);
      tr.add(seg_sum(g < ng ? leaf : 0.0f, L), i);
      if (i == ni - 1u) {
        const float v = tr.sum(ni);
        const u32 r = (blockIdx.x + j * gridDim.x) * rpg + wv * rpw + q;
        if (l == 0u && r < rows) {
          float o = v;
          if (op.bias) o = o + __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rb, 4u * r, 0, CPOL_SC1));
          if (op.res) o = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rr, 4u * r, 0, CPOL_SC1)) + o;
          __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(u32, o), ry, 4u * r, 0, CPOL_SC1);
        }
      }
    }
  }
  __syncthreads(); // the LDS vector is free for the next operation
}

// the quantization of op.a (nb blocks of 32 floats) into the Q8 buffer op.b,
// blocks 32 p .. 32 p + 31 by workgroup p, + 32 gridDim.x, ... (8 lanes per
// block, 4 values per lane; the arithmetic of amdc_quant_q8)
// A Q8_0 / Q6_K GEMV operation of the chain: the decode kernel's item loads
// and arithmetic (gemv2_body, the same lanes per row: bit-equal results), one
// item at a time, the Q8 vector written by other workgroups (coherent loads),
// the rows of the workgroup as the GEMV operations above; no weight preload
// before a barrier.
template <int KIND>
__device__ __forceinline__ void chain_gemv_k8(const ChainOp &op, uint8_t *smem) {
  const uint8_t *W = (const uint8_t *)op.a, *xq = (const uint8_t *)op.b;
  const u32 rows = op.rows, nb = op.nb, L = op.L, ng = amdc_ngroups(nb), tid = threadIdx.x, lane = tid & 63u, wv = tid >> 6;
  const u32 l = lane & (L - 1u), q = lane / L, rpw = 64u / L, rpg = 4u * rpw;
  const u32 nrg = (rows + rpg - 1u) / rpg, ni = (ng + L - 1u) / L, nblk = 8u * ng;
  const u32 mine = blockIdx.x < nrg ? (nrg - blockIdx.x + gridDim.x - 1u) / gridDim.x : 0u, nit = mine * ni;
  const u32 RB = (u32)amdc_row_bytes_k(KIND, nb), NR = rows * RB; // the host checks NR + RB < 2^32
  u32x4 *s_lo = (u32x4 *)smem;
  u32x4 *s_hi = s_lo + nblk;
  float *s_d = (float *)(s_hi + nblk);
  u32 *s_as = (u32 *)(s_d + nblk);
  const __amdgpu_buffer_rsrc_t rw = rsrc(W, NR);
  typename ItemOf<KIND>::type A;
  auto ld = [&](typename ItemOf<KIND>::type &it, u32 f) {
    const u32 j = f / ni, i = f - j * ni, g = l + L * i, r = (blockIdx.x + j * gridDim.x) * rpg + wv * rpw + q;
    item_load<KIND, 0>(it, rw, f < nit && g < ng && r < rows ? r * RB : NR, g, ng);
  };
  if (nit) ld(A, 0u);
  __asm__ volatile("" ::: "memory"); // the weight loads ahead of the activation loads
  const __amdgpu_buffer_rsrc_t rq = rsrc(xq, 40u * nb);
  for (u32 j = tid; j < nblk; j += NT) { // the Q8 vector, written by other workgroups: coherent loads
    const u32 p = (j & 7u) * ng + (j >> 3);
    u32x4 lo = (u32x4)(0u), hi = (u32x4)(0u);
    float d = 0.0f;
    if (j < nb) {
      lo = __builtin_amdgcn_raw_buffer_load_b128(rq, 32u * j, 0, CPOL_SC1);
      hi = __builtin_amdgcn_raw_buffer_load_b128(rq, 32u * j + 16u, 0, CPOL_SC1);
      d = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rq, 32u * nb + 4u * j, 0, CPOL_SC1));
    }
    s_lo[p] = lo, s_hi[p] = hi, s_d[p] = d;
    if constexpr (KIND == AMDC_Q6_K) // 32 x the sum of each half of the block, as gemv2_body stages it
      ((u32x2 *)s_as)[p] = (u32x2){32u * (u32)hsum16(lo), 32u * (u32)hsum16(hi)};
  }
  __syncthreads();
  const __amdgpu_buffer_rsrc_t ry = rsrc(op.y, 4u * rows), rb = rsrc(op.bias, 4u * rows), rr = rsrc(op.res, 4u * rows);
  ItemTree tr;
  auto comp = [&](const typename ItemOf<KIND>::type &it, u32 f) {
    const u32 j = f / ni, i = f - j * ni, g = l + L * i;
    const float leaf = item_dot<KIND>(it, g < ng ? g : 0u, ng, s_lo, s_hi, s_d, s_as, 0.0f);
    tr.add(seg_sum(g < ng ? leaf : 0.0f, L), i);
    if (i == ni - 1u) {
      const float v = tr.sum(ni);
      const u32 r = (blockIdx.x + j * gridDim.x) * rpg + wv * rpw + q;
      if (l == 0u && r < rows) {
        float o = v;
        if (op.bias) o = o + __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rb, 4u * r, 0, CPOL_SC1));
        if (op.res) o = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rr, 4u * r, 0, CPOL_SC1)) + o;
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(u32, o), ry, 4u * r, 0, CPOL_SC1);
      }
    }
  };
  for (u32 f = 0; f < nit; f++) { // one item at a time (the chain kernel's registers hold no second Q8_0 item)
    comp(A, f);
    if (f + 1u < nit) ld(A, f + 1u);
  }
  __syncthreads(); // the LDS vector is free for the next operation
}

// The Q8 producers as chain operations: amdc_rmsnorm_q8 / amdc_swiglu_q8 of one token (the same device
// code: bit-equal), every workgroup taking blocks of 8 (RMSNorm: each first computes the whole scale,
// as every workgroup of the separate launch does), inputs and outputs agent-coherent.
__device__ __forceinline__ void chain_rmsnorm(const ChainOp &op) {
  __shared__ float s_ss[4];
  const u32 nb = op.nb, n = 32u * nb, tid = threadIdx.x;
  const float *x = (const float *)op.a, *w = op.bias;
  const float s = rms_scale<true, 2u>(x, n, __builtin_bit_cast(float, op.pad), s_ss);
  const __amdgpu_buffer_rsrc_t rx = rsrc(x, 4u * n), rw = rsrc(w, 4u * n), ry = rsrc(op.y, 4u * n);
  for (u32 b0 = 8u * blockIdx.x; b0 < nb; b0 += 8u * gridDim.x) {
    const u32 b = b0 + (tid >> 5);
    if (b < nb) { // whole 32-lane halves
      const u32 i = 32u * b + (tid & 31u);
      const float v = ldf<true>(x, rx, i) * s * ldf<true>(w, rw, i);
      __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(u32, v), ry, 4u * i, 0, CPOL_SC1);
      if (op.b) quant_half<true>(v, b, (uint8_t *)op.b, nb);
    }
  }
}
__device__ __forceinline__ void chain_swiglu(const ChainOp &op) {
  const u32 nb = op.nb, n = 32u * nb;
  const float *u = (const float *)op.a;
  const __amdgpu_buffer_rsrc_t rg = rsrc(op.y, 4u * n), ru = rsrc(u, 4u * n);
  for (u32 i0 = NT * blockIdx.x; i0 < n; i0 += NT * gridDim.x) {
    const u32 i = i0 + threadIdx.x;
    if (i < n) { // n is a multiple of 32: whole halves
      const float v = swiglu1(ldf<true>(op.y, rg, i), ldf<true>(u, ru, i));
      __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(u32, v), rg, 4u * i, 0, CPOL_SC1);
      if (op.b) quant_half<true>(v, i >> 5, (uint8_t *)op.b, nb);
    }
  }
}

__device__ __forceinline__ void chain_quant(const ChainOp &op) {
  const u32 nb = op.nb, tid = threadIdx.x, e = tid & 7u;
  const __amdgpu_buffer_rsrc_t rx = rsrc(op.a, 128u * nb), rq = rsrc(op.b, 40u * nb);
  for (u32 b0 = 32u * blockIdx.x; b0 < nb; b0 += 32u * gridDim.x) {
    const u32 b = b0 + (tid >> 3);
    const v4f v = __builtin_bit_cast(v4f, __builtin_amdgcn_raw_buffer_load_b128(rx, b < nb ? 128u * b + 16u * e : 0xFFFFFFF0u, 0, CPOL_SC1));
    float a = __builtin_fmaxf(__builtin_fmaxf(__builtin_fabsf(v.x), __builtin_fabsf(v.y)), __builtin_fmaxf(__builtin_fabsf(v.z), __builtin_fabsf(v.w)));
    a = __builtin_fmaxf(a, dpp<0xB1>(a));
    a = __builtin_fmaxf(a, dpp<0x4E>(a));
    a = __builtin_fmaxf(a, dpp<0x141>(a));
    const float d = a / 127.0f;
    int qi[4];
    q8_round4(v, d, qi);
    const u32 word = (u32)(qi[0] & 255) | (u32)(qi[1] & 255) << 8 | (u32)(qi[2] & 255) << 16 | (u32)qi[3] << 24;
    u32 sum = (u32)qi[0] + (u32)qi[1] + (u32)qi[2] + (u32)qi[3];
    sum += (u32)__builtin_amdgcn_update_dpp(0, (int)sum, 0xB1, 0xF, 0xF, false);
    sum += (u32)__builtin_amdgcn_update_dpp(0, (int)sum, 0x4E, 0xF, 0xF, false);
    sum += (u32)__builtin_amdgcn_update_dpp(0, (int)sum, 0x141, 0xF, 0xF, false);
    if (b < nb) {
      __builtin_amdgcn_raw_buffer_store_b32(word, rq, 32u * b + 4u * e, 0, CPOL_SC1);
      if (e == 0u) {
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(u32, d), rq, 32u * nb + 4u * b, 0, CPOL_SC1);
        __builtin_amdgcn_raw_buffer_store_b32(sum, rq, 36u * nb + 4u * b, 0, CPOL_SC1);
      }
    }
  }
}

// the first item of op (a GEMV) for this workgroup, loaded ahead (false if it has none)
__device__ __forceinline__ bool chain_preload(const ChainOp &op, Item &cur) {
  const u32 L = op.L, ng = amdc_ngroups(op.nb), lane = threadIdx.x & 63u, wv = threadIdx.x >> 6;
  const u32 l = lane & (L - 1u), q = lane / L, rpw = 64u / L, rpg = 4u * rpw, nrg = (op.rows + rpg - 1u) / rpg;
  if (blockIdx.x >= nrg || op.type > 4u) return false; // Q8_0 / Q6_K operations load their own first items
  const u32 r = blockIdx.x * rpg + wv * rpw + q;
  const uint8_t *wr = (const uint8_t *)op.a + (u64)(r < op.rows ? r : op.rows - 1u) * amdc_row_bytes(op.nb);
  if (op.type == 1u || op.type == 3u) load_item<AMDC_Q4_0>(cur, wr, ng, l, l < ng);
  else load_item<AMDC_Q4_K>(cur, wr, ng, l, l < ng);
  return true;
}

extern "C" __global__ __launch_bounds__(256, 2) void amdc_chain(const ChainOp *__restrict__ ops, u32 n, u32 *sync, u32 spin_ns) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  u32 nbar = 0, pre = 0xFFFFFFFFu; // pre: the operation whose first item it[0] holds
  Item it[CHI];
  for (u32 k = 0; k < n; k++) {
    const ChainOp op = ops[k];
    if (op.type == 0u) chain_quant(op);
    else if (op.type == 1u) chain_gemv<AMDC_Q4_0, false>(op, it, pre == k, smem);
    else if (op.type == 2u) chain_gemv<AMDC_Q4_K, false>(op, it, pre == k, smem);
    else if (op.type == 3u) chain_gemv<AMDC_Q4_0, true>(op, it, pre == k, smem);
    else if (op.type == 4u) chain_gemv<AMDC_Q4_K, true>(op, it, pre == k, smem);
    else if (op.type == 5u) chain_gemv_k8<AMDC_Q8_0>(op, smem);
    else if (op.type == 6u) chain_gemv_k8<AMDC_Q6_K>(op, smem);
    else if (op.type == 7u) chain_rmsnorm(op);
    else chain_swiglu(op);
    if (op.sync && k + 1u < n) {
      // the next GEMV's first weights go out before the wait (quantizations and producers between do
      // not touch it[])
      u32 j = k + 1u;
      while (j < n && (ops[j].type == 0u || ops[j].type >= 7u)) j++;
      if (j < n && pre != j && chain_preload(ops[j], it[0])) pre = j;
      nbar++;
      if (!chain_barrier(sync, nbar, spin_ns)) break;
    }
  }
  // the end: one more arrival; the last one sets the counters back to zero
  // (not the abort flag: the host reads it)
  __syncthreads();
  if (threadIdx.x == 0u && chain_arrive(sync, nbar + 1u)) {
    for (u32 g = 0; g < NGRP + 2u; g++) __hip_atomic_store(sync + SYNC_LINE * g, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// ------------------------------------------------------------------ the streaming chain

// The GEMV chain, streaming form (amdc_chain_s_q4_0 / _q4_k: every GEMV of
// the list of one kind): one workgroup of 768 threads per CU, in two roles.
// - 8 compute waves issue nothing but weight loads. Wave gw = 8 blockIdx.x +
//   (wave - 4) of the GW = 8 gridDim.x compute waves takes the wave row
//   groups (64 / L rows each) gw, gw + GW, ... of every GEMV, each as
//   ceil(ng / L) items of one super-group per lane (the decode kernels' lane
//   split, block arithmetic and summation order: bit-equal results). A wave
//   keeps NBUF item buffers (2 for Q4_0, 3 for Q4_K, as the registers allow):
//   right after it computes an item it loads the next one of its sequence
//   into the freed buffer, whichever operation that item belongs to, so while
//   the workgroup passes an operation boundary the weights of the next NBUF
//   items of every compute wave are in flight. Row results go to the LDS.
// - 4 staging waves do the rest: they write the workgroup's results of an
//   operation to memory (with bias and residual), take part in the grid
//   barrier, quantize or load the next operation's vector into the LDS, and
//   run the quantize operations.
// A wave's vector memory operations complete in issue order; with the roles
// apart, no barrier poll, vector load or output store waits behind weight
// loads. The operation list is copied to the LDS once (the compute waves'
// cursors read it there). Outputs and the vectors between operations are
// coherent (sc1) accesses, as in amdc_chain.
#define CS_NS 4u // staging waves per workgroup
#define CS_NC 8u // compute waves per workgroup

__device__ __forceinline__ bool chain_wait(u32 *sync, u32 nbar, u32 spin_ns) {
  const u64 t0 = __builtin_amdgcn_s_memrealtime(), lim = spin_ns / 10u;
  for (u32 it = 0;; it++) {
    if ((int)(__hip_atomic_load(sync + SYNC_LINE * (NGRP + 1u), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) - nbar) >= 0) return true;
    if ((it & 15u) == 15u) {
      if (__hip_atomic_load(sync + SYNC_LINE * (NGRP + 2u), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) return false;
      if (__builtin_amdgcn_s_memrealtime() - t0 > lim) {
        __hip_atomic_store(sync + SYNC_LINE * (NGRP + 2u), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return false;
      }
    }
    __builtin_amdgcn_s_sleep(1);
  }
}

// The per-operation values of a GEMV of the streaming chain for one compute wave.
struct CsOp {
  const uint8_t *W;
  u64 RB;
  u32 rows, nb, ng, L, ni, rpw, nwr, nit;
};
__device__ __forceinline__ CsOp cs_op(const ChainOp &op, u32 gw, u32 GW) {
  CsOp c;
  c.W = (const uint8_t *)op.a, c.rows = op.rows, c.nb = op.nb, c.ng = amdc_ngroups(op.nb), c.L = op.L ? op.L : 64u; // L = 0: a quantization
  c.RB = amdc_row_bytes(op.nb), c.ni = (c.ng + c.L - 1u) / c.L, c.rpw = 64u / c.L;
  c.nwr = (c.rows + c.rpw - 1u) / c.rpw; // wave row groups
  c.nit = op.type >= 1u && op.type <= 4u && gw < c.nwr ? (c.nwr - gw + GW - 1u) / GW * c.ni : 0u;
  return c;
}

// An operation of the list, read through the constant address space: scalar
// loads (counted apart from the vector memory operations, so that reading the
// list never waits for weight loads), every word uniform.
typedef const __attribute__((address_space(4))) ChainOp *cops_t;
__device__ __forceinline__ ChainOp ld_op(cops_t p) { return *p; }

// The load cursor of a compute wave: operation kl, its item fl (of cl.nit
// items), ahead of the computation. Once the wave's sequence is done it loads
// its last item again (unused), so that every call issues the same 9 loads
// and no load is under a branch.
struct CsCursor {
  cops_t ops;
  u32 n, gw, GW, kl, fl;
  CsOp cl;
  // the first item at or after operation k (false: none)
  __device__ __forceinline__ bool seek(u32 k) {
    for (; k < n; k++) {
      const CsOp c = cs_op(ld_op(ops + k), gw, GW);
      if (c.nit) {
        cl = c, kl = k, fl = 0;
        return true;
      }
    }
    return false;
  }
  // the host puts a GEMV operation in every streaming chain: a wave without
  // items loads (clamped) addresses of the first one
  __device__ __forceinline__ void init(cops_t o, u32 n_, u32 gw_, u32 GW_) {
    ops = o, n = n_, gw = gw_, GW = GW_, kl = n, fl = 0;
    if (!seek(0)) {
      u32 k = 0;
      while (k + 1u < n && (ld_op(ops + k).type < 1u || ld_op(ops + k).type > 4u)) k++;
      cl = cs_op(ld_op(ops + k), gw, GW);
    }
  }
  // the next item of the sequence into it
  __device__ __forceinline__ void issue(Item &it) {
    typedef const __attribute__((address_space(1))) u32x4 *gp;
    const u32 lane = threadIdx.x & 63u, j = fl / cl.ni, i = fl - j * cl.ni, l = lane & (cl.L - 1u), q = lane / cl.L, g = l + cl.L * i;
    const u32 r = (gw + GW * j) * cl.rpw + q, gg = g < cl.ng ? g : 0u;
    const uint8_t *wr = cl.W + (u64)(r < cl.rows ? r : cl.rows - 1u) * cl.RB;
    it.h = __builtin_nontemporal_load((gp)(wr + amdc_header_off(gg))); // the loads of load_item, as global (not flat) accesses
#pragma unroll
    for (u32 kk = 0; kk < 8u; kk++) it.n[kk] = __builtin_nontemporal_load((gp)(wr + amdc_nib_off(cl.ng, gg, kk)));
    if (kl < n && ++fl == cl.nit) {
      const CsOp keep = cl;
      fl--;
      if (!seek(kl + 1u)) kl = n, cl = keep; // done: the last item again
    }
  }
};

// The quantization of nb blocks of the f32 vector op.a into the Q8 buffer
// op.b, blocks b0 + 32 p .. by the staging threads of workgroup p (the
// arithmetic of amdc_quant_q8).
__device__ __forceinline__ void cs_quant_op(const ChainOp &op, u32 t) {
  const u32 nb = op.nb, e = t & 7u;
  const __amdgpu_buffer_rsrc_t rx = rsrc(op.a, 128u * nb), rq = rsrc(op.b, 40u * nb);
  for (u32 b0 = 32u * blockIdx.x; b0 < nb; b0 += 32u * gridDim.x) {
    const u32 b = b0 + (t >> 3);
    const v4f v = __builtin_bit_cast(v4f, __builtin_amdgcn_raw_buffer_load_b128(rx, b < nb ? 128u * b + 16u * e : 0xFFFFFFF0u, 0, CPOL_SC1));
    float a = __builtin_fmaxf(__builtin_fmaxf(__builtin_fabsf(v.x), __builtin_fabsf(v.y)), __builtin_fmaxf(__builtin_fabsf(v.z), __builtin_fabsf(v.w)));
    a = __builtin_fmaxf(a, dpp<0xB1>(a));
    a = __builtin_fmaxf(a, dpp<0x4E>(a));
    a = __builtin_fmaxf(a, dpp<0x141>(a));
    const float d = a / 127.0f;
    int qi[4];
    q8_round4(v, d, qi);
    const u32 word = (u32)(qi[0] & 255) | (u32)(qi[1] & 255) << 8 | (u32)(qi[2] & 255) << 16 | (u32)qi[3] << 24;
    u32 sum = (u32)qi[0] + (u32)qi[1] + (u32)qi[2] + (u32)qi[3];
    sum += (u32)__builtin_amdgcn_update_dpp(0, (int)sum, 0xB1, 0xF, 0xF, false);
    sum += (u32)__builtin_amdgcn_update_dpp(0, (int)sum, 0x4E, 0xF, 0xF, false);
    sum += (u32)__builtin_amdgcn_update_dpp(0, (int)sum, 0x141, 0xF, 0xF, false);
    if (b < nb) {
      __builtin_amdgcn_raw_buffer_store_b32(word, rq, 32u * b + 4u * e, 0, CPOL_SC1);
      if (e == 0u) {
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(u32, d), rq, 32u * nb + 4u * b, 0, CPOL_SC1);
        __builtin_amdgcn_raw_buffer_store_b32(sum, rq, 36u * nb + 4u * b, 0, CPOL_SC1);
      }
    }
  }
}

// The vector of GEMV operation op, by the staging threads (t < 256): a Q8
// vector into the LDS (vec), permuted as the weights; an f32 vector raw into
// the LDS (xr, 128 nb bytes), up to 16 loads of 16 bytes per thread in
// flight at once, for cs_quant_lds.
__device__ __forceinline__ void cs_stage(const ChainOp &op, u32 t, uint8_t *vec, float *xr) {
  const u32 nb = op.nb, ng = amdc_ngroups(nb), nblk = 8u * ng;
  if (op.type >= 3u) {
    constexpr u32 NL = 16u;
    const __amdgpu_buffer_rsrc_t rx = rsrc(op.b, 128u * nb);
    const u32 nw = 8u * nb; // 16-byte words
    for (u32 w0 = 0; w0 < nw; w0 += 256u * NL) {
      u32x4 v[NL];
#pragma unroll
      for (u32 i = 0; i < NL; i++) {
        const u32 wi = w0 + 256u * i + t;
        v[i] = __builtin_amdgcn_raw_buffer_load_b128(rx, wi < nw ? 16u * wi : 0xFFFFFFF0u, 0, CPOL_SC1);
      }
#pragma unroll
      for (u32 i = 0; i < NL; i++) {
        const u32 wi = w0 + 256u * i + t;
        if (wi < nw) ((u32x4 *)xr)[wi] = v[i];
      }
    }
    return;
  }
  u32x4 *s_lo = (u32x4 *)vec, *s_hi = s_lo + nblk;
  float *s_d = (float *)(s_hi + nblk);
  u32 *s_as = (u32 *)(s_d + nblk);
  const __amdgpu_buffer_rsrc_t rq = rsrc(op.b, 40u * nb);
  for (u32 j = t; j < nblk; j += 256u) {
    const u32 p = (j & 7u) * ng + (j >> 3);
    const bool in = j < nb;
    s_lo[p] = __builtin_amdgcn_raw_buffer_load_b128(rq, in ? 32u * j : 0xFFFFFFF0u, 0, CPOL_SC1);
    s_hi[p] = __builtin_amdgcn_raw_buffer_load_b128(rq, in ? 32u * j + 16u : 0xFFFFFFF0u, 0, CPOL_SC1);
    s_d[p] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rq, in ? 32u * nb + 4u * j : 0xFFFFFFF0u, 0, CPOL_SC1));
    s_as[p] = __builtin_amdgcn_raw_buffer_load_b32(rq, in ? 36u * nb + 4u * j : 0xFFFFFFF0u, 0, CPOL_SC1);
  }
}

// The quantization of the raw f32 vector xr (nb blocks) into vec, by all NT_
// threads of the workgroup (the arithmetic of amdc_quant_q8 and FusedQ8T: 8
// lanes per block, blocks past nb up to the super-group end are zeros).
template <u32 NT_>
__device__ __forceinline__ void cs_quant_lds(const float *xr, u32 nb, uint8_t *vec) {
  const u32 ng = amdc_ngroups(nb), nblk = 8u * ng, tid = threadIdx.x, e = tid & 7u;
  u32x4 *s_lo = (u32x4 *)vec, *s_hi = s_lo + nblk;
  float *s_d = (float *)(s_hi + nblk);
  u32 *s_as = (u32 *)(s_d + nblk);
  for (u32 b0 = 0; b0 < nblk; b0 += NT_ / 8u) {
    const u32 b = b0 + (tid >> 3);
    const v4f x = b < nb ? ((const v4f *)xr)[8u * b + e] : (v4f){0.0f, 0.0f, 0.0f, 0.0f};
    float a = __builtin_fmaxf(__builtin_fmaxf(__builtin_fabsf(x.x), __builtin_fabsf(x.y)), __builtin_fmaxf(__builtin_fabsf(x.z), __builtin_fabsf(x.w)));
    a = __builtin_fmaxf(a, dpp<0xB1>(a));
    a = __builtin_fmaxf(a, dpp<0x4E>(a));
    a = __builtin_fmaxf(a, dpp<0x141>(a));
    const float d = a / 127.0f;
    int qi[4];
    q8_round4(x, d, qi);
    const u32 word = (u32)(qi[0] & 255) | (u32)(qi[1] & 255) << 8 | (u32)(qi[2] & 255) << 16 | (u32)qi[3] << 24;
    u32 sum = (u32)qi[0] + (u32)qi[1] + (u32)qi[2] + (u32)qi[3];
    sum += (u32)__builtin_amdgcn_update_dpp(0, (int)sum, 0xB1, 0xF, 0xF, false);
    sum += (u32)__builtin_amdgcn_update_dpp(0, (int)sum, 0x4E, 0xF, 0xF, false);
    sum += (u32)__builtin_amdgcn_update_dpp(0, (int)sum, 0x141, 0xF, 0xF, false);
    if (b < nblk) {
      const u32 p = (b & 7u) * ng + (b >> 3);
      ((u32 *)(e < 4u ? &s_lo[p] : &s_hi[p]))[e & 3u] = word;
      if (e == 0u) s_d[p] = d, s_as[p] = sum;
    }
  }
}

// LDS: the results of the workgroup's rows of one operation (outb bytes:
// compute wave w, its row group j, row q at float (w mj + j) rpw + q, mj =
// the most row groups of a compute wave), the vector (vecb bytes: the
// staged Q8 vector), then the raw f32 vector of an f32-input operation. Every operation boundary is four workgroup barriers, met by every
// wave in the same order (a compute wave may meet them after either of its
// buffers): B1 the compute waves' results of operation k are in the LDS; Bw
// the staging waves' stores of them are complete; Br the grid barrier has
// passed (thread 0); Bx the next operation's vector (raw f32 or Q8) is in the
// LDS; B2 it is quantized (all waves quantize an f32 vector between Bx and
// B2). After the last operation only B1.
// Each workgroup arrives once more after its last grid barrier (the last
// arrival sets the counters back to zero, while the last operation runs).
// trace (or NULL): per workgroup 2 + 4 n + 64 words of the 100 MHz clock:
// the start, B2 of the start, B1 Bw Br B2 of each operation (thread 0), then
// the time each of the first 64 items of the first compute wave is computed.
template <int KIND, u32 NBUF>
__device__ __forceinline__ void chain_s_body(const ChainOp *__restrict__ gops, u32 n, u32 *sync, u32 spin_ns, u32 outb, u32 vecb,
                                             u64 *trace) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  __shared__ u32 s_ok;
  const cops_t ops = (cops_t)gops;
  float *outs = (float *)smem;
  uint8_t *vec = smem + outb;
  float *xr = (float *)(smem + outb + vecb);
  constexpr u32 NT_ = (CS_NS + CS_NC) * 64u;
  const u32 tid = threadIdx.x, lane = tid & 63u, wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const u32 GW = CS_NC * gridDim.x;
  u64 *tr0 = trace ? trace + (u64)blockIdx.x * (2u + 4u * n + 64u) : nullptr;
  if (tr0 && tid == 0u) tr0[0] = __builtin_amdgcn_s_memrealtime();
  if (tid == 0u) s_ok = 1u;
  u32 nsync = 0; // grid barriers in the list
  for (u32 k = 0; k + 1u < n; k++) nsync += ld_op(ops + k).sync ? 1u : 0u;
  u32 nbar = 0;
  if (wv >= CS_NS) { // ---------------- a compute wave
    const u32 w = wv - CS_NS, gw = CS_NC * blockIdx.x + w;
    CsCursor cur;
    cur.init(ops, n, gw, GW);
    Item A, B, C; // C: the third buffer (NBUF 3)
    cur.issue(A);
    cur.issue(B);
    if (NBUF == 3) cur.issue(C);
    __syncthreads(); // Bx of the start
    if (ld_op(ops).type >= 3u) cs_quant_lds<NT_>(xr, ld_op(ops).nb, vec);
    __syncthreads(); // B2 of the start: operation 0's vector
    u32 nt_ = 0;      // items computed (trace)
    u32 k = 0, f = 0;
    CsOp c = cs_op(ld_op(ops), gw, GW);
    bool live = s_ok != 0u;
    // past the operation boundaries this wave has reached; false when the list is done or aborted
    auto next = [&]() {
      while (live && f == c.nit) {
        __syncthreads(); // B1
        if (k + 1u == n) { // the last operation: the staging waves write the results and end
          live = false;
          break;
        }
        __syncthreads(); // Bw
        __syncthreads(); // Br
        __syncthreads(); // Bx
        live = s_ok != 0u && ++k < n;
        if (live) {
          const ChainOp nx = ld_op(ops + k);
          if (nx.type >= 3u) cs_quant_lds<NT_>(xr, nx.nb, vec);
        }
        __syncthreads(); // B2
        if (live) c = cs_op(ld_op(ops + k), gw, GW), f = 0;
      }
      return live;
    };
    ItemTree tr;
    auto step = [&](Item &it) {
      const u32 ng = c.ng, nblk = 8u * ng, L = c.L, l = lane & (L - 1u), q = lane / L, ni = c.ni;
      const u32x4 *s_lo = (const u32x4 *)vec, *s_hi = s_lo + nblk;
      const float *s_d = (const float *)(s_hi + nblk);
      const u32 *s_as = (const u32 *)(s_d + nblk);
      const u32 j = f / ni, i = f - j * ni, g = l + L * i, mj = (c.nwr + GW - 1u) / GW;
      const float leaf = item_dot<KIND>(it, g < ng ? g : 0u, ng, s_lo, s_hi, s_d, s_as, 0.0f);
      tr.add(seg_sum(g < ng ? leaf : 0.0f, L), i);
      if (i == ni - 1u && l == 0u) outs[(w * mj + j) * c.rpw + q] = tr.sum(ni);
      if (tr0 && w == 0u && lane == 0u && nt_ < 64u) tr0[2u + 4u * n + nt_] = __builtin_amdgcn_s_memrealtime();
      nt_++;
      cur.issue(it);
      f++;
    };
    for (;;) {
      if (!next()) break;
      step(A);
      if (!next()) break;
      step(B);
      if (NBUF == 3) {
        if (!next()) break;
        step(C);
      }
    }
    return;
  }
  // ---------------- a staging wave (threads tid < 256)
  {
    const ChainOp op = ld_op(ops);
    if (op.type == 0u) cs_quant_op(op, tid);
    else cs_stage(op, tid, vec, xr);
  }
  __syncthreads(); // Bx of the start
  if (ld_op(ops).type >= 3u) cs_quant_lds<NT_>(xr, ld_op(ops).nb, vec);
  __syncthreads(); // B2 of the start
  auto stamp = [&](u32 i) {
    if (tr0 && tid == 0u) tr0[i] = __builtin_amdgcn_s_memrealtime();
  };
  stamp(1u);
  if (nsync == 0u && tid == 0u && chain_arrive(sync, 1u)) // no grid barrier: the end's arrival now
    for (u32 g = 0; g < NGRP + 2u; g++) __hip_atomic_store(sync + SYNC_LINE * g, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  for (u32 k = 0; k < n; k++) {
    const ChainOp op = ld_op(ops + k);
    const CsOp c = cs_op(op, 0u, GW);
    __syncthreads(); // B1
    stamp(2u + 4u * k);
    if (op.type != 0u) { // the workgroup's results of operation k
      const __amdgpu_buffer_rsrc_t ry = rsrc(op.y, 4u * c.rows), rb = rsrc(op.bias, 4u * c.rows), rr = rsrc(op.res, 4u * c.rows);
      const u32 mj = (c.nwr + GW - 1u) / GW, per = mj * c.rpw;
      for (u32 s = tid; s < CS_NC * per; s += CS_NS * 64u) {
        const u32 ww = s / per, j = (s - ww * per) / c.rpw, q = s - ww * per - j * c.rpw;
        const u32 r = ((CS_NC * blockIdx.x + ww) + GW * j) * c.rpw + q;
        if (r < c.rows) {
          float o = outs[s];
          if (op.bias) o = o + __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rb, 4u * r, 0, CPOL_SC1));
          if (op.res) o = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rr, 4u * r, 0, CPOL_SC1)) + o;
          __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(u32, o), ry, 4u * r, 0, CPOL_SC1);
        }
      }
    }
    if (k + 1u == n) break; // the end: the stores complete with the launch
    __builtin_amdgcn_s_waitcnt(0); // this wave's stores (results, quantizations) are complete
    __syncthreads();               // Bw: ... and those of the other staging waves
    stamp(3u + 4u * k);
    if (tid == 0u && op.sync) {
      nbar++;
      if (chain_arrive(sync, nbar)) __hip_atomic_store(sync + SYNC_LINE * (NGRP + 1u), nbar, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      s_ok = chain_wait(sync, nbar, spin_ns) ? 1u : 0u;
      // after the last grid barrier, the end's arrival (the last one sets the counters back to zero)
      if (s_ok && nbar == nsync && chain_arrive(sync, nbar + 1u))
        for (u32 g = 0; g < NGRP + 2u; g++) __hip_atomic_store(sync + SYNC_LINE * g, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads(); // Br
    stamp(4u + 4u * k);
    const bool live = s_ok != 0u;
    const ChainOp nx = ld_op(ops + k + 1u);
    if (live) {
      if (nx.type == 0u) cs_quant_op(nx, tid);
      else cs_stage(nx, tid, vec, xr);
    }
    __syncthreads(); // Bx
    if (live && nx.type >= 3u) cs_quant_lds<NT_>(xr, nx.nb, vec);
    __syncthreads(); // B2
    stamp(5u + 4u * k);
    if (!live) break;
  }
  // an aborted launch leaves the counters as they are: the host reads them
}

extern "C" __global__ __launch_bounds__(768, 1) void amdc_chain_s_q4_0(const ChainOp *__restrict__ ops, u32 n, u32 *sync, u32 spin_ns, u32 outb,
                                                                       u32 vecb, u64 *trace) {
  chain_s_body<AMDC_Q4_0, 2u>(ops, n, sync, spin_ns, outb, vecb, trace);
}
extern "C" __global__ __launch_bounds__(768, 1) void amdc_chain_s_q4_k(const ChainOp *__restrict__ ops, u32 n, u32 *sync, u32 spin_ns, u32 outb,
                                                                       u32 vecb, u64 *trace) {
  chain_s_body<AMDC_Q4_K, 3u>(ops, n, sync, spin_ns, outb, vecb, trace);
}

// ------------------------------------------------------------------ bandwidth probes

// Plain streaming kernels of known traffic, the yardsticks of the GEMV: read
// n 16-byte words (a grid-stride loop, 4 loads in flight per lane, the xor
// of all words stored per workgroup) and copy n 16-byte words.
extern "C" __global__ __launch_bounds__(256) void amdc_probe_read(const u32x4 *__restrict__ src, u64 n, u32 *__restrict__ out) {
  u32x4 a = (u32x4)(0u);
  const u64 stride = (u64)gridDim.x * NT;
  u64 i = (u64)blockIdx.x * NT + threadIdx.x;
  for (; i + 3u * stride < n; i += 4u * stride) {
    const u32x4 v0 = __builtin_nontemporal_load(src + i), v1 = __builtin_nontemporal_load(src + i + stride);
    const u32x4 v2 = __builtin_nontemporal_load(src + i + 2u * stride), v3 = __builtin_nontemporal_load(src + i + 3u * stride);
    a ^= v0 ^ v1 ^ v2 ^ v3;
  }
  for (; i < n; i += stride) a ^= src[i];
  const u32 x = a.x ^ a.y ^ a.z ^ a.w;
  if (x == 0x9E3779B9u) out[blockIdx.x] = x; // practically never: keeps the loads
}
extern "C" __global__ __launch_bounds__(256) void amdc_probe_copy(const u32x4 *__restrict__ src, u32x4 *__restrict__ dst, u64 n) {
  const u64 stride = (u64)gridDim.x * NT;
  for (u64 i = (u64)blockIdx.x * NT + threadIdx.x; i < n; i += stride) dst[i] = src[i];
}

// ------------------------------------------------------------------ block dots (parity)

// out[r * nb + b] = the int32 dot of block b of row r with Q8 block b:
// Q4_0 sum (q - 8) a (ie_q4q8_block), Q4_K sum q a (ie_q4k_dot), computed by
// nib_dot as in the GEMV kernels. One thread per block.
template <int KIND>
__device__ __forceinline__ void dots_body(const uint8_t *W, const uint8_t *xq, int *out, u32 rows, u32 nb) {
  const u64 i = (u64)blockIdx.x * NT + threadIdx.x;
  if (i >= (u64)rows * nb) return;
  const u32 r = (u32)(i / nb), b = (u32)(i - (u64)r * nb), ng = amdc_ngroups(nb);
  const u32x4 w = *(const u32x4 *)(W + (u64)r * amdc_row_bytes(nb) + amdc_nib_off(ng, b >> 3, b & 7u));
  const u32x4 lo = *(const u32x4 *)(xq + 32u * b), hi = *(const u32x4 *)(xq + 32u * b + 16u);
  const int dq = nib_dot(w, lo, hi);
  out[i] = KIND == AMDC_Q4_0 ? (int)((u32)dq - 8u * ((const u32 *)(xq + 36u * nb))[b]) : dq;
}
extern "C" __global__ __launch_bounds__(256) void amdc_dots_q4_0(const uint8_t *W, const uint8_t *xq, int *out, u32 rows, u32 nb) {
  dots_body<AMDC_Q4_0>(W, xq, out, rows, nb);
}
extern "C" __global__ __launch_bounds__(256) void amdc_dots_q4_k(const uint8_t *W, const uint8_t *xq, int *out, u32 rows, u32 nb) {
  dots_body<AMDC_Q4_K>(W, xq, out, rows, nb);
}
// Q8_0: out[r * nb + b] = sum q a (ie_q8q8_block). Q6_K: out[(r * nb + b) * 2
// + h] = sum over half h of (q - 32) a (ie_q6k_dots), by the integer steps
// of the GEMV (q8_dot, q6k_dots, hsum16). One thread per block.
extern "C" __global__ __launch_bounds__(256) void amdc_dots_q8_0(const uint8_t *W, const uint8_t *xq, int *out, u32 rows, u32 nb) {
  const u64 i = (u64)blockIdx.x * NT + threadIdx.x;
  if (i >= (u64)rows * nb) return;
  const u32 r = (u32)(i / nb), b = (u32)(i - (u64)r * nb), ng = amdc_ngroups(nb);
  const uint8_t *wr = W + (u64)r * amdc_q8_row_bytes(nb);
  const u32x4 w0 = *(const u32x4 *)(wr + amdc_q8_off(ng, b >> 3, 2u * (b & 7u)));
  const u32x4 w1 = *(const u32x4 *)(wr + amdc_q8_off(ng, b >> 3, 2u * (b & 7u) + 1u));
  const u32x4 lo = *(const u32x4 *)(xq + 32u * b), hi = *(const u32x4 *)(xq + 32u * b + 16u);
  const int dq = q8_dot(w0, w1, lo, hi);
  out[i] = dq;
}
extern "C" __global__ __launch_bounds__(256) void amdc_dots_q6_k(const uint8_t *W, const uint8_t *xq, int *out, u32 rows, u32 nb) {
  const u64 i = (u64)blockIdx.x * NT + threadIdx.x;
  if (i >= (u64)rows * nb) return;
  const u32 r = (u32)(i / nb), b = (u32)(i - (u64)r * nb), ng = nb / 8u, k = b & 7u;
  const uint8_t *wr = W + (u64)r * amdc_q6k_row_bytes(nb);
  const u32x4 nw = *(const u32x4 *)(wr + amdc_q6k_nib_off(ng, b >> 3, k));
  const u32x2 hw = *(const u32x2 *)(wr + amdc_q6k_hi_off(ng, b >> 3, k >> 1) + 8u * (k & 1u));
  const u32x4 lo = *(const u32x4 *)(xq + 32u * b), hi = *(const u32x4 *)(xq + 32u * b + 16u);
  int d0, d1;
  q6k_dots(nw, hw.x, hw.y, lo, hi, d0, d1);
  const int s0 = hsum16(lo), s1 = hsum16(hi);
  out[2u * i] = d0 - 32 * s0;
  out[2u * i + 1u] = d1 - 32 * s1;
}

// ------------------------------------------------------------------ prefill GEMM

// Y[t][r] = sum over sub-blocks b of (d sc)_rb da_tb dq_rtb - (dmin mn)_rb
// da_tb asum_tb for Q4_K weights and T Q8 token rows (ie_gemm_q4kr), then
// the epilogue. The integer dq (sum q a over the 32 weights of a sub-block)
// comes exact from v_mfma_i32_16x16x32_i8; the min term, a small
// contraction over the blocks, from v_mfma_f32_16x16x4_f32 in f32 (the
// reference uses fp16 there: not within 1e-5).
//
// Workgroup tile: 64 rows x NTT tokens, 4 waves; wave w: rows 16w..16w+15,
// all NTT tokens (NTT / 16 MFMA tiles). K loop: tile t of 8 super-groups
// (header of each row staged in LDS), then plane k = 0..7 of the tile: the
// 8 blocks b = 8 (8t + gl) + k, gl < gt, whose nibbles are 128 contiguous
// bytes per row. MFMA operand mapping (lane = 16 h + i): A lane holds row i,
// K bytes 8h..8h+7 = nibbles (h & 1) * 8 .. + 7, low nibble if h < 2 else
// high; B lane holds token i, activation bytes 8h..8h+7: both sides use the
// same K order. Output lane: rows 4h + v (v < 4), token i.
template <int NTT>
__device__ __forceinline__ void gemm_body(const uint8_t *__restrict__ W, const uint8_t *__restrict__ xq, float *__restrict__ y,
                                          u32 rows, u32 nb, const float *__restrict__ bias, const float *__restrict__ res, u32 T, u32 xs,
                                          u32 ys, u32 rs) {
  constexpr u32 NJ = NTT / 16;
  __shared__ __attribute__((aligned(16))) u32x4 sh_hdr[8][64];        // headers of the tile [gl][row]
  __shared__ __attribute__((aligned(16))) u32x4 sh_a[8][64];          // plane nibbles [gl][row]
  __shared__ __attribute__((aligned(16))) u32x4 sh_b[8][NTT][2];      // activations [gl][token][lo/hi]
  __shared__ __attribute__((aligned(16))) float sh_da[8][NTT];        // d_a [gl][token]
  __shared__ __attribute__((aligned(16))) float sh_xa[8][NTT];        // d_a * asum [gl][token]
  __shared__ __attribute__((aligned(16))) float sh_s[8][64];          // d sc [gl][row]
  __shared__ __attribute__((aligned(16))) float sh_m[8][64];          // -(dmin mn) [gl][row]

  const u32 ng = amdc_ngroups(nb), ntile = (ng + 7u) >> 3, tid = threadIdx.x, lane = tid & 63u, w = tid >> 6;
  const u32 i16 = lane & 15u, h = lane >> 4;
  const u32 ntt = (T + NTT - 1u) / NTT, tt = blockIdx.x % ntt, rt = blockIdx.x / ntt;
  const u32 rbase = rt * 64u, tbase = tt * NTT;
  const u64 RB = amdc_row_bytes(nb);

  v4f acc[NJ];
#pragma unroll
  for (u32 j = 0; j < NJ; j++) acc[j] = (v4f){0.0f, 0.0f, 0.0f, 0.0f};

  for (u32 t = 0; t < ntile; t++) {
    const u32 gt = ng - 8u * t < 8u ? ng - 8u * t : 8u;
    __syncthreads();
    for (u32 i = tid; i < 64u * gt; i += NT) { // the headers of the tile
      const u32 gl = i >> 6, r = i & 63u, rr = rbase + r < rows ? rbase + r : rows - 1u;
      sh_hdr[gl][r] = *(const u32x4 *)(W + (u64)rr * RB + amdc_header_off(8u * t + gl));
    }
    for (u32 k = 0; k < 8u; k++) {
      __syncthreads();
      for (u32 i = tid; i < 64u * gt; i += NT) { // plane k: nibbles and row scales
        const u32 gl = i >> 6, r = i & 63u, rr = rbase + r < rows ? rbase + r : rows - 1u;
        sh_a[gl][r] = *(const u32x4 *)(W + (u64)rr * RB + amdc_nib_off(ng, 8u * t + gl, k));
        const u32x4 hd = sh_hdr[gl][r];
        sh_s[gl][r] = h2f(hd.x) * (float)q4k_sc(hd, k);
        sh_m[gl][r] = -(h2f(hd.x >> 16) * (float)q4k_mn(hd, k));
      }
      for (u32 i = tid; i < NTT * gt * 2u; i += NT) { // activations of blocks 8 (8t + gl) + k
        const u32 half = i & 1u, tk = (i >> 1) % NTT, gl = (i >> 1) / NTT;
        const u32 gtk = tbase + tk < T ? tbase + tk : T - 1u, b = 8u * (8u * t + gl) + k;
        const uint8_t *xt = xq + (u64)gtk * xs;
        sh_b[gl][tk][half] = *(const u32x4 *)(xt + 32u * b + 16u * half);
        if (half == 0u) {
          const float da = ((const float *)(xt + 32u * nb))[b];
          sh_da[gl][tk] = da;
          sh_xa[gl][tk] = da * (float)(int)((const u32 *)(xt + 36u * nb))[b];
        }
      }
      __syncthreads();
      for (u32 gl = 0; gl < gt; gl++) {
        const u32x4 wa = sh_a[gl][16u * w + i16];
        const u32 w0 = (h & 1u) ? wa.z : wa.x, w1 = (h & 1u) ? wa.w : wa.y, sft = (h >> 1) * 4u;
        const long af = (long)(((u64)((w1 >> sft) & 0x0F0F0F0Fu) << 32) | ((w0 >> sft) & 0x0F0F0F0Fu));
        const v4f s4 = *(const v4f *)&sh_s[gl][16u * w + 4u * h];
#pragma unroll
        for (u32 j = 0; j < NJ; j++) {
          const u32x4 bv = sh_b[gl][16u * j + i16][h >> 1];
          const long bf = (long)((h & 1u) ? (((u64)bv.w << 32) | bv.z) : (((u64)bv.y << 32) | bv.x));
          const v4i c = __builtin_amdgcn_mfma_i32_16x16x32_i8(af, bf, (v4i){0, 0, 0, 0}, 0, 0, 0);
          const float da = sh_da[gl][16u * j + i16];
#pragma unroll
          for (u32 v = 0; v < 4u; v++) acc[j][v] = __builtin_fmaf(s4[v] * da, (float)c[v], acc[j][v]);
        }
      }
      // the min term of the plane's blocks: K = gl (zero past gt)
#pragma unroll
      for (u32 kk = 0; kk < 8u; kk += 4u) {
        const u32 gl = kk + h;
        const float am = gl < gt ? sh_m[gl][16u * w + i16] : 0.0f;
#pragma unroll
        for (u32 j = 0; j < NJ; j++) {
          const float bx = gl < gt ? sh_xa[gl][16u * j + i16] : 0.0f;
          acc[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(am, bx, acc[j], 0, 0, 0);
        }
      }
    }
  }
#pragma unroll
  for (u32 j = 0; j < NJ; j++) {
    const u32 tk = tbase + 16u * j + i16;
    if (tk >= T) continue;
#pragma unroll
    for (u32 v = 0; v < 4u; v++) {
      const u32 r = rbase + 16u * w + 4u * h + v;
      if (r < rows) {
        float o = acc[j][v];
        if (bias) o = o + bias[r];
        if (res) o = res[(u64)tk * rs + r] + o;
        y[(u64)tk * ys + r] = o;
      }
    }
  }
}

extern "C" __global__ __launch_bounds__(256) void amdc_gemm_q4_k_n128(const uint8_t *W, const uint8_t *xq, float *y, u32 rows, u32 nb,
                                                                     const float *bias, const float *res, u32 T, u32 xs, u32 ys,
                                                                     u32 rs) {
  gemm_body<128>(W, xq, y, rows, nb, bias, res, T, xs, ys, rs);
}
extern "C" __global__ __launch_bounds__(256) void amdc_gemm_q4_k_n64(const uint8_t *W, const uint8_t *xq, float *y, u32 rows, u32 nb,
                                                                    const float *bias, const float *res, u32 T, u32 xs, u32 ys,
                                                                    u32 rs) {
  gemm_body<64>(W, xq, y, rows, nb, bias, res, T, xs, ys, rs);
}

// ------------------------------------------------------------------ prefill GEMM on the f16 MFMA, exact integer sums

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));

// The prefill activations as the GEMM reads them, from the Q8 buffers of T
// tokens (token t at xq + t xs): xh[t][32 nb] = the int8 values as f16
// (exact), da[b][t] = d_a, xa[b][t] = d_a * asum, for t < Tp; tokens T..Tp-1
// are zeros. One thread per (token, block).
extern "C" __global__ __launch_bounds__(256) void amdc_q8_prep(const uint8_t *__restrict__ xq, u32 nb, u32 T, u32 xs,
                                                               _Float16 *__restrict__ xh, float *__restrict__ da, float *__restrict__ xa,
                                                               u32 Tp) {
  // a workgroup: 8 blocks x 32 tokens; thread (token tid / 8, block tid % 8) converts its block (a
  // token's 8 blocks are 256 contiguous bytes of xq and 512 of xh), and the scales go to da / xa
  // through the LDS, 32 consecutive tokens of a block per store
  constexpr u32 BB = 8u, TT = 32u;
  __shared__ float sd[2][BB][TT + 1u];
  const u32 nbb = (nb + BB - 1u) / BB, b0 = (blockIdx.x % nbb) * BB, t0 = (blockIdx.x / nbb) * TT;
  const u32 tl = threadIdx.x / BB, bl = threadIdx.x % BB, t = t0 + tl, b = b0 + bl;
  if (b < nb) {
    u32x4 o[4] = {(u32x4)(0u), (u32x4)(0u), (u32x4)(0u), (u32x4)(0u)};
    float d = 0.0f, x = 0.0f;
    if (t < T) {
      const uint8_t *xt = xq + (u64)t * xs;
      const u32x4 lo = *(const u32x4 *)(xt + 32u * b), hi = *(const u32x4 *)(xt + 32u * b + 16u);
      const u32 w[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
#pragma unroll
      for (u32 k = 0; k < 16u; k++) {
        const int e0 = (int)(int8_t)(w[k >> 1] >> (16u * (k & 1u))), e1 = (int)(int8_t)(w[k >> 1] >> (16u * (k & 1u) + 8u));
        const u32 v = (u32)__builtin_bit_cast(unsigned short, (_Float16)e0) | ((u32)__builtin_bit_cast(unsigned short, (_Float16)e1) << 16);
        o[k >> 2][k & 3u] = v;
      }
      d = ((const float *)(xt + 32u * nb))[b];
      x = d * (float)(int)((const u32 *)(xt + 36u * nb))[b];
    }
    u32x4 *dst = (u32x4 *)(xh + ((u64)t * nb + b) * 32u);
#pragma unroll
    for (u32 k = 0; k < 4u; k++) dst[k] = o[k];
    sd[0][bl][tl] = d;
    sd[1][bl][tl] = x;
  }
  __syncthreads();
  const u32 tw = threadIdx.x % TT, bw = threadIdx.x / TT; // 32 tokens of block b0 + bw
  if (b0 + bw < nb) {
    da[(u64)(b0 + bw) * Tp + t0 + tw] = sd[0][bw][tw];
    xa[(u64)(b0 + bw) * Tp + t0 + tw] = sd[1][bw][tw];
  }
}

// Four nibbles (bytes 0..15 of n) -> two f16 pairs (1024 + q): each byte
// below 0x64, the exponent byte of 1024 (v_perm_b32 picks the bytes).
__device__ __forceinline__ void nib_to_h(u32 n, h2 &a, h2 &b) {
  a = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, n, 0x04010400u));
  b = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, n, 0x04030402u));
}

// The A operand of one 16 x 32 block tile: lane (row i, h) holds weights
// 8h..8h+7 of its row's block, q sc as f16 (exact: q sc <= 945). w0, w1: the
// 8 nibble bytes (h & 1) * 8 .. + 7 of the block; the low nibbles for h < 2.
__device__ __forceinline__ h8 a_frag(u32 w0, u32 w1, u32 h, _Float16 sc) {
  const u32 sft = (h >> 1) * 4u;
  const u32 n0 = (w0 >> sft) & 0x0F0F0F0Fu, n1 = (w1 >> sft) & 0x0F0F0F0Fu;
  h2 p0, p1, p2, p3;
  nib_to_h(n0, p0, p1);
  nib_to_h(n1, p2, p3);
  const h2 s2 = {sc, sc}, c2 = {(_Float16)(-1024.0f) * sc, (_Float16)(-1024.0f) * sc}; // (1024 + q) sc - 1024 sc, one rounding
  p0 = __builtin_elementwise_fma(p0, s2, c2);
  p1 = __builtin_elementwise_fma(p1, s2, c2);
  p2 = __builtin_elementwise_fma(p2, s2, c2);
  p3 = __builtin_elementwise_fma(p3, s2, c2);
  return (h8){p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
}

// The A operand of a Q8_0 block tile: lane (row i, h) holds weights
// 8h..8h+7, the int8 bytes w0, w1 (plane h >> 1, bytes 8 (h & 1) ..) as f16:
// byte ^ 0x80 = w + 128 in the mantissa of 1024, then - 1152 (exact).
__device__ __forceinline__ h8 a_frag_q8(u32 w0, u32 w1) {
  h2 p0, p1, p2, p3;
  nib_to_h(w0 ^ 0x80808080u, p0, p1);
  nib_to_h(w1 ^ 0x80808080u, p2, p3);
  const h2 c = {(_Float16)-1152.0f, (_Float16)-1152.0f};
  p0 += c, p1 += c, p2 += c, p3 += c;
  return (h8){p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
}

// The A operand of a Q4_0 block tile: lane (row i, h) holds weights 8h..8h+7
// as q - 8 in f16 (exact): the nibbles of bytes 8 (h & 1) .. + 7 (low for
// h < 2), in the mantissa of 1024, then - 1032.
__device__ __forceinline__ h8 a_frag_q40(u32 w0, u32 w1, u32 h) {
  const u32 sft = (h >> 1) * 4u;
  h2 p0, p1, p2, p3;
  nib_to_h((w0 >> sft) & 0x0F0F0F0Fu, p0, p1);
  nib_to_h((w1 >> sft) & 0x0F0F0F0Fu, p2, p3);
  const h2 c = {(_Float16)-1032.0f, (_Float16)-1032.0f};
  p0 += c, p1 += c, p2 += c, p3 += c;
  return (h8){p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
}

// The A operands of a Q6_K sub-block tile: lane (row i, h) holds weights
// 8h..8h+7, of half h >> 1, as (q - 32) sc split into hi = (q - 32) 16 (sc >> 4)
// and lo = (q - 32) (sc & 15), both exact in f16 (|.| <= 4096, multiples of
// 16; |.| <= 480), so that the two MFMAs add the integer (q - 32) sc a exactly
// (every partial sum stays under 128 * 32 * 32 * 127 < 2^24). w0, w1: nibble
// bytes 8 (h & 1) .. + 7 (the low 4 bits of the half's weights in the low
// nibble for h < 2, else the high); hw: the half's high-bit word (weight
// 4i + e at bits 8e + 2i, i = 2 (h & 1) for w0's weights, + 1 for w1's).
__device__ __forceinline__ void a_frag_q6(u32 w0, u32 w1, u32 hw, u32 h, int sc, h8 &ahi, h8 &alo) {
  const u32 sft = (h >> 1) * 4u, hs = 4u * (h & 1u);
  const u32 q0 = ((w0 >> sft) & 0x0F0F0F0Fu) | (((hw >> hs) & 0x03030303u) << 4);
  const u32 q1 = ((w1 >> sft) & 0x0F0F0F0Fu) | (((hw >> (hs + 2u)) & 0x03030303u) << 4);
  h2 p[4];
  nib_to_h(q0, p[0], p[1]);
  nib_to_h(q1, p[2], p[3]);
  const _Float16 fl = (_Float16)(float)(sc & 15), fh = (_Float16)(float)(sc - (sc & 15));
  const h2 c = {(_Float16)-1056.0f, (_Float16)-1056.0f}, l2 = {fl, fl}, h2v = {fh, fh};
#pragma unroll
  for (u32 m = 0; m < 4u; m++) p[m] += c; // q - 32, exact
  h2 hi[4], lo[4];
#pragma unroll
  for (u32 m = 0; m < 4u; m++) hi[m] = p[m] * h2v, lo[m] = p[m] * l2;
  ahi = (h8){hi[0][0], hi[0][1], hi[1][0], hi[1][1], hi[2][0], hi[2][1], hi[3][0], hi[3][1]};
  alo = (h8){lo[0][0], lo[0][1], lo[1][0], lo[1][1], lo[2][0], lo[2][1], lo[3][0], lo[3][1]};
}

// Y[t][r] for Q4_K weights and T tokens (the arguments of ie_gemm_q4kr plus the
// prepared activations of amdc_q8_prep): per sub-block b of super-block g
//   X_rtb = sum_k (q sc)_rk a_tk          v_mfma_f32_16x16x32_f16, exact
//   tmp_rt += da_tb X_rtb                  one fma per element and block
//   acc_rt += d_rg tmp_rt                  per super-block
//   acc_rt -= sum_b (dmin mn)_rb xa_tb     v_mfma_f32_16x16x4_f32 per super-block
// the reference's terms (d sc)_rb da_tb dq_rtb - (dmin mn)_rb da_tb asum_tb
// regrouped, the integer sums sc dq kept exact.
//
// Workgroup: 4 waves, 2 x 2; wave (wm, wn): 32 rows (2 row tiles of 16) x
// 16 NJ tokens; the workgroup tile is 64 rows x 32 NJ tokens. K in stages of
// 2 blocks; a super-block is 4 stages. The stage's f16 activations, d_a and
// d_a asum are written to LDS (double buffer, one barrier per stage) from
// registers loaded a stage ahead; each wave reads its weights' nibble bytes
// straight from memory, also a stage ahead (the stage loop is unrolled by
// two, so the prefetched registers alternate instead of being copied). All
// global addresses are a workgroup-uniform base plus a 32-bit lane offset.
// Inside a block all MFMAs are issued before their results are used.
// Schedule (nfull, nks): blocks [0, nfull) are tiles 0 .. nfull - 1 over the
// whole K, written to y; the other blocks, nfull + j, are the tail tiles,
// tile nfull + j % tail and K split j / tail of nks (super-blocks [g0, g1)),
// whose partial sums go to part[split][t][r - r0] (r0 the tail's first row,
// row stride rows - r0) for amdc_gemm_reduce to add in split order. nfull is
// a whole number of row tiles; nfull = 0 splits every tile.
template <int NJ, int KIND, u32 MW = 2u>
__device__ __forceinline__ void gemmh_body(const uint8_t *__restrict__ W, const _Float16 *__restrict__ xh, const float *__restrict__ DA,
                                           const float *__restrict__ XA, float *__restrict__ y, u32 rows, u32 nb,
                                           const float *__restrict__ bias, const float *__restrict__ res, u32 T, u32 Tp, u32 ys, u32 rs,
                                           float *__restrict__ part, u32 nfull, u32 nsplit) {
  constexpr u32 NTH = 128u * MW, MR = 32u * MW, NTT = 32u * NJ; // MW waves of 32 rows x 2 of 16 NJ tokens
  constexpr u32 BSTR = 72u; // halves per token per stage: 2 blocks x 32 + 8 of padding
  __shared__ __attribute__((aligned(16))) _Float16 sb[2][NTT * BSTR];
  __shared__ __attribute__((aligned(16))) float sda[2][2][NTT];
  __shared__ __attribute__((aligned(16))) float sxa[2][8][NTT]; // d_a asum of a super-block's 8 blocks, by parity
  __shared__ float sspare[2][2u * NTT < NTH ? NTH : 1u];
  constexpr bool PB = KIND == AMDC_Q8_0 || KIND == AMDC_Q4_0;     // a d per (row, block): applied per block
  __shared__ __attribute__((aligned(16))) float sdw[PB ? 2u * MW : 1][2][8][16]; // per wave: d [row tile][block][row]
  const u32 ng = KIND == AMDC_Q8_0 || KIND == AMDC_Q4_0 ? amdc_ngroups(nb) : nb >> 3, tid = threadIdx.x, lane = tid & 63u, w = tid >> 6, wm = w % MW, wn = w / MW;
  const u32 i16 = lane & 15u, h = lane >> 4;
  const u32 ntt = (T + NTT - 1u) / NTT, b = blockIdx.x, full = b < nfull;
  const u32 tail = (rows + MR - 1u) / MR * ntt - nfull, tj = b - nfull; // tail tiles; a tail block's index among the tail blocks
  // whole-K tiles: the ntt token tiles of a row tile go to one XCD (workgroups are dealt to the 8 XCDs
  // in turn), 8 workgroups apart, so that the second reads the row tile's weights from that XCD's L2
  const u32 xg = 8u * ntt, xq = b / xg, xj = b % xg;
  const u32 tile = full ? (ntt > 1u && nfull % xg == 0u ? (8u * xq + xj % 8u) * ntt + xj / 8u : b) : nfull + tj % tail;
  const u32 tt = tile % ntt, rt = tile / ntt;
  const u32 tbase = tt * NTT, twave = 16u * NJ * wn;
  const u32 ks = full ? 0u : tj / tail, nks = full ? 1u : nsplit, g0 = ng * ks / nks, g1 = ng * (ks + 1u) / nks;
  const u32 r0 = nfull / ntt * MR; // the tail's first row
  const u32 RB = (u32)amdc_row_bytes_k(KIND, nb), K2 = 64u * nb; // bytes per weight row, per activation row
  // uniform bases (buffer resources), 32-bit lane offsets
  const uint8_t *wbase = W + (u64)rt * MR * RB;
  const __amdgpu_buffer_rsrc_t rw = rsrc(wbase, (u32)min((u64)(rows - rt * MR) * RB, (u64)0xFFFFFFF0u));
  const __amdgpu_buffer_rsrc_t rx = rsrc((const uint8_t *)xh + (u64)tbase * K2, (u32)min((u64)(Tp - tbase) * K2, (u64)0xFFFFFFF0u));
  const __amdgpu_buffer_rsrc_t rda = rsrc(DA, (u32)min((u64)nb * Tp * 4u, (u64)0xFFFFFFF0u));
  const __amdgpu_buffer_rsrc_t rxa = rsrc(XA, (u32)min((u64)nb * Tp * 4u, (u64)0xFFFFFFF0u));
  // lane offsets: the A rows of this lane (clamped), the B chunks of this thread
  u32 wo[2];
#pragma unroll
  for (u32 i = 0; i < 2u; i++) {
    const u32 rl = 32u * wm + 16u * i + i16, r = rt * MR + rl;
    wo[i] = (r < rows ? rl : rows - 1u - rt * MR) * RB;
  }
  constexpr u32 NCH = NTT * 8u / NTH; // 16-byte chunks of activations per thread and stage (128 bytes per token)
  u32 xo[NCH];
#pragma unroll
  for (u32 c = 0; c < NCH; c++) {
    const u32 ch = tid + c * NTH;
    xo[c] = (ch >> 3) * K2 + 16u * (ch & 7u);
  }
  const u32 dao = ((tid / NTT) * Tp + tbase + tid % NTT) * 4u; // d_a of (block 2s + tid / NTT, token tid % NTT)
  v4f acc[2][NJ], tmp[2][NJ];
#pragma unroll
  for (u32 i = 0; i < 2u; i++)
#pragma unroll
    for (u32 j = 0; j < NJ; j++) acc[i][j] = (v4f){0.0f, 0.0f, 0.0f, 0.0f}, tmp[i][j] = acc[i][j];

  u32x4 rb[NCH];
  float rd = 0.0f, rxv = 0.0f; // d_a, d_a asum: threads < 2 NTT, one (block, token) each
  // every load of a stage is issued by every thread (threads past 2 NTT read past the resource: zeros,
  // unused), and the loop issues them unconditionally: the compiler then counts the loads in flight
  // statically, and a wait for one stage's data does not become a wait for the next stage's loads
  const u32 daoa = tid < 2u * NTT ? dao : 0xFFFFFFF0u;
  auto fetch = [&](u32 s) { // stage s = blocks 2s, 2s+1
#pragma unroll
    for (u32 c = 0; c < NCH; c++) rb[c] = __builtin_amdgcn_raw_buffer_load_b128(rx, xo[c], 128u * s, 0);
    rd = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rda, daoa, 8u * s * Tp, 0));
    rxv = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rxa, daoa, 8u * s * Tp, 0));
  };
  auto store = [&](u32 bf, u32 s) {
#pragma unroll
    for (u32 c = 0; c < NCH; c++) {
      const u32 ch = tid + c * NTH;
      *(u32x4 *)(&sb[bf][(ch >> 3) * BSTR + 8u * (ch & 7u)]) = rb[c];
    }
    // every thread stores (threads past 2 NTT into a spare word): with the store conditional the
    // compiler moved the d_a loads into its branch, after the stage's compute, and waited for them there
    const bool hv = tid < 2u * NTT;
    float *pd = hv ? &sda[bf][tid / NTT][tid % NTT] : &sspare[0][tid];
    float *px = hv ? &sxa[(s >> 2) & 1u][2u * (s & 3u) + tid / NTT][tid % NTT] : &sspare[1][tid]; // the next super-block writes the other half
    *pd = rd;
    *px = rxv;
  };
  // the lane's 8 weight bytes (nibbles, or int8), 2 blocks x 2 row tiles, and
  // for Q6_K the high-bit word of its half
  auto load_w = [&](u32 s, u32 (&wv)[2][2][3]) {
    const u32 g = s >> 2, kb = 2u * (s & 3u);
#pragma unroll
    for (u32 bb = 0; bb < 2u; bb++) {
      const u32 k = kb + bb;
      const u32 so = KIND == AMDC_Q8_0   ? (u32)amdc_q8_off(ng, g, 2u * k + (h >> 1))
                     : KIND == AMDC_Q6_K ? (u32)amdc_q6k_nib_off(ng, g, k)
                                         : (u32)amdc_nib_off(ng, g, k);
#pragma unroll
      for (u32 i = 0; i < 2u; i++) {
        const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(rw, wo[i] + 8u * (h & 1u), so, 0);
        wv[bb][i][0] = v.x, wv[bb][i][1] = v.y;
        if constexpr (KIND == AMDC_Q6_K)
          wv[bb][i][2] = __builtin_amdgcn_raw_buffer_load_b32(rw, wo[i] + 4u * (h >> 1), (u32)amdc_q6k_hi_off(ng, g, k >> 1) + 8u * (k & 1u), 0);
      }
    }
  };
  u32x4 hd[2], hn[2]; // the super-group header of the lane's A rows (scales; Q8_0: the 8 d), and the next one's
  u32 hdd[2], hnd[2];  // Q6_K: f16 d
  auto load_h = [&](u32 g, u32x4(&hx)[2], u32(&hxd)[2]) {
#pragma unroll
    for (u32 i = 0; i < 2u; i++) {
      hx[i] = __builtin_amdgcn_raw_buffer_load_b128(rw, wo[i], 16u * g, 0);
      if constexpr (KIND == AMDC_Q6_K) hxd[i] = __builtin_amdgcn_raw_buffer_load_b16(rw, wo[i], 16u * ng + 2u * g, 0);
    }
  };

  // one stage: the MFMAs and fmas of blocks kb, kb + 1 of the super-block (kb
  // a constant) from LDS buffer bf and the nibbles wv
  // the A operands of block k from its weight words (Q6_K: two, hi and lo)
  auto frag = [&](const u32(&wk)[3], u32 i, u32 k, h8 &a0, h8 &a1) {
    if constexpr (KIND == AMDC_Q8_0) {
      a0 = a_frag_q8(wk[0], wk[1]);
    } else if constexpr (KIND == AMDC_Q4_0) {
      a0 = a_frag_q40(wk[0], wk[1], h);
    } else if constexpr (KIND == AMDC_Q6_K) {
      const int sc = (int)(int8_t)(hword(hd[i], k >> 1) >> (16u * (k & 1u) + 8u * (h >> 1)));
      a_frag_q6(wk[0], wk[1], wk[2], h, sc, a0, a1);
    } else {
      a0 = a_frag(wk[0], wk[1], h, (_Float16)(float)q4k_sc(hd[i], k));
    }
  };
  auto compute = [&](u32 kb, u32 bf, const u32(&wv)[2][2][3]) {
    if constexpr (PB) {
      if (kb == 0u) { // a super-group's first stage: the d's of the lane's A rows into the wave's table (blocks 2h, 2h + 1)
#pragma unroll
        for (u32 i = 0; i < 2u; i++)
#pragma unroll
          for (u32 e = 0; e < 2u; e++) sdw[w][i][2u * h + e][i16] = h2f(hword(hd[i], h) >> (16u * e));
        __asm__ volatile("" ::: "memory"); // the table's stores stay ahead of its loads (one wave: LDS keeps their order)
      }
    }
    const _Float16 *lb = &sb[bf][(twave + i16) * BSTR + 8u * h];
    h8 bq[NJ];
#pragma unroll
    for (u32 j = 0; j < NJ; j++) bq[j] = *(const h8 *)(lb + 16u * j * BSTR);
    h8 af[2], al[2];
#pragma unroll
    for (u32 i = 0; i < 2u; i++) frag(wv[0][i], i, kb, af[i], al[i]);
#pragma unroll
    for (u32 bb = 0; bb < 2u; bb++) {
      float dj[NJ];
#pragma unroll
      for (u32 j = 0; j < NJ; j++) dj[j] = sda[bf][bb][twave + 16u * j + i16];
      v4f dw[2]; // Q8_0, Q4_0: the block's d of the C rows 4h + v of each row tile
      if constexpr (PB) {
#pragma unroll
        for (u32 i = 0; i < 2u; i++) dw[i] = *(const v4f *)&sdw[w][i][kb + bb][4u * h];
      }
#pragma unroll
      for (u32 i = 0; i < 2u; i++) { // a row tile at a time: NJ MFMAs in flight, then their fmas
        v4f x[NJ];
#pragma unroll
        for (u32 j = 0; j < NJ; j++) {
          if constexpr (KIND == AMDC_Q6_K) {
            x[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bq[j], (v4f){0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
            x[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[i], bq[j], x[j], 0, 0, 0);
          } else {
            x[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bq[j], (v4f){0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
          }
        }
        if (bb == 0u && i == 1u) { // the second block's operands while the MFMAs run
#pragma unroll
          for (u32 j = 0; j < NJ; j++) bq[j] = *(const h8 *)(lb + 16u * j * BSTR + 32u);
#pragma unroll
          for (u32 i2 = 0; i2 < 2u; i2++) frag(wv[1][i2], i2, kb + 1u, af[i2], al[i2]);
        }
#pragma unroll
        for (u32 j = 0; j < NJ; j++)
#pragma unroll
          for (u32 v = 0; v < 4u; v++) {
            if constexpr (KIND == AMDC_Q8_0 || KIND == AMDC_Q4_0) // (d_w d_a) dot, as src/cpu.c:81, 168
              acc[i][j][v] = __builtin_fmaf(dw[i][v] * dj[j], x[j][v], acc[i][j][v]);
            else
              tmp[i][j][v] = __builtin_fmaf(dj[j], x[j][v], tmp[i][j][v]);
          }
      }
    }
  };
  // the end of a super-block: d, and the min term from the 8 blocks' d_a asum
  auto close_group = [&](u32 gp) {
    if constexpr (KIND == AMDC_Q8_0 || KIND == AMDC_Q4_0) return;
#pragma unroll
    for (u32 i = 0; i < 2u; i++) {
      const float dmine = KIND == AMDC_Q6_K ? h2f(hdd[i]) : h2f(hd[i].x), dmn = h2f(hd[i].x >> 16);
      float dv[4];
#pragma unroll
      for (u32 v = 0; v < 4u; v++) dv[v] = __shfl(dmine, (int)(4u * h + v));
      float am[2];
#pragma unroll
      for (u32 q = 0; q < 2u; q++) am[q] = -(dmn * (float)q4k_mn(hd[i], 4u * q + h));
#pragma unroll
      for (u32 j = 0; j < NJ; j++) {
#pragma unroll
        for (u32 v = 0; v < 4u; v++) acc[i][j][v] = __builtin_fmaf(dv[v], tmp[i][j][v], acc[i][j][v]);
        tmp[i][j] = (v4f){0.0f, 0.0f, 0.0f, 0.0f};
        if constexpr (KIND == AMDC_Q4_K) {
#pragma unroll
          for (u32 q = 0; q < 2u; q++)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(am[q], sxa[gp][4u * q + h][twave + 16u * j + i16], acc[i][j], 0, 0, 0);
        }
      }
    }
  };

  // stages in pairs: s (LDS buffer 0, nibbles wa), s + 1 (buffer 1, nibbles
  // wb); the activations and the nibbles of the next stage are in flight
  // during a stage
  const u32 s0 = 4u * g0, s1 = 4u * g1;
  u32 wa[2][2][3], wb[2][2][3];
  if (s0 < s1) { // a split may own no super-block (then its partial sums are 0)
    fetch(s0);
    store(0, s0);
    load_w(s0, wa);
    load_h(g0, hn, hnd);
  }
  __syncthreads();
  for (u32 s = s0; s < s1; s += 2u) {
#pragma unroll
    for (u32 i = 0; i < 2u; i++) hd[i] = hn[i], hdd[i] = hnd[i]; // the header of stages s, s + 1 (loaded a stage ago)
    fetch(s + 1u);
    load_w(s + 1u, wb);
    compute(2u * (s & 3u), 0, wa);
    store(1, s + 1u);
    __syncthreads();
    const bool more = s + 2u < s1;
    load_h((s + 2u) >> 2, hn, hnd); // the super-group header of stage s + 2 (the current one's again inside a super-group)
    __asm__ volatile("" ::: "memory"); // issued before the stage's other loads: waiting for it does not wait for them
    fetch(s + 2u);                     // past the range: unused bytes (or zeros past the resource)
    load_w(s + 2u, wa);
    compute(2u * ((s + 1u) & 3u), 1, wb);
    if (((s + 1u) & 3u) == 3u) close_group((s >> 2) & 1u);
    if (more) store(0, s + 2u);
    __syncthreads();
  }
#pragma unroll
  for (u32 i = 0; i < 2u; i++)
#pragma unroll
    for (u32 j = 0; j < NJ; j++) {
      const u32 tk = tbase + twave + 16u * j + i16;
      if (tk >= T) continue;
#pragma unroll
      for (u32 v = 0; v < 4u; v++) {
        const u32 r = rt * MR + 32u * wm + 16u * i + 4u * h + v;
        if (r >= rows) continue;
        if (!full) {
          part[((u64)ks * T + tk) * (rows - r0) + (r - r0)] = acc[i][j][v];
        } else {
          float o = acc[i][j][v];
          if (bias) o = o + bias[r];
          if (res) o = res[(u64)tk * rs + r] + o;
          y[(u64)tk * ys + r] = o;
        }
      }
    }
}

#define GEMMH_KERNEL(NAME, NJ, KIND)                                                                                               \
  extern "C" __global__ __launch_bounds__(256) void NAME(const uint8_t *W, const _Float16 *xh, const float *DA, const float *XA,  \
                                                         float *y, u32 rows, u32 nb, const float *bias, const float *res, u32 T,  \
                                                         u32 Tp, u32 ys, u32 rs, float *part, u32 nfull, u32 nsplit) {            \
    gemmh_body<NJ, KIND>(W, xh, DA, XA, y, rows, nb, bias, res, T, Tp, ys, rs, part, nfull, nsplit);                              \
  }
GEMMH_KERNEL(amdc_gemmh_m64_n128, 4, AMDC_Q4_K)
GEMMH_KERNEL(amdc_gemmh_m64_n64, 2, AMDC_Q4_K)
GEMMH_KERNEL(amdc_gemmh_q8_0_m64_n128, 4, AMDC_Q8_0)
GEMMH_KERNEL(amdc_gemmh_q8_0_m64_n64, 2, AMDC_Q8_0)
GEMMH_KERNEL(amdc_gemmh_q6_k_m64_n128, 4, AMDC_Q6_K)
GEMMH_KERNEL(amdc_gemmh_q6_k_m64_n64, 2, AMDC_Q6_K)
GEMMH_KERNEL(amdc_gemmh_q4_0_m64_n128, 4, AMDC_Q4_0)
GEMMH_KERNEL(amdc_gemmh_q4_0_m64_n64, 2, AMDC_Q4_0)
// 128-row tiles, 8 waves (4 x 2): the stage's activations in the LDS shared by twice the rows (Q4_K,
// T > 64, the default below 65536 rows; measured on MI355X, T = 256, us per call with the prep, 64 /
// 128-row tiles: 5120 x 17408 185.6 / 161.3, 17408 x 5120 161.5 / 158.1, 34816 x 5120 305 / 288, 4096 x
// 11008 99.2 / 90.2, 6144 x 5120 82.1 / 76.3, 152064 x 5120 1116 / 1161; 128 rows x 64 tokens, 124
// VGPRs and two workgroups per CU: 170-266 TOPS, slower everywhere)
extern "C" __global__ __launch_bounds__(512) void amdc_gemmh_m128_n128(const uint8_t *W, const _Float16 *xh, const float *DA, const float *XA,
                                                                      float *y, u32 rows, u32 nb, const float *bias, const float *res, u32 T,
                                                                      u32 Tp, u32 ys, u32 rs, float *part, u32 nfull, u32 nsplit) {
  gemmh_body<4, AMDC_Q4_K, 4u>(W, xh, DA, XA, y, rows, nb, bias, res, T, Tp, ys, rs, part, nfull, nsplit);
}

// The split-K sums: y[t][r] = the pairwise tree (adjacent splits first, a
// split past nks counting as +0.0) of part[0][t][r], part[1][t][r], ...,
// then the epilogue. nks (1..16) is uniform: one branch on it, then nks loads
// in flight, then the adds. The host clamps the split count to 16 (the
// default case reads 16 splits). The verify kernels' K ranges are aligned
// subtrees of their tile tree, so this tree completes it; for the GEMM any
// fixed order would do.
template <u32 N, bool AT = false> __device__ __forceinline__ float split_sum(const float *__restrict__ part, u64 step, u64 i) {
  float v[N];
#pragma unroll
  for (u32 k = 0; k < N; k++)
    v[k] = AT ? __hip_atomic_load(part + k * step + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : part[k * step + i];
#pragma unroll
  for (u32 m = N; m > 1u; m = (m + 1u) / 2u) {
#pragma unroll
    for (u32 k = 0; k < m / 2u; k++) v[k] = v[2u * k] + v[2u * k + 1u];
    if (m & 1u) v[m / 2u] = v[m - 1u]; // an odd one out pairs with +0.0
  }
  return v[0];
}

template <bool AT = false>
__device__ __forceinline__ float split_sum_n(const float *__restrict__ part, u32 nks, u64 step, u64 i) {
  switch (nks) {
  case 1: return split_sum<1, AT>(part, step, i);
  case 2: return split_sum<2, AT>(part, step, i);
  case 3: return split_sum<3, AT>(part, step, i);
  case 4: return split_sum<4, AT>(part, step, i);
  case 5: return split_sum<5, AT>(part, step, i);
  case 6: return split_sum<6, AT>(part, step, i);
  case 7: return split_sum<7, AT>(part, step, i);
  case 8: return split_sum<8, AT>(part, step, i);
  case 9: return split_sum<9, AT>(part, step, i);
  case 10: return split_sum<10, AT>(part, step, i);
  case 11: return split_sum<11, AT>(part, step, i);
  case 12: return split_sum<12, AT>(part, step, i);
  case 13: return split_sum<13, AT>(part, step, i);
  case 14: return split_sum<14, AT>(part, step, i);
  case 15: return split_sum<15, AT>(part, step, i);
  default: return split_sum<16, AT>(part, step, i);
  }
}

extern "C" __global__ __launch_bounds__(256) void amdc_gemm_reduce(const float *__restrict__ part, u32 nks, float *__restrict__ y, u32 rows,
                                                                   u32 T, const float *__restrict__ bias, const float *__restrict__ res,
                                                                   u32 ys, u32 rs) {
  const u64 i = (u64)blockIdx.x * NT + threadIdx.x;
  if (i >= (u64)rows * T) return;
  const u32 t = (u32)(i / rows), r = (u32)(i - (u64)t * rows);
  float o = split_sum_n(part, nks, (u64)rows * T, i);
  if (bias) o = o + bias[r];
  if (res) o = res[(u64)t * rs + r] + o;
  y[(u64)t * ys + r] = o;
}

// Split K without a reduction launch (the verify kernels when the host passes
// the counters): each workgroup of a row tile stores its partial sums, then
// arrives on the tile's counter; the last of the nks to arrive adds the
// tile's partial sums (split_sum's tree, as amdc_gemm_reduce) and writes y,
// and sets the counter back to 0 for the next launch. Launches that use the
// counters must not overlap.
// Memory order: the partial sums are stored and loaded as agent-scope relaxed
// atomics (split_put, split_sum's loads), which the hardware performs at the
// agent's coherence point instead of in one XCD's L2 (the workgroups of a
// tile run on different XCDs); every thread waits for its stores' completion
// before the barrier that precedes the arrival, and the last workgroup loads
// after the barrier that follows it. No cache-wide writeback or invalidation
// is needed (agent-scope fences, one per workgroup, made the launch 2x slower).
__device__ __align__(256) u32 split_count[AMDC_SPLIT_TILES];
// the arrival counter of the GEMVs with the fused RMSNorm tail (norm_tail; 0 between launches)
__device__ __align__(256) u32 norm_count[64];

__device__ __forceinline__ void split_put(float *p, float v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }

__device__ __forceinline__ bool split_arrive(u32 *cnt, u32 nks) {
  __shared__ u32 s_last;
  __builtin_amdgcn_s_waitcnt(0x0F70); // vmcnt(0): this thread's partial stores are complete
  __syncthreads();
  if (threadIdx.x == 0u) {
    const u32 old = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const bool last = old + 1u == nks;
    if (last) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = last ? 1u : 0u;
  }
  __syncthreads();
  return s_last != 0u;
}

// The last workgroup's sums: rows [rt0, rt0 + 64) of every token, NTH threads.
template <u32 NTH>
__device__ __forceinline__ void split_finish(const float *__restrict__ part, u32 nks, float *__restrict__ y, u32 rows, u32 rt0, u32 T,
                                             const float *__restrict__ bias, const float *__restrict__ res, u32 ys, u32 rs) {
  for (u32 e = threadIdx.x; e < 64u * T; e += NTH) {
    const u32 t = e >> 6, r = rt0 + (e & 63u);
    if (r >= rows) continue;
    float o = split_sum_n<true>(part, nks, (u64)rows * T, (u64)t * rows + r);
    if (bias) o = o + bias[r];
    if (res) o = res[(u64)t * rs + r] + o;
    y[(u64)t * ys + r] = o;
  }
}


// The decode GEMV with K split over gridDim.y (amdc_gemv_{q4_0,q4_k}_k / _xk: matrices of few rows
// and long rows, which leave the CUs short of loads in flight): workgroup (row group, ks) takes the
// super-groups [ks R, ks R + R) of its rows, R = L a power of two (one super-group per lane, L lanes
// per row); it stages (_k) or quantizes from the f32 vector (_xk) only that slice of the vector, so
// the per-workgroup prologue shrinks with the split; the range's leaves go through seg_sum (the
// range's subtree of the row's super-group tree). The ranges' sums are stored as agent-scope atomics
// (part[ks][r]) and the last workgroup of the row group to arrive on its counter adds them with
// split_sum's tree (adjacent first), which completes the row tree: the bits of every other form.
// gridDim.y = 1 writes y directly.
template <int KIND, bool FQ>
__device__ __forceinline__ void gemvk_body(const uint8_t *__restrict__ W, const uint8_t *__restrict__ xq, float *__restrict__ y, u32 rows,
                                           u32 nb, const float *__restrict__ bias, const float *__restrict__ res, u32 L,
                                           const float *__restrict__ xf, uint8_t *__restrict__ q8out, float *__restrict__ part,
                                           u32 *__restrict__ arrive) {
  constexpr u32 NTH = 256u;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const u32 ng = amdc_ngroups(nb), tid = threadIdx.x, lane = tid & 63u, wv = tid >> 6;
  const u32 l = lane & (L - 1u), q = lane / L, rpw = 64u / L, rpg = 4u * rpw;
  const u32 sg0 = blockIdx.y * L, g = sg0 + l; // the range's first super-group, the lane's
  const u64 RB = amdc_row_bytes(nb);
  u32x4 *s_lo = (u32x4 *)smem;
  u32x4 *s_hi = s_lo + 8u * L;
  float *s_d = (float *)(s_hi + 8u * L);
  u32 *s_as = (u32 *)(s_d + 8u * L);
  const u32 r = blockIdx.x * rpg + wv * rpw + q;
  const uint8_t *wr = W + (u64)(r < rows ? r : rows - 1u) * RB;
  FusedQ8T<4u, NTH> fq;
  fq.sgb = sg0, fq.gc = L;
  if (FQ) {
    fq.load(xf, nb, 8u * sg0);
    __asm__ volatile("" ::: "memory"); // the activation loads ahead of the weight loads
  }
  Item it;
  load_item<KIND>(it, wr, ng, g, g < ng);
  if (FQ) {
    const u32 bend = 8u * (sg0 + L);
    fq.quant(8u * sg0, nb, ng, s_lo, s_hi, s_d, s_as, q8out);
    for (u32 b0 = 8u * sg0 + fq.bp * 4u; b0 < bend; b0 += fq.bp * 4u) {
      fq.load(xf, nb, b0);
      fq.quant(b0, nb, ng, s_lo, s_hi, s_d, s_as, q8out);
    }
  } else {
    for (u32 j = tid; j < 8u * L; j += NTH) { // block b = 8 (sg0 + j % L) + j / L of the row at LDS slot j
      const u32 b = 8u * (sg0 + j % L) + j / L;
      u32x4 lo = (u32x4)(0u), hi = (u32x4)(0u);
      float d = 0.0f;
      u32 as = 0;
      if (b < nb) {
        lo = *(const u32x4 *)(xq + 32u * b);
        hi = *(const u32x4 *)(xq + 32u * b + 16u);
        d = ((const float *)(xq + 32u * nb))[b];
        as = ((const u32 *)(xq + 36u * nb))[b];
      }
      s_lo[j] = lo, s_hi[j] = hi, s_d[j] = d, s_as[j] = as;
    }
  }
  __syncthreads();
  const float leaf = item_dot<KIND>(it, l, L, s_lo, s_hi, s_d, s_as, 0.0f);
  const float v = seg_sum(g < ng ? leaf : 0.0f, L);
  if (gridDim.y == 1u) {
    if (l == 0u && r < rows) {
      float o = v;
      if (bias) o = o + bias[r];
      if (res) o = res[r] + o;
      y[r] = o;
    }
    return;
  }
  if (l == 0u && r < rows) split_put(&part[(u64)blockIdx.y * rows + r], v);
  if (split_arrive(arrive + blockIdx.x, gridDim.y)) {
    for (u32 rr = tid; rr < rpg; rr += NTH) {
      const u32 ro = blockIdx.x * rpg + rr;
      if (ro >= rows) continue;
      float o = split_sum_n<true>(part, gridDim.y, rows, ro);
      if (bias) o = o + bias[ro];
      if (res) o = res[ro] + o;
      y[ro] = o;
    }
  }
}

#define GEMVK_KERNELS(KN, KIND)                                                                                                        \
  extern "C" __global__ __launch_bounds__(256) void amdc_gemv_##KN##_k(const uint8_t *W, const uint8_t *xq, float *y, u32 rows, u32 nb, \
                                                                        const float *bias, const float *res, u32 L, float *part,       \
                                                                        u32 *cnt) {                                                    \
    gemvk_body<KIND, false>(W, xq, y, rows, nb, bias, res, L, nullptr, nullptr, part, cnt);                                            \
  }                                                                                                                                    \
  extern "C" __global__ __launch_bounds__(256) void amdc_gemv_##KN##_xk(const uint8_t *W, const float *x, float *y, u32 rows, u32 nb,  \
                                                                         const float *bias, const float *res, u32 L, uint8_t *q8,       \
                                                                         float *part, u32 *cnt) {                                      \
    gemvk_body<KIND, true>(W, nullptr, y, rows, nb, bias, res, L, x, q8, part, cnt);                                                   \
  }
GEMVK_KERNELS(q4_0, AMDC_Q4_0)
GEMVK_KERNELS(q4_k, AMDC_Q4_K)

// ------------------------------------------------------------------ verify GEMV on int8 MFMA (T <= 8)

// y_t = W x_t for T <= 8 Q8 vectors, the weights read once: per pair of
// sub-blocks (g, k), (g + 1, k) of one plane, v_mfma_i32_16x16x64_i8 with
//   A (16 rows x 64): lane (row i, h) = the nibbles of block (g + h / 2, k),
//     low (h even) or high (h odd) half: weights 16 (h & 1) .. + 15
//   B (64 x 16 columns n = t + 8 pp): the 32 activations of token t, block
//     (g + pp, k), in K half pp, zeros in the other half (LDS holds only the
//     nonzero half of each column; the lanes of the other half use 0)
// so that C[r][t + 8 pp] is the exact integer dot of block (g + pp, k) with
// vector t (Q4_K: sum q a; Q4_0: sum q a, then - 8 asum; Q8_0: the int8
// weights of planes 2k, 2k + 1 as A, sum w a).
//
// The float steps are the decode GEMV's, in its order (the super-group tree
// order above), so that y_t equals the decode GEMV of vector t bit for bit
// (the reference's guarantee for its multi-token kernels,
// kernels/ie_kernels.c:481-482): each lane keeps the leaf of each super-group
// of its column (pair p: super-group 2 p + pp of the tile), and per block
//   Q4_0: leaf += (d_w d_a) (dq - 8 asum); Q8_0: leaf += (d_w d_a) dq
//   Q4_K: leaf = fma(-(dmin mn), d_a asum, fma((d sc) dq, d_a, leaf))
// After the tile's 8 planes the leaves of a pair are joined across the two
// columns (a DPP row_ror:8: super-groups 2p, 2p + 1), then the pairs
// ((0 + 1) + (2 + 3)): the tile's subtree of 8 leaves. The tiles of a
// workgroup's K range (an aligned range of S <= 4 tiles, S a power of two) go
// into a pairwise tree kept as a stack (ItemTree's tree, over tiles); the
// ranges' sums are added by amdc_gemm_reduce in the same tree.
//
// Workgroup: 4 row groups of 16 rows (a 64-row tile), each with WS waves: one
// (Q8_0) or two (Q4_0, Q4_K: each wave takes 2 of a tile's 4 pairs of super-
// groups, so that the dependent chain of LDS reads, MFMAs and scale arithmetic
// per plane is half as long; the second wave's tile sum goes to the first
// through the LDS, which adds it in the order above). K in tiles of 8
// super-groups (64 blocks): the tile's activations are staged in LDS,
// B-ready (the zero halves written once), with d_a, d_a asum (or asum) per
// (block, token); each wave builds its scale tables from the headers.
// The weights go from memory straight into LDS (buffer_load ... lds) in whole
// lines: plane k of a tile is 128 contiguous bytes of a row, and each load
// instruction moves 8 rows x 128 bytes (one wave per row group) or 16 rows x
// 64 bytes (two) (register loads in the MFMA's lane order touch 16 rows x 32
// bytes per instruction, which held the vector memory pipeline to about 2.5
// TB/s); the A operand is then read from LDS in lane order. Per wave a ring of
// NS plane steps (Q4: one plane of its rows and columns, 2 or 1 KB; Q8_0: the
// two half planes of a block, 4 KB). The compiler's own waits for loads into
// the LDS are not relied on (it missed one after the loop's back edge): before
// each plane the wave waits explicitly for the loads issued before the plane's
// step (vm_wait, counted from the fixed issue order). Within a wave's plane,
// row i's 16-byte column c holds super-group c ^ swz(i), so that the A reads
// (16 rows, one column pair) fall on distinct banks.
// NH token halves of 8 (T <= 8 NH): the _v16 kernels take two, each A operand
// then feeds two MFMAs.
// Split K over gridDim.y: split ks takes tiles [ks S, ks S + S) (S = tps, at
// most 4), partial sums to part.
__device__ __forceinline__ u32 v8_swz(u32 i) { return (i & 7u) ^ ((i >> 3) & 1u); }
// A workgroup barrier for LDS written with ds_write only: the waves' LDS
// writes are complete (lgkmcnt 0), the compiler keeps memory accesses on their
// side; unlike __syncthreads it does not wait for the loads into LDS in
// flight (each wave's weight ring is its own).
__device__ __forceinline__ void v8_barrier() {
  __builtin_amdgcn_s_waitcnt(0xC07F); // lgkmcnt(0)
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// Wait until at most n vector memory loads of the wave are in flight (gfx9 s_waitcnt: vmcnt in bits
// 3:0 and 15:14, expcnt and lgkmcnt at their maxima). The loads complete in order, so this is how a
// wave knows that its loads into the LDS issued before the last n have landed. n is a constant once
// the caller's loop is unrolled. expcnt(6) marks these waits in the built code (these kernels have no
// exports, so it waits for nothing): tests/test_isa.py finds them there and checks each count against
// the vector memory instructions the compiler actually issued.
__device__ __forceinline__ void vm_wait(u32 n) {
  __asm__ volatile("" ::: "memory");
  switch (n) {
#define VMW(N)                                                                                                                     \
  case N: __builtin_amdgcn_s_waitcnt(0x0F60 | ((N) & 15) | (((N) >> 4) << 14)); break;
    VMW(0) VMW(1) VMW(2) VMW(3) VMW(4) VMW(5) VMW(6) VMW(7) VMW(8) VMW(9) VMW(10) VMW(11) VMW(12) VMW(13) VMW(14) VMW(15)
    VMW(16) VMW(17) VMW(18) VMW(19) VMW(20) VMW(21) VMW(22) VMW(23) VMW(24) VMW(25) VMW(26) VMW(27) VMW(28) VMW(29) VMW(30)
#undef VMW
  default: __builtin_amdgcn_s_waitcnt(0x0F60); break;
  }
  __asm__ volatile("" ::: "memory");
}

// The column swizzle of the verify kernels' B operands in the LDS (sB[..][pair
// p + 4 k][quarter q][column]): column n of (k, q) sits at n ^ v8_bswz(k, q).
// The staging writes of 16 consecutive threads (the 8 blocks k of a
// super-group, both 16-byte halves) then land in 16 distinct 16-byte columns
// instead of one (a 16-way bank conflict), and a quarter-wave's reads of one
// (k, q) stay a permutation of 16 consecutive columns.
__device__ __forceinline__ u32 v8_bswz(u32 k, u32 q) { return ((k << 1) | (q & 1u)) & 15u; }

// A 16-byte-per-lane load into the LDS (lane i's bytes at d + 16 i; d wave-uniform) through an
// inline-asm buffer load, out of the compiler's sight: the compiler waits for every in-flight load into
// the LDS (vmcnt 0) before an LDS read it cannot tell apart from the load's target, which drained the
// verify kernels' weight ring twice per tile. gemv8_body waits for these loads itself (vm_wait,
// from the fixed issue order); the compiler's own vmcnt waits for its register loads only grow
// stronger with loads it does not count (loads complete in issue order). m0 is set and used inside
// the one statement; it is a reserved register the compiler does not let a clobber list preserve, and
// the kernels that use this hold nothing else in it (their built code sets m0 only here). An SALU write
// of m0 needs one wait state before a buffer load with lds = 1 reads it (the gfx9 hazard the compiler
// covers with s_nop 0 for its own LDS loads; the assembler does not insert it into inline asm).
__device__ __forceinline__ void lds_load16(__amdgpu_buffer_rsrc_t rs, __attribute__((address_space(3))) void *d, u32 voff) {
  const u32 m = __builtin_amdgcn_readfirstlane((u32)(__UINTPTR_TYPE__)d);
  __asm__ volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds" ::"s"(m), "v"(voff), "s"(rs) : "memory");
}

template <int KIND, int NS, int NH, int WS>
__device__ __forceinline__ void gemv8_body(const uint8_t *__restrict__ W, const uint8_t *__restrict__ xq, float *__restrict__ y, u32 rows,
                                           u32 nb, const float *__restrict__ bias, const float *__restrict__ res, u32 T, u32 xs, u32 ys,
                                           u32 rs, float *__restrict__ part, u32 tps, u32 *__restrict__ arrive) {
  constexpr u32 SC = KIND == AMDC_Q8_0 ? 2u : 1u; // 2 KB chunks (planes of 16 rows) per step
  static_assert(WS == 1 || SC == 1, "the pair split is built for the nibble kinds");
  constexpr bool K4 = KIND == AMDC_Q4_K;
  constexpr u32 NW = 4u * WS, NTH = 64u * NW; // waves, threads
  constexpr u32 CW = 8u / WS;                 // 16-byte columns (super-groups of the tile) of a plane line per wave
  constexpr u32 SL = SC * 16u * CW;           // u32x4 per ring slot: 16 rows x CW columns (x SC)
  constexpr u32 NPW = 4u / WS;                // pairs of super-groups per wave
  typedef __attribute__((address_space(3))) void lds_t;
  __shared__ __attribute__((aligned(16))) u32x4 sw0[NW][SL];
  __shared__ __attribute__((aligned(16))) u32x4 sw1[NW][SL];
  __shared__ __attribute__((aligned(16))) u32x4 sw2[NS > 2 ? NW : 1][NS > 2 ? SL : 1u];
  __shared__ __attribute__((aligned(16))) u32x4 sw3[NS > 2 ? NW : 1][NS > 2 ? SL : 1u];
  constexpr u32 NTK = 8u * NH;                                      // tokens per launch: NH halves of 8
  // [token half][pair p + 4 k][K quarter][column]: the B operands, read by every lane as they are (the
  // quarters outside a column's half of K hold zeros, written once)
  __shared__ __attribute__((aligned(16))) u32x4 sB[NH][32][4][16];
  __shared__ __attribute__((aligned(16))) float sda[64][NTK];      // d_a [block of tile][token]
  __shared__ __attribute__((aligned(16))) float sxa[64][NTK];      // Q4_K: d_a asum; Q4_0: asum (as int bits)
  // per wave and plane (double-buffered): s (Q4_K d sc, Q4_0 / Q8_0 d) and Q4_K -(dmin mn) [the wave's
  // super-group of the tile][row]
  __shared__ __attribute__((aligned(16))) float ssc[NW][2][CW][16];
  __shared__ __attribute__((aligned(16))) float smn[K4 ? NW : 1][2][CW][16];
  __shared__ __attribute__((aligned(16))) float sx[WS > 1 ? 4 : 1][NH][4][64]; // split pairs: the second wave's tile sums
  const u32 ng = amdc_ngroups(nb), nt = (ng + 7u) >> 3, tid = threadIdx.x, lane = tid & 63u, w = tid >> 6;
  const u32 wr = w & 3u, wp = w >> 2; // the wave's 16 rows, its half of the pairs (WS = 2)
  const u32 i16 = lane & 15u, h = lane >> 4, n = i16, tk = n & 7u, pp = n >> 3;
  const u32 RB = (u32)amdc_row_bytes_k(KIND, nb);
  const u32 rt0 = blockIdx.x * 64u, r0 = rt0 + 16u * wr;
  auto clamp_row = [&](u32 r) { return (r < rows ? r : rows - 1u) - rt0; };
  // a workgroup-uniform resource over the tile's rows; a lane's row in the 32-bit offset
  const __amdgpu_buffer_rsrc_t rw = rsrc(W + (u64)rt0 * RB, (u32)min((u64)(rows - rt0) * RB, (u64)0xFFFFFFF0u));
  const u32 wo = clamp_row(r0 + i16) * RB; // row i16 (headers)
  // the plane loads: one wave: rows lane / 8 and 8 + lane / 8, column lane & 7 (2 instructions); split
  // pairs: row lane / 4, column lane & 3 of the wave's half (1 instruction); column c of row i holds
  // super-group c ^ swz(i) of the wave's columns
  auto swz = [](u32 i) -> u32 { return WS == 1 ? v8_swz(i) : (i >> 1) & 3u; };
  const u32 wl0 = WS == 1 ? clamp_row(r0 + (lane >> 3)) * RB : clamp_row(r0 + (lane >> 2)) * RB;
  const u32 wl1 = clamp_row(r0 + 8u + (lane >> 3)) * RB;
  const u32 g0 = WS == 1 ? (lane & 7u) ^ v8_swz(lane >> 3) : CW * wp + ((lane & 3u) ^ swz(lane >> 2));
  const u32 g1 = (lane & 7u) ^ v8_swz(8u + (lane >> 3));
  const u32 xn = (u32)min((u64)T * xs, (u64)0xFFFFFFF0u);
  const __amdgpu_buffer_rsrc_t rxq = rsrc(xq, xn); // the T Q8 rows
  constexpr u32 OOB = 0xFFFFFFF0u;                 // an offset past every resource: the load returns zeros
  const u32 ks = blockIdx.y, t0 = ks * tps, t1 = t0 + tps < nt ? t0 + tps : nt;
  auto gtile = [&](u32 t) { return ng - 8u * t < 8u ? ng - 8u * t : 8u; };
  auto slot = [&](u32 s) -> u32x4 * {
    if (s == 0u) return sw0[w];
    if (s == 1u) return sw1[w];
    if (s == 2u) return sw2[NS > 2 ? w : 0u];
    return sw3[NS > 2 ? w : 0u];
  };
  // step k of tile t into slot s: chunk c = plane k (Q4) or 2k + c (Q8_0)
  // The compiler does not order LDS reads against these loads into the LDS: the fences keep every read
  // of a slot's previous step ahead of its refill.
  auto issue = [&](u32 t, u32 k, u32 s, bool on) {
    const u32 gt = on ? gtile(t) : 0u; // off: every load out of range (zeros into the slot)
    __asm__ volatile("" ::: "memory");
#pragma unroll
    for (u32 c = 0; c < SC; c++) {
      const u32 pl = SC == 1u ? k : 2u * k + c;
      const u32 base = (KIND == AMDC_Q8_0 ? 2048u : 1024u) * t + 16u * ng + 16u * pl * gt;
      lds_t *d = (lds_t *)(slot(s) + 128u * c);
      lds_load16(rw, d, g0 < gt ? wl0 + base + 16u * g0 : OOB);
      if constexpr (WS == 1)
        lds_load16(rw, (lds_t *)(slot(s) + 128u * c + 64u), g1 < gt ? wl1 + base + 16u * g1 : OOB);
    }
    __asm__ volatile("" ::: "memory");
  };
  // activations of tile t in registers (thread: the 16-byte halves and (block, token) scale pairs i = tid +
  // c NTH); the lane offsets of tile 0 computed once: tile t adds 2048 t (halves), 4 t (scales), 128 t
  // (headers), and a load is valid while its block of the tile is under lim(t)
  constexpr u32 NC4 = 4u * NH / WS, NCS = 2u * NH / WS, NQH = 2u / WS; // halves, scale pairs, headers per thread
  constexpr u32 NFT = NC4 + 2u * NCS + NQH, DPS = SC * (WS == 1 ? 2u : 1u); // loads of fetch_tile, of one ring step
  constexpr u32 FP = 1u; // fetch_tile goes out after plane FP's ring step (plane 0's LDS reads do not wait for it)
  u32x4 ra4[NC4];
  float rd[NCS];
  u32 rx[NCS];
  u32x4 rh[NQH]; // the next tile's headers of row i16: super-groups h + 4 (q + wp) (one wave: h, h + 4)
  u32 xo[NC4], xb[NC4], so[NCS], sbl[NCS];
#pragma unroll
  for (u32 c = 0; c < NC4; c++) {
    const u32 i = tid + c * NTH, half = i & 1u, bl = (i >> 1) & 63u, tok = i >> 7;
    xo[c] = tok < T ? tok * xs + 32u * bl + 16u * half : OOB;
    xb[c] = tok < T ? bl : 64u;
  }
#pragma unroll
  for (u32 c = 0; c < NCS; c++) {
    const u32 i = tid + c * NTH, tok = i & (NTK - 1u), bl = i / NTK;
    so[c] = tok * xs + 4u * bl;
    sbl[c] = tok < T ? bl : 64u;
  }
  auto hgl = [&](u32 q) { return h + 4u * (q + (WS > 1 ? wp : 0u)); }; // the super-group of header q
  auto fetch_tile = [&](u32 t, bool on) {
    const u32 lim = on ? min(8u * gtile(t), nb - 64u * t) : 0u; // blocks of tile t (off: every load out of range)
#pragma unroll
    for (u32 c = 0; c < NC4; c++)
      ra4[c] = __builtin_amdgcn_raw_buffer_load_b128(rxq, xb[c] < lim ? xo[c] + 2048u * t : OOB, 0, 0);
#pragma unroll
    for (u32 c = 0; c < NCS; c++) {
      const bool ok = sbl[c] < lim;
      rd[c] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rxq, ok ? so[c] + 32u * nb + 256u * t : OOB, 0, 0));
      rx[c] = __builtin_amdgcn_raw_buffer_load_b32(rxq, ok ? so[c] + 36u * nb + 256u * t : OOB, 0, 0);
    }
#pragma unroll
    for (u32 q = 0; q < NQH; q++) {
      const u32 gl = hgl(q);
      rh[q] = __builtin_amdgcn_raw_buffer_load_b128(rw, 8u * gl < lim ? wo + 16u * (8u * t + gl) : OOB, 0, 0);
    }
  };
  u32x4 hc[NQH];    // the current tile's headers (rh is refilled with the next tile's during this one)
  float dd[NQH][2]; // Q4_K: d, dmin of hc[q]
  // the scale table of plane k into buffer k & 1: this lane's entries (its headers' super-groups, row i16);
  // the same products as the decode GEMV's (exact: an f16 times a 6-bit integer)
  auto scales = [&](u32 k) {
#pragma unroll
    for (u32 q = 0; q < NQH; q++) {
      const u32 gx = hgl(q) & (CW - 1u);
      if (K4) {
        ssc[w][k & 1u][gx][i16] = dd[q][0] * (float)q4k_sc(hc[q], k);
        smn[K4 ? w : 0u][k & 1u][gx][i16] = -(dd[q][1] * (float)q4k_mn(hc[q], k));
      } else {
        ssc[w][k & 1u][gx][i16] = h2f(hword(hc[q], k >> 1) >> (16u * (k & 1u)));
      }
    }
  };
  auto stage_tile = [&]() {
#pragma unroll
    for (u32 c = 0; c < NC4; c++) { // block (gl, k) of token tok: quarter 2 (gl & 1) + half of column tok % 8 + 8 (gl & 1)
      const u32 i = tid + c * NTH, half = i & 1u, bl = (i >> 1) & 63u, tok = i >> 7, gl = bl >> 3, k = bl & 7u;
      const u32 q_ = 2u * (gl & 1u) + half;
      sB[tok >> 3][(gl >> 1) + 4u * k][q_][((tok & 7u) + 8u * (gl & 1u)) ^ v8_bswz(k, q_)] = ra4[c];
    }
#pragma unroll
    for (u32 c = 0; c < NCS; c++) {
      const u32 i = tid + c * NTH, tok = i & (NTK - 1u), bl = i / NTK;
      sda[bl][tok] = rd[c];
      sxa[bl][tok] = K4 ? rd[c] * (float)(int)rx[c] : __builtin_bit_cast(float, rx[c]);
    }
#pragma unroll
    for (u32 q = 0; q < NQH; q++) {
      hc[q] = rh[q];
      if (K4) dd[q][0] = h2f(hc[q].x), dd[q][1] = h2f(hc[q].x >> 16);
    }
    scales(0u);
  };
  float lf[NH][NPW][4]; // the leaves: [token half][the wave's pair pl (pair NPW wp + pl): super-group 2 p + pp][row 4 h + v]
  // the MFMAs of plane step k (the wave's pairs of the tile) from slot s: pair pl + 1's MFMAs go out before
  // pair pl's results are used (two result sets live)
  // Every pair is computed, also past a partial tile's super-groups: their weights, activations and
  // scales are zeros, so their leaves stay +0 (the value of a leaf not visited), and the code has no
  // branch (the loads and MFMAs of consecutive planes can overlap).
  auto plane = [&](u32 k, u32 s) {
    const u32 pw0 = WS > 1 ? NPW * wp : 0u; // the wave's first pair
    const u32x4 *sl = slot(s);
    const u32 cs = SC == 2u ? 128u * (h & 1u) : 0u; // Q8_0: lanes h odd read the second half plane
    v4i c[NH][2];
    auto mfma = [&](u32 pl) {
      const u32 p = pw0 + pl;
      const u32x4 wq = sl[cs + CW * i16 + ((2u * pl + (h >> 1)) ^ swz(i16))];
      const u32x4 a = KIND == AMDC_Q8_0 ? wq : (wq >> (4u * (h & 1u))) & 0x0F0F0F0Fu;
#pragma unroll
      for (u32 th = 0; th < (u32)NH; th++) {
        const u32x4 bq = sB[th][p + 4u * k][h][n ^ v8_bswz(k, h)];
        c[th][pl & 1u] = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(v4i, a), __builtin_bit_cast(v4i, bq), (v4i){0, 0, 0, 0}, 0, 0, 0);
      }
    };
    mfma(0u);
#pragma unroll
    for (u32 pl = 0; pl < NPW; pl++) {
      if (pl + 1u < NPW) mfma(pl + 1u);
      if (pl == 0u && k + 1u < 8u) scales(k + 1u); // the next plane's table, while the MFMAs run
      const u32 gl = 2u * (pw0 + pl) + pp, bl = 8u * gl + k; // this lane's super-group and block (column pp)
      const v4f s4 = *(const v4f *)&ssc[w][k & 1u][gl & (CW - 1u)][4u * h];
      v4f m4 = {};
      if (K4) m4 = *(const v4f *)&smn[K4 ? w : 0u][k & 1u][gl & (CW - 1u)][4u * h];
#pragma unroll
      for (u32 th = 0; th < (u32)NH; th++) {
        const v4i cp = c[th][pl & 1u];
        const float da = sda[bl][tk + 8u * th];
        if (KIND == AMDC_Q4_0) {
          const u32 as = __builtin_bit_cast(u32, sxa[bl][tk + 8u * th]);
#pragma unroll
          for (u32 v = 0; v < 4u; v++) lf[th][pl][v] += (s4[v] * da) * (float)(int)((u32)cp[v] - 8u * as);
        } else if (KIND == AMDC_Q8_0) {
#pragma unroll
          for (u32 v = 0; v < 4u; v++) lf[th][pl][v] += (s4[v] * da) * (float)cp[v];
        } else {
          const float xa = sxa[bl][tk + 8u * th];
#pragma unroll
          for (u32 v = 0; v < 4u; v++) lf[th][pl][v] = __builtin_fmaf(m4[v], xa, __builtin_fmaf(s4[v] * (float)cp[v], da, lf[th][pl][v]));
        }
      }
    }
  };

  // the tree over the range's tiles: st[j] holds a pending subtree of 2^j tiles, out the range's sum
  float st[2][NH][4], out[NH][4];
#pragma unroll
  for (u32 th = 0; th < (u32)NH; th++)
#pragma unroll
    for (u32 v = 0; v < 4u; v++) out[th][v] = 0.0f, st[0][th][v] = st[1][th][v] = 0.0f;

  // software pipeline over (tile, step): step k uses slot k % NS and, once
  // used, the slot is reloaded with step k + NS (of this tile or the next)
  // the zero quarters of the B operands (column n: the quarters of the other block's half of K)
#pragma unroll
  for (u32 c = 0; c < NC4; c++) {
    const u32 i = tid + c * NTH, n_ = i & 15u, qz = (i >> 4) & 1u, pk = (i >> 5) & 31u, th = i >> 10;
    const u32 q_ = 2u * (1u - (n_ >> 3)) + qz;
    sB[th][pk][q_][n_ ^ v8_bswz(pk >> 2, q_)] = (u32x4)(0u);
  }
  if (t0 < t1) {
    fetch_tile(t0, true);
#pragma unroll
    for (u32 k = 0; k < (u32)NS; k++) issue(t0, k, k, true);
  }
  for (u32 t = t0; t < t1; t++) {
    const bool more = t + 1u < t1;
    v8_barrier(); // the previous tile's readers are done
    stage_tile();
    v8_barrier();
#pragma unroll
    for (u32 th = 0; th < (u32)NH; th++)
#pragma unroll
      for (u32 p = 0; p < NPW; p++)
#pragma unroll
        for (u32 v = 0; v < 4u; v++) lf[th][p][v] = 0.0f;
#pragma unroll
    for (u32 k = 0; k < 8u; k++) {
      // step k's loads into its slot have landed: issued after them are the NS - 1 later steps' and, for
      // steps FP + 1 .. FP + NS, the next tile's activation loads (issued after plane FP's step)
      vm_wait((NS - 1u) * DPS + (k > FP && k <= FP + (u32)NS ? NFT : 0u));
      plane(k, k % (u32)NS);
      // issued also after the range's last tile (as zeros), so that the waits count statically
      if (k + (u32)NS < 8u) issue(t, k + (u32)NS, k % (u32)NS, true);
      else issue(t + 1u, k + (u32)NS - 8u, k % (u32)NS, more);
      if (k == FP) fetch_tile(t + 1u, more); // in flight during this tile (issued also past the range)
    }
    // the tile's subtree: super-groups (2p, 2p + 1) across the two columns, then ((0 + 1) + (2 + 3))
    // (split pairs: the second wave's (2 + 3) through the LDS), then into the tree over tiles (c: the
    // tiles before this one in the range)
    float x[NH][4];
#pragma unroll
    for (u32 th = 0; th < (u32)NH; th++)
#pragma unroll
      for (u32 v = 0; v < 4u; v++) {
        float pr[NPW];
#pragma unroll
        for (u32 p = 0; p < NPW; p++) pr[p] = lf[th][p][v] + dpp<0x128>(lf[th][p][v]); // row_ror:8
        x[th][v] = NPW == 4u ? (pr[0] + pr[1]) + (pr[2 % NPW] + pr[3 % NPW]) : pr[0] + pr[1];
      }
    if constexpr (WS > 1) {
      if (wp) {
#pragma unroll
        for (u32 th = 0; th < (u32)NH; th++)
#pragma unroll
          for (u32 v = 0; v < 4u; v++) sx[wr][th][v][lane] = x[th][v];
      }
      v8_barrier();
      if (!wp) {
#pragma unroll
        for (u32 th = 0; th < (u32)NH; th++)
#pragma unroll
          for (u32 v = 0; v < 4u; v++) x[th][v] = x[th][v] + sx[wr][th][v][lane];
      }
    }
    const u32 c = t - t0;
#pragma unroll
    for (u32 th = 0; th < (u32)NH; th++) {
#pragma unroll
      for (u32 v = 0; v < 4u; v++) {
        float xv = x[th][v];
        if (c & 1u) {
          xv = st[0][th][v] + xv;
          if (c & 2u) out[th][v] = st[1][th][v] + xv; // a range of 4 tiles is complete
          else st[1][th][v] = xv;
        } else {
          st[0][th][v] = xv;
        }
      }
    }
  }
  // a range of fewer than 4 tiles: its pending subtrees, from the lowest level up (zero tiles past the range)
  const u32 cnt = t1 > t0 ? t1 - t0 : 0u;
  if (cnt < 4u) {
#pragma unroll
    for (u32 th = 0; th < (u32)NH; th++)
#pragma unroll
      for (u32 v = 0; v < 4u; v++) out[th][v] = cnt == 3u ? st[1][th][v] + st[0][th][v] : cnt == 2u ? st[1][th][v] : st[0][th][v];
  }
#pragma unroll
  for (u32 th = 0; th < (u32)NH; th++) {
    const u32 tt = tk + 8u * th;
    if (!(WS > 1 && wp) && pp == 0u && tt < T) { // the first wave of the rows holds the sums
#pragma unroll
      for (u32 v = 0; v < 4u; v++) {
        const u32 r = r0 + 4u * h + v;
        if (r >= rows) continue;
        if (part) {
          split_put(&part[((u64)ks * T + tt) * rows + r], out[th][v]);
        } else {
          float o = out[th][v];
          if (bias) o = o + bias[r];
          if (res) o = res[(u64)tt * rs + r] + o;
          y[(u64)tt * ys + r] = o;
        }
      }
    }
  }
  if (part && arrive && split_arrive(arrive + blockIdx.x, gridDim.y))
    split_finish<NTH>(part, gridDim.y, y, rows, rt0, T, bias, res, ys, rs);
}

extern "C" __global__ __launch_bounds__(512) void amdc_gemv_q4_0_v8(const uint8_t *W, const uint8_t *xq, float *y, u32 rows, u32 nb,
                                                                   const float *bias, const float *res, u32 T, u32 xs, u32 ys, u32 rs,
                                                                   float *part, u32 tps, u32 *cnt) {
  gemv8_body<AMDC_Q4_0, 2, 1, 2>(W, xq, y, rows, nb, bias, res, T, xs, ys, rs, part, tps, cnt);
}
extern "C" __global__ __launch_bounds__(512) void amdc_gemv_q4_k_v8(const uint8_t *W, const uint8_t *xq, float *y, u32 rows, u32 nb,
                                                                   const float *bias, const float *res, u32 T, u32 xs, u32 ys, u32 rs,
                                                                   float *part, u32 tps, u32 *cnt) {
  gemv8_body<AMDC_Q4_K, 2, 1, 2>(W, xq, y, rows, nb, bias, res, T, xs, ys, rs, part, tps, cnt);
}
extern "C" __global__ __launch_bounds__(256) void amdc_gemv_q8_0_v8(const uint8_t *W, const uint8_t *xq, float *y, u32 rows, u32 nb,
                                                                   const float *bias, const float *res, u32 T, u32 xs, u32 ys, u32 rs,
                                                                   float *part, u32 tps, u32 *cnt) {
  gemv8_body<AMDC_Q8_0, 2, 1, 1>(W, xq, y, rows, nb, bias, res, T, xs, ys, rs, part, tps, cnt);
}
// the same for up to 16 vectors (two token halves per MFMA A operand)
extern "C" __global__ __launch_bounds__(512) void amdc_gemv_q4_0_v16(const uint8_t *W, const uint8_t *xq, float *y, u32 rows, u32 nb,
                                                                   const float *bias, const float *res, u32 T, u32 xs, u32 ys, u32 rs,
                                                                   float *part, u32 tps, u32 *cnt) {
  gemv8_body<AMDC_Q4_0, 2, 2, 2>(W, xq, y, rows, nb, bias, res, T, xs, ys, rs, part, tps, cnt);
}
extern "C" __global__ __launch_bounds__(512) void amdc_gemv_q4_k_v16(const uint8_t *W, const uint8_t *xq, float *y, u32 rows, u32 nb,
                                                                   const float *bias, const float *res, u32 T, u32 xs, u32 ys, u32 rs,
                                                                   float *part, u32 tps, u32 *cnt) {
  gemv8_body<AMDC_Q4_K, 2, 2, 2>(W, xq, y, rows, nb, bias, res, T, xs, ys, rs, part, tps, cnt);
}
extern "C" __global__ __launch_bounds__(256) void amdc_gemv_q8_0_v16(const uint8_t *W, const uint8_t *xq, float *y, u32 rows, u32 nb,
                                                                   const float *bias, const float *res, u32 T, u32 xs, u32 ys, u32 rs,
                                                                   float *part, u32 tps, u32 *cnt) {
  gemv8_body<AMDC_Q8_0, 1, 2, 1>(W, xq, y, rows, nb, bias, res, T, xs, ys, rs, part, tps, cnt);
}

// The verify GEMV for Q6_K (T <= 8). A Q6_K weight's scale changes every 16
// weights, so each K quarter of v_mfma_i32_16x16x64_i8 is one half sub-block
// and each of the 16 columns one (quarter, token) pair:
//   A (16 rows x 64): lane (row i, h) = q - 32 of the 16 weights of half h & 1
//     of sub-block (g + h / 2, k) (a pair of super-groups, one plane, as the Q4
//     pair kernel): its 16 nibble bytes and its half's high-bit word, then
//     ((v | 0x80) - 0x20) ^ 0x80 per byte
//   B (64 x 16 columns n = 4 q + t): the 16 activations of quarter q for token
//     t (4 tokens per MFMA, two MFMAs for 8), zeros in the other quarters (LDS
//     holds only the nonzero quarter of each column; the other lanes use 0)
// so that C[r][4 q + t] is the exact half dot sum (q - 32) a of ie_q6k_dots for
// quarter q. The float steps are the decode GEMV's, in its order (bit-equal to
// it): the lanes of quarter 0 (2) take quarter 1's (3's) dot from the lane 4
// columns up and apply leaf = fma(fma(s1, d1, s0 d0), d_a, leaf) per block
// (src/cpu.c:142, s = d sc), a leaf per super-group; the tile's 8 leaves join
// as ((g0 + g1) + (g2 + g3)) + ... (row_ror:8 for the pairs), and the tiles of
// a range and the ranges as gemv8_body's (the super-group tree).
// Tiles of 8 super-groups as gemv8_body: activations and d_a staged in LDS in
// B form. The weights go into LDS as in gemv8_body, in whole 128-byte lines: a
// ring step is the nibble planes 2m, 2m + 1 and high-bit plane m of the wave's
// 16 rows (6 KB), 2 steps per wave. The scales: each wave's table of the int8
// sc per (sub-block, half, row) and d per (super-group, row); s = d sc (exact).
// Split K over gridDim.y.
template <int NQ, int NS>
__device__ __forceinline__ void gemv8_q6k_body(const uint8_t *__restrict__ W, const uint8_t *__restrict__ xq, float *__restrict__ y,
                                               u32 rows, u32 nb, const float *__restrict__ bias, const float *__restrict__ res, u32 T,
                                               u32 xs, u32 ys, u32 rs, float *__restrict__ part, u32 tps, u32 *__restrict__ arrive) {
  constexpr u32 NTK = 4u * NQ; // tokens per launch: NQ groups of 4
  typedef __attribute__((address_space(3))) void lds_t;
  constexpr u32 CH = 128u; // u32x4 per 2 KB chunk (16 rows x 128 bytes)
  __shared__ __attribute__((aligned(16))) u32x4 sw0[4][3u * CH]; // per wave: nibble planes 2m, 2m + 1, high plane m
  __shared__ __attribute__((aligned(16))) u32x4 sw1[NS > 1 ? 4 : 1][NS > 1 ? 3u * CH : 1u];
  __shared__ __attribute__((aligned(16))) u32x4 sB[NQ][32][16]; // [token group][pair p + 4 k][column]: the column's nonzero quarter
  __shared__ __attribute__((aligned(16))) float sda[64][NTK];      // d_a [sub-block][token]
  __shared__ __attribute__((aligned(16))) uint8_t ssc[4][64][2][16]; // per wave: the int8 sc [sub-block][half][row]
  __shared__ __attribute__((aligned(16))) float sd[4][8][16];        // per wave: d [super-group][row]
  const u32 ng = nb >> 3, nt = (ng + 7u) >> 3, tid = threadIdx.x, lane = tid & 63u, w = tid >> 6;
  const u32 i16 = lane & 15u, h = lane >> 4, n = i16, qn = n >> 2, tq = n & 3u;
  const u32 RB = (u32)amdc_q6k_row_bytes(nb), D = amdc_q6k_dpad(ng);
  const u32 rt0 = blockIdx.x * 64u, r0 = rt0 + 16u * w;
  auto clamp_row = [&](u32 r) { return (r < rows ? r : rows - 1u) - rt0; };
  const __amdgpu_buffer_rsrc_t rw = rsrc(W + (u64)rt0 * RB, (u32)min((u64)(rows - rt0) * RB, (u64)0xFFFFFFF0u));
  const u32 wo = clamp_row(r0 + i16) * RB;
  const u32 wl0 = clamp_row(r0 + (lane >> 3)) * RB, wl1 = clamp_row(r0 + 8u + (lane >> 3)) * RB; // the plane loads' rows
  const u32 lcol = lane & 7u, g0 = lcol ^ v8_swz(lane >> 3), g1 = lcol ^ v8_swz(8u + (lane >> 3));
  const __amdgpu_buffer_rsrc_t rxq = rsrc(xq, (u32)min((u64)T * xs, (u64)0xFFFFFFF0u));
  constexpr u32 OOB = 0xFFFFFFF0u;
  const u32 ks = blockIdx.y, t0 = ks * tps, t1 = t0 + tps < nt ? t0 + tps : nt;
  auto gtile = [&](u32 t) { return ng - 8u * t < 8u ? ng - 8u * t : 8u; };
  auto slot = [&](u32 s) -> u32x4 * {
    if (s == 0u || NS == 1) return sw0[w];
    return sw1[NS > 1 ? w : 0u];
  };
  // step m of tile t into slot s (off: every load out of range). The slot was read by the planes just
  // before: the wave's LDS reads are complete (lgkmcnt 0) and ordered before the refill (the compiler
  // does not order LDS reads against these loads into the LDS; with a ring of one step the last reads
  // sit right before the refill)
  auto issue = [&](u32 t, u32 m, u32 s, bool on) {
    const u32 gt = on ? gtile(t) : 0u;
    __builtin_amdgcn_s_waitcnt(0xC07F); // lgkmcnt(0)
    __asm__ volatile("" ::: "memory");
#pragma unroll
    for (u32 c = 0; c < 3u; c++) {
      const u32 base = c < 2u ? 16u * ng + D + 1024u * t + 16u * (2u * m + c) * gt : 144u * ng + D + 512u * t + 16u * m * gt;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, (lds_t *)(slot(s) + CH * c), 16, g0 < gt ? wl0 + base + 16u * g0 : OOB, 0, 0, 0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, (lds_t *)(slot(s) + CH * c + 64u), 16, g1 < gt ? wl1 + base + 16u * g1 : OOB, 0, 0, 0);
    }
    __asm__ volatile("" ::: "memory");
  };
  u32x4 ra4[2 * NQ];
  float rd[NQ];
  u32x4 rh[2];
  u32 rdd[2];
  // the tile's activations, d_a and headers into registers (on false: every load past the resource,
  // zeros, so that the loads in flight count statically)
  constexpr u32 NFT = 3u * NQ + 4u; // its loads
  auto fetch_tile = [&](u32 t, bool on) {
    const u32 gt = on ? gtile(t) : 0u;
#pragma unroll
    for (u32 c = 0; c < 2u * NQ; c++) {
      const u32 i = tid + c * NT, half = i & 1u, bl = (i >> 1) & 63u, tok = i >> 7, b = 64u * t + bl;
      const bool ok = tok < T && (bl >> 3) < gt;
      ra4[c] = __builtin_amdgcn_raw_buffer_load_b128(rxq, ok ? tok * xs + 32u * b + 16u * half : OOB, 0, 0);
    }
#pragma unroll
    for (u32 c = 0; c < (u32)NQ; c++) {
      const u32 i = tid + c * NT, tok = i & (NTK - 1u), bl = i / NTK, b = 64u * t + bl;
      const bool ok = tok < T && (bl >> 3) < gt;
      rd[c] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rxq, ok ? tok * xs + 32u * nb + 4u * b : OOB, 0, 0));
    }
#pragma unroll
    for (u32 q = 0; q < 2u; q++) {
      const u32 gl = h + 4u * q, g = 8u * t + gl;
      rh[q] = __builtin_amdgcn_raw_buffer_load_b128(rw, gl < gt ? wo + 16u * g : OOB, 0, 0);
      rdd[q] = __builtin_amdgcn_raw_buffer_load_b16(rw, gl < gt ? wo + (u32)amdc_q6k_d_off(ng, g) : OOB, 0, 0);
    }
  };
  auto stage_tile = [&]() {
#pragma unroll
    for (u32 c = 0; c < 2u * NQ; c++) { // (half, sub-block (gl, k), token) -> quarter 2 (gl & 1) + half of pair gl / 2
      const u32 i = tid + c * NT, half = i & 1u, bl = (i >> 1) & 63u, tok = i >> 7, gl = bl >> 3, k = bl & 7u;
      const u32 q = 2u * (gl & 1u) + half;
      sB[tok >> 2][(gl >> 1) + 4u * k][4u * q + (tok & 3u)] = ra4[c];
    }
#pragma unroll
    for (u32 c = 0; c < (u32)NQ; c++) {
      const u32 i = tid + c * NT;
      sda[i / NTK][i % NTK] = rd[c];
    }
#pragma unroll
    for (u32 q = 0; q < 2u; q++) { // this wave's tables: row i16, super-groups h, h + 4
      const u32 gl = h + 4u * q;
      sd[w][gl][i16] = h2f(rdd[q]);
#pragma unroll
      for (u32 k = 0; k < 8u; k++)
#pragma unroll
        for (u32 e = 0; e < 2u; e++)
          ssc[w][8u * gl + k][e][i16] = (uint8_t)(hword(rh[q], k >> 1) >> (16u * (k & 1u) + 8u * e));
    }
  };
  float lf[NQ][4][4]; // the leaves: [token group][pair p: super-group 2 p + qn / 2 (lanes of an even quarter qn)][row 4 h + v]
  const u32 nth = (T + 3u) >> 2; // token groups with tokens (group 0 always: T >= 1)
  // the MFMAs of plane k = 2 m + e from slot s
  auto plane = [&](u32 m, u32 e, u32 npair, u32 s) {
    const u32 k = 2u * m + e;
    const u32x4 *sl = slot(s);
    v4i c[NQ][2];
    const u32 sft = 4u * (h & 1u);
    auto mfma = [&](u32 p) {
      const u32 col = (2u * p + (h >> 1)) ^ v8_swz(i16);
      const u32x4 wq = sl[CH * e + 8u * i16 + col];
      const u32 hq = ((const u32 *)(sl + 2u * CH + 8u * i16 + col))[2u * e + (h & 1u)];
      u32 a[4];
#pragma unroll
      for (u32 i = 0; i < 4u; i++) {
        const u32 v = ((wq[i] >> sft) & 0x0F0F0F0Fu) | (((hq >> (2u * i)) & 0x03030303u) << 4);
        a[i] = ((v | 0x80808080u) - 0x20202020u) ^ 0x80808080u;
      }
      const v4i av = {(int)a[0], (int)a[1], (int)a[2], (int)a[3]};
#pragma unroll
      for (u32 th = 0; th < (u32)NQ; th++)
        if (th == 0u || th < nth)
          c[th][p & 1u] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, h == qn ? __builtin_bit_cast(v4i, sB[th][p + 4u * k][n]) : (v4i){0, 0, 0, 0},
                                                                 (v4i){0, 0, 0, 0}, 0, 0, 0);
    };
    // pair p + 1's MFMAs go out before pair p's results are used (two result sets live)
    mfma(0u);
#pragma unroll
    for (u32 p = 0; p < 4u; p++) {
      if (p >= npair) break;
      if (p + 1u < npair) mfma(p + 1u);
      // the lanes of an even quarter qn (half 0 of super-group 2 p + qn / 2) take half 1's dot from the
      // lane 4 columns up (row_ror:12) and apply the decode GEMV's block step, src/cpu.c:142:
      // leaf = fma(fma(s1, d1, s0 d0), d_a, leaf), s = d sc (the lanes of odd quarters compute unused values)
      const u32 bl = 8u * (2u * p + (qn >> 1)) + k; // this lane's sub-block
      // d of this lane's 4 rows, read per pair (kept in registers for the 4 pairs it costs the kernel the
      // 256-VGPR limit of two waves per SIMD: 264 VGPRs)
      const v4f dp = *(const v4f *)&sd[w][2u * p + (qn >> 1)][4u * h];
      const u32 sc0 = *(const u32 *)&ssc[w][bl][0][4u * h], sc1 = *(const u32 *)&ssc[w][bl][1][4u * h];
      v4f s0, s1;
#pragma unroll
      for (u32 v = 0; v < 4u; v++) {
        s0[v] = dp[v] * (float)(int)(int8_t)(sc0 >> (8u * v)); // d sc, exact (as the decode GEMV's dsc * sc)
        s1[v] = dp[v] * (float)(int)(int8_t)(sc1 >> (8u * v));
      }
#pragma unroll
      for (u32 th = 0; th < (u32)NQ; th++) {
        if (th > 0u && th >= nth) break;
        const float da = sda[bl][tq + 4u * th];
#pragma unroll
        for (u32 v = 0; v < 4u; v++) {
          const int d0 = c[th][p & 1u][v], d1 = __builtin_amdgcn_update_dpp(0, d0, 0x12C, 0xF, 0xF, false); // row_ror:12: column n + 4
          lf[th][p][v] = __builtin_fmaf(__builtin_fmaf(s1[v], (float)d1, s0[v] * (float)d0), da, lf[th][p][v]);
        }
      }
    }
  };
  // the tree over the range's tiles, as gemv8_body: st[j] a pending subtree of 2^j tiles, out the range's sum
  float st[2][NQ][4], out[NQ][4];
#pragma unroll
  for (u32 th = 0; th < (u32)NQ; th++)
#pragma unroll
    for (u32 v = 0; v < 4u; v++) out[th][v] = 0.0f, st[0][th][v] = st[1][th][v] = 0.0f;
  if (t0 < t1) {
    fetch_tile(t0, true);
#pragma unroll
    for (u32 m = 0; m < (u32)NS; m++) issue(t0, m, m, true);
  }
  for (u32 t = t0; t < t1; t++) {
    const bool more = t + 1u < t1;
    const u32 npair = (gtile(t) + 1u) >> 1;
    v8_barrier(); // the previous tile's readers are done
    stage_tile();
    v8_barrier();
#pragma unroll
    for (u32 th = 0; th < (u32)NQ; th++)
#pragma unroll
      for (u32 p = 0; p < 4u; p++)
#pragma unroll
        for (u32 v = 0; v < 4u; v++) lf[th][p][v] = 0.0f;
#pragma unroll
    for (u32 m = 0; m < 4u; m++) {
      // step m's loads into its slot have landed: issued after them, in this fixed order, are the next
      // step's 6 (NS = 2) and, for steps 1 and 2 (NS = 2) or 1 (NS = 1), the next tile's activation loads
      // (issued after step 0). The compiler's own waits are not relied on: it takes a 1 KB load into the
      // LDS for a 16-byte store and moved the high-bit word read of a freshly refilled slot above its
      // wait (with a one-step ring that read the previous step's bits)
      vm_wait(NS == 2 ? 6u + (m == 1u || m == 2u ? NFT : 0u) : (m == 1u ? NFT : 0u));
      plane(m, 0u, npair, m % (u32)NS);
      plane(m, 1u, npair, m % (u32)NS);
      // issued also after the range's last tile (as zeros), so that the waits count statically
      if (m + (u32)NS < 4u) issue(t, m + (u32)NS, m % (u32)NS, true);
      else issue(t + 1u, m + (u32)NS - 4u, m % (u32)NS, more);
      if (m == 0u) fetch_tile(t + 1u, more); // in flight during this tile (issued also past the range)
    }
    // the tile's subtree: super-groups (2 p, 2 p + 1) from quarters 0 and 2 (row_ror:8), then ((0 + 1) + (2 + 3)),
    // then into the tree over tiles (c: the tiles before this one in the range)
    const u32 c = t - t0;
#pragma unroll
    for (u32 th = 0; th < (u32)NQ; th++)
#pragma unroll
      for (u32 v = 0; v < 4u; v++) {
        float pr[4];
#pragma unroll
        for (u32 p = 0; p < 4u; p++) pr[p] = lf[th][p][v] + dpp<0x128>(lf[th][p][v]); // row_ror:8
        float xv = (pr[0] + pr[1]) + (pr[2] + pr[3]);
        if (c & 1u) {
          xv = st[0][th][v] + xv;
          if (c & 2u) out[th][v] = st[1][th][v] + xv; // a range of 4 tiles is complete
          else st[1][th][v] = xv;
        } else {
          st[0][th][v] = xv;
        }
      }
  }
  // a range of fewer than 4 tiles: its pending subtrees, from the lowest level up (zero tiles past the range)
  const u32 cnt = t1 > t0 ? t1 - t0 : 0u;
  if (cnt < 4u) {
#pragma unroll
    for (u32 th = 0; th < (u32)NQ; th++)
#pragma unroll
      for (u32 v = 0; v < 4u; v++) out[th][v] = cnt == 3u ? st[1][th][v] + st[0][th][v] : cnt == 2u ? st[1][th][v] : st[0][th][v];
  }
  float acc[NQ][4];
#pragma unroll
  for (u32 th = 0; th < (u32)NQ; th++)
#pragma unroll
    for (u32 v = 0; v < 4u; v++) acc[th][v] = out[th][v];
  if (qn == 0u) {
#pragma unroll
    for (u32 th = 0; th < (u32)NQ; th++) {
      const u32 tk = tq + 4u * th;
      if (tk >= T) continue;
#pragma unroll
      for (u32 v = 0; v < 4u; v++) {
        const u32 r = r0 + 4u * h + v;
        if (r >= rows) continue;
        if (part) {
          split_put(&part[((u64)ks * T + tk) * rows + r], acc[th][v]);
        } else {
          float o = acc[th][v];
          if (bias) o = o + bias[r];
          if (res) o = res[(u64)tk * rs + r] + o;
          y[(u64)tk * ys + r] = o;
        }
      }
    }
  }
  if (part && arrive && split_arrive(arrive + blockIdx.x, gridDim.y))
    split_finish<256u>(part, gridDim.y, y, rows, rt0, T, bias, res, ys, rs);
}

extern "C" __global__ __launch_bounds__(256) void amdc_gemv_q6_k_v8(const uint8_t *W, const uint8_t *xq, float *y, u32 rows, u32 nb,
                                                                   const float *bias, const float *res, u32 T, u32 xs, u32 ys, u32 rs,
                                                                   float *part, u32 tps, u32 *cnt) {
  gemv8_q6k_body<2, 2>(W, xq, y, rows, nb, bias, res, T, xs, ys, rs, part, tps, cnt);
}
// up to 16 vectors: four token groups per A operand, a ring of one step (72 KB of LDS, 2 workgroups per CU)
extern "C" __global__ __launch_bounds__(256) void amdc_gemv_q6_k_v16(const uint8_t *W, const uint8_t *xq, float *y, u32 rows, u32 nb,
                                                                    const float *bias, const float *res, u32 T, u32 xs, u32 ys, u32 rs,
                                                                    float *part, u32 tps, u32 *cnt) {
  gemv8_q6k_body<4, 1>(W, xq, y, rows, nb, bias, res, T, xs, ys, rs, part, tps, cnt);
}
