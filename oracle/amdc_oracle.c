/* amdc_oracle.c -- TEST INFRASTRUCTURE ONLY: the checker of the HIP path.
 *
 * A from-scratch C restatement of the reference's CPU backend for the
 * quantized GEMV path (hanw/amd.c src/cpu.c:36-118, core/ie_core.h,
 * src/model.c:24-31,98-107,142-171,205-219,246-267, src/common.c:25-67).
 * Compiled with -ffp-contract=off and without FMA code generation, as the
 * reference's cpu.c is (plain gcc -O2 on x86-64), so every float operation
 * rounds where the reference's does; explicit fused multiply-adds are fmaf,
 * as in src/cpu.c:112.
 *
 * Integer arithmetic follows core/ie_core.h: u32, wrapping mod 2^32. */
#include "amdc_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

typedef uint32_t u32;

/* ---------------------------------------------------------------- f16 */

/* IEEE binary16 -> binary32, exact (the reference: src/common.c:25-46). */
float or_f16_to_f32(uint16_t h) {
  const u32 s = h >> 15, e = (h >> 10) & 31u, m = h & 1023u;
  float v;
  if (e == 0) v = ldexpf((float)m, -24); /* zero and subnormals: m * 2^-24 */
  else if (e == 31) v = m ? NAN : INFINITY;
  else v = ldexpf((float)(m | 1024u), (int)e - 25);
  return s ? -v : v;
}

/* binary32 -> binary16, round to nearest even (src/common.c:48-67). */
uint16_t or_f32_to_f16(float f) {
  u32 x;
  memcpy(&x, &f, 4);
  const u32 sign = (x >> 16) & 0x8000u, ax = x & 0x7FFFFFFFu;
  if (ax > 0x7F800000u) return (uint16_t)(sign | 0x7E00u);  /* nan */
  if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u); /* >= 65520 (or inf): inf */
  const int e = (int)(ax >> 23) - 127;
  if (e < -14) { /* subnormal half (or zero): units of 2^-24 */
    if (e < -25) return (uint16_t)sign;
    const u32 m = (ax & 0x7FFFFFu) | 0x800000u; /* value = m * 2^(e-23) */
    const int sh = -e - 1;                      /* 14..24: m >> sh = units of 2^-24 */
    u32 q = m >> sh;
    const u32 rem = m & ((1u << sh) - 1u), half = 1u << (sh - 1);
    if (rem > half || (rem == half && (q & 1u))) q++;
    return (uint16_t)(sign | q);
  }
  u32 q = (((u32)(e + 15)) << 10) | ((ax >> 13) & 1023u);
  const u32 rem = ax & 0x1FFFu;
  if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++; /* a carry into the exponent is right */
  return (uint16_t)(sign | q);
}

/* ---------------------------------------------------------------- Q8 */

/* src/cpu.c:36-53: per block of 32, amax = max |x|, d = amax / 127,
 * q = (int)roundf(x / d) (0 if d == 0), asum = the u32 sum of the q. */
void or_quant_q8(const float *x, uint8_t *q, uint32_t nb) {
  int8_t *qv = (int8_t *)q;
  float *dv = (float *)(q + 32u * (size_t)nb);
  u32 *sv = (u32 *)(q + 36u * (size_t)nb);
  for (u32 b = 0; b < nb; b++) {
    const float *xb = x + 32u * (size_t)b;
    float amax = 0.0f;
    for (int j = 0; j < 32; j++) {
      const float a = fabsf(xb[j]);
      amax = fmaxf(amax, a);
    }
    const float d = amax / 127.0f;
    u32 s = 0;
    for (int j = 0; j < 32; j++) {
      const int v = d != 0.0f ? (int)roundf(xb[j] / d) : 0;
      qv[32u * (size_t)b + j] = (int8_t)v;
      s += (u32)v;
    }
    dv[b] = d;
    sv[b] = s;
  }
}

/* src/cpu.c:276-281: the sum of squares in element order, one division, one
 * square root, then (x s) w per element. */
void or_rmsnorm(const float *x, const float *w, float *y, uint32_t n, float eps) {
  float ss = 0.0f;
  for (uint32_t i = 0; i < n; i++) ss += x[i] * x[i];
  const float s = 1.0f / sqrtf(ss / (float)n + eps);
  for (uint32_t i = 0; i < n; i++) y[i] = x[i] * s * w[i];
}

/* src/cpu.c:580 */
void or_swiglu(float *a, const float *b, uint32_t n) {
  for (uint32_t j = 0; j < n; j++) a[j] = a[j] / (1.0f + expf(-a[j])) * b[j];
}

/* ---------------------------------------------------------------- repack */

/* GGUF Q4_0 (18-byte blocks: f16 d, 16 nibble bytes) -> MAT_Q4: word w of
 * block b of row r = nibble bytes 4w..4w+3, little endian
 * (src/model.c:205-219 with core/ie_core.h:69-91). */
void or_repack_q4(const uint8_t *src, uint32_t rows, uint32_t nb, uint32_t *qw, uint16_t *qs) {
  for (size_t i = 0; i < (size_t)rows * nb; i++) {
    const uint8_t *blk = src + 18u * i;
    qs[i] = (uint16_t)(blk[0] | (blk[1] << 8));
    for (u32 w = 0; w < 4; w++)
      qw[4u * i + w] = (u32)blk[2 + 4 * w] | ((u32)blk[3 + 4 * w] << 8) | ((u32)blk[4 + 4 * w] << 16) | ((u32)blk[5 + 4 * w] << 24);
  }
}

/* The 6-bit scale and min of sub-block j (< 8) from the 12 scale bytes of a
 * Q4_K super-block (ggml's get_scale_min_k4; src/model.c:24-31). */
static void q4k_scale_min(u32 j, const uint8_t *s, u32 *sc, u32 *mn) {
  if (j < 4) {
    *sc = s[j] & 63u;
    *mn = s[j + 4] & 63u;
  } else {
    *sc = (s[j + 4] & 15u) | ((u32)(s[j - 4] >> 6) << 4);
    *mn = (u32)(s[j + 4] >> 4) | ((u32)(s[j] >> 6) << 4);
  }
}

size_t or_q4k_qs_n(uint32_t rows, uint32_t nb) { return (size_t)rows * nb + (size_t)rows * (nb / 8u) * 2u; }

/* GGUF Q4_K (144-byte super-blocks: f16 d, f16 dmin, 12 scale bytes, 128
 * nibble bytes; sub-blocks 2k and 2k+1 are the low and high nibbles of bytes
 * 32k..32k+31) -> MAT_Q4K (src/model.c:246-267, core/ie_core.h:258-275):
 * each sub-block as a Q4_0-order block (byte j: weights j (low) and j+16
 * (high)); qs[r*nb + b] = sc | mn << 8; the (d, dmin) pair of super-block s
 * of row r at rows*nb + (r*(nb/8) + s)*2. */
void or_repack_q4k(const uint8_t *src, uint32_t rows, uint32_t nb, uint32_t *qw, uint16_t *qs) {
  const u32 ns = nb / 8u;
  for (u32 r = 0; r < rows; r++)
    for (u32 s = 0; s < ns; s++) {
      const uint8_t *blk = src + ((size_t)r * ns + s) * 144u;
      const size_t dd = (size_t)rows * nb + ((size_t)r * ns + s) * 2u;
      qs[dd] = (uint16_t)(blk[0] | (blk[1] << 8));
      qs[dd + 1] = (uint16_t)(blk[2] | (blk[3] << 8));
      for (u32 k = 0; k < 8; k++) {
        const u32 b = s * 8u + k;
        u32 sc, mn;
        q4k_scale_min(k, blk + 4, &sc, &mn);
        qs[(size_t)r * nb + b] = (uint16_t)(sc | (mn << 8));
        const uint8_t *nib = blk + 16 + 32u * (k / 2u); /* the 32 bytes of the pair */
        uint8_t by[16];
        for (u32 j = 0; j < 16; j++) {
          const u32 lo = (k & 1u) ? (u32)nib[j] >> 4 : nib[j] & 15u;           /* weight j */
          const u32 hi = (k & 1u) ? (u32)nib[j + 16] >> 4 : nib[j + 16] & 15u; /* weight j + 16 */
          by[j] = (uint8_t)(lo | (hi << 4));
        }
        u32 *dst = qw + ((size_t)r * nb + b) * 4u;
        for (u32 w = 0; w < 4; w++)
          dst[w] = (u32)by[4 * w] | ((u32)by[4 * w + 1] << 8) | ((u32)by[4 * w + 2] << 16) | ((u32)by[4 * w + 3] << 24);
      }
    }
}

/* GGUF Q8_0 (34-byte blocks: f16 d, 32 int8) -> MAT_Q8: word w of block b
 * of row r = int8 bytes 4w..4w+3 at (r*nb + b)*8 + w; qs[r*nb + b] = d
 * (src/model.c:221-237, core/ie_core.h:187-198). */
void or_repack_q8(const uint8_t *src, uint32_t rows, uint32_t nb, uint32_t *qw, uint16_t *qs) {
  for (size_t i = 0; i < (size_t)rows * nb; i++) {
    const uint8_t *blk = src + 34u * i;
    qs[i] = (uint16_t)(blk[0] | (blk[1] << 8));
    for (u32 w = 0; w < 8; w++)
      qw[8u * i + w] = (u32)blk[2 + 4 * w] | ((u32)blk[3 + 4 * w] << 8) | ((u32)blk[4 + 4 * w] << 16) | ((u32)blk[5 + 4 * w] << 24);
  }
}

size_t or_q6k_qs_n(uint32_t rows, uint32_t nb) { return (size_t)rows * nb + (size_t)rows * (nb / 8u); }

/* The 6-bit q (0..63) of weight e (< 256) of a GGUF Q6_K super-block
 * (210 bytes: ql[128], qh[64], int8 sc[16], f16 d): e = 128 n + 32 m + l,
 * low 4 bits = nibble (m < 2: low, else high) of ql[64 n + 32 (m & 1) + l],
 * high 2 bits = (qh[32 n + l] >> 2 m) & 3 (core/ie_core.h:309-313, 338-341). */
static u32 q6k_q(const uint8_t *blk, u32 e) {
  const u32 n = e / 128u, m = (e / 32u) % 4u, l = e % 32u;
  const uint8_t lo = blk[64u * n + 32u * (m & 1u) + l];
  const u32 nib = m < 2u ? (lo & 15u) : (u32)(lo >> 4);
  return nib | ((((u32)blk[128u + 32u * n + l] >> (2u * m)) & 3u) << 4);
}

/* GGUF Q6_K -> MAT_Q6K (src/model.c:269-292, core/ie_core.h:314-349): the
 * low 4 bits of sub-block b as a Q4_0-order block at qw word (r*nb + b)*4;
 * the high 2 bits in two words per sub-block at rows*nb*4 + (r*nb + b)*2 + h,
 * weight 16h + 4k + i at bits 8i + 2k; qs[r*nb + b] = sc[2b'] | sc[2b'+1] << 8
 * (b' = b % 8), then the f16 d of super-block s of row r at rows*nb + r*(nb/8) + s. */
void or_repack_q6k(const uint8_t *src, uint32_t rows, uint32_t nb, uint32_t *qw, uint16_t *qs) {
  const u32 ns = nb / 8u;
  for (u32 r = 0; r < rows; r++)
    for (u32 s = 0; s < ns; s++) {
      const uint8_t *blk = src + ((size_t)r * ns + s) * 210u;
      qs[(size_t)rows * nb + (size_t)r * ns + s] = (uint16_t)(blk[208] | (blk[209] << 8));
      for (u32 k = 0; k < 8; k++) {
        const u32 b = s * 8u + k;
        u32 q[32];
        for (u32 j = 0; j < 32; j++) q[j] = q6k_q(blk, 32u * k + j);
        u32 *dst = qw + ((size_t)r * nb + b) * 4u;
        for (u32 w = 0; w < 4; w++) {
          dst[w] = 0;
          for (u32 i = 0; i < 4; i++) dst[w] |= ((q[4 * w + i] & 15u) | ((q[4 * w + i + 16] & 15u) << 4)) << (8 * i);
        }
        u32 *hw = qw + (size_t)rows * nb * 4u + ((size_t)r * nb + b) * 2u;
        for (u32 h = 0; h < 2; h++) {
          hw[h] = 0;
          for (u32 e = 0; e < 16; e++) hw[h] |= (q[16 * h + e] >> 4) << (8u * (e % 4u) + 2u * (e / 4u));
        }
        qs[(size_t)r * nb + b] = (uint16_t)(blk[192 + 2 * k] | (blk[193 + 2 * k] << 8));
      }
    }
}

/* ---------------------------------------------------------------- integer dots */

static inline u32 sext8(u32 v) { return (v & 128u) ? (v | 0xFFFFFF00u) : (v & 255u); }

/* acc + sum over the 4 bytes of (unsigned byte of a) * (signed byte of b),
 * mod 2^32 (the model of the dot4 instruction, core/ie_core.h:113-127). */
static inline u32 dot4_us(u32 acc, u32 a, u32 b) {
  for (u32 e = 0; e < 4; e++) acc += ((a >> (8 * e)) & 255u) * sext8((b >> (8 * e)) & 255u);
  return acc;
}

/* Sum over j < 32 of nibble_j * a_j for the 4 nibble words w and the 8
 * activation words a (core/ie_core.h:137-139, 281-286). */
static inline u32 q4k_dot(const u32 *w, const u32 *a) {
  u32 acc = 0;
  for (u32 k = 0; k < 4; k++) {
    acc = dot4_us(acc, w[k] & 0x0F0F0F0Fu, a[k]);
    acc = dot4_us(acc, (w[k] >> 4) & 0x0F0F0F0Fu, a[k + 4]);
  }
  return acc;
}

/* The Q4_0 block dot: sum (q - 8) a = q4k_dot - 8 asum (core/ie_core.h:161-167). */
static inline u32 q4q8_block(const u32 *w, const u32 *a, u32 asum) { return q4k_dot(w, a) - 8u * asum; }

void or_block_dots_q4(const uint32_t *qw, uint32_t rows, uint32_t nb, const uint8_t *xq, int32_t *out) {
  const u32 *aw = (const u32 *)xq, *asum = (const u32 *)(xq + 36u * (size_t)nb);
  for (size_t r = 0; r < rows; r++)
    for (u32 b = 0; b < nb; b++) out[r * nb + b] = (int32_t)q4q8_block(qw + (r * nb + b) * 4u, aw + 8u * b, asum[b]);
}

void or_block_dots_q4k(const uint32_t *qw, uint32_t rows, uint32_t nb, const uint8_t *xq, int32_t *out) {
  const u32 *aw = (const u32 *)xq;
  for (size_t r = 0; r < rows; r++)
    for (u32 b = 0; b < nb; b++) out[r * nb + b] = (int32_t)q4k_dot(qw + (r * nb + b) * 4u, aw + 8u * b);
}

/* acc + the signed-by-signed dot4 (core/ie_core.h:205-218). */
static inline u32 dot4_ss(u32 acc, u32 a, u32 b) {
  for (u32 e = 0; e < 4; e++) acc += sext8((a >> (8 * e)) & 255u) * sext8((b >> (8 * e)) & 255u);
  return acc;
}

/* The Q8_0 block dot: 8 dot4 of the int8 words (core/ie_core.h:222-233). */
static inline u32 q8q8_block(const u32 *w, const u32 *a) {
  u32 acc = 0;
  for (u32 k = 0; k < 8; k++) acc = dot4_ss(acc, w[k], a[k]);
  return acc;
}

/* Half h of a MAT_Q6K sub-block: sum over its 16 weights of (q - 32) a, by 4
 * signed dot4 of the q - 32 bytes ((v | 0x80) - 0x20) ^ 0x80 per byte, where
 * v = nibble | high bits << 4 (core/ie_core.h:355-389). */
static inline u32 q6k_half(const u32 *nw, u32 hword, const u32 *a, u32 h) {
  u32 acc = 0;
  for (u32 k = 0; k < 4; k++) {
    const u32 nib = h == 0 ? nw[k] & 0x0F0F0F0Fu : (nw[k] >> 4) & 0x0F0F0F0Fu;
    const u32 v = nib | (((hword >> (2u * k)) & 0x03030303u) << 4);
    acc = dot4_ss(acc, ((v | 0x80808080u) - 0x20202020u) ^ 0x80808080u, a[4 * h + k]);
  }
  return acc;
}

void or_block_dots_q8(const uint32_t *qw, uint32_t rows, uint32_t nb, const uint8_t *xq, int32_t *out) {
  const u32 *aw = (const u32 *)xq;
  for (size_t r = 0; r < rows; r++)
    for (u32 b = 0; b < nb; b++) out[r * nb + b] = (int32_t)q8q8_block(qw + (r * nb + b) * 8u, aw + 8u * b);
}

void or_block_dots_q6k(const uint32_t *qw, uint32_t rows, uint32_t nb, const uint8_t *xq, int32_t *out) {
  const u32 *aw = (const u32 *)xq;
  for (size_t r = 0; r < rows; r++)
    for (u32 b = 0; b < nb; b++)
      for (u32 h = 0; h < 2; h++)
        out[(r * nb + b) * 2u + h] =
            (int32_t)q6k_half(qw + (r * nb + b) * 4u, qw[(size_t)rows * nb * 4u + (r * nb + b) * 2u + h], aw + 8u * b, h);
}

/* Nibble j (< 32) of block/sub-block b of row r, straight from the GGUF bytes. */
static u32 gguf_nib(int kind, const uint8_t *src, u32 r, u32 b, u32 j, u32 nb) {
  if (kind == 2) {
    const uint8_t q = src[((size_t)r * nb + b) * 18u + 2u + (j & 15u)];
    return j < 16 ? (q & 15u) : (u32)(q >> 4);
  }
  const uint8_t q = src[((size_t)r * (nb / 8u) + b / 8u) * 144u + 16u + 32u * ((b % 8u) / 2u) + j];
  return (b & 1u) ? (u32)(q >> 4) : (q & 15u);
}

void or_block_dots_gguf(int kind, const uint8_t *src, uint32_t rows, uint32_t nb, const uint8_t *xq, int32_t *out) {
  const int8_t *qa = (const int8_t *)xq;
  for (u32 r = 0; r < rows; r++)
    for (u32 b = 0; b < nb; b++) {
      int64_t s[2] = {0, 0};
      for (u32 j = 0; j < 32; j++) {
        int64_t q;
        if (kind == 8) q = (int8_t)src[((size_t)r * nb + b) * 34u + 2u + j];
        else if (kind == 14) q = (int64_t)q6k_q(src + ((size_t)r * (nb / 8u) + b / 8u) * 210u, 32u * (b % 8u) + j) - 32;
        else q = (int64_t)gguf_nib(kind, src, r, b, j, nb) - (kind == 2 ? 8 : 0);
        s[j / 16u] += q * qa[32u * (size_t)b + j];
      }
      if (kind == 14) out[((size_t)r * nb + b) * 2u] = (int32_t)s[0], out[((size_t)r * nb + b) * 2u + 1u] = (int32_t)s[1];
      else out[(size_t)r * nb + b] = (int32_t)(s[0] + s[1]);
    }
}

/* ---------------------------------------------------------------- GEMV */

/* The 32 lane sums added by the wave tree: shuffle down by 16, 8, 4, 2, 1
 * (src/cpu.c:56-62, core/ie_core.h:438-441). */
static float tree32(float v[32]) {
  for (u32 off = 16; off >= 1; off >>= 1)
    for (u32 i = 0; i < off; i++) v[i] = v[i] + v[i + off];
  return v[0];
}

static void gemv_q4_rows(const uint32_t *qw, const uint16_t *qs, uint32_t r0, uint32_t r1, uint32_t nb, const uint8_t *xq, float *y) {
  const u32 *aw = (const u32 *)xq, *asum = (const u32 *)(xq + 36u * (size_t)nb);
  const float *da = (const float *)(xq + 32u * (size_t)nb);
  for (u32 r = r0; r < r1; r++) {
    float lane[32];
    for (u32 l = 0; l < 32; l++) {
      float acc = 0.0f;
      for (u32 b = l; b < nb; b += 32) {
        const int32_t dot = (int32_t)q4q8_block(qw + ((size_t)r * nb + b) * 4u, aw + 8u * b, asum[b]);
        const float dw = or_f16_to_f32(qs[(size_t)r * nb + b]);
        const float sc = dw * da[b];
        const float t = sc * (float)dot;
        acc = acc + t; /* src/cpu.c:81 */
      }
      lane[l] = acc;
    }
    y[r] = tree32(lane);
  }
}

static void gemv_q4k_rows(const uint32_t *qw, const uint16_t *qs, uint32_t rows, uint32_t r0, uint32_t r1, uint32_t nb, const uint8_t *xq,
                          float *y) {
  const u32 *aw = (const u32 *)xq, *asum = (const u32 *)(xq + 36u * (size_t)nb);
  const float *da = (const float *)(xq + 32u * (size_t)nb);
  for (u32 r = r0; r < r1; r++) {
    float lane[32];
    for (u32 l = 0; l < 32; l++) {
      float acc = 0.0f;
      for (u32 b = l; b < nb; b += 32) {
        const int dq = (int)q4k_dot(qw + ((size_t)r * nb + b) * 4u, aw + 8u * b);
        const u32 sm = qs[(size_t)r * nb + b];
        const size_t dd = (size_t)rows * nb + ((size_t)r * (nb / 8u) + b / 8u) * 2u;
        const float s = or_f16_to_f32(qs[dd]) * (float)(sm & 63u);
        const float mm = or_f16_to_f32(qs[dd + 1]) * (float)(sm >> 8);
        const float x = da[b] * (float)(int)asum[b];
        const float t = s * (float)dq;
        acc = fmaf(-mm, x, fmaf(t, da[b], acc)); /* src/cpu.c:112 */
      }
      lane[l] = acc;
    }
    y[r] = tree32(lane);
  }
}

static void gemv_q8_rows(const uint32_t *qw, const uint16_t *qs, uint32_t r0, uint32_t r1, uint32_t nb, const uint8_t *xq, float *y) {
  const u32 *aw = (const u32 *)xq;
  const float *da = (const float *)(xq + 32u * (size_t)nb);
  for (u32 r = r0; r < r1; r++) {
    float lane[32];
    for (u32 l = 0; l < 32; l++) {
      float acc = 0.0f;
      for (u32 b = l; b < nb; b += 32) {
        const int32_t dot = (int32_t)q8q8_block(qw + ((size_t)r * nb + b) * 8u, aw + 8u * b);
        const float dw = or_f16_to_f32(qs[(size_t)r * nb + b]);
        const float sc = dw * da[b];
        acc = acc + sc * (float)dot; /* src/cpu.c:168 */
      }
      lane[l] = acc;
    }
    y[r] = tree32(lane);
  }
}

static void gemv_q6k_rows(const uint32_t *qw, const uint16_t *qs, uint32_t rows, uint32_t r0, uint32_t r1, uint32_t nb, const uint8_t *xq,
                          float *y) {
  const u32 *aw = (const u32 *)xq;
  const float *da = (const float *)(xq + 32u * (size_t)nb);
  for (u32 r = r0; r < r1; r++) {
    float lane[32];
    for (u32 l = 0; l < 32; l++) {
      float acc = 0.0f;
      for (u32 b = l; b < nb; b += 32) {
        const size_t i = (size_t)r * nb + b;
        const u32 *hw = qw + (size_t)rows * nb * 4u + i * 2u;
        const int d0 = (int)q6k_half(qw + i * 4u, hw[0], aw + 8u * b, 0);
        const int d1 = (int)q6k_half(qw + i * 4u, hw[1], aw + 8u * b, 1);
        const u32 sc = qs[i];
        const float d = or_f16_to_f32(qs[(size_t)rows * nb + (size_t)r * (nb / 8u) + b / 8u]);
        const float s0 = d * (float)(int8_t)(sc & 255u), s1 = d * (float)(int8_t)(sc >> 8);
        acc = fmaf(fmaf(s1, (float)d1, s0 * (float)d0), da[b], acc); /* src/cpu.c:142 */
      }
      lane[l] = acc;
    }
    y[r] = tree32(lane);
  }
}

void or_gemv_q8(const uint32_t *qw, const uint16_t *qs, uint32_t rows, uint32_t nb, const uint8_t *xq, float *y) {
  gemv_q8_rows(qw, qs, 0, rows, nb, xq, y);
}

void or_gemv_q6k(const uint32_t *qw, const uint16_t *qs, uint32_t rows, uint32_t nb, const uint8_t *xq, float *y) {
  gemv_q6k_rows(qw, qs, rows, 0, rows, nb, xq, y);
}

void or_gemv_q4(const uint32_t *qw, const uint16_t *qs, uint32_t rows, uint32_t nb, const uint8_t *xq, float *y) {
  gemv_q4_rows(qw, qs, 0, rows, nb, xq, y);
}

void or_gemv_q4k(const uint32_t *qw, const uint16_t *qs, uint32_t rows, uint32_t nb, const uint8_t *xq, float *y) {
  gemv_q4k_rows(qw, qs, rows, 0, rows, nb, xq, y);
}

void or_epilogue(float *y, uint32_t rows, const float *bias, const float *res) {
  for (u32 r = 0; r < rows; r++) {
    float v = y[r];
    if (bias) v = v + bias[r];
    if (res) v = res[r] + v;
    y[r] = v;
  }
}

/* ---------------------------------------------------------------- dequant, f64 */

void or_dequant(int kind, const uint8_t *src, uint64_t first, uint64_t n, float *out) {
  for (uint64_t i = 0; i < n; i++) {
    const uint64_t e = first + i;
    if (kind == 8) { /* src/model.c:89-97 */
      const uint8_t *blk = src + e / 32 * 34;
      out[i] = or_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8))) * (float)(int8_t)blk[2 + e % 32];
    } else if (kind == 14) { /* src/model.c:108-140: d * sc[e / 16] * (q - 32) */
      const uint8_t *blk = src + e / 256 * 210;
      const u32 k = (u32)(e % 256);
      const float d = or_f16_to_f32((uint16_t)(blk[208] | (blk[209] << 8)));
      out[i] = d * (float)(int8_t)blk[192 + k / 16] * (float)((int)q6k_q(blk, k) - 32);
    } else if (kind == 2) { /* src/model.c:98-107 */
      const uint8_t *blk = src + e / 32 * 18;
      const u32 j = (u32)(e % 32), q = j < 16 ? (blk[2 + j] & 15u) : (u32)(blk[2 + j - 16] >> 4);
      out[i] = or_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8))) * (float)((int)q - 8);
    } else { /* Q4_K, src/model.c:142-171 */
      const uint8_t *blk = src + e / 256 * 144;
      const u32 k = (u32)(e % 256), sub = k / 32, j = k % 32;
      u32 sc, mn;
      q4k_scale_min(sub, blk + 4, &sc, &mn);
      const float d = or_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8))), dmin = or_f16_to_f32((uint16_t)(blk[2] | (blk[3] << 8)));
      const uint8_t qb = blk[16 + 32 * (sub / 2) + j];
      const u32 q = (sub & 1u) ? (u32)(qb >> 4) : (qb & 15u);
      const float d1 = d * (float)sc, m1 = dmin * (float)mn;
      out[i] = d1 * (float)q - m1;
    }
  }
}

void or_gemv_f64(int kind, const uint8_t *src, uint32_t rows, uint32_t nb, const uint8_t *xq, double *y_ref, double *mag) {
  const int8_t *qa = (const int8_t *)xq;
  const float *da = (const float *)(xq + 32u * (size_t)nb);
  float *w = malloc((size_t)nb * 32u * sizeof(float));
  for (u32 r = 0; r < rows; r++) {
    or_dequant(kind, src, (uint64_t)r * nb * 32u, (uint64_t)nb * 32u, w);
    double acc = 0, m = 0;
    for (u32 b = 0; b < nb; b++)
      for (u32 j = 0; j < 32; j++) {
        const double t = (double)w[32u * b + j] * (double)da[b] * (double)qa[32u * (size_t)b + j];
        acc += t;
        m += fabs(t);
      }
    y_ref[r] = acc;
    mag[r] = m;
  }
  free(w);
}

/* ---------------------------------------------------------------- threads */

typedef struct {
  const uint32_t *qw;
  const uint16_t *qs;
  uint32_t rows, r0, r1, nb;
  const uint8_t *xq;
  float *y;
  int kind; /* 0 Q4_0, 2 Q8_0, 3 Q4_K, 4 Q6_K */
} job;

static void *run_job(void *p) {
  const job *j = p;
  switch (j->kind) {
    case 3: gemv_q4k_rows(j->qw, j->qs, j->rows, j->r0, j->r1, j->nb, j->xq, j->y); break;
    case 4: gemv_q6k_rows(j->qw, j->qs, j->rows, j->r0, j->r1, j->nb, j->xq, j->y); break;
    case 2: gemv_q8_rows(j->qw, j->qs, j->r0, j->r1, j->nb, j->xq, j->y); break;
    default: gemv_q4_rows(j->qw, j->qs, j->r0, j->r1, j->nb, j->xq, j->y);
  }
  return NULL;
}

static void gemv_mt(int kind, const uint32_t *qw, const uint16_t *qs, uint32_t rows, uint32_t nb, const uint8_t *xq, float *y, int nt) {
  if (nt < 1) nt = 1;
  if (nt > 256) nt = 256;
  pthread_t th[256];
  job jb[256];
  for (int i = 0; i < nt; i++) {
    jb[i] = (job){qw, qs, rows, (u32)((uint64_t)rows * i / nt), (u32)((uint64_t)rows * (i + 1) / nt), nb, xq, y, kind};
    if (i > 0) pthread_create(&th[i], NULL, run_job, &jb[i]);
  }
  run_job(&jb[0]);
  for (int i = 1; i < nt; i++) pthread_join(th[i], NULL);
}

void or_gemv_q4_mt(const uint32_t *qw, const uint16_t *qs, uint32_t rows, uint32_t nb, const uint8_t *xq, float *y, int nthreads) {
  gemv_mt(0, qw, qs, rows, nb, xq, y, nthreads);
}
void or_gemv_q4k_mt(const uint32_t *qw, const uint16_t *qs, uint32_t rows, uint32_t nb, const uint8_t *xq, float *y, int nthreads) {
  gemv_mt(3, qw, qs, rows, nb, xq, y, nthreads);
}
void or_gemv_q8_mt(const uint32_t *qw, const uint16_t *qs, uint32_t rows, uint32_t nb, const uint8_t *xq, float *y, int nthreads) {
  gemv_mt(2, qw, qs, rows, nb, xq, y, nthreads);
}
void or_gemv_q6k_mt(const uint32_t *qw, const uint16_t *qs, uint32_t rows, uint32_t nb, const uint8_t *xq, float *y, int nthreads) {
  gemv_mt(4, qw, qs, rows, nb, xq, y, nthreads);
}

/* or_dequant over up to 256 threads, each a range of whole 256-weight groups. */
typedef struct {
  int kind;
  const uint8_t *src;
  uint64_t first, n;
  float *out;
} dq_job;

static void *run_dq(void *p) {
  const dq_job *j = p;
  or_dequant(j->kind, j->src, j->first, j->n, j->out + j->first);
  return NULL;
}

void or_dequant_mt(int kind, const uint8_t *src, uint64_t n, float *out, int nt) {
  if (nt < 1) nt = 1;
  if (nt > 256) nt = 256;
  pthread_t th[256];
  dq_job jb[256];
  const uint64_t groups = (n + 255u) / 256u;
  for (int i = 0; i < nt; i++) {
    const uint64_t a = groups * (uint64_t)i / (uint64_t)nt * 256u, b = groups * (uint64_t)(i + 1) / (uint64_t)nt * 256u;
    jb[i] = (dq_job){kind, src, a < n ? a : n, (b < n ? b : n) - (a < n ? a : n), out};
    if (i > 0) pthread_create(&th[i], NULL, run_dq, &jb[i]);
  }
  run_dq(&jb[0]);
  for (int i = 1; i < nt; i++) pthread_join(th[i], NULL);
}
