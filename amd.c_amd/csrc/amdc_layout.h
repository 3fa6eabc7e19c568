/* amdc_layout.h -- the CDNA4 weight layout of the quantized GEMV/GEMM path,
 * shared by the host repack (C) and the HIP kernels.
 *
 * A matrix has rows x (32 nb) weights: nb blocks of 32 per row (Q4_0 blocks,
 * or the 32-weight sub-blocks of Q4_K). Blocks are grouped into super-groups
 * of 8 blocks (256 weights; for Q4_K exactly its super-block), ng =
 * ceil(nb / 8) per row. Each row takes 144 ng bytes (= 18 nb, the GGUF size,
 * when nb % 8 == 0), rows one after the other:
 *
 *   header panel  ng x 16 bytes: the scales of super-group g at 16 g
 *     Q4_0: 8 x f16 d (block 8g + k at bytes 2k)
 *     Q4_K: u32 (f16 d | f16 dmin << 16), then the 8 six-bit scales sc_k
 *           packed little endian (sc_k at bit 6k of bytes 4..9) and the 8
 *           six-bit mins mn_k the same way in bytes 10..15
 *   nibble panel  ng x 128 bytes from byte 16 ng: the 16 nibble bytes of
 *     block b = 8g + k (byte j: weight j in the low nibble, weight j + 16 in
 *     the high nibble, the GGUF Q4_0 order) in tiles of 8 super-groups: tile
 *     t = g / 8 holds gt = min(8, ng - 8t) super-groups, plane-major: block
 *     (g, k) at 16 ng + 1024 t + 16 (k gt + g % 8).
 *
 * Why: lane l of a wave owns whole super-groups. It reads its 16-byte header
 * once (lanes l, l+1, ... read consecutive headers) and, for plane k, 16
 * bytes that sit next to those of lanes l +- 1 (consecutive super-groups of
 * one plane are consecutive in a tile): every load is 128 bits wide and every
 * wave load is a run of whole 128-byte lines. The prefill GEMM reads one plane
 * of one tile (8 blocks, 128 contiguous bytes per row) per K step.
 * Blocks past nb (Q4_0 with nb % 8 != 0) are zero bytes with scale 0.
 *
 * Q8_0 (amdc_q8_*): the same super-groups, row = 272 ng bytes (= 34 nb, the
 * GGUF size, when nb % 8 == 0):
 *   header panel  ng x 16 bytes: 8 x f16 d, as Q4_0
 *   int8 panel    ng x 256 bytes from byte 16 ng: 16 planes of 16 bytes per
 *     super-group (plane 2k + h: bytes 16h .. 16h + 15 of block 8g + k), in
 *     tiles of 8 super-groups, plane-major: (g, p) at 16 ng + 2048 t +
 *     16 (p gt + g % 8).
 * Q6_K (amdc_q6k_*, nb % 8 == 0: a super-group is a Q6_K super-block), row =
 * 208 ng + D bytes, D = 2 ng rounded up to 16 (= 210 ng + < 16 padding):
 *   scale panel   ng x 16 bytes: the 16 int8 scales of super-group g at 16 g
 *     (scale 2k + h: half h of sub-block k, the GGUF order)
 *   d panel       ng x 2 bytes from 16 ng: f16 d of super-group g at 2 g
 *   nibble panel  ng x 128 bytes from 16 ng + D: the low 4 bits of each
 *     weight as a Q4_0-order block, placed as the Q4 nibble panel (tiles of
 *     1024 bytes)
 *   high panel    ng x 64 bytes from 144 ng + D: the high 2 bits, two words
 *     per sub-block (word h: weights 16h .. 16h + 15, weight 16h + 4i + e at
 *     bits 8e + 2i, the reference's MAT_Q6K packing, core/ie_core.h:314-349);
 *     plane p (< 4) = the 4 words of sub-blocks 2p, 2p + 1, in tiles of 8
 *     super-groups: (g, p) at 144 ng + D + 512 t + 16 (p gt + g % 8).
 * A lane owning super-group g reads it in 17 (Q8_0) or 13 loads of 128 bits
 * plus one of 16 bits (Q6_K), each a part of a wave-wide run of lines. */
#ifndef AMDC_LAYOUT_H
#define AMDC_LAYOUT_H

#ifdef __cplusplus
#define AMDC_INLINE __host__ __device__ static inline
#else
#define AMDC_INLINE static inline
#endif

#include <stddef.h>
#include <stdint.h>

enum { AMDC_Q4_0 = 0, AMDC_Q8_0 = 2, AMDC_Q4_K = 3, AMDC_Q6_K = 4 }; /* the reference's MAT_* (src/model.h:15) */

/* The size of the kernels' fixed workspace (the device array `scratch`); the same definition as
 * in include/amdc_q4.h, where the host reads it. */
#define AMDC_SCRATCH_BYTES ((size_t)64 << 20)
/* per-tile arrival counters of the split-K verify launches that add their own partial sums */
#define AMDC_SPLIT_TILES 4096u

AMDC_INLINE uint32_t amdc_ngroups(uint32_t nb) { return (nb + 7u) >> 3; }
AMDC_INLINE uint64_t amdc_row_bytes(uint32_t nb) { return 144ull * amdc_ngroups(nb); }
AMDC_INLINE uint64_t amdc_header_off(uint32_t g) { return 16ull * g; }
/* byte offset (inside a row) of the 16 nibble bytes of block k of super-group g */
AMDC_INLINE uint64_t amdc_nib_off(uint32_t ng, uint32_t g, uint32_t k) {
  const uint32_t t = g >> 3, gt = (ng - 8u * t) < 8u ? (ng - 8u * t) : 8u;
  return 16ull * ng + 1024ull * t + 16ull * (k * gt + (g & 7u));
}

/* tile t of 8 super-groups holds gt of them */
AMDC_INLINE uint32_t amdc_tile_gt(uint32_t ng, uint32_t t) { return (ng - 8u * t) < 8u ? (ng - 8u * t) : 8u; }

AMDC_INLINE uint64_t amdc_q8_row_bytes(uint32_t nb) { return 272ull * amdc_ngroups(nb); }
/* plane p (< 16) of super-group g */
AMDC_INLINE uint64_t amdc_q8_off(uint32_t ng, uint32_t g, uint32_t p) {
  return 16ull * ng + 2048ull * (g >> 3) + 16ull * (p * amdc_tile_gt(ng, g >> 3) + (g & 7u));
}

AMDC_INLINE uint32_t amdc_q6k_dpad(uint32_t ng) { return (2u * ng + 15u) & ~15u; }
AMDC_INLINE uint64_t amdc_q6k_row_bytes(uint32_t nb) { return 208ull * amdc_ngroups(nb) + amdc_q6k_dpad(amdc_ngroups(nb)); }
AMDC_INLINE uint64_t amdc_q6k_d_off(uint32_t ng, uint32_t g) { return 16ull * ng + 2ull * g; }
AMDC_INLINE uint64_t amdc_q6k_nib_off(uint32_t ng, uint32_t g, uint32_t k) {
  return 16ull * ng + amdc_q6k_dpad(ng) + 1024ull * (g >> 3) + 16ull * (k * amdc_tile_gt(ng, g >> 3) + (g & 7u));
}
AMDC_INLINE uint64_t amdc_q6k_hi_off(uint32_t ng, uint32_t g, uint32_t p) {
  return 144ull * ng + amdc_q6k_dpad(ng) + 512ull * (g >> 3) + 16ull * (p * amdc_tile_gt(ng, g >> 3) + (g & 7u));
}

/* bytes of a row of any kind */
AMDC_INLINE uint64_t amdc_row_bytes_k(int kind, uint32_t nb) {
  return kind == AMDC_Q8_0 ? amdc_q8_row_bytes(nb) : kind == AMDC_Q6_K ? amdc_q6k_row_bytes(nb) : amdc_row_bytes(nb);
}

#endif
