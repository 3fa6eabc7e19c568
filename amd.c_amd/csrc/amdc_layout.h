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
 * Blocks past nb (Q4_0 with nb % 8 != 0) are zero bytes with scale 0. */
#ifndef AMDC_LAYOUT_H
#define AMDC_LAYOUT_H

#ifdef __cplusplus
#define AMDC_INLINE __host__ __device__ static inline
#else
#define AMDC_INLINE static inline
#endif

#include <stddef.h>
#include <stdint.h>

enum { AMDC_Q4_0 = 0, AMDC_Q4_K = 3 }; /* the reference's MAT_Q4 / MAT_Q4K (src/model.h:15) */

AMDC_INLINE uint32_t amdc_ngroups(uint32_t nb) { return (nb + 7u) >> 3; }
AMDC_INLINE uint64_t amdc_row_bytes(uint32_t nb) { return 144ull * amdc_ngroups(nb); }
AMDC_INLINE uint64_t amdc_header_off(uint32_t g) { return 16ull * g; }
/* byte offset (inside a row) of the 16 nibble bytes of block k of super-group g */
AMDC_INLINE uint64_t amdc_nib_off(uint32_t ng, uint32_t g, uint32_t k) {
  const uint32_t t = g >> 3, gt = (ng - 8u * t) < 8u ? (ng - 8u * t) : 8u;
  return 16ull * ng + 1024ull * t + 16ull * (k * gt + (g & 7u));
}

#endif
