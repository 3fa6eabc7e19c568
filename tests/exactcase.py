"""Weights and activations on which every float step of the GEMV / GEMM is exact.

All scales (f16 d, dmin) are powers of two (Q4_0, Q8_0: {1/2, 1, 2}; Q4_K,
Q6_K: {1/2, 1}), the Q4_K sub-block scales are 1..3 and mins 0..3, the Q6_K
int8 scales -2..2, the Q8_0 weights -16..16, and every activation block holds
integers in [-2, 2] with one element at +-127, so that cpu_quant_q8 gives
d_a = 127 / 127 = 1 and q = x. Every product of the reference's per-block
arithmetic (src/cpu.c:81, 111-112, 142, 168) is then a multiple of 1/2, and
so is every sum of them. ``bound`` is the largest magnitude any sum of a
row's products can take (a block's |sum q a| <= max |q| sum |a| <= max |q|
189, times the largest scale, plus the min term); below 2^23 every partial
sum, in any order and of any grouping (tree, split K, f16-MFMA tiles, fma
chains), is a float32 without rounding. The
result of a correct kernel is therefore one number, bit for bit, and a
kernel whose integer block sum is off by one differs from it by at least 1/2.
"""
import numpy as np

from amdc import synth

POW2 = np.array([0.5, 1.0, 2.0], dtype=np.float16)
AMAX = 127 + 31 * 2  # the largest sum |a| of a block
# the largest |d sc q| + |dmin mn| of a weight, per kind
WMAX = {synth.KIND_Q4_0: 2 * 8, synth.KIND_Q8_0: 2 * 16, synth.KIND_Q4_K: 1 * 3 * 15 + 1 * 3, synth.KIND_Q6_K: 1 * 2 * 32}


def bound(kind, nb):
    return nb * WMAX[kind] * AMAX


def _rng(seed):
    return np.random.Generator(np.random.PCG64(seed))


def gguf(kind, rows, cols, seed):
    """GGUF bytes of an exact case (the layouts of synth.py)."""
    g = _rng(seed)
    if kind in (synth.KIND_Q4_0, synth.KIND_Q8_0):
        n = rows * (cols // 32)
        size = 18 if kind == synth.KIND_Q4_0 else 34
        blk = np.empty((n, size), dtype=np.uint8)
        blk[:, 0:2] = POW2[g.integers(0, 3, n)].view(np.uint8).reshape(n, 2)
        if kind == synth.KIND_Q4_0:
            blk[:, 2:] = g.integers(0, 256, size=(n, 16), dtype=np.uint8)
        else:
            blk[:, 2:] = g.integers(-16, 17, size=(n, 32)).astype(np.int8).view(np.uint8)
        return blk.reshape(-1)
    n = rows * (cols // 256)
    if kind == synth.KIND_Q4_K:
        blk = np.empty((n, 144), dtype=np.uint8)
        blk[:, 0:4] = POW2[g.integers(0, 2, (n, 2))].view(np.uint8).reshape(n, 4)
        sc = g.integers(1, 4, (n, 8))
        mn = g.integers(0, 4, (n, 8))
        # get_scale_min_k4 (src/model.c:24-31) for values below 16: bytes 0..3 = sc 0..3, 4..7 = mn 0..3,
        # 8..11 = sc 4..7 | mn 4..7 << 4 (the 2-bit high parts stay 0)
        blk[:, 4:8] = sc[:, 0:4]
        blk[:, 8:12] = mn[:, 0:4]
        blk[:, 12:16] = sc[:, 4:8] | (mn[:, 4:8] << 4)
        blk[:, 16:] = g.integers(0, 256, size=(n, 128), dtype=np.uint8)
        return blk.reshape(-1)
    assert kind == synth.KIND_Q6_K
    blk = np.empty((n, 210), dtype=np.uint8)
    blk[:, 0:192] = g.integers(0, 256, size=(n, 192), dtype=np.uint8)
    blk[:, 192:208] = g.integers(-2, 3, size=(n, 16)).astype(np.int8).view(np.uint8)
    blk[:, 208:210] = POW2[g.integers(0, 2, n)].view(np.uint8).reshape(n, 2)
    return blk.reshape(-1)


def activations(T, cols, seed):
    """T vectors of integers in [-2, 2], one +-127 per block of 32 (so d_a = 1)."""
    g = _rng(seed)
    x = g.integers(-2, 3, size=(T, cols // 32, 32)).astype(np.float32)
    pos = g.integers(0, 32, size=(T, cols // 32))
    sign = np.where(g.integers(0, 2, size=(T, cols // 32)) == 1, 127.0, -127.0).astype(np.float32)
    np.put_along_axis(x, pos[..., None], sign[..., None], axis=2)
    return x.reshape(T, cols)


def exact_y(orc, kind, src, rows, nb, xq):
    """The exact result of one vector: the oracle's float64 sum, checked to be exact in float32."""
    assert bound(kind, nb) < 2 ** 23, "the case is not exact at this nb"
    y64, _ = orc.gemv_f64(synth.GGML[kind], src, rows, nb, xq)
    y = y64.astype(np.float32)
    assert np.array_equal(y.astype(np.float64), y64), "the float64 sum is not a float32"
    return y
