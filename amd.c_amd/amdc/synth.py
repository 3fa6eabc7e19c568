"""Seeded synthetic GGUF weights and activations for the configurations of the
benchmark (weights: uniform nibbles; Q4_0 f16 d = |N(0,1)| * 0.02; Q4_K f16
d, dmin = |N(0,1)| * 0.01 and uniform 6-bit scales and mins; activations
f32 N(0,1)). numpy's float32 -> float16 cast rounds to nearest even, as the
reference's ie_f32_to_f16 (hanw/amd.c src/common.c:48-67).

GGUF Q4_0 block (18 bytes): f16 d, 16 nibble bytes (core/ie_core.h:66-68).
GGUF Q4_K super-block (144 bytes): f16 d, f16 dmin, 12 bytes of 6-bit scales
and mins, 128 nibble bytes (core/ie_core.h:247-251).
GGUF Q8_0 block (34 bytes): f16 d, 32 int8 (core/ie_core.h:187-192): f16 d =
|N(0,1)| * 0.004, uniform bytes (-128 included).
GGUF Q6_K super-block (210 bytes): ql[128], qh[64], int8 scales[16], f16 d
(core/ie_core.h:309-313): uniform bytes, uniform int8 scales, f16 d =
|N(0,1)| * 0.0005.
"""
import numpy as np

KIND_Q4_0, KIND_Q8_0, KIND_Q4_K, KIND_Q6_K = 0, 2, 3, 4  # the reference's MAT_* (src/model.h:15)
GGML = {KIND_Q4_0: 2, KIND_Q8_0: 8, KIND_Q4_K: 12, KIND_Q6_K: 14}
# GGUF bytes per 32 weights, and the weights per GGUF block
BYTES_PER_32 = {KIND_Q4_0: 18.0, KIND_Q8_0: 34.0, KIND_Q4_K: 18.0, KIND_Q6_K: 26.25}
BLOCK_WEIGHTS = {KIND_Q4_0: 32, KIND_Q8_0: 32, KIND_Q4_K: 256, KIND_Q6_K: 256}


def rng(seed):
    return np.random.Generator(np.random.PCG64(seed))


def gguf_q4_0(rows, cols, seed, scale=0.02):
    """rows x cols Q4_0 weights as GGUF bytes (rows * cols / 32 * 18)."""
    assert cols % 32 == 0
    g = rng(seed)
    n = rows * (cols // 32)
    blk = np.empty((n, 18), dtype=np.uint8)
    d = (np.abs(g.standard_normal(n, dtype=np.float32)) * np.float32(scale)).astype(np.float16)
    blk[:, 0:2] = d.view(np.uint8).reshape(n, 2)
    blk[:, 2:] = g.integers(0, 256, size=(n, 16), dtype=np.uint8)
    return blk.reshape(-1)


def gguf_q4_k(rows, cols, seed, scale=0.01):
    """rows x cols Q4_K weights as GGUF bytes (rows * cols / 256 * 144)."""
    assert cols % 256 == 0
    g = rng(seed)
    n = rows * (cols // 256)
    blk = np.empty((n, 144), dtype=np.uint8)
    dd = (np.abs(g.standard_normal((n, 2), dtype=np.float32)) * np.float32(scale)).astype(np.float16)
    blk[:, 0:4] = dd.view(np.uint8).reshape(n, 4)
    blk[:, 4:] = g.integers(0, 256, size=(n, 140), dtype=np.uint8)
    return blk.reshape(-1)


def gguf_q8_0(rows, cols, seed, scale=0.004):
    """rows x cols Q8_0 weights as GGUF bytes (rows * cols / 32 * 34)."""
    assert cols % 32 == 0
    g = rng(seed)
    n = rows * (cols // 32)
    blk = np.empty((n, 34), dtype=np.uint8)
    d = (np.abs(g.standard_normal(n, dtype=np.float32)) * np.float32(scale)).astype(np.float16)
    blk[:, 0:2] = d.view(np.uint8).reshape(n, 2)
    blk[:, 2:] = g.integers(0, 256, size=(n, 32), dtype=np.uint8)
    return blk.reshape(-1)


def gguf_q6_k(rows, cols, seed, scale=0.0005):
    """rows x cols Q6_K weights as GGUF bytes (rows * cols / 256 * 210)."""
    assert cols % 256 == 0
    g = rng(seed)
    n = rows * (cols // 256)
    blk = np.empty((n, 210), dtype=np.uint8)
    blk[:, 0:208] = g.integers(0, 256, size=(n, 208), dtype=np.uint8)
    d = (np.abs(g.standard_normal(n, dtype=np.float32)) * np.float32(scale)).astype(np.float16)
    blk[:, 208:210] = d.view(np.uint8).reshape(n, 2)
    return blk.reshape(-1)


_GEN = {KIND_Q4_0: gguf_q4_0, KIND_Q8_0: gguf_q8_0, KIND_Q4_K: gguf_q4_k, KIND_Q6_K: gguf_q6_k}


def gguf(kind, rows, cols, seed):
    return _GEN[kind](rows, cols, seed)


def activations(T, cols, seed):
    """T f32 ~ N(0,1) vectors of cols elements."""
    return rng(seed).standard_normal((T, cols), dtype=np.float32)


def gguf_bytes(kind, rows, cols):
    return int(rows * cols // 32 * BYTES_PER_32[kind])


# The configurations (rows x cols = N outputs x K inputs).
CONFIGS = {
    "c0": {"kind": KIND_Q4_0, "T": 1, "shapes": [("q4096x4096", 4096, 4096)]},
    "c1": {"kind": KIND_Q4_0, "T": 1, "shapes": [
        ("q", 4096, 4096), ("k", 4096, 4096), ("v", 4096, 4096), ("o", 4096, 4096),
        ("gate", 11008, 4096), ("up", 11008, 4096), ("down", 4096, 11008), ("lm_head", 32000, 4096)]},
    "c2": {"kind": KIND_Q4_K, "T": 1, "shapes": [
        ("ffn_gate", 17408, 5120), ("ffn_up", 17408, 5120), ("ffn_down", 5120, 17408),
        ("attn_in", 6144, 5120), ("attn_out", 5120, 6144), ("lm_head", 152064, 5120)]},
    "c3": {"T": 8, "shapes": [
        ("q4k_ffn_up", 17408, 5120, KIND_Q4_K), ("q4k_ffn_down", 5120, 17408, KIND_Q4_K),
        ("q4_0_gate", 11008, 4096, KIND_Q4_0)]},
    "c4": {"kind": KIND_Q4_K, "T": 256, "shapes": [("ffn_up", 17408, 5120), ("ffn_down", 5120, 17408)]},
}
