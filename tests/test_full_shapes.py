"""Q4_0 / Q4_K parity at the full shapes of every benchmark configuration (c0-c4), through the
entry points a caller uses and the host's own choices (decode form, lanes per row, workgroups,
verify K split and tile ranges, GEMM tile and K split): no tuning overrides.

Every row of every token is compared with the oracle (the reference's cpu.c order, src/cpu.c:64-118)
within 1e-5 of sum |terms| (|W| |x| from the dequantized weights), and the verify results of each
token equal the decode GEMV of that token bit for bit (the reference's multi-token guarantee,
kernels/ie_kernels.c:481-482).
"""
import os

import numpy as np
import pytest

from amdc import synth

pytestmark = pytest.mark.gpu
TOL = 1e-5
CPUS = min(16, os.cpu_count() or 1)
Q40, Q4K = synth.KIND_Q4_0, synth.KIND_Q4_K


def q8_stride(nb):
    return (40 * nb + 255) // 256 * 256  # token rows 256-aligned (src/model.c:1194)


class Mat:
    """One seeded matrix on the host (GGUF bytes, the reference layout, |W|) and the device."""

    def __init__(self, dev, orc, kind, rows, cols, seed):
        self.kind, self.rows, self.nb = kind, rows, cols // 32
        self.tt = synth.GGML[kind]
        self.src = synth.gguf(kind, rows, cols, seed)
        self.qw, self.qs = orc.repack(self.tt, self.src, rows, self.nb)
        self.absw = np.abs(orc.dequant(self.tt, self.src, rows * cols, threads=CPUS)).reshape(rows, cols)
        self.W = dev.DevBuf.of(dev.repack(kind, self.src, rows, cols))
        self.orc = orc

    def oracle(self, xq):
        return self.orc.gemv(self.tt, self.qw, self.qs, self.rows, self.nb, xq, threads=CPUS)

    def mag(self, xq):
        """sum |terms| per row for each Q8 vector of xq [T, 40 nb]: |W| |q d_a|."""
        nb = self.nb
        q = xq[:, :32 * nb].view(np.int8).astype(np.float32).reshape(-1, nb, 32)
        d = xq[:, 32 * nb:36 * nb].copy().view(np.float32)
        a = np.abs(q * d[:, :, None]).reshape(-1, 32 * nb)
        return (self.absw @ a.T).T.astype(np.float64)

    def free(self):
        self.W.free()


def check(y, want, mag, what):
    err = np.abs(y.astype(np.float64) - want.astype(np.float64)) / np.maximum(mag, 1e-30)
    i = int(np.argmax(err))
    assert err.flat[i] < TOL, f"{what}: rel err {err.flat[i]:.3e} at {np.unravel_index(i, err.shape)}"


def decode_case(dev, orc, kind, rows, cols, seed):
    m = Mat(dev, orc, kind, rows, cols, seed)
    x = synth.activations(1, cols, seed + 1)
    xq = orc.quant_q8(x)
    want, mag = m.oracle(xq[0]), m.mag(xq)[0]
    X, Q, Y, Y2 = dev.DevBuf.of(x), dev.DevBuf(q8_stride(m.nb)), dev.DevBuf(4 * rows), dev.DevBuf(4 * rows)
    print(f"decode kind {kind} {rows}x{cols}", flush=True)
    Q.fill(0)
    dev.gemv_x(kind, m.W, X, Y, rows, m.nb, q8=Q)  # the f32-input decode (the bench's step)
    assert np.array_equal(Q.download(np.uint8)[:40 * m.nb], xq[0])
    check(Y.download(np.float32), want, mag, "gemv_x")
    dev.op_gemv(kind, m.W, Q, Y2, rows, m.nb, 1, q8_stride(m.nb), rows)  # the dispatcher at T = 1
    check(Y2.download(np.float32), want, mag, "op_gemv")
    assert np.array_equal(Y.download(np.uint32), Y2.download(np.uint32))
    m.free()


C1 = [(4096, 4096), (11008, 4096), (4096, 11008), (32000, 4096), (12288, 4096), (22016, 4096)]
C2 = [(17408, 5120), (5120, 17408), (6144, 5120), (5120, 6144), (34816, 5120), (152064, 5120)]


@pytest.mark.parametrize("rows,cols", C1, ids=[f"{r}x{c}" for r, c in C1])
def test_c0_c1_decode(dev, orc, rows, cols):
    """c0 (4096 x 4096) and the c1 Llama-7B Q4_0 shapes, with the merged wqkv and wgu."""
    decode_case(dev, orc, Q40, rows, cols, seed=rows + cols)


@pytest.mark.parametrize("rows,cols", C2, ids=[f"{r}x{c}" for r, c in C2])
def test_c2_decode(dev, orc, rows, cols):
    """The c2 27B-class Q4_K shapes, with the merged ffn gate/up and the 152064-row lm_head."""
    decode_case(dev, orc, Q4K, rows, cols, seed=rows + cols + 1)


C3 = [(Q4K, 17408, 5120), (Q4K, 5120, 17408), (Q40, 11008, 4096),
      # the unsplit one-round T = 8 launches: 6 row groups per workgroup (250 workgroups), 4 (256),
      # 5 with a ragged last workgroup and a partial tile of K (nb = 65)
      (Q40, 24000, 4096), (Q4K, 16384, 5120), (Q40, 19990, 2080)]


@pytest.mark.parametrize("kind,rows,cols", C3, ids=[f"k{k}-{r}x{c}" for k, r, c in C3])
def test_c3_verify(dev, orc, kind, rows, cols):
    """c3: T = 8 and T = 16 vectors through op_gemv (the verify kernels, the host's K split) against the
    oracle, and each token bit-equal to its own decode GEMV."""
    m = Mat(dev, orc, kind, rows, cols, seed=rows + 3)
    nb, xs = m.nb, q8_stride(m.nb)
    x = synth.activations(16, cols, seed=cols + 5)
    xq = orc.quant_q8(x)
    mag = m.mag(xq)
    want = np.stack([m.oracle(xq[t]) for t in range(16)])
    X, Q = dev.DevBuf.of(x), dev.DevBuf(16 * xs)
    Y, Y1 = dev.DevBuf(16 * rows * 4), dev.DevBuf(rows * 4)
    dev.quant_q8(X, Q, nb, 16, 128 * nb, xs)
    dec = []
    for t in range(16):
        dev.gemv(kind, m.W, Q.ptr + t * xs, Y1, rows, nb)
        dec.append(Y1.download(np.uint32))
    dec = np.stack(dec)
    check(dec.view(np.float32), want, mag, "decode")
    for T in (8, 16):
        print(f"verify kind {kind} {rows}x{cols} T={T}", flush=True)
        Y.fill(0xFF)
        dev.op_gemv(kind, m.W, Q, Y, rows, nb, T, xs, rows)
        y = Y.download(np.float32).reshape(16, rows)[:T]
        check(y, want[:T], mag[:T], f"T={T}")
        same = y.view(np.uint32) == dec[:T]
        assert same.all(), f"T={T}: {int((~same).sum())} outputs differ from the decode GEMV"
    m.free()


C4 = [(17408, 5120), (5120, 17408)]


@pytest.mark.parametrize("rows,cols", C4, ids=[f"{r}x{c}" for r, c in C4])
def test_c4_gemm(dev, orc, rows, cols):
    """c4: the T = 256 prefill chunk through op_gemv (the GEMM, the host's tile and K split), every token and
    row against the oracle."""
    T = 256
    m = Mat(dev, orc, Q4K, rows, cols, seed=rows + 4)
    nb, xs = m.nb, q8_stride(m.nb)
    x = synth.activations(T, cols, seed=cols + 6)
    xq = orc.quant_q8(x)
    X, Q, Y = dev.DevBuf.of(x), dev.DevBuf(T * xs), dev.DevBuf(T * rows * 4)
    dev.quant_q8(X, Q, nb, T, 128 * nb, xs)
    print(f"gemm {rows}x{cols} T={T}", flush=True)
    dev.op_gemv(Q4K, m.W, Q, Y, rows, nb, T, xs, rows)
    y = Y.download(np.float32).reshape(T, rows)
    mag = m.mag(xq)
    for t in range(T):
        check(y[t], m.oracle(xq[t]), mag[t], f"token {t}")
    m.free()
