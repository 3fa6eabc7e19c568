"""Integer exactness of every GEMV / GEMM path, observed bit for bit.

On the cases of ``exactcase`` every float step is exact, so the one correct
result is the exact sum: each path -- the decode forms at every lane count,
the fused-quantization decode, the int8-MFMA verify kernels at every K split
and T = 1..16, the prefill GEMMs (f16-MFMA and int8-MFMA, with and without
split K) -- must return it bit for bit. A block sum off by one (a wrong
nibble, a wrong half of an MFMA operand, a wrong scale index) moves y by at
least 1/2. The CPU test pins the cases: the oracle (the reference's cpu.c
order) gives the exact sum too.
"""
import numpy as np
import pytest

import exactcase
from amdc import synth

KINDS = {0: "q4_0", 2: "q8_0", 3: "q4_k", 4: "q6_k"}
# (kind, rows, nb): Q4_0 rows of 344 blocks (c1 down) and 128; Q4_K rows of 544 (c2 ffn_down) and 160
SHAPES = [(0, 150, 344), (0, 200, 128), (3, 130, 544), (3, 200, 160), (2, 100, 344), (4, 70, 544)]


def q8_stride(nb):
    return (40 * nb + 255) // 256 * 256


class Exact:
    def __init__(self, orc, kind, rows, nb, T, seed, dev=None):
        self.kind, self.rows, self.nb, self.T = kind, rows, nb, T
        self.src = exactcase.gguf(kind, rows, 32 * nb, seed)
        self.x = exactcase.activations(T, 32 * nb, seed + 1)
        self.xq = orc.quant_q8(self.x)
        assert np.all(self.xq[:, 32 * nb:36 * nb].view(np.float32) == 1.0)  # d_a = 1 in every block
        self.want = np.stack([exactcase.exact_y(orc, kind, self.src, rows, nb, self.xq[t]) for t in range(T)])
        self.xs = q8_stride(nb)
        if dev is not None:
            self.W = dev.DevBuf.of(dev.repack(kind, self.src, rows, 32 * nb))
            self.X = dev.DevBuf.of(self.x)
            self.Q = dev.DevBuf(T * self.xs)
            self.Q.fill(0)
            dev.quant_q8(self.X, self.Q, nb, T, 128 * nb, self.xs)
            q = self.Q.download(np.uint8).reshape(T, self.xs)[:, :40 * nb]
            assert np.array_equal(q, self.xq)
            self.Y = dev.DevBuf(T * rows * 4)

    def y(self):
        return self.Y.download(np.float32).reshape(self.T, self.rows)


def mismatch(y, want):
    bad = np.nonzero(y.view(np.uint32) != want.view(np.uint32))
    if len(bad[0]) == 0:
        return None
    i = tuple(b[0] for b in bad)
    return f"{len(bad[0])} differ, first at {i}: {y[i]!r} != {want[i]!r}"


@pytest.mark.parametrize("kind,rows,nb", SHAPES)
def test_oracle_exact(orc, kind, rows, nb):
    """cpu.c's order on the exact cases gives the exact sum (pins the cases)."""
    e = Exact(orc, kind, rows, nb, 2, seed=kind * 100 + nb)
    qw, qs = orc.repack(synth.GGML[kind], e.src, rows, nb)
    for t in range(2):
        y = orc.gemv(synth.GGML[kind], qw, qs, rows, nb, e.xq[t])
        assert mismatch(y, e.want[t]) is None


@pytest.mark.gpu
@pytest.mark.parametrize("kind,rows,nb", SHAPES)
def test_exact_decode(dev, orc, kind, rows, nb):
    """Every decode form and lane count (and the fused-quantization form) returns the exact sum."""
    e = Exact(orc, kind, rows, nb, 1, seed=kind * 10 + nb, dev=dev)
    try:
        tried = []
        for form in (0, 1, 2, 3):
            for lanes in (0, 4, 8, 16, 32, 64):
                if kind in (2, 4) and form == 1:
                    continue  # Q8_0 / Q6_K have the second form only
                dev.set_tuning(lanes=lanes, form=form)
                e.Y.fill(0xFF)
                dev.gemv(kind, e.W, e.Q, e.Y, rows, nb)
                m = mismatch(e.y()[0], e.want[0])
                assert m is None, (form, lanes, m)
                tried.append((form, lanes))
        dev.set_tuning()
        e.Y.fill(0xFF)
        dev.gemv_x(kind, e.W, e.X, e.Y, rows, nb)
        assert mismatch(e.y()[0], e.want[0]) is None, "gemv_x"
    finally:
        dev.set_tuning()


@pytest.mark.gpu
@pytest.mark.parametrize("kind,rows,nb", SHAPES)
def test_exact_verify(dev, orc, kind, rows, nb):
    """The int8-MFMA verify kernels at T = 1..16 and every K split return the exact sums."""
    e = Exact(orc, kind, rows, nb, 16, seed=kind * 20 + nb, dev=dev)
    nt = (nb + 63) // 64
    try:
        for ks in sorted({0, 1, 2, 3, nt}):
            dev.set_tuning(gemm_ksplit=ks)
            for T in range(1, 17):
                e.Y.fill(0xFF)
                dev.gemv_t(kind, e.W, e.Q, e.Y, rows, nb, T, e.xs, rows)
                m = mismatch(e.y()[:T], e.want[:T])
                assert m is None, (ks, T, m)
    finally:
        dev.set_tuning()


@pytest.mark.gpu
@pytest.mark.parametrize("kind,rows,nb", SHAPES)
def test_exact_gemm(dev, orc, kind, rows, nb):
    """The prefill GEMMs (f16-MFMA 64 / 128-token tiles, 128-row tiles for Q4_K, the int8-MFMA Q4_K kernels) with and without split K
    return the exact sums."""
    T = 80
    e = Exact(orc, kind, rows, nb, T, seed=kind * 30 + nb, dev=dev)
    kerns = [(0, 0), (3, 0), (4, 0), (3, 2), (4, 4), (3, 8)] + ([(1, 0), (2, 0), (5, 0), (5, 3)] if kind == 3 else [])
    try:
        for kern, ks in kerns:
            dev.set_tuning(gemm_kernel=kern, gemm_ksplit=ks)
            e.Y.fill(0xFF)
            dev.gemm(kind, e.W, e.Q, e.Y, rows, nb, T, e.xs, rows)
            m = mismatch(e.y(), e.want)
            assert m is None, (kern, ks, m)
    finally:
        dev.set_tuning()
