"""Parity of the HIP path (libamdc_q4.so + amdc_kernels.hsaco, through the C
ABI) with the oracle, on an MI355X.

The bar: Q8 buffers, repacked nibbles and the
per-block int32 dot products bit-exact; f32 outputs within 1e-5 relative
error, measured as |y_gpu - y_oracle| / sum |terms| per row (the reference's
tests/kernel_test.c:59-80 metric: summation order differs, the terms do not).
"""
import os

import numpy as np
import pytest

from amdc import synth

pytestmark = pytest.mark.gpu
TOL = 1e-5
CPUS = min(16, os.cpu_count() or 1)


def ttype(kind):
    return synth.GGML[kind]


def q8_stride(nb):
    return (40 * nb + 255) // 256 * 256  # token rows of the Q8 buffer 256-aligned (src/model.c:1194)


@pytest.fixture(autouse=True)
def _tuning_reset(dev):
    dev.set_tuning()
    yield
    dev.set_tuning()


class Case:
    """Seeded weights and T activation vectors, on the host and the device."""

    def __init__(self, dev, orc, kind, rows, nb, T=1, seed=1, xscale=1.0, upload=True):
        self.dev, self.orc, self.kind, self.rows, self.nb, self.T = dev, orc, kind, rows, nb, T
        cols = 32 * nb
        self.src = synth.gguf(kind, rows, cols, seed)
        self.x = synth.activations(T, cols, seed + 1) * np.float32(xscale)
        self.qw, self.qs = orc.repack(ttype(kind), self.src, rows, nb)
        self.xq = orc.quant_q8(self.x)  # [T, 40 nb]
        self.xs = q8_stride(nb)
        if upload:
            self.W = dev.DevBuf.of(dev.repack(kind, self.src, rows, cols))
            self.X = dev.DevBuf.of(self.x)
            self.Q = dev.DevBuf(T * self.xs)
            self.Q.fill(0)
            self.Y = dev.DevBuf(T * rows * 4)

    def quant(self):
        self.dev.quant_q8(self.X, self.Q, self.nb, self.T, 128 * self.nb, self.xs)
        q = self.Q.download(np.uint8).reshape(self.T, self.xs)[:, :40 * self.nb]
        return q

    def y_oracle(self, t):
        return self.orc.gemv(ttype(self.kind), self.qw, self.qs, self.rows, self.nb, self.xq[t], threads=CPUS)

    def mag(self, t):
        return self.orc.gemv_f64(ttype(self.kind), self.src, self.rows, self.nb, self.xq[t])[1]

    def y_gpu(self):
        return self.Y.download(np.float32).reshape(self.T, self.rows)


def rel_err(y, yref, mag):
    return float((np.abs(y.astype(np.float64) - yref.astype(np.float64)) / np.maximum(mag, 1e-30)).max())


# ---------------------------------------------------------------- Q8

@pytest.mark.parametrize("nb,T", [(1, 1), (3, 2), (33, 1), (128, 5), (544, 3)])
def test_quant_q8_bitexact(dev, orc, nb, T):
    c = Case(dev, orc, 0, 1, nb, T, seed=nb + T, xscale=2.0)
    x = c.x.copy()
    if nb >= 4:  # special blocks: zeros, a single nonzero, .5 ties, tiny values
        x[0, 0:32] = 0
        x[0, 32:64] = 0
        x[0, 40] = -3.25
        x[0, 64:96] = np.arange(-16, 16, dtype=np.float32) * np.float32(127.0 / 32.0)
        x[0, 96:128] *= np.float32(1e-30)
        c.X.upload(x)
        c.xq = orc.quant_q8(x)
    q = c.quant()
    assert np.array_equal(q, c.xq.reshape(T, -1))


# ---------------------------------------------------------------- integer dots

@pytest.mark.parametrize("kind,rows,nb", [(0, 1, 1), (0, 7, 3), (0, 9, 11), (0, 13, 33), (0, 3, 100), (0, 2, 511), (0, 5, 128),
                                          (3, 1, 8), (3, 7, 16), (3, 9, 40), (3, 5, 72), (3, 3, 544)])
def test_block_dots_bitexact(dev, orc, kind, rows, nb):
    c = Case(dev, orc, kind, rows, nb, seed=rows * 31 + nb, xscale=3.0)
    c.quant()
    out = dev.DevBuf(rows * nb * 4)
    dev.block_dots(kind, c.W, c.Q, out, rows, nb)
    got = out.download(np.int32).reshape(rows, nb)
    assert np.array_equal(got, orc.block_dots(ttype(kind), c.qw, rows, nb, c.xq[0]))
    assert np.array_equal(got, orc.block_dots_gguf(ttype(kind), c.src, rows, nb, c.xq[0]))


# ---------------------------------------------------------------- decode GEMV (T = 1)

SHAPES_Q4_0 = [(1, 1), (7, 3), (9, 11), (8, 32), (13, 33), (17, 36), (5, 64), (3, 100), (2, 511), (64, 128), (33, 344)]
SHAPES_Q4_K = [(1, 8), (7, 16), (9, 40), (3, 64), (5, 72), (37, 160), (19, 544), (8, 192)]


@pytest.mark.parametrize("kind,rows,nb", [(0, r, n) for r, n in SHAPES_Q4_0] + [(3, r, n) for r, n in SHAPES_Q4_K])
def test_gemv_t1(dev, orc, kind, rows, nb):
    c = Case(dev, orc, kind, rows, nb, seed=rows + 100 * nb)
    assert np.array_equal(c.quant()[0], c.xq[0])
    dev.gemv(kind, c.W, c.Q, c.Y, rows, nb)
    err = rel_err(c.y_gpu()[0], c.y_oracle(0), c.mag(0))
    assert err < TOL, err


@pytest.mark.parametrize("lanes", [4, 8, 16, 32, 64])
@pytest.mark.parametrize("unroll,form", [(0, 0), (0, 1), (0, 2)])
@pytest.mark.parametrize("wgs", [0, 3])  # 3 workgroups: each loops over several row groups
@pytest.mark.parametrize("kind,rows,nb", [(0, 70, 344), (0, 33, 300), (3, 45, 160), (3, 6, 544)])
def test_gemv_t1_tunings(dev, orc, kind, rows, nb, lanes, unroll, form, wgs):
    c = Case(dev, orc, kind, rows, nb, seed=lanes + unroll + form)
    c.quant()
    dev.set_tuning(lanes, unroll, wgs, form=form)
    dev.gemv(kind, c.W, c.Q, c.Y, rows, nb)
    err = rel_err(c.y_gpu()[0], c.y_oracle(0), c.mag(0))
    assert err < TOL, err


@pytest.mark.parametrize("kind", [0, 3])
@pytest.mark.parametrize("form", [1, 2])
def test_gemv_epilogue_bias_res(dev, orc, kind, form):
    rows, nb = 50, 64
    c = Case(dev, orc, kind, rows, nb, seed=77)
    c.quant()
    dev.set_tuning(form=form)
    g = np.random.default_rng(5)
    bias, res = g.standard_normal(rows).astype(np.float32), g.standard_normal(rows).astype(np.float32)
    B, R = dev.DevBuf.of(bias), dev.DevBuf.of(res)
    dev.gemv(kind, c.W, c.Q, c.Y, rows, nb, bias=B, res=R)
    want = orc.epilogue(c.y_oracle(0), bias, res)
    err = rel_err(c.y_gpu()[0], want, c.mag(0) + np.abs(bias) + np.abs(res))
    assert err < TOL, err
    dev.gemv(kind, c.W, c.Q, c.Y, rows, nb, res=R)
    err = rel_err(c.y_gpu()[0], orc.epilogue(c.y_oracle(0), None, res), c.mag(0) + np.abs(res))
    assert err < TOL, err
    dev.gemv(kind, c.W, c.Q, c.Y, rows, nb, bias=B)
    err = rel_err(c.y_gpu()[0], orc.epilogue(c.y_oracle(0), bias, None), c.mag(0) + np.abs(bias))
    assert err < TOL, err


# ---------------------------------------------------------------- multi-vector GEMV (verify)

@pytest.mark.parametrize("path", [0, 1])  # 0: the int8-MFMA verify kernels (16 vectors per launch); 1: a decode launch per vector
@pytest.mark.parametrize("T", [2, 5, 8, 9, 16, 19])
@pytest.mark.parametrize("kind,rows,nb", [(0, 40, 128), (0, 130, 43), (3, 33, 160), (3, 21, 544), (3, 200, 72)])
def test_gemv_multi(dev, orc, kind, rows, nb, T, path):
    dev.set_tuning(unroll=path)
    c = Case(dev, orc, kind, rows, nb, T, seed=T * 13 + nb)
    assert np.array_equal(c.quant(), c.xq)
    res = np.random.default_rng(T).standard_normal((T, rows)).astype(np.float32)
    R = dev.DevBuf.of(res)
    dev.gemv_t(kind, c.W, c.Q, c.Y, rows, nb, T, c.xs, rows, rows, res=R)
    y = c.y_gpu()
    # and the single-vector kernel per token: within the bound of the oracle, and the same bits
    Y1 = dev.DevBuf(rows * 4)
    for t in range(T):
        want = orc.epilogue(c.y_oracle(t), None, res[t])
        mag = c.mag(t) + np.abs(res[t])
        assert rel_err(y[t], want, mag) < TOL, t
        dev.gemv(kind, c.W, c.Q.ptr + t * c.xs, Y1, rows, nb, res=R.ptr + 4 * t * rows)
        assert np.array_equal(Y1.download(np.uint32), y[t].view(np.uint32)), t


# ---------------------------------------------------------------- prefill GEMM

@pytest.mark.parametrize("kern,ks", [(0, 0), (1, 0), (2, 0), (3, 1), (4, 2), (3, 4), (4, 3), (5, 1), (5, 3)])
@pytest.mark.parametrize("rows,nb,T", [(1, 8, 17), (63, 16, 64), (64, 160, 65), (130, 40, 130), (300, 24, 256), (70, 544, 33)])
def test_gemm_q4k(dev, orc, rows, nb, T, kern, ks):
    c = Case(dev, orc, 3, rows, nb, T, seed=rows + T)
    assert np.array_equal(c.quant(), c.xq)
    g = np.random.default_rng(T)
    bias = g.standard_normal(rows).astype(np.float32)
    B = dev.DevBuf.of(bias)
    if ks and nb // 8 < ks:
        pytest.skip("fewer super-blocks than splits")
    dev.set_tuning(gemm_kernel=kern, gemm_ksplit=ks)
    dev.gemm_q4k(c.W, c.Q, c.Y, rows, nb, T, c.xs, rows, bias=B)
    y = c.y_gpu()
    for t in range(T):
        want = orc.epilogue(c.y_oracle(t), bias, None)
        assert rel_err(y[t], want, c.mag(t) + np.abs(bias)) < TOL, t


def test_op_gemv_dispatch(dev, orc):
    rows, nb = 48, 64
    for kind, T in ((0, 1), (3, 1), (0, 8), (3, 8), (0, 19), (3, 19), (0, 20), (3, 20), (0, 40), (3, 40)):
        c = Case(dev, orc, kind, rows, nb, T, seed=T + kind)
        c.quant()
        dev.op_gemv(kind, c.W, c.Q, c.Y, rows, nb, T, c.xs, rows)
        y = c.y_gpu()
        for t in range(T):
            assert rel_err(y[t], c.y_oracle(t), c.mag(t)) < TOL, (kind, T, t)


def test_errors_do_not_launch(dev, orc):
    c = Case(dev, orc, 3, 8, 16, seed=3)
    with pytest.raises(dev.AmdcError):
        dev.gemv_q4k(c.W, c.Q, c.Y, 8, 12)  # Q4_K nb % 8 != 0
    with pytest.raises(dev.AmdcError):
        dev.gemv_q4(c.W.ptr + 4, c.Q, c.Y, 8, 16)  # misaligned weights
    with pytest.raises(dev.AmdcError):
        dev.gemv_q4k_t(c.W, c.Q, c.Y, 8, 16, 2, 100, 8)  # xs not a multiple of 16


def test_graph_replay_matches_eager(dev, orc):
    """A captured op sequence (quant, decode GEMV, multi-vector GEMV, GEMM) replayed several times, with eager
    work and synchronizations between the replays: every replay equals the eager run bit for bit."""
    rows, nb, T = 100, 160, 20
    c = Case(dev, orc, 3, rows, nb, T, seed=4)
    Y1, YT, YG = dev.DevBuf(4 * rows), dev.DevBuf(4 * rows * T), dev.DevBuf(4 * rows * T)
    S = dev.Stream()

    def ops(s):
        dev.quant_q8(c.X, c.Q, nb, T, 128 * nb, c.xs, stream=s)
        dev.gemv_q4k(c.W, c.Q, Y1, rows, nb, stream=s)
        dev.gemv_q4k_t(c.W, c.Q, YT, rows, nb, 8, c.xs, rows, stream=s)
        dev.gemm_q4k(c.W, c.Q, YG, rows, nb, T, c.xs, rows, stream=s)

    for b in (c.Q, Y1, YT, YG):
        b.fill(0)  # YT is written for 8 of its 20 token rows: the rest must not hold stale memory
    dev.sync()
    ops(S.s)
    S.sync()
    want = [b.download(np.uint32) for b in (c.Q, Y1, YT, YG)]
    g = dev.Graph(S, ops)
    other = Case(dev, orc, 0, 64, 128, seed=9)
    for rep in range(3):
        for b in (c.Q, Y1, YT, YG):
            b.fill(0)
        other.quant()
        dev.gemv_q4(other.W, other.Q, other.Y, 64, 128)  # eager work between replays
        dev.sync()
        g.launch()
        S.sync()
        for b, w in zip((c.Q, Y1, YT, YG), want):
            assert np.array_equal(b.download(np.uint32), w), rep
    assert rel_err(Y1.download(np.float32), c.y_oracle(0), c.mag(0)) < TOL


@pytest.mark.parametrize("kern,ks", [(0, 0), (1, 0), (3, 2), (4, 4), (5, 2)])
def test_gemm_deterministic(dev, orc, kern, ks):
    """Repeated GEMMs give the same bits: the kernels have a fixed summation order, so any
    difference between runs would be a race between waves."""
    rows, nb, T = 300, 544, 96
    c = Case(dev, orc, 3, rows, nb, T, seed=11)
    c.quant()
    dev.set_tuning(gemm_kernel=kern, gemm_ksplit=ks)
    first = None
    for _ in range(6):
        c.Y.fill(0)
        dev.gemm_q4k(c.W, c.Q, c.Y, rows, nb, T, c.xs, rows)
        got = c.Y.download(np.uint32)
        if first is None:
            first = got
        assert np.array_equal(got, first)
    y = first.view(np.float32).reshape(T, rows)
    for t in (0, T - 1):
        assert rel_err(y[t], c.y_oracle(t), c.mag(t)) < TOL


@pytest.mark.parametrize("kind,rows,nb", [(0, 70, 13), (0, 300, 128), (0, 64, 344), (3, 45, 160), (3, 20, 544)])
def test_gemv_fused_quant(dev, orc, kind, rows, nb):
    """The decode GEMV that quantizes its f32 input itself: its Q8 output equals cpu_quant_q8 bit for
    bit, and y equals the separate quantize + GEMV launches bit for bit."""
    c = Case(dev, orc, kind, rows, nb, seed=rows + nb, xscale=2.0)
    g = np.random.default_rng(nb)
    bias, res = g.standard_normal(rows).astype(np.float32), g.standard_normal(rows).astype(np.float32)
    B, R = dev.DevBuf.of(bias), dev.DevBuf.of(res)
    Q2, Y2 = dev.DevBuf(c.xs), dev.DevBuf(rows * 4)
    Q2.fill(0)
    dev.gemv_x(kind, c.W, c.X, Y2, rows, nb, bias=B, res=R, q8=Q2)
    assert np.array_equal(Q2.download(np.uint8)[:40 * nb], c.xq[0])
    c.quant()
    dev.gemv(kind, c.W, c.Q, c.Y, rows, nb, bias=B, res=R)
    assert np.array_equal(Y2.download(np.uint32), c.Y.download(np.uint32))
    want = orc.epilogue(c.y_oracle(0), bias, res)
    assert rel_err(Y2.download(np.float32), want, c.mag(0) + np.abs(bias) + np.abs(res)) < TOL
    dev.gemv_x(kind, c.W, c.X, Y2, rows, nb)  # without the Q8 output
    assert rel_err(Y2.download(np.float32), c.y_oracle(0), c.mag(0)) < TOL


@pytest.mark.gpu
@pytest.mark.parametrize("kind,nb", [(0, 120), (3, 120), (0, 136), (3, 136)])
def test_gemv_fused_quant_special_blocks(dev, orc, kind, nb):
    """The fused quantization on blocks that stress rounding: an all-zero block (d = 0), a block of
    exact .5 ties of x / d, a single non-zero value, and denormal-sized values; its Q8 output equals
    cpu_quant_q8 bit for bit."""
    rows = 96
    c = Case(dev, orc, kind, rows, nb, seed=7)
    x = c.x.copy()
    x[0, 0:32] = 0.0
    x[0, 32:64] = np.arange(32, dtype=np.float32) - 15.5  # d = 1 below: every x / d a tie
    x[0, 63] = 127.0
    x[0, 64:96] = 0.0
    x[0, 70] = -3.0
    x[0, 96:128] = np.float32(1e-42) * np.arange(1, 33, dtype=np.float32)
    x[0, 32 * (nb - 1):] *= 1e6
    want_q = orc.quant_q8(x)[0]
    X, Q2, Y2 = dev.DevBuf.of(x), dev.DevBuf(c.xs), dev.DevBuf(rows * 4)
    Q2.fill(0)
    dev.gemv_x(kind, c.W, X, Y2, rows, nb, q8=Q2)
    assert np.array_equal(Q2.download(np.uint8)[:40 * nb], want_q)
    Q1, Y1 = dev.DevBuf(c.xs), dev.DevBuf(rows * 4)
    dev.quant_q8(X, Q1, nb)
    assert np.array_equal(Q1.download(np.uint8)[:40 * nb], want_q)
    dev.gemv(kind, c.W, Q1, Y1, rows, nb)
    assert np.array_equal(Y2.download(np.uint32), Y1.download(np.uint32))


@pytest.mark.gpu
@pytest.mark.parametrize("kind", [0, 3])
@pytest.mark.parametrize("T", [8, 11, 16])
def test_verify_splitk(dev, orc, kind, T):
    """The verify kernels (T <= 8, and the 16-vector form for T = 9..16) with K split over workgroups
    (aligned tile ranges, their sums added in a tree by the reduce kernel): calls in a row with different
    splits, bias and residual all match the oracle, and every split gives the same bits."""
    rows, nb = 200, 544
    c = Case(dev, orc, kind, rows, nb, T, seed=21)
    c.quant()
    g = np.random.default_rng(3)
    bias = g.standard_normal(rows).astype(np.float32)
    res = g.standard_normal((T, rows)).astype(np.float32)
    B, R = dev.DevBuf.of(bias), dev.DevBuf.of(res)
    bits = {}
    for ks in (1, 9, 4, 9, 2, 4):
        dev.set_tuning(gemm_ksplit=ks)
        c.Y.fill(0)
        dev.gemv_t(kind, c.W, c.Q, c.Y, rows, nb, T, c.xs, rows, rs=rows, bias=B, res=R)
        y = c.y_gpu()
        for t in range(T):
            want = orc.epilogue(c.y_oracle(t), bias, res[t])
            assert rel_err(y[t], want, c.mag(t) + np.abs(bias) + np.abs(res[t])) < TOL, (ks, t)
        u = y.view(np.uint32).copy()
        for k, b in bits.items():
            assert np.array_equal(u, b), (ks, k)
        bits[ks] = u


def test_graph_survives_workspace_growth(dev, orc):
    """A graph captured while the library's workspace is small keeps replaying correctly after a larger
    call has grown the workspace (the smaller allocation stays alive until amdc_close)."""
    small = Case(dev, orc, 3, 64, 40, 32, seed=31)
    small.quant()
    S = dev.Stream()
    dev.gemm_q4k(small.W, small.Q, small.Y, 64, 40, 32, small.xs, 64)  # sizes the workspace for this call
    dev.sync()
    want = small.Y.download(np.uint32)
    g = dev.Graph(S, lambda s: dev.gemm_q4k(small.W, small.Q, small.Y, 64, 40, 32, small.xs, 64, stream=s))
    big = Case(dev, orc, 3, 300, 544, 256, seed=32)
    big.quant()
    dev.gemm_q4k(big.W, big.Q, big.Y, 300, 544, 256, big.xs, 300)  # grows the workspace
    dev.sync()
    for _ in range(3):
        small.Y.fill(0)
        g.launch()
        S.sync()
        assert np.array_equal(small.Y.download(np.uint32), want)
    y = big.y_gpu()
    assert rel_err(y[255], big.y_oracle(255), big.mag(255)) < TOL


@pytest.mark.gpu
@pytest.mark.parametrize("kind,T", [(0, 24), (3, 32), (3, 33)])
def test_op_gemv_dispatch_large(dev, orc, kind, T):
    """op_gemv on a matrix of more than 2^24 weights: T = 24 and 32 run the verify kernels (16 + 8,
    16 + 16 vectors), T = 33 the GEMM; every token matches the oracle."""
    rows, nb = 1040, 520
    c = Case(dev, orc, kind, rows, nb, T, seed=T + 7 * kind)
    c.quant()
    dev.op_gemv(kind, c.W, c.Q, c.Y, rows, nb, T, c.xs, rows)
    y = c.y_gpu()
    for t in range(T):
        assert rel_err(y[t], c.y_oracle(t), c.mag(t)) < TOL, (kind, T, t)
