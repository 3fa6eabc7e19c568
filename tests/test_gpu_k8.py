"""Parity of the Q8_0 and Q6_K decode GEMV (amdc_gemv_q8 / amdc_gemv_q6k and
their multi-vector and f32-input forms, through the C ABI) with the oracle's
restatement of cpu_gemv_q8 / cpu_gemv_q6k (hanw/amd.c src/cpu.c:120-175), on
an MI355X. The same bar as the Q4 kinds: the per-block int32 dots (Q6_K: the
two half dots of ie_q6k_dots) bit-exact against the oracle and an int64 brute
force over the GGUF bytes; f32 outputs within 1e-5 of sum |terms| per row.
"""
import numpy as np
import pytest

from amdc import synth
from test_gpu_parity import TOL, Case, rel_err, ttype

pytestmark = pytest.mark.gpu
Q8, Q6 = synth.KIND_Q8_0, synth.KIND_Q6_K


@pytest.fixture(autouse=True)
def _tuning_reset(dev):
    dev.set_tuning()
    yield
    dev.set_tuning()


@pytest.mark.parametrize("kind,rows,nb", [(Q8, 1, 1), (Q8, 7, 3), (Q8, 9, 11), (Q8, 13, 33), (Q8, 2, 511), (Q8, 5, 128),
                                          (Q6, 1, 8), (Q6, 7, 16), (Q6, 9, 40), (Q6, 5, 72), (Q6, 3, 544)])
def test_block_dots_bitexact(dev, orc, kind, rows, nb):
    c = Case(dev, orc, kind, rows, nb, seed=rows * 31 + nb, xscale=3.0)
    c.quant()
    h = 2 if kind == Q6 else 1
    out = dev.DevBuf(rows * nb * 4 * h)
    dev.block_dots(kind, c.W, c.Q, out, rows, nb)
    got = out.download(np.int32).reshape((rows, nb, 2) if h == 2 else (rows, nb))
    assert np.array_equal(got, orc.block_dots(ttype(kind), c.qw, rows, nb, c.xq[0]))
    assert np.array_equal(got, orc.block_dots_gguf(ttype(kind), c.src, rows, nb, c.xq[0]))


SHAPES_Q8 = [(1, 1), (7, 3), (9, 11), (8, 32), (13, 33), (17, 36), (3, 100), (2, 511), (64, 128), (33, 344), (5, 2048)]
SHAPES_Q6 = [(1, 8), (7, 16), (9, 40), (3, 64), (37, 160), (19, 544), (8, 192), (3, 1792)]


@pytest.mark.parametrize("kind,rows,nb", [(Q8, r, n) for r, n in SHAPES_Q8] + [(Q6, r, n) for r, n in SHAPES_Q6])
def test_gemv_t1(dev, orc, kind, rows, nb):
    c = Case(dev, orc, kind, rows, nb, seed=rows + 100 * nb)
    assert np.array_equal(c.quant()[0], c.xq[0])
    dev.gemv(kind, c.W, c.Q, c.Y, rows, nb)
    assert rel_err(c.y_gpu()[0], c.y_oracle(0), c.mag(0)) < TOL


@pytest.mark.parametrize("lanes", [4, 8, 16, 32, 64])
@pytest.mark.parametrize("wgs", [0, 3])
@pytest.mark.parametrize("kind,rows,nb", [(Q8, 70, 344), (Q8, 33, 300), (Q6, 45, 160), (Q6, 6, 544)])
def test_gemv_t1_tunings(dev, orc, kind, rows, nb, lanes, wgs):
    c = Case(dev, orc, kind, rows, nb, seed=lanes + wgs)
    c.quant()
    dev.set_tuning(lanes, 0, wgs)
    dev.gemv(kind, c.W, c.Q, c.Y, rows, nb)
    assert rel_err(c.y_gpu()[0], c.y_oracle(0), c.mag(0)) < TOL


@pytest.mark.parametrize("kind", [Q8, Q6])
def test_gemv_epilogue_bias_res(dev, orc, kind):
    rows, nb = 50, 64
    c = Case(dev, orc, kind, rows, nb, seed=77)
    c.quant()
    g = np.random.default_rng(5)
    bias, res = g.standard_normal(rows).astype(np.float32), g.standard_normal(rows).astype(np.float32)
    B, R = dev.DevBuf.of(bias), dev.DevBuf.of(res)
    for b, r in ((bias, res), (None, res), (bias, None)):
        dev.gemv(kind, c.W, c.Q, c.Y, rows, nb, bias=None if b is None else B, res=None if r is None else R)
        mag = c.mag(0) + (0 if b is None else np.abs(b)) + (0 if r is None else np.abs(r))
        assert rel_err(c.y_gpu()[0], orc.epilogue(c.y_oracle(0), b, r), mag) < TOL


@pytest.mark.parametrize("kind,rows,nb,T", [(Q8, 40, 128, 3), (Q8, 130, 43, 9), (Q6, 33, 160, 5), (Q6, 21, 544, 2)])
def test_gemv_multi_and_dispatch(dev, orc, kind, rows, nb, T):
    c = Case(dev, orc, kind, rows, nb, T, seed=T * 13 + nb)
    assert np.array_equal(c.quant(), c.xq)
    res = np.random.default_rng(T).standard_normal((T, rows)).astype(np.float32)
    R = dev.DevBuf.of(res)
    dev.gemv_t(kind, c.W, c.Q, c.Y, rows, nb, T, c.xs, rows, rows, res=R)
    y = c.y_gpu()
    for t in range(T):
        assert rel_err(y[t], orc.epilogue(c.y_oracle(t), None, res[t]), c.mag(t) + np.abs(res[t])) < TOL, t
    c.Y.fill(0)
    dev.op_gemv(kind, c.W, c.Q, c.Y, rows, nb, T, c.xs, rows)
    y = c.y_gpu()
    for t in range(T):
        assert rel_err(y[t], c.y_oracle(t), c.mag(t)) < TOL, t


@pytest.mark.parametrize("kind,rows,nb", [(Q8, 70, 13), (Q8, 64, 344), (Q6, 45, 160)])
def test_gemv_x_equals_quant_then_gemv(dev, orc, kind, rows, nb):
    c = Case(dev, orc, kind, rows, nb, seed=rows + nb, xscale=2.0)
    Q2, Y2 = dev.DevBuf(c.xs), dev.DevBuf(rows * 4)
    dev.gemv_x(kind, c.W, c.X, Y2, rows, nb, q8=Q2)
    assert np.array_equal(Q2.download(np.uint8)[:40 * nb], c.xq[0])
    c.quant()
    dev.gemv(kind, c.W, c.Q, c.Y, rows, nb)
    assert np.array_equal(Y2.download(np.uint32), c.Y.download(np.uint32))
    dev.gemv_x(kind, c.W, c.X, Y2, rows, nb)  # the library's workspace for the Q8 vector
    assert np.array_equal(Y2.download(np.uint32), c.Y.download(np.uint32))


@pytest.mark.parametrize("kind,rows,cols", [(Q8, 4096, 4096), (Q6, 5120, 17408), (Q6, 152064, 5120)])
def test_gemv_full_size(dev, orc, kind, rows, cols):
    """The shapes of real decode matrices (a Q8_0 attention projection, Q6_K ffn_down and lm_head of
    the Q4_K_M configuration): every row within the bound, and a second run gives the same bits."""
    nb = cols // 32
    c = Case(dev, orc, kind, rows, nb, seed=3)
    c.quant()
    dev.gemv(kind, c.W, c.Q, c.Y, rows, nb)
    first = c.Y.download(np.uint32)
    assert rel_err(first.view(np.float32), c.y_oracle(0), c.mag(0)) < TOL
    c.Y.fill(0)
    dev.gemv(kind, c.W, c.Q, c.Y, rows, nb)
    assert np.array_equal(c.Y.download(np.uint32), first)


def test_errors_do_not_launch(dev, orc):
    c = Case(dev, orc, Q6, 8, 16, seed=3)
    with pytest.raises(dev.AmdcError):
        dev.gemv_q6k(c.W, c.Q, c.Y, 8, 12)  # Q6_K nb % 8 != 0
    with pytest.raises(dev.AmdcError):
        dev.gemv_q8(c.W.ptr + 4, c.Q, c.Y, 8, 16)  # misaligned weights
    with pytest.raises(dev.AmdcError):
        dev.Chain([dev.chain_gemv_x(Q6, c.W, c.X, c.Y, 8, 16)])  # f32-input chain GEMVs take the Q4 kinds only


@pytest.mark.parametrize("kind,rows,nb,T", [(Q8, 1, 1, 17), (Q8, 63, 13, 64), (Q8, 130, 128, 65), (Q8, 70, 344, 33), (Q8, 300, 40, 256),
                                            (Q6, 1, 8, 17), (Q6, 63, 16, 64), (Q6, 64, 160, 65), (Q6, 130, 40, 130), (Q6, 70, 544, 33),
                                            (0, 1, 1, 17), (0, 63, 13, 64), (0, 130, 128, 65), (0, 70, 344, 33), (0, 300, 40, 256)])
@pytest.mark.parametrize("ks", [0, 3])
def test_gemm(dev, orc, kind, rows, nb, T, ks):
    """The prefill GEMM (f16 MFMA, exact integer block sums) against the oracle per token row, with a
    bias, with and without split K; Q8_0, Q6_K and the Q4_0 form (no reference kernel: the reference
    runs one GEMV per token)."""
    c = Case(dev, orc, kind, rows, nb, T, seed=rows + T + kind)
    assert np.array_equal(c.quant(), c.xq)
    ng = (nb + 7) // 8
    if ks and ng < ks:
        pytest.skip("fewer super-groups than splits")
    bias = np.random.default_rng(T).standard_normal(rows).astype(np.float32)
    B = dev.DevBuf.of(bias)
    dev.set_tuning(gemm_ksplit=ks)
    dev.gemm(kind, c.W, c.Q, c.Y, rows, nb, T, c.xs, rows, bias=B)
    y = c.y_gpu()
    for t in range(T):
        assert rel_err(y[t], orc.epilogue(c.y_oracle(t), bias, None), c.mag(t) + np.abs(bias)) < TOL, t


@pytest.mark.parametrize("kind", [Q8, Q6])
def test_gemm_extreme_values(dev, orc, kind):
    """Weights and activations at the ends of their ranges, where the exactness of the f16 sums is
    tightest: Q6_K q = 0 (q - 32 = -32) with scales -128 / 127, Q8_0 weights -128 / 127; activations
    of one block all +-127 (x = +-1)."""
    rows, nb, T = 64, 16, 32
    c = Case(dev, orc, kind, rows, nb, T, seed=5, upload=False)
    src = c.src.copy()
    if kind == Q6:
        blk = src.reshape(-1, 210)
        blk[:, 0:192] = 0  # q = 0 everywhere
        blk[0::2, 192:208] = 0x80  # sc = -128
        blk[1::2, 192:208] = 0x7F  # sc = 127
    else:
        blk = src.reshape(-1, 34)
        blk[0::2, 2:] = 0x80
        blk[1::2, 2:] = 0x7F
    x = c.x.copy()
    x[:, 0:32] = 1.0
    x[1::2, 32:64] = -1.0
    c.src, c.x = src, x
    c.qw, c.qs = orc.repack(ttype(kind), src, rows, nb)
    c.xq = orc.quant_q8(x)
    c.W = dev.DevBuf.of(dev.repack(kind, src, rows, 32 * nb))
    c.X = dev.DevBuf.of(x)
    c.Q = dev.DevBuf(T * c.xs)
    c.Y = dev.DevBuf(T * rows * 4)
    assert np.array_equal(c.quant(), c.xq)
    dev.gemm(kind, c.W, c.Q, c.Y, rows, nb, T, c.xs, rows)
    y = c.y_gpu()
    for t in range(T):
        assert rel_err(y[t], c.y_oracle(t), c.mag(t)) < TOL, t


@pytest.mark.parametrize("kind,rows,nb", [(Q8, 200, 544), (Q8, 77, 13), (Q6, 200, 544), (Q6, 70, 24)])
@pytest.mark.parametrize("T", [1, 2, 7, 8, 12, 16])
def test_verify_splitk(dev, orc, kind, rows, nb, T):
    """The verify kernels (int8 MFMA, T <= 16 per launch, Q6_K T <= 8; Q6_K one half sub-block per
    K quarter, half dots in separate columns) with K split over workgroups: several splits in a row, with bias and residual, all
    within the bound and a repeated split gives the same bits; the per-vector decode kernel
    (tuning unroll=1) agrees within the bound."""
    c = Case(dev, orc, kind, rows, nb, T, seed=21 + T)
    c.quant()
    g = np.random.default_rng(3)
    bias = g.standard_normal(rows).astype(np.float32)
    res = g.standard_normal((T, rows)).astype(np.float32)
    B, R = dev.DevBuf.of(bias), dev.DevBuf.of(res)
    bits = {}
    for ks in (1, 9, 4, 9, 2, 1):
        dev.set_tuning(gemm_ksplit=ks)
        c.Y.fill(0)
        dev.gemv_t(kind, c.W, c.Q, c.Y, rows, nb, T, c.xs, rows, rs=rows, bias=B, res=R)
        y = c.y_gpu()
        for t in range(T):
            want = orc.epilogue(c.y_oracle(t), bias, res[t])
            assert rel_err(y[t], want, c.mag(t) + np.abs(bias) + np.abs(res[t])) < TOL, (ks, t)
        u = y.view(np.uint32).copy()
        if ks in bits:
            assert np.array_equal(u, bits[ks]), ks
        bits[ks] = u
    dev.set_tuning(unroll=1)
    c.Y.fill(0)
    dev.gemv_t(kind, c.W, c.Q, c.Y, rows, nb, T, c.xs, rows, rs=rows, bias=B, res=R)
    y = c.y_gpu()
    for t in range(T):
        assert rel_err(y[t], orc.epilogue(c.y_oracle(t), bias, res[t]), c.mag(t) + np.abs(bias) + np.abs(res[t])) < TOL, t


def test_graph_replay_matches_eager(dev, orc):
    """Q8_0 / Q6_K decode, split-K verify and GEMM (and the Q4_0 GEMM) captured in one graph and replayed
    several times, with eager work and synchronizations between the replays: every replay equals the
    eager run bit for bit (no node of the graph depends on memory set outside it)."""
    cases = [Case(dev, orc, Q8, 96, 136, 20, seed=4), Case(dev, orc, Q6, 80, 160, 20, seed=5), Case(dev, orc, 0, 64, 72, 20, seed=6)]
    outs = []
    for c in cases:
        c.quant()
        outs.append((dev.DevBuf(4 * c.rows), dev.DevBuf(4 * c.rows * 8), dev.DevBuf(4 * c.rows * c.T)))
    S = dev.Stream()

    def ops(s):
        for c, (Y1, Y8, YG) in zip(cases, outs):
            if c.kind != 0:
                dev.gemv(c.kind, c.W, c.Q, Y1, c.rows, c.nb, stream=s)
                dev.gemv_t(c.kind, c.W, c.Q, Y8, c.rows, c.nb, 8, c.xs, c.rows, stream=s)
            dev.gemm(c.kind, c.W, c.Q, YG, c.rows, c.nb, c.T, c.xs, c.rows, stream=s)

    bufs = [b for o in outs for b in o]
    for b in bufs:
        b.fill(0)
    dev.set_tuning(gemm_ksplit=3)  # split K in the verify kernels and the GEMMs: partial sums in the workspace
    ops(None)
    dev.sync()
    want = [b.download(np.uint32) for b in bufs]
    g = dev.Graph(S, ops)
    other = Case(dev, orc, Q6, 64, 64, seed=9)
    for rep in range(3):
        for b in bufs:
            b.fill(0)
        other.quant()
        dev.gemv(Q6, other.W, other.Q, other.Y, 64, 64)  # eager work between replays
        dev.sync()
        g.launch()
        S.sync()
        for b, w in zip(bufs, want):
            assert np.array_equal(b.download(np.uint32), w), rep
    for c, (Y1, _, YG) in zip(cases, outs):
        if c.kind != 0:
            assert rel_err(Y1.download(np.float32), c.y_oracle(0), c.mag(0)) < TOL
        y = YG.download(np.float32).reshape(c.T, c.rows)
        assert rel_err(y[c.T - 1], c.y_oracle(c.T - 1), c.mag(c.T - 1)) < TOL


@pytest.mark.parametrize("kind,nb", [(0, 511), (0, 2048), (synth.KIND_Q4_K, 2040), (Q8, 2047), (Q6, 2040)])
def test_max_sizes(dev, orc, kind, nb):
    """The largest rows the reference's loader accepts for each kind (core/ie_core.h:60, 187, 258-260:
    Q4_0 nb < 512, Q8_0 nb < 2048, Q4_K / Q6_K nb < 2048 with nb % 8 == 0; Q4_0 also past the
    reference's limit, up to this library's 2048 blocks): decode, verify (T = 8) and GEMM (T = 32).
    2049 blocks are refused before any launch."""
    rows = 37
    c = Case(dev, orc, kind, rows, nb, 32, seed=nb)
    c.quant()
    dev.gemv(kind, c.W, c.Q, c.Y, rows, nb)
    assert rel_err(c.y_gpu()[0], c.y_oracle(0), c.mag(0)) < TOL
    dev.gemv_t(kind, c.W, c.Q, c.Y, rows, nb, 8, c.xs, rows)
    y = c.y_gpu()
    for t in (0, 7):
        assert rel_err(y[t], c.y_oracle(t), c.mag(t)) < TOL, t
    dev.op_gemv(kind, c.W, c.Q, c.Y, rows, nb, 32, c.xs, rows)
    y = c.y_gpu()
    for t in (0, 31):
        assert rel_err(y[t], c.y_oracle(t), c.mag(t)) < TOL, t
    with pytest.raises(dev.AmdcError, match="2048 blocks"):
        dev.gemv(kind, c.W, c.Q, c.Y, rows, 2056)
