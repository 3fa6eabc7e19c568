"""The GEMV chain (amdc_chain_*): a list of quantize, decode-GEMV and Q8-producer operations in one
persistent launch with grid barriers, and its recorder (amdc_chain_record_begin / _end, the reference's
mk_put / mk_flush, src/hip.c:475-567). Every result equals the separate launches (amdc_quant_q8, then
amdc_gemv_q4 / _q4k with the same lane split, amdc_gemv_q8 / _q6k, amdc_rmsnorm_q8, amdc_swiglu_q8) bit for
bit, across repeated launches and graph replays, and the GEMVs match the oracle to the GEMV tolerance."""
import numpy as np
import pytest

from amdc import synth
from test_gpu_parity import Case, rel_err, TOL, q8_stride, ttype as synth_ttype

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _form1(dev):
    dev.set_tuning(form=1)  # the separate launches with the chain's lane split (bitwise comparison)
    yield
    dev.set_tuning()


def test_chain_equals_separate_launches(dev, orc):
    """x0 -> Q8 -> GEMV A (Q4_0, nb 13: a partial super-group) -> y1 -> Q8 -> GEMV B (Q4_K, with bias and
    residual) -> y2 -> Q8 -> GEMV C and D (Q4_0, one input, no barrier between them)."""
    g = np.random.default_rng(0)
    A = Case(dev, orc, 0, 256, 13, seed=1)  # 416 -> 256 (each output feeds the next stage's input)
    B = Case(dev, orc, 3, 1024, 8, seed=2)  # 256 -> 1024
    C_ = Case(dev, orc, 0, 77, 32, seed=3)  # 1024 -> 77
    D = Case(dev, orc, 0, 300, 32, seed=4)  # 1024 -> 300
    x0 = dev.DevBuf.of(A.x[0])
    q0, q1, q2 = dev.DevBuf(q8_stride(13)), dev.DevBuf(q8_stride(8)), dev.DevBuf(q8_stride(32))
    y1, y2, y3, y4 = (dev.DevBuf(4 * r) for r in (256, 1024, 77, 300))
    bias = dev.DevBuf.of(g.standard_normal(1024).astype(np.float32))
    res = dev.DevBuf.of(g.standard_normal(1024).astype(np.float32))
    ops = [dev.chain_quant(x0, q0, 13),
           dev.chain_gemv(0, A.W, q0, y1, 256, 13),
           dev.chain_quant(y1, q1, 8),
           dev.chain_gemv(3, B.W, q1, y2, 1024, 8, bias=bias, res=res),
           dev.chain_quant(y2, q2, 32),
           dev.chain_gemv(0, C_.W, q2, y3, 77, 32, sync=False),
           dev.chain_gemv(0, D.W, q2, y4, 300, 32)]
    ch = dev.Chain(ops)
    # the separate launches
    r0, r1, r2 = dev.DevBuf(q8_stride(13)), dev.DevBuf(q8_stride(8)), dev.DevBuf(q8_stride(32))
    z1, z2, z3, z4 = (dev.DevBuf(4 * r) for r in (256, 1024, 77, 300))
    dev.quant_q8(x0, r0, 13)
    dev.gemv(0, A.W, r0, z1, 256, 13)
    dev.quant_q8(z1, r1, 8)
    dev.gemv(3, B.W, r1, z2, 1024, 8, bias=bias, res=res)
    dev.quant_q8(z2, r2, 32)
    dev.gemv(0, C_.W, r2, z3, 77, 32)
    dev.gemv(0, D.W, r2, z4, 300, 32)
    want = [b.download(np.uint32) for b in (r0, z1, r1, z2, r2, z3, z4)]
    for rep in range(3):
        for b in (q0, q1, q2, y1, y2, y3, y4):
            b.fill(0)
        ch.launch()
        ch.check()
        got = [b.download(np.uint32) for b in (q0, y1, q1, y2, q2, y3, y4)]
        for i, (gt, wt) in enumerate(zip(got, want)):
            n = 10 * (13, 8, 32)[i // 2] if i in (0, 2, 4) else gt.size  # Q8 buffers: their 40 nb bytes
            assert np.array_equal(gt[:n], wt[:n]), (rep, i)
    # the first GEMV against the oracle
    yA = y1.download(np.float32)
    assert rel_err(yA, A.y_oracle(0), A.mag(0)) < TOL


@pytest.mark.parametrize("form", ["persistent", "streaming"])
def test_chain_graph_replay(dev, orc, form):
    """A chain captured in a HIP graph and replayed, with eager work between replays, equals the eager chain."""
    A = Case(dev, orc, 3, 3000, 160, seed=5)
    x0 = dev.DevBuf.of(A.x[0])
    q0, y = dev.DevBuf(q8_stride(160)), dev.DevBuf(4 * 3000)
    fm = dev.CHAIN_PERSISTENT if form == "persistent" else dev.CHAIN_STREAMING
    ch = dev.Chain([dev.chain_quant(x0, q0, 160), dev.chain_gemv(3, A.W, q0, y, 3000, 160)], form=fm)
    ch.launch()
    ch.check()
    want = y.download(np.uint32)
    assert rel_err(y.download(np.float32), A.y_oracle(0), A.mag(0)) < TOL
    S = dev.Stream()
    gph = dev.Graph(S, lambda s: ch.launch(s))
    other = Case(dev, orc, 0, 64, 128, seed=9)
    for rep in range(3):
        y.fill(0)
        other.quant()
        dev.sync()
        gph.launch()
        S.sync()
        assert np.array_equal(y.download(np.uint32), want), rep
    ch.check()


def test_chain_rejects_read_before_sync(dev, orc):
    A = Case(dev, orc, 0, 64, 8, seed=6)
    x0, q0, y = dev.DevBuf.of(A.x[0]), dev.DevBuf(q8_stride(8)), dev.DevBuf(4 * 64)
    with pytest.raises(dev.AmdcError, match="without a sync"):
        dev.Chain([dev.chain_quant(x0, q0, 8, sync=False), dev.chain_gemv(0, A.W, q0, y, 64, 8)])
    # overlapping byte ranges, not only equal pointers: the GEMV's input starts inside the Q8 bytes being written
    Qb = dev.DevBuf(2 * q8_stride(8))
    with pytest.raises(dev.AmdcError, match="without a sync"):
        dev.Chain([dev.chain_quant(x0, Qb, 8, sync=False), dev.chain_gemv(0, A.W, Qb.ptr + 256, y, 64, 8)])
    # a write after a read in one segment (the GEMV may still read q0 while the quantization overwrites it)
    with pytest.raises(dev.AmdcError, match="without a sync"):
        dev.Chain([dev.chain_gemv(0, A.W, q0, y, 64, 8, sync=False), dev.chain_quant(x0, q0, 8)])
    # disjoint ranges of one buffer in one segment are accepted
    ch = dev.Chain([dev.chain_quant(x0, Qb, 8, sync=False), dev.chain_gemv(0, A.W, Qb.ptr + q8_stride(8), y, 64, 8)])
    del ch
    with pytest.raises(dev.AmdcError, match="type"):
        op = dev.chain_quant(x0, q0, 8)
        op.type = 7
        dev.Chain([op])


def test_chain_fused_quant_equals_separate_launches(dev, orc):
    """GEMV operations on f32 vectors (AMDC_CHAIN_GEMV_X: every workgroup quantizes its input into LDS, no
    Q8 buffer, no barrier between quantization and GEMV): x0 -> A (Q4_0, nb 13) -> y1 -> B (Q4_K, bias and
    residual) -> y2 -> C and D (one input, no barrier between them), then E (Q4_0, nb 600: the quantization
    in two passes) on x0 again. Each output equals amdc_quant_q8 + amdc_gemv with the same lane split, bit
    for bit, across repeated launches."""
    g = np.random.default_rng(5)
    A = Case(dev, orc, 0, 256, 13, seed=11)
    B = Case(dev, orc, 3, 1024, 8, seed=12)
    C_ = Case(dev, orc, 0, 77, 32, seed=13)
    D = Case(dev, orc, 3, 300, 32, seed=14)
    E = Case(dev, orc, 0, 90, 600, seed=15)
    x0 = dev.DevBuf.of(A.x[0])
    xe = dev.DevBuf.of(E.x[0])
    y1, y2, y3, y4, y5 = (dev.DevBuf(4 * r) for r in (256, 1024, 77, 300, 90))
    bias = dev.DevBuf.of(g.standard_normal(1024).astype(np.float32))
    res = dev.DevBuf.of(g.standard_normal(1024).astype(np.float32))
    ops = [dev.chain_gemv_x(0, A.W, x0, y1, 256, 13),
           dev.chain_gemv_x(3, B.W, y1, y2, 1024, 8, bias=bias, res=res),
           dev.chain_gemv_x(0, C_.W, y2, y3, 77, 32, sync=False),
           dev.chain_gemv_x(3, D.W, y2, y4, 300, 32),
           dev.chain_gemv_x(0, E.W, xe, y5, 90, 600)]
    ch = dev.Chain(ops)
    want = []
    q = dev.DevBuf(q8_stride(600))
    z1, z2, z3, z4, z5 = (dev.DevBuf(4 * r) for r in (256, 1024, 77, 300, 90))
    dev.quant_q8(x0, q, 13)
    dev.gemv(0, A.W, q, z1, 256, 13)
    dev.quant_q8(z1, q, 8)
    dev.gemv(3, B.W, q, z2, 1024, 8, bias=bias, res=res)
    dev.quant_q8(z2, q, 32)
    dev.gemv(0, C_.W, q, z3, 77, 32)
    dev.gemv(3, D.W, q, z4, 300, 32)
    dev.quant_q8(xe, q, 600)
    dev.gemv(0, E.W, q, z5, 90, 600)
    want = [b.download(np.uint32) for b in (z1, z2, z3, z4, z5)]
    for rep in range(3):
        for b in (y1, y2, y3, y4, y5):
            b.fill(0)
        ch.launch()
        ch.check()
        got = [b.download(np.uint32) for b in (y1, y2, y3, y4, y5)]
        for i, (gt, wt) in enumerate(zip(got, want)):
            assert np.array_equal(gt, wt), (rep, i)
    assert rel_err(y5.download(np.float32), E.y_oracle(0), E.mag(0)) < TOL


def test_chain_q8_0_q6_k_equals_separate_launches(dev, orc):
    """Q8_0 and Q6_K GEMV operations in a chain (the matrices of a Q4_K_M file besides Q4_K): x0 -> Q8 ->
    GEMV A (Q8_0, nb 13) -> y1 -> Q8 -> GEMV B (Q6_K, bias and residual) -> y2 -> Q8 -> GEMV C (Q4_K) and D
    (Q8_0) on one input. Each output equals amdc_quant_q8 + amdc_gemv of the kind, bit for bit, across
    repeated launches; A and B match the oracle."""
    g = np.random.default_rng(9)
    Q8, Q6 = synth.KIND_Q8_0, synth.KIND_Q6_K
    A = Case(dev, orc, Q8, 256, 13, seed=21)
    B = Case(dev, orc, Q6, 1024, 8, seed=22)
    C_ = Case(dev, orc, 3, 300, 32, seed=23)
    D = Case(dev, orc, Q8, 77, 32, seed=24)
    x0 = dev.DevBuf.of(A.x[0])
    q0, q1, q2 = dev.DevBuf(q8_stride(13)), dev.DevBuf(q8_stride(8)), dev.DevBuf(q8_stride(32))
    y1, y2, y3, y4 = (dev.DevBuf(4 * r) for r in (256, 1024, 300, 77))
    bias = dev.DevBuf.of(g.standard_normal(1024).astype(np.float32))
    res = dev.DevBuf.of(g.standard_normal(1024).astype(np.float32))
    ops = [dev.chain_quant(x0, q0, 13),
           dev.chain_gemv(Q8, A.W, q0, y1, 256, 13),
           dev.chain_quant(y1, q1, 8),
           dev.chain_gemv(Q6, B.W, q1, y2, 1024, 8, bias=bias, res=res),
           dev.chain_quant(y2, q2, 32),
           dev.chain_gemv(3, C_.W, q2, y3, 300, 32, sync=False),
           dev.chain_gemv(Q8, D.W, q2, y4, 77, 32)]
    ch = dev.Chain(ops)
    r0, r1, r2 = dev.DevBuf(q8_stride(13)), dev.DevBuf(q8_stride(8)), dev.DevBuf(q8_stride(32))
    z1, z2, z3, z4 = (dev.DevBuf(4 * r) for r in (256, 1024, 300, 77))
    dev.quant_q8(x0, r0, 13)
    dev.gemv(Q8, A.W, r0, z1, 256, 13)
    dev.quant_q8(z1, r1, 8)
    dev.gemv(Q6, B.W, r1, z2, 1024, 8, bias=bias, res=res)
    dev.quant_q8(z2, r2, 32)
    dev.gemv(3, C_.W, r2, z3, 300, 32)
    dev.gemv(Q8, D.W, r2, z4, 77, 32)
    want = [b.download(np.uint32) for b in (z1, z2, z3, z4)]
    for rep in range(3):
        for b in (y1, y2, y3, y4):
            b.fill(0)
        ch.launch()
        ch.check()
        got = [b.download(np.uint32) for b in (y1, y2, y3, y4)]
        for i, (gt, wt) in enumerate(zip(got, want)):
            assert np.array_equal(gt, wt), (rep, i)
    assert rel_err(y1.download(np.float32), A.y_oracle(0), A.mag(0)) < TOL
    # B's input is the quantized y1 (not B's own activations): check it through the oracle on that input
    xq1 = r1.download(np.uint8)[:40 * 8]
    yb = orc.gemv(synth.GGML[Q6], B.qw, B.qs, 1024, 8, xq1)
    mag = orc.gemv_f64(synth.GGML[Q6], B.src, 1024, 8, xq1)[1]
    yb = orc.epilogue(yb, bias.download(np.float32), res.download(np.float32))
    assert rel_err(y2.download(np.float32), yb, mag + np.abs(bias.download(np.float32)) + np.abs(res.download(np.float32))) < TOL


def test_chain_rejects_f32_input_for_q8_0(dev, orc):
    A = Case(dev, orc, synth.KIND_Q8_0, 64, 8, seed=5)
    x0 = dev.DevBuf.of(A.x[0])
    y = dev.DevBuf(4 * 64)
    with pytest.raises(dev.AmdcError):
        dev.Chain([dev.chain_gemv_x(synth.KIND_Q8_0, A.W, x0, y, 64, 8)])


@pytest.mark.parametrize("kind", [0, 3])
def test_chain_streaming_equals_separate_launches(dev, orc, kind):
    """The streaming form (one workgroup of 768 threads per CU, each wave's next two items in flight across
    operations and barriers, split barriers, the f32 input quantized once per CU) on a list of one kind:
    x0 -> Q8 -> A (Q8 input) -> y1 -> B (f32 input, bias and residual) -> y2 -> C and D (one input, no
    barrier between them), then E (nb 600: the quantization in several passes) on its own vector. Each
    output equals amdc_quant_q8 + amdc_gemv bit for bit, across repeated launches; the auto form picks the
    streaming kernel for such a list, and the streaming form refuses a list of two kinds."""
    g = np.random.default_rng(17 + kind)
    nbA = 13 if kind == 0 else 16
    A = Case(dev, orc, kind, 256, nbA, seed=31)
    B = Case(dev, orc, kind, 1024, 8, seed=32)
    C_ = Case(dev, orc, kind, 77, 32, seed=33)
    D = Case(dev, orc, kind, 300, 32, seed=34)
    E = Case(dev, orc, kind, 90, 600, seed=35)
    x0, xe = dev.DevBuf.of(A.x[0]), dev.DevBuf.of(E.x[0])
    q0 = dev.DevBuf(q8_stride(nbA))
    y1, y2, y3, y4, y5 = (dev.DevBuf(4 * r) for r in (256, 1024, 77, 300, 90))
    bias = dev.DevBuf.of(g.standard_normal(1024).astype(np.float32))
    res = dev.DevBuf.of(g.standard_normal(1024).astype(np.float32))
    ops = [dev.chain_quant(x0, q0, nbA),
           dev.chain_gemv(kind, A.W, q0, y1, 256, nbA),
           dev.chain_gemv_x(kind, B.W, y1, y2, 1024, 8, bias=bias, res=res),
           dev.chain_gemv_x(kind, C_.W, y2, y3, 77, 32, sync=False),
           dev.chain_gemv_x(kind, D.W, y2, y4, 300, 32),
           dev.chain_gemv_x(kind, E.W, xe, y5, 90, 600)]
    q = dev.DevBuf(q8_stride(600))
    z0 = dev.DevBuf(q8_stride(nbA))
    z1, z2, z3, z4, z5 = (dev.DevBuf(4 * r) for r in (256, 1024, 77, 300, 90))
    dev.quant_q8(x0, z0, nbA)
    dev.gemv(kind, A.W, z0, z1, 256, nbA)
    dev.quant_q8(z1, q, 8)
    dev.gemv(kind, B.W, q, z2, 1024, 8, bias=bias, res=res)
    dev.quant_q8(z2, q, 32)
    dev.gemv(kind, C_.W, q, z3, 77, 32)
    dev.gemv(kind, D.W, q, z4, 300, 32)
    dev.quant_q8(xe, q, 600)
    dev.gemv(kind, E.W, q, z5, 90, 600)
    want = [b.download(np.uint32) for b in (z0, z1, z2, z3, z4, z5)]
    for fm in (dev.CHAIN_STREAMING, dev.CHAIN_AUTO):
        ch = dev.Chain(ops, form=fm)
        for rep in range(3):
            for b in (q0, y1, y2, y3, y4, y5):
                b.fill(0)
            ch.launch()
            ch.check()
            got = [b.download(np.uint32) for b in (q0, y1, y2, y3, y4, y5)]
            assert np.array_equal(got[0][:10 * nbA], want[0][:10 * nbA]), (fm, rep)
            for i in range(1, 6):
                assert np.array_equal(got[i], want[i]), (fm, rep, i)
        del ch
    assert rel_err(y5.download(np.float32), E.y_oracle(0), E.mag(0)) < TOL
    other = Case(dev, orc, 3 - kind, 64, 8, seed=36)
    with pytest.raises(dev.AmdcError, match="streaming form"):
        dev.Chain(ops + [dev.chain_gemv_x(3 - kind, other.W, x0, y3, 64, 8)], form=dev.CHAIN_STREAMING)


MODEL_CHAINS = {
    # (kind, [(name, rows, cols)]): each GEMV reads the previous one's output (its first cols values)
    "c1": (0, [("qkv", 12288, 4096), ("o", 4096, 4096), ("gate_up", 22016, 4096), ("down", 4096, 11008), ("lm_head", 32000, 4096)]),
    "c2": (3, [("gate_up", 34816, 5120), ("down", 5120, 17408), ("attn_in", 6144, 5120), ("attn_out", 5120, 6144),
               ("lm_head", 152064, 5120)]),
}


@pytest.mark.parametrize("cfg", ["c1", "c2"])
@pytest.mark.parametrize("form", ["persistent", "streaming"])
def test_chain_model_shapes(dev, orc, cfg, form):
    """A decode step's GEMVs at the c1 (Q4_0, Llama-7B) and c2 (Q4_K, 27B) shapes as one chain of dependent
    operations: each GEMV quantizes the previous GEMV's output (its first cols values) in the chain
    (AMDC_CHAIN_GEMV_X) and waits for it at a barrier, so a missing or early barrier changes the result.
    The waves hold up to about 25 items each (the 152064-row lm_head), so the streaming form's weight
    loads run ahead across every operation boundary. Every output equals amdc_quant_q8 + amdc_gemv bit for
    bit over three launches; the first and last GEMVs also match the oracle."""
    kind, shapes = MODEL_CHAINS[cfg]
    fm = dev.CHAIN_PERSISTENT if form == "persistent" else dev.CHAIN_STREAMING
    cases = [Case(dev, orc, kind, r, c // 32, seed=40 + i) for i, (_, r, c) in enumerate(shapes)]
    x0 = dev.DevBuf.of(cases[0].x[0])
    ys = [dev.DevBuf(4 * r) for _, r, _ in shapes]
    ops, src = [], x0
    for i, (_, r, c) in enumerate(shapes):
        ops.append(dev.chain_gemv_x(kind, cases[i].W, src, ys[i], r, c // 32))
        src = ys[i]
    q = dev.DevBuf(q8_stride(max(c for _, _, c in shapes) // 32))
    zs = [dev.DevBuf(4 * r) for _, r, _ in shapes]
    src = x0
    for i, (_, r, c) in enumerate(shapes):
        dev.quant_q8(src, q, c // 32)
        dev.gemv(kind, cases[i].W, q, zs[i], r, c // 32)
        src = zs[i]
    want = [z.download(np.uint32) for z in zs]
    ch = dev.Chain(ops, form=fm)
    for rep in range(3):
        for y in ys:
            y.fill(0)
        ch.launch()
        ch.check()
        for i, y in enumerate(ys):
            assert np.array_equal(y.download(np.uint32), want[i]), (rep, shapes[i][0])
    del ch
    # the first GEMV against the oracle; the last one on the oracle's quantization of its real input
    assert rel_err(ys[0].download(np.float32), cases[0].y_oracle(0), cases[0].mag(0)) < TOL
    last = cases[-1]
    xin = ys[-2].download(np.float32)[:32 * last.nb][None, :]
    xq = orc.quant_q8(xin)[0]
    yref = orc.gemv(synth_ttype(kind), last.qw, last.qs, last.rows, last.nb, xq, threads=16)
    mag = orc.gemv_f64(synth_ttype(kind), last.src, last.rows, last.nb, xq)[1]
    assert rel_err(ys[-1].download(np.float32), yref, mag) < TOL


def test_chain_trace(dev, orc):
    """amdc_chain_trace (the streaming form's timeline, as the reference megakernel's IE_MK_TRACE): every
    workgroup records its start, the first vector staged and the four boundary points of every operation
    in order, and the first compute wave's item times; the results do not change; the persistent form
    refuses a timeline."""
    A = Case(dev, orc, 0, 4096, 128, seed=51)
    B = Case(dev, orc, 0, 1000, 128, seed=52)
    x0 = dev.DevBuf.of(A.x[0])
    y1, y2 = dev.DevBuf(4 * 4096), dev.DevBuf(4 * 1000)
    ops = [dev.chain_gemv_x(0, A.W, x0, y1, 4096, 128), dev.chain_gemv_x(0, B.W, y1, y2, 1000, 128)]
    ch = dev.Chain(ops, form=dev.CHAIN_STREAMING)
    ch.launch()
    ch.check()
    want = y2.download(np.uint32)
    nw = ch.trace_words()
    grid = dev.cu_count()
    n, per = 2, 2 + 4 * 2 + 64
    assert nw == grid * per
    TB = dev.DevBuf(8 * nw)
    TB.fill(0)
    ch.trace(TB)
    ch.launch()
    ch.check()
    ch.trace(None)
    assert np.array_equal(y2.download(np.uint32), want)
    t = TB.download(np.uint64).reshape(grid, per).astype(np.int64)
    # start, B2 of the start, op 0: B1 Bw Br B2, op 1: B1 (the last operation records only B1)
    marks = t[:, [0, 1, 2, 3, 4, 5, 6]]
    assert (marks > 0).all()
    assert (np.diff(marks, axis=1) >= 0).all()
    # every workgroup passed the grid barrier after every workgroup's stores of op 0 completed
    assert marks[:, 4].min() >= marks[:, 3].max()
    items = t[:, 2 + 4 * n:]
    # the first compute wave of workgroup b is wave 8 b of the grid's compute waves: it has items of op 0
    # (4096 rows of 4 per wave: 1024 wave row groups) for 8 b < 1024
    nb_ = min(grid, 128)
    assert (items[:nb_, 0] > 0).all() and (items[grid:, 0] if grid > 128 else items[:0, 0]).size == 0
    ch2 = dev.Chain(ops, form=dev.CHAIN_PERSISTENT)
    with pytest.raises(dev.AmdcError, match="timeline"):
        ch2.trace(TB)


def _layer(dev, orc, seed):
    """The buffers of a decode layer's tail: x -> RMSNorm+Q8 -> gate, up (Q4_K) -> SwiGLU+Q8 -> down (Q6_K,
    residual x) -> y -> RMSNorm+Q8 -> a Q8_0 GEMV -> z."""
    nbD, nbH = 16, 48
    D, H = 32 * nbD, 32 * nbH
    g = np.random.default_rng(seed)
    L = {"nbD": nbD, "nbH": nbH, "D": D, "H": H}
    L["Wg"] = Case(dev, orc, 3, H, nbD, seed=seed + 1).W
    L["Wu"] = Case(dev, orc, 3, H, nbD, seed=seed + 2).W
    L["Wd"] = Case(dev, orc, 4, D, nbH, seed=seed + 3).W
    L["Wo"] = Case(dev, orc, 2, 96, nbD, seed=seed + 4).W
    L["x"] = dev.DevBuf.of(g.standard_normal(D).astype(np.float32))
    L["wn"] = dev.DevBuf.of((1.0 + 0.1 * g.standard_normal(D)).astype(np.float32))
    return L


def _outs(dev, L):
    nbD, nbH, D, H = L["nbD"], L["nbH"], L["D"], L["H"]
    o = {"xn": dev.DevBuf(4 * D), "q1": dev.DevBuf(q8_stride(nbD)), "gt": dev.DevBuf(4 * H), "up": dev.DevBuf(4 * H),
         "q2": dev.DevBuf(q8_stride(nbH)), "y": dev.DevBuf(4 * D), "yn": dev.DevBuf(4 * D), "q3": dev.DevBuf(q8_stride(nbD)),
         "z": dev.DevBuf(4 * 96)}
    for b in o.values():
        b.fill(0)
    return o


def _run_layer(dev, L, o, stream=None):
    """The layer as operator calls (launched, or recorded when a recording is on for `stream`)."""
    S = stream.s if stream is not None else None
    nbD, nbH, D, H = L["nbD"], L["nbH"], L["D"], L["H"]
    dev.rmsnorm_q8(L["x"], L["wn"], o["xn"], D, 1e-5, q=o["q1"], stream=S)
    dev.gemv(3, L["Wg"], o["q1"], o["gt"], H, nbD, stream=S)
    dev.gemv(3, L["Wu"], o["q1"], o["up"], H, nbD, stream=S)
    dev.swiglu_q8(o["gt"], o["up"], H, q=o["q2"], stream=S)
    dev.gemv(4, L["Wd"], o["q2"], o["y"], D, nbH, res=L["x"], stream=S)
    dev.rmsnorm_q8(o["y"], L["wn"], o["yn"], D, 1e-5, q=o["q3"], stream=S)
    dev.gemv(2, L["Wo"], o["q3"], o["z"], 96, nbD, stream=S)


def _same(dev, L, a, b):
    for k in a:
        n = {"q1": 40 * L["nbD"], "q3": 40 * L["nbD"], "q2": 40 * L["nbH"]}.get(k)
        x, y = a[k].download(np.uint8), b[k].download(np.uint8)
        if n:
            x, y = x[:n], y[:n]
        assert np.array_equal(x, y), k


def test_chain_producers_equal_separate_launches(dev, orc):
    """AMDC_CHAIN_RMSNORM_Q8 and AMDC_CHAIN_SWIGLU_Q8 in a persistent chain with GEMVs of three kinds: every
    float and Q8 output equals the separate launches (amdc_rmsnorm_q8, amdc_swiglu_q8, the GEMVs) bit for
    bit, over repeated launches; gate and up run in one segment (no barrier between them)."""
    L = _layer(dev, orc, 40)
    want = _outs(dev, L)
    _run_layer(dev, L, want)
    dev.sync()
    o = _outs(dev, L)
    nbD, nbH, D, H = L["nbD"], L["nbH"], L["D"], L["H"]
    ops = [dev.chain_rmsnorm_q8(L["x"], L["wn"], o["xn"], nbD, 1e-5, q=o["q1"]),
           dev.chain_gemv(3, L["Wg"], o["q1"], o["gt"], H, nbD, sync=False),
           dev.chain_gemv(3, L["Wu"], o["q1"], o["up"], H, nbD),
           dev.chain_swiglu_q8(o["gt"], o["up"], nbH, q=o["q2"]),
           dev.chain_gemv(4, L["Wd"], o["q2"], o["y"], D, nbH, res=L["x"]),
           dev.chain_rmsnorm_q8(o["y"], L["wn"], o["yn"], nbD, 1e-5, q=o["q3"]),
           dev.chain_gemv(2, L["Wo"], o["q3"], o["z"], 96, nbD)]
    ch = dev.Chain(ops)
    for rep in range(3):
        for b in o.values():
            b.fill(0)
        ch.launch()
        ch.check()
        _same(dev, L, o, want)
    # the streaming form takes no producer operation
    with pytest.raises(dev.AmdcError, match="streaming form"):
        dev.Chain(ops, form=dev.CHAIN_STREAMING)
    # a producer that reads what the operation before it writes, without a barrier, is refused
    bad = list(ops)
    bad[2] = dev.chain_gemv(3, L["Wu"], o["q1"], o["up"], H, nbD, sync=False)
    with pytest.raises(dev.AmdcError, match="without a sync"):
        dev.Chain(bad)


def test_chain_recorder(dev, orc):
    """amdc_chain_record_begin / _end: the same operator calls on a recording stream build a chain (barriers
    placed from the operands' byte ranges) whose launch equals the calls launched, bit for bit, also as a
    replayed HIP graph; a call that cannot be recorded fails, and so does the recording."""
    L = _layer(dev, orc, 50)
    want = _outs(dev, L)
    _run_layer(dev, L, want)
    dev.sync()
    o = _outs(dev, L)
    S = dev.Stream()
    with dev.ChainRecorder(S) as rec:
        _run_layer(dev, L, o, stream=S)
    dev.sync()
    for b in o.values():  # nothing ran while recording
        assert not b.download(np.uint8).any()
    rec.chain.launch(S.s)
    S.sync()
    rec.chain.check()
    _same(dev, L, o, want)
    gph = dev.Graph(S, lambda s: rec.chain.launch(s))
    for rep in range(3):
        for b in o.values():
            b.fill(0)
        dev.sync()
        gph.launch()
        S.sync()
        _same(dev, L, o, want)
    rec.chain.check()
    # an f32-input GEMV records as one operation (Q4_0 / Q4_K) or, with q8, as quantize + GEMV
    A = Case(dev, orc, 3, 300, 32, seed=61)
    x = dev.DevBuf.of(A.x[0])
    y0, y1, y2, q8 = dev.DevBuf(4 * 300), dev.DevBuf(4 * 300), dev.DevBuf(4 * 300), dev.DevBuf(q8_stride(32))
    dev.gemv_x(3, A.W, x, y0, 300, 32)
    with dev.ChainRecorder(S) as rec2:
        dev.gemv_x(3, A.W, x, y1, 300, 32, stream=S.s)
        dev.gemv_x(3, A.W, x, y2, 300, 32, q8=q8, stream=S.s)
    rec2.chain.launch(S.s)
    S.sync()
    w0 = y0.download(np.uint32)
    assert np.array_equal(y1.download(np.uint32), w0) and np.array_equal(y2.download(np.uint32), w0)
    assert rel_err(y0.download(np.float32), A.y_oracle(0), A.mag(0)) < TOL
    # refused: a verify GEMV (T = 2) on the recording stream; the recording then yields no chain
    B = Case(dev, orc, 3, 64, 8, T=2, seed=62)
    B.quant()
    with pytest.raises(dev.AmdcError, match="refused|cannot be recorded"):
        with dev.ChainRecorder(S):
            dev.gemv_t(3, B.W, B.Q, B.Y, 64, 8, 2, B.xs, 64, stream=S.s)
    # other streams launch as usual during a recording
    with dev.ChainRecorder(S) as rec3:
        dev.gemv(3, B.W, B.Q, B.Y, 64, 8)
        dev.gemv(3, B.W, B.Q, B.Y, 64, 8, stream=S.s)
    del rec3


@pytest.mark.parametrize("nb", [1, 13, 200])
def test_chain_producers_ragged(dev, nb):
    """The producer operations at block counts that are not multiples of a workgroup's 8 (and a single
    block): equal to amdc_rmsnorm_q8 / amdc_swiglu_q8 bit for bit."""
    n = 32 * nb
    g = np.random.default_rng(nb)
    x = dev.DevBuf.of(g.standard_normal(n).astype(np.float32))
    w = dev.DevBuf.of((1.0 + 0.1 * g.standard_normal(n)).astype(np.float32))
    a0 = g.standard_normal(n).astype(np.float32)
    b = dev.DevBuf.of(g.standard_normal(n).astype(np.float32))
    y0, q0, q1 = dev.DevBuf(4 * n), dev.DevBuf(q8_stride(nb)), dev.DevBuf(q8_stride(nb))
    a = dev.DevBuf.of(a0)
    dev.rmsnorm_q8(x, w, y0, n, 1e-6, q=q0)
    dev.swiglu_q8(a, b, n, q=q1)
    dev.sync()
    want = [y0.download(np.uint8), q0.download(np.uint8)[:40 * nb], a.download(np.uint8), q1.download(np.uint8)[:40 * nb]]
    y1, r0, r1 = dev.DevBuf(4 * n), dev.DevBuf(q8_stride(nb)), dev.DevBuf(q8_stride(nb))
    a2 = dev.DevBuf.of(a0)
    ch = dev.Chain([dev.chain_rmsnorm_q8(x, w, y1, nb, 1e-6, q=r0, sync=False), dev.chain_swiglu_q8(a2, b, nb, q=r1)])
    ch.launch()
    ch.check()
    got = [y1.download(np.uint8), r0.download(np.uint8)[:40 * nb], a2.download(np.uint8), r1.download(np.uint8)[:40 * nb]]
    for i, (gt, wt) in enumerate(zip(got, want)):
        assert np.array_equal(gt, wt), i
