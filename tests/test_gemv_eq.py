"""One summation order for every GEMV form: results equal bit for bit.

The reference's multi-token kernels give each token exactly the bits of the
single-token kernel (kernels/ie_kernels.c:481-482, checked by its
tools/gemv_eq.c), which its MTP speculative decode relies on to emit exactly
the greedy tokens (README.md:515-522). Here every decode form (persistent first
form, second form, single-shot form, K-split form, at any lane count, and the fused-quantization forms) and the int8-MFMA
verify kernels (T = 1..16, any K split, all four kinds) follow the super-group
tree order, so on ordinary (rounding) data they all return the same bits; the
oracle check of these values is in test_gpu_parity.py and test_gpu_k8.py.
"""
import numpy as np
import pytest

from amdc import synth

pytestmark = pytest.mark.gpu


def q8_stride(nb):
    return (40 * nb + 255) // 256 * 256


# (kind, rows, nb): ragged rows, Q4_0 partial super-groups (nb % 8 != 0), short and long rows, a partial last tile
SHAPES = [(0, 70, 13), (0, 130, 43), (0, 200, 128), (0, 150, 344), (0, 33, 511), (3, 90, 40), (3, 130, 160),
          (3, 77, 544), (3, 64, 1024), (2, 100, 100), (2, 70, 344), (4, 100, 160), (4, 70, 544), (4, 64, 40), (4, 130, 1024)]


def setup(dev, kind, rows, nb, T, seed):
    src = synth.gguf(kind, rows, 32 * nb, seed)
    x = synth.activations(T, 32 * nb, seed + 1)
    xs = q8_stride(nb)
    W = dev.DevBuf.of(dev.repack(kind, src, rows, 32 * nb))
    X = dev.DevBuf.of(x)
    Q = dev.DevBuf(T * xs)
    Q.fill(0)
    dev.quant_q8(X, Q, nb, T, 128 * nb, xs)
    return W, X, Q, xs


@pytest.mark.parametrize("kind,rows,nb", SHAPES)
def test_decode_forms_equal(dev, kind, rows, nb):
    """Every decode form and lane count gives the same bits (and gemv_x the same as gemv)."""
    W, X, Q, xs = setup(dev, kind, rows, nb, 1, seed=rows + nb)
    Y = dev.DevBuf(4 * rows)
    ref = None
    try:
        for form in (0, 1, 2, 3):
            for lanes in (0, 4, 8, 16, 32, 64):
                for wgs in (0, 5):
                    dev.set_tuning(lanes=lanes, form=form, wgs=wgs)
                    Y.fill(0xFF)
                    dev.gemv(kind, W, Q, Y, rows, nb)
                    got = Y.download(np.uint32)
                    if ref is None:
                        ref = got
                    assert np.array_equal(got, ref), (form, lanes, wgs, int((got != ref).sum()))
        for form in (0, 1, 3):  # the fused-quantization forms: persistent (x1) and single-shot (xs)
            for lanes in (0, 8, 16):
                dev.set_tuning(form=form, lanes=lanes)
                Y.fill(0xFF)
                dev.gemv_x(kind, W, X, Y, rows, nb)
                assert np.array_equal(Y.download(np.uint32), ref), ("gemv_x", form, lanes)
        if kind in (0, 3):  # the K-split form (form 4): ranges of 4 .. 64 super-groups, Q8 and f32 input
            for lanes in (4, 8, 16, 32, 64):
                dev.set_tuning(form=4, lanes=lanes)
                for fx in (False, True):
                    Y.fill(0xFF)
                    if fx:
                        dev.gemv_x(kind, W, X, Y, rows, nb)
                    else:
                        dev.gemv(kind, W, Q, Y, rows, nb)
                    assert np.array_equal(Y.download(np.uint32), ref), ("split", lanes, fx)
    finally:
        dev.set_tuning()


@pytest.mark.parametrize("kind,rows,nb", [(0, 4096, 344), (3, 5120, 544), (3, 1000, 160), (0, 700, 13)])
def test_gemv_ksplit_epilogue_and_q8(dev, kind, rows, nb):
    """The K-split form with bias and residual (added once, by the last range to arrive) and the Q8 copy of
    its f32 input (each range writes its slice) equal quant_q8 + the single-shot GEMV, on two calls in a
    row (the tile counters are left at zero)."""
    W, X, Q, xs = setup(dev, kind, rows, nb, 1, seed=rows)
    g = np.random.default_rng(rows)
    B = dev.DevBuf.of(g.standard_normal(rows).astype(np.float32))
    R = dev.DevBuf.of(g.standard_normal(rows).astype(np.float32))
    Y, Y2, Q2 = dev.DevBuf(4 * rows), dev.DevBuf(4 * rows), dev.DevBuf(xs)
    dev.gemv(kind, W, Q, Y, rows, nb, bias=B, res=R)
    want = Y.download(np.uint32)
    try:
        for lanes in (8, 16):
            dev.set_tuning(form=4, lanes=lanes)
            for rep in range(2):
                Y2.fill(0xFF)
                Q2.fill(0xFF)
                dev.gemv_x(kind, W, X, Y2, rows, nb, bias=B, res=R, q8=Q2)
                assert np.array_equal(Y2.download(np.uint32), want), (lanes, rep)
                assert np.array_equal(Q2.download(np.uint8)[:40 * nb], Q.download(np.uint8)[:40 * nb]), (lanes, rep)
    finally:
        dev.set_tuning()


# shapes whose f32-input GEMV takes the workgroup-per-CU kernels (amdc_gemv_*_xw1 / _xw2: 5 to 16 waves
# of rows per CU on 256 CUs): ragged row counts, a partial super-group, long rows (344 and 544 blocks:
# the quantization in one and in two load batches), with bias and residual
XW_SHAPES = [(0, 5003, 128), (0, 12288, 128), (0, 4096, 344), (0, 3001, 344), (0, 30000, 13), (3, 6144, 160), (3, 5121, 192),
             (3, 3000, 544)]


@pytest.mark.parametrize("kind,rows,nb", XW_SHAPES)
def test_gemv_x_workgroup_per_cu(dev, kind, rows, nb):
    """gemv_x on the workgroup-per-CU fused-quantization kernels equals quant_q8 + gemv bit for bit (the
    Q8 copy too), with and without bias and residual."""
    W, X, Q, xs = setup(dev, kind, rows, nb, 1, seed=5 * rows + nb)
    g = np.random.default_rng(rows)
    B = dev.DevBuf.of(g.standard_normal(rows).astype(np.float32))
    R = dev.DevBuf.of(g.standard_normal(rows).astype(np.float32))
    Y, Y2, Q2 = dev.DevBuf(4 * rows), dev.DevBuf(4 * rows), dev.DevBuf(xs)
    for bias, res in ((None, None), (B, R)):
        dev.gemv(kind, W, Q, Y, rows, nb, bias=bias, res=res)
        Y2.fill(0xFF)
        Q2.fill(0)
        dev.gemv_x(kind, W, X, Y2, rows, nb, bias=bias, res=res, q8=Q2)
        assert np.array_equal(Y2.download(np.uint32), Y.download(np.uint32)), (bias is None,)
        assert np.array_equal(Q2.download(np.uint8)[:40 * nb], Q.download(np.uint8)[:40 * nb])


@pytest.mark.parametrize("kind,rows,nb", SHAPES)
def test_verify_equals_decode(dev, kind, rows, nb):
    """gemv_t (T = 1..16, every K split the host can take, bias and residual) gives each token the bits of
    the decode GEMV of that token (gemv_eq)."""
    T = 16
    W, X, Q, xs = setup(dev, kind, rows, nb, T, seed=3 * rows + nb)
    g = np.random.default_rng(nb)
    bias = g.standard_normal(rows).astype(np.float32)
    res = g.standard_normal((T, rows)).astype(np.float32)
    B, R = dev.DevBuf.of(bias), dev.DevBuf.of(res)
    Y1, Y = dev.DevBuf(4 * rows), dev.DevBuf(4 * rows * T)
    dec = []
    for t in range(T):
        dev.gemv(kind, W, Q.ptr + t * xs, Y1, rows, nb, bias=B, res=R.ptr + 4 * t * rows)
        dec.append(Y1.download(np.uint32))
    dec = np.stack(dec)
    nt = (nb + 63) // 64
    try:
        for ks in sorted({0, 1, 2, 3, 5, nt}):
            dev.set_tuning(gemm_ksplit=ks)
            for Tn in range(1, T + 1):
                Y.fill(0xFF)
                dev.gemv_t(kind, W, Q, Y, rows, nb, Tn, xs, rows, rs=rows, bias=B, res=R)
                got = Y.download(np.uint32).reshape(T, rows)[:Tn]
                same = got == dec[:Tn]
                assert same.all(), (ks, Tn, int((~same).sum()))
    finally:
        dev.set_tuning()


def halfway_vector(nb, seed):
    """Activations whose quotients x / d fall on and next to the half-integers, where a quantization that
    does not divide could round the other way: per block, amax 127 d for a random or a unit d, and the
    other values (k + 0.5) d, moved by 0..3 ulp either way; some blocks with a tiny d (1e-39 .. 1e-30:
    a denormal amax and the reciprocal's range)."""
    g = np.random.default_rng(seed)
    x = np.zeros((nb, 32), np.float32)
    for b in range(nb):
        d = np.float32(1.0) if b % 3 == 0 else np.float32(g.uniform(0.01, 50.0))
        if b % 7 == 6:
            d = np.float32(10.0 ** g.uniform(-41, -32))
        x[b, 0] = np.float32(127.0) * d
        k = g.integers(-127, 127, 31).astype(np.float32) + np.float32(0.5)
        v = (k * d).astype(np.float32)
        steps = g.integers(-3, 4, 31)
        v = np.array([np.float32(np.nextafter(vi, np.float32(np.inf) if s > 0 else np.float32(-np.inf))) if s else vi
                      for vi, s in zip(v, steps)], np.float32)
        for _ in range(2):  # up to 3 ulp
            v = np.where(np.abs(steps) > 1, np.nextafter(v, np.where(steps > 0, np.inf, -np.inf).astype(np.float32)), v)
            steps = np.sign(steps) * np.maximum(np.abs(steps) - 1, 0)
        x[b, 1:] = np.clip(v, -np.float32(127.0) * d, np.float32(127.0) * d)
        g.shuffle(x[b])
    return x.reshape(-1)


@pytest.mark.parametrize("kind,rows,nb", [(0, 200, 128), (0, 12288, 128), (0, 4096, 344), (3, 6144, 160)])
def test_fused_quant_halfway(dev, orc, kind, rows, nb):
    """The fused quantizations (the GEMV prologue of the 256-thread and workgroup-per-CU kernels, and the
    streaming chain's) give the bits of the oracle's quantization (the reference's IEEE division and
    roundf) on values at and next to the rounding boundaries, and tiny scales."""
    x = halfway_vector(nb, seed=rows + nb)
    want = orc.quant_q8(x[None, :])[0]
    src = synth.gguf(kind, rows, 32 * nb, seed=rows)
    W = dev.DevBuf.of(dev.repack(kind, src, rows, 32 * nb))
    X = dev.DevBuf.of(x)
    Q, Qs = dev.DevBuf(q8_stride(nb)), dev.DevBuf(q8_stride(nb))
    Y, Y2, Y3 = dev.DevBuf(4 * rows), dev.DevBuf(4 * rows), dev.DevBuf(4 * rows)
    Q.fill(0)
    dev.gemv_x(kind, W, X, Y, rows, nb, q8=Q)
    assert np.array_equal(Q.download(np.uint8)[:40 * nb], want)
    dev.quant_q8(X, Qs, nb)
    assert np.array_equal(Qs.download(np.uint8)[:40 * nb], want)
    dev.gemv(kind, W, Qs, Y2, rows, nb)
    assert np.array_equal(Y.download(np.uint32), Y2.download(np.uint32))
    ch = dev.Chain([dev.chain_gemv_x(kind, W, X, Y3, rows, nb)], form=dev.CHAIN_STREAMING)
    ch.launch()
    ch.check()
    assert np.array_equal(Y3.download(np.uint32), Y2.download(np.uint32))


@pytest.mark.parametrize("kind,rows,nb", [(0, 16400, 128), (3, 17000, 160), (0, 20000, 13)])
def test_decode_512_thread_single_shot_equal(dev, kind, rows, nb):
    """From 16384 rows the one-item single-shot GEMV runs on 512-thread workgroups (amdc_gemv_*_s1w): its
    bits equal the persistent form's (form 1) and the 256-thread single-shot form's (a partial last
    workgroup included)."""
    W, X, Q, xs = setup(dev, kind, rows, nb, 1, seed=rows)
    Y = dev.DevBuf(4 * rows)
    dev.gemv(kind, W, Q, Y, rows, nb)
    assert dev.last_kernel().endswith("_s1w"), dev.last_kernel()
    got = Y.download(np.uint32)
    try:
        for form in (1, 2):
            dev.set_tuning(form=form)
            Y.fill(0xFF)
            dev.gemv(kind, W, Q, Y, rows, nb)
            assert np.array_equal(Y.download(np.uint32), got), form
    finally:
        dev.set_tuning()
