"""One summation order for every GEMV form: results equal bit for bit.

The reference's multi-token kernels give each token exactly the bits of the
single-token kernel (kernels/ie_kernels.c:481-482, checked by its
tools/gemv_eq.c), which its MTP speculative decode relies on to emit exactly
the greedy tokens (README.md:515-522). Here every decode form (persistent first
form, second form, single-shot form, at any lane count, and the fused-quantization forms) and the int8-MFMA
verify kernels (T = 1..16, any K split) follow the super-group tree order, so
on ordinary (rounding) data they all return the same bits; the oracle check
of these values is in test_gpu_parity.py. Q6_K's verify kernel joins a
block's two half sums in another order (within the 1e-5 bound, not bit-equal)
and is left out.
"""
import numpy as np
import pytest

from amdc import synth

pytestmark = pytest.mark.gpu


def q8_stride(nb):
    return (40 * nb + 255) // 256 * 256


# (kind, rows, nb): ragged rows, Q4_0 partial super-groups (nb % 8 != 0), short and long rows, a partial last tile
SHAPES = [(0, 70, 13), (0, 130, 43), (0, 200, 128), (0, 150, 344), (0, 33, 511), (3, 90, 40), (3, 130, 160),
          (3, 77, 544), (3, 64, 1024), (2, 100, 100), (2, 70, 344)]


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
    finally:
        dev.set_tuning()


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
