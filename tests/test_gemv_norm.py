"""The decode GEMV with the fused RMSNorm tail (amdc_gemv_norm; the reference's GEMV launch with NW / NY /
NQ, src/hip.c:928-931, and its tail gemv_norm_tail, kernels/ie_kernels.c:267-283): y equals the plain
decode GEMV of the kind bit for bit, and ny / nq equal amdc_rmsnorm_q8 of that y bit for bit (the same
device code), on the single-shot kernels and the second form, over back-to-back launches (the arrival
counter returns to 0) and graph replays. The plain GEMV and amdc_rmsnorm_q8 are themselves held to the
oracle by test_gpu_parity / test_gpu_k8 / test_producers; y is also checked against the oracle here."""
import numpy as np
import pytest

from test_gpu_parity import Case, rel_err, TOL, q8_stride

pytestmark = pytest.mark.gpu

# (kind, rows, nb): Q4_0 / Q4_K on the single-shot kernels (1 to 4 super-groups per lane, a partial
# super-group, the longest row), Q8_0 and Q6_K on the second form
SHAPES = [(0, 512, 128), (0, 96, 13), (3, 1024, 64), (3, 256, 1024), (3, 160, 2048), (2, 256, 64), (4, 320, 96), (4, 4096, 160)]


@pytest.mark.parametrize("kind,rows,nb", SHAPES)
def test_gemv_norm_equals_gemv_then_rmsnorm(dev, orc, kind, rows, nb):
    A = Case(dev, orc, kind, rows, nb, seed=rows + nb)
    A.quant()
    g = np.random.default_rng(nb)
    nw = dev.DevBuf.of((1.0 + 0.1 * g.standard_normal(rows)).astype(np.float32))
    res = dev.DevBuf.of(g.standard_normal(rows).astype(np.float32))
    y0, n0, q0 = dev.DevBuf(4 * rows), dev.DevBuf(4 * rows), dev.DevBuf(q8_stride(rows // 32))
    dev.gemv(kind, A.W, A.Q, y0, rows, nb, res=res)
    dev.rmsnorm_q8(y0, nw, n0, rows, 1e-5, q=q0)
    dev.sync()
    want = [b.download(np.uint8) for b in (y0, n0)] + [q0.download(np.uint8)[:40 * (rows // 32)]]
    y, ny, nq = dev.DevBuf(4 * rows), dev.DevBuf(4 * rows), dev.DevBuf(q8_stride(rows // 32))

    def check(tag):
        got = [b.download(np.uint8) for b in (y, ny)] + [nq.download(np.uint8)[:40 * (rows // 32)]]
        for name, a, b in zip(("y", "ny", "nq"), got, want):
            assert np.array_equal(a, b), (tag, name)

    for rep in range(3):
        for b in (y, ny, nq):
            b.fill(0)
        dev.gemv_norm(kind, A.W, A.Q, y, rows, nb, nw, ny, 1e-5, nq=nq, res=res)
        dev.sync()
        check(rep)
    S = dev.Stream()
    gph = dev.Graph(S, lambda s: dev.gemv_norm(kind, A.W, A.Q, y, rows, nb, nw, ny, 1e-5, nq=nq, res=res, stream=s))
    for rep in range(3):
        for b in (y, ny, nq):
            b.fill(0)
        dev.sync()
        gph.launch()
        S.sync()
        check(f"graph {rep}")
    # without the Q8 copy
    ny.fill(0)
    dev.gemv_norm(kind, A.W, A.Q, y, rows, nb, nw, ny, 1e-5, res=res)
    dev.sync()
    assert np.array_equal(ny.download(np.uint8), want[1])
    # y against the oracle (the residual added)
    yo = A.y_oracle(0) + res.download(np.float32)
    assert rel_err(y.download(np.float32), yo, A.mag(0) + np.abs(res.download(np.float32))) < TOL


def test_gemv_norm_rejects(dev, orc):
    A = Case(dev, orc, 0, 100, 8, seed=3)
    nw, ny = dev.DevBuf(400), dev.DevBuf(400)
    with pytest.raises(dev.AmdcError, match="multiple of 32"):
        dev.gemv_norm(0, A.W, A.Q, A.Y, 100, 8, nw, ny, 1e-5)
    with pytest.raises(dev.AmdcError, match="required"):
        dev.gemv_norm(0, A.W, A.Q, A.Y, 96, 8, None, ny, 1e-5)
