"""A seeded sweep of the verify GEMV (amdc_gemv_*_t: the int8-MFMA kernels, up to 16 vectors per
launch, weights through LDS) over random shapes of every kind against the oracle's restatement of
cpu_gemv_q4 / _q4k / _q8 / _q6k (hanw/amd.c src/cpu.c:64-175): ragged row counts (partial 16-row
waves and 64-row tiles), partial super-group tiles, T = 1..24 (one to two launches), with and
without bias and residual, and several K splits. Every token's output is within the 1e-5 bound of
sum |terms|."""
import numpy as np
import pytest

from amdc import synth
from test_gpu_parity import TOL, Case, rel_err

pytestmark = pytest.mark.gpu

KINDS = [synth.KIND_Q4_0, synth.KIND_Q8_0, synth.KIND_Q4_K, synth.KIND_Q6_K]


def _shapes(n, seed):
    g = np.random.default_rng(seed)
    out = []
    for i in range(n):
        kind = KINDS[i % 4]
        rows = int(g.integers(1, 260))
        if kind in (synth.KIND_Q4_K, synth.KIND_Q6_K):
            nb = 8 * int(g.integers(1, 90))  # whole super-blocks: 1..89 (up to 12 tiles of 8)
        else:
            nb = int(g.integers(1, 700))
        T = int(g.integers(1, 25))
        out.append((kind, rows, nb, T, int(g.integers(0, 4)), int(g.integers(0, 2))))
    return out


@pytest.mark.parametrize("kind,rows,nb,T,ks,epi", _shapes(24, 2027))
def test_verify_random_shapes(dev, orc, kind, rows, nb, T, ks, epi):
    c = Case(dev, orc, kind, rows, nb, T, seed=rows * 7 + nb * 3 + T)
    c.quant()
    g = np.random.default_rng(rows + nb)
    bias = g.standard_normal(rows).astype(np.float32) if epi else None
    res = g.standard_normal((T, rows)).astype(np.float32) if epi else None
    B = dev.DevBuf.of(bias) if epi else None
    R = dev.DevBuf.of(res) if epi else None
    dev.set_tuning(gemm_ksplit=ks)
    try:
        dev.gemv_t(kind, c.W, c.Q, c.Y, rows, nb, T, c.xs, rows, rs=rows, bias=B, res=R)
        y = c.y_gpu()
    finally:
        dev.set_tuning()
    for t in range(T):
        want = orc.epilogue(c.y_oracle(t), bias, None if res is None else res[t])
        mag = c.mag(t) + (0 if bias is None else np.abs(bias)) + (0 if res is None else np.abs(res[t]))
        assert rel_err(y[t], want, mag) < TOL, (kind, rows, nb, T, ks, epi, t)
