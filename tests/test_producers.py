"""The fused Q8 producers: RMSNorm + Q8 and SwiGLU + Q8 (the reference's OP_RMSNORM / OP_SWIGLU with a
Q8 output). CPU: the oracle restatements (src/cpu.c:276-281, 580) against float64 formulas and closed
forms. GPU: the float result within 1e-5 (relative, per element) of the float64 formula and of the
oracle; the Q8 copy equals cpu_quant_q8 of the kernel's own float result bit for bit."""
import numpy as np
import pytest

EPS = 1e-6


def rms64(x, w, eps):
    x = x.astype(np.float64)
    s = 1.0 / np.sqrt((x * x).mean(axis=-1, keepdims=True) + eps)
    return x * s * w.astype(np.float64)


def silu64(a, b):
    a = a.astype(np.float64)
    return a / (1.0 + np.exp(-a)) * b.astype(np.float64)


# ---------------------------------------------------------------- oracle (CPU)

def test_oracle_rmsnorm_pins(orc):
    g = np.random.default_rng(1)
    for n in (32, 4096, 5120):
        x = g.standard_normal((3, n)).astype(np.float32) * np.float32(3.0)
        w = (1.0 + 0.1 * g.standard_normal(n)).astype(np.float32)
        y = orc.rmsnorm(x, w, EPS)
        want = rms64(x, w, EPS)
        assert np.all(np.abs(y - want) <= 1e-5 * np.abs(want) + 1e-30)
        # with unit weights the output has unit root mean square
        y1 = orc.rmsnorm(x, np.ones(n, np.float32), 0.0)
        assert np.allclose(np.sqrt((y1.astype(np.float64) ** 2).mean(axis=1)), 1.0, rtol=1e-5)
        # scale invariance (eps 0) and the zero vector (eps > 0)
        assert np.allclose(orc.rmsnorm(x * np.float32(8.0), w, 0.0), orc.rmsnorm(x, w, 0.0), rtol=1e-6, atol=0)
    assert np.array_equal(orc.rmsnorm(np.zeros((1, 64), np.float32), np.ones(64, np.float32), EPS), np.zeros((1, 64), np.float32))


def test_oracle_swiglu_pins(orc):
    g = np.random.default_rng(2)
    a = (g.standard_normal(4096) * 4).astype(np.float32)
    b = g.standard_normal(4096).astype(np.float32)
    v = orc.swiglu(a, b)
    want = silu64(a, b)
    assert np.all(np.abs(v - want) <= 2e-6 * np.abs(want) + 1e-30)
    special = orc.swiglu(np.array([0.0, 60.0, -120.0], np.float32), np.array([5.0, 2.0, 3.0], np.float32))
    assert special[0] == 0.0 and special[1] == np.float32(120.0) and abs(special[2]) < 1e-40


# ---------------------------------------------------------------- GPU

@pytest.mark.gpu
@pytest.mark.parametrize("n,T", [(32, 1), (4096, 1), (5120, 3), (11008, 2), (17408, 1)])
def test_rmsnorm_q8(dev, orc, n, T):
    g = np.random.default_rng(n + T)
    x = (g.standard_normal((T, n)) * 2.0).astype(np.float32)
    x[0, :32] = 0.0  # a zero block: d = 0 in the Q8 copy
    w = (1.0 + 0.1 * g.standard_normal(n)).astype(np.float32)
    nb = n // 32
    qs = (40 * nb + 255) // 256 * 256
    X, Wd, Y, Q = dev.DevBuf.of(x), dev.DevBuf.of(w), dev.DevBuf(4 * T * n), dev.DevBuf(T * qs)
    Q.fill(0)
    dev.rmsnorm_q8(X, Wd, Y, n, EPS, Q, T, 4 * n, 4 * n, qs)
    y = Y.download(np.float32).reshape(T, n)
    want = rms64(x, w, EPS)
    assert np.all(np.abs(y - want) <= 1e-5 * np.abs(want) + 1e-30)
    ref = orc.rmsnorm(x, w, EPS)
    assert np.all(np.abs(y - ref) <= 1e-5 * np.abs(ref) + 1e-30)
    q = Q.download(np.uint8).reshape(T, qs)[:, :40 * nb]
    assert np.array_equal(q, orc.quant_q8(y))
    Y2 = dev.DevBuf(4 * T * n)
    dev.rmsnorm_q8(X, Wd, Y2, n, EPS, None, T, 4 * n, 4 * n, 0)  # without the Q8 copy
    assert np.array_equal(Y2.download(np.uint32), Y.download(np.uint32))


@pytest.mark.gpu
@pytest.mark.parametrize("n,T", [(32, 1), (11008, 1), (17408, 2)])
def test_swiglu_q8(dev, orc, n, T):
    g = np.random.default_rng(n * 3 + T)
    a = (g.standard_normal((T, n)) * 4.0).astype(np.float32)
    b = g.standard_normal((T, n)).astype(np.float32)
    a[0, :3] = (0.0, 60.0, -120.0)
    nb = n // 32
    qs = (40 * nb + 255) // 256 * 256
    A, B, Q = dev.DevBuf.of(a), dev.DevBuf.of(b), dev.DevBuf(T * qs)
    Q.fill(0)
    dev.swiglu_q8(A, B, n, Q, T, 4 * n, qs)
    v = A.download(np.float32).reshape(T, n)
    want = silu64(a, b)
    assert np.all(np.abs(v - want) <= 1e-5 * np.abs(want) + 1e-30)
    assert np.all(np.abs(v - orc.swiglu(a, b)) <= 1e-5 * np.abs(want) + 1e-30)
    q = Q.download(np.uint8).reshape(T, qs)[:, :40 * nb]
    assert np.array_equal(q, orc.quant_q8(v))


@pytest.mark.gpu
def test_producers_reject_bad_sizes(dev):
    X = dev.DevBuf(4 * 64)
    with pytest.raises(dev.AmdcError, match="multiple of 32"):
        dev.rmsnorm_q8(X, X, X, 40, EPS)
    with pytest.raises(dev.AmdcError, match="strides"):
        dev.swiglu_q8(X, X, 32, X, 2, 64, 40)
