"""The C ABI driven from C: tests/capi/launch_op.c, built with gcc against include/amdc_q4.h,
runs the reference's launch_op for OP_QUANT and OP_GEMV_Q4 / _Q4K / _Q8 / _Q6K
(src/hip.c:922-1089) over T tokens in an arena with 256-byte token strides, on its own stream,
eagerly and as a replayed HIP graph, with IE_GEMM_MIN=17 (the reference's default,
src/hip.c:972-974) or unset (the library's rule).

Checked here: every token's Q8 buffer equals the oracle's cpu_quant_q8 bit for bit; every output
is within 1e-5 of sum |terms| of the oracle (src/cpu.c order) plus the bias / residual epilogue;
below the GEMM threshold (the decode and multi-vector kernels) every output equals the decode
GEMV of its token bit for bit (Q6_K's verify kernel excepted).
"""
import os
import subprocess

import numpy as np
import pytest

from amdc import synth

HERE = os.path.dirname(os.path.abspath(__file__))
EXE = os.path.join(HERE, "capi", "launch_op")
TOL = 1e-5


def test_launch_op_built():
    """The host test is built (by build()) and rejects a bad command line without touching a GPU."""
    assert os.access(EXE, os.X_OK), "tests/capi/launch_op is not built: run __graft_entry__.build()"
    r = subprocess.run([EXE], capture_output=True, text=True, timeout=30)
    assert r.returncode == 1 and "usage" in r.stderr


def gemm_taken(T, gmin, rows, cols):
    if T == 1:
        return False
    if gmin is not None:
        return T >= int(gmin)
    return T >= 33 or (T >= 20 and rows * cols <= 1 << 24)


CASES = [(k, T, g) for k in (synth.KIND_Q4_0, synth.KIND_Q4_K, synth.KIND_Q8_0, synth.KIND_Q6_K)
         for T in (1, 6, 16, 17, 40) for g in ("17", None)]


@pytest.mark.gpu
@pytest.mark.parametrize("kind,T,gmin", CASES, ids=[f"k{k}-T{T}-min{g}" for k, T, g in CASES])
def test_launch_op(dev, orc, tmp_path, kind, T, gmin):
    rows, cols = 300, 2048 if kind != synth.KIND_Q4_0 else 2080  # Q4_0: a ragged last super-group
    nb, tt = cols // 32, synth.GGML[kind]
    seed = 7 * kind + T
    src = synth.gguf(kind, rows, cols, seed)
    x = synth.activations(T, cols, seed + 1)
    g = np.random.default_rng(seed)
    bias = g.standard_normal(rows).astype(np.float32)
    res = g.standard_normal((T, rows)).astype(np.float32)
    src.tofile(tmp_path / "w.gguf")
    x.tofile(tmp_path / "x.f32")
    bias.tofile(tmp_path / "bias.f32")
    res.tofile(tmp_path / "res.f32")
    env = dict(os.environ)
    env.pop("IE_GEMM_MIN", None)
    if gmin is not None:
        env["IE_GEMM_MIN"] = gmin
    print(f"launch_op kind {kind} {rows}x{cols} T={T} IE_GEMM_MIN={gmin}", flush=True)
    r = subprocess.run([EXE, str(kind), str(rows), str(cols), str(T), str(tmp_path)], capture_output=True, text=True,
                       timeout=60, env=env)
    assert r.returncode == 0, r.stdout + r.stderr
    q8 = np.fromfile(tmp_path / "q8.bin", dtype=np.uint8).reshape(T, 40 * nb)
    y = np.fromfile(tmp_path / "y.f32", dtype=np.float32).reshape(T, rows)

    xq = orc.quant_q8(x)
    assert np.array_equal(q8, xq), "OP_QUANT differs from cpu_quant_q8"
    qw, qs = orc.repack(tt, src, rows, nb)
    for t in range(T):
        want = orc.epilogue(orc.gemv(tt, qw, qs, rows, nb, xq[t]), bias, res[t])
        mag = orc.gemv_f64(tt, src, rows, nb, xq[t])[1] + np.abs(bias) + np.abs(res[t])
        err = np.abs(y[t].astype(np.float64) - want) / np.maximum(mag, 1e-30)
        assert err.max() < TOL, f"token {t}: rel err {err.max():.3e} at row {int(err.argmax())}"

    if gemm_taken(T, gmin, rows, cols) or (kind == synth.KIND_Q6_K and T > 1):
        return
    W = dev.DevBuf.of(dev.repack(kind, src, rows, cols))
    xs = (40 * nb + 255) // 256 * 256
    qpad = np.zeros((T, xs), dtype=np.uint8)
    qpad[:, :40 * nb] = xq
    Q, Y = dev.DevBuf.of(qpad), dev.DevBuf(4 * rows)
    B, R = dev.DevBuf.of(bias), dev.DevBuf.of(res)
    for t in range(T):
        dev.gemv(kind, W, Q.ptr + t * xs, Y, rows, nb, bias=B, res=R.ptr + 4 * t * rows)
        same = Y.download(np.uint32) == y[t].view(np.uint32)
        assert same.all(), f"token {t}: {int((~same).sum())} outputs differ from the decode GEMV"
    for b in (W, Q, Y, B, R):
        b.free()
