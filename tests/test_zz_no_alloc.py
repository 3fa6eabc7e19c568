"""amdc_op_gemv_noalloc: amdc_op_gemv with the code object's fixed scratch array as its workspace
(no device allocation). Through the C ABI, its outputs equal amdc_op_gemv's bit for bit (the same
kernels, launch choices and summation order) on two calls in a row, the second on a smaller
input, for the paths that use a workspace (the split-K verify GEMV and the prefill GEMM, with
split-K partial sums) and one that does not (decode); a first-seen size captured into a HIP graph
and replayed gives the eager bits on every replay; a call whose workspace exceeds the array is
rejected before any launch (its output untouched).
"""
import numpy as np
import pytest

from amdc import synth

pytestmark = pytest.mark.gpu


def q8_stride(nb):
    return (40 * nb + 255) // 256 * 256


class Case:
    def __init__(self, dev, kind, rows, cols, T, seed):
        self.kind, self.rows, self.nb, self.T = kind, rows, cols // 32, T
        self.xs = q8_stride(self.nb)
        src = synth.gguf(kind, rows, cols, seed)
        x = synth.activations(T, cols, seed + 1)
        g = np.random.default_rng(seed)
        self.W = dev.DevBuf.of(dev.repack(kind, src, rows, cols))
        self.X = dev.DevBuf.of(x)
        self.Q = dev.DevBuf(T * self.xs)
        self.B = dev.DevBuf.of(g.standard_normal(rows).astype(np.float32))
        self.R = dev.DevBuf.of(g.standard_normal((T, rows)).astype(np.float32))
        self.Y = dev.DevBuf(4 * T * rows)
        dev.quant_q8(self.X, self.Q, self.nb, T, 128 * self.nb, self.xs)

    def run(self, fn, stream=None):
        fn(self.kind, self.W, self.Q, self.Y, self.rows, self.nb, self.T, self.xs, self.rows, self.rows, bias=self.B,
           res=self.R, stream=stream)

    def out(self):
        return self.Y.download(np.uint32)

    def free(self):
        for b in (self.W, self.X, self.Q, self.B, self.R, self.Y):
            b.free()


# pairs (first call, second call on a smaller input): the verify GEMV with split-K partial sums, the
# prefill GEMM (c4 shapes, split K), the decode GEMV (no workspace)
PAIRS = [
    ((synth.KIND_Q4_K, 17408, 5120, 8), (synth.KIND_Q4_K, 6144, 5120, 5)),
    ((synth.KIND_Q4_0, 4096, 11008, 16), (synth.KIND_Q4_0, 4096, 4096, 3)),
    ((synth.KIND_Q4_K, 5120, 17408, 256), (synth.KIND_Q4_K, 17408, 5120, 64)),
    ((synth.KIND_Q6_K, 5120, 17408, 256), (synth.KIND_Q8_0, 4096, 4096, 40)),
    ((synth.KIND_Q4_0, 11008, 4096, 1), (synth.KIND_Q4_K, 5120, 6144, 1)),
]


@pytest.mark.parametrize("first,second", PAIRS, ids=[f"{a[0]}-{a[1]}x{a[2]}-T{a[3]}" for a, _ in PAIRS])
def test_noalloc_equals_op_gemv(dev, first, second):
    for i, (kind, rows, cols, T) in enumerate((first, second)):
        print(f"noalloc kind {kind} {rows}x{cols} T={T}", flush=True)
        c = Case(dev, kind, rows, cols, T, seed=rows + cols + T + i)
        c.Y.fill(0xFF)
        c.run(dev.op_gemv)
        want = c.out()
        c.Y.fill(0xFF)
        c.run(dev.op_gemv_noalloc)
        got = c.out()
        assert np.array_equal(got, want), f"call {i}: {int((got != want).sum())} outputs differ from amdc_op_gemv"
        c.free()


def test_noalloc_graph_capture(dev):
    """A size never seen before, captured and replayed: no allocation happens inside the capture."""
    c = Case(dev, synth.KIND_Q4_K, 2560, 6656, 12, seed=11)
    s = dev.Stream()
    g = dev.Graph(s, lambda st: c.run(dev.op_gemv_noalloc, stream=st))
    c.Y.fill(0xFF)
    c.run(dev.op_gemv)
    want = c.out()
    for r in range(3):
        c.Y.fill(0xFF)
        g.launch()
        s.sync()
        got = c.out()
        assert np.array_equal(got, want), f"replay {r}: {int((got != want).sum())} outputs differ"
    del g
    c.free()


def test_noalloc_rejects_oversize(dev):
    """5120 x 17408 Q4_K at T = 2048 needs about 97 MB of workspace (64 MiB available): an error, no launch."""
    c = Case(dev, synth.KIND_Q4_K, 5120, 17408, 2048, seed=5)
    c.Y.fill(0x7F)
    with pytest.raises(dev.AmdcError, match="scratch array holds"):
        c.run(dev.op_gemv_noalloc)
    dev.sync()
    assert np.all(c.Y.download(np.uint8) == 0x7F)
    c.free()
