"""Write the golden vectors of the quantized GEMV path from the reference's own
CPU code (hanw/amd.c src/cpu.c cpu_quant_q8 / cpu_gemv_q4 / cpu_gemv_q4k /
cpu_gemv_q8 / cpu_gemv_q6k and src/model.c model_mat_from_gguf), compiled from the reference sources by
oracle/Makefile into oracle/_ref/libref_cpu.so. Run here, where /root/reference
exists:  make -C oracle && python tests/golden/make_golden.py

Each fixture (golden_<name>.npz, no pickles) holds the seeded inputs (GGUF
bytes, f32 activations) and the reference's outputs (Q8 buffer, repacked qw /
qs, y as float32 bits). Shapes: the Q4_0 shapes of tests/kernel_test.c:28
(nb < 32, = 32, > 32, 511, rows % 8 != 0), Q4_K shapes with nb % 8 == 0, and
the K sizes of the benchmark configurations with a few rows; Q8_0 as Q4_0 and
Q6_K as Q4_K. A fixture that exists is kept (pass --force to rewrite all).
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [os.path.join(ROOT, "oracle"), os.path.join(ROOT, "amd.c_amd")]

from oracle import RefCPU  # noqa: E402
from amdc import synth  # noqa: E402

Q4_0_SHAPES = [(1, 1), (7, 3), (9, 11), (8, 32), (13, 33), (17, 36), (5, 64), (3, 100), (2, 511), (5, 128), (3, 344)]
Q4_K_SHAPES = [(1, 8), (7, 16), (9, 40), (3, 64), (5, 72), (2, 160), (2, 544), (3, 192)]
Q8_0_SHAPES = [(1, 1), (7, 3), (9, 11), (8, 32), (13, 33), (3, 100), (2, 511), (5, 128)]
Q6_K_SHAPES = [(1, 8), (7, 16), (9, 40), (3, 64), (2, 160), (2, 544), (3, 192)]
NAMES = {synth.KIND_Q4_0: "q4_0", synth.KIND_Q4_K: "q4_k", synth.KIND_Q8_0: "q8_0", synth.KIND_Q6_K: "q6_k"}


def special_activations(cols, seed):
    """N(0,1) with special blocks: all zero, one nonzero, exact .5 ties, huge/tiny."""
    x = synth.activations(1, cols, seed)[0] * np.float32(1.5)
    nb = cols // 32
    if nb >= 4:
        x[0:32] = 0.0                       # d = 0 -> q = 0
        x[32:64] = 0.0
        x[32 + 5] = -3.25                   # a single nonzero -> q = -127
        x[64:96] = np.arange(-16, 16, dtype=np.float32) * np.float32(127.0 / 16.0) / np.float32(2.0)  # ties
        x[96:128] *= np.float32(1e-30)      # tiny
    return x


def main():
    force = "--force" in sys.argv
    ref = RefCPU()
    out_dir = HERE
    n = 0
    for kind, shapes in ((synth.KIND_Q4_0, Q4_0_SHAPES), (synth.KIND_Q4_K, Q4_K_SHAPES), (synth.KIND_Q8_0, Q8_0_SHAPES),
                         (synth.KIND_Q6_K, Q6_K_SHAPES)):
        for i, (rows, nb) in enumerate(shapes):
            name = f"golden_{NAMES[kind]}_{rows}x{nb}.npz"
            if os.path.exists(os.path.join(out_dir, name)) and not force:
                continue
            cols = 32 * nb
            seed = 1000 * (kind + 1) + i
            src = synth.gguf(kind, rows, cols, seed)
            x = special_activations(cols, seed + 7)
            xq = ref.quant_q8(x)
            m = ref.mat(synth.GGML[kind], src, rows, cols)
            qw, qs = m.arrays()
            y = m.gemv(xq)
            m.free()
            np.savez_compressed(os.path.join(out_dir, name), kind=np.int32(kind), rows=np.int32(rows), nb=np.int32(nb), seed=np.int64(seed),
                                gguf=src, x=x, xq=xq, qw=qw, qs=qs, y_bits=y.view(np.uint32))
            n += 1
    print(f"wrote {n} fixtures to {out_dir}")


if __name__ == "__main__":
    main()
