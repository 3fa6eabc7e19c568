"""The oracle (oracle/amdc_oracle.c) pinned before it is trusted:

- bit for bit against the golden vectors written by the reference's own
  compiled cpu.c / model.c (tests/golden, make_golden.py);
- against oracle/_ref (the reference compiled here) on fresh seeds, when built;
- the integer block dots against an int64 brute force over the GGUF bytes;
- the float GEMV against a float64 element loop over the GGUF bytes, rel err
  < 1e-5 of sum |terms| (the reference's tests/kernel_test.c:59-80 check);
- f16 conversions against numpy over all 65536 halves / RNE edge cases;
- Q8 invariants: asum = sum q, |q| <= 127, max |q| = 127, d = 0 -> q = 0.
"""
import glob
import os

import numpy as np
import pytest

from amdc import synth
from oracle import GGML_Q4_0, GGML_Q4_K, GGML_Q6_K, GGML_Q8_0, RefCPU

GOLDEN = sorted(glob.glob(os.path.join(os.path.dirname(__file__), "golden", "golden_*.npz")))


def ttype(kind):
    return synth.GGML[kind]


def test_golden_present():
    assert len(GOLDEN) >= 34
    for name in ("q4_0", "q4_k", "q8_0", "q6_k"):
        assert any(f"golden_{name}_" in p for p in GOLDEN), name


@pytest.mark.parametrize("path", GOLDEN, ids=[os.path.basename(p)[7:-4] for p in GOLDEN])
def test_oracle_matches_reference_golden(orc, path):
    g = np.load(path)  # no pickles (allow_pickle=False)
    kind, rows, nb = int(g["kind"]), int(g["rows"]), int(g["nb"])
    xq = orc.quant_q8(g["x"])
    assert np.array_equal(xq.reshape(-1), g["xq"].reshape(-1)), "Q8 buffer differs from cpu_quant_q8"
    qw, qs = orc.repack(ttype(kind), g["gguf"], rows, nb)
    assert np.array_equal(qw, g["qw"]) and np.array_equal(qs, g["qs"]), "repack differs from the reference"
    y = orc.gemv(ttype(kind), qw, qs, rows, nb, xq.reshape(-1))
    assert np.array_equal(y.view(np.uint32), g["y_bits"]), "GEMV differs from cpu_gemv (bitwise)"
    # multi-threaded rows: same per-row arithmetic, same bits
    y8 = orc.gemv(ttype(kind), qw, qs, rows, nb, xq.reshape(-1), threads=4)
    assert np.array_equal(y8.view(np.uint32), g["y_bits"])


@pytest.mark.skipif(not RefCPU.available(), reason="oracle/_ref not built (needs /root/reference)")
@pytest.mark.parametrize("kind,rows,nb", [(0, 37, 129), (0, 64, 344), (3, 33, 96), (3, 16, 544), (2, 37, 129), (2, 16, 448),
                                         (4, 33, 96), (4, 16, 448)])
def test_oracle_matches_compiled_reference(orc, kind, rows, nb):
    ref = RefCPU()
    src = synth.gguf(kind, rows, 32 * nb, seed=rows * 7 + nb)
    x = synth.activations(3, 32 * nb, seed=nb)
    m = ref.mat(ttype(kind), src, rows, 32 * nb)
    qw_r, qs_r = m.arrays()
    qw, qs = orc.repack(ttype(kind), src, rows, nb)
    assert np.array_equal(qw, qw_r) and np.array_equal(qs, qs_r)
    for t in range(3):
        xq = orc.quant_q8(x[t])
        assert np.array_equal(xq, ref.quant_q8(x[t]))
        assert np.array_equal(orc.gemv(ttype(kind), qw, qs, rows, nb, xq).view(np.uint32), m.gemv(xq).view(np.uint32))


@pytest.mark.parametrize("kind,rows,nb", [(0, 5, 1), (0, 9, 37), (0, 3, 511), (3, 4, 8), (3, 7, 168), (2, 5, 1), (2, 9, 37),
                                         (4, 4, 8), (4, 7, 168)])
def test_block_dots_brute_force(orc, kind, rows, nb):
    src = synth.gguf(kind, rows, 32 * nb, seed=11 + nb)
    xq = orc.quant_q8(synth.activations(1, 32 * nb, seed=nb)[0] * 4)
    qw, _ = orc.repack(ttype(kind), src, rows, nb)
    assert np.array_equal(orc.block_dots(ttype(kind), qw, rows, nb, xq), orc.block_dots_gguf(ttype(kind), src, rows, nb, xq))


@pytest.mark.parametrize("kind,rows,nb", [(0, 13, 33), (0, 4, 344), (3, 6, 160), (3, 3, 544), (2, 13, 33), (2, 4, 344),
                                         (4, 6, 160), (4, 3, 544)])
def test_gemv_vs_float64(orc, kind, rows, nb):
    src = synth.gguf(kind, rows, 32 * nb, seed=5 + nb)
    x = synth.activations(1, 32 * nb, seed=9)[0]
    xq = orc.quant_q8(x)
    qw, qs = orc.repack(ttype(kind), src, rows, nb)
    y = orc.gemv(ttype(kind), qw, qs, rows, nb, xq)
    yref, mag = orc.gemv_f64(ttype(kind), src, rows, nb, xq)
    err = np.abs(y.astype(np.float64) - yref) / np.maximum(mag, 1e-30)
    assert err.max() < 1e-5


def test_dequant_q4_0_closed_form(orc):
    # one block: d = 0.5, nibble byte j = j | (15 - j) << 4 -> weights (j - 8) * 0.5, (7 - j) * 0.5
    blk = np.zeros(18, dtype=np.uint8)
    blk[0:2] = np.array([0.5], dtype=np.float16).view(np.uint8)
    blk[2:] = [(j | ((15 - j) << 4)) for j in range(16)]
    w = orc.dequant(GGML_Q4_0, blk, 32)
    want = np.array([(j - 8) * 0.5 for j in range(16)] + [(7 - j) * 0.5 for j in range(16)], dtype=np.float32)
    assert np.array_equal(w, want)


def test_dequant_q4_k_closed_form(orc):
    # d = 2, dmin = 1, all 12 scale bytes 0x41 (sc = 1 | ..): sub-block j < 4: sc = 0x41 & 63 = 1, mn = 1;
    # j >= 4: sc = (0x41 & 15) | (0x41 >> 6) << 4 = 1 | 16 = 17, mn = (0x41 >> 4) | 16 = 4 | 16 = 20
    blk = np.zeros(144, dtype=np.uint8)
    blk[0:4] = np.array([2.0, 1.0], dtype=np.float16).view(np.uint8)
    blk[4:16] = 0x41
    blk[16:] = 0x5A  # low nibble 10, high nibble 5
    w = orc.dequant(GGML_Q4_K, blk, 256)
    for sub in range(8):
        sc, mn = (1, 1) if sub < 4 else (17, 20)
        q = 10 if sub % 2 == 0 else 5
        assert np.all(w[32 * sub:32 * sub + 32] == np.float32(2.0 * sc * q - 1.0 * mn)), sub


def test_dequant_q8_0_closed_form(orc):
    # d = 0.5, q_j = j - 16 (bytes 240..255, 0..15) -> weights (j - 16) * 0.5
    blk = np.zeros(34, dtype=np.uint8)
    blk[0:2] = np.array([0.5], dtype=np.float16).view(np.uint8)
    blk[2:] = (np.arange(32) - 16).astype(np.int8).view(np.uint8)
    assert np.array_equal(orc.dequant(GGML_Q8_0, blk, 32), (np.arange(32, dtype=np.float32) - 16) * np.float32(0.5))


def test_dequant_q6_k_closed_form(orc):
    # The GGUF Q6_K super-block spelled out by hand: weight e = 128 n + 32 m + l
    # takes its low 4 bits from ql[64 n + 32 (m & 1) + l] (low nibble for m < 2,
    # high for m >= 2) and its high 2 bits from qh[32 n + l] >> 2m; value =
    # d * sc[e / 16] * (q - 32). ql: n=0 bytes 0..31 = 0x21, 32..63 = 0x65; n=1
    # 0x43, 0x87 -> low bits by (n, m): [1, 5, 2, 6], [3, 7, 4, 8]. qh: n=0 0xE4
    # (high bits m), n=1 0x1B (3 - m). sc[i] = i - 8, d = 0.25.
    blk = np.zeros(210, dtype=np.uint8)
    blk[0:32], blk[32:64], blk[64:96], blk[96:128] = 0x21, 0x65, 0x43, 0x87
    blk[128:160], blk[160:192] = 0xE4, 0x1B
    blk[192:208] = (np.arange(16) - 8).astype(np.int8).view(np.uint8)
    blk[208:210] = np.array([0.25], dtype=np.float16).view(np.uint8)
    low = [[1, 5, 2, 6], [3, 7, 4, 8]]
    want = np.zeros(256, dtype=np.float32)
    for e in range(256):
        n, m = e // 128, (e // 32) % 4
        q = low[n][m] | ((m if n == 0 else 3 - m) << 4)
        want[e] = np.float32(0.25) * np.float32(e // 16 - 8) * np.float32(q - 32)
    assert np.array_equal(orc.dequant(GGML_Q6_K, blk, 256), want)


def test_q6_k_half_dots_closed_form(orc):
    # One sub-block of all-equal q against activations a_j = 1: each half dot
    # is 16 (q - 32), whatever the packing. q = 0 (-> -512), 63 (-> 496), 32 (-> 0).
    for qv, want in ((0, -512), (63, 496), (32, 0)):
        blk = np.zeros(210, dtype=np.uint8)
        lo, hi = qv & 15, qv >> 4
        blk[0:128] = lo | (lo << 4)
        blk[128:192] = hi | (hi << 2) | (hi << 4) | (hi << 6)
        x = np.ones(256, dtype=np.float32)
        xq = orc.quant_q8(x)  # d = 1/127, q = 127
        qw, _ = orc.repack(GGML_Q6_K, blk, 1, 8)
        dots = orc.block_dots(GGML_Q6_K, qw, 1, 8, xq)
        assert np.all(dots == want * 127), (qv, dots)


def test_f16_to_f32_all_halves(orc):
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = h.view(np.float16).astype(np.float32)
    got = np.array([orc.f16_to_f32(int(v)) for v in h], dtype=np.float32)
    fin = np.isfinite(want)
    assert np.array_equal(got[fin].view(np.uint32), want[fin].view(np.uint32))
    assert np.all(np.isnan(got[np.isnan(want)]))


def test_f32_to_f16_rne(orc):
    g = np.random.default_rng(3)
    vals = np.concatenate([g.standard_normal(3000).astype(np.float32) * 0.02,
                           np.float32(2.0) ** g.integers(-26, 17, 2000).astype(np.float32) * g.uniform(1, 2, 2000).astype(np.float32),
                           np.array([0.0, -0.0, 65504.0, 65519.0, 65520.0, 1e-8, 2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -26], dtype=np.float32)])
    with np.errstate(over="ignore"):  # 65520 and the largest values round to inf, as they should
        want = vals.astype(np.float16).view(np.uint16)
    got = np.array([orc.f32_to_f16(float(v)) for v in vals], dtype=np.uint16)
    assert np.array_equal(got, want)


def test_quant_q8_invariants(orc):
    x = synth.activations(1, 32 * 64, seed=4)[0] * 3
    x[0:32] = 0
    x[32:64] = 0
    x[40] = -2.5
    q = orc.quant_q8(x)
    nb = 64
    qv = q[:32 * nb].view(np.int8).reshape(nb, 32).astype(np.int64)
    d = q[32 * nb:36 * nb].view(np.float32)
    asum = q[36 * nb:].view(np.uint32)
    assert np.array_equal((qv.sum(1) % 2 ** 32).astype(np.uint32), asum)
    assert d[0] == 0 and not qv[0].any()
    assert qv[1, 8] == -127 and np.count_nonzero(qv[1]) == 1
    assert np.abs(qv).max() <= 127 and np.all(np.abs(qv[2:]).max(1) == 127)
