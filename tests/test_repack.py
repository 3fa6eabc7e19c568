"""The load-time repack into the CDNA4 layout (amd.c_amd/csrc/amdc_layout.h),
checked on the CPU against the reference's own repacked arrays (golden
fixtures: repack_q4 / repack_q4k of src/model.c) and the GGUF bytes:

- nibble bytes: bit for bit (every nibble of every block, via the layout's
  inverse map, equals the reference's MAT_Q4 / MAT_Q4K word bytes);
- scales: the f16 d of Q4_0, and Q4_K's f16 d, dmin and 6-bit sc / mn equal the
  reference's qs entries;
- the nibble map is a bijection onto the panel; padding blocks are zero;
- Q8_0 and Q6_K (repack_q8 / repack_q6k of src/model.c:221-292): the int8
  words, the Q6_K nibble and high-bit words, scales and d equal the
  reference's MAT_Q8 / MAT_Q6K arrays through the layout's inverse maps, and
  every map covers its panel exactly once.
"""
import glob
import os

import numpy as np
import pytest

import amdc
from amdc import synth
from oracle import GGML_Q4_0, GGML_Q4_K

GOLDEN_ALL = sorted(glob.glob(os.path.join(os.path.dirname(__file__), "golden", "golden_*.npz")))
GOLDEN = [p for p in GOLDEN_ALL if "_q4_" in os.path.basename(p)]
GOLDEN_K8 = [p for p in GOLDEN_ALL if "_q8_0_" in os.path.basename(p) or "_q6_k_" in os.path.basename(p)]


def tile(ng, g):
    return g // 8, min(8, ng - 8 * (g // 8))


def q8_off(ng, g, p):
    t, gt = tile(ng, g)
    return 16 * ng + 2048 * t + 16 * (p * gt + g % 8)


def q6k_dpad(ng):
    return (2 * ng + 15) // 16 * 16


def q6k_nib_off(ng, g, k):
    t, gt = tile(ng, g)
    return 16 * ng + q6k_dpad(ng) + 1024 * t + 16 * (k * gt + g % 8)


def q6k_hi_off(ng, g, p):
    t, gt = tile(ng, g)
    return 144 * ng + q6k_dpad(ng) + 512 * t + 16 * (p * gt + g % 8)


def nib_off(ng, g, k):
    """byte offset of block (g, k) inside a row (the map of amdc_layout.h)."""
    t = g // 8
    gt = min(8, ng - 8 * t)
    return 16 * ng + 1024 * t + 16 * (k * gt + g % 8)


def decode(kind, packed, rows, nb):
    """CDNA4 layout -> (nibble bytes [rows, nb, 16], header bytes [rows, ng, 16])."""
    ng = (nb + 7) // 8
    rb = 144 * ng
    m = packed.reshape(rows, rb)
    nib = np.empty((rows, nb, 16), dtype=np.uint8)
    for b in range(nb):
        o = nib_off(ng, b // 8, b % 8)
        nib[:, b, :] = m[:, o:o + 16]
    return nib, m[:, :16 * ng].reshape(rows, ng, 16)


@pytest.mark.parametrize("path", GOLDEN, ids=[os.path.basename(p)[7:-4] for p in GOLDEN])
def test_repack_matches_reference_arrays(path):
    g = np.load(path)
    kind, rows, nb = int(g["kind"]), int(g["rows"]), int(g["nb"])
    packed = amdc.repack(kind, g["gguf"], rows, 32 * nb)
    assert packed.size == amdc.mat_bytes(kind, rows, 32 * nb) == rows * 144 * ((nb + 7) // 8)
    nib, hdr = decode(kind, packed, rows, nb)
    ref_words = g["qw"].reshape(rows, nb, 4)
    assert np.array_equal(nib.view(np.uint32).reshape(rows, nb, 4), ref_words), "nibble bytes differ from the reference repack"
    qs = g["qs"]
    if kind == synth.KIND_Q4_0:
        d = hdr.reshape(rows, -1).view(np.uint16)[:, :nb]
        assert np.array_equal(d.reshape(-1), qs)
        pad = hdr.reshape(rows, -1).view(np.uint16)[:, nb:]
        assert not pad.any()
    else:
        ng = nb // 8
        h32 = hdr.reshape(rows, ng, 4, 4).view(np.uint32).reshape(rows, ng, 4)
        dd = qs[rows * nb:].reshape(rows, ng, 2)
        assert np.array_equal((h32[:, :, 0] & 0xFFFF).astype(np.uint16), dd[:, :, 0])
        assert np.array_equal((h32[:, :, 0] >> 16).astype(np.uint16), dd[:, :, 1])
        f1 = h32[:, :, 1].astype(np.uint64) | (h32[:, :, 2].astype(np.uint64) << np.uint64(32))
        f2 = h32[:, :, 2].astype(np.uint64) | (h32[:, :, 3].astype(np.uint64) << np.uint64(32))
        sm = qs[:rows * nb].reshape(rows, ng, 8)
        for k in range(8):
            sc = (f1 >> np.uint64(6 * k)) & np.uint64(63)
            mn = (f2 >> np.uint64(16 + 6 * k)) & np.uint64(63)
            assert np.array_equal(sc.astype(np.uint16), sm[:, :, k] & 63), k
            assert np.array_equal(mn.astype(np.uint16), sm[:, :, k] >> 8), k


@pytest.mark.parametrize("nb", [1, 7, 8, 9, 63, 64, 65, 128, 344, 511, 544])
def test_nibble_map_bijection(nb):
    ng = (nb + 7) // 8
    offs = sorted(nib_off(ng, g, k) for g in range(ng) for k in range(8))
    assert offs == list(range(16 * ng, 144 * ng, 16))


def test_padding_blocks_zero():
    rows, nb = 3, 13
    src = synth.gguf(0, rows, 32 * nb, seed=2)
    packed = amdc.repack(0, src, rows, 32 * nb).reshape(rows, -1)
    ng = 2
    for b in range(nb, 16):
        o = nib_off(ng, b // 8, b % 8)
        assert not packed[:, o:o + 16].any()


def test_repack_rejects_bad_shapes():
    with pytest.raises(amdc.AmdcError):
        amdc.repack(3, np.zeros(144, np.uint8), 1, 128)  # Q4_K needs cols % 256 == 0
    with pytest.raises(amdc.AmdcError):
        amdc.mat_bytes(0, 1, 33)


@pytest.mark.parametrize("path", GOLDEN_K8, ids=[os.path.basename(p)[7:-4] for p in GOLDEN_K8])
def test_repack_k8_matches_reference_arrays(path):
    g = np.load(path)
    kind, rows, nb = int(g["kind"]), int(g["rows"]), int(g["nb"])
    ng = (nb + 7) // 8
    packed = amdc.repack(kind, g["gguf"], rows, 32 * nb)
    qw, qs = g["qw"], g["qs"]
    if kind == synth.KIND_Q8_0:
        rb = 272 * ng
        assert packed.size == amdc.mat_bytes(kind, rows, 32 * nb) == rows * rb
        m = packed.reshape(rows, rb)
        words = np.empty((rows, nb, 32), dtype=np.uint8)
        for b in range(nb):
            words[:, b, :16] = m[:, q8_off(ng, b // 8, 2 * (b % 8)):][:, :16]
            words[:, b, 16:] = m[:, q8_off(ng, b // 8, 2 * (b % 8) + 1):][:, :16]
        assert np.array_equal(words.view(np.uint32).reshape(-1), qw), "int8 words differ from the reference repack"
        d = m[:, :16 * ng].view(np.uint16)
        assert np.array_equal(d[:, :nb].reshape(-1), qs)
        assert not d[:, nb:].any()
        for b in range(nb, 8 * ng):  # padding blocks: zero weights
            for h in range(2):
                o = q8_off(ng, b // 8, 2 * (b % 8) + h)
                assert not m[:, o:o + 16].any(), b
    else:
        rb = 208 * ng + q6k_dpad(ng)
        assert packed.size == amdc.mat_bytes(kind, rows, 32 * nb) == rows * rb
        m = packed.reshape(rows, rb)
        nib = np.empty((rows, nb, 16), dtype=np.uint8)
        hw = np.empty((rows, nb, 8), dtype=np.uint8)
        for b in range(nb):
            gg, k = b // 8, b % 8
            nib[:, b] = m[:, q6k_nib_off(ng, gg, k):][:, :16]
            hw[:, b] = m[:, q6k_hi_off(ng, gg, k // 2) + 8 * (k % 2):][:, :8]
        assert np.array_equal(nib.view(np.uint32).reshape(-1), qw[:rows * nb * 4]), "low bits differ"
        assert np.array_equal(hw.view(np.uint32).reshape(-1), qw[rows * nb * 4:]), "high-bit words differ"
        sc = m[:, :16 * ng].view(np.uint16).reshape(-1)  # (sc0 | sc1 << 8) per sub-block
        assert np.array_equal(sc, qs[:rows * nb])
        d = m[:, 16 * ng:16 * ng + 2 * ng].view(np.uint16).reshape(-1)
        assert np.array_equal(d, qs[rows * nb:])
        assert not m[:, 18 * ng:16 * ng + q6k_dpad(ng)].any()


@pytest.mark.parametrize("nb", [1, 7, 8, 9, 63, 64, 65, 128, 344, 511, 544])
def test_q8_map_bijection(nb):
    ng = (nb + 7) // 8
    offs = sorted(q8_off(ng, g, p) for g in range(ng) for p in range(16))
    assert offs == list(range(16 * ng, 272 * ng, 16))


@pytest.mark.parametrize("ng", [1, 2, 7, 8, 9, 20, 56, 68])
def test_q6k_maps_bijection(ng):
    D = q6k_dpad(ng)
    nibs = sorted(q6k_nib_off(ng, g, k) for g in range(ng) for k in range(8))
    assert nibs == list(range(16 * ng + D, 144 * ng + D, 16))
    his = sorted(q6k_hi_off(ng, g, p) for g in range(ng) for p in range(4))
    assert his == list(range(144 * ng + D, 208 * ng + D, 16))


def test_repack_k8_rejects_bad_shapes():
    with pytest.raises(amdc.AmdcError):
        amdc.repack(4, np.zeros(210, np.uint8), 1, 128)  # Q6_K needs cols % 256 == 0
    with pytest.raises(amdc.AmdcError):
        amdc.mat_bytes(2, 1, 48)
