"""The GGUF reader and matrix load of libamdc_q4.so (include/amdc_gguf.h),
which replace the reference's src/gguf.c and the load_mat_src / gpu_sink pair
(src/model.c:401-494, src/hip.c:274-309) for this path.

CPU: files written by tests/gguf_writer.py (the GGUF v3 layout) read back key
by key and tensor by tensor; every truncation of a file, a bad magic, version,
alignment, value type, dimension count, a misaligned or out-of-file tensor are
refused with an error code (the reference exits the process instead); the
host repack of a tensor equals amdc.repack of its bytes at any thread count.
GPU: the streaming load (pinned double buffer, chunks of rows) puts the same
bytes on the device, and a GEMV over it matches the oracle."""
import os
import struct

import numpy as np
import pytest

import amdc
import gguf_writer as gw
from amdc import synth

KINDS = [(synth.KIND_Q4_0, 2, 37, 96), (synth.KIND_Q8_0, 8, 21, 160), (synth.KIND_Q4_K, 12, 19, 512), (synth.KIND_Q6_K, 14, 13, 256)]


def sample_file(tmp_path, alignment=32):
    kvs = [("general.architecture", gw.STR, "llama"), ("general.alignment", gw.U32, alignment),
           ("u8", gw.U8, 200), ("i8", gw.I8, -100), ("u16", gw.U16, 60000), ("i16", gw.I16, -30000),
           ("u32", gw.U32, 4000000000), ("i32", gw.I32, -2000000000), ("f32", gw.F32, 1.5), ("bool", gw.BOOL, 1),
           ("u64", gw.U64, 2 ** 63 + 5), ("i64", gw.I64, -(2 ** 62)), ("f64", gw.F64, -2.25), ("empty", gw.STR, ""),
           ("ints", gw.ARR, (gw.I32, [1, -2, 3])), ("toks", gw.ARR, (gw.STR, ["a", "", "hello"])),
           ("nested", gw.ARR, (gw.ARR, [(gw.U8, [1, 2]), (gw.STR, ["x"])]))]
    tensors, srcs = [], {}
    for kind, gt, rows, cols in KINDS:
        src = synth.gguf(kind, rows, cols, seed=rows + cols)
        name = f"blk.0.{gt}.weight"
        tensors.append((name, gt, (cols, rows), src.tobytes()))
        srcs[name] = (kind, rows, cols, src)
    f32 = np.arange(24, dtype=np.float32)
    tensors.append(("norm.weight", 0, (24,), f32.tobytes()))
    tensors.append(("cube", 2, (32, 2, 2), bytes(4 * 18)))
    path = os.path.join(tmp_path, "m.gguf")
    b = gw.write(path, kvs, tensors, alignment=alignment)
    return path, b, srcs, f32


@pytest.mark.parametrize("alignment", [32, 64, 1024])
def test_read_back_keys_and_tensors(tmp_path, alignment):
    path, b, srcs, f32 = sample_file(tmp_path, alignment)
    with amdc.Gguf(path) as g:
        assert g.version == 3 and g.alignment == alignment and g.data_offset % alignment == 0
        assert [k for k, _ in g.keys()][:3] == ["general.architecture", "general.alignment", "u8"]
        assert g.get_str("general.architecture") == "llama" and g.get_str("empty") == ""
        assert g.get_int("u8") == 200 and g.get_int("i8") == -100 and g.get_int("u16") == 60000
        assert g.get_int("i16") == -30000 and g.get_int("u32") == 4000000000 and g.get_int("i32") == -2000000000
        assert g.get_int("bool") == 1 and g.get_int("i64") == -(2 ** 62)
        assert g.get_int("u64") == (2 ** 63 + 5) - 2 ** 64  # int64 view of the u64 (as the reference's gguf_get_int)
        assert g.get_float("f32") == 1.5 and g.get_float("f64") == -2.25 and g.get_float("i32") == -2e9
        assert g.get_int("f32") is None and g.get_str("u8") is None and g.get_int("missing") is None
        t, n, arr = g.get_arr("ints")
        assert t == gw.I32 and n == 3 and list(arr) == [1, -2, 3]
        t, n, arr = g.get_arr("toks")
        assert t == gw.STR and n == 3 and arr is None
        assert [g.get_arr_str("toks", i) for i in range(3)] == ["a", "", "hello"] and g.get_arr_str("toks", 3) is None
        assert g.get_arr("nested")[:2] == (gw.ARR, 2)
        ts = g.tensors()
        assert len(ts) == len(srcs) + 2
        for t in ts[:len(srcs)]:
            kind, rows, cols, src = srcs[t.name.decode()]
            assert t.n_dims == 2 and list(t.ne) == [cols, rows, 1, 1] and t.type == synth.GGML[kind]
            assert t.nbytes == src.size and t.offset % alignment == 0
            assert np.array_equal(np.frombuffer(bytes((b[g.data_offset + t.offset:g.data_offset + t.offset + t.nbytes])), np.uint8), src)
        nt = ts[len(srcs)]
        assert nt.name == b"norm.weight" and nt.type == 0 and nt.nbytes == 96
        assert g.find("norm.weight") == len(srcs) and g.find("nope") == -1


@pytest.mark.parametrize("threads", [1, 3, 16, 0])
def test_repack_equals_amdc_repack(tmp_path, threads):
    path, _, srcs, _ = sample_file(tmp_path)
    with amdc.Gguf(path) as g:
        for name, (kind, rows, cols, src) in srcs.items():
            m, dst = g.repack(name, threads)
            assert (m.kind, m.rows, m.cols, m.nb) == (kind, rows, cols, cols // 32)
            assert np.array_equal(dst, amdc.repack(kind, src, rows, cols)), name


def test_mat_info_refuses_other_tensors(tmp_path):
    path, _, _, _ = sample_file(tmp_path)
    with amdc.Gguf(path) as g:
        for name in ("norm.weight", "cube", "missing"):
            with pytest.raises(amdc.AmdcError):
                g.mat_info(name)
    assert [amdc.lib().amdc_gguf_mat_kind(t) for t in (0, 1, 2, 8, 12, 13, 14, 23)] == [-1, -1, 0, 2, 3, -1, 4, -1]
    assert amdc.lib().amdc_ggml_nbytes(12, 256) == 144 and amdc.lib().amdc_ggml_nbytes(12, 255) == 0
    assert amdc.lib().amdc_ggml_nbytes(14, 512) == 420 and amdc.lib().amdc_ggml_nbytes(99, 32) == 0


def small_file():
    kvs = [("a", gw.STR, "xyz"), ("arr", gw.ARR, (gw.STR, ["p", "q"])), ("n", gw.U32, 7)]
    src = synth.gguf(synth.KIND_Q4_0, 2, 64, seed=1)
    return gw.gguf_bytes(kvs, [("w", 2, (64, 2), src.tobytes())])


def opens(tmp_path, data, name="x.gguf"):
    p = os.path.join(tmp_path, name)
    with open(p, "wb") as f:
        f.write(data)
    try:
        amdc.Gguf(p).close()
        return True
    except amdc.AmdcError:
        return False


def test_every_truncation_refused(tmp_path):
    """Every prefix that cuts the header or the tensor data is refused; the padding after the last
    tensor is not needed."""
    b = small_file()
    assert opens(tmp_path, b)
    p = os.path.join(tmp_path, "x.gguf")
    with amdc.Gguf(p) as g:
        t = g.tensors()[0]
        end = g.data_offset + t.offset + t.nbytes
    assert end < len(b)
    for n in range(len(b)):
        assert opens(tmp_path, b[:n]) == (n >= end), n


def test_malformed_files_refused(tmp_path):
    src = synth.gguf(synth.KIND_Q4_0, 2, 64, seed=1).tobytes()
    t = [("w", 2, (64, 2), src)]
    assert not opens(tmp_path, gw.gguf_bytes([], t, magic=b"GGUX"))
    assert not opens(tmp_path, gw.gguf_bytes([], t, version=2))
    assert not opens(tmp_path, gw.gguf_bytes([("general.alignment", gw.U32, 48)], t, alignment=48))  # not a power of two
    assert not opens(tmp_path, gw.gguf_bytes([], t, offsets=[16]))  # misaligned tensor
    assert not opens(tmp_path, gw.gguf_bytes([], [("w", 2, (64, 4), src)]))  # 4 rows of data for 2: outside the file
    good = gw.gguf_bytes([("k", gw.U8, 1)], t)
    assert opens(tmp_path, good)
    bad_type = bytearray(good)
    ktype_at = 4 + 4 + 8 + 8 + 8 + 1  # after magic, version, counts, key length and "k"
    bad_type[ktype_at:ktype_at + 4] = struct.pack("<I", 13)
    assert not opens(tmp_path, bytes(bad_type))
    dims5 = gw.gguf_bytes([], [("w", 2, (32, 1, 1, 1, 2), src)])
    assert not opens(tmp_path, dims5)
    huge = bytearray(good)
    huge[8:16] = struct.pack("<Q", 2 ** 60)  # tensor count
    assert not opens(tmp_path, bytes(huge))
    assert not opens(tmp_path, b"")
    with pytest.raises(amdc.AmdcError):
        amdc.Gguf(os.path.join(tmp_path, "does-not-exist.gguf"))


@pytest.mark.gpu
@pytest.mark.parametrize("chunk_kb", [0, 1, 64])
def test_load_to_device(dev, orc, tmp_path, chunk_kb, monkeypatch):
    """The streaming load: the device holds the repacked bytes (several chunks of rows when the chunk
    is small: 1 KiB = a few rows per chunk), and a GEMV over the loaded matrix matches the oracle."""
    if chunk_kb:
        monkeypatch.setenv("AMDC_LOAD_CHUNK_KB", str(chunk_kb))
    path, _, srcs, _ = sample_file(tmp_path)
    with amdc.Gguf(path) as g:
        for name, (kind, rows, cols, src) in srcs.items():
            M = g.load(name, threads=2)
            assert np.array_equal(M.download(), amdc.repack(kind, src, rows, cols)), name
            nb = cols // 32
            x = synth.activations(1, cols, seed=rows)[0]
            X, Q, Y = dev.DevBuf.of(x), dev.DevBuf((40 * nb + 255) // 256 * 256), dev.DevBuf(4 * rows)
            dev.quant_q8(X, Q, nb)
            dev.gemv(kind, M, Q, Y, rows, nb)
            xq = orc.quant_q8(x)
            qw, qs = orc.repack(synth.GGML[kind], src, rows, nb)
            want = orc.gemv(synth.GGML[kind], qw, qs, rows, nb, xq)
            mag = orc.gemv_f64(synth.GGML[kind], src, rows, nb, xq)[1]
            assert float((np.abs(Y.download(np.float32) - want) / np.maximum(mag, 1e-30)).max()) < 1e-5
            M.free()


def test_mutated_files_never_crash(tmp_path):
    """Random byte, bit, length and 8-byte-field mutations of a small file with every kind of tensor:
    each open either fails with an error or yields a file whose tensors repack (the library also ran
    clean under AddressSanitizer and UBSan on 20000 such mutations, host-only build)."""
    kvs = [("a", gw.STR, "xyz"), ("arr", gw.ARR, (gw.STR, ["p", "q"])), ("n", gw.U32, 7), ("nest", gw.ARR, (gw.ARR, [(gw.U8, [1, 2])]))]
    t = [("w", 2, (64, 2), synth.gguf(0, 2, 64, 1).tobytes()), ("k", 12, (256, 2), synth.gguf(3, 2, 256, 2).tobytes()),
         ("s", 14, (256, 1), synth.gguf(4, 1, 256, 3).tobytes()), ("q", 8, (64, 1), synth.gguf(2, 1, 64, 4).tobytes())]
    base = gw.gguf_bytes(kvs, t)
    rng = np.random.default_rng(7)
    p = os.path.join(tmp_path, "m.gguf")
    opened = 0
    for _ in range(1500):
        m = bytearray(base)
        for _ in range(int(rng.integers(1, 5))):
            k, pos = int(rng.integers(0, 4)), int(rng.integers(0, len(m)))
            if k == 0:
                m[pos] = int(rng.integers(0, 256))
            elif k == 1:
                m[pos] ^= 1 << int(rng.integers(0, 8))
            elif k == 2:
                del m[int(rng.integers(0, len(m))):]
            elif len(m) > 8:
                q = int(rng.integers(0, len(m) - 8))
                m[q:q + 8] = struct.pack("<Q", int(rng.integers(0, 2 ** 40)) << int(rng.integers(0, 24)))
            if not m:
                break
        with open(p, "wb") as f:
            f.write(bytes(m))
        try:
            g = amdc.Gguf(p)
        except amdc.AmdcError:
            continue
        opened += 1
        for tt in g.tensors():
            try:
                g.repack(tt.name, 2)
            except amdc.AmdcError:
                pass
        for k, ty in g.keys():
            g.get_int(k), g.get_float(k), g.get_str(k), g.get_arr(k)
            if ty == gw.ARR:
                g.get_arr_str(k, 0)
        g.close()
    assert opened > 100
