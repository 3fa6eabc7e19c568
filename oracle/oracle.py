"""TEST INFRASTRUCTURE ONLY: ctypes access to the CPU checkers.

- ``liboracle.so``: the C restatement of the reference's CPU path
  (``amdc_oracle.c``: hanw/amd.c src/cpu.c:36-118, src/model.c:205-267).
- ``_ref/libref_cpu.so``: the reference's own src/{common,gguf,model,plan,cpu}.c
  compiled where they lie (``Makefile``), present only where /root/reference
  was (it travels with the tree as a built file).

Only tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg use
this module: it checks the HIP path and is never the thing measured or shipped.
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
GGML_Q4_0, GGML_Q8_0, GGML_Q4_K, GGML_Q6_K = 2, 8, 12, 14
# words of qw per 32-weight block in the reference layouts
_QW_PER = {GGML_Q4_0: 4, GGML_Q8_0: 8, GGML_Q4_K: 4, GGML_Q6_K: 6}


def qs_len(kind, rows, nb):
    """u16 entries of qs in the reference layouts (src/model.c:356-362)."""
    extra = {GGML_Q4_K: rows * (nb // 8) * 2, GGML_Q6_K: rows * (nb // 8)}.get(kind, 0)
    return rows * nb + extra

_P = C.c_void_p
_U32 = C.c_uint32


def _ptr(a):
    return a.ctypes.data_as(_P)


class Oracle:
    def __init__(self, path=None):
        path = path or os.path.join(HERE, "liboracle.so")
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} is not built (make -C oracle)")
        L = self.lib = C.CDLL(path)
        L.or_f16_to_f32.restype = C.c_float
        L.or_f16_to_f32.argtypes = [C.c_uint16]
        L.or_f32_to_f16.restype = C.c_uint16
        L.or_f32_to_f16.argtypes = [C.c_float]
        L.or_quant_q8.argtypes = [_P, _P, _U32]
        for f in (L.or_repack_q4, L.or_repack_q4k, L.or_repack_q8, L.or_repack_q6k):
            f.argtypes = [_P, _U32, _U32, _P, _P]
        for f in (L.or_gemv_q4, L.or_gemv_q4k, L.or_gemv_q8, L.or_gemv_q6k):
            f.argtypes = [_P, _P, _U32, _U32, _P, _P]
        for f in (L.or_gemv_q4_mt, L.or_gemv_q4k_mt, L.or_gemv_q8_mt, L.or_gemv_q6k_mt):
            f.argtypes = [_P, _P, _U32, _U32, _P, _P, C.c_int]
        L.or_epilogue.argtypes = [_P, _U32, _P, _P]
        for f in (L.or_block_dots_q4, L.or_block_dots_q4k, L.or_block_dots_q8, L.or_block_dots_q6k):
            f.argtypes = [_P, _U32, _U32, _P, _P]
        L.or_block_dots_gguf.argtypes = [C.c_int, _P, _U32, _U32, _P, _P]
        L.or_dequant.argtypes = [C.c_int, _P, C.c_uint64, C.c_uint64, _P]
        L.or_dequant_mt.argtypes = [C.c_int, _P, C.c_uint64, _P, C.c_int]
        L.or_gemv_f64.argtypes = [C.c_int, _P, _U32, _U32, _P, _P, _P]
        L.or_q4k_qs_n.restype = C.c_size_t
        L.or_q4k_qs_n.argtypes = [_U32, _U32]
        L.or_rmsnorm.argtypes = [_P, _P, _P, _U32, C.c_float]
        L.or_swiglu.argtypes = [_P, _P, _U32]

    # -- Q8
    def quant_q8(self, x):
        """x: float32 [..., 32 nb] -> uint8 [..., 40 nb] Q8 buffers (src/cpu.c:36-53)."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        n = x.shape[-1]
        assert n % 32 == 0
        nb = n // 32
        flat = x.reshape(-1, n)
        out = np.zeros((flat.shape[0], 40 * nb), dtype=np.uint8)
        for i in range(flat.shape[0]):
            self.lib.or_quant_q8(_ptr(flat[i]), _ptr(out[i]), nb)
        return out.reshape(x.shape[:-1] + (40 * nb,))

    # -- the producers of Q8 vectors (float part; their Q8 copy is quant_q8 of the result)
    def rmsnorm(self, x, w, eps):
        """y = x s w per row of x (src/cpu.c:276-281)."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        w = np.ascontiguousarray(w, dtype=np.float32)
        flat = x.reshape(-1, x.shape[-1])
        out = np.empty_like(flat)
        for i in range(flat.shape[0]):
            self.lib.or_rmsnorm(_ptr(flat[i]), _ptr(w), _ptr(out[i]), flat.shape[1], C.c_float(eps))
        return out.reshape(x.shape)

    def swiglu(self, a, b):
        """a / (1 + expf(-a)) * b per element (src/cpu.c:580)."""
        a = np.array(a, dtype=np.float32, copy=True)
        b = np.ascontiguousarray(b, dtype=np.float32)
        self.lib.or_swiglu(_ptr(a), _ptr(b), a.size)
        return a

    # -- repack to the reference layouts
    _SUF = {GGML_Q4_0: "q4", GGML_Q8_0: "q8", GGML_Q4_K: "q4k", GGML_Q6_K: "q6k"}

    def _fn(self, stem, kind):
        return getattr(self.lib, f"or_{stem}_{self._SUF[kind]}")

    def repack(self, kind, src, rows, nb):
        """GGUF bytes -> the reference's (qw, qs) (src/model.c:205-292)."""
        src = np.ascontiguousarray(src, dtype=np.uint8)
        qw = np.zeros(rows * nb * _QW_PER[kind], dtype=np.uint32)
        qs = np.zeros(qs_len(kind, rows, nb), dtype=np.uint16)
        self._fn("repack", kind)(_ptr(src), rows, nb, _ptr(qw), _ptr(qs))
        return qw, qs

    def gemv(self, kind, qw, qs, rows, nb, xq, threads=1):
        """y = W x in the reference's order, bit for bit (src/cpu.c:64-175)."""
        xq = np.ascontiguousarray(xq, dtype=np.uint8)
        y = np.zeros(rows, dtype=np.float32)
        if threads > 1:
            getattr(self.lib, f"or_gemv_{self._SUF[kind]}_mt")(_ptr(qw), _ptr(qs), rows, nb, _ptr(xq), _ptr(y), threads)
        else:
            self._fn("gemv", kind)(_ptr(qw), _ptr(qs), rows, nb, _ptr(xq), _ptr(y))
        return y

    def epilogue(self, y, bias=None, res=None):
        y = np.array(y, dtype=np.float32)
        b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
        r = None if res is None else np.ascontiguousarray(res, dtype=np.float32)
        self.lib.or_epilogue(_ptr(y), y.size, _ptr(b) if b is not None else None, _ptr(r) if r is not None else None)
        return y

    def block_dots(self, kind, qw, rows, nb, xq):
        """int32 [rows, nb] block dots; Q6_K: [rows, nb, 2] half dots."""
        h = 2 if kind == GGML_Q6_K else 1
        out = np.zeros(rows * nb * h, dtype=np.int32)
        self._fn("block_dots", kind)(_ptr(qw), rows, nb, _ptr(np.ascontiguousarray(xq)), _ptr(out))
        return out.reshape((rows, nb, 2) if h == 2 else (rows, nb))

    def block_dots_gguf(self, kind, src, rows, nb, xq):
        h = 2 if kind == GGML_Q6_K else 1
        out = np.zeros(rows * nb * h, dtype=np.int32)
        self.lib.or_block_dots_gguf(kind, _ptr(np.ascontiguousarray(src)), rows, nb, _ptr(np.ascontiguousarray(xq)), _ptr(out))
        return out.reshape((rows, nb, 2) if h == 2 else (rows, nb))

    def dequant(self, kind, src, n, threads=1):
        out = np.zeros(n, dtype=np.float32)
        if threads > 1:
            self.lib.or_dequant_mt(kind, _ptr(np.ascontiguousarray(src)), n, _ptr(out), threads)
        else:
            self.lib.or_dequant(kind, _ptr(np.ascontiguousarray(src)), 0, n, _ptr(out))
        return out

    def gemv_f64(self, kind, src, rows, nb, xq):
        """(y_ref float64, sum |terms| per row) from the GGUF bytes (tests/kernel_test.c:59-80)."""
        y = np.zeros(rows, dtype=np.float64)
        m = np.zeros(rows, dtype=np.float64)
        self.lib.or_gemv_f64(kind, _ptr(np.ascontiguousarray(src)), rows, nb, _ptr(np.ascontiguousarray(xq)), _ptr(y), _ptr(m))
        return y, m

    def f16_to_f32(self, h):
        return self.lib.or_f16_to_f32(int(h))

    def f32_to_f16(self, f):
        return self.lib.or_f32_to_f16(float(f))


class RefCPU:
    """The reference's own cpu.c / model.c (oracle/_ref/libref_cpu.so)."""

    def __init__(self, path=None):
        path = path or os.path.join(HERE, "_ref", "libref_cpu.so")
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} is not built (make -C oracle ref, needs /root/reference)")
        L = self.lib = C.CDLL(path)
        L.ref_quant_q8.argtypes = [_P, _P, _U32]
        L.ref_mat_new.restype = _P
        L.ref_mat_new.argtypes = [C.c_int, _P, _U32, _U32]
        L.ref_mat_kind.argtypes = [_P]
        L.ref_mat_copy.argtypes = [_P, _P, _P]
        L.ref_mat_gemv.argtypes = [_P, _P, _P]
        L.ref_mat_free.argtypes = [_P]

    @staticmethod
    def available(path=None):
        return os.path.exists(path or os.path.join(HERE, "_ref", "libref_cpu.so"))

    def quant_q8(self, x):
        x = np.ascontiguousarray(x, dtype=np.float32)
        nb = x.shape[-1] // 32
        flat = x.reshape(-1, x.shape[-1])
        out = np.zeros((flat.shape[0], 40 * nb), dtype=np.uint8)
        for i in range(flat.shape[0]):
            self.lib.ref_quant_q8(_ptr(flat[i]), _ptr(out[i]), nb)
        return out.reshape(x.shape[:-1] + (40 * nb,))

    def mat(self, ttype, src, rows, cols):
        src = np.ascontiguousarray(src, dtype=np.uint8)
        h = self.lib.ref_mat_new(ttype, _ptr(src), rows, cols)
        if not h:
            raise ValueError("not a MAT_Q4 / MAT_Q8 / MAT_Q4K / MAT_Q6K matrix")
        return RefMat(self, h, ttype, rows, cols // 32)


class RefMat:
    def __init__(self, ref, h, ttype, rows, nb):
        self.ref, self.h, self.ttype, self.rows, self.nb = ref, h, ttype, rows, nb

    def arrays(self):
        qw = np.zeros(self.rows * self.nb * _QW_PER[self.ttype], dtype=np.uint32)
        qs = np.zeros(qs_len(self.ttype, self.rows, self.nb), dtype=np.uint16)
        self.ref.lib.ref_mat_copy(self.h, _ptr(qw), _ptr(qs))
        return qw, qs

    def gemv(self, xq, y=None):
        y = np.zeros(self.rows, dtype=np.float32) if y is None else y
        self.ref.lib.ref_mat_gemv(self.h, _ptr(np.ascontiguousarray(xq)), _ptr(y))
        return y

    def free(self):
        if self.h:
            self.ref.lib.ref_mat_free(self.h)
            self.h = None

    def __del__(self):
        self.free()
