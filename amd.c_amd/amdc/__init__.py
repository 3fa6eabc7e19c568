"""Python access to libamdc_q4.so, the MI355X quantized GEMV/GEMM path.

A thin ctypes mirror of include/amdc_q4.h for the test harness and bench.py:
the computation is in the HIP kernels (amdc_kernels.hsaco) that the C host
launches. There is no fallback: without the built library, or without a GPU,
every operator raises ``AmdcError``.

Names follow the reference's operators (hanw/amd.c src/backend.h:61-64,
src/hip.c:922-1026): ``quant_q8``, ``gemv_q4``, ``gemv_q4k``, the multi-vector
``gemv_q4_t`` / ``gemv_q4k_t``, the prefill ``gemm_q4k`` and the dispatcher
``op_gemv``; ``repack_q4`` / ``repack_q4k`` replace the load-time repack of
src/model.c:205-267. The Q8_0 and Q6_K kinds (``gemv_q8`` / ``gemv_q6k``,
``repack_q8`` / ``repack_q6k``) follow OP_GEMV_Q8 / OP_GEMV_Q6K
(src/hip.c:934-962, 1027-1089) and src/model.c:221-292.
"""
import ctypes as C
import os

import numpy as np

PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(PKG_DIR, "libamdc_q4.so")
HSACO_PATH = os.path.join(PKG_DIR, "amdc_kernels.hsaco")

KIND_Q4_0, KIND_Q8_0, KIND_Q4_K, KIND_Q6_K = 0, 2, 3, 4
_SUF = {KIND_Q4_0: "q4", KIND_Q8_0: "q8", KIND_Q4_K: "q4k", KIND_Q6_K: "q6k"}
_P, _U32 = C.c_void_p, C.c_uint32

_I64, _U64 = C.c_int64, C.c_uint64
_PP = C.POINTER(C.c_void_p)


class GgufTensor(C.Structure):
    """amdc_gguf_tensor (include/amdc_gguf.h)."""
    _fields_ = [("name", C.c_char_p), ("type", C.c_uint32), ("n_dims", C.c_uint32), ("ne", C.c_uint64 * 4),
                ("offset", C.c_uint64), ("nbytes", C.c_uint64), ("data", C.c_void_p)]


class Mat(C.Structure):
    """amdc_mat (include/amdc_gguf.h): a matrix in the CDNA4 layout."""
    _fields_ = [("kind", C.c_int), ("rows", C.c_uint32), ("cols", C.c_uint32), ("nb", C.c_uint32), ("bytes", C.c_uint64),
                ("w", C.c_void_p)]


# every function of include/amdc_q4.h and include/amdc_gguf.h: name -> (restype, argtypes)
ABI = {
    "amdc_gguf_open": (C.c_int, [C.c_char_p, _PP]),
    "amdc_gguf_close": (None, [_P]),
    "amdc_gguf_version": (C.c_uint32, [_P]),
    "amdc_gguf_alignment": (C.c_uint32, [_P]),
    "amdc_gguf_data_offset": (_U64, [_P]),
    "amdc_gguf_n_kv": (_U64, [_P]),
    "amdc_gguf_n_tensors": (_U64, [_P]),
    "amdc_gguf_key_at": (C.c_int, [_P, _U64, C.POINTER(C.c_char_p), C.POINTER(C.c_uint32)]),
    "amdc_gguf_get_int": (C.c_int, [_P, C.c_char_p, C.POINTER(_I64)]),
    "amdc_gguf_get_float": (C.c_int, [_P, C.c_char_p, C.POINTER(C.c_double)]),
    "amdc_gguf_get_str": (C.c_int, [_P, C.c_char_p, _PP, C.POINTER(_U64)]),
    "amdc_gguf_get_arr": (C.c_int, [_P, C.c_char_p, C.POINTER(C.c_uint32), C.POINTER(_U64), _PP]),
    "amdc_gguf_get_arr_str": (C.c_int, [_P, C.c_char_p, _U64, _PP, C.POINTER(_U64)]),
    "amdc_gguf_tensor_at": (C.c_int, [_P, _U64, C.POINTER(GgufTensor)]),
    "amdc_gguf_find_tensor": (_I64, [_P, C.c_char_p]),
    "amdc_ggml_nbytes": (_U64, [C.c_uint32, _U64]),
    "amdc_gguf_mat_kind": (C.c_int, [C.c_uint32]),
    "amdc_gguf_mat_info": (C.c_int, [_P, C.c_char_p, C.POINTER(Mat)]),
    "amdc_gguf_repack": (C.c_int, [_P, C.c_char_p, C.c_int, C.POINTER(Mat), _P]),
    "amdc_gguf_load": (C.c_int, [_P, C.c_char_p, C.c_int, C.POINTER(Mat), _P]),
    "amdc_mat_release": (C.c_int, [C.POINTER(Mat)]),
    "amdc_last_error": (C.c_char_p, []),
    "amdc_mat_bytes": (C.c_size_t, [C.c_int, _U32, _U32]),
    "amdc_repack_q4": (C.c_int, [_P, _U32, _U32, _P]),
    "amdc_repack_q4k": (C.c_int, [_P, _U32, _U32, _P]),
    "amdc_repack_q8": (C.c_int, [_P, _U32, _U32, _P]),
    "amdc_repack_q6k": (C.c_int, [_P, _U32, _U32, _P]),
    "amdc_open": (C.c_int, [C.c_char_p]),
    "amdc_close": (None, []),
    "amdc_cu_count": (C.c_int, []),
    "amdc_malloc": (C.c_int, [C.POINTER(_P), C.c_size_t]),
    "amdc_free": (C.c_int, [_P]),
    "amdc_memcpy_h2d": (C.c_int, [_P, _P, C.c_size_t]),
    "amdc_memcpy_d2h": (C.c_int, [_P, _P, C.c_size_t]),
    "amdc_memcpy_d2d": (C.c_int, [_P, _P, C.c_size_t]),
    "amdc_memset": (C.c_int, [_P, C.c_int, C.c_size_t]),
    "amdc_sync": (C.c_int, []),
    "amdc_event_create": (C.c_int, [C.POINTER(_P)]),
    "amdc_event_destroy": (C.c_int, [_P]),
    "amdc_event_record": (C.c_int, [_P, _P]),
    "amdc_event_elapsed_ms": (C.c_int, [C.POINTER(C.c_float), _P, _P]),
    "amdc_stream_create": (C.c_int, [C.POINTER(_P)]),
    "amdc_stream_destroy": (C.c_int, [_P]),
    "amdc_stream_sync": (C.c_int, [_P]),
    "amdc_stream_wait_event": (C.c_int, [_P, _P]),
    "amdc_graph_begin": (C.c_int, [_P]),
    "amdc_graph_end": (C.c_int, [_P, C.POINTER(_P)]),
    "amdc_graph_launch": (C.c_int, [_P, _P]),
    "amdc_graph_destroy": (C.c_int, [_P]),
    "amdc_quant_q8": (C.c_int, [_P, _P, _U32, _U32, _U32, _U32, _P]),
    "amdc_gemv_q4": (C.c_int, [_P, _P, _P, _U32, _U32, _P, _P, _P]),
    "amdc_gemv_q4k": (C.c_int, [_P, _P, _P, _U32, _U32, _P, _P, _P]),
    "amdc_gemm_q4": (C.c_int, [_P, _P, _P, _U32, _U32, _P, _P, _U32, _U32, _U32, _U32, _P]),
    "amdc_gemm_q8": (C.c_int, [_P, _P, _P, _U32, _U32, _P, _P, _U32, _U32, _U32, _U32, _P]),
    "amdc_gemm_q6k": (C.c_int, [_P, _P, _P, _U32, _U32, _P, _P, _U32, _U32, _U32, _U32, _P]),
    "amdc_gemv_q8": (C.c_int, [_P, _P, _P, _U32, _U32, _P, _P, _P]),
    "amdc_gemv_q6k": (C.c_int, [_P, _P, _P, _U32, _U32, _P, _P, _P]),
    "amdc_gemv_q8_x": (C.c_int, [_P, _P, _P, _U32, _U32, _P, _P, _P, _P]),
    "amdc_gemv_q6k_x": (C.c_int, [_P, _P, _P, _U32, _U32, _P, _P, _P, _P]),
    "amdc_gemv_q8_t": (C.c_int, [_P, _P, _P, _U32, _U32, _P, _P, _U32, _U32, _U32, _U32, _P]),
    "amdc_gemv_q6k_t": (C.c_int, [_P, _P, _P, _U32, _U32, _P, _P, _U32, _U32, _U32, _U32, _P]),
    "amdc_gemv_q4_x": (C.c_int, [_P, _P, _P, _U32, _U32, _P, _P, _P, _P]),
    "amdc_gemv_q4k_x": (C.c_int, [_P, _P, _P, _U32, _U32, _P, _P, _P, _P]),
    "amdc_gemv_q4_t": (C.c_int, [_P, _P, _P, _U32, _U32, _P, _P, _U32, _U32, _U32, _U32, _P]),
    "amdc_gemv_q4k_t": (C.c_int, [_P, _P, _P, _U32, _U32, _P, _P, _U32, _U32, _U32, _U32, _P]),
    "amdc_gemm_q4k": (C.c_int, [_P, _P, _P, _U32, _U32, _P, _P, _U32, _U32, _U32, _U32, _P]),
    "amdc_op_gemv": (C.c_int, [C.c_int, _P, _P, _P, _U32, _U32, _P, _P, _U32, _U32, _U32, _U32, _P]),
    "amdc_last_kernel": (C.c_char_p, []),
    "amdc_op_gemv_noalloc": (C.c_int, [C.c_int, _P, _P, _P, _U32, _U32, _P, _P, _U32, _U32, _U32, _U32, _P]),
    "amdc_block_dots": (C.c_int, [C.c_int, _P, _P, _P, _U32, _U32, _P]),
    "amdc_set_tuning": (C.c_int, [C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int]),
    "amdc_probe_read": (C.c_int, [_P, C.c_size_t, _P, _U32, _P]),
    "amdc_probe_copy": (C.c_int, [_P, _P, C.c_size_t, _U32, _P]),
    "amdc_rmsnorm_q8": (C.c_int, [_P, _P, _P, _U32, C.c_float, _P, _U32, _U32, _U32, _U32, _P]),
    "amdc_swiglu_q8": (C.c_int, [_P, _P, _U32, _P, _U32, _U32, _U32, _P]),
    "amdc_chain_create": (C.c_int, [_P, _U32, C.POINTER(_P)]),
    "amdc_chain_create_form": (C.c_int, [_P, _U32, C.c_int, C.POINTER(_P)]),
    "amdc_chain_trace": (C.c_int, [_P, _P]),
    "amdc_chain_trace_words": (_U32, [_P]),
    "amdc_chain_launch": (C.c_int, [_P, _P]),
    "amdc_chain_check": (C.c_int, [_P]),
    "amdc_chain_destroy": (C.c_int, [_P]),
    "amdc_gemv_norm": (C.c_int, [C.c_int, _P, _P, _P, _U32, _U32, _P, _P, _P, _P, _P, C.c_float, _P]),
    "amdc_chain_record_begin": (C.c_int, [_P]),
    "amdc_chain_record_end": (C.c_int, [_P, C.c_int, C.POINTER(_P)]),
}

CHAIN_QUANT, CHAIN_GEMV, CHAIN_GEMV_X, CHAIN_RMSNORM_Q8, CHAIN_SWIGLU_Q8 = 0, 1, 2, 3, 4


class ChainOp(C.Structure):
    """amdc_chain_op of include/amdc_q4.h."""
    _fields_ = [("type", C.c_int), ("kind", C.c_int), ("sync", C.c_int), ("rows", _U32), ("nb", _U32),
                ("w", _P), ("x", _P), ("q", _P), ("xq", _P), ("y", _P), ("bias", _P), ("res", _P), ("eps", C.c_float)]


class AmdcError(RuntimeError):
    pass


_lib = None


def lib():
    """The loaded libamdc_q4.so (raises if it is not built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise AmdcError(f"{LIB_PATH} is not built: run __graft_entry__.build() (make -C amd.c_amd)")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in ABI.items():
            f = getattr(L, name)
            f.restype, f.argtypes = res, args
        _lib = L
    return _lib


def _check(rc):
    if rc:
        raise AmdcError(lib().amdc_last_error().decode(errors="replace"))


_opened = False


def open_device(hsaco=None):
    """amdc_open: HIP runtime, device 0, the kernel code object."""
    global _opened
    if not _opened:
        _check(lib().amdc_open((hsaco or HSACO_PATH).encode()))
        _opened = True


def cu_count():
    return lib().amdc_cu_count()


def set_tuning(lanes=0, unroll=0, wgs=0, gemm_kernel=0, gemm_ksplit=0, form=0):
    _check(lib().amdc_set_tuning(lanes, unroll, wgs, gemm_kernel, gemm_ksplit, form))


def sync():
    _check(lib().amdc_sync())


class DevBuf:
    """A device allocation (hipMalloc through the library)."""

    def __init__(self, nbytes):
        open_device()
        p = _P()
        _check(lib().amdc_malloc(C.byref(p), max(int(nbytes), 1)))
        self.ptr, self.nbytes = p.value, int(nbytes)

    @classmethod
    def of(cls, a):
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        b.upload(a)
        return b

    def upload(self, a, offset=0):
        a = np.ascontiguousarray(a)
        assert offset + a.nbytes <= self.nbytes
        _check(lib().amdc_memcpy_h2d(self.ptr + offset, a.ctypes.data_as(_P), a.nbytes))

    def download(self, dtype, count=None, offset=0):
        dtype = np.dtype(dtype)
        count = (self.nbytes - offset) // dtype.itemsize if count is None else count
        out = np.empty(count, dtype=dtype)
        _check(lib().amdc_memcpy_d2h(out.ctypes.data_as(_P), self.ptr + offset, out.nbytes))
        return out

    def fill(self, v=0):
        _check(lib().amdc_memset(self.ptr, v, self.nbytes))

    def free(self):
        if self.ptr:
            _check(lib().amdc_free(self.ptr))
            self.ptr = None

    def __del__(self):
        try:
            if self.ptr and _lib is not None:
                _lib.amdc_free(self.ptr)
        except Exception:
            pass


def _p(x):
    if x is None:
        return None
    return x.ptr if isinstance(x, (DevBuf, DevMat)) else int(x)


class Event:
    def __init__(self):
        open_device()
        p = _P()
        _check(lib().amdc_event_create(C.byref(p)))
        self.ev = p.value

    def record(self, stream=None):
        _check(lib().amdc_event_record(self.ev, stream))

    def elapsed_ms(self, later):
        ms = C.c_float()
        _check(lib().amdc_event_elapsed_ms(C.byref(ms), self.ev, later.ev))
        return ms.value

    def __del__(self):
        try:
            if self.ev and _lib is not None:
                _lib.amdc_event_destroy(self.ev)
        except Exception:
            pass


class Stream:
    """A HIP stream (default priority)."""

    def __init__(self):
        open_device()
        p = _P()
        _check(lib().amdc_stream_create(C.byref(p)))
        self.s = p.value

    def sync(self):
        _check(lib().amdc_stream_sync(self.s))

    def wait(self, event):
        """Later work on this stream waits for `event` (an Event recorded on another stream)."""
        _check(lib().amdc_stream_wait_event(self.s, event.ev))

    def __del__(self):
        try:
            if self.s and _lib is not None:
                _lib.amdc_stream_destroy(self.s)
        except Exception:
            pass


class Graph:
    """The operators that fn(stream) launches on `stream`, captured once; launch() replays them."""

    def __init__(self, stream, fn):
        self.stream = stream
        _check(lib().amdc_graph_begin(stream.s))
        try:
            fn(stream.s)
        finally:
            p = _P()
            rc = lib().amdc_graph_end(stream.s, C.byref(p))
        _check(rc)
        self.exec = p.value

    def launch(self):
        _check(lib().amdc_graph_launch(self.exec, self.stream.s))

    def __del__(self):
        try:
            if self.exec and _lib is not None:
                _lib.amdc_graph_destroy(self.exec)
        except Exception:
            pass


# ---------------------------------------------------------------- load time (host)

def mat_bytes(kind, rows, cols):
    n = lib().amdc_mat_bytes(kind, rows, cols)
    if not n:
        raise AmdcError(f"kind {kind}: {rows}x{cols} is not a valid shape")
    return n


def repack(kind, gguf, rows, cols):
    """GGUF bytes -> the CDNA4 layout (host numpy uint8)."""
    src = np.ascontiguousarray(gguf, dtype=np.uint8)
    dst = np.empty(mat_bytes(kind, rows, cols), dtype=np.uint8)
    f = getattr(lib(), "amdc_repack_" + _SUF[kind])
    _check(f(src.ctypes.data_as(_P), rows, cols, dst.ctypes.data_as(_P)))
    return dst


def repack_q4(gguf, rows, cols):
    return repack(KIND_Q4_0, gguf, rows, cols)


def repack_q4k(gguf, rows, cols):
    return repack(KIND_Q4_K, gguf, rows, cols)


def repack_q8(gguf, rows, cols):
    return repack(KIND_Q8_0, gguf, rows, cols)


def repack_q6k(gguf, rows, cols):
    return repack(KIND_Q6_K, gguf, rows, cols)


# ---------------------------------------------------------------- operators (device pointers)

def quant_q8(x, q, nb, T=1, xs=0, qs=0, stream=None):
    _check(lib().amdc_quant_q8(_p(x), _p(q), nb, T, xs, qs, stream))


def gemv_q4(w, xq, y, rows, nb, bias=None, res=None, stream=None):
    _check(lib().amdc_gemv_q4(_p(w), _p(xq), _p(y), rows, nb, _p(bias), _p(res), stream))


def gemv_q4k(w, xq, y, rows, nb, bias=None, res=None, stream=None):
    _check(lib().amdc_gemv_q4k(_p(w), _p(xq), _p(y), rows, nb, _p(bias), _p(res), stream))


def gemv_q8(w, xq, y, rows, nb, bias=None, res=None, stream=None):
    _check(lib().amdc_gemv_q8(_p(w), _p(xq), _p(y), rows, nb, _p(bias), _p(res), stream))


def gemv_q6k(w, xq, y, rows, nb, bias=None, res=None, stream=None):
    _check(lib().amdc_gemv_q6k(_p(w), _p(xq), _p(y), rows, nb, _p(bias), _p(res), stream))


def gemv(kind, w, xq, y, rows, nb, bias=None, res=None, stream=None):
    f = getattr(lib(), "amdc_gemv_" + _SUF[kind])
    _check(f(_p(w), _p(xq), _p(y), rows, nb, _p(bias), _p(res), stream))


def gemv_x(kind, w, x, y, rows, nb, bias=None, res=None, q8=None, stream=None):
    """Decode GEMV on the f32 vector x (quantized in the kernel where a workgroup per CU holds the rows or
    nb <= 128, else quantize + GEMV; q8: optional Q8 output)."""
    f = getattr(lib(), f"amdc_gemv_{_SUF[kind]}_x")
    _check(f(_p(w), _p(x), _p(y), rows, nb, _p(bias), _p(res), _p(q8), stream))


def gemv_q4_t(w, xq, y, rows, nb, T, xs, ys, rs=0, bias=None, res=None, stream=None):
    _check(lib().amdc_gemv_q4_t(_p(w), _p(xq), _p(y), rows, nb, _p(bias), _p(res), T, xs, ys, rs, stream))


def gemv_q4k_t(w, xq, y, rows, nb, T, xs, ys, rs=0, bias=None, res=None, stream=None):
    _check(lib().amdc_gemv_q4k_t(_p(w), _p(xq), _p(y), rows, nb, _p(bias), _p(res), T, xs, ys, rs, stream))


def gemv_t(kind, w, xq, y, rows, nb, T, xs, ys, rs=0, bias=None, res=None, stream=None):
    f = getattr(lib(), f"amdc_gemv_{_SUF[kind]}_t")
    _check(f(_p(w), _p(xq), _p(y), rows, nb, _p(bias), _p(res), T, xs, ys, rs, stream))


def gemm_q4k(w, xq, y, rows, nb, T, xs, ys, rs=0, bias=None, res=None, stream=None):
    _check(lib().amdc_gemm_q4k(_p(w), _p(xq), _p(y), rows, nb, _p(bias), _p(res), T, xs, ys, rs, stream))


def gemm(kind, w, xq, y, rows, nb, T, xs, ys, rs=0, bias=None, res=None, stream=None):
    """The prefill GEMM of a matrix of any kind."""
    f = getattr(lib(), "amdc_gemm_" + _SUF[kind])
    _check(f(_p(w), _p(xq), _p(y), rows, nb, _p(bias), _p(res), T, xs, ys, rs, stream))


def op_gemv(kind, w, xq, y, rows, nb, T, xs, ys, rs=0, bias=None, res=None, stream=None):
    _check(lib().amdc_op_gemv(kind, _p(w), _p(xq), _p(y), rows, nb, _p(bias), _p(res), T, xs, ys, rs, stream))


def op_gemv_noalloc(kind, w, xq, y, rows, nb, T, xs, ys, rs=0, bias=None, res=None, stream=None):
    """op_gemv with the code object's fixed workspace (no device allocation; SCRATCH_BYTES at most)."""
    _check(lib().amdc_op_gemv_noalloc(kind, _p(w), _p(xq), _p(y), rows, nb, _p(bias), _p(res), T, xs, ys, rs, stream))


SCRATCH_BYTES = 64 << 20


def last_kernel():
    """The kernel the library launched last."""
    return lib().amdc_last_kernel().decode()  # AMDC_SCRATCH_BYTES of include/amdc_q4.h


def block_dots(kind, w, xq, out, rows, nb, stream=None):
    _check(lib().amdc_block_dots(kind, _p(w), _p(xq), _p(out), rows, nb, stream))


def probe_read(src, nbytes, scratch, grid, stream=None):
    _check(lib().amdc_probe_read(_p(src), nbytes, _p(scratch), grid, stream))


def probe_copy(dst, src, nbytes, grid, stream=None):
    _check(lib().amdc_probe_copy(_p(dst), _p(src), nbytes, grid, stream))


def rmsnorm_q8(x, w, y, n, eps, q=None, T=1, xs=0, ys=0, qs=0, stream=None):
    """amdc_rmsnorm_q8: y = rmsnorm(x) w and, when q is given, its Q8 copy."""
    _check(lib().amdc_rmsnorm_q8(_p(x), _p(w), _p(y), n, eps, _p(q), T, xs, ys, qs, stream))


def gemv_norm(kind, w, xq, y, rows, nb, nw, ny, eps, nq=None, bias=None, res=None, stream=None):
    """amdc_gemv_norm: the decode GEMV y and, from its last workgroup, ny = rmsnorm(y) nw and its Q8 copy nq."""
    _check(lib().amdc_gemv_norm(kind, _p(w), _p(xq), _p(y), rows, nb, _p(bias), _p(res), _p(nw), _p(ny), _p(nq), eps, stream))


def swiglu_q8(a, b, n, q=None, T=1, as_=0, qs=0, stream=None):
    """amdc_swiglu_q8: a = silu(a) b in place and, when q is given, its Q8 copy."""
    _check(lib().amdc_swiglu_q8(_p(a), _p(b), n, _p(q), T, as_, qs, stream))


def chain_quant(x, q, nb, sync=True):
    """A quantize operation of a GEMV chain: x (f32) -> q (Q8)."""
    return ChainOp(CHAIN_QUANT, 0, int(sync), 0, nb, None, _p(x), _p(q), None, None, None, None)


def chain_gemv(kind, w, xq, y, rows, nb, bias=None, res=None, sync=True):
    """A decode-GEMV operation of a GEMV chain: w, xq (Q8) -> y."""
    return ChainOp(CHAIN_GEMV, kind, int(sync), rows, nb, _p(w), None, None, _p(xq), _p(y), _p(bias), _p(res))


def chain_gemv_x(kind, w, x, y, rows, nb, bias=None, res=None, sync=True):
    """A decode-GEMV operation on the f32 vector x (quantized inside the operation): w, x -> y."""
    return ChainOp(CHAIN_GEMV_X, kind, int(sync), rows, nb, _p(w), _p(x), None, None, _p(y), _p(bias), _p(res))


def chain_rmsnorm_q8(x, w, y, nb, eps, q=None, sync=True):
    """An RMSNorm + Q8 operation of a chain (amdc_rmsnorm_q8 of one token): x, w -> y and, with q, its Q8 copy."""
    return ChainOp(CHAIN_RMSNORM_Q8, 0, int(sync), 0, nb, _p(w), _p(x), _p(q), None, _p(y), None, None, eps)


def chain_swiglu_q8(a, b, nb, q=None, sync=True):
    """A SwiGLU + Q8 operation of a chain (amdc_swiglu_q8 of one token): a = silu(a) b in place and, with q,
    its Q8 copy."""
    return ChainOp(CHAIN_SWIGLU_Q8, 0, int(sync), 0, nb, None, _p(b), _p(q), None, _p(a), None, None, 0.0)


CHAIN_AUTO, CHAIN_PERSISTENT, CHAIN_STREAMING = 0, 1, 2


class Chain:
    """amdc_chain_create_form / _launch / _check / _destroy: a list of ChainOp run by one launch (form:
    CHAIN_AUTO, CHAIN_PERSISTENT or CHAIN_STREAMING)."""

    def __init__(self, ops, form=CHAIN_AUTO):
        arr = (ChainOp * len(ops))(*ops)
        h = _P()
        _check(lib().amdc_chain_create_form(C.cast(arr, _P), len(ops), form, C.byref(h)))
        self.h = h

    def launch(self, stream=None):
        _check(lib().amdc_chain_launch(self.h, stream))

    def check(self):
        _check(lib().amdc_chain_check(self.h))

    def trace(self, buf):
        """amdc_chain_trace: record the timeline of later launches into buf (a DevBuf of trace_words()
        u64 words), or stop (None)."""
        _check(lib().amdc_chain_trace(self.h, buf.ptr if buf is not None else None))

    def trace_words(self):
        return lib().amdc_chain_trace_words(self.h)

    @classmethod
    def _adopt(cls, h):
        c = cls.__new__(cls)
        c.h = h
        return c

    def __del__(self):
        if getattr(self, "h", None) and _lib is not None:
            lib().amdc_chain_destroy(self.h)
            self.h = None


class ChainRecorder:
    """amdc_chain_record_begin / _end as a context: the recordable operators called on `stream` inside the
    block are appended to a chain instead of launched; `.chain` holds it after the block."""

    def __init__(self, stream, form=CHAIN_AUTO):
        self.stream, self.form, self.chain = stream, form, None

    def __enter__(self):
        _check(lib().amdc_chain_record_begin(self.stream.s))
        return self

    def __exit__(self, et, ev, tb):
        h = _P()
        rc = lib().amdc_chain_record_end(self.stream.s, self.form, C.byref(h))
        if et is None:
            _check(rc)
            self.chain = Chain._adopt(h)
        elif h.value:
            lib().amdc_chain_destroy(h)
        return False


# ---------------------------------------------------------------- GGUF files (include/amdc_gguf.h)

def _k(name):
    """A key or tensor name as the C strings of the file (any bytes round-trip through str)."""
    return name.encode(errors="surrogateescape") if isinstance(name, str) else bytes(name)


class Gguf:
    """A GGUF v3 file opened by amdc_gguf_open (memory-mapped). Keys and names are str (bytes that are
    not UTF-8 kept as surrogate escapes) or bytes."""

    def __init__(self, path):
        h = _P()
        _check(lib().amdc_gguf_open(os.fsencode(path), C.byref(h)))
        self.h = h

    def close(self):
        if getattr(self, "h", None) and _lib is not None:
            lib().amdc_gguf_close(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    @property
    def version(self):
        return lib().amdc_gguf_version(self.h)

    @property
    def alignment(self):
        return lib().amdc_gguf_alignment(self.h)

    @property
    def data_offset(self):
        return lib().amdc_gguf_data_offset(self.h)

    def keys(self):
        out = []
        for i in range(lib().amdc_gguf_n_kv(self.h)):
            k, t = C.c_char_p(), C.c_uint32()
            _check(lib().amdc_gguf_key_at(self.h, i, C.byref(k), C.byref(t)))
            out.append((k.value.decode(errors="surrogateescape"), t.value))
        return out

    def get_int(self, key):
        v = _I64()
        return v.value if lib().amdc_gguf_get_int(self.h, _k(key), C.byref(v)) else None

    def get_float(self, key):
        v = C.c_double()
        return v.value if lib().amdc_gguf_get_float(self.h, _k(key), C.byref(v)) else None

    def get_str(self, key):
        p, n = C.c_void_p(), _U64()
        if not lib().amdc_gguf_get_str(self.h, _k(key), C.byref(p), C.byref(n)):
            return None
        return C.string_at(p.value, n.value).decode(errors="surrogateescape") if n.value else ""

    def get_arr(self, key):
        """(element type, count, numpy view of the packed scalars or None)."""
        t, n, d = C.c_uint32(), _U64(), C.c_void_p()
        if not lib().amdc_gguf_get_arr(self.h, _k(key), C.byref(t), C.byref(n), C.byref(d)):
            return None
        dt = {0: np.uint8, 1: np.int8, 2: np.uint16, 3: np.int16, 4: np.uint32, 5: np.int32, 6: np.float32, 7: np.uint8,
              10: np.uint64, 11: np.int64, 12: np.float64}.get(t.value)
        arr = None
        if d.value and dt is not None:
            arr = np.frombuffer(C.string_at(d.value, n.value * np.dtype(dt).itemsize), dtype=dt)
        return t.value, n.value, arr

    def get_arr_str(self, key, i):
        p, n = C.c_void_p(), _U64()
        if not lib().amdc_gguf_get_arr_str(self.h, _k(key), i, C.byref(p), C.byref(n)):
            return None
        return C.string_at(p.value, n.value).decode(errors="surrogateescape") if n.value else ""

    def tensors(self):
        out = []
        for i in range(lib().amdc_gguf_n_tensors(self.h)):
            t = GgufTensor()
            _check(lib().amdc_gguf_tensor_at(self.h, i, C.byref(t)))
            out.append(t)
        return out

    def find(self, name):
        return lib().amdc_gguf_find_tensor(self.h, _k(name))

    def mat_info(self, name):
        m = Mat()
        _check(lib().amdc_gguf_mat_info(self.h, _k(name), C.byref(m)))
        return m

    def repack(self, name, threads=0):
        """The tensor repacked into the CDNA4 layout on the host: (Mat, uint8 array)."""
        m = self.mat_info(name)
        dst = np.empty(m.bytes, dtype=np.uint8)
        _check(lib().amdc_gguf_repack(self.h, _k(name), threads, C.byref(m), dst.ctypes.data_as(_P)))
        return m, dst

    def load(self, name, threads=0, stream=None):
        """The streaming load to the device (amdc_gguf_load): a DevMat owning the device memory."""
        m = Mat()
        _check(lib().amdc_gguf_load(self.h, _k(name), threads, C.byref(m), stream))
        return DevMat(m)


class DevMat:
    """A device matrix from Gguf.load; .ptr is the weights, .m the amdc_mat."""

    def __init__(self, m):
        self.m = m
        self.ptr = m.w

    def download(self):
        out = np.empty(self.m.bytes, dtype=np.uint8)
        _check(lib().amdc_memcpy_d2h(out.ctypes.data_as(_P), self.ptr, self.m.bytes))
        return out

    def free(self):
        if self.m.w and _lib is not None:
            lib().amdc_mat_release(C.byref(self.m))
            self.ptr = None

    def __del__(self):
        self.free()
