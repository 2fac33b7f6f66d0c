"""ctypes binding of the MI355X bitsqz_llm library (lib/libbitsqz_llm_lib.so).

The library is the product: a C-ABI shared library built from csrc/ by
build.py.  This module only binds it for Python callers (the tests and
bench.py): it defines the packed-object structs with the reference's byte
layout (include/bitsqz_llm.hpp:48-93), a small device-buffer helper over the
library's own hipMalloc wrappers, and thin functions named after the
reference's operators.  It never computes anything itself: every function
either calls the library or fails loudly when the library is missing.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib", "libbitsqz_llm_lib.so")

QUANT_NONE, NF4_DQ, NF4 = -1, 10, 11
INPUT_HOST, INPUT_DEVICE = 0, 1
FLAG_SVD, FLAG_OUTLIER, FLAG_ERROR = 1, 2, 4
SECTION_NONE, SECTION_FP32, SECTION_QUANT, SECTION_TOPK = 0, 1, 2, 3


class Section(C.Structure):
    _fields_ = [("offset", C.c_uint64), ("size", C.c_uint64), ("storage", C.c_uint8),
                ("reserved", C.c_uint8 * 7)]


class PackedHeader(C.Structure):
    """bitsqz_llm_array_t (reference include/bitsqz_llm.hpp:55-83), 200 bytes."""
    _fields_ = [
        ("num_rows", C.c_uint16), ("num_columns", C.c_uint16), ("num_elements", C.c_uint32),
        ("outlier_topk_ratio", C.c_float), ("error_correction_topk_ratio", C.c_float),
        ("svd_ranks", C.c_int16), ("svd_niters", C.c_int16), ("effective_rank", C.c_int16),
        ("reserved0", C.c_int16),
        ("svd_uv_format", C.c_int32), ("svd_s_format", C.c_int32),
        ("quantization_only_format", C.c_int32), ("reserved1", C.c_int32),
        ("flags", C.c_uint32),
        ("section_u", Section), ("section_s", Section), ("section_v", Section),
        ("section_direct", Section), ("section_outlier_topk", Section),
        ("section_error_topk", Section),
        ("payload", C.c_void_p),
    ]


assert C.sizeof(PackedHeader) == 200 and PackedHeader.section_u.offset == 48
assert PackedHeader.payload.offset == 192


class Profile(C.Structure):
    """bitsqz_llm_compress_profile_t (reference include/bitsqz_llm.hpp:85-93)."""
    _fields_ = [(n, C.c_double) for n in (
        "topk_separation_latency_ms", "svd_lowrank_cuda_latency_ms",
        "quantization_compress_latency_ms", "reconsturct_quantization_decompress_latency_ms",
        "reconstruct_svd_latency_ms", "error_extraction_latency_ms", "other_latency_ms")]


class DevicePacked(C.Structure):
    """bsq_device_packed_t (include/bitsqz_llm_c.h)."""
    _fields_ = [
        ("header", PackedHeader),
        ("d_flags", C.c_void_p),
        ("d_dense", C.c_void_p * 4), ("d_scales_f32", C.c_void_p * 4),
        ("d_scales_u8", C.c_void_p * 4), ("d_dq_scale", C.c_void_p * 4),
        ("d_codes", C.c_void_p * 4), ("count", C.c_uint64 * 4),
        ("d_topk_idx", C.c_void_p * 2), ("d_topk_val", C.c_void_p * 2),
        ("topk_k", C.c_uint16 * 2),
    ]


_lib = None
P = C.c_void_p


def lib():
    """The loaded library; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} missing: run `python bitsqueeze-llm_amd/build.py`")
    L = C.CDLL(LIB_PATH)
    u16, u32, u64, f32, i32 = C.c_uint16, C.c_uint32, C.c_uint64, C.c_float, C.c_int
    sig = {
        "bsq_last_error": (C.c_char_p, []),
        "bsq_version": (C.c_char_p, []),
        "bsq_compress_initialize": (i32, [u16, u16, f32, f32, i32, i32, i32, i32, i32, i32]),
        "bsq_compress_release": (None, []),
        "bsq_decompress_initialize": (i32, [u16, u16, f32, f32, i32, i32, i32, i32]),
        "bsq_decompress_release": (None, []),
        "bsq_compress": (i32, [P, C.POINTER(C.POINTER(PackedHeader)), C.POINTER(Profile)]),
        "bsq_decompress": (i32, [P, P, u32]),
        "bsq_get_packed_size": (u64, [P]),
        "bsq_load_from_buffer": (C.POINTER(PackedHeader), [P, u64]),
        "bsq_free": (None, [P]),
        "bsq_compress_set_sketch": (i32, [P]),
        "bsq_device_compress": (i32, [P, C.POINTER(DevicePacked)]),
        "bsq_device_decompress": (i32, [C.POINTER(DevicePacked), P, u32]),
        "bsq_device_synchronize": (i32, []),
        "bsq_runtime_stream": (P, []),
        "bsq_lanes_initialize": (i32, [i32, u16, u16, f32, f32, i32, i32, i32, i32, i32]),
        "bsq_lanes_roundtrip": (i32, [i32, P, P]),
        "bsq_lanes_stream": (P, [i32]),
        "bsq_lanes_synchronize": (i32, []),
        "bsq_lanes_release": (None, []),
        "bsq_topk_num_columns": (i32, [u16, f32, C.POINTER(u16)]),
        "bsq_topk_select": (i32, [P, u16, u16, u16, P, P, P, P]),
        "bsq_topk_scatter": (i32, [P, P, u16, u16, u16, P, i32, P]),
        "bsq_quant_compress": (i32, [P, u64, i32, P, P, P, P, P]),
        "bsq_quant_decompress": (i32, [u64, i32, P, P, P, P, P, P]),
        "bsq_quant_nf4_codes": (i32, [P, u64, P, P]),
        "bsq_quant_e4m3_encode": (i32, [P, u64, P, P]),
        "bsq_quant_e4m3_decode": (i32, [P, u64, P, P]),
        "bsq_quant_nf4_code_sweep": (i32, [u64, u64, P, P, P]),
        "bsq_nf4_thresholds": (None, [P]),
        "bsq_svd_lowrank": (i32, [P, i32, i32, i32, i32, P, u64, P, P, P, P]),
        "bsq_svd_lowrank_noalloc": (i32, [P, i32, i32, i32, i32, P, u64, P, P, P, P]),
        "bsq_reconstruct_lowrank": (i32, [P, P, P, i32, i32, i32, P, P]),
        "bsq_gaussian_fill": (i32, [P, u64, u64, P]),
        "bsq_device_count": (i32, [C.POINTER(i32)]),
        "bsq_device_malloc": (i32, [C.POINTER(P), u64]),
        "bsq_device_free": (i32, [P]),
        "bsq_memcpy_h2d": (i32, [P, P, u64]),
        "bsq_memcpy_d2h": (i32, [P, P, u64]),
        "bsq_memcpy_d2d": (i32, [P, P, u64]),
        "bsq_device_memset": (i32, [P, i32, u64]),
        "bsq_host_malloc": (i32, [C.POINTER(P), u64]),
        "bsq_host_free": (i32, [P]),
        "bsq_memcpy_h2d_async": (i32, [P, P, u64, P]),
        "bsq_stream_synchronize": (i32, [P]),
        "bsq_event_create": (i32, [C.POINTER(P)]),
        "bsq_event_destroy": (i32, [P]),
        "bsq_event_record": (i32, [P, P]),
        "bsq_event_elapsed_ms": (i32, [P, P, C.POINTER(f32)]),
        "bsq_kernel_timer_start": (i32, []),
        "bsq_copy_kernel": (i32, [P, P, u64, P]),
        "bsq_kernel_timer_stop": (i32, [C.POINTER(C.c_double), C.POINTER(i32)]),
        "bsq_kernel_timer_read": (i32, [i32, C.POINTER(C.c_double), C.POINTER(i32)]),
        "bsq_legacy_compress": (i32, [i32, P, u64, C.POINTER(P)]),
        "bsq_legacy_decompress": (i32, [P, P, u64]),
        "bsq_legacy_packed_size": (C.c_longlong, [P]),
        "bsq_legacy_load": (P, [P, C.c_longlong]),
        "bsq_legacy_free": (None, [P]),
        "bsq_legacy_payload_bytes": (C.c_longlong, [i32, u64]),
        "bsq_legacy_encode_device": (i32, [i32, P, u64, P, P]),
        "bsq_legacy_decode_device": (i32, [i32, P, u64, P, P]),
        "bsq_legacy_sweep": (i32, [i32, u64, u64, P, P]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


class BsqError(RuntimeError):
    pass


def check(rc: int, what: str):
    if rc != 0:
        raise BsqError(f"{what} failed: {lib().bsq_last_error().decode()}")


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(C.c_void_p)


# ---------------------------------------------------------------------------
# device memory
# ---------------------------------------------------------------------------
class DeviceBuffer:
    """A hipMalloc'd buffer owned by Python."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        self.ptr = C.c_void_p()
        if self.nbytes:
            check(lib().bsq_device_malloc(C.byref(self.ptr), self.nbytes), "hipMalloc")

    @classmethod
    def from_array(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        b.upload(a)
        return b

    def upload(self, a: np.ndarray):
        a = np.ascontiguousarray(a)
        assert a.nbytes <= self.nbytes
        if a.nbytes:
            check(lib().bsq_memcpy_h2d(self.ptr, _ptr(a), a.nbytes), "H2D")

    def download(self, dtype, count: int) -> np.ndarray:
        out = np.empty(count, dtype)
        if out.nbytes:
            assert out.nbytes <= self.nbytes
            check(lib().bsq_memcpy_d2h(_ptr(out), self.ptr, out.nbytes), "D2H")
        return out

    def zero(self):
        if self.nbytes:
            check(lib().bsq_device_memset(self.ptr, 0, self.nbytes), "memset")

    @property
    def value(self):
        return self.ptr.value

    def free(self):
        if self.ptr and self.ptr.value:
            lib().bsq_device_free(self.ptr)
        self.ptr = C.c_void_p()

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class PinnedBuffer:
    """hipHostMalloc'd (page-locked) host memory owned by Python, viewed as a
    flat numpy array of `dtype`."""

    def __init__(self, count: int, dtype=np.float32):
        self.dtype = np.dtype(dtype)
        self.nbytes = int(count) * self.dtype.itemsize
        self.ptr = C.c_void_p()
        check(lib().bsq_host_malloc(C.byref(self.ptr), max(self.nbytes, 1)), "hipHostMalloc")
        buf = (C.c_char * max(self.nbytes, 1)).from_address(self.ptr.value)
        self.array = np.frombuffer(buf, dtype=self.dtype, count=int(count))

    def copy_to_device_async(self, dst: DeviceBuffer, stream=None):
        check(lib().bsq_memcpy_h2d_async(dst.ptr, self.ptr, self.nbytes, stream), "H2D async")

    def free(self):
        if self.ptr and self.ptr.value:
            self.array = None
            lib().bsq_host_free(self.ptr)
        self.ptr = C.c_void_p()

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


TIMER_RECONSTRUCT, TIMER_RANGE_FINDER = 0, 1
TIMER_TOPK_OUTLIER, TIMER_TOPK_ERROR, TIMER_DIRECT_ENCODE, TIMER_DIRECT_DECODE = 2, 3, 4, 5


def kernel_timer_start() -> None:
    """Bracket the timed launch classes of the pipelines (TIMER_*) with HIP events."""
    check(lib().bsq_kernel_timer_start(), "kernel timer start")


def kernel_timer_stop() -> tuple[float, int]:
    """Stop bracketing; returns (summed ms, launches) of the reconstruction GEMMs since the start."""
    ms, n = C.c_double(), C.c_int()
    check(lib().bsq_kernel_timer_stop(C.byref(ms), C.byref(n)), "kernel timer stop")
    return ms.value, n.value


def kernel_timer_read(timer_class: int) -> tuple[float, int]:
    """After kernel_timer_stop: (summed ms, launches) of one class (TIMER_*)."""
    ms, n = C.c_double(), C.c_int()
    check(lib().bsq_kernel_timer_read(timer_class, C.byref(ms), C.byref(n)), "kernel timer read")
    return ms.value, n.value


def device_count() -> int:
    n = C.c_int(0)
    rc = lib().bsq_device_count(C.byref(n))
    return n.value if rc == 0 else 0


class Event:
    def __init__(self):
        self.h = C.c_void_p()
        check(lib().bsq_event_create(C.byref(self.h)), "event create")

    def record(self, stream=None):
        check(lib().bsq_event_record(self.h, stream), "event record")

    def elapsed_ms(self, stop: "Event") -> float:
        ms = C.c_float()
        check(lib().bsq_event_elapsed_ms(self.h, stop.h, C.byref(ms)), "event elapsed")
        return ms.value

    def __del__(self):
        try:
            lib().bsq_event_destroy(self.h)
        except Exception:
            pass


# ---------------------------------------------------------------------------
# public ABI (bitsqz_llm.hpp) through the extern "C" twins
# ---------------------------------------------------------------------------
def compress_initialize(rows, cols, outlier_ratio=0.0, error_ratio=0.0, svd_ranks=-1, svd_niters=2,
                        uv_format=QUANT_NONE, s_format=QUANT_NONE, direct_format=QUANT_NONE,
                        input_location=INPUT_DEVICE) -> int:
    return lib().bsq_compress_initialize(rows, cols, outlier_ratio, error_ratio, svd_ranks, svd_niters,
                                         uv_format, s_format, direct_format, input_location)


def decompress_initialize(rows, cols, outlier_ratio=0.0, error_ratio=0.0, svd_ranks=-1,
                          uv_format=QUANT_NONE, s_format=QUANT_NONE, direct_format=QUANT_NONE) -> int:
    return lib().bsq_decompress_initialize(rows, cols, outlier_ratio, error_ratio, svd_ranks, uv_format,
                                           s_format, direct_format)


def compress_release():
    lib().bsq_compress_release()


def decompress_release():
    lib().bsq_decompress_release()


def packed_bytes(ptr) -> bytes:
    """Bytes of a library-owned packed object (header + payload)."""
    vp = C.cast(ptr, C.c_void_p)
    n = lib().bsq_get_packed_size(vp)
    return C.string_at(vp, n)


def compress(src, profile: bool = False):
    """bitsqz_llm_compress: `src` is a host float32 array (HOST runtime) or a
    DeviceBuffer (DEVICE runtime).  Returns the packed bytes (and profile)."""
    out = C.POINTER(PackedHeader)()
    prof = Profile() if profile else None  # no struct: the two-argument form
    if isinstance(src, DeviceBuffer):
        p = src.ptr
    else:
        src = np.ascontiguousarray(src, np.float32)
        p = _ptr(src)
    check(lib().bsq_compress(p, C.byref(out), C.byref(prof) if profile else None), "bitsqz_llm_compress")
    try:
        data = packed_bytes(out)
    finally:
        lib().bsq_free(C.cast(out, C.c_void_p))
    return (data, prof) if profile else data


def load(buf: bytes):
    """load_bitsqz_llm_from_buffer -> owned pointer (free with free_packed) or None."""
    b = C.create_string_buffer(bytes(buf), len(buf))
    p = lib().bsq_load_from_buffer(b, len(buf))
    return p if p else None


def free_packed(p):
    lib().bsq_free(C.cast(p, C.c_void_p))


def decompress_to_device(buf: bytes, dst: DeviceBuffer, dst_num_elements: int) -> int:
    """bitsqz_llm_decompress of host bytes into `dst`; returns the ABI status."""
    p = load(buf)
    if p is None:
        return 1
    vp = C.cast(p, C.c_void_p)
    try:
        return lib().bsq_decompress(vp, dst.ptr, dst_num_elements)
    finally:
        lib().bsq_free(vp)


def decompress(buf: bytes, rows: int, cols: int) -> np.ndarray:
    dst = DeviceBuffer(rows * cols * 4)
    check(decompress_to_device(buf, dst, rows * cols), "bitsqz_llm_decompress")
    return dst.download(np.float32, rows * cols).reshape(rows, cols)


def topk_num_columns(cols: int, ratio: float) -> int:
    k = C.c_uint16()
    check(lib().bsq_topk_num_columns(cols, ratio, C.byref(k)), "topk_num_columns")
    return k.value


# ---------------------------------------------------------------------------
# module operators
# ---------------------------------------------------------------------------
def topk_select(x: np.ndarray, k: int, separate: bool = False):
    """Per-row top-k: returns (indices u16 rows x k, values f32 rows x k[, residual])."""
    x = np.ascontiguousarray(x, np.float32)
    rows, cols = x.shape
    dx = DeviceBuffer.from_array(x)
    di = DeviceBuffer(max(1, rows * k * 2))
    dv = DeviceBuffer(max(1, rows * k * 4))
    dr = DeviceBuffer(x.nbytes) if separate else None
    check(lib().bsq_topk_select(dx.ptr, rows, cols, k, di.ptr, dv.ptr, dr.ptr if dr else None, None),
          "topk_select")
    check(lib().bsq_stream_synchronize(None), "sync")
    idx = di.download(np.uint16, rows * k).reshape(rows, k)
    val = dv.download(np.float32, rows * k).reshape(rows, k)
    if separate:
        return idx, val, dr.download(np.float32, rows * cols).reshape(rows, cols)
    return idx, val


def topk_scatter(idx: np.ndarray, val: np.ndarray, dense: np.ndarray, accumulate: bool = True) -> np.ndarray:
    dense = np.ascontiguousarray(dense, np.float32)
    rows, cols = dense.shape
    k = idx.shape[1]
    dd = DeviceBuffer.from_array(dense)
    di = DeviceBuffer.from_array(np.ascontiguousarray(idx, np.uint16))
    dv = DeviceBuffer.from_array(np.ascontiguousarray(val, np.float32))
    check(lib().bsq_topk_scatter(di.ptr, dv.ptr, rows, cols, k, dd.ptr, int(accumulate), None), "topk_scatter")
    check(lib().bsq_stream_synchronize(None), "sync")
    return dd.download(np.float32, rows * cols).reshape(rows, cols)


def quant_compress(x: np.ndarray, method: int):
    """Returns (scales, codes, dq): scales f32 (NF4) or u8 (NF4_DQ)."""
    x = np.ascontiguousarray(x, np.float32).ravel()
    n = x.size
    nb, nc = (n + 63) // 64, (n + 1) // 2
    dx = DeviceBuffer.from_array(x)
    dsf = DeviceBuffer(nb * 4)
    dsu = DeviceBuffer(nb)
    ddq = DeviceBuffer(4)
    dc = DeviceBuffer(nc)
    check(lib().bsq_quant_compress(dx.ptr, n, method, dsf.ptr, dsu.ptr, ddq.ptr, dc.ptr, None), "quant_compress")
    check(lib().bsq_stream_synchronize(None), "sync")
    codes = dc.download(np.uint8, nc)
    if method == NF4:
        return dsf.download(np.float32, nb), codes, 0.0
    return dsu.download(np.uint8, nb), codes, float(ddq.download(np.float32, 1)[0])


def quant_decompress(n: int, method: int, scales: np.ndarray, codes: np.ndarray, dq: float = 0.0) -> np.ndarray:
    nb = (n + 63) // 64
    dsf = DeviceBuffer.from_array(np.ascontiguousarray(scales, np.float32)) if method == NF4 else DeviceBuffer(4)
    dsu = DeviceBuffer.from_array(np.ascontiguousarray(scales, np.uint8)) if method == NF4_DQ else DeviceBuffer(4)
    ddq = DeviceBuffer.from_array(np.array([dq], np.float32))
    dc = DeviceBuffer.from_array(np.ascontiguousarray(codes, np.uint8))
    out = DeviceBuffer(n * 4)
    assert scales.size == nb
    check(lib().bsq_quant_decompress(n, method, dsf.ptr, dsu.ptr, ddq.ptr, dc.ptr, out.ptr, None), "quant_decompress")
    check(lib().bsq_stream_synchronize(None), "sync")
    return out.download(np.float32, n)


def _batch(fn_name, src: np.ndarray, out_dtype):
    dsrc = DeviceBuffer.from_array(src)
    dout = DeviceBuffer(max(1, src.size * np.dtype(out_dtype).itemsize))
    check(getattr(lib(), fn_name)(dsrc.ptr, src.size, dout.ptr, None), fn_name)
    check(lib().bsq_stream_synchronize(None), "sync")
    return dout.download(out_dtype, src.size)


def nf4_codes(v: np.ndarray) -> np.ndarray:
    return _batch("bsq_quant_nf4_codes", np.ascontiguousarray(v, np.float32).ravel(), np.uint8)


def e4m3_encode(v: np.ndarray) -> np.ndarray:
    return _batch("bsq_quant_e4m3_encode", np.ascontiguousarray(v, np.float32).ravel(), np.uint8)


def e4m3_decode(c: np.ndarray) -> np.ndarray:
    return _batch("bsq_quant_e4m3_decode", np.ascontiguousarray(c, np.uint8).ravel(), np.float32)


def nf4_code_sweep(lo: int, hi: int):
    dh = DeviceBuffer(16 * 8)
    dc = DeviceBuffer(8)
    check(lib().bsq_quant_nf4_code_sweep(lo, hi, dh.ptr, dc.ptr, None), "nf4 sweep")
    check(lib().bsq_stream_synchronize(None), "sync")
    return dh.download(np.uint64, 16), int(dc.download(np.uint64, 1)[0])


def nf4_thresholds() -> np.ndarray:
    out = np.zeros(15, np.float32)
    lib().bsq_nf4_thresholds(_ptr(out))
    return out


def svd_lowrank(A: np.ndarray, q: int, niter: int, sketch: np.ndarray | None = None, seed: int = 1241):
    A = np.ascontiguousarray(A, np.float32)
    m, n = A.shape
    k = max(1, min(q, m, n))
    dA = DeviceBuffer.from_array(A)
    dR = DeviceBuffer.from_array(np.ascontiguousarray(sketch, np.float32)) if sketch is not None else None
    dU, dS, dV = DeviceBuffer(m * k * 4), DeviceBuffer(k * 4), DeviceBuffer(n * k * 4)
    check(lib().bsq_svd_lowrank(dA.ptr, m, n, q, niter, dR.ptr if dR else None, seed, dU.ptr, dS.ptr, dV.ptr,
                                None), "svd_lowrank")
    return (dU.download(np.float32, m * k).reshape(m, k), dS.download(np.float32, k),
            dV.download(np.float32, n * k).reshape(n, k))


def reconstruct(U: np.ndarray, S: np.ndarray, V: np.ndarray) -> np.ndarray:
    U = np.ascontiguousarray(U, np.float32)
    V = np.ascontiguousarray(V, np.float32)
    m, k = U.shape
    n = V.shape[0]
    dU, dS, dV = DeviceBuffer.from_array(U), DeviceBuffer.from_array(np.ascontiguousarray(S, np.float32)), \
        DeviceBuffer.from_array(V)
    out = DeviceBuffer(m * n * 4)
    check(lib().bsq_reconstruct_lowrank(dU.ptr, dS.ptr, dV.ptr, m, n, k, out.ptr, None), "reconstruct")
    check(lib().bsq_stream_synchronize(None), "sync")
    return out.download(np.float32, m * n).reshape(m, n)


def gaussian(n: int, seed: int) -> np.ndarray:
    d = DeviceBuffer(n * 4)
    check(lib().bsq_gaussian_fill(d.ptr, n, seed, None), "gaussian_fill")
    check(lib().bsq_stream_synchronize(None), "sync")
    return d.download(np.float32, n)


# ---------------------------------------------------------------------------
# device-resident pipeline
# ---------------------------------------------------------------------------
def device_compress(src: DeviceBuffer) -> DevicePacked:
    out = DevicePacked()
    check(lib().bsq_device_compress(src.ptr, C.byref(out)), "bsq_device_compress")
    return out


def device_decompress(packed: DevicePacked, dst: DeviceBuffer, n: int):
    check(lib().bsq_device_decompress(C.byref(packed), dst.ptr, n), "bsq_device_decompress")


def device_synchronize():
    check(lib().bsq_device_synchronize(), "bsq_device_synchronize")


def runtime_stream():
    return lib().bsq_runtime_stream()


# ---------------------------------------------------------------------------
# legacy quantisation formats (include/quantization.hpp)
# ---------------------------------------------------------------------------
LEGACY_Q8_0, LEGACY_Q4_0, LEGACY_Q2_K, LEGACY_BF16, LEGACY_FP16, LEGACY_FP8, LEGACY_FP4 = 0, 1, 2, 3, 4, 5, 6
LEGACY_MXFP8, LEGACY_MXFP4, LEGACY_NVFP4, LEGACY_NF4_DQ, LEGACY_NF4, LEGACY_Q2_K_FAST = 7, 8, 9, 10, 11, 12


def legacy_compress_handle(method: int, x: np.ndarray):
    """quantization_compress of host floats; returns (rc, buffer pointer)."""
    x = np.ascontiguousarray(x, np.float32).ravel()
    out = C.c_void_p()
    rc = lib().bsq_legacy_compress(method, _ptr(x) if x.size else None, x.size, C.byref(out))
    return rc, out


def legacy_compress(method: int, x: np.ndarray) -> bytes:
    """The serialised buffer (quantization_get_packed_size bytes)."""
    rc, h = legacy_compress_handle(method, x)
    check(rc, "quantization_compress")
    try:
        size = lib().bsq_legacy_packed_size(h)
        assert size > 0
        return C.string_at(h, size)
    finally:
        lib().bsq_legacy_free(h)


def legacy_decompress(buf: bytes, n: int, dst_n: int | None = None):
    """load_quantization_from_buffer + quantization_decompress; returns
    (rc, floats) with rc = -1 when the load is refused."""
    raw = C.create_string_buffer(buf, len(buf))
    h = lib().bsq_legacy_load(raw, len(buf))
    if not h:
        return -1, None
    try:
        out = np.zeros(max(n, 1), np.float32)
        rc = lib().bsq_legacy_decompress(h, _ptr(out), n if dst_n is None else dst_n)
        return rc, out[:n]
    finally:
        lib().bsq_legacy_free(h)


def legacy_payload_bytes(method: int, n: int) -> int:
    return int(lib().bsq_legacy_payload_bytes(method, n))


def legacy_encode_device(method: int, x: np.ndarray) -> bytes:
    """Payload image written by the device encoder (pointer fields as the
    device left them)."""
    x = np.ascontiguousarray(x, np.float32).ravel()
    size = legacy_payload_bytes(method, x.size)
    src = DeviceBuffer.from_array(x)
    img = DeviceBuffer(size)
    check(lib().bsq_legacy_encode_device(method, src.ptr, x.size, img.ptr, None), "legacy encode")
    check(lib().bsq_stream_synchronize(None), "sync")
    return img.download(np.uint8, size).tobytes()


def legacy_decode_device(method: int, payload: bytes, n: int) -> np.ndarray:
    img = DeviceBuffer.from_array(np.frombuffer(payload, np.uint8))
    dst = DeviceBuffer(4 * n)
    check(lib().bsq_legacy_decode_device(method, img.ptr, n, dst.ptr, None), "legacy decode")
    check(lib().bsq_stream_synchronize(None), "sync")
    return dst.download(np.float32, n)


def legacy_sweep(kind: int, lo: int, hi: int) -> int:
    d = DeviceBuffer(8)
    d.zero()
    check(lib().bsq_legacy_sweep(kind, lo, hi, d.ptr, None), "legacy sweep")
    check(lib().bsq_stream_synchronize(None), "sync")
    return int(d.download(np.uint64, 1)[0])
