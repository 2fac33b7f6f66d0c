"""Legacy CPU codecs of the reference -- TEST INFRASTRUCTURE ONLY.

Python side of ``oracle/legacy_oracle.c``: the packed-buffer layout of the
reference's legacy dispatcher (``quantization_buffer_t`` followed by one
format struct and its arrays, legacy_modules/quantization/src/
quantization.cpp:5-12, 14-90) and ctypes wrappers of the C restatement of the
eleven codecs.  Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import this module.

Pointer fields (the ``payload`` pointer of the outer header and the array
pointers of each format struct) hold addresses of the process that wrote the
buffer; ``mask_pointers`` zeroes them so buffers from different writers can
be compared byte for byte.
"""
from __future__ import annotations

import ctypes
import struct
import threading

import numpy as np

from . import oracle as _o

# quantization_method_t (modules/quantization_cuda/include/quantization_cuda/
# quantization_method.hpp:5-19)
Q8_0, Q4_0, Q2_K, BF16, FP16, FP8, FP4, MXFP8, MXFP4, NVFP4, NF4_DQ, NF4, Q2_K_FAST = range(13)
NAMES = {Q8_0: "Q8_0", Q4_0: "Q4_0", Q2_K: "Q2_K", BF16: "BF16", FP16: "FP16", FP8: "FP8", FP4: "FP4",
         MXFP8: "MXFP8", MXFP4: "MXFP4", NVFP4: "NVFP4", NF4_DQ: "NF4_DQ", NF4: "NF4", Q2_K_FAST: "Q2_K_FAST"}
ALL = tuple(range(13))

OUTER = struct.Struct("<i4xQQ")  # quantization_buffer_t: method, shape.num_elements, payload*
assert OUTER.size == 24

# format struct of each method: (struct, indices of pointer fields)
_BLOCK3 = struct.Struct("<QQQQQ")        # n, num_blocks, block_size, ptr, ptr (40)
_BLOCK3F = struct.Struct("<QQQf4xQQ")    # n, num_blocks, block_size, f32, ptr, ptr (48)
_Q2K = struct.Struct("<QQI4xQ")          # n, n_aligned, num_super_blocks, ptr (32)
_ELEM = struct.Struct("<QQ")             # n, ptr (16)
_ELEMF = struct.Struct("<Qf4xQ")         # n, f32 scale, ptr (24)
assert (_BLOCK3.size, _BLOCK3F.size, _Q2K.size, _ELEM.size, _ELEMF.size) == (40, 48, 32, 16, 24)
Q2K_RECORD = 84
BLOCK = {Q8_0: 32, Q4_0: 32, MXFP8: 32, MXFP4: 32, NVFP4: 16, NF4: 64, NF4_DQ: 64}


def header_struct(method: int):
    """(struct, byte offsets of the pointer fields) of the format struct."""
    if method in (Q8_0, Q4_0, MXFP8, MXFP4, NF4):
        return _BLOCK3, (24, 32)
    if method in (NVFP4, NF4_DQ):
        return _BLOCK3F, (32, 40)
    if method in (Q2_K, Q2_K_FAST):
        return _Q2K, (24,)
    if method in (BF16, FP16):
        return _ELEM, (8,)
    if method in (FP8, FP4):
        return _ELEMF, (16,)
    raise ValueError(method)


def payload_size(method: int, n: int) -> int:
    """Size of the format struct plus its arrays (the get_*_array_size
    functions, e.g. q8_0_impl.cpp:3-6, q2_k_impl.cpp:39-42)."""
    h = header_struct(method)[0].size
    half = (n + 1) // 2
    if method in (Q2_K, Q2_K_FAST):
        return h + ((n + 255) // 256) * Q2K_RECORD
    if method in (BF16, FP16):
        return h + 2 * n
    if method == FP8:
        return h + n
    if method == FP4:
        return h + half
    nb = (n + BLOCK[method] - 1) // BLOCK[method]
    return h + {Q8_0: 4 * nb + n, Q4_0: 4 * nb + half, MXFP8: nb + n, MXFP4: nb + half,
                NVFP4: nb + half, NF4: 4 * nb + half, NF4_DQ: nb + half}[method]


def mask_pointers(method: int, packed: bytes) -> bytes:
    """The packed buffer with the outer payload pointer and the format
    struct's array pointers zeroed."""
    b = bytearray(packed)
    b[16:24] = bytes(8)
    for off in header_struct(method)[1]:
        b[24 + off:24 + off + 8] = bytes(8)
    return bytes(b)


# ---------------------------------------------------------------------------
# C restatement
# ---------------------------------------------------------------------------
_configured = None
_lock = threading.Lock()


def _lib():
    """The oracle library with the legacy functions' signatures set (once
    per loaded handle, under a lock: worker threads may make the first
    call)."""
    global _configured
    with _lock:
        L = _o.lib()
        if _configured is L:
            return L
        P, U64, F = ctypes.c_void_p, ctypes.c_uint64, ctypes.c_float
        for name in ("q8_0", "q4_0", "mxfp8", "mxfp4"):
            getattr(L, f"oracle_{name}_encode").argtypes = [P, U64, P, P]
            getattr(L, f"oracle_{name}_decode").argtypes = [P, P, U64, P]
        for name in ("fp8", "fp4"):
            getattr(L, f"oracle_{name}_encode").argtypes = [P, U64, P, P]
            getattr(L, f"oracle_{name}_decode").argtypes = [F, P, U64, P]
        L.oracle_nvfp4_encode.argtypes = [P, U64, P, P, P]
        L.oracle_nvfp4_decode.argtypes = [F, P, P, U64, P]
        L.oracle_q2k_encode.argtypes = [P, U64, ctypes.c_int, P]
        L.oracle_q2k_decode.argtypes = [P, U64, P]
        for name in ("bf16", "fp16"):
            getattr(L, f"oracle_{name}_encode").argtypes = [P, U64, P]
            getattr(L, f"oracle_{name}_decode").argtypes = [P, U64, P]
        L.oracle_legacy_sweep.restype = ctypes.c_uint64
        L.oracle_legacy_sweep.argtypes = [ctypes.c_int, U64, U64]
        L.oracle_fp16_from_f32.restype = ctypes.c_uint16
        L.oracle_fp16_from_f32.argtypes = [F]
        L.oracle_fp16_to_f32.restype = F
        L.oracle_fp16_to_f32.argtypes = [ctypes.c_uint16]
        L.oracle_legacy_e4m3_encode.restype = ctypes.c_uint8
        L.oracle_legacy_e4m3_encode.argtypes = [F]
        L.oracle_legacy_e4m3_decode.restype = F
        L.oracle_legacy_e4m3_decode.argtypes = [ctypes.c_uint8]
        L.oracle_e2m1_encode.restype = ctypes.c_uint8
        L.oracle_e2m1_encode.argtypes = [F]
        L.oracle_e2m1_decode.restype = F
        L.oracle_e2m1_decode.argtypes = [ctypes.c_uint8]
        L.oracle_mx_scale_exp.restype = ctypes.c_int8
        L.oracle_mx_scale_exp.argtypes = [F, F]
        _configured = L
        return L


def _p(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def encode(method: int, x: np.ndarray) -> bytes:
    """The payload (format struct with zero pointers, then the arrays) that
    quantization_compress writes for `x`."""
    x = np.ascontiguousarray(x, np.float32).ravel()
    n = x.size
    if n == 0:
        raise ValueError("empty input")
    if method in (NF4, NF4_DQ):
        q = _o.quant_compress(x, method)
        nb = (n + 63) // 64
        if method == NF4:
            return (_BLOCK3.pack(n, nb, 64, 0, 0) + np.asarray(q.scales, np.float32).tobytes()
                    + np.asarray(q.codes, np.uint8).tobytes())
        return (_BLOCK3F.pack(n, nb, 64, float(q.dq), 0, 0) + np.asarray(q.scales, np.uint8).tobytes()
                + np.asarray(q.codes, np.uint8).tobytes())
    L = _lib()
    half = (n + 1) // 2
    if method in (Q8_0, Q4_0, MXFP8, MXFP4):
        nb = (n + 31) // 32
        sc = np.zeros(nb, np.float32 if method in (Q8_0, Q4_0) else np.int8)
        q = np.zeros(n if method in (Q8_0, MXFP8) else half, np.uint8)
        getattr(L, f"oracle_{NAMES[method].lower()}_encode")(_p(x), n, _p(sc), _p(q))
        return _BLOCK3.pack(n, nb, 32, 0, 0) + sc.tobytes() + q.tobytes()
    if method in (FP8, FP4):
        s = np.zeros(1, np.float32)
        q = np.zeros(n if method == FP8 else half, np.uint8)
        getattr(L, f"oracle_{NAMES[method].lower()}_encode")(_p(x), n, _p(s), _p(q))
        return _ELEMF.pack(n, float(s[0]), 0) + q.tobytes()
    if method == NVFP4:
        nb = (n + 15) // 16
        s = np.zeros(1, np.float32)
        bs = np.zeros(nb, np.uint8)
        q = np.zeros(half, np.uint8)
        L.oracle_nvfp4_encode(_p(x), n, _p(s), _p(bs), _p(q))
        return _BLOCK3F.pack(n, nb, 16, float(s[0]), 0, 0) + bs.tobytes() + q.tobytes()
    if method in (Q2_K, Q2_K_FAST):
        nsb = (n + 255) // 256
        rec = np.zeros(nsb * Q2K_RECORD, np.uint8)
        L.oracle_q2k_encode(_p(x), n, 1 if method == Q2_K_FAST else 0, _p(rec))
        return _Q2K.pack(n, nsb * 256, nsb, 0) + rec.tobytes()
    if method in (BF16, FP16):
        q = np.zeros(n, np.uint16)
        getattr(L, f"oracle_{NAMES[method].lower()}_encode")(_p(x), n, _p(q))
        return _ELEM.pack(n, 0) + q.tobytes()
    raise ValueError(method)


def packed(method: int, x: np.ndarray) -> bytes:
    """quantization_buffer_t (zero payload pointer) followed by the payload."""
    x = np.ascontiguousarray(x, np.float32).ravel()
    return OUTER.pack(method, x.size, 0) + encode(method, x)


def decode(method: int, payload: bytes, n: int) -> np.ndarray:
    """quantization_decompress of a well-formed payload of `n` elements."""
    L = _lib()
    out = np.zeros(n, np.float32)
    h = header_struct(method)[0]
    fields = h.unpack_from(payload, 0)
    body = np.frombuffer(payload, np.uint8, offset=h.size)
    half = (n + 1) // 2
    if method in (NF4, NF4_DQ):
        nb = (n + 63) // 64
        ss = 4 * nb if method == NF4 else nb
        scales = body[:ss].view(np.float32).copy() if method == NF4 else body[:ss].copy()
        dq = float(fields[3]) if method == NF4_DQ else 0.0
        return _o.quant_decompress(_o.Quant(method, n, scales, body[ss:ss + half].copy(), dq))
    if method in (Q8_0, Q4_0, MXFP8, MXFP4):
        nb = (n + 31) // 32
        ss = 4 * nb if method in (Q8_0, Q4_0) else nb
        sc = body[:ss].copy()
        q = body[ss:].copy()
        getattr(L, f"oracle_{NAMES[method].lower()}_decode")(_p(sc), _p(q), n, _p(out))
        return out
    if method in (FP8, FP4):
        q = body.copy()
        getattr(L, f"oracle_{NAMES[method].lower()}_decode")(ctypes.c_float(fields[1]), _p(q), n, _p(out))
        return out
    if method == NVFP4:
        nb = (n + 15) // 16
        bs, q = body[:nb].copy(), body[nb:nb + half].copy()
        L.oracle_nvfp4_decode(ctypes.c_float(fields[3]), _p(bs), _p(q), n, _p(out))
        return out
    if method in (Q2_K, Q2_K_FAST):
        rec = body.copy()
        L.oracle_q2k_decode(_p(rec), n, _p(out))
        return out
    if method in (BF16, FP16):
        q = body[:2 * n].view(np.uint16).copy()
        getattr(L, f"oracle_{NAMES[method].lower()}_decode")(_p(q), n, _p(out))
        return out
    raise ValueError(method)


def sweep(kind: int, lo: int, hi: int) -> int:
    """Checksum of the oracle's FP16 (0), BF16 (1) conversion or MX exponent
    (2: max 448, 3: max 6) over every float pattern in [lo, hi)."""
    return int(_lib().oracle_legacy_sweep(kind, lo, hi))
