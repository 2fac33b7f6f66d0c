"""bitsqz_llm CPU oracle -- TEST INFRASTRUCTURE ONLY.

Restates the reference's compress / decompress hot path on the CPU so that the
HIP library can be checked against it.  Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
this module, and only as the checker (or the timed CPU baseline), never as the
product path.

Integer / byte work (NF4, NF4_DQ, E4M3, top-k) runs in the C restatement
``oracle/bsq_oracle.c`` (built into ``oracle/liboracle.so``); the byte layouts
of the packed object are written here with ``struct``; the randomised SVD and
the low-rank reconstruction are restated in float64 numpy.

Pinning (see tests/test_oracle.py):
  * NF4 / NF4_DQ / E4M3 codecs: golden vectors written by the reference's own
    legacy codec compiled from its sources (tests/golden/gen_golden.py), an
    exhaustive 2^32 sweep of the code function, and closed forms.
  * top-k: the reference's three known-answer tests and brute force.
  * packed layouts: the reference's offsetof-verified header layout and the
    section blob definitions (byte offsets asserted in tests).
  * SVD: exact recovery of exact low-rank inputs, orthonormality, agreement
    with numpy's dense SVD once the power iteration has converged, and the
    basis invariance of U S V^T.  The reference's own SVD (cuSOLVER/cuRAND)
    cannot be run anywhere in this pipeline, so U/S/V parity is defined with an
    injected sketch matrix.
"""
from __future__ import annotations

import ctypes
import os
import struct
from dataclasses import dataclass, field

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))

# ---------------------------------------------------------------------------
# enums / constants (reference include/bitsqz_llm.hpp:17-46, src/bitsqz_llm.cu:25-29)
# ---------------------------------------------------------------------------
QUANT_NONE = -1
NF4_DQ = 10
NF4 = 11
SECTION_NONE, SECTION_FP32, SECTION_QUANT, SECTION_TOPK = 0, 1, 2, 3
INPUT_HOST, INPUT_DEVICE = 0, 1
FLAG_SVD, FLAG_OUTLIER, FLAG_ERROR = 1, 2, 4
QUANT_MAGIC = 0x51544355        # quantization_cuda.cuh:12
QUANT_VERSION = 1               # quantization_cuda.cuh:13
BLOCK = 64                      # quantization_cuda.cuh:10
FLT_EPSILON = np.float32(np.finfo(np.float32).eps)

HEADER_SIZE = 200
_HDR = struct.Struct("<HHIffhhhhiiiiI4x")          # 48 bytes, bitsqz_llm.hpp:55-73
_SEC = struct.Struct("<QQB7x")                     # 24 bytes, bitsqz_llm.hpp:48-53
_QHDR = struct.Struct("<IHHiIQQQfI")               # 48 bytes, quantization_cuda.cuh:15-26
_THDR = struct.Struct("<HHHH")                     # 8 bytes, topk_cuda.cuh:16-21
assert _HDR.size == 48 and _SEC.size == 24 and _QHDR.size == 48 and _THDR.size == 8

SECTION_NAMES = ("u", "s", "v", "direct", "outlier", "error")

# ---------------------------------------------------------------------------
# C restatement
# ---------------------------------------------------------------------------
_lib = None


def lib():
    global _lib
    if _lib is None:
        path = os.path.join(_HERE, "liboracle.so")
        if not os.path.exists(path):
            raise RuntimeError("oracle/liboracle.so missing: run `make -C oracle`")
        L = ctypes.CDLL(path)
        P, U64 = ctypes.c_void_p, ctypes.c_uint64
        L.oracle_nf4_code.restype = ctypes.c_uint8
        L.oracle_nf4_code.argtypes = [ctypes.c_float]
        L.oracle_e4m3_encode.restype = ctypes.c_uint8
        L.oracle_e4m3_encode.argtypes = [ctypes.c_float]
        L.oracle_e4m3_decode.restype = ctypes.c_float
        L.oracle_e4m3_decode.argtypes = [ctypes.c_uint8]
        L.oracle_nf4_compress.argtypes = [P, U64, P, P]
        L.oracle_nf4_decompress.argtypes = [P, P, U64, P]
        L.oracle_nf4dq_compress.argtypes = [P, U64, P, P, P]
        L.oracle_nf4dq_decompress.argtypes = [ctypes.c_float, P, P, U64, P]
        L.oracle_nf4_code_batch.argtypes = [P, U64, P]
        L.oracle_e4m3_encode_batch.argtypes = [P, U64, P]
        L.oracle_nf4_code_sweep.argtypes = [U64, U64, P, P]
        L.oracle_topk_rows.argtypes = [P, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32, P, P]
        L.oracle_topk_num_columns.restype = ctypes.c_int
        L.oracle_topk_num_columns.argtypes = [ctypes.c_uint16, ctypes.c_float]
        L.oracle_nf4_levels.restype = ctypes.POINTER(ctypes.c_float)
        L.oracle_nf4_threshold_mismatches.restype = ctypes.c_uint64
        L.oracle_nf4_threshold_mismatches.argtypes = [P, U64, U64]
        L.oracle_nf4_table_mismatches.restype = ctypes.c_uint64
        L.oracle_nf4_table_mismatches.argtypes = [P, U64, U64]
        _lib = L
    return _lib


def _p(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def nf4_levels() -> np.ndarray:
    ptr = lib().oracle_nf4_levels()
    return np.array([ptr[i] for i in range(16)], dtype=np.float32)


def nf4_codes(v: np.ndarray) -> np.ndarray:
    v = np.ascontiguousarray(v, dtype=np.float32)
    out = np.empty(v.size, np.uint8)
    lib().oracle_nf4_code_batch(_p(v), v.size, _p(out))
    return out


def e4m3_encode(v: np.ndarray) -> np.ndarray:
    v = np.ascontiguousarray(v, dtype=np.float32)
    out = np.empty(v.size, np.uint8)
    lib().oracle_e4m3_encode_batch(_p(v), v.size, _p(out))
    return out


def e4m3_decode_table() -> np.ndarray:
    return np.array([lib().oracle_e4m3_decode(i) for i in range(256)], dtype=np.float32)


def nf4_code_sweep(lo: int, hi: int):
    hist = np.zeros(16, np.uint64)
    cs = np.zeros(1, np.uint64)
    lib().oracle_nf4_code_sweep(lo, hi, _p(hist), _p(cs))
    return hist, int(cs[0])


def nf4_threshold_mismatches(thresholds: np.ndarray, lo: int = 0, hi: int = 1 << 32) -> int:
    """Floats with |v| < 2 in [lo, hi) where code = #{T <= v} differs from the scan."""
    t = np.ascontiguousarray(thresholds, dtype=np.float32)
    assert t.size == 15
    return int(lib().oracle_nf4_threshold_mismatches(_p(t), lo, hi))


def nf4_table_mismatches(thresholds: np.ndarray, lo: int = 0, hi: int = 1 << 32) -> int:
    """Floats with |v| < 2 in [lo, hi) where the device's 256-bin table rule
    differs from the scan."""
    t = np.ascontiguousarray(thresholds, dtype=np.float32)
    assert t.size == 15
    return int(lib().oracle_nf4_table_mismatches(_p(t), lo, hi))


@dataclass
class Quant:
    """One quantised section: reference quantization_cuda_array_t contents."""
    method: int
    count: int
    scales: np.ndarray          # f32 (NF4) or u8 E4M3 codes (NF4_DQ)
    codes: np.ndarray           # u8, ceil(count/2)
    dq: float = 0.0             # NF4_DQ global scale; 0.0 for NF4 (header field)


def quant_compress(x: np.ndarray, method: int) -> Quant:
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    n = x.size
    nb, nc = (n + BLOCK - 1) // BLOCK, (n + 1) // 2
    codes = np.zeros(nc, np.uint8)
    if method == NF4:
        scales = np.zeros(nb, np.float32)
        lib().oracle_nf4_compress(_p(x), n, _p(scales), _p(codes))
        return Quant(NF4, n, scales, codes, 0.0)
    if method == NF4_DQ:
        scales = np.zeros(nb, np.uint8)
        dq = np.zeros(1, np.float32)
        lib().oracle_nf4dq_compress(_p(x), n, _p(dq), _p(scales), _p(codes))
        return Quant(NF4_DQ, n, scales, codes, float(dq[0]))
    raise ValueError("unsupported method %r" % method)


def quant_decompress(q: Quant) -> np.ndarray:
    out = np.zeros(q.count, np.float32)
    if q.method == NF4:
        lib().oracle_nf4_decompress(_p(q.scales), _p(q.codes), q.count, _p(out))
    elif q.method == NF4_DQ:
        lib().oracle_nf4dq_decompress(ctypes.c_float(q.dq), _p(q.scales), _p(q.codes), q.count,
                                      _p(out))
    else:
        raise ValueError(q.method)
    return out


def topk_num_columns(cols: int, ratio: float) -> int:
    """topk_compute_num_topk_columns (topk_cuda.cu:53-69); -1 on a bad ratio."""
    return lib().oracle_topk_num_columns(cols, ctypes.c_float(ratio))


def topk_rows(x: np.ndarray, k: int):
    """Per-row top-k of |x| ordered (|x| desc, column asc), NaN ranked lowest
    (topk_cuda_utils.cuh:51-93 with CUB's stable descending sort)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, cols = x.shape
    idx = np.zeros((rows, k), np.uint16)
    val = np.zeros((rows, k), np.float32)
    if k:
        lib().oracle_topk_rows(_p(x), rows, cols, k, _p(idx), _p(val))
    return idx, val


# ---------------------------------------------------------------------------
# byte layouts
# ---------------------------------------------------------------------------
def quant_section_size(method: int, count: int) -> int:
    """quantization_cuda_get_packed_size_for_shape (quantization_cuda.cu:665-679)."""
    nb = (count + BLOCK - 1) // BLOCK
    return 48 + (nb * 4 if method == NF4 else nb) + (count + 1) // 2


def pack_quant(q: Quant) -> bytes:
    """quantization_cuda_pack_to_buffer (quantization_cuda.cu:736-807)."""
    nb = (q.count + BLOCK - 1) // BLOCK
    hdr = _QHDR.pack(QUANT_MAGIC, QUANT_VERSION, 0, q.method, 0, q.count, nb, BLOCK,
                     np.float32(q.dq if q.method == NF4_DQ else 0.0), 0)
    return hdr + q.scales.tobytes() + q.codes.tobytes()


def unpack_quant(buf: bytes) -> Quant:
    """quantization_cuda_validate_packed_buffer + unpack (quantization_cuda.cu:691-734, 809-876)."""
    if len(buf) < 48:
        raise ValueError("short quant section")
    magic, ver, _r0, method, _r1, count, nb, bs, dq, _r2 = _QHDR.unpack_from(buf, 0)
    if magic != QUANT_MAGIC or ver != QUANT_VERSION or method not in (NF4, NF4_DQ):
        raise ValueError("bad quant header")
    if count == 0 or bs != BLOCK or nb != (count + BLOCK - 1) // BLOCK:
        raise ValueError("bad quant shape")
    if len(buf) != quant_section_size(method, count):
        raise ValueError("bad quant size")
    ssz = nb * 4 if method == NF4 else nb
    sc = np.frombuffer(buf, np.float32 if method == NF4 else np.uint8, nb, 48).copy()
    codes = np.frombuffer(buf, np.uint8, (count + 1) // 2, 48 + ssz).copy()
    return Quant(method, count, sc, codes, float(dq))


def topk_blob_size(rows: int, cols: int, k: int) -> int:
    """topk_get_packed_size_for_shape (topk_cuda.cu:235-243)."""
    return 8 + rows * k * 6


def pack_topk(rows: int, cols: int, idx: np.ndarray, val: np.ndarray) -> bytes:
    """topk_pack_to_buffer (topk_cuda.cu:284-330)."""
    k = idx.shape[1] if idx.ndim == 2 else 0
    return (_THDR.pack(rows, cols, k, 0) + np.ascontiguousarray(idx, np.uint16).tobytes()
            + np.ascontiguousarray(val, np.float32).tobytes())


def unpack_topk(buf: bytes):
    """topk_validate_packed_buffer + unpack (topk_cuda.cu:255-282, 332-383)."""
    rows, cols, k, _ = _THDR.unpack_from(buf, 0)
    if rows == 0 or cols == 0 or k > cols or len(buf) != topk_blob_size(rows, cols, k):
        raise ValueError("bad top-k blob")
    idx = np.frombuffer(buf, np.uint16, rows * k, 8).reshape(rows, k).copy()
    val = np.frombuffer(buf, np.float32, rows * k, 8 + rows * k * 2).reshape(rows, k).copy()
    return rows, cols, k, idx, val


@dataclass
class Packed:
    rows: int
    cols: int
    outlier_ratio: float
    error_ratio: float
    svd_ranks: int
    svd_niters: int
    effective_rank: int
    uv_format: int
    s_format: int
    direct_format: int
    flags: int
    sections: dict = field(default_factory=dict)   # name -> (storage, bytes)

    def to_bytes(self, payload_pointer: int = 0) -> bytes:
        """Header + payload in the section order of src/bitsqz_llm.cu:1078-1247."""
        payload = bytearray()
        descs = []
        for name in SECTION_NAMES:
            if name in self.sections:
                storage, blob = self.sections[name]
                descs.append(_SEC.pack(len(payload), len(blob), storage))
                payload += blob
            else:
                descs.append(_SEC.pack(0, 0, SECTION_NONE))
        hdr = _HDR.pack(self.rows, self.cols, self.rows * self.cols,
                        np.float32(self.outlier_ratio), np.float32(self.error_ratio),
                        self.svd_ranks, self.svd_niters, self.effective_rank, 0,
                        self.uv_format, self.s_format, self.direct_format, 0, self.flags)
        out = hdr + b"".join(descs) + struct.pack("<Q", payload_pointer) + bytes(payload)
        assert len(out) == HEADER_SIZE + len(payload)
        return out


def parse_packed(buf: bytes) -> Packed:
    """Header fields + sections of a packed object (bitsqz_llm.hpp:55-83)."""
    (rows, cols, _n, ro, re, sr, sn, er, _r0, uvf, sf, df, _r1, flags) = _HDR.unpack_from(buf, 0)
    p = Packed(rows, cols, ro, re, sr, sn, er, uvf, sf, df, flags)
    payload = buf[HEADER_SIZE:]
    for i, name in enumerate(SECTION_NAMES):
        off, size, storage = _SEC.unpack_from(buf, 48 + 24 * i)
        if storage != SECTION_NONE:
            p.sections[name] = (storage, bytes(payload[off:off + size]))
    return p


_U64 = (1 << 64) - 1


def section_bounds_ok(offset: int, size: int, storage: int, payload_size: int) -> bool:
    """validate_section_bounds (src/bitsqz_llm.cu:319-332), u64 operands."""
    if storage == SECTION_NONE:
        return size == 0
    if size == 0 or offset > payload_size or size > payload_size - offset:
        return False
    return storage in (SECTION_FP32, SECTION_QUANT, SECTION_TOPK)


def packed_size(buf: bytes) -> int:
    """bitsqz_llm_get_packed_size (src/bitsqz_llm.cu:1395-1415): 200 + the largest
    offset + size of the non-NONE sections, summed in wrapping u64 arithmetic."""
    end = 0
    for i in range(6):
        off, size, storage = _SEC.unpack_from(buf, 48 + 24 * i)
        if storage != SECTION_NONE:
            end = max(end, (off + size) & _U64)
    return (HEADER_SIZE + end) & _U64


def load_accepts(buf: bytes) -> bool:
    """Whether load_bitsqz_llm_from_buffer accepts `buf` (src/bitsqz_llm.cu:
    1417-1450: at least a header, packed size within the buffer, every section
    inside the payload), plus the one check this build adds: the payload end is
    formed without wrapping and lies inside the buffer (the reference's wrapping
    sum accepts sections that end within 200 bytes of 2^64)."""
    n = len(buf)
    if n < HEADER_SIZE:
        return False
    packed = packed_size(buf)
    if packed == 0 or n < packed:
        return False
    payload = (packed - HEADER_SIZE) & _U64
    secs = [_SEC.unpack_from(buf, 48 + 24 * i) for i in range(6)]
    if not all(section_bounds_ok(off, size, st, payload) for off, size, st in secs):
        return False
    return all(st == SECTION_NONE or off + size <= n - HEADER_SIZE for off, size, st in secs)


def mask_pointer(buf: bytes) -> bytes:
    """Packed bytes with the process-address payload pointer (bytes 192-199) zeroed."""
    b = bytearray(buf)
    b[192:200] = b"\0" * 8
    return bytes(b)


# ---------------------------------------------------------------------------
# randomised SVD + reconstruction (float64 restatement)
# ---------------------------------------------------------------------------
def svd_work_shape(m: int, n: int, q: int):
    """configure_context (svd_lowrank_cuda.cu:129-137)."""
    k = max(1, min(q, m, n))
    transposed = m < n
    return k, transposed, (n if transposed else m), (m if transposed else n)


def normalize_signs(U: np.ndarray, V: np.ndarray):
    """Sign convention shared with the HIP library: flip each singular pair so
    that the entry of largest magnitude of the U column (first such row) is
    positive.  The reference's signs come from cusolverDnSgesvdj and cannot be
    reproduced; comparisons against it are sign-aligned anyway."""
    U = U.copy()
    V = V.copy()
    for j in range(U.shape[1]):
        i = int(np.argmax(np.abs(U[:, j])))
        if U[i, j] < 0:
            U[:, j] *= -1
            V[:, j] *= -1
    return U, V


def svd_lowrank(A: np.ndarray, q: int, niter: int, sketch: np.ndarray):
    """Rank-q randomised SVD with `niter` power iterations, QR after every
    product and no oversampling (svd_lowrank_cuda.cu:284-426, 478-524),
    evaluated in float64 with Householder QR (numpy).  `sketch` is the
    N_work x k Gaussian matrix (the reference draws it from cuRAND).
    Returns row-major U (m x k), S (k), V (n x k) in float64, signs
    normalised by normalize_signs."""
    m, n = A.shape
    k, transposed, Mw, Nw = svd_work_shape(m, n, q)
    Aw = (A.T if transposed else A).astype(np.float64)
    R = np.asarray(sketch, np.float64).reshape(Nw, k)
    X = Aw @ R
    Q, _ = np.linalg.qr(X)
    for _ in range(max(0, niter)):
        Qn, _ = np.linalg.qr(Aw.T @ Q)
        Q, _ = np.linalg.qr(Aw @ Qn)
    B = Q.T @ Aw                                     # k x Nw
    Uh, S, Vht = np.linalg.svd(B, full_matrices=False)
    Uw = Q @ Uh                                      # Mw x k
    Vh = Vht.T                                       # Nw x k
    U, V = (Vh, Uw) if transposed else (Uw, Vh)
    U, V = normalize_signs(U, V)
    return U, S, V


def reconstruct(U: np.ndarray, S: np.ndarray, V: np.ndarray) -> np.ndarray:
    """U diag(S) V^T (reconstruct_lowrank_cuda.cu:21-62), in float64."""
    U = np.asarray(U, np.float64)
    return (U * np.asarray(S, np.float64)[None, :]) @ np.asarray(V, np.float64).T


# ---------------------------------------------------------------------------
# whole pipeline (src/bitsqz_llm.cu:981-1393)
# ---------------------------------------------------------------------------
@dataclass
class Config:
    rows: int
    cols: int
    outlier_ratio: float = 0.0
    error_ratio: float = 0.0
    svd_ranks: int = -1
    svd_niters: int = 2
    uv_format: int = QUANT_NONE
    s_format: int = QUANT_NONE
    direct_format: int = QUANT_NONE

    @property
    def k_outlier(self):
        return topk_num_columns(self.cols, self.outlier_ratio)

    @property
    def k_error(self):
        return topk_num_columns(self.cols, self.error_ratio)


def _encode_section(x: np.ndarray, fmt: int):
    """append_quantized_section / append_dense_section_from_device
    (src/bitsqz_llm.cu:440-537): returns (storage, bytes, dequantised values
    as the decoder will see them)."""
    x = np.ascontiguousarray(x, np.float32).ravel()
    if fmt == QUANT_NONE:
        return SECTION_FP32, x.tobytes(), x.copy()
    q = quant_compress(x, fmt)
    return SECTION_QUANT, pack_quant(q), quant_decompress(q)


def compress(A: np.ndarray, cfg: Config, sketch: np.ndarray | None = None,
             svd_result=None) -> Packed:
    """bitsqz_llm_compress (src/bitsqz_llm.cu:981-1302).  For the SVD path
    pass `sketch` (the injected Gaussian matrix) or a precomputed
    `svd_result` = (U, S, V) float32 arrays."""
    A = np.ascontiguousarray(A, np.float32)
    m, n = A.shape
    assert (m, n) == (cfg.rows, cfg.cols)
    residual = A.copy()
    flags = 0
    p = Packed(m, n, cfg.outlier_ratio, cfg.error_ratio, cfg.svd_ranks, cfg.svd_niters, 0,
               cfg.uv_format, cfg.s_format, cfg.direct_format, 0)
    out_idx = out_val = None
    if cfg.outlier_ratio > 0.0:
        ko = cfg.k_outlier
        out_idx, out_val = topk_rows(residual, ko)
        rr = np.repeat(np.arange(m), ko)
        residual[rr, out_idx.ravel().astype(np.int64)] = 0.0
        if ko > 0:
            flags |= FLAG_OUTLIER
    approx = None
    if cfg.svd_ranks >= 1:
        flags |= FLAG_SVD
        q = max(1, min(cfg.svd_ranks, m, n))
        if svd_result is None:
            U, S, V = svd_lowrank(residual, q, cfg.svd_niters, sketch)
        else:
            U, S, V = svd_result
        U = np.asarray(U, np.float32)
        S = np.asarray(S, np.float32)
        V = np.asarray(V, np.float32)
        p.effective_rank = q
        su, bu, du = _encode_section(U, cfg.uv_format)
        ss, bs, ds = _encode_section(S, cfg.s_format)
        sv, bv, dv = _encode_section(V, cfg.uv_format)
        p.sections["u"] = (su, bu)
        p.sections["s"] = (ss, bs)
        p.sections["v"] = (sv, bv)
        if cfg.error_ratio > 0.0:
            approx = reconstruct(du.reshape(m, q), ds, dv.reshape(n, q)).astype(np.float32)
    else:
        sd, bd, dd = _encode_section(residual, cfg.direct_format)
        p.sections["direct"] = (sd, bd)
        if cfg.error_ratio > 0.0 and cfg.direct_format != QUANT_NONE:
            approx = dd.reshape(m, n)
    if out_idx is not None and (flags & FLAG_OUTLIER):
        p.sections["outlier"] = (SECTION_TOPK, pack_topk(m, n, out_idx, out_val))
    if approx is not None:
        err = residual - approx
        if np.any(np.abs(err) > FLT_EPSILON):
            ke = cfg.k_error
            ei, ev = topk_rows(err, ke)
            if ke > 0:
                flags |= FLAG_ERROR
                p.sections["error"] = (SECTION_TOPK, pack_topk(m, n, ei, ev))
    p.flags = flags
    return p


def _decode_dense(storage: int, blob: bytes, fmt: int, count: int) -> np.ndarray:
    if storage == SECTION_FP32:
        return np.frombuffer(blob, np.float32, count).copy()
    q = unpack_quant(blob)
    assert q.method == fmt and q.count == count
    return quant_decompress(q)


def decompress(p: Packed) -> np.ndarray:
    """bitsqz_llm_decompress (src/bitsqz_llm.cu:1304-1393): dense part, then
    error top-k, then outlier top-k, each added in float32."""
    m, n = p.rows, p.cols
    if p.flags & FLAG_SVD:
        q = p.effective_rank
        U = _decode_dense(*p.sections["u"], p.uv_format, m * q).reshape(m, q)
        S = _decode_dense(*p.sections["s"], p.s_format, q)
        V = _decode_dense(*p.sections["v"], p.uv_format, n * q).reshape(n, q)
        out = reconstruct(U, S, V).astype(np.float32)
    else:
        out = _decode_dense(*p.sections["direct"], p.direct_format, m * n).reshape(m, n)
    # scatter_add_topk_kernel (topk_cuda_utils.cuh:132-149) writes at the flat
    # position row * cols + index, so an index >= cols of a loaded object lands
    # in a later row; positions past the matrix (outside the reference's
    # buffer) are dropped here
    flat = out.reshape(-1)
    for name, flag in (("error", FLAG_ERROR), ("outlier", FLAG_OUTLIER)):
        if p.flags & flag:
            _, _, k, idx, val = unpack_topk(p.sections[name][1])
            pos = np.repeat(np.arange(m, dtype=np.int64), k) * n + idx.ravel().astype(np.int64)
            keep = pos < m * n
            np.add.at(flat, pos[keep], val.ravel()[keep])
    return out
