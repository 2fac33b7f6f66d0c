"""Shared helpers of the GPU tests of the SVD path: the BASELINE matrix
generators, an ABI round trip with an optional injected sketch, and the
section-by-section check of a packed object against the oracle."""
import numpy as np

import bitsqz_amd as B
from oracle import oracle as O


def rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


def align(U, V, Ur, Vr):
    """Flip columns of (U, V) to match the signs of (Ur, Vr)."""
    s = np.sign(np.sum(U.astype(np.float64) * Ur, axis=0))
    s[s == 0] = 1
    return U * s, V * s


def lowrank(m, n, r, decay, noise, seed=0):
    """A diag(sigma) B^T with Gaussian A (m x r), B (n x r), sigma_i = i^-decay,
    plus N(0, noise^2) (the BASELINE configs' generator)."""
    rng = np.random.default_rng(seed)
    A = rng.standard_normal((m, r)).astype(np.float32)
    Bm = rng.standard_normal((n, r)).astype(np.float32)
    sig = (np.arange(1, r + 1, dtype=np.float64) ** -decay).astype(np.float32)
    x = (A * sig) @ Bm.T
    if noise:
        x += np.float32(noise) * rng.standard_normal((m, n)).astype(np.float32)
    return np.ascontiguousarray(x, np.float32)


def outlier_columns(x, count, scale, seed=1):
    x[:, np.random.default_rng(seed).permutation(x.shape[1])[:count]] *= np.float32(scale)
    return x


def abi_round_trip(x, ro, re, q, it, uv, s, loc=B.INPUT_DEVICE, sketch=None):
    """bitsqz_llm_compress + bitsqz_llm_decompress of `x` through the ABI;
    `sketch` (min(m,n) x k) replaces the built-in Gaussian sketch."""
    rows, cols = x.shape
    B.compress_release()
    B.decompress_release()
    assert B.compress_initialize(rows, cols, ro, re, q, it, uv, s, B.QUANT_NONE, loc) == 0, \
        B.lib().bsq_last_error()
    kq = max(1, min(q, rows, cols))
    assert B.decompress_initialize(rows, cols, ro, re, kq, uv, s, B.QUANT_NONE) == 0
    dsk = None
    if sketch is not None:
        dsk = B.DeviceBuffer.from_array(np.ascontiguousarray(sketch, np.float32))
        assert B.lib().bsq_compress_set_sketch(dsk.ptr) == 0
    src = B.DeviceBuffer.from_array(x) if loc == B.INPUT_DEVICE else x
    data = B.compress(src)
    del src
    out = B.decompress(data, rows, cols)
    if dsk is not None:
        B.lib().bsq_compress_set_sketch(None)
    return data, out


def check_sections(x, data, out, ro, re, q, uv, s, factors=None):
    """Every section except the SVD factors' values is checked bit for bit:
    the outlier section is the oracle top-k of x; U/S/V sections re-pack
    exactly; when `factors` (the same SVD computed standalone) is given, the
    U/S/V sections equal the oracle's encoding of those factors; the error
    section is the oracle top-k of residual - (GPU reconstruction of the
    decoded factors); the decode equals that reconstruction plus the error
    set, then the outlier set.  Returns the decoded (U, S, V), the residual
    and the reconstruction."""
    rows, cols = x.shape
    p = O.parse_packed(data)
    k = p.effective_rank
    assert k == max(1, min(q, rows, cols)) and (p.flags & O.FLAG_SVD)
    dec = {}
    for i, (name, fmt, cnt) in enumerate((("u", uv, rows * k), ("s", s, k), ("v", uv, cols * k))):
        storage, blob = p.sections[name]
        if factors is not None:
            st, b, _ = O._encode_section(factors[i], fmt)
            assert storage == st and blob == b, f"section {name} differs from the oracle encoding"
        if fmt == O.QUANT_NONE:
            assert storage == O.SECTION_FP32
            dec[name] = np.frombuffer(blob, np.float32).copy()
        else:
            qz = O.unpack_quant(blob)
            assert O.pack_quant(qz) == blob
            dec[name] = O.quant_decompress(qz)
    U, S, V = dec["u"].reshape(rows, k), dec["s"], dec["v"].reshape(cols, k)
    residual = x.copy()
    if ro > 0:
        ko = O.topk_num_columns(cols, ro)
        oi, ov = O.topk_rows(x, ko)
        assert p.sections["outlier"][1] == O.pack_topk(rows, cols, oi, ov)
        np.put_along_axis(residual, oi.astype(np.int64), 0.0, axis=1)
    recon = B.reconstruct(U, S, V)
    err = residual - recon
    expect = recon.copy()
    if re > 0 and np.any(np.abs(err) > O.FLT_EPSILON):
        ke = O.topk_num_columns(cols, re)
        ei, ev = O.topk_rows(err, ke)
        assert p.flags & O.FLAG_ERROR
        assert p.sections["error"][1] == O.pack_topk(rows, cols, ei, ev)
        rr = np.repeat(np.arange(rows), ke)
        expect[rr, ei.astype(np.int64).ravel()] += ev.ravel()
    else:
        assert not (p.flags & O.FLAG_ERROR)
    if ro > 0:
        expect[np.repeat(np.arange(rows), ko), oi.astype(np.int64).ravel()] += ov.ravel()
    assert out.tobytes() == expect.tobytes()
    return (U, S, V), residual, recon
