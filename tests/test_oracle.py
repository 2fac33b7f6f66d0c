"""Pins the CPU oracle (oracle/bsq_oracle.c + oracle/oracle.py).

Every oracle function used as a checker is tested here against something that
is not the oracle itself: the golden vectors written by the reference's own
legacy codec (tests/golden/gen_golden.py), the reference's top-k known-answer
tests, closed forms and brute force.
"""
import math
import struct

import numpy as np
import pytest

from oracle import oracle as O


# --------------------------------------------------------------------- NF4 --
@pytest.mark.parametrize("name", ["edge", "unif"])
def test_nf4_matches_reference_codec(golden, name):
    g = golden["nf4"]
    x = g["nf4_%s_x" % name]
    q = O.quant_compress(x, O.NF4)
    assert q.scales.tobytes() == g["nf4_%s_scales" % name].tobytes()
    assert q.codes.tobytes() == g["nf4_%s_codes" % name].tobytes()
    assert O.quant_decompress(q).tobytes() == g["nf4_%s_out" % name].tobytes()


@pytest.mark.parametrize("name", ["edge", "unif"])
def test_nf4dq_matches_reference_codec(golden, name):
    g = golden["nf4"]
    x = g["nf4dq_%s_x" % name]
    q = O.quant_compress(x, O.NF4_DQ)
    assert np.float32(q.dq).tobytes() == g["nf4dq_%s_dq" % name].tobytes()
    assert q.scales.tobytes() == g["nf4dq_%s_scales" % name].tobytes()
    assert q.codes.tobytes() == g["nf4dq_%s_codes" % name].tobytes()
    assert O.quant_decompress(q).tobytes() == g["nf4dq_%s_out" % name].tobytes()


def test_e4m3_probes_match_reference(golden):
    g = golden["nf4"]
    assert O.e4m3_encode(g["e4m3_probe_x"]).tobytes() == g["e4m3_probe_code"].tobytes()


def test_e4m3_decode_closed_form():
    """E4M3 decode = (-1)^s * (ef ? (1+m/8) 2^(ef-7) : (m/8) 2^-6), 0x7F -> 480."""
    t = O.e4m3_decode_table()
    for c in range(256):
        s, ef, mf = c >> 7, (c >> 3) & 15, c & 7
        v = (1 + mf / 8) * 2.0 ** (ef - 7) if ef else (mf / 8) * 2.0 ** -6
        assert t[c] == np.float32(-v if s else v), c
    assert t[0x7F] == 480.0


def test_e4m3_encode_round_trips_representable_values():
    """Every non-negative representable value up to 448 encodes to its own code
    (up to the sub-normal mantissa clamp at 7 and +0)."""
    t = O.e4m3_decode_table()
    codes = np.arange(1, 0x7F, dtype=np.uint8)
    vals = t[codes]
    enc = O.e4m3_encode(vals)
    keep = vals <= 448.0
    assert np.array_equal(enc[keep], codes[keep])


def test_nf4_code_is_first_nearest_level():
    """Brute force with exact (float64) distances: the code is the nearest
    level, and on exact float32 ties the lower index."""
    rng = np.random.default_rng(1)
    lv = O.nf4_levels()
    v = np.concatenate([rng.uniform(-1.2, 1.2, 20000), (lv[:-1] + lv[1:]) / 2]).astype(np.float32)
    codes = O.nf4_codes(v)
    for x, c in zip(v, codes):
        e = np.abs(np.float32(x) - lv)         # float32 subtraction, as the codec
        assert c == int(np.argmin(e)), (x, c)  # argmin -> first minimum


def test_nf4_code_nonfinite_maps_to_zero_level():
    v = np.array([np.nan, np.inf, -np.inf, 0.0, -0.0], np.float32)
    assert list(O.nf4_codes(v)) == [7, 7, 7, 7, 7]


def test_nf4_code_sweep_partitions():
    """The sweep helper used by the GPU exhaustive test counts every pattern."""
    hist, cs = O.nf4_code_sweep(0x3F000000, 0x3F000000 + 4096)
    assert int(hist.sum()) == 4096 and cs > 0


# ------------------------------------------------------------------- top-k --
@pytest.mark.parametrize("name", ["extract", "sep0", "sep001", "sep1", "pack", "ties"])
def test_topk_known_answers(golden, name):
    g = golden["topk"]
    x = g[name + "_x"]
    k = int(g[name + "_k"][0])
    assert O.topk_num_columns(x.shape[1], float(g[name + "_ratio"][0])) == k
    idx, val = O.topk_rows(x, k)
    assert np.array_equal(idx, g[name + "_idx"])
    assert val.tobytes() == g[name + "_val"].tobytes()


def test_topk_extraction_sets_from_reference_test(golden):
    g = golden["topk"]
    idx, _ = O.topk_rows(g["extract_x"], 3)
    for r in range(3):
        assert set(idx[r].tolist()) == set(g["extract_sets"][r].tolist())


def test_topk_num_columns_cases(golden):
    g = golden["topk"]
    for (c, k), r in zip(g["k_cases"], g["k_ratios"]):
        assert O.topk_num_columns(int(c), float(r)) == int(k), (c, r)
    assert O.topk_num_columns(10, -0.1) == -1
    assert O.topk_num_columns(10, float("nan")) == -1
    assert O.topk_num_columns(10, 1.5) == -1


def test_topk_brute_force_random():
    rng = np.random.default_rng(7)
    x = rng.standard_normal((37, 129)).astype(np.float32)
    x[:, 5] = x[:, 6]                      # ties
    x[3, 10] = np.nan
    x[4, :] = 0.0
    k = 17
    idx, val = O.topk_rows(x, k)
    for r in range(x.shape[0]):
        keys = [(-math.inf if math.isnan(abs(float(a))) else abs(float(a))) for a in x[r]]
        order = sorted(range(x.shape[1]), key=lambda c: (-keys[c], c))
        assert idx[r].tolist() == order[:k]
        assert val[r].tobytes() == x[r, order[:k]].tobytes()


# ----------------------------------------------------------------- layouts --
def test_header_layout_offsets():
    p = O.Packed(3, 5, 0.25, 0.5, 7, 2, 7, O.NF4, O.QUANT_NONE, O.NF4_DQ, 5)
    p.sections["u"] = (O.SECTION_QUANT, b"\1" * 11)
    p.sections["error"] = (O.SECTION_TOPK, b"\2" * 14)
    b = p.to_bytes(payload_pointer=0x1122334455667788)
    assert len(b) == 200 + 25
    assert struct.unpack_from("<HHI", b, 0) == (3, 5, 15)
    assert struct.unpack_from("<ff", b, 8) == (0.25, 0.5)
    assert struct.unpack_from("<hhhh", b, 16) == (7, 2, 7, 0)
    assert struct.unpack_from("<iiiiI", b, 24) == (O.NF4, -1, O.NF4_DQ, 0, 5)
    assert b[44:48] == b"\0\0\0\0"
    assert struct.unpack_from("<QQB", b, 48) == (0, 11, O.SECTION_QUANT)       # section_u
    assert struct.unpack_from("<QQB", b, 168) == (11, 14, O.SECTION_TOPK)      # section_error
    assert struct.unpack_from("<Q", b, 192)[0] == 0x1122334455667788
    q = O.parse_packed(b)
    assert q.sections["u"][1] == b"\1" * 11 and q.sections["error"][1] == b"\2" * 14


def test_quant_section_round_trip():
    rng = np.random.default_rng(3)
    for method in (O.NF4, O.NF4_DQ):
        for n in (1, 63, 64, 65, 1001):
            q = O.quant_compress(rng.standard_normal(n).astype(np.float32), method)
            blob = O.pack_quant(q)
            assert len(blob) == O.quant_section_size(method, n)
            r = O.unpack_quant(blob)
            assert r.scales.tobytes() == q.scales.tobytes() and r.codes.tobytes() == q.codes.tobytes()
            assert np.float32(r.dq) == np.float32(q.dq)


def test_section_sizes_of_configs():
    """Appendix sizes: C1 direct NF4 section and C2 NF4_DQ + outlier blob."""
    assert O.quant_section_size(O.NF4, 2048 * 4096) == 4718640
    assert O.quant_section_size(O.NF4_DQ, 4096 * 4096) == 8650800
    assert O.topk_blob_size(4096, 4096, 20) == 491528


# --------------------------------------------------------------------- SVD --
def _lowrank(m, n, r, seed, decay=1.0, noise=0.0):
    rng = np.random.default_rng(seed)
    a = rng.standard_normal((m, r))
    b = rng.standard_normal((n, r))
    s = np.arange(1, r + 1, dtype=np.float64) ** -decay
    A = (a * s) @ b.T
    if noise:
        A = A + noise * rng.standard_normal((m, n))
    return A.astype(np.float32)


@pytest.mark.parametrize("shape", [(96, 160), (160, 96)])
def test_svd_exact_low_rank_recovery(shape):
    """q >= rank(A): the randomised SVD is exact (as the reference's own test
    builds exact rank-32 inputs, test_svd_lowrank_cuda.cu:70-84)."""
    m, n = shape
    A = _lowrank(m, n, 8, 0)
    rng = np.random.default_rng(1)
    k = 12
    R = rng.standard_normal((min(m, n), k))
    U, S, V = O.svd_lowrank(A, k, 1, R)
    rec = O.reconstruct(U, S, V)
    assert np.linalg.norm(rec - A) / np.linalg.norm(A) < 1e-6
    assert np.allclose(U.T @ U, np.eye(k), atol=1e-10)
    assert np.allclose(V.T @ V, np.eye(k), atol=1e-10)
    assert np.all(np.diff(S) <= 0) and np.all(S >= 0)
    dense = np.linalg.svd(A.astype(np.float64), compute_uv=False)[:8]
    assert np.allclose(S[:8], dense, rtol=1e-9)


def test_svd_converged_matches_dense_svd():
    """With a large spectral gap and enough power iterations the leading
    triplets equal numpy's dense SVD (signs normalised)."""
    m, n, k = 120, 200, 6
    rng = np.random.default_rng(5)
    a, _ = np.linalg.qr(rng.standard_normal((m, k)))
    b, _ = np.linalg.qr(rng.standard_normal((n, k)))
    s = np.array([50, 40, 30, 20, 10, 5], np.float64)
    A = (a * s) @ b.T + 1e-3 * rng.standard_normal((m, n))
    R = rng.standard_normal((min(m, n), k))
    U, S, V = O.svd_lowrank(A, k, 4, R)
    Ud, Sd, Vdt = np.linalg.svd(A)
    Ud, Vd = O.normalize_signs(Ud[:, :k], Vdt[:k].T)
    assert np.allclose(S, Sd[:k], rtol=1e-6)
    assert np.allclose(U, Ud, atol=1e-5) and np.allclose(V, Vd, atol=1e-5)


def test_svd_reconstruction_is_projection():
    """U S V^T = Q Q^T A_w (basis invariance) -- the property the GPU
    reconstruction is compared on."""
    A = _lowrank(64, 100, 30, 9, decay=0.5, noise=0.01).astype(np.float64)
    rng = np.random.default_rng(2)
    k = 10
    R = rng.standard_normal((64, k))
    U, S, V = O.svd_lowrank(A, k, 2, R)
    Aw = A.T
    Q, _ = np.linalg.qr(Aw @ R)
    for _ in range(2):
        Qn, _ = np.linalg.qr(Aw.T @ Q)
        Q, _ = np.linalg.qr(Aw @ Qn)
    proj = (Q @ (Q.T @ Aw)).T
    assert np.allclose(O.reconstruct(U, S, V), proj, atol=1e-9)


@pytest.mark.parametrize("shape", [(40, 60), (60, 40)])
@pytest.mark.parametrize("it", [0, 1, 2])
def test_svd_iteration_semantics_closed_form(shape, it):
    """The oracle's range-finder basis spans orth((A_w A_w^T)^it A_w R), with
    A_w = A for m >= n and A^T for m < n (svd_lowrank_cuda.cu:129-137,
    284-386): its projector equals the one of that product formed directly in
    float64, with no intermediate QR, on a spectrum mild enough that the
    direct power is well conditioned.  The same check against it - 1 and
    it + 1 iterations and against the sketch applied on the other side shows
    the case tells those apart."""
    m, n = shape
    k, r = 8, 30
    rng = np.random.default_rng(m * 7 + it)
    a, _ = np.linalg.qr(rng.standard_normal((m, r)))
    b, _ = np.linalg.qr(rng.standard_normal((n, r)))
    A = (a * (0.85 ** np.arange(r))) @ b.T
    transposed = m < n
    Aw = A.T if transposed else A
    R = rng.standard_normal((min(m, n), k))
    U, S, V = O.svd_lowrank(A, k, it, R)
    basis = V if transposed else U  # U_w = Q U_hat: the range-finder basis, in A_w's row space

    def projector(Y):
        Y = np.asarray(Y, np.float64)
        return Y @ np.linalg.solve(Y.T @ Y, Y.T)

    def direct(p):
        Y = Aw @ R
        for _ in range(p):
            Y = Aw @ (Aw.T @ Y)
        return projector(Y)

    P = basis @ basis.T
    assert np.linalg.norm(P - direct(it)) < 1e-9
    for p in (it - 1, it + 1):
        if p >= 0:
            assert np.linalg.norm(P - direct(p)) > 1e-3
    # the sketch on the other side: A_w^T R' spans a subspace of the other
    # dimension; its row-space image A_w (A_w^T R') is a different subspace
    Rw = rng.standard_normal((Aw.shape[0], k))
    assert np.linalg.norm(P - projector(Aw @ (Aw.T @ Rw))) > 1e-3


# ---------------------------------------------------------------- pipeline --
def test_pipeline_direct_round_trip():
    rng = np.random.default_rng(11)
    A = rng.standard_normal((16, 128)).astype(np.float32)
    A[:, 7] *= 60
    cfg = O.Config(16, 128, outlier_ratio=0.02, error_ratio=0.05, direct_format=O.NF4_DQ)
    p = O.compress(A, cfg)
    assert p.flags == (O.FLAG_OUTLIER | O.FLAG_ERROR)
    b = p.to_bytes()
    out = O.decompress(O.parse_packed(b))
    err = np.abs(out - A)
    # the outliers are stored exactly
    assert np.all(err[:, 7] == 0)
    assert np.linalg.norm(err) / np.linalg.norm(A) < 0.1


def test_pipeline_dense_direct_is_exact():
    rng = np.random.default_rng(12)
    A = rng.standard_normal((8, 64)).astype(np.float32)
    p = O.compress(A, O.Config(8, 64, error_ratio=0.1))
    assert p.flags == 0            # dense section: no error extraction
    assert np.array_equal(O.decompress(p), A)


# ------------------------------------------------- pipeline composition pins --
# These pin oracle.compress / oracle.decompress (the restatement of
# src/bitsqz_llm.cu:981-1393) with checks that do not reuse the oracle's own
# pipeline code: the top-k is recomputed with numpy's stable sort, and the
# decoded values are written as explicit float32 operations.  A swapped apply
# order, an error measured against the raw residual, a `>=` FLT_EPSILON gate
# or a misplaced section each fail one of them.
def _stable_topk(err: np.ndarray, k: int):
    """Per row the k largest |err| (ties to the lower column) by numpy's
    stable sort: an independent brute force of topk_cuda_utils.cuh:51-93."""
    key = np.abs(err.astype(np.float32))
    key = np.where(np.isnan(key), -np.inf, key)
    order = np.argsort(-key, axis=1, kind="stable")[:, :k]
    return order.astype(np.uint16), np.take_along_axis(err, order, axis=1).astype(np.float32)


def _sections(p: "O.Packed", buf: bytes):
    """(name -> (offset, size)) read back from the serialized header."""
    out = {}
    for i, name in enumerate(O.SECTION_NAMES):
        off, size, st = struct.unpack_from("<QQB", buf, 48 + 24 * i)
        if st:
            out[name] = (off, size, st)
    return out


@pytest.mark.parametrize("method", [O.NF4, O.NF4_DQ])
def test_composition_direct_error_is_topk_of_residual_minus_dequant(method):
    """Direct path (src/bitsqz_llm.cu:1183-1227): the error section holds the
    k_e largest |x - deq(x)| per row, and the decode there is
    fl(deq + fl(x - deq)) -- the residual minus the *dequantised* section."""
    rng = np.random.default_rng(21)
    rows, cols = 12, 320
    x = rng.standard_normal((rows, cols)).astype(np.float32)
    cfg = O.Config(rows, cols, error_ratio=0.05, direct_format=method)
    ke = O.topk_num_columns(cols, 0.05)
    p = O.compress(x, cfg)
    deq = O.quant_decompress(O.quant_compress(x, method)).reshape(rows, cols)
    err = (x - deq).astype(np.float32)
    ei, ev = _stable_topk(err, ke)
    assert p.flags == O.FLAG_ERROR
    assert p.sections["error"][1] == struct.pack("<HHHH", rows, cols, ke, 0) + ei.tobytes() + ev.tobytes()
    out = O.decompress(O.parse_packed(p.to_bytes()))
    expect = deq.copy()
    for r in range(rows):
        for j in range(ke):
            c = int(ei[r, j])
            expect[r, c] = np.float32(deq[r, c] + np.float32(x[r, c] - deq[r, c]))
    assert out.tobytes() == expect.tobytes()
    # section order: direct first, then the error blob, no gaps
    secs = _sections(p, p.to_bytes())
    assert secs["direct"][0] == 0 and secs["error"][0] == secs["direct"][1]


def test_composition_outliers_are_exact_and_zeroed_before_quantisation():
    """Outliers are the k_o largest |x| per row; they are zeroed in the
    residual before the direct section is encoded, and decode to x exactly."""
    rng = np.random.default_rng(22)
    rows, cols = 8, 256
    x = rng.standard_normal((rows, cols)).astype(np.float32)
    x[:, 17] *= 80.0
    x[3, 200] = -900.0
    ko = O.topk_num_columns(cols, 0.01)
    p = O.compress(x, O.Config(rows, cols, outlier_ratio=0.01, error_ratio=0.02, direct_format=O.NF4))
    oi, ov = _stable_topk(x, ko)
    assert p.sections["outlier"][1] == struct.pack("<HHHH", rows, cols, ko, 0) + oi.tobytes() + ov.tobytes()
    residual = x.copy()
    np.put_along_axis(residual, oi.astype(np.int64), 0.0, axis=1)
    q = O.quant_compress(residual, O.NF4)
    assert p.sections["direct"][1] == O.pack_quant(q)
    out = O.decompress(O.parse_packed(p.to_bytes()))
    assert np.array_equal(np.take_along_axis(out, oi.astype(np.int64), axis=1), ov)
    secs = _sections(p, p.to_bytes())
    assert secs["direct"][0] == 0
    assert secs["outlier"][0] == secs["direct"][1]
    assert secs["error"][0] == secs["outlier"][0] + secs["outlier"][1]


def test_composition_error_then_outlier_apply_order():
    """src/bitsqz_llm.cu:1373-1387 adds the error set before the outlier set.
    Crafted so the two orders round differently: at column 0 the outlier is
    2^24, the reconstruction 1 and the error -1; error first gives
    (1 + -1) + 2^24 = 2^24, outlier first gives (1 + 2^24) - 1 = 2^24 - 1."""
    x = np.ones((1, 8), np.float32)
    x[0, 0] = np.float32(2.0 ** 24)
    U = np.ones((1, 1), np.float32)
    S = np.ones(1, np.float32)
    V = np.ones((8, 1), np.float32)
    cfg = O.Config(1, 8, outlier_ratio=0.125, error_ratio=0.125, svd_ranks=1, svd_niters=1)
    p = O.compress(x, cfg, svd_result=(U, S, V))
    _, _, ko, oi, ov = O.unpack_topk(p.sections["outlier"][1])
    _, _, ke, ei, ev = O.unpack_topk(p.sections["error"][1])
    assert (ko, int(oi[0, 0]), float(ov[0, 0])) == (1, 0, 2.0 ** 24)
    # the residual is 0 at the outlier, the reconstruction 1: error -1 there
    assert (ke, int(ei[0, 0]), float(ev[0, 0])) == (1, 0, -1.0)
    out = O.decompress(O.parse_packed(p.to_bytes()))
    error_first = np.float32(np.float32(np.float32(1.0) + np.float32(-1.0)) + np.float32(2.0 ** 24))
    outlier_first = np.float32(np.float32(np.float32(1.0) + np.float32(2.0 ** 24)) + np.float32(-1.0))
    assert error_first != outlier_first
    assert out[0, 0] == error_first
    assert np.all(out[0, 1:] == 1.0)


def test_composition_svd_error_uses_dequantised_factors():
    """With quantised U/V the error is measured against the reconstruction of
    the *dequantised* factors (src/bitsqz_llm.cu:1078-1163, 506-512)."""
    rng = np.random.default_rng(23)
    rows, cols, q = 16, 96, 4
    U = rng.standard_normal((rows, q)).astype(np.float32)
    S = np.array([4.0, 3.0, 2.0, 1.0], np.float32)
    V = rng.standard_normal((cols, q)).astype(np.float32)
    x = ((U * S) @ V.T).astype(np.float32)
    cfg = O.Config(rows, cols, error_ratio=0.05, svd_ranks=q, svd_niters=1, uv_format=O.NF4)
    p = O.compress(x, cfg, svd_result=(U, S, V))
    du = O.quant_decompress(O.quant_compress(U, O.NF4)).reshape(rows, q).astype(np.float64)
    dv = O.quant_decompress(O.quant_compress(V, O.NF4)).reshape(cols, q).astype(np.float64)
    approx = ((du * S.astype(np.float64)) @ dv.T).astype(np.float32)
    ke = O.topk_num_columns(cols, 0.05)
    ei, ev = _stable_topk((x - approx).astype(np.float32), ke)
    assert p.sections["error"][1] == struct.pack("<HHHH", rows, cols, ke, 0) + ei.tobytes() + ev.tobytes()
    # U, S, V sections in that order at the front of the payload
    secs = _sections(p, p.to_bytes())
    assert secs["u"][0] == 0 and secs["s"][0] == secs["u"][1] and secs["v"][0] == secs["s"][0] + secs["s"][1]


@pytest.mark.parametrize("bump,present", [(False, False), (True, True)])
def test_composition_flt_epsilon_gate(bump, present):
    """The error top-k runs only if some |err| > FLT_EPSILON (strictly;
    src/bitsqz_llm.cu:175-184, 410).  A block holding 1.0 has scale 1, so an
    entry of FLT_EPSILON quantises to level 0 and leaves an error of exactly
    FLT_EPSILON (no error section); the next float up leaves one."""
    x = np.zeros((2, 64), np.float32)
    x[:, 0] = 1.0
    e = np.float32(O.FLT_EPSILON)
    x[1, 5] = np.nextafter(e, np.float32(1.0)) if bump else e
    p = O.compress(x, O.Config(2, 64, error_ratio=0.05, direct_format=O.NF4))
    deq = O.quant_decompress(O.quant_compress(x, O.NF4)).reshape(2, 64)
    assert deq[1, 5] == 0.0 and np.float32(x[1, 5] - deq[1, 5]) == x[1, 5]
    assert bool(p.flags & O.FLAG_ERROR) == present
    assert ("error" in p.sections) == present


@pytest.mark.parametrize("dq", [0.0, -0.0, float("nan"), float("inf"), float("-inf"), 1e-45])
def test_nf4dq_decode_guards_dq_like_the_device_decoder(dq):
    """quantization_cuda.cu:322-327: a dq of 0 or non-finite decodes as 1;
    any other value (a subnormal included) is used as it is."""
    rng = np.random.default_rng(24)
    x = rng.standard_normal(200).astype(np.float32)
    q = O.quant_compress(x, O.NF4_DQ)
    q.dq = dq
    out = O.quant_decompress(q)
    eff = np.float32(1.0) if (dq == 0.0 or not math.isfinite(dq)) else np.float32(dq)
    lv = O.nf4_levels()
    e4 = O.e4m3_decode_table()
    expect = np.empty(200, np.float32)
    for i in range(200):
        s = np.float32(eff * e4[q.scales[i // 64]])
        if s == 0.0 or not np.isfinite(s):
            s = np.float32(1.0)
        c = (q.codes[i // 2] >> 4) if i % 2 == 0 else (q.codes[i // 2] & 15)
        expect[i] = np.float32(s * lv[c])
    assert out.tobytes() == expect.tobytes()


def test_decompress_wide_index_flat_position():
    """An index >= cols adds at row * cols + index (topk_cuda_utils.cuh:
    132-149); one past the end of the matrix is dropped."""
    rows, cols = 3, 64
    p = O.Packed(rows, cols, 1.0 / 64, 0.0, -1, 2, 0, O.QUANT_NONE, O.QUANT_NONE, O.QUANT_NONE, O.FLAG_OUTLIER)
    p.sections["direct"] = (O.SECTION_FP32, np.zeros(rows * cols, np.float32).tobytes())
    idx = np.array([[cols + 3], [5], [cols + 1]], np.uint16)
    val = np.array([[2.5], [4.0], [9.0]], np.float32)
    p.sections["outlier"] = (O.SECTION_TOPK, O.pack_topk(rows, cols, idx, val))
    out = O.decompress(O.parse_packed(p.to_bytes()))
    expect = np.zeros((rows, cols), np.float32)
    expect[1, 3] = 2.5
    expect[1, 5] = 4.0
    assert np.array_equal(out, expect)
