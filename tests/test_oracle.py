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
