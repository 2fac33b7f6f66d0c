"""Randomised SVD, reconstruction and the SVD path of the pipeline on the GPU.

Parity is defined with the sketch injected (the reference draws it from
cuRAND, modules/svd_lowrank_cuda/src/svd_lowrank_cuda.cu:289-291): U, S, V are
compared with the FP64 oracle restatement (oracle/oracle.py svd_lowrank, the
algorithm of svd_lowrank_cuda.cu:284-426) after sign alignment, and the
reconstructions U diag(S) V^T are compared directly.  Tolerances (relative
Frobenius) are written per test; the bar is 1e-4 on the reconstruction."""
import numpy as np
import pytest

import bitsqz_amd as B
from oracle import oracle as O

pytestmark = pytest.mark.gpu


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
    rng = np.random.default_rng(seed)
    A = rng.standard_normal((m, r)).astype(np.float32)
    Bm = rng.standard_normal((n, r)).astype(np.float32)
    sig = (np.arange(1, r + 1, dtype=np.float64) ** -decay).astype(np.float32)
    x = (A * sig) @ Bm.T
    if noise:
        x += noise * rng.standard_normal((m, n)).astype(np.float32)
    return np.ascontiguousarray(x, np.float32)


@pytest.mark.parametrize("m,n,k", [(256, 384, 64), (100, 37, 5), (1000, 513, 130), (33, 2000, 17)])
def test_reconstruct_matches_fp64(m, n, k):
    rng = np.random.default_rng(m + n + k)
    U = rng.standard_normal((m, k)).astype(np.float32)
    S = rng.random(k).astype(np.float32)
    V = rng.standard_normal((n, k)).astype(np.float32)
    out = B.reconstruct(U, S, V)
    ref = O.reconstruct(U, S, V)
    assert rel(out, ref) < 2e-6


def test_gaussian_sketch_moments_and_determinism():
    a = B.gaussian(1 << 20, 1234)
    b = B.gaussian(1 << 20, 1234)
    c = B.gaussian(1 << 20, 1241)
    assert np.array_equal(a, b) and not np.array_equal(a, c)
    assert abs(a.mean()) < 5e-3 and abs(a.var() - 1.0) < 1e-2
    assert abs(np.mean(a ** 4) - 3.0) < 0.05


@pytest.mark.parametrize("m,n", [(512, 2048), (2048, 512)])
def test_exact_low_rank_recovery(m, n):
    """Rank-32 input with q = 64 and 2 iterations (the reference's own SVD
    test shape family, tests/svd_lowrank_cuda/test_svd_lowrank_cuda.cu:70-128):
    U S V^T reproduces A, U and V have orthonormal columns on the signal part."""
    A = lowrank(m, n, 32, 0.0, 0.0, seed=m)
    U, S, V = B.svd_lowrank(A, 64, 2)
    assert np.all(np.diff(S) <= 0)
    assert rel(O.reconstruct(U, S, V), A) < 1e-5
    Us, Vs = U[:, :32].astype(np.float64), V[:, :32].astype(np.float64)
    assert np.abs(Us.T @ Us - np.eye(32)).max() < 1e-5
    assert np.abs(Vs.T @ Vs - np.eye(32)).max() < 1e-5


@pytest.mark.parametrize("m,n,q,it,decay", [(1024, 2752, 128, 2, 1.2), (2752, 1024, 64, 1, 1.0),
                                          (777, 1500, 40, 3, 0.8), (600, 600, 100, 0, 1.2),
                                          # ranks that leave padding inside the 16 x 16 tiles of
                                          # the Cholesky kernel (47) and a single padded block (1)
                                          (300, 500, 47, 2, 1.2), (90, 64, 1, 2, 1.0)])
def test_svd_matches_oracle_with_injected_sketch(m, n, q, it, decay):
    A = lowrank(m, n, 512 if min(m, n) > 512 else min(m, n), decay, 0.01, seed=q)
    k = max(1, min(q, m, n))
    R = np.random.default_rng(3).standard_normal((min(m, n), k)).astype(np.float32)
    U, S, V = B.svd_lowrank(A, q, it, sketch=R)
    Ur, Sr, Vr = O.svd_lowrank(A, q, it, R)
    U, V = align(U, V, Ur, Vr)
    # reconstruction
    assert rel(O.reconstruct(U, S, V), O.reconstruct(Ur, Sr, Vr)) < 1e-4
    assert rel(S, Sr) < 1e-5
    # factors, sign-aligned, relative Frobenius over the whole matrix
    assert rel(U, Ur) < 1e-3
    assert rel(V, Vr) < 1e-3
    assert np.abs(U.astype(np.float64).T @ U - np.eye(k)).max() < 1e-4


@pytest.mark.parametrize("m,n,q,r", [(1200, 700, 300, 120), (900, 2000, 512, 200), (600, 400, 257, 257)])
def test_two_level_cholesky_low_rank_recovery(m, n, q, r):
    """Ranks 257 .. 512 orthonormalise with the two-level Cholesky (the
    256-rank blocked factorisation of the leading block and of the Schur
    complement, FP64 products between them).  A rank-r input with r < q makes
    both Gram blocks singular, so each block's factorisation restarts with a
    diagonal shift; the basis still spans the input, so U S V^T reproduces it
    and the signal part of U is orthonormal.  r = q = 257 leaves a one-column
    second block."""
    A = lowrank(m, n, r, 0.3, 0.0, seed=q + r)
    U, S, V = B.svd_lowrank(A, q, 2)
    assert U.shape == (m, q) and V.shape == (n, q)
    assert np.all(np.diff(S) <= 0) and np.all(np.isfinite(U)) and np.all(np.isfinite(V))
    assert rel(O.reconstruct(U, S, V), A) < 1e-5
    rr = min(r, q)
    Us = U[:, :rr].astype(np.float64)
    assert np.abs(Us.T @ Us - np.eye(rr)).max() < 1e-4
    Z = np.zeros((m, n), np.float32)
    U, S, V = B.svd_lowrank(Z, q, 1)
    assert np.all(S == 0) and np.all(np.isfinite(U)) and np.all(np.isfinite(V))


def test_svd_config3_full_size():
    """BASELINE config 3 (4096 x 11008, rank-512 spectrum i^-1.2 + noise 0.01,
    q = 128, 2 power iterations) with an injected sketch."""
    A = lowrank(4096, 11008, 512, 1.2, 0.01, seed=0)
    R = np.random.default_rng(3).standard_normal((4096, 128)).astype(np.float32)
    U, S, V = B.svd_lowrank(A, 128, 2, sketch=R)
    Ur, Sr, Vr = O.svd_lowrank(A, 128, 2, R)
    U, V = align(U, V, Ur, Vr)
    e_rec = rel(O.reconstruct(U, S, V), O.reconstruct(Ur, Sr, Vr))
    print(f"C3: rec {e_rec:.2e} S {rel(S, Sr):.2e} U {rel(U, Ur):.2e} V {rel(V, Vr):.2e}")
    assert e_rec < 1e-4
    assert rel(S, Sr) < 1e-5


def test_svd_zero_and_rank_one():
    Z = np.zeros((64, 96), np.float32)
    U, S, V = B.svd_lowrank(Z, 8, 2)
    assert np.all(S == 0) and np.all(np.isfinite(U)) and np.all(np.isfinite(V))
    x = np.outer(np.arange(1, 65, dtype=np.float32), np.linspace(-1, 1, 96, dtype=np.float32))
    U, S, V = B.svd_lowrank(x, 8, 2)
    assert rel(O.reconstruct(U, S, V), x) < 1e-5


def test_svd_rank_one_repeated_between_other_ranks():
    """Regression: the triangular inverse's last column block (every rank
    <= 32) read its LDS copy of the diagonal inverse before the other waves
    had written it, so the rank-one case below came out with an unnormalised
    basis (S around 1e21) now and then, most often right after a larger-rank
    call.  Every repetition must give the same factors."""
    x = np.outer(np.arange(1, 65, dtype=np.float32), np.linspace(-1, 1, 96, dtype=np.float32))
    rng = np.random.default_rng(0)
    U0, S0, V0 = B.svd_lowrank(x, 8, 2)
    assert rel(O.reconstruct(U0, S0, V0), x) < 1e-5
    for it in range(40):
        if it % 2:
            B.svd_lowrank(rng.standard_normal((300, 500)).astype(np.float32), 47, 2)
        else:
            B.svd_lowrank(np.zeros((64, 96), np.float32), 8, 2)
        U, S, V = B.svd_lowrank(x, 8, 2)
        assert np.array_equal(S, S0) and np.array_equal(U, U0) and np.array_equal(V, V0), it


# ------------------------------------------------------------ pipeline ----
def svd_case(x, ro, re, q, it, uv, s, loc=B.INPUT_DEVICE):
    rows, cols = x.shape
    B.compress_release()
    B.decompress_release()
    assert B.compress_initialize(rows, cols, ro, re, q, it, uv, s, B.QUANT_NONE, loc) == 0
    kq = max(1, min(q, rows, cols))
    assert B.decompress_initialize(rows, cols, ro, re, kq, uv, s, B.QUANT_NONE) == 0
    src = B.DeviceBuffer.from_array(x) if loc == B.INPUT_DEVICE else x
    data = B.compress(src)
    out = B.decompress(data, rows, cols)
    return data, out


def check_svd_pipeline(x, ro, re, q, it, uv, s, loc=B.INPUT_DEVICE):
    """Every section except U/S/V (whose values come from the SVD) is checked
    bit for bit: U/S/V sections are re-encoded by the oracle from the decoded
    factors, the error section is the oracle top-k of residual - (GPU
    reconstruction of the decoded factors), and the decode equals that
    reconstruction plus the two scatter-adds in the reference's order."""
    rows, cols = x.shape
    data, out = svd_case(x, ro, re, q, it, uv, s, loc)
    p = O.parse_packed(data)
    k = p.effective_rank
    assert k == max(1, min(q, rows, cols)) and (p.flags & O.FLAG_SVD)
    dec = {}
    for name, fmt, cnt in (("u", uv, rows * k), ("s", s, k), ("v", uv, cols * k)):
        storage, blob = p.sections[name]
        if fmt == O.QUANT_NONE:
            assert storage == O.SECTION_FP32
            dec[name] = np.frombuffer(blob, np.float32).copy()
        else:
            qz = O.unpack_quant(blob)
            assert O.pack_quant(qz) == blob
            dec[name] = O.quant_decompress(qz)
    U, S, V = dec["u"].reshape(rows, k), dec["s"], dec["v"].reshape(cols, k)
    # outlier separation, exact
    residual = x.copy()
    if ro > 0:
        ko = O.topk_num_columns(cols, ro)
        oi, ov = O.topk_rows(x, ko)
        assert p.sections["outlier"][1] == O.pack_topk(rows, cols, oi, ov)
        np.put_along_axis(residual, oi.astype(np.int64), 0.0, axis=1)
    # sections U/S/V re-encoded from the decoded values must equal the payload
    # (quantisation of a dequantised section is not the identity in general,
    # so instead check the factors are a good SVD of the residual)
    recon = B.reconstruct(U, S, V)
    assert rel(recon, O.reconstruct(U, S, V)) < 2e-6
    err = residual - recon
    if re > 0 and np.any(np.abs(err) > O.FLT_EPSILON):
        ke = O.topk_num_columns(cols, re)
        ei, ev = O.topk_rows(err, ke)
        assert p.flags & O.FLAG_ERROR
        assert p.sections["error"][1] == O.pack_topk(rows, cols, ei, ev)
        expect = recon.copy()
        rr = np.repeat(np.arange(rows), ke)
        expect[rr, ei.astype(np.int64).ravel()] += ev.ravel()
    else:
        assert not (p.flags & O.FLAG_ERROR)
        expect = recon.copy()
    if ro > 0:
        expect[np.repeat(np.arange(rows), ko), oi.astype(np.int64).ravel()] += ov.ravel()
    assert out.tobytes() == expect.tobytes()
    return U, S, V, residual


CASES = [
    # reference tests/bitsqz_llm/test_svd.cpp:590-615 shapes at 512x8192 sin/cos
    ("svd_only", 0.0, 0.0, B.QUANT_NONE, B.QUANT_NONE, 128, 2, B.INPUT_DEVICE),
    ("svd_only_host", 0.0, 0.0, B.QUANT_NONE, B.QUANT_NONE, 128, 2, B.INPUT_HOST),
    ("svd_quantization_nf4", 0.0, 0.0, B.NF4, B.NF4, 128, 2, B.INPUT_DEVICE),
    ("svd_error", 0.0, 0.10, B.QUANT_NONE, B.QUANT_NONE, 128, 2, B.INPUT_DEVICE),
    ("svd_quantization_error_nf4", 0.0, 0.10, B.NF4, B.NF4, 128, 2, B.INPUT_DEVICE),
    ("outlier_svd", 0.05, 0.0, B.QUANT_NONE, B.QUANT_NONE, 128, 2, B.INPUT_DEVICE),
    ("outlier_svd_error", 0.05, 0.10, B.QUANT_NONE, B.QUANT_NONE, 128, 2, B.INPUT_DEVICE),
    ("outlier_svd_quantization_error_nf4_dq", 0.05, 0.10, B.NF4_DQ, B.NF4, 128, 2, B.INPUT_DEVICE),
    ("best_nf4_dq", 0.001, 0.015, B.NF4_DQ, B.QUANT_NONE, 128, 2, B.INPUT_DEVICE),
    ("best_nf4_dq_iter6", 0.001, 0.015, B.NF4_DQ, B.QUANT_NONE, 128, 6, B.INPUT_DEVICE),
]


def sincos_source(rows, cols):
    idx = np.arange(rows * cols, dtype=np.int64).reshape(rows, cols)
    r = np.arange(rows)[:, None]
    c = np.arange(cols)[None, :]
    return (np.sin(np.float32(0.11) * idx.astype(np.float32)) +
            np.cos(np.float32(0.07) * (r + c).astype(np.float32))).astype(np.float32)


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_svd_pipeline_reference_cases(case):
    name, ro, re, uv, s, q, it, loc = case
    x = sincos_source(512, 8192)
    check_svd_pipeline(x, ro, re, q, it, uv, s, loc)


def test_svd_pipeline_config4_like():
    """Config-4 knobs (outlier 0.005, error 0.01, q=256, it=2, UV NF4) on a
    2048x4096 low-rank matrix with outlier columns."""
    x = lowrank(2048, 4096, 512, 1.0, 0.01, seed=5)
    x[:, np.random.default_rng(1).permutation(4096)[:8]] *= 50.0
    U, S, V, residual = check_svd_pipeline(x, 0.005, 0.01, 256, 2, B.NF4, B.QUANT_NONE)
    assert rel(O.reconstruct(U, S, V), residual) < 0.2


@pytest.mark.parametrize("q", [16, 48, 80])
def test_svd_pipeline_error_short_rank(q):
    """The fused reconstruction - residual epilogue with 1, 3 and 5 K-slices
    (the minuend is requested behind the last operand slice, in the prologue
    when there are at most three) and a row count that is not a multiple of
    the 128-row tile."""
    x = lowrank(200, 1000, 160, 0.8, 0.01, seed=q)
    check_svd_pipeline(x, 0.0, 0.05, q, 1, B.QUANT_NONE, B.QUANT_NONE)


def test_walkthrough_example_8x8():
    """examples/bitsqz_llm_walkthrough.cpp: 8x8 host input, rank 4, NF4 U/V and S."""
    i = np.arange(64)
    x = ((i % 8) * 0.25 + (i // 8) * 0.5).astype(np.float32).reshape(8, 8)
    check_svd_pipeline(x, 0.0, 0.0, 4, 2, B.NF4, B.NF4, B.INPUT_HOST)


def test_rank_mismatch_rejected():
    x = sincos_source(64, 256)
    data, _ = svd_case(x, 0.0, 0.0, 16, 2, B.QUANT_NONE, B.QUANT_NONE)
    dst = B.DeviceBuffer(x.nbytes)
    for r in (15, 17):
        assert B.decompress_initialize(64, 256, 0.0, 0.0, r, B.QUANT_NONE, B.QUANT_NONE, B.QUANT_NONE) == 0
        assert B.decompress_to_device(data, dst, x.size) == 1
    assert B.decompress_initialize(64, 256, 0.0, 0.0, 16, B.QUANT_NONE, B.QUANT_NONE, B.QUANT_NONE) == 0
    assert B.decompress_to_device(data, dst, x.size) == 0
    B.decompress_release()
    B.compress_release()
