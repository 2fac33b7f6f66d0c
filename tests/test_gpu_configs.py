"""The BASELINE configurations C4, C5 and the headline workload through the
reference ABI on the GPU, and the randomised SVD at ranks above 256.

SVD parity is defined with the sketch injected (the reference draws it from
cuRAND, modules/svd_lowrank_cuda/src/svd_lowrank_cuda.cu:289-291): the
GPU's U, S, V for the residual are compared with the FP64 oracle restatement
of svd_lowrank_cuda.cu:284-426 (reconstruction <= 1e-4 relative Frobenius,
S <= 1e-5), and the packed object is checked section by section against the
oracle's encoding of those same factors (bit-exact for every section, and for
the decode)."""
import time

import numpy as np
import pytest

import bitsqz_amd as B
from oracle import oracle as O
from _svdcase import abi_round_trip, align, check_sections, lowrank, outlier_columns, rel

pytestmark = pytest.mark.gpu


def svd_parity(A, q, it, R, tol_rec=1e-4, tol_s=1e-5):
    t0 = time.time()
    U, S, V = B.svd_lowrank(A, q, it, sketch=R)
    t1 = time.time()
    Ur, Sr, Vr = O.svd_lowrank(A, q, it, R)
    t2 = time.time()
    Ua, Va = align(U, V, Ur, Vr)
    e_rec = rel(O.reconstruct(Ua, S, Va), O.reconstruct(Ur, Sr, Vr))
    e_s = rel(S, Sr)
    k = S.size
    orth = np.abs(U.astype(np.float64).T @ U - np.eye(k)).max()
    print(f"svd {A.shape} q={q} it={it}: rec {e_rec:.2e} S {e_s:.2e} U^T U - I {orth:.1e} "
          f"(gpu {t1 - t0:.1f} s, oracle {t2 - t1:.1f} s)", flush=True)
    assert np.all(np.diff(S) <= 0)
    assert e_rec < tol_rec
    assert e_s < tol_s
    assert orth < 1e-4
    return U, S, V


@pytest.mark.parametrize("m,n,q,it,decay", [
    (1200, 3000, 257, 2, 1.0),   # one past the register-resident kernels, transposed branch
    (2600, 1100, 300, 1, 1.2),   # m > n branch
    (2048, 14336, 512, 3, 0.8),  # C5's rank and iterations on its 8-way row share
    (900, 1500, 449, 1, 1.1),    # an odd rank: the per-column kernels' last lanes idle
])
def test_svd_rank_above_256_matches_oracle(m, n, q, it, decay):
    """Ranks 257 .. 512 run the two-level Cholesky, the per-column
    tridiagonalisation over a global-memory working copy (linalg.hip
    trd_step_kernel + trd_col_kernel, reflectors row-wise) and the row-wise
    back-transformation (backtransform_rows_kernel<8, 16>)."""
    A = lowrank(m, n, min(1024, m, n), decay, 0.02, seed=q)
    k = max(1, min(q, m, n))
    R = np.random.default_rng(3).standard_normal((min(m, n), k)).astype(np.float32)
    svd_parity(A, q, it, R)


def _full_pipeline(x, ro, re, q, it, uv, s, loc, seed=3):
    rows, cols = x.shape
    print(f"pipeline {x.shape}: input generated", flush=True)
    k = max(1, min(q, rows, cols))
    R = np.random.default_rng(seed).standard_normal((min(rows, cols), k)).astype(np.float32)
    residual = x.copy()
    if ro > 0:
        oi, _ = O.topk_rows(x, O.topk_num_columns(cols, ro))
        np.put_along_axis(residual, oi.astype(np.int64), 0.0, axis=1)
    print(f"pipeline {x.shape}: oracle outliers separated", flush=True)
    factors = svd_parity(residual, q, it, R)
    t0 = time.time()
    data, out = abi_round_trip(x, ro, re, q, it, uv, s, loc, sketch=R)
    t1 = time.time()
    print(f"pipeline {x.shape}: ABI round trip done in {t1 - t0:.1f} s", flush=True)
    _, res2, recon = check_sections(x, data, out, ro, re, q, uv, s, factors=factors)
    assert np.array_equal(res2, residual)
    e = rel(out, x)
    print(f"pipeline {x.shape}: packed {len(data)} B, round trip {t1 - t0:.1f} s, "
          f"rel error of the decode vs the input {e:.4f}", flush=True)
    return data, out, e


@pytest.mark.timeout(900)
def test_config4_full_pipeline():
    """BASELINE C4: 8192 x 4096 (m > n), rank-512 spectrum i^-1.0 + noise 0.01,
    8 columns x50; outlier 0.005 (k_o = 20), error 0.01 (k_e = 41), q = 256,
    2 iterations, UV NF4, S FP32."""
    x = outlier_columns(lowrank(8192, 4096, 512, 1.0, 0.01, seed=0), 8, 50.0)
    assert O.topk_num_columns(4096, 0.005) == 20 and O.topk_num_columns(4096, 0.01) == 41
    data, _, e = _full_pipeline(x, 0.005, 0.01, 256, 2, B.NF4, B.QUANT_NONE, B.INPUT_DEVICE)
    assert len(data) == 200 + 4768880
    assert e < 0.2


@pytest.mark.timeout(900)
def test_config3_full_pipeline_fp32_factors():
    """BASELINE C3 through the ABI at full size: 4096 x 11008, rank-512
    spectrum i^-1.2 + noise 0.01, q = 128, 2 iterations, U / S / V stored as
    FP32 sections, no top-k.  The sections equal the standalone SVD's factors
    (which match the FP64 oracle to 1e-4), and the decode is their
    reconstruction, byte for byte."""
    x = lowrank(4096, 11008, 512, 1.2, 0.01, seed=0)
    data, _, e = _full_pipeline(x, 0.0, 0.0, 128, 2, B.QUANT_NONE, B.QUANT_NONE, B.INPUT_DEVICE)
    assert len(data) == 200 + 7733760
    assert e < 0.2


@pytest.mark.timeout(900)
def test_headline_full_pipeline():
    """The headline workload: 4096 x 11008 with the C3 generator and 8 columns
    x50, C4's knobs (k_o = 55, k_e = 110, q = 256, it = 2, UV NF4)."""
    x = outlier_columns(lowrank(4096, 11008, 512, 1.2, 0.01, seed=0), 8, 50.0)
    data, _, e = _full_pipeline(x, 0.005, 0.01, 256, 2, B.NF4, B.QUANT_NONE, B.INPUT_DEVICE)
    assert len(data) == 200 + 6231152
    assert e < 0.2


@pytest.mark.timeout(1200)
def test_config5_full_pipeline_host_input():
    """BASELINE C5: 16384 x 14336, rank-1024 spectrum i^-0.8 + noise 0.02, 32
    columns x80; outlier 0.002 (k_o = 29), error 0.005 (k_e = 72), q = 512,
    3 iterations, UV NF4_DQ, S FP32, HOST input (the 939.5 MB H2D staging
    copy of src/bitsqz_llm.cu:1022-1034)."""
    x = outlier_columns(lowrank(16384, 14336, 1024, 0.8, 0.02, seed=0), 32, 80.0)
    assert O.topk_num_columns(14336, 0.002) == 29 and O.topk_num_columns(14336, 0.005) == 72
    data, _, e = _full_pipeline(x, 0.002, 0.005, 512, 3, B.NF4_DQ, B.QUANT_NONE, B.INPUT_HOST)
    assert len(data) == 200 + 18040944
    assert e < 0.3
