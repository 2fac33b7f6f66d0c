"""Shapes the reference accepts with no limit of its own: top-k with k above
8192 (topk_compute_num_topk_columns allows any k <= cols, topk_cuda.cu:53-69)
and SVD ranks above 4096 (k = max(1, min(q, m, n)), svd_lowrank_cuda.cu:
129-137).  Outputs are checked against the oracle as everywhere else."""
import numpy as np
import pytest

import bitsqz_amd as B
from oracle import oracle as O
from _svdcase import align, lowrank, rel

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("rows,cols,k", [(4, 9000, 8193), (3, 11008, 11008), (2, 16384, 12000),
                                         (2, 20000, 20000), (2, 65535, 40000)])
def test_topk_above_8192_matches_oracle(rows, cols, k):
    """Bands of 8192 ranks; rows cached in LDS up to 16384 columns, read from
    HBM beyond.  Includes heavy ties (integers) so the column tie-break is
    exercised across band boundaries."""
    rng = np.random.default_rng(rows * cols + k)
    x = rng.standard_normal((rows, cols)).astype(np.float32)
    x[0] = rng.integers(-5, 6, cols).astype(np.float32)
    idx, val, res = B.topk_select(x, k, separate=True)
    ei, ev = O.topk_rows(x, k)
    assert idx.tobytes() == ei.tobytes()
    assert val.tobytes() == ev.tobytes()
    expect = x.copy()
    np.put_along_axis(expect, ei.astype(np.int64), 0.0, axis=1)
    assert res.tobytes() == expect.tobytes()


def test_outlier_ratio_one_on_11008_columns():
    """outlier_topk_ratio = 1.0 on 11008 columns (k = 11008): every entry is an
    outlier, the direct section encodes zeros, and the decode is exact."""
    rows, cols = 16, 11008
    x = np.random.default_rng(7).standard_normal((rows, cols)).astype(np.float32)
    B.compress_release()
    B.decompress_release()
    assert B.compress_initialize(rows, cols, 1.0, 0.0, -1, 2, B.QUANT_NONE, B.QUANT_NONE, B.NF4,
                                 B.INPUT_HOST) == 0, B.lib().bsq_last_error()
    assert B.decompress_initialize(rows, cols, 1.0, 0.0, -1, B.QUANT_NONE, B.QUANT_NONE, B.NF4) == 0
    data = B.compress(x)
    out = B.decompress(data, rows, cols)
    p = O.compress(x, O.Config(rows, cols, outlier_ratio=1.0, direct_format=O.NF4))
    assert O.mask_pointer(data) == O.mask_pointer(p.to_bytes())
    assert out.tobytes() == O.decompress(p).tobytes()
    assert np.array_equal(out, x)
    B.compress_release()
    B.decompress_release()


def test_svd_ranks_above_4096_small_rows_accepted():
    """svd_ranks = 5000 on a 64-row matrix: the effective rank is 64."""
    x = lowrank(64, 8192, 64, 1.0, 0.01, seed=2)
    B.compress_release()
    B.decompress_release()
    assert B.compress_initialize(64, 8192, 0.0, 0.0, 5000, 2, B.QUANT_NONE, B.QUANT_NONE, B.QUANT_NONE,
                                 B.INPUT_HOST) == 0
    assert B.decompress_initialize(64, 8192, 0.0, 0.0, 64, B.QUANT_NONE, B.QUANT_NONE, B.QUANT_NONE) == 0
    data = B.compress(x)
    p = O.parse_packed(data)
    assert p.effective_rank == 64 and p.svd_ranks == 5000
    out = B.decompress(data, 64, 8192)
    assert rel(out, x) < 1e-5
    B.compress_release()
    B.decompress_release()


@pytest.mark.timeout(600)
def test_svd_effective_rank_above_4096_matches_oracle():
    """k = 4100 (both dimensions above 4096): the unblocked global-memory
    Cholesky, the one-workgroup tridiagonalisation (sytrd_kernel), the
    column-wise back-transformation and the eigensolver kernels with their
    global-memory vectors."""
    m, n, q = 4160, 4300, 4100
    A = lowrank(m, n, min(m, n), 0.5, 0.0, seed=9)
    R = np.random.default_rng(3).standard_normal((m, q)).astype(np.float32)
    U, S, V = B.svd_lowrank(A, q, 1, sketch=R)
    Ur, Sr, Vr = O.svd_lowrank(A, q, 1, R)
    U, V = align(U, V, Ur, Vr)
    e_rec = rel(O.reconstruct(U, S, V), O.reconstruct(Ur, Sr, Vr))
    print(f"rank {q}: rec {e_rec:.2e} S {rel(S, Sr):.2e}", flush=True)
    assert e_rec < 1e-4
    assert rel(S, Sr) < 1e-5
