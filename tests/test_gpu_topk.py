"""Per-row top-k on the GPU vs the reference's known-answer tests and the CPU
oracle (stable descending sort by |x|, NaN lowest, ties to the lower column;
reference modules/topk_cuda/src/topk_cuda_utils.cuh:51-149).  Indices and
values must be bit-exact."""
import numpy as np
import pytest

import bitsqz_amd as B
from oracle import oracle as O

pytestmark = pytest.mark.gpu

KATS = ["extract", "sep0", "sep001", "sep1", "pack", "ties"]


@pytest.mark.parametrize("name", KATS)
def test_reference_kats(golden, name):
    g = golden["topk"]
    x = g[name + "_x"]
    k = int(g[name + "_k"][0])
    assert B.topk_num_columns(x.shape[1], float(g[name + "_ratio"][0])) == k
    if k == 0:
        return
    idx, val, res = B.topk_select(x, k, separate=True)
    assert idx.tobytes() == g[name + "_idx"].tobytes()
    assert val.tobytes() == g[name + "_val"].tobytes()
    # separation zeroes exactly the selected entries, the rest unchanged
    # (test_topk_cuda_separation.cpp), and scatter-add restores the input
    expect = x.copy()
    np.put_along_axis(expect, idx.astype(np.int64), 0.0, axis=1)
    assert res.tobytes() == expect.tobytes()
    back = B.topk_scatter(idx, val, res, accumulate=True)
    assert np.array_equal(back, x, equal_nan=True)
    dense = B.topk_scatter(idx, val, np.full_like(x, 7.0), accumulate=False)
    exp = np.zeros_like(x)
    np.put_along_axis(exp, idx.astype(np.int64), val, axis=1)
    assert np.array_equal(dense, exp, equal_nan=True)


def _check(x, k):
    idx, val = B.topk_select(x, k)
    ei, ev = O.topk_rows(x, k)
    assert idx.tobytes() == ei.tobytes()
    assert val.tobytes() == ev.tobytes()


@pytest.mark.parametrize("rows,cols,k", [(64, 4096, 20), (32, 11008, 55), (32, 11008, 110), (16, 14336, 72),
                                         (8, 100, 100), (8, 1000, 300), (4, 20000, 29), (4, 40000, 2000),
                                         (2, 9000, 8192), (3, 65535, 1)])
def test_random_rows(rows, cols, k):
    x = np.random.default_rng(rows * cols + k).standard_normal((rows, cols)).astype(np.float32)
    _check(x, k)


def test_ties_nan_inf_zero_rows():
    rng = np.random.default_rng(11)
    x = rng.integers(-3, 4, (32, 600)).astype(np.float32)   # heavy ties incl. +-0
    x[0] = 0.0
    x[1] = np.nan
    x[2, ::3] = np.nan
    x[3, 5] = np.inf
    x[3, 9] = -np.inf
    x[4] = -0.0
    x[5, :300] = 1e-42
    for k in (1, 7, 64, 256, 257, 600):
        _check(x, k)


@pytest.mark.parametrize("cols", [600, 4096, 8000, 11008, 12000, 14336, 16000, 20000])
def test_ties_at_threshold_every_kernel(cols):
    """Heavy ties in magnitude (integers -3..3 and their negatives, so equal
    |v| sits on both sides of the k-th entry), NaN / inf / +-0 / subnormal
    rows, at widths served by each kernel variant (register rows of 2, 4, 8,
    11 and 14 quads per lane, the last also part-filled at 12000 columns,
    then the LDS-cached kernel at 16000 and the uncached one at 20000); the
    separation residual zeroes exactly the selected entries."""
    rng = np.random.default_rng(cols)
    x = rng.integers(-3, 4, (12, cols)).astype(np.float32)
    x[0] = 0.0
    x[1] = np.nan
    x[2, ::3] = np.nan
    x[3, 5] = np.inf
    x[3, 9] = -np.inf
    x[4] = -0.0
    x[5, : cols // 2] = 1e-42
    x[6] = rng.standard_normal(cols).astype(np.float32)
    x[7, ::2] = np.nan
    x[7, 1::2] = 2.0
    for k in (1, 64, 256):
        idx, val, res = B.topk_select(x, k, separate=True)
        ei, ev = O.topk_rows(x, k)
        assert idx.tobytes() == ei.tobytes() and val.tobytes() == ev.tobytes()
        expect = x.copy()
        np.put_along_axis(expect, ei.astype(np.int64), 0.0, axis=1)
        assert res.tobytes() == expect.tobytes()


def test_outlier_columns_like_config2():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((512, 4096)).astype(np.float32)
    cols = np.random.default_rng(1).permutation(4096)[:16]
    x[:, cols] *= 60.0
    _check(x, 20)


def test_separation_in_place_large():
    x = np.random.default_rng(2).standard_normal((128, 20000)).astype(np.float32)
    idx, val, res = B.topk_select(x, 40, separate=True)
    ei, ev = O.topk_rows(x, 40)
    assert idx.tobytes() == ei.tobytes() and val.tobytes() == ev.tobytes()
    expect = x.copy()
    np.put_along_axis(expect, ei.astype(np.int64), 0.0, axis=1)
    assert res.tobytes() == expect.tobytes()


@pytest.mark.parametrize("k", [16, 110, 256])
def test_filter_fallback_and_separation(k):
    """Rows whose largest entries all fall on the same 256-column residues
    (column % 256 < k) defeat the per-thread-maximum filter (about 43 k
    candidates), so the radix select takes over; other rows in the same launch
    take the filter path.  Both must give the oracle's bytes, including the
    separation residual."""
    rng = np.random.default_rng(k)
    x = rng.standard_normal((8, 11008)).astype(np.float32)
    big = (np.arange(11008) % 256) < k
    x[::2, big] = (rng.standard_normal(int(big.sum())) * 100.0).astype(np.float32)  # even rows: fallback
    idx, val, res = B.topk_select(x, k, separate=True)
    ei, ev = O.topk_rows(x, k)
    assert idx.tobytes() == ei.tobytes() and val.tobytes() == ev.tobytes()
    expect = x.copy()
    np.put_along_axis(expect, ei.astype(np.int64), 0.0, axis=1)
    assert res.tobytes() == expect.tobytes()
