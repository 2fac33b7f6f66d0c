"""The pipeline composition of src/bitsqz_llm.cu:981-1393 on the GPU, on
crafted inputs whose expected bytes are written out explicitly (the same
cases pin the oracle in tests/test_oracle.py):
  * direct path: error = top-k of x - dequant(x), decoded as fl(deq + err);
  * the strict FLT_EPSILON gate of the error extraction;
  * error set applied before the outlier set on decode;
  * NF4_DQ decode with a loaded dq of 0 / -0 / NaN / +-inf / subnormal
    (quantization_cuda.cu:322-327);
  * top-k indices >= cols in a loaded object land at the flat position
    r * cols + idx, as the reference's scatter_add_topk_kernel writes them
    (topk_cuda_utils.cuh:132-149)."""
import struct

import numpy as np
import pytest

import bitsqz_amd as B
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def direct_round_trip(x, ro, re, fmt):
    rows, cols = x.shape
    B.compress_release()
    B.decompress_release()
    assert B.compress_initialize(rows, cols, ro, re, -1, 2, B.QUANT_NONE, B.QUANT_NONE, fmt, B.INPUT_HOST) == 0
    assert B.decompress_initialize(rows, cols, ro, re, -1, B.QUANT_NONE, B.QUANT_NONE, fmt) == 0
    data = B.compress(x)
    return data, B.decompress(data, rows, cols)


@pytest.mark.parametrize("method", [B.NF4, B.NF4_DQ])
def test_direct_error_is_topk_of_residual_minus_dequant(method):
    rng = np.random.default_rng(21)
    rows, cols = 12, 320
    x = rng.standard_normal((rows, cols)).astype(np.float32)
    ke = O.topk_num_columns(cols, 0.05)
    data, out = direct_round_trip(x, 0.0, 0.05, method)
    deq = O.quant_decompress(O.quant_compress(x, method)).reshape(rows, cols)
    err = (x - deq).astype(np.float32)
    order = np.argsort(-np.abs(err), axis=1, kind="stable")[:, :ke]
    p = O.parse_packed(data)
    assert p.sections["error"][1] == (struct.pack("<HHHH", rows, cols, ke, 0) + order.astype(np.uint16).tobytes()
                                      + np.take_along_axis(err, order, axis=1).astype(np.float32).tobytes())
    expect = deq.copy()
    for r in range(rows):
        for c in order[r]:
            expect[r, c] = np.float32(deq[r, c] + np.float32(x[r, c] - deq[r, c]))
    assert out.tobytes() == expect.tobytes()


@pytest.mark.parametrize("bump,present", [(False, False), (True, True)])
def test_flt_epsilon_gate(bump, present):
    x = np.zeros((2, 64), np.float32)
    x[:, 0] = 1.0
    e = np.float32(O.FLT_EPSILON)
    x[1, 5] = np.nextafter(e, np.float32(1.0)) if bump else e
    data, out = direct_round_trip(x, 0.0, 0.05, B.NF4)
    p = O.parse_packed(data)
    assert bool(p.flags & O.FLAG_ERROR) == present
    assert ("error" in p.sections) == present
    assert O.mask_pointer(data) == O.mask_pointer(O.compress(x, O.Config(2, 64, error_ratio=0.05,
                                                                          direct_format=O.NF4)).to_bytes())


def _decode_on_gpu(buf: bytes, rows, cols, ro, re, rank, uv, s, direct):
    B.decompress_release()
    assert B.decompress_initialize(rows, cols, ro, re, rank, uv, s, direct) == 0
    dst = B.DeviceBuffer(rows * cols * 4)
    assert B.decompress_to_device(buf, dst, rows * cols) == 0, B.lib().bsq_last_error()
    return dst.download(np.float32, rows * cols).reshape(rows, cols)


def test_error_then_outlier_apply_order():
    """Outlier 2^24, reconstruction 1, error -1 at column 0: error first gives
    2^24, outlier first 2^24 - 1 (the packed object is written by the oracle
    from explicit factors U = 1, S = 1, V = 1)."""
    x = np.ones((1, 8), np.float32)
    x[0, 0] = np.float32(2.0 ** 24)
    cfg = O.Config(1, 8, outlier_ratio=0.125, error_ratio=0.125, svd_ranks=1, svd_niters=1)
    p = O.compress(x, cfg, svd_result=(np.ones((1, 1), np.float32), np.ones(1, np.float32),
                                       np.ones((8, 1), np.float32)))
    out = _decode_on_gpu(p.to_bytes(), 1, 8, 0.125, 0.125, 1, B.QUANT_NONE, B.QUANT_NONE, B.QUANT_NONE)
    assert out[0, 0] == np.float32(2.0 ** 24)
    assert np.all(out[0, 1:] == 1.0)
    assert out.tobytes() == O.decompress(p).tobytes()


@pytest.mark.parametrize("dq", [0.0, -0.0, float("nan"), float("inf"), float("-inf"), 1e-45, 3.0e-3])
def test_nf4dq_decode_of_loaded_dq(dq):
    rng = np.random.default_rng(25)
    rows, cols = 4, 200
    x = rng.standard_normal((rows, cols)).astype(np.float32)
    data, _ = direct_round_trip(x, 0.0, 0.0, B.NF4_DQ)
    p = O.parse_packed(data)
    off, size, st = struct.unpack_from("<QQB", data, 48 + 24 * 3)
    assert st == O.SECTION_QUANT
    buf = bytearray(data)
    struct.pack_into("<f", buf, 200 + off + 40, dq)  # dq_scale field of the quant header
    out = _decode_on_gpu(bytes(buf), rows, cols, 0.0, 0.0, -1, B.QUANT_NONE, B.QUANT_NONE, B.NF4_DQ)
    ref = O.decompress(O.parse_packed(bytes(buf)))
    assert out.tobytes() == ref.tobytes()


def test_wide_topk_index_lands_at_flat_position():
    """A loaded outlier set whose row-0 index is cols + 3 adds into row 1,
    column 3, as r * cols + idx does in the reference; an index past the end
    of the matrix (last row) is skipped where the reference would write
    outside the buffer."""
    rows, cols = 3, 64
    x = np.zeros((rows, cols), np.float32)
    p = O.Packed(rows, cols, 1.0 / 64, 0.0, -1, 2, 0, O.QUANT_NONE, O.QUANT_NONE, O.QUANT_NONE, O.FLAG_OUTLIER)
    p.sections["direct"] = (O.SECTION_FP32, x.tobytes())
    idx = np.array([[cols + 3], [5], [cols + 1]], np.uint16)
    val = np.array([[2.5], [4.0], [9.0]], np.float32)
    p.sections["outlier"] = (O.SECTION_TOPK, O.pack_topk(rows, cols, idx, val))
    out = _decode_on_gpu(p.to_bytes(), rows, cols, 1.0 / 64, 0.0, -1, B.QUANT_NONE, B.QUANT_NONE, B.QUANT_NONE)
    expect = x.copy()
    expect[1, 3] += 2.5
    expect[1, 5] += 4.0
    assert out.tobytes() == expect.tobytes()
    assert out.tobytes() == O.decompress(p).tobytes()
