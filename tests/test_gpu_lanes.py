"""Lanes (bsq_lanes_*): independent compress + decompress runtime pairs on
their own streams.  Round trips enqueued on two lanes at once, on different
matrices and repeated, must give byte for byte the decode that the single
device-resident runtime (bsq_device_compress + bsq_device_decompress) gives
for each matrix."""
import numpy as np
import pytest

import bitsqz_amd as B
from _svdcase import lowrank, outlier_columns

pytestmark = pytest.mark.gpu


def _single(x, cfg):
    rows, cols = x.shape
    ro, re, svd, it, uv, s, direct = cfg
    B.compress_release()
    B.decompress_release()
    B.check(B.compress_initialize(rows, cols, ro, re, svd, it, uv, s, direct, B.INPUT_DEVICE), "compress init")
    q = max(1, min(svd, rows, cols)) if svd >= 1 else -1
    B.check(B.decompress_initialize(rows, cols, ro, re, q, uv, s, direct), "decompress init")
    src = B.DeviceBuffer.from_array(x)
    dst = B.DeviceBuffer(x.nbytes)
    p = B.device_compress(src)
    B.device_decompress(p, dst, rows * cols)
    B.device_synchronize()
    out = dst.download(np.float32, rows * cols)
    B.compress_release()
    B.decompress_release()
    return out


@pytest.mark.parametrize("shape,cfg", [
    ((512, 4096), (0.01, 0.02, -1, 2, B.QUANT_NONE, B.QUANT_NONE, B.NF4_DQ)),
    ((1024, 2752), (0.005, 0.01, 128, 2, B.NF4, B.QUANT_NONE, B.QUANT_NONE)),
    ((700, 1200), (0.0, 0.0, 64, 1, B.QUANT_NONE, B.QUANT_NONE, B.QUANT_NONE)),
])
def test_four_lanes_match_the_single_runtime(shape, cfg):
    rows, cols = shape
    nl = 4
    xs = [outlier_columns(lowrank(rows, cols, 256, 1.1, 0.01, seed=s), 4, 30.0, seed=s + 1) for s in range(nl)]
    refs = [_single(x, cfg) for x in xs]
    ro, re, svd, it, uv, s, direct = cfg
    L = B.lib()
    B.check(L.bsq_lanes_initialize(nl, rows, cols, ro, re, svd, it, uv, s, direct), "lanes init")
    try:
        src = [B.DeviceBuffer.from_array(x) for x in xs]
        dst = [B.DeviceBuffer(rows * cols * 4) for _ in xs]
        for rep in range(3):
            for d in dst:
                d.zero()
            for lane in range(nl):
                # rotate which matrix each lane gets
                i = (lane + rep) % nl
                B.check(L.bsq_lanes_roundtrip(lane, src[i].ptr, dst[i].ptr), "lanes roundtrip")
            B.check(L.bsq_lanes_synchronize(), "lanes sync")
            for i in range(nl):
                got = dst[i].download(np.float32, rows * cols)
                assert got.tobytes() == refs[i].tobytes(), f"repetition {rep}, matrix {i}"
    finally:
        L.bsq_lanes_release()


def test_lanes_arguments_rejected():
    L = B.lib()
    assert L.bsq_lanes_initialize(0, 64, 64, 0.0, 0.0, -1, 2, B.QUANT_NONE, B.QUANT_NONE, B.NF4) == 1
    assert L.bsq_lanes_initialize(9, 64, 64, 0.0, 0.0, -1, 2, B.QUANT_NONE, B.QUANT_NONE, B.NF4) == 1
    assert L.bsq_lanes_initialize(1, 64, 64, 1.5, 0.0, -1, 2, B.QUANT_NONE, B.QUANT_NONE, B.NF4) == 1
    B.check(L.bsq_lanes_initialize(1, 64, 64, 0.0, 0.0, -1, 2, B.QUANT_NONE, B.QUANT_NONE, B.NF4), "init")
    d = B.DeviceBuffer(64 * 64 * 4)
    assert L.bsq_lanes_roundtrip(1, d.ptr, d.ptr) == 1  # no such lane
    assert L.bsq_lanes_roundtrip(0, None, d.ptr) == 1
    L.bsq_lanes_release()
    assert L.bsq_lanes_roundtrip(0, d.ptr, d.ptr) == 1  # released
