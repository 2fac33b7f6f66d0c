"""The reconstruction from packed NF4 / NF4_DQ factors decoded inline
(recon.hip) on the GPU.

  * Through the ABI, every section and the decode are checked bit for bit
    against the oracle by `check_sections`: the decompress side decodes U and
    V inside the reconstruction, and the result must equal the FP32
    reconstruction of the decoded factors plus the error set, then the
    outlier set (src/bitsqz_llm.cu:1341-1387).
  * The device-resident decompress (packed U and V taken straight from the
    compress runtime) must give the same bytes.

Shapes are ragged (rows and columns off the 128-wide tiles), both branches of
the SVD (m < n and m > n), ranks 64 .. 512, S in FP32 and packed."""
import numpy as np
import pytest

import bitsqz_amd as B
from _svdcase import abi_round_trip, check_sections, lowrank, outlier_columns

pytestmark = pytest.mark.gpu

CASES = [
    # rows, cols, q, uv, s, outlier ratio, error ratio
    (300, 700, 64, B.NF4, B.QUANT_NONE, 0.02, 0.05),
    (520, 1030, 128, B.NF4_DQ, B.NF4, 0.01, 0.03),
    (1000, 300, 64, B.NF4, B.NF4_DQ, 0.05, 0.0),
    (200, 2000, 192, B.NF4_DQ, B.QUANT_NONE, 0.0, 0.02),
    (1024, 3000, 256, B.NF4, B.QUANT_NONE, 0.005, 0.01),
    (640, 1536, 512, B.NF4_DQ, B.QUANT_NONE, 0.004, 0.008),
]


@pytest.mark.parametrize("rows,cols,q,uv,s,ro,re", CASES)
def test_fused_reconstruction_bit_exact(rows, cols, q, uv, s, ro, re):
    x = lowrank(rows, cols, min(256, rows, cols), 1.0, 0.01, seed=q + rows)
    x = outlier_columns(x, 4, 40.0, seed=cols)
    print(f"fused recon case {rows}x{cols} q={q} uv={uv} s={s} ro={ro} re={re}", flush=True)
    data, out = abi_round_trip(x, ro, re, q, 2, uv, s)
    check_sections(x, data, out, ro, re, q, uv, s)
    # the device-resident twin: same compress, scatter fused into the reconstruction
    src = B.DeviceBuffer.from_array(x)
    dst = B.DeviceBuffer(rows * cols * 4)
    packed = B.device_compress(src)
    B.device_decompress(packed, dst, rows * cols)
    B.device_synchronize()
    dev = dst.download(np.float32, rows * cols).reshape(rows, cols)
    assert dev.tobytes() == out.tobytes()
    B.compress_release()
    B.decompress_release()
