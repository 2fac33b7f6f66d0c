"""NF4 / NF4_DQ / E4M3 on the GPU vs the CPU oracle, bit for bit.

The oracle (oracle/bsq_oracle.c) is itself pinned to the reference's legacy
codec by tests/test_oracle.py; the reference requires its CUDA codec to equal
that codec exactly (tests/quantization_cuda/test_nf4_cuda.cu:109-114), so bit
equality here is equality with the reference's device path."""
import numpy as np
import pytest

import bitsqz_amd as B
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _nf4_check(x):
    scales, codes, _ = B.quant_compress(x, B.NF4)
    q = O.quant_compress(x, O.NF4)
    assert scales.tobytes() == q.scales.tobytes()
    assert codes.tobytes() == q.codes.tobytes()
    out = B.quant_decompress(x.size, B.NF4, scales, codes)
    assert out.tobytes() == O.quant_decompress(q).tobytes()


def _nf4dq_check(x):
    scales, codes, dq = B.quant_compress(x, B.NF4_DQ)
    q = O.quant_compress(x, O.NF4_DQ)
    assert np.float32(dq).tobytes() == np.float32(q.dq).tobytes()
    assert scales.tobytes() == q.scales.tobytes()
    assert codes.tobytes() == q.codes.tobytes()
    out = B.quant_decompress(x.size, B.NF4_DQ, scales, codes, dq)
    assert out.tobytes() == O.quant_decompress(q).tobytes()


@pytest.mark.parametrize("name", ["edge", "unif"])
def test_nf4_golden(golden, name):
    g = golden["nf4"]
    x = g["nf4_%s_x" % name]
    scales, codes, _ = B.quant_compress(x, B.NF4)
    assert scales.tobytes() == g["nf4_%s_scales" % name].tobytes()
    assert codes.tobytes() == g["nf4_%s_codes" % name].tobytes()
    out = B.quant_decompress(x.size, B.NF4, scales, codes)
    assert out.tobytes() == g["nf4_%s_out" % name].tobytes()


@pytest.mark.parametrize("name", ["edge", "unif"])
def test_nf4dq_golden(golden, name):
    g = golden["nf4"]
    x = g["nf4dq_%s_x" % name]
    scales, codes, dq = B.quant_compress(x, B.NF4_DQ)
    assert np.float32(dq).tobytes() == g["nf4dq_%s_dq" % name].tobytes()
    assert scales.tobytes() == g["nf4dq_%s_scales" % name].tobytes()
    assert codes.tobytes() == g["nf4dq_%s_codes" % name].tobytes()
    out = B.quant_decompress(x.size, B.NF4_DQ, scales, codes, dq)
    assert out.tobytes() == g["nf4dq_%s_out" % name].tobytes()


def test_e4m3_golden_probes(golden):
    g = golden["nf4"]
    assert B.e4m3_encode(g["e4m3_probe_x"]).tobytes() == g["e4m3_probe_code"].tobytes()


def test_e4m3_decode_all_codes():
    codes = np.arange(256, dtype=np.uint8)
    assert B.e4m3_decode(codes).tobytes() == O.e4m3_decode_table().tobytes()


def test_e4m3_encode_random_bit_patterns():
    rng = np.random.default_rng(7)
    bits = rng.integers(0, 2 ** 32, 1 << 20, dtype=np.uint64).astype(np.uint32)
    v = bits.view(np.float32)
    assert B.e4m3_encode(v).tobytes() == O.e4m3_encode(v).tobytes()


def test_nf4_code_exhaustive_sweep():
    """Every one of the 2^32 float bit patterns: histogram + checksum of the
    device code function equal the CPU oracle's linear scan."""
    h_gpu, cs_gpu = B.nf4_code_sweep(0, 1 << 32)
    h_cpu, cs_cpu = O.nf4_code_sweep(0, 1 << 32)
    assert list(h_gpu) == list(h_cpu)
    assert cs_gpu == cs_cpu


def test_nf4_code_random_values():
    rng = np.random.default_rng(3)
    v = np.concatenate([rng.uniform(-1.5, 1.5, 1 << 18), rng.standard_normal(1 << 16) * 1e6,
                        np.array([np.nan, np.inf, -np.inf, 0.0, -0.0, 2.0, -2.0, 1e30, -1e30, 8388608.0,
                                  16777216.0, 3e38], np.float32)]).astype(np.float32)
    assert B.nf4_codes(v).tobytes() == O.nf4_codes(v).tobytes()


@pytest.mark.parametrize("n", [1, 2, 63, 64, 65, 127, 1000, 1023, 1024, 1025, 4097, 100003,
                               # past one pass of the contiguous-load encode's grid (2048 workgroups x
                               # 4 tiles of 1024 on 256 CUs), with a partial last tile and an odd count
                               3 * 4 * 1024 * 2048 + 777])
def test_nf4_partial_blocks(n):
    rng = np.random.default_rng(n)
    x = rng.standard_normal(n).astype(np.float32)
    _nf4_check(x)
    _nf4dq_check(x)


def test_nf4_config1_2048x4096():
    """2048x4096 i.i.d. N(0,1), NF4 block 64."""
    x = np.random.default_rng(0).standard_normal((2048, 4096)).astype(np.float32)
    _nf4_check(x)


def test_nf4dq_config2_outlier_columns():
    """BASELINE config 2 shape (4096x4096) with 16 columns scaled x60."""
    rng = np.random.default_rng(0)
    x = rng.standard_normal((4096, 4096)).astype(np.float32)
    cols = np.random.default_rng(1).permutation(4096)[:16]
    x[:, cols] *= 60.0
    _nf4dq_check(x)


def test_nf4_special_values():
    x = np.zeros(64 * 6, np.float32)
    x[64:128] = np.nan
    x[130] = np.inf
    x[131] = -np.inf
    x[192:256] = 1e-42        # denormal block
    x[256:320] = np.linspace(-3e38, 3e38, 64)
    x[320:] = -0.0
    _nf4_check(x)
    _nf4dq_check(x)


def test_nf4dq_tiny_blocks_next_to_huge():
    """Blocks whose absmax/dq underflows E4M3 decode with scale 1 (and push
    the code search into its large-|v| branch)."""
    x = np.random.default_rng(5).standard_normal(64 * 8).astype(np.float32)
    x[:64] *= 1e30
    x[64:128] *= 1e6
    x[128:192] *= 1e-3
    _nf4dq_check(x)
