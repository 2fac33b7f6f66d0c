"""The public ABI end to end on the GPU (direct path): packed bytes equal the
oracle's packed bytes (payload pointer masked), decoded matrices equal the
oracle's decode bit for bit, and the lifecycle / negative-path contract of the
reference's ABI tests (tests/bitsqz_llm/test_quantization.cpp:129-461)."""
import ctypes as C

import numpy as np
import pytest

import bitsqz_amd as B
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def ref_source(rows, cols, a=0.11, b=0.07):
    """The reference ABI tests' matrix: sin(a*idx) + cos(b*(r+c)) in float32
    (test_quantization.cpp:487-492)."""
    idx = np.arange(rows * cols, dtype=np.int64).reshape(rows, cols)
    r = np.arange(rows)[:, None]
    c = np.arange(cols)[None, :]
    return (np.sin(np.float32(a) * idx.astype(np.float32)) +
            np.cos(np.float32(b) * (r + c).astype(np.float32))).astype(np.float32)


def run_direct(x, outlier=0.0, error=0.0, fmt=B.NF4, loc=B.INPUT_DEVICE):
    rows, cols = x.shape
    B.compress_release()
    B.decompress_release()
    assert B.compress_initialize(rows, cols, outlier, error, -1, 2, B.QUANT_NONE, B.QUANT_NONE, fmt, loc) == 0
    assert B.decompress_initialize(rows, cols, outlier, error, -1, B.QUANT_NONE, B.QUANT_NONE, fmt) == 0
    src = B.DeviceBuffer.from_array(x) if loc == B.INPUT_DEVICE else x
    data, prof = B.compress(src, profile=True)
    out = B.decompress(data, rows, cols)
    return data, out, prof


def oracle_direct(x, outlier=0.0, error=0.0, fmt=B.NF4):
    cfg = O.Config(x.shape[0], x.shape[1], outlier, error, -1, 2, O.QUANT_NONE, O.QUANT_NONE, fmt)
    p = O.compress(x, cfg)
    return p.to_bytes(), O.decompress(p)


CASES = [
    # (name, rows, cols, outlier, error, fmt, location)  -- reference test_quantization.cpp:515-519
    ("quantization_only_nf4", 512, 8192, 0.0, 0.0, B.NF4, B.INPUT_DEVICE),
    ("quantization_only_nf4_host", 512, 8192, 0.0, 0.0, B.NF4, B.INPUT_HOST),
    ("quantization_plus_error_nf4", 512, 8192, 0.0, 0.10, B.NF4, B.INPUT_DEVICE),
    ("outlier_plus_quantization_nf4_dq", 512, 8192, 0.05, 0.0, B.NF4_DQ, B.INPUT_DEVICE),
    ("outlier_quantization_error_nf4_dq", 512, 8192, 0.05, 0.10, B.NF4_DQ, B.INPUT_DEVICE),
    ("fp32_direct_outlier", 256, 1000, 0.02, 0.0, B.QUANT_NONE, B.INPUT_HOST),
    ("fp32_direct_plain", 64, 64, 0.0, 0.3, B.QUANT_NONE, B.INPUT_DEVICE),
    ("odd_shape_nf4_error", 37, 101, 0.03, 0.07, B.NF4, B.INPUT_DEVICE),
    ("odd_shape_nf4dq_error", 33, 99, 0.0, 0.5, B.NF4_DQ, B.INPUT_HOST),
    # the headline width: 11 column quads per lane in the register top-k
    ("wide_nf4dq_outlier_error", 128, 11008, 0.005, 0.01, B.NF4_DQ, B.INPUT_DEVICE),
    ("wide_nf4_error", 64, 11008, 0.0, 0.01, B.NF4, B.INPUT_DEVICE),
]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_direct_path_bytes_and_decode(case):
    name, rows, cols, ro, re, fmt, loc = case
    x = ref_source(rows, cols)
    data, out, prof = run_direct(x, ro, re, fmt, loc)
    exp_bytes, exp_out = oracle_direct(x, ro, re, fmt)
    assert len(data) == len(exp_bytes)
    assert O.mask_pointer(data) == O.mask_pointer(exp_bytes)
    assert out.tobytes() == exp_out.tobytes()
    assert prof.other_latency_ms >= 0.0


def test_config1_2048x4096_nf4():
    x = np.random.default_rng(0).standard_normal((2048, 4096)).astype(np.float32)
    data, out, _ = run_direct(x, 0.0, 0.0, B.NF4)
    exp_bytes, exp_out = oracle_direct(x, 0.0, 0.0, B.NF4)
    assert len(data) == 4718840
    assert O.mask_pointer(data) == O.mask_pointer(exp_bytes)
    assert out.tobytes() == exp_out.tobytes()


def test_config2_4096x4096_nf4dq_outliers():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((4096, 4096)).astype(np.float32)
    cols = np.random.default_rng(1).permutation(4096)[:16]
    x[:, cols] *= 60.0
    data, out, _ = run_direct(x, 0.005, 0.0, B.NF4_DQ)
    exp_bytes, exp_out = oracle_direct(x, 0.005, 0.0, B.NF4_DQ)
    assert len(data) == 9142528
    assert O.mask_pointer(data) == O.mask_pointer(exp_bytes)
    assert out.tobytes() == exp_out.tobytes()


def test_direct_full_4096x11008_nf4dq_outlier_error():
    """The benched direct workload at full size: the headline matrix (rank-512
    spectrum i^-1.2 + noise 0.01, 8 columns x50) through the direct path with
    NF4_DQ, outlier top-k 0.005 (55 per row) and error top-k 0.01 (110 per
    row): packed bytes and decode equal the oracle's, through the ABI and the
    device-resident twin."""
    from _svdcase import lowrank, outlier_columns
    x = outlier_columns(lowrank(4096, 11008, 512, 1.2, 0.01, seed=0), 8, 50.0)
    rows, cols = x.shape
    data, out, _ = run_direct(x, 0.005, 0.01, B.NF4_DQ)
    exp_bytes, exp_out = oracle_direct(x, 0.005, 0.01, B.NF4_DQ)
    assert len(data) == len(exp_bytes)
    assert O.mask_pointer(data) == O.mask_pointer(exp_bytes)
    assert out.tobytes() == exp_out.tobytes()
    src = B.DeviceBuffer.from_array(x)
    dst = B.DeviceBuffer(rows * cols * 4)
    packed = B.device_compress(src)
    B.device_decompress(packed, dst, rows * cols)
    B.device_synchronize()
    assert dst.download(np.float32, rows * cols).reshape(rows, cols).tobytes() == exp_out.tobytes()
    B.compress_release()
    B.decompress_release()


@pytest.mark.parametrize("rows,cols,hot", [
    (48, 4096, 24), (40, 1000, 20), (16, 11008, 8),
    (42, 4096, 41),     # rows % 4 != 0: the maxima go through the reduce launch
    (4096, 128, 4095),  # the most rows the encode kernels reduce themselves, largest in the last
    (4096, 128, 2900),  # ... largest in the last of each lane's four loads
    (4100, 128, 4099),  # more rows: the reduce launch
])
def test_nf4dq_global_scale_from_the_outlier_separation(rows, cols, hot):
    """The direct NF4_DQ section's global scale comes from the outlier
    separation kernel's per-row block maxima when cols % 64 == 0 (and from the
    separate reduction otherwise), reduced inside the encode pass for up to
    4096 rows (a multiple of 4) and by a reduce launch beyond: bytes and
    decode equal the oracle's with all-zero blocks (which count as 1), NaN and
    infinity left in the residual (sanitised to 0), and the largest block
    absmax in row `hot`, through the fused encode + error pass and through
    the encode alone (no error set)."""
    rng = np.random.default_rng(rows + cols)
    x = (rng.standard_normal((rows, cols)) * 0.01).astype(np.float32)
    x[0, :192] = 0.0                        # all-zero blocks in row 0
    x[hot] *= 500.0                          # the largest residual block sits in one row
    x[1, 5], x[2, 70] = np.nan, np.inf       # NaN is never an outlier; +inf is
    x[3, 9] = -np.inf
    for re in (0.02, 0.0):
        data, out, _ = run_direct(x, 0.01, re, B.NF4_DQ)
        exp_bytes, exp_out = oracle_direct(x, 0.01, re, B.NF4_DQ)
        assert O.mask_pointer(data) == O.mask_pointer(exp_bytes)
        assert out.tobytes() == exp_out.tobytes()
    # no outlier selection: the separate reduction
    data, out, _ = run_direct(x, 0.0, 0.02, B.NF4_DQ)
    exp_bytes, exp_out = oracle_direct(x, 0.0, 0.02, B.NF4_DQ)
    assert O.mask_pointer(data) == O.mask_pointer(exp_bytes)
    assert out.tobytes() == exp_out.tobytes()


def test_error_section_absent_when_exact():
    """A matrix the NF4 codec reproduces exactly has no error section even with
    error top-k enabled (has_nonzero gate, src/bitsqz_llm.cu:1210-1225)."""
    x = np.tile(np.array([1.0, -1.0, 0.0, 0.5626170039176941], np.float32), (8, 16))
    data, out, _ = run_direct(x, 0.0, 0.25, B.NF4)
    p = O.parse_packed(data)
    assert not (p.flags & O.FLAG_ERROR) and "error" not in p.sections
    exp_bytes, exp_out = oracle_direct(x, 0.0, 0.25, B.NF4)
    assert O.mask_pointer(data) == O.mask_pointer(exp_bytes)
    assert out.tobytes() == exp_out.tobytes()


def test_reload_and_negative_paths():
    """run_case's reload and failure checks (test_quantization.cpp:330-421)."""
    rows, cols, ro, re, fmt = 128, 512, 0.02, 0.03, B.NF4
    x = ref_source(rows, cols, 0.09, 0.05)
    data, out, _ = run_direct(x, ro, re, fmt)
    dst = B.DeviceBuffer(rows * cols * 4)
    # reload consistency
    assert B.decompress_to_device(data, dst, rows * cols) == 0
    assert np.array_equal(dst.download(np.float32, rows * cols).reshape(rows, cols), out)
    # destination too small
    assert B.decompress_to_device(data, dst, rows * cols - 1) == 1
    # after release
    B.decompress_release()
    assert B.decompress_to_device(data, dst, rows * cols) == 1
    # shape mismatch
    assert B.decompress_initialize(rows, cols - 1, ro, re, -1, B.QUANT_NONE, B.QUANT_NONE, fmt) == 0
    assert B.decompress_to_device(data, dst, rows * cols) == 1
    # no quantisation runtime
    assert B.decompress_initialize(rows, cols, ro, re, -1, B.QUANT_NONE, B.QUANT_NONE, B.QUANT_NONE) == 0
    assert B.decompress_to_device(data, dst, rows * cols) == 1
    # insufficient top-k capacity (smaller_topk_ratio, test_quantization.cpp:43-55)
    def smaller(ratio):
        k = B.topk_num_columns(cols, ratio)
        return 0.0 if k <= 1 else (np.float32(k - 1) - np.float32(0.49)) / np.float32(cols)
    assert B.decompress_initialize(rows, cols, float(smaller(ro)), float(smaller(re)), -1, B.QUANT_NONE,
                                   B.QUANT_NONE, fmt) == 0
    assert B.decompress_to_device(data, dst, rows * cols) == 1
    # corrupted quant magic
    bad = bytearray(data)
    bad[200] ^= 0xFF
    assert B.decompress_initialize(rows, cols, ro, re, -1, B.QUANT_NONE, B.QUANT_NONE, fmt) == 0
    assert B.decompress_to_device(bytes(bad), dst, rows * cols) == 1
    # flags / section mismatch
    bad = bytearray(data)
    bad[40] |= 1  # claims SVD
    assert B.decompress_to_device(bytes(bad), dst, rows * cols) == 1
    assert B.decompress_to_device(data, dst, rows * cols) == 0
    B.decompress_release()
    B.compress_release()


def test_lifecycle():
    """run_lifecycle_checks (test_quantization.cpp:129-230)."""
    rows, cols = 128, 512
    x = ref_source(rows, cols, 0.09, 0.05)
    src = B.DeviceBuffer.from_array(x)
    dst = B.DeviceBuffer(rows * cols * 4)
    B.compress_release()
    B.decompress_release()
    with pytest.raises(B.BsqError):
        B.compress(src)
    args = (rows, cols, 0.02, 0.03)
    assert B.compress_initialize(*args, -1, 2, B.QUANT_NONE, B.QUANT_NONE, B.NF4, B.INPUT_DEVICE) == 0
    assert B.decompress_initialize(*args, -1, B.QUANT_NONE, B.QUANT_NONE, B.NF4) == 0
    data = B.compress(src)
    assert B.decompress_to_device(data, dst, rows * cols) == 0
    B.compress_release()
    with pytest.raises(B.BsqError):
        B.compress(src)
    assert B.decompress_to_device(data, dst, rows * cols) == 0       # survives compressor release
    assert B.compress_initialize(*args, -1, 2, B.QUANT_NONE, B.QUANT_NONE, B.NF4, B.INPUT_DEVICE) == 0
    B.decompress_release()
    assert B.decompress_to_device(data, dst, rows * cols) == 1
    data2 = B.compress(src)                                            # survives decompressor release
    assert O.mask_pointer(data2) == O.mask_pointer(data)
    # *out must be null on entry
    out = C.POINTER(B.PackedHeader)(B.PackedHeader())
    assert B.lib().bsq_compress(src.ptr, C.byref(out), None) == 1
    B.compress_release()


@pytest.mark.parametrize("fmt,ro,re", [(B.NF4, 0.0, 0.0), (B.NF4_DQ, 0.005, 0.01), (B.NF4, 0.02, 0.05)])
def test_device_resident_matches_abi(fmt, ro, re):
    rows, cols = 256, 4096
    x = np.random.default_rng(4).standard_normal((rows, cols)).astype(np.float32)
    data, out, _ = run_direct(x, ro, re, fmt)
    src = B.DeviceBuffer.from_array(x)
    dst = B.DeviceBuffer(rows * cols * 4)
    packed = B.device_compress(src)
    B.device_decompress(packed, dst, rows * cols)
    B.device_synchronize()
    assert np.array_equal(dst.download(np.float32, rows * cols).reshape(rows, cols), out)
    B.compress_release()
    B.decompress_release()


@pytest.mark.parametrize("ro", [0.0, 0.02])
def test_fused_encode_blocks_below_the_scale_range(ro):
    """NF4_DQ blocks far below the global maximum get E4M3 scale code 0,
    replaced by 1, so their scaled values leave the table's |w| < 2 range and
    take the exact nearest-level scan inside the fused encode + error pass
    (cols % 64 == 0, with and without the selection bitmap of an outlier
    separation); bytes and decode equal the oracle's."""
    rows, cols = 16, 1024
    rng = np.random.default_rng(5)
    x = rng.standard_normal((rows, cols)).astype(np.float32)
    x[0] *= 1e9                                  # sets the global scale
    x[3, :64] *= 1e-3                            # blocks at, below and far below the E4M3 range
    x[5, 128:256] *= 1e-7
    x[7, 512:576] = np.float32(1e-30)
    data, out, _ = run_direct(x, ro, 0.05, B.NF4_DQ)
    exp_bytes, exp_out = oracle_direct(x, ro, 0.05, B.NF4_DQ)
    assert O.mask_pointer(data) == O.mask_pointer(exp_bytes)
    assert out.tobytes() == exp_out.tobytes()
    B.compress_release()
    B.decompress_release()


def test_reused_host_objects_alternating_error_sections():
    """Packed objects freed with bitsqz_llm_free are reused by the next
    compress: alternating an input with an error section and one the codec
    reproduces exactly (no error section, a smaller object in the same
    block), with and without a profile struct, every object equals the
    oracle's bytes and decodes like it (objects of about 1.8 MB: large
    enough to be kept)."""
    rows, cols = 1024, 2048
    rng = np.random.default_rng(21)
    x_err = rng.standard_normal((rows, cols)).astype(np.float32)
    x_exact = np.tile(np.array([1.0, -1.0, 0.0, 0.5626170039176941], np.float32), (rows, cols // 4))
    B.compress_release()
    B.decompress_release()
    assert B.compress_initialize(rows, cols, 0.0, 0.05, -1, 2, B.QUANT_NONE, B.QUANT_NONE, B.NF4, B.INPUT_HOST) == 0
    assert B.decompress_initialize(rows, cols, 0.0, 0.05, -1, B.QUANT_NONE, B.QUANT_NONE, B.NF4) == 0
    expect = {name: oracle_direct(x, 0.0, 0.05, B.NF4) for name, x in (("err", x_err), ("exact", x_exact))}
    assert len(expect["exact"][0]) < len(expect["err"][0])
    for i in range(6):
        name, x = ("err", x_err) if i % 2 == 0 else ("exact", x_exact)
        got = B.compress(x, profile=(i % 3 == 0))
        data = got[0] if isinstance(got, tuple) else got
        assert O.mask_pointer(data) == O.mask_pointer(expect[name][0]), (i, name)
        out = B.decompress(data, rows, cols)
        assert out.tobytes() == expect[name][1].tobytes(), (i, name)
    B.compress_release()
    B.decompress_release()


def _device_flags(packed):
    out = np.zeros(1, np.uint32)
    B.check(B.lib().bsq_memcpy_d2h(out.ctypes.data_as(C.c_void_p), C.c_void_p(packed.d_flags), 4), "D2H")
    return int(out[0])


@pytest.mark.parametrize("fmt", [B.NF4, B.NF4_DQ])
def test_device_flags_word_of_each_direct_variant(fmt):
    """The device flags word of bsq_device_compress: bit 2 (error section
    present) set after a compress with an error pass, and the word 0 after a
    quant-only one (cleared by the encode kernel itself there, not by a fill)
    even right after a compress that set it."""
    rows, cols = 64, 4096
    x = np.random.default_rng(9).standard_normal((rows, cols)).astype(np.float32)
    for ro, re, want in [(0.0, 0.1, 4), (0.0, 0.0, 0), (0.02, 0.1, 4), (0.02, 0.0, 0), (0.0, 0.0, 0)]:
        run_direct(x, ro, re, fmt)
        src = B.DeviceBuffer.from_array(x)
        for _ in range(2):
            packed = B.device_compress(src)
            B.device_synchronize()
            word = _device_flags(packed)
            assert (word & 4 if want else word) == want, (ro, re, word)
        src.free()
    B.compress_release()
    B.decompress_release()


@pytest.mark.parametrize("rows,cols,fmt,ro,re", [
    (37, 101, B.NF4, 0.03, 0.07),        # ragged width: element-wise decode of the fused row pass
    (33, 99, B.NF4_DQ, 0.02, 0.5),
    (16, 4096, B.NF4, 0.15, 0.2),        # k = 614 and 819 per row: entries past the first 512
    (8, 4096, B.NF4, 0.0, 0.3),          # error set only
    (24, 4096, B.NF4_DQ, 0.05, 0.0),     # outlier set only
    (32, 4096, B.NF4, 0.05, 0.0),        # outlier set only, NF4: the encode reads the input and the selection bitmap
    (12, 2048, B.NF4, 0.2, 0.1),         # k_o = 409 per row: the separation writes a residual (LDS kernel)
    (64, 11008, B.NF4_DQ, 0.005, 0.01),  # the headline width
])
def test_device_resident_direct_decode_fused_with_the_scatter(rows, cols, fmt, ro, re):
    """bsq_device_decompress decodes a direct section and adds both top-k sets
    in one pass over the rows (error set gated by the compress flags, then the
    outlier set); the result equals the host ABI's decode + scatter and the
    oracle's decode bit for bit."""
    x = ref_source(rows, cols, 0.13, 0.05)
    x[::5, ::7] *= 40.0  # outlier columns in some rows
    data, out, _ = run_direct(x, ro, re, fmt)
    _, exp_out = oracle_direct(x, ro, re, fmt)
    assert out.tobytes() == exp_out.tobytes()
    src = B.DeviceBuffer.from_array(x)
    dst = B.DeviceBuffer(rows * cols * 4)
    dst.zero()
    packed = B.device_compress(src)
    B.device_decompress(packed, dst, rows * cols)
    B.device_synchronize()
    assert dst.download(np.float32, rows * cols).reshape(rows, cols).tobytes() == exp_out.tobytes()
    B.compress_release()
    B.decompress_release()


@pytest.mark.parametrize("fmt", [B.NF4, B.NF4_DQ])
def test_direct_separation_keys_edge_rows(fmt):
    """The quantised direct path with an outlier separation and an error
    pass (cols % 64 == 0: the encode and the error top-k run as one fused
    pass over the residual).  Rows whose k-th entry is a NaN (fewer than k
    numbers: every number and the lowest-column NaNs are separated), ties at
    the k-th magnitude (lower columns win), infinities, all-zero and
    signed-zero rows give the oracle's bytes and decode, through the ABI and
    the device-resident twin."""
    rows, cols = 24, 512
    rng = np.random.default_rng(11)
    x = rng.standard_normal((rows, cols)).astype(np.float32)
    x[0, :] = np.nan
    x[0, rng.permutation(cols)[:10]] = rng.standard_normal(10).astype(np.float32)  # 10 numbers < k
    x[1, :] = np.where(np.arange(cols) % 2 == 0, 1.0, -1.0).astype(np.float32)    # all tied
    x[2, rng.permutation(cols)[:30]] = np.float32(np.inf)
    x[2, 7] = -np.inf
    x[3, :] = 0.0
    x[4, :] = np.where(np.arange(cols) % 3 == 0, -0.0, 0.0).astype(np.float32)
    x[5, 100:140] = np.float32(3.5)  # a tie run straddling the k-th rank
    ro, re = 0.05, 0.1
    assert O.topk_num_columns(cols, ro) == 26 and O.topk_num_columns(cols, re) == 51
    data, out, _ = run_direct(x, ro, re, fmt)
    exp_bytes, exp_out = oracle_direct(x, ro, re, fmt)
    assert O.mask_pointer(data) == O.mask_pointer(exp_bytes)
    assert out.tobytes() == exp_out.tobytes()
    src = B.DeviceBuffer.from_array(x)
    dst = B.DeviceBuffer(rows * cols * 4)
    packed = B.device_compress(src)
    B.device_decompress(packed, dst, rows * cols)
    B.device_synchronize()
    assert dst.download(np.float32, rows * cols).reshape(rows, cols).tobytes() == exp_out.tobytes()
    B.compress_release()
    B.decompress_release()
