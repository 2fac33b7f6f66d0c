"""CPU-side checks of the built library: it loads, exports every symbol the
headers declare (the nine C++-linkage names of the reference ABI with their
exact mangling, reference include/bitsqz_llm.hpp:95-141), and its host-only
entry points (argument validation, packed-size, load) behave as the
reference's (src/bitsqz_llm.cu:785-804, 887-897, 981-987, 1304-1310,
1395-1455).  No GPU work is started here."""
import ctypes as C
import os
import re
import struct
import subprocess
import sys

import numpy as np
import pytest

import bitsqz_amd as B

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

# Mangled names of the reference's C++-linkage ABI (bitsqz_llm.hpp:95-141)
# plus topk_compute_num_topk_columns (topk_cuda.cuh, linked by the reference's
# ABI tests).
MANGLED = [
    "_Z30bitsqz_llm_compress_initializettffii21quantization_method_tS_S_27bitsqz_llm_input_location_t",
    "_Z27bitsqz_llm_compress_releasev",
    "_Z32bitsqz_llm_decompress_initializettffi21quantization_method_tS_S_",
    "_Z29bitsqz_llm_decompress_releasev",
    "_Z19bitsqz_llm_compressPKfPP16bitsqz_llm_arrayP29bitsqz_llm_compress_profile_t",
    "_Z21bitsqz_llm_decompressPK16bitsqz_llm_arrayPfj",
    "_Z26bitsqz_llm_get_packed_sizePK16bitsqz_llm_array",
    "_Z27load_bitsqz_llm_from_bufferPKvm",
    "_Z15bitsqz_llm_freeP16bitsqz_llm_array",
    "_Z29topk_compute_num_topk_columnstf",
]


def exported():
    out = subprocess.run(["nm", "-D", "--defined-only", B.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    return {line.split()[-1] for line in out.splitlines() if line.strip()}


def c_header_functions():
    txt = open(os.path.join(ROOT, "include", "bitsqz_llm_c.h")).read()
    return set(re.findall(r"BSQ_API\s+[\w\s\*]+?\b(bsq_\w+)\s*\(", txt))


def test_library_built_and_loads():
    assert os.path.exists(B.LIB_PATH)
    assert B.lib().bsq_version().decode().startswith("bitsqz_llm")


def test_exports_reference_mangled_abi():
    syms = exported()
    missing = [m for m in MANGLED if m not in syms]
    assert not missing, missing


def test_exports_every_c_header_function():
    syms = exported()
    decl = c_header_functions()
    assert len(decl) >= 30
    missing = sorted(d for d in decl if d not in syms)
    assert not missing, missing


def test_soname_matches_reference_library():
    out = subprocess.run(["readelf", "-d", B.LIB_PATH], capture_output=True, text=True, check=True).stdout
    assert "libbitsqz_llm_lib.so.0" in out


def test_struct_layout():
    assert C.sizeof(B.PackedHeader) == 200
    offs = [getattr(B.PackedHeader, n).offset for n in
            ("section_u", "section_s", "section_v", "section_direct", "section_outlier_topk",
             "section_error_topk", "payload")]
    assert offs == [48, 72, 96, 120, 144, 168, 192]
    assert C.sizeof(B.Profile) == 56


def test_topk_num_columns_matches_reference_rounding():
    # roundf(cols * ratio), clamped to [1, cols] for ratio > 0 (topk_cuda.cu:53-69)
    cases = {(4096, 0.005): 20, (4096, 0.01): 41, (14336, 0.002): 29, (14336, 0.005): 72,
             (11008, 0.005): 55, (11008, 0.01): 110, (6, 0.5): 3, (8, 0.01): 1, (8, 1.0): 8, (8, 0.0): 0,
             (5, 0.4): 2, (512, 0.03): 15}
    for (cols, r), k in cases.items():
        assert B.topk_num_columns(cols, r) == k, (cols, r)
    with pytest.raises(B.BsqError):
        B.topk_num_columns(8, 1.5)


def test_compress_initialize_rejects_invalid_arguments():
    bad = [
        dict(rows=0, cols=8), dict(rows=8, cols=0),
        dict(rows=8, cols=8, outlier_ratio=-0.1), dict(rows=8, cols=8, error_ratio=1.5),
        dict(rows=8, cols=8, outlier_ratio=float("nan")),
        dict(rows=8, cols=8, uv_format=0),  # Q8_0 is rejected (test_quantization.cpp:469-483)
        dict(rows=8, cols=8, direct_format=5),
        dict(rows=8, cols=8, input_location=2),
        dict(rows=8, cols=8, svd_niters=0),
    ]
    for kw in bad:
        rows, cols = kw.pop("rows"), kw.pop("cols")
        assert B.compress_initialize(rows, cols, **kw) == 1, kw
    assert B.decompress_initialize(8, 8, uv_format=3) == 1
    assert B.decompress_initialize(0, 8) == 1


def test_calls_before_initialize_fail():
    B.compress_release()
    B.decompress_release()
    out = C.POINTER(B.PackedHeader)()
    x = np.zeros(64, np.float32)
    assert B.lib().bsq_compress(x.ctypes.data_as(C.c_void_p), C.byref(out), None) == 1
    hdr = B.PackedHeader()
    assert B.lib().bsq_decompress(C.cast(C.pointer(hdr), C.c_void_p), C.c_void_p(16), 64) == 1


def _fake_object(sections):
    """A packed object whose header has the given (offset, size, storage) sections."""
    hdr = B.PackedHeader()
    hdr.num_rows, hdr.num_columns, hdr.num_elements = 2, 4, 8
    names = ["section_u", "section_s", "section_v", "section_direct", "section_outlier_topk",
             "section_error_topk"]
    end = 0
    for name, (off, size, st) in zip(names, sections):
        s = getattr(hdr, name)
        s.offset, s.size, s.storage = off, size, st
        if st:
            end = max(end, off + size)
    return bytes(hdr) + bytes(end), end


def test_get_packed_size_and_load_validation():
    L = B.lib()
    assert L.bsq_get_packed_size(None) == 0
    buf, end = _fake_object([(0, 0, 0)] * 3 + [(0, 32, 1), (0, 0, 0), (0, 0, 0)])
    b = C.create_string_buffer(buf, len(buf))
    p = L.bsq_load_from_buffer(b, len(buf))
    assert p
    vp = C.cast(p, C.c_void_p)
    assert L.bsq_get_packed_size(vp) == 200 + 32
    # the payload pointer is re-pointed at the copy's own payload
    assert p.contents.payload == vp.value + 200
    L.bsq_free(vp)
    # truncated buffer, short header, bad storage kind, NONE with a size
    assert not L.bsq_load_from_buffer(b, len(buf) - 1)
    assert not L.bsq_load_from_buffer(b, 100)
    for secs in ([(0, 0, 0)] * 3 + [(0, 32, 7), (0, 0, 0), (0, 0, 0)],
                 [(0, 0, 0)] * 3 + [(0, 0, 1), (0, 0, 0), (0, 0, 0)],
                 [(0, 4, 0)] + [(0, 0, 0)] * 2 + [(0, 32, 1), (0, 0, 0), (0, 0, 0)]):
        buf2, _ = _fake_object(secs)
        b2 = C.create_string_buffer(buf2, max(len(buf2), 200))
        assert not L.bsq_load_from_buffer(b2, max(len(buf2), 200)), secs


def test_device_thresholds_pinned_against_reference_scan():
    """The device NF4 code function uses code = #{T <= v} for |v| < 2; the
    thresholds it uses agree with the reference's linear scan on every float
    with |v| < 2 (2^31 bit patterns, CPU oracle)."""
    from oracle import oracle as O
    t = B.nf4_thresholds()
    assert np.all(np.diff(t) > 0)
    lv = O.nf4_levels()
    assert np.all((t > lv[:-1]) & (t < lv[1:]))
    assert O.nf4_threshold_mismatches(t) == 0


def test_device_code_table_pinned_against_reference_scan():
    """The device NF4 code function reads code = lo[b] + (v >= thr[b]) from a
    256-bin table over [-1, 1] (clamped outside); built with the same float
    arithmetic, the rule equals the reference's linear scan on every float
    with |v| < 2 (2^31 bit patterns, CPU oracle)."""
    from oracle import oracle as O
    assert O.nf4_table_mismatches(B.nf4_thresholds()) == 0
    # a plausible slip is caught: one threshold moved by one ulp
    t = B.nf4_thresholds().copy()
    t[7] = np.nextafter(t[7], np.float32(1.0))
    assert O.nf4_table_mismatches(t) > 0


def _valid_object() -> bytes:
    """A well-formed packed object (SVD sections U, S, V as NF4 / FP32 / NF4, an
    outlier blob), built by the oracle's byte-layout restatement."""
    from oracle import oracle as O
    rng = np.random.default_rng(7)
    rows, cols, q = 16, 24, 4
    U = rng.standard_normal(rows * q).astype(np.float32)
    V = rng.standard_normal(cols * q).astype(np.float32)
    S = np.abs(rng.standard_normal(q)).astype(np.float32)
    idx = np.tile(np.arange(2, dtype=np.uint16), (rows, 1))
    val = rng.standard_normal((rows, 2)).astype(np.float32)
    p = O.Packed(rows, cols, 0.1, 0.0, q, 2, q, O.NF4, O.QUANT_NONE, O.QUANT_NONE, 0b011)
    p.sections["u"] = (O.SECTION_QUANT, O.pack_quant(O.quant_compress(U, O.NF4)))
    p.sections["s"] = (O.SECTION_FP32, S.tobytes())
    p.sections["v"] = (O.SECTION_QUANT, O.pack_quant(O.quant_compress(V, O.NF4)))
    p.sections["outlier"] = (O.SECTION_TOPK, O.pack_topk(rows, cols, idx, val))
    return p.to_bytes()


def test_load_fuzz_corpus_matches_reference_checks():
    """Seeded corruptions of a valid object's section table and length: the
    library's load_bitsqz_llm_from_buffer accepts exactly the buffers that the
    reference's checks accept (oracle load_accepts restates
    src/bitsqz_llm.cu:319-332, 1395-1450), reports the same packed size for
    them, and copies every byte except the re-pointed payload pointer."""
    from oracle import oracle as O
    L = B.lib()
    base = _valid_object()
    assert O.load_accepts(base)
    rng = np.random.default_rng(20260101)
    U64 = (1 << 64) - 1
    payload = len(base) - 200
    special = [0, 1, 2, 7, payload - 1, payload, payload + 1, payload // 2, 1 << 32, 1 << 63, U64, U64 - 150,
               U64 - 199, U64 - 200, U64 - 201, U64 - payload]
    accepted = rejected = 0
    for case in range(3000):
        b = bytearray(base)
        for _ in range(int(rng.integers(1, 4))):
            kind = int(rng.integers(0, 5))
            sec = 48 + 24 * int(rng.integers(0, 6))
            if kind == 0:    # offset
                v = special[int(rng.integers(len(special)))] if rng.random() < 0.6 else int(rng.integers(0, 2 * payload))
                struct.pack_into("<Q", b, sec, v & U64)
            elif kind == 1:  # size
                v = special[int(rng.integers(len(special)))] if rng.random() < 0.6 else int(rng.integers(0, 2 * payload))
                struct.pack_into("<Q", b, sec + 8, v & U64)
            elif kind == 2:  # storage kind
                b[sec + 16] = int(rng.choice([0, 1, 2, 3, 4, 255]))
            elif kind == 3:  # length
                cut = int(rng.integers(-64, 65))
                b = b[:max(0, len(b) + cut)] if cut < 0 else b + bytes(cut)
            else:            # a random byte of the section table
                b[48 + int(rng.integers(0, 144))] = int(rng.integers(0, 256))
        buf = bytes(b)
        want = O.load_accepts(buf)
        cb = C.create_string_buffer(buf, max(len(buf), 1))
        p = L.bsq_load_from_buffer(cb, len(buf))
        assert bool(p) == want, (case, [struct.unpack_from("<QQB", buf, 48 + 24 * i) for i in range(6)]
                                 if len(buf) >= 192 else len(buf))
        if p:
            accepted += 1
            vp = C.cast(p, C.c_void_p)
            assert L.bsq_get_packed_size(vp) == O.packed_size(buf)
            got = C.string_at(vp.value, len(buf))
            assert O.mask_pointer(got) == O.mask_pointer(buf)
            assert struct.unpack_from("<Q", got, 192)[0] == vp.value + 200
            L.bsq_free(vp)
        else:
            rejected += 1
    assert accepted > 100 and rejected > 100, (accepted, rejected)


def test_load_rejects_wrapped_payload_end():
    """A section ending within 200 bytes of 2^64 makes the reference's wrapping
    packed size fall below 200, so its checks accept a header whose section lies
    far outside the buffer; this build rejects it (the one intended difference)."""
    from oracle import oracle as O
    buf = bytearray(_valid_object())
    for i in range(6):
        struct.pack_into("<QQB", buf, 48 + 24 * i, 0, 0, 0)
    U64 = (1 << 64) - 1
    struct.pack_into("<QQB", buf, 48, U64 - 150, 100, 1)  # FP32 section at 2^64 - 150
    buf = bytes(buf)
    payload = (O.packed_size(buf) - 200) & U64
    assert O.packed_size(buf) < 200 and O.section_bounds_ok(U64 - 150, 100, 1, payload)
    assert not O.load_accepts(buf)
    cb = C.create_string_buffer(buf, len(buf))
    assert not B.lib().bsq_load_from_buffer(cb, len(buf))


# ------------------------------------------------------- installed package --
INSTALL = os.path.join(ROOT, "bitsqueeze-llm_amd", "_install")
CONSUMER = os.path.join(ROOT, "tests", "cmake_consumer", "_build", "bsq_consumer")


def test_installed_cmake_package_layout():
    """The package the reference's downstream users consume
    (CMakeLists.txt:60-124, cmake/bitsqz_llmConfig.cmake.in:1-13): the
    versioned library with the reference's SONAME, both headers, and a config
    exporting bitsqz_llm::bitsqz_llm with hip::host as a public dependency."""
    lib = os.path.join(INSTALL, "lib")
    cm = os.path.join(lib, "cmake", "bitsqz_llm")
    for f in ("libbitsqz_llm_lib.so.0.1.0", "libbitsqz_llm_lib.so.0", "libbitsqz_llm_lib.so"):
        assert os.path.exists(os.path.join(lib, f)), f
    assert os.path.realpath(os.path.join(lib, "libbitsqz_llm_lib.so")).endswith("libbitsqz_llm_lib.so.0.1.0")
    for f in ("bitsqz_llm.hpp", "bitsqz_llm_c.h"):
        assert os.path.exists(os.path.join(INSTALL, "include", f)), f
    cfg = open(os.path.join(cm, "bitsqz_llmConfig.cmake")).read()
    assert "find_dependency(hip" in cfg
    targets = open(os.path.join(cm, "bitsqz_llmTargets.cmake")).read()
    assert "bitsqz_llm::bitsqz_llm" in targets and "hip::host" in targets
    assert 'PACKAGE_VERSION "0.1.0"' in open(os.path.join(cm, "bitsqz_llmConfigVersion.cmake")).read()
    out = subprocess.run(["readelf", "-d", os.path.join(lib, "libbitsqz_llm_lib.so.0.1.0")], capture_output=True,
                         text=True, check=True).stdout
    assert "[libbitsqz_llm_lib.so.0]" in out
    syms = subprocess.run(["nm", "-D", "--defined-only", os.path.join(lib, "libbitsqz_llm_lib.so.0.1.0")],
                          capture_output=True, text=True, check=True).stdout
    assert all(m in syms for m in MANGLED)


def test_consumer_links_the_nine_mangled_functions():
    """The downstream program (tests/cmake_consumer, built through
    find_package against the installed package) binds all nine C++-linkage
    functions by their reference mangling and loads the installed library."""
    undef = subprocess.run(["nm", "--undefined-only", CONSUMER], capture_output=True, text=True,
                           check=True).stdout
    assert all(m in undef for m in MANGLED[:9])
    dyn = subprocess.run(["readelf", "-d", CONSUMER], capture_output=True, text=True, check=True).stdout
    assert "libbitsqz_llm_lib.so.0" in dyn and os.path.join(INSTALL, "lib") in dyn


def test_bench_refuses_more_than_one_gpu():
    """bench.py measures one GPU: --gpus above 1 exits with status 2 and a
    message that says so, before anything touches a device."""
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, os.path.join(root, "bench.py"), "--gpus", "2"], cwd=root,
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 2
    assert "one GPU" in (r.stdout + r.stderr)
    assert r.stdout.strip() == ""  # no JSON line
