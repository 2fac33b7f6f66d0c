"""The legacy-format oracle (oracle/legacy_oracle.c, oracle/legacy.py) pinned
on the CPU, and the host-only paths of the legacy dispatcher ABI.

Pins of every encoder and decoder of the eleven formats restated in C:
  * tests/golden/legacy_golden.npz, written by the reference's own legacy
    library (legacy_modules/quantization/src/quantization.cpp + impl/*.cpp,
    built into oracle/_ref/libref_legacy.so) on seeded, edge and boundary
    inputs: serialised buffers byte for byte (pointer fields zeroed) and
    decoded floats bit for bit;
  * that library directly, where it is built, on fresh random inputs;
  * closed forms: FP16 against numpy's IEEE binary16 conversion, BF16 against
    an integer round-to-nearest-even, the E2M1 level table, checksums of the
    FP16 / BF16 conversions over all 2^32 float patterns against the
    reference's conversions.
"""
import concurrent.futures as cf
import ctypes
import os

import numpy as np
import pytest

import bitsqz_amd as B
from oracle import legacy as LG

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLD = np.load(os.path.join(ROOT, "tests", "golden", "legacy_golden.npz"))
REF_SO = os.path.join(ROOT, "oracle", "_ref", "libref_legacy.so")


def golden_cases():
    off = GOLD["x_off"]
    return [GOLD["x"][off[i]:off[i + 1]] for i in range(off.size - 1)]


def golden(method, i):
    po, xo = GOLD[f"packed_off_{method}"], GOLD["x_off"]
    return (GOLD[f"packed_{method}"][po[i]:po[i + 1]].tobytes(),
            GOLD[f"decoded_{method}"][xo[i]:xo[i + 1]])


CASES = golden_cases()


@pytest.mark.parametrize("method", LG.ALL, ids=[LG.NAMES[m] for m in LG.ALL])
def test_oracle_matches_reference_goldens(method):
    for i, x in enumerate(CASES):
        packed, decoded = golden(method, i)
        assert len(packed) == 24 + LG.payload_size(method, x.size)
        assert LG.packed(method, x) == packed, f"{LG.NAMES[method]} case {i} (n={x.size}) encode"
        got = LG.decode(method, packed[24:], x.size)
        assert got.tobytes() == decoded.tobytes(), f"{LG.NAMES[method]} case {i} (n={x.size}) decode"


def _ref():
    if not os.path.exists(REF_SO):
        pytest.skip("oracle/_ref/libref_legacy.so not built (no reference tree)")
    L = ctypes.CDLL(REF_SO)
    P, U, LL = ctypes.c_void_p, ctypes.c_ulonglong, ctypes.c_longlong
    L.ref_legacy_compress.restype = LL
    L.ref_legacy_compress.argtypes = [ctypes.c_int, P, U, P, LL]
    L.ref_legacy_decompress.argtypes = [P, LL, P, U]
    L.ref_legacy_sweep.restype = U
    L.ref_legacy_sweep.argtypes = [ctypes.c_int, U, U]
    L.ref_legacy_set_threads(1)
    return L


@pytest.mark.parametrize("seed", [1, 2])
def test_oracle_matches_reference_library_on_random_inputs(seed):
    L = _ref()
    rng = np.random.default_rng(seed)
    for method in LG.ALL:
        for n in (int(rng.integers(1, 300)), int(rng.integers(300, 5000))):
            x = (rng.standard_normal(n) * np.exp(rng.uniform(-8, 8, n))).astype(np.float32)
            cap = 24 + LG.payload_size(method, n)
            buf = np.zeros(cap, np.uint8)
            assert L.ref_legacy_compress(method, x.ctypes.data, n, buf.ctypes.data, cap) == cap
            ref = LG.mask_pointers(method, buf.tobytes())
            assert LG.packed(method, x) == ref, (LG.NAMES[method], n)
            out = np.zeros(n, np.float32)
            assert L.ref_legacy_decompress(buf.tobytes(), cap, out.ctypes.data, n) == 0
            assert LG.decode(method, ref[24:], n).tobytes() == out.tobytes()


def _sweep_parallel(fn, kind, hi):
    bounds = [(i << 28, min((i + 1) << 28, hi)) for i in range(16) if (i << 28) < hi]
    with cf.ThreadPoolExecutor(8) as ex:
        return sum(ex.map(lambda b: fn(kind, b[0], b[1]), bounds)) % (1 << 64)


@pytest.mark.parametrize("kind", [0, 1, 2, 3])
def test_exhaustive_conversion_checksums(kind):
    """FP16 / BF16 conversions of every float pattern and the MX exponent of
    every positive finite float equal the reference's (checksums written by
    the reference's conversions; the MX exponent by the same libm call)."""
    hi = (1 << 32) if kind < 2 else 0x7F800000
    assert _sweep_parallel(LG.sweep, kind, hi) == int(GOLD[f"sweep_{kind}"][0])


def test_fp16_and_bf16_closed_forms():
    rng = np.random.default_rng(5)
    bits = np.concatenate([rng.integers(0, 1 << 32, 200000, dtype=np.uint64).astype(np.uint32),
                           np.arange(0x33000000 - 64, 0x33000000 + 64, dtype=np.uint32),
                           np.arange(0x477FE000, 0x47800010, 0x100, dtype=np.uint32)])
    f = bits.view(np.float32)
    L = LG._lib()
    fin = ~np.isnan(f)
    got16 = np.array([L.oracle_fp16_from_f32(float(v)) for v in f[fin][:20000]], np.uint16)
    with np.errstate(over="ignore"):
        assert np.array_equal(got16, f[fin][:20000].astype(np.float16).view(np.uint16))
    nan16 = [L.oracle_fp16_from_f32(float(v)) for v in f[~fin][:100]]
    assert all((h & 0x7FFF) == 0x7E00 for h in nan16)
    # every half pattern widens exactly (NaNs: payload up 13 bits, quiet bit set)
    h = np.arange(1 << 16, dtype=np.uint16)
    wide = np.array([L.oracle_fp16_to_f32(int(v)) for v in h], np.float32)
    ok = ~np.isnan(h.view(np.float16))
    assert np.array_equal(wide[ok].view(np.uint32), h[ok].view(np.float16).astype(np.float32).view(np.uint32))
    hn = h[~ok].astype(np.uint32)
    assert np.array_equal(wide[~ok].view(np.uint32),
                          ((hn & 0x8000) << 16) | 0x7FC00000 | ((hn & 0x3FF) << 13))
    # BF16: round to nearest even on the low half, NaN quieted
    u = bits.astype(np.uint64)
    low, odd = u & np.uint64(0xFFFF), (u >> np.uint64(16)) & np.uint64(1)
    bump = np.where((low > 0x8000) | ((low == 0x8000) & (odd == 1)), np.uint64(0x10000), np.uint64(0))
    rne = ((u + bump) >> np.uint64(16)) & np.uint64(0xFFFF)
    isnan = ((u & np.uint64(0x7F800000)) == 0x7F800000) & ((u & np.uint64(0x7FFFFF)) != 0)
    expect = np.where(isnan, (u >> np.uint64(16)) | np.uint64(0x40), rne).astype(np.uint16)
    q = np.zeros(bits.size, np.uint16)
    L.oracle_bf16_encode(f.ctypes.data, f.size, q.ctypes.data)
    assert np.array_equal(q, expect)


def test_e2m1_and_e4m3_tables():
    L = LG._lib()
    levels = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0]
    for c in range(16):
        v = L.oracle_e2m1_decode(c)
        assert v == (-1 if c & 8 else 1) * levels[c & 7] and np.signbit(v) == bool(c & 8)
        assert L.oracle_e2m1_encode(v) == c
    # midpoints go to the lower level; above 6 saturates; NaN -> 6 (sign kept)
    assert [L.oracle_e2m1_encode(v) for v in (0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0, 7.0, 1e30)] == \
        [0, 1, 2, 3, 4, 5, 6, 7, 7]
    assert L.oracle_e2m1_encode(float("nan")) & 7 == 7
    # E4M3: every code that is not 0x7F / 0xFF round-trips; 0x7F decodes to 480
    for c in range(256):
        v = L.oracle_legacy_e4m3_decode(c)
        if c & 0x7F == 0x7F:
            assert abs(v) == 480.0
        else:
            assert L.oracle_legacy_e4m3_encode(v) == c
    assert L.oracle_legacy_e4m3_encode(1e9) == 0x7E and L.oracle_legacy_e4m3_encode(float("inf")) == 0x7E


def test_library_payload_sizes_match_the_reference_layout():
    """bsq_legacy_payload_bytes (no GPU needed) equals the reference's
    get_*_array_size of the struct its compress writes."""
    for m in LG.ALL:
        for n in (1, 2, 31, 32, 33, 255, 256, 257, 1 << 20, (1 << 20) + 3):
            assert B.legacy_payload_bytes(m, n) == LG.payload_size(m, n)
    assert B.legacy_payload_bytes(13, 10) == -1 and B.legacy_payload_bytes(0, 0) == -1


def test_host_only_dispatcher_paths():
    """load / packed size / free and the argument checks that return before
    any device work (quantization.cpp:125-130, 384-487)."""
    L = B.lib()
    x = CASES[20]
    for m in LG.ALL:
        packed, _ = golden(m, 20)
        raw = ctypes.create_string_buffer(packed, len(packed))
        h = L.bsq_legacy_load(raw, len(packed))
        assert h
        assert L.bsq_legacy_packed_size(h) == len(packed)
        # the loaded copy's pointers point into itself
        body = ctypes.string_at(h, len(packed))
        hdr, ptr_offs = LG.header_struct(m)
        assert LG.mask_pointers(m, body) == packed
        base = ctypes.cast(h, ctypes.c_void_p).value
        for off in ptr_offs:
            p = int.from_bytes(body[24 + off:32 + off], "little")
            assert base + 24 + hdr.size <= p <= base + len(packed)
        assert int.from_bytes(body[16:24], "little") == base + 24
        L.bsq_legacy_free(h)
        # one byte short, or a header cut off: refused
        assert not L.bsq_legacy_load(raw, len(packed) - 1)
        assert not L.bsq_legacy_load(raw, 24 + hdr.size - 1)
        # decode into too few elements: 1 (quantization.cpp:392-394), no device work
        h = L.bsq_legacy_load(raw, len(packed))
        out = np.zeros(x.size, np.float32)
        assert L.bsq_legacy_decompress(h, out.ctypes.data, x.size - 1) == 1
        L.bsq_legacy_free(h)
    bad = bytearray(golden(0, 0)[0])
    bad[0:4] = (13).to_bytes(4, "little")
    assert not L.bsq_legacy_load(bytes(bad), len(bad))
    # compress argument checks
    one = np.ones(4, np.float32)
    h = ctypes.c_void_p()
    assert L.bsq_legacy_compress(13, one.ctypes.data, 4, ctypes.byref(h)) == 1
    assert L.bsq_legacy_compress(0, one.ctypes.data, 0, ctypes.byref(h)) == 1
    assert L.bsq_legacy_compress(0, None, 4, ctypes.byref(h)) == 1
    h = ctypes.c_void_p(8)
    assert L.bsq_legacy_compress(0, one.ctypes.data, 4, ctypes.byref(h)) == 1  # *out must be NULL
    assert L.bsq_legacy_decompress(None, one.ctypes.data, 4) == 1
    # a Q2_K buffer with zero super-blocks: 1 (q2_k_impl.cpp:349-351)
    q = bytearray(golden(LG.Q2_K, 0)[0])
    q[24 + 16:24 + 20] = bytes(4)
    raw = ctypes.create_string_buffer(bytes(q), len(q))
    h = L.bsq_legacy_load(raw, len(q))
    assert h
    assert L.bsq_legacy_decompress(h, one.ctypes.data, 4) == 1
    L.bsq_legacy_free(h)
