"""The legacy quantisation formats on the GPU (csrc/legacy.hip), bit-exact
against the reference's legacy dispatcher.

  * Host ABI (quantization_compress / load_quantization_from_buffer /
    quantization_decompress, include/quantization.hpp): every method on every
    golden case gives the serialised buffer the reference's library wrote
    (tests/golden/legacy_golden.npz, pointer fields zeroed) and decodes the
    reference's buffers to the reference's floats.
  * Device entry points: the payload image equals the reference's payload
    apart from the pointer fields, also for unaligned input / output pointers;
    decode of the reference's payloads.
  * Larger inputs (up to the reference benches' 4 194 304 elements) against
    the CPU oracle, which the CPU suite pins to the reference.
  * Exhaustive: the device FP16 / BF16 conversions of all 2^32 float patterns
    and the MX exponent of every positive finite float, as checksums against
    the reference's.
  * Error behaviour of quantization_decompress on inconsistent buffers.
"""
import ctypes

import numpy as np
import pytest

import bitsqz_amd as B
from oracle import legacy as LG
from test_legacy_oracle import CASES, GOLD, golden

pytestmark = pytest.mark.gpu
IDS = [LG.NAMES[m] for m in LG.ALL]


def mask_payload(method, payload: bytes) -> bytes:
    """The payload with the format struct's pointer fields zeroed."""
    b = bytearray(payload)
    for off in LG.header_struct(method)[1]:
        b[off:off + 8] = bytes(8)
    return bytes(b)


@pytest.mark.parametrize("method", LG.ALL, ids=IDS)
def test_host_abi_matches_reference_goldens(method):
    print(f"legacy host ABI {LG.NAMES[method]}", flush=True)
    for i, x in enumerate(CASES):
        packed, decoded = golden(method, i)
        got = B.legacy_compress(method, x)
        assert LG.mask_pointers(method, got) == packed, f"{LG.NAMES[method]} case {i} (n={x.size}) encode"
        rc, out = B.legacy_decompress(packed, x.size)
        assert rc == 0
        assert out.tobytes() == decoded.tobytes(), f"{LG.NAMES[method]} case {i} (n={x.size}) decode"
        # our own buffer round-trips through load as well
        rc, out2 = B.legacy_decompress(got, x.size)
        assert rc == 0 and out2.tobytes() == decoded.tobytes()


def _dev_encode(method, x, src_shift=0):
    """Device encode with the input `src_shift` floats into its buffer."""
    L = B.lib()
    n = x.size
    size = B.legacy_payload_bytes(method, n)
    src = B.DeviceBuffer(4 * (n + src_shift))
    src.upload(np.concatenate([np.zeros(src_shift, np.float32), x]))
    img = B.DeviceBuffer(size)
    B.check(L.bsq_legacy_encode_device(method, src.value + 4 * src_shift, n, img.ptr, None), "encode")
    B.check(L.bsq_stream_synchronize(None), "sync")
    return img.download(np.uint8, size).tobytes()


def _dev_decode(method, payload, n, dst_shift=0):
    L = B.lib()
    img = B.DeviceBuffer.from_array(np.frombuffer(payload, np.uint8))
    dst = B.DeviceBuffer(4 * (n + dst_shift))
    dst.zero()
    B.check(L.bsq_legacy_decode_device(method, img.ptr, n, dst.value + 4 * dst_shift, None), "decode")
    B.check(L.bsq_stream_synchronize(None), "sync")
    return dst.download(np.float32, n + dst_shift)[dst_shift:]


@pytest.mark.parametrize("method", LG.ALL, ids=IDS)
def test_device_entry_points_match_reference_payloads(method):
    print(f"legacy device {LG.NAMES[method]}", flush=True)
    for i, x in enumerate(CASES):
        packed, decoded = golden(method, i)
        shift = i % 3  # 16-byte aligned, 4-aligned and 8-aligned inputs / outputs
        assert mask_payload(method, _dev_encode(method, x, shift)) == packed[24:], f"case {i} encode"
        assert _dev_decode(method, packed[24:], x.size, shift).tobytes() == decoded.tobytes(), f"case {i} decode"


@pytest.mark.parametrize("method", LG.ALL, ids=IDS)
@pytest.mark.parametrize("n", [4097, 1 << 20, 4194304])
def test_large_inputs_match_oracle(method, n):
    print(f"legacy large {LG.NAMES[method]} n={n}", flush=True)
    rng = np.random.default_rng(n + method)
    x = rng.uniform(-10.0, 10.0, n).astype(np.float32)  # the reference benches' inputs
    x[rng.integers(0, n, 16)] = (rng.standard_normal(16) * 1e4).astype(np.float32)
    expect = LG.encode(method, x)
    got = _dev_encode(method, x)
    assert mask_payload(method, got) == expect
    assert _dev_decode(method, expect, n).tobytes() == LG.decode(method, expect, n).tobytes()


@pytest.mark.parametrize("kind", [0, 1, 2, 3])
def test_exhaustive_device_conversions(kind):
    print(f"legacy sweep kind {kind}", flush=True)
    hi = (1 << 32) if kind < 2 else 0x7F800000
    assert B.legacy_sweep(kind, 0, hi) == int(GOLD[f"sweep_{kind}"][0])


def test_decompress_rejects_inconsistent_buffers():
    L = B.lib()
    x = CASES[20]
    for m in LG.ALL:
        packed, _ = golden(m, 20)
        hdr = LG.header_struct(m)[0]
        if hdr.size >= 24 and m not in (LG.FP8, LG.FP4, LG.Q2_K, LG.Q2_K_FAST):
            # a block size other than the format's: refused (the reference's
            # compress never writes one)
            bad = bytearray(packed)
            bs = int.from_bytes(bad[24 + 16:24 + 24], "little")
            bad[24 + 16:24 + 24] = (bs * 2).to_bytes(8, "little")
            raw = ctypes.create_string_buffer(bytes(bad), len(bad))
            h = L.bsq_legacy_load(raw, len(bad))
            assert h
            out = np.zeros(x.size, np.float32)
            assert L.bsq_legacy_decompress(h, out.ctypes.data, x.size) == 1
            assert L.bsq_last_error()
            L.bsq_legacy_free(h)
    # a decode into exactly n elements of a buffer of n + 0 works; the library
    # keeps serving after a refused call
    rc, out = B.legacy_decompress(golden(LG.Q8_0, 20)[0], x.size)
    assert rc == 0 and out.tobytes() == golden(LG.Q8_0, 20)[1].tobytes()
