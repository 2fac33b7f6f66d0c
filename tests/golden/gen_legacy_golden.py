"""Writes tests/golden/legacy_golden.npz (run in the build container only).

The vectors come from the reference's legacy dispatcher and its CPU codecs
(legacy_modules/quantization/src/quantization.cpp and src/impl/*.cpp),
compiled from the reference's own sources into oracle/_ref/libref_legacy.so
by oracle/Makefile and run single-threaded (the reference's FP4 encoder writes
each byte from two loop iterations, which OpenMP may split across threads).

For every method and input case the file holds the serialised buffer
(quantization_get_packed_size bytes, pointer fields zeroed) and the decoded
floats of load_quantization_from_buffer + quantization_decompress.  It also
holds checksums over every float bit pattern of the reference's FP16 and BF16
conversions (datatype/fp16/fp16.hpp, datatype/bf16.hpp) and of the MX block
exponent ceil(log2f(absmax / max_norm)) narrowed to int8, the last computed by
oracle/legacy_oracle.c with the same libm call the reference makes (the
reference's helper is file-static).

Only data is written (.npz without pickles).
Usage:  python tests/golden/gen_legacy_golden.py
"""
import concurrent.futures as cf
import ctypes
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
from oracle import legacy as LG  # noqa: E402

REF_SO = os.path.join(ROOT, "oracle", "_ref", "libref_legacy.so")


def ref():
    if not os.path.exists(REF_SO):
        sys.exit("oracle/_ref/libref_legacy.so missing: run `make -C oracle` where /root/reference exists")
    L = ctypes.CDLL(REF_SO)
    P, U, LL = ctypes.c_void_p, ctypes.c_ulonglong, ctypes.c_longlong
    L.ref_legacy_compress.restype = LL
    L.ref_legacy_compress.argtypes = [ctypes.c_int, P, U, P, LL]
    L.ref_legacy_decompress.argtypes = [P, LL, P, U]
    L.ref_legacy_sweep.restype = U
    L.ref_legacy_sweep.argtypes = [ctypes.c_int, U, U]
    L.ref_legacy_set_threads.argtypes = [ctypes.c_int]
    return L


def ref_roundtrip(L, method, x):
    x = np.ascontiguousarray(x, np.float32)
    cap = 24 + LG.payload_size(method, x.size) + 64
    buf = np.zeros(cap, np.uint8)
    size = L.ref_legacy_compress(method, x.ctypes.data, x.size, buf.ctypes.data, cap)
    assert size == 24 + LG.payload_size(method, x.size), (method, size)
    packed = buf[:size].tobytes()
    out = np.zeros(x.size, np.float32)
    assert L.ref_legacy_decompress(packed, size, out.ctypes.data, x.size) == 0
    return LG.mask_pointers(method, packed), out


def cases():
    rng = np.random.default_rng(20250214)
    c = []
    for n in (1, 2, 3, 7, 8, 15, 16, 17, 31, 32, 33, 64, 65, 255, 256, 257, 511, 1000):
        c.append(rng.uniform(-10.0, 10.0, n).astype(np.float32))  # the reference benches' distribution
    e = rng.standard_normal(777).astype(np.float32)
    e[::53] = 0.0
    e[3], e[4], e[5], e[6] = np.nan, np.inf, -np.inf, -0.0
    e[100:132] = 0.0                                  # an all-zero block of 32
    e[200:216] = np.float32(3e-39)                    # subnormal block
    e[300:340] = np.float32(-2.5)                     # constant run
    e[400] = np.float32(1e-44)
    e[500:516] = np.float32(65504.0)                  # FP16 max
    e[520] = np.float32(65520.0)                      # rounds to FP16 infinity
    e[530] = np.float32(1e38)
    c.append(e)
    c.append((rng.standard_normal(1024) * np.exp(rng.uniform(-40, 40, 1024))).astype(np.float32))
    c.append(np.zeros(70, np.float32))
    c.append(np.full(300, -2.5, np.float32))
    c.append(np.full(33, np.float32(1e-42)))
    # MX block maxima near max_norm * 2^k (ceil(log2) boundaries)
    mx = []
    for norm in (448.0, 6.0):
        for k in range(-140, 128, 9):
            base = np.float32(norm * 2.0 ** k) if norm * 2.0 ** k < 3.4e38 else np.float32(3.0e38)
            for d in (-2, -1, 0, 1, 2, 5):
                v = np.frombuffer(np.array([base], np.float32).tobytes(), np.uint32)[0]
                m = np.array([max(1, int(v) + d)], np.uint32).view(np.float32)[0]
                blk = np.zeros(32, np.float32)  # zeros keep the fixture small
                blk[rng.integers(0, 32)] = m if rng.integers(0, 2) else -m
                blk[rng.integers(0, 32)] = np.float32(m * rng.uniform(-0.9, 0.9))
                mx.append(blk)
    c.append(np.concatenate(mx))
    # NVFP4: one large value and tiny blocks (block scale codes of 0)
    t = (rng.standard_normal(160) * 1e-30).astype(np.float32)
    t[7] = 1e6
    c.append(t)
    return c


def main():
    L = ref()
    L.ref_legacy_set_threads(1)
    xs = cases()
    x_all = np.concatenate(xs)
    x_off = np.cumsum([0] + [x.size for x in xs]).astype(np.int64)
    out = {"x": x_all, "x_off": x_off}
    for m in LG.ALL:
        packs, decs = [], []
        for x in xs:
            p, d = ref_roundtrip(L, m, x)
            packs.append(np.frombuffer(p, np.uint8))
            decs.append(d)
        out[f"packed_{m}"] = np.concatenate(packs)
        out[f"packed_off_{m}"] = np.cumsum([0] + [p.size for p in packs]).astype(np.int64)
        out[f"decoded_{m}"] = np.concatenate(decs)
    # checksums over every float pattern, in 16 slices
    bounds = [(i << 28, (i + 1) << 28) for i in range(16)]
    with cf.ThreadPoolExecutor(8) as ex:
        for kind in (0, 1):
            parts = list(ex.map(lambda b: L.ref_legacy_sweep(kind, b[0], b[1]), bounds))
            out[f"sweep_{kind}"] = np.array([sum(parts) % (1 << 64)], np.uint64)
        pos = [(b[0], min(b[1], 0x7F800000)) for b in bounds if b[0] < 0x7F800000]
        for kind in (2, 3):
            parts = list(ex.map(lambda b: LG.sweep(kind, b[0], b[1]), pos))
            out[f"sweep_{kind}"] = np.array([sum(parts) % (1 << 64)], np.uint64)
    path = os.path.join(HERE, "legacy_golden.npz")
    np.savez_compressed(path, **out)
    print("wrote", path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
