"""Writes the golden vectors under tests/golden/ (run in the build container only).

NF4 / NF4_DQ / E4M3 vectors come from the reference's legacy CPU codec
(legacy_modules/quantization/src/impl/nf4_impl.cpp, nf4_dq_impl.cpp), compiled
from the reference's own sources into oracle/_ref/libref_nf4.so by
oracle/Makefile.  The reference's CUDA codec is required to equal that codec bit
for bit by the reference's own test (tests/quantization_cuda/test_nf4_cuda.cu:
109-114), so these vectors pin the device codec too.

Top-k vectors restate the reference's three known-answer tests
(tests/topk_cuda/test_topk_cuda_extraction.cpp:70-74,
test_topk_cuda_separation.cpp:142-149, test_topk_cuda_pack_roundtrip.cpp:49-57)
plus tie / NaN / zero rows; their expected outputs are computed here by
Python's stable `sorted` (independent of oracle/bsq_oracle.c).

Only data is written (inputs and expected outputs, .npz without pickles).
Usage:  python tests/golden/gen_golden.py
"""
import ctypes
import math
import os
import struct
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
REF_SO = os.path.join(ROOT, "oracle", "_ref", "libref_nf4.so")


def ref():
    if not os.path.exists(REF_SO):
        sys.exit("oracle/_ref/libref_nf4.so missing: run `make -C oracle` where /root/reference exists")
    L = ctypes.CDLL(REF_SO)
    P, U = ctypes.c_void_p, ctypes.c_ulonglong
    L.ref_nf4_compress.argtypes = [P, U, P, P]
    L.ref_nf4_decompress.argtypes = [P, P, U, P]
    L.ref_nf4dq_compress.argtypes = [P, U, P, P, P]
    L.ref_nf4dq_decompress.argtypes = [ctypes.c_float, P, P, U, P]
    return L


def p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def f32(bits):
    return struct.unpack("<f", struct.pack("<I", bits & 0xFFFFFFFF))[0]


LEVELS = [-1.0, -0.6961928009986877, -0.5250730514526367, -0.39491748809814453,
          -0.28444138169288635, -0.18477343022823334, -0.09105003625154495, 0.0,
          0.07958029955625534, 0.16093020141124725, 0.24611230194568634, 0.33791524171829224,
          0.44070982933044434, 0.5626170039176941, 0.7229568362236023, 1.0]


def nf4_edge_input(rng):
    """Blocks of 64 exercising the codec's special cases, then an odd tail."""
    blocks = []
    lv = np.array(LEVELS, np.float32)
    mids = (lv[:-1] + lv[1:]) / np.float32(2)
    # 1. values at, one ulp below and above every NF4 midpoint (block scale 1)
    b = np.concatenate([mids, np.nextafter(mids, np.float32(-2)), np.nextafter(mids, np.float32(2))])
    b = np.concatenate([b, [1.0, -1.0, 0.0, -0.0]]).astype(np.float32)
    blocks.append(np.resize(b, 64))
    blocks.append(np.resize(np.concatenate([lv, -lv * np.float32(0.999)]), 64))
    # 2. non-finite values mixed with finite
    b = rng.standard_normal(64).astype(np.float32)
    b[[1, 9, 17, 33]] = [np.nan, np.inf, -np.inf, np.nan]
    blocks.append(b)
    # 3. all zero, all -0.0
    blocks.append(np.zeros(64, np.float32))
    blocks.append(np.full(64, -0.0, np.float32))
    # 4. sub-normal block (scale sub-normal -> reciprocal overflows to inf)
    blocks.append((rng.standard_normal(64) * 1e-42).astype(np.float32))
    blocks.append(np.array([f32(0x00000001 + i) for i in range(64)], np.float32))
    # 5. tiny and huge scales
    blocks.append((rng.standard_normal(64) * 1e-37).astype(np.float32))
    blocks.append((rng.standard_normal(64) * 1e37).astype(np.float32))
    blocks.append(np.full(64, 3.4028235e38, np.float32))
    # 6. a block that is a single spike
    b = np.zeros(64, np.float32)
    b[13] = -7.25
    blocks.append(b)
    # 7. midpoints scaled by a non-power-of-two absmax
    b = np.resize(mids * np.float32(3.3), 63).astype(np.float32)
    blocks.append(np.concatenate([b, [np.float32(3.3)]]).astype(np.float32))
    # 8. random normal / uniform blocks
    for _ in range(6):
        blocks.append(rng.standard_normal(64).astype(np.float32))
    blocks.append(rng.uniform(-10, 10, 64).astype(np.float32))
    x = np.concatenate(blocks + [rng.standard_normal(37).astype(np.float32)])  # odd partial tail
    return x.astype(np.float32)


def nf4dq_edge_input(rng):
    """NF4_DQ: block absmax ratios hitting the E4M3 boundaries and the code-0
    (scale -> 1) path, with a 1e30 block fixing dq = 1e30/448."""
    blocks = []
    dq = np.float32(1e30) / np.float32(448.0)
    ratios = [448.0, 447.0, 240.0, 2.0 ** -6, 7.5 / 512, 7.49 / 512, 6.5 / 512, 0.5 / 512,
              0.51 / 512, 0.49 / 512, 1e-6, 1e-12, 1.0, 1.0625, 1.03125, 0.9, 17.0, 300.0]
    for r in ratios:
        b = rng.standard_normal(64).astype(np.float32)
        b = b / np.float32(np.max(np.abs(b))) * np.float32(r) * dq
        blocks.append(b.astype(np.float32))
    b = np.zeros(64, np.float32)
    b[0] = np.float32(1e30)
    blocks.append(b)
    b = np.zeros(64, np.float32)
    b[5] = np.float32(1e20)       # ratio ~4.5e-8 -> E4M3 code 0 -> scale 1 -> |v| ~ 1e20
    b[6] = np.float32(-3e19)
    b[7] = np.float32(16777216.0)
    b[8] = np.float32(2.5e7)
    blocks.append(b)
    blocks.append(np.zeros(64, np.float32))
    b = rng.standard_normal(64).astype(np.float32)
    b[3] = np.nan
    b[4] = -np.inf
    blocks.append(b * np.float32(1e25))
    x = np.concatenate(blocks + [rng.standard_normal(21).astype(np.float32)])
    return x.astype(np.float32)


def run_nf4(L, x):
    n = x.size
    nb, nc = (n + 63) // 64, (n + 1) // 2
    sc = np.zeros(nb, np.float32)
    cd = np.zeros(nc, np.uint8)
    assert L.ref_nf4_compress(p(x), n, p(sc), p(cd)) == 0
    out = np.zeros(n, np.float32)
    assert L.ref_nf4_decompress(p(sc), p(cd), n, p(out)) == 0
    return sc, cd, out


def run_nf4dq(L, x):
    n = x.size
    nb, nc = (n + 63) // 64, (n + 1) // 2
    dq = np.zeros(1, np.float32)
    sc = np.zeros(nb, np.uint8)
    cd = np.zeros(nc, np.uint8)
    assert L.ref_nf4dq_compress(p(x), n, p(dq), p(sc), p(cd)) == 0
    out = np.zeros(n, np.float32)
    assert L.ref_nf4dq_decompress(ctypes.c_float(dq[0]), p(sc), p(cd), n, p(out)) == 0
    return dq, sc, cd, out


def e4m3_table(L):
    """E4M3 encode of boundary values through the reference codec: a two-block
    NF4_DQ whose first block fixes dq and whose second block's absmax / dq
    equals the probe value exposes the scale code the reference writes."""
    probes, codes = [], []
    for v in [2.0 ** -6, 7.5 / 512, 7.49 / 512, 0.5 / 512, 0.51 / 512, 1.0, 1.0625, 1.03125,
              1.09375, 1.1, 240.0, 247.9, 248.0, 300.0, 447.9, 3.0, 0.0625, 0.015625, 0.01,
              1e-3, 2.0 ** -9, 3.0 * 2 ** -9, 1.5, 1.9375, 1.96875, 2.0]:
        # two blocks: block 0 absmax 448*t fixes dq = t, block 1 absmax v*t
        t = np.float32(0.5)
        x = np.zeros(128, np.float32)
        x[0] = np.float32(448.0) * t
        x[64] = np.float32(v) * t
        dq, sc, _, _ = run_nf4dq(L, x)
        assert dq[0] == t
        probes.append(np.float32(v))
        codes.append(sc[1])
    return np.array(probes, np.float32), np.array(codes, np.uint8)


def topk_expected(x, k):
    """Stable sort of each row by |x| descending (NaN ranked as -inf)."""
    rows, cols = x.shape
    idx = np.zeros((rows, k), np.uint16)
    val = np.zeros((rows, k), np.float32)
    for r in range(rows):
        keys = []
        for c in range(cols):
            a = abs(float(x[r, c]))
            keys.append(-math.inf if math.isnan(a) else a)
        order = sorted(range(cols), key=lambda c: -keys[c])   # stable: ties keep column order
        for j in range(k):
            idx[r, j] = order[j]
            val[r, j] = x[r, order[j]]
    return idx, val


def k_of(cols, ratio):
    """roundf(float(cols) * ratio) clamped to [1, cols] for ratio > 0."""
    raw = float(np.float32(cols) * np.float32(ratio))   # exact float32 product
    kk = math.floor(raw + 0.5)                           # roundf for raw >= 0 (double is exact here)
    kk = min(kk, cols)
    if kk == 0 and ratio > 0:
        kk = 1
    return kk


def main():
    L = ref()
    rng = np.random.default_rng(20260405)
    out = {}
    x = nf4_edge_input(rng)
    sc, cd, deq = run_nf4(L, x)
    out.update(nf4_edge_x=x, nf4_edge_scales=sc, nf4_edge_codes=cd, nf4_edge_out=deq)
    x = rng.uniform(-10, 10, 8191).astype(np.float32)
    sc, cd, deq = run_nf4(L, x)
    out.update(nf4_unif_x=x, nf4_unif_scales=sc, nf4_unif_codes=cd, nf4_unif_out=deq)
    x = nf4dq_edge_input(rng)
    dq, sc, cd, deq = run_nf4dq(L, x)
    out.update(nf4dq_edge_x=x, nf4dq_edge_dq=dq, nf4dq_edge_scales=sc, nf4dq_edge_codes=cd,
               nf4dq_edge_out=deq)
    x = rng.uniform(-10, 10, 8193).astype(np.float32)
    dq, sc, cd, deq = run_nf4dq(L, x)
    out.update(nf4dq_unif_x=x, nf4dq_unif_dq=dq, nf4dq_unif_scales=sc, nf4dq_unif_codes=cd,
               nf4dq_unif_out=deq)
    probes, codes = e4m3_table(L)
    out.update(e4m3_probe_x=probes, e4m3_probe_code=codes)
    np.savez_compressed(os.path.join(HERE, "nf4_golden.npz"), **out)

    # ---- top-k known answers ------------------------------------------------
    tk = {}
    cases = {
        # test_topk_cuda_extraction.cpp:70-74, ratio 0.5
        "extract": (np.array([[0.4, -9.3, 2.1, -5.2, 7.8, -1.0],
                              [-6.6, 1.3, 8.4, -2.5, 0.7, 3.9],
                              [4.2, -0.8, 5.1, -7.7, 2.6, 9.9]], np.float32), 0.5),
        # test_topk_cuda_separation.cpp:142-149 at ratios 0, 0.01, 1.0
        "sep0": (np.array([[1.0, -2.0, 3.0, -4.0, 5.0, -6.0, 7.0, -8.0],
                           [-1.1, 2.2, -3.3, 4.4, -5.5, 6.6, -7.7, 8.8]], np.float32), 0.0),
        "sep001": (None, 0.01),
        "sep1": (None, 1.0),
        # test_topk_cuda_pack_roundtrip.cpp:49-57, ratio 0.4
        "pack": (np.array([[1.0, -5.0, 0.2, 7.0, -3.0],
                           [2.0, 4.0, -8.0, 0.5, 1.5],
                           [-9.0, 0.1, 3.0, 2.0, -4.0],
                           [6.0, -7.0, 8.0, -1.0, 0.3]], np.float32), 0.4),
        # ties (+-equal magnitudes), NaNs, zeros, +-0, inf
        "ties": (np.array([[1.0, -1.0, 2.0, -2.0, 2.0, 1.0, -0.0, 0.0],
                           [np.nan, 3.0, np.nan, -3.0, np.inf, -np.inf, 0.0, 1.0],
                           [0.0, -0.0, 0.0, 0.0, -0.0, 0.0, 0.0, 0.0],
                           [np.nan] * 8], np.float32), 0.75),
    }
    cases["sep001"] = (cases["sep0"][0], 0.01)
    cases["sep1"] = (cases["sep0"][0], 1.0)
    for name, (xx, ratio) in cases.items():
        k = k_of(xx.shape[1], ratio)
        idx, val = topk_expected(xx, k)
        tk[name + "_x"] = xx
        tk[name + "_ratio"] = np.array([ratio], np.float32)
        tk[name + "_k"] = np.array([k], np.int32)
        tk[name + "_idx"] = idx
        tk[name + "_val"] = val
    # the reference test's own expected index sets (extraction KAT)
    tk["extract_sets"] = np.array([[1, 4, 3], [2, 0, 5], [5, 3, 2]], np.int32)
    # k = roundf(cols*ratio) values named in the survey for the configs
    kc = [(4096, 0.005), (4096, 0.01), (14336, 0.002), (14336, 0.005), (11008, 0.005),
          (11008, 0.01), (8192, 0.02), (8192, 0.03), (8192, 0.05), (8192, 0.10), (512, 0.02),
          (512, 0.03), (6, 0.5), (8, 0.01), (8, 1.0), (5, 0.4), (3, 0.0001), (65535, 1.0)]
    tk["k_cases"] = np.array([[c, k_of(c, r)] for c, r in kc], np.int64)
    tk["k_ratios"] = np.array([r for _, r in kc], np.float32)
    np.savez_compressed(os.path.join(HERE, "topk_golden.npz"), **tk)
    for f in ("nf4_golden.npz", "topk_golden.npz"):
        print(f, os.path.getsize(os.path.join(HERE, f)), "bytes")


if __name__ == "__main__":
    main()
