"""Throughput of the bitsqz_llm compress + decompress hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]

A step is one device-resident compress followed by one device-resident
decompress of a synthetic FP32 matrix that is already in HBM, on each of L
lanes (bsq_lanes_roundtrip, --lanes, default 4): L independent runtime pairs
on their own streams, each with its own copy of the matrix, so the one-CU
stages of one matrix's randomised SVD run beside another's matrix-core GEMMs.
`value` is GB/s of FP32 input (4*rows*cols*L*K / time of the K timed steps);
`single_lane` gives the same pipeline one matrix at a time
(bsq_device_compress + bsq_device_decompress on the process-global runtimes,
the reference ABI's model).  Every lane's decode is checked byte for byte
against the single-lane decode.  Prints one JSON line with the roofline
figure of the dominant kernel and the reference's CPU codec timed on this
host.  For the HOST-input workload (c5) the lanes' figure is device-resident
like the others, and `host_input_step` adds the H2D to a single-lane step.

Dominant kernel: on the SVD workloads, the FP32-MFMA GEMMs that touch the
full matrix (the range finder's 2 + 2 it products and the low-rank
reconstructions, 2 * rows * cols * rank flops each); on the direct
workloads, the HBM-bound stage with the largest time per step (outlier
separation, direct encode, error top-k or direct decode), at its
algorithmic bytes.  Every one of them is bracketed with HIP events on the
runtime stream inside the timed steps (bsq_kernel_timer_*).  `traffic` is
the HBM bytes per launch of that class from the committed rocprofv3 --pmc
summary of the workload, used only when the summary's recorded source hash
equals the hash of the kernel sources this run was built from.

    python bench.py --calibrate-copy   # also launches the plain copy kernel
                                       # (for rocprofv3 --pmc calibration runs)
    python bench.py --legacy           # the legacy formats' device codecs
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import re
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "bitsqueeze-llm_amd")
for _p in (ROOT, PKG):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import bitsqz_amd as B  # noqa: E402

METRIC = "compress+decompress GB/s (FP32 in) at 4096×11008; % HBM/MFMA roofline"
HBM_PEAK_GBS = 8000.0
FP32_MFMA_PEAK_TFLOPS = 157.3

# name -> (rows, cols, outlier ratio, error ratio, svd_ranks, svd_niters, uv, s, direct, generator, input)
# generator: "normal", "outlier_cols", or ("lowrank", rank, decay, noise std, outlier columns, their scale)
HEADLINE_GEN = ("lowrank", 512, 1.2, 0.01, 8, 50.0)
WORKLOADS = {
    # BASELINE headline: 4096x11008 low-rank + noise + outlier columns with config-4 knobs
    "headline": (4096, 11008, 0.005, 0.01, 256, 2, B.NF4, B.QUANT_NONE, B.QUANT_NONE, HEADLINE_GEN, "device"),
    # the same matrix through the direct path (NF4_DQ + outlier + error top-k)
    "direct_full": (4096, 11008, 0.005, 0.01, -1, 2, B.QUANT_NONE, B.QUANT_NONE, B.NF4_DQ, HEADLINE_GEN, "device"),
    "supplement": (4096, 11008, 0.0, 0.0, -1, 2, B.QUANT_NONE, B.QUANT_NONE, B.NF4, "normal", "device"),
    "c1": (2048, 4096, 0.0, 0.0, -1, 2, B.QUANT_NONE, B.QUANT_NONE, B.NF4, "normal", "device"),
    "c2": (4096, 4096, 0.005, 0.0, -1, 2, B.QUANT_NONE, B.QUANT_NONE, B.NF4_DQ, "outlier_cols", "device"),
    # SVD-only, FP32 factors: rank-512 spectrum i^-1.2 + noise 0.01, q = 128, it = 2
    "c3": (4096, 11008, 0.0, 0.0, 128, 2, B.QUANT_NONE, B.QUANT_NONE, B.QUANT_NONE,
           ("lowrank", 512, 1.2, 0.01, 0, 0.0), "device"),
    # full pipeline: rank-512 spectrum i^-1.0 + noise 0.01 + 8 columns x50, q = 256, it = 2, UV NF4
    "c4": (8192, 4096, 0.005, 0.01, 256, 2, B.NF4, B.QUANT_NONE, B.QUANT_NONE,
           ("lowrank", 512, 1.0, 0.01, 8, 50.0), "device"),
    # large full pipeline: rank-1024 spectrum i^-0.8 + noise 0.02 + 32 columns x80, q = 512, it = 3,
    # UV NF4_DQ, HOST input
    "c5": (16384, 14336, 0.002, 0.005, 512, 3, B.NF4_DQ, B.QUANT_NONE, B.QUANT_NONE,
           ("lowrank", 1024, 0.8, 0.02, 32, 80.0), "host"),
}


def make_input(rows, cols, gen, seed=0):
    rng = np.random.default_rng(seed)
    if gen == "normal":
        return rng.standard_normal((rows, cols), dtype=np.float32)
    if gen == "outlier_cols":
        x = rng.standard_normal((rows, cols), dtype=np.float32)
        x[:, np.random.default_rng(1).permutation(cols)[:16]] *= 60.0
        return x
    # low-rank A diag(sigma) B^T (sigma_i = i^-decay) + N(0, noise^2) + outlier columns
    _, r, decay, noise, n_out, scale = gen
    A = rng.standard_normal((rows, r), dtype=np.float32)
    Bm = np.random.default_rng(seed + 1).standard_normal((cols, r), dtype=np.float32)
    sig = (np.arange(1, r + 1, dtype=np.float32) ** np.float32(-decay)).astype(np.float32)
    x = (A * sig[None, :]) @ Bm.T
    x += np.float32(noise) * np.random.default_rng(seed + 2).standard_normal((rows, cols), dtype=np.float32)
    if n_out:
        x[:, np.random.default_rng(seed + 3).permutation(cols)[:n_out]] *= np.float32(scale)
    return np.ascontiguousarray(x, np.float32)


def packed_payload_bytes(p: B.DevicePacked, err_present: bool) -> int:
    h = p.header
    total = 0
    for name in ("section_u", "section_s", "section_v", "section_direct", "section_outlier_topk"):
        s = getattr(h, name)
        if s.storage:
            total += s.size
    if err_present and h.section_error_topk.storage:
        total += h.section_error_topk.size
    return total


def abi_leg(src, ddst, n, wl, reps=5):
    """Wall clock of the reference ABI calls bitsqz_llm_compress (host packed
    object: includes the payload D2H) + bitsqz_llm_decompress (includes the
    payload H2D); returns (GB/s of FP32 input, ms per step).  `src` is the
    device buffer, or for a HOST-input workload the host matrix (the compress
    runtime is re-initialised for HOST input, so its H2D is inside the call)."""
    L = B.lib()
    rows, cols, ro, rerr, svd, nit, uv, s, direct, _, loc = wl
    if loc == "host":
        B.compress_release()
        B.check(B.compress_initialize(rows, cols, ro, rerr, svd, nit, uv, s, direct, B.INPUT_HOST), "compress init")
        src_ptr = src.ctypes.data_as(C.c_void_p)
    else:
        src_ptr = src.ptr
    times = []
    for i in range(reps + 1):
        out = C.POINTER(B.PackedHeader)()
        t0 = time.perf_counter()
        # no profile struct: the reference's two-argument bitsqz_llm_compress
        B.check(L.bsq_compress(src_ptr, C.byref(out), None), "bitsqz_llm_compress")
        B.check(L.bsq_decompress(C.cast(out, C.c_void_p), ddst.ptr, n), "bitsqz_llm_decompress")
        dt = time.perf_counter() - t0
        L.bsq_free(C.cast(out, C.c_void_p))
        if i:
            times.append(dt)
    ms = 1e3 * float(np.median(times))
    return 4.0 * n / (ms * 1e-3) / 1e9, ms


def sources_sha256() -> str:
    """SHA-256 over the kernel and runtime sources, the public headers and the
    build script (file names and contents, in name order): the identity of
    the code a profile summary was collected from."""
    import hashlib

    h = hashlib.sha256()
    files = []
    for d, exts in ((os.path.join(PKG, "csrc"), (".hip", ".hpp")), (os.path.join(ROOT, "include"), (".h", ".hpp"))):
        files += [os.path.join(d, f) for f in sorted(os.listdir(d)) if f.endswith(exts)]
    files.append(os.path.join(PKG, "build.py"))
    for f in files:
        h.update(os.path.relpath(f, ROOT).encode())
        h.update(open(f, "rb").read())
    return h.hexdigest()


def committed_traffic(workload: str, cls: str):
    """HBM bytes per launch of timing class `cls` at `workload`
    (FETCH_SIZE + WRITE_SIZE of every kernel the class launches, each
    calibrated against the copy kernel), from profiles/<workload>_pmc.md when
    that summary was collected from these exact sources; else None and why."""
    path = os.path.join(ROOT, "profiles", f"{workload}_pmc.md")
    if not os.path.exists(path):
        return None, "no pmc summary for this workload"
    text = open(path).read()
    m = re.search(r"^sources_sha256\s*=\s*([0-9a-f]{64})", text, re.M)
    if not m or m.group(1) != sources_sha256():
        return None, "pmc summary collected from other sources"
    m = re.search(r"^traffic_bytes_per_launch\[" + re.escape(cls) + r"\]\s*=\s*(\d+)", text, re.M)
    if not m:
        return None, f"pmc summary has no {cls} class"
    return int(m.group(1)), os.path.relpath(path, ROOT)


def roofline_time_ms(rows, cols, svd, nit, q, err_on, payload_bytes):
    """T_roof of the whole step: MFMA time of the GEMMs over the m x n matrix
    (2 N q (2 + 2 it) + 2 N q (1 + [error top-k])) for the SVD path, HBM time
    of 8N + 2P bytes for the direct path."""
    n = rows * cols
    if svd >= 1:
        flops = 2.0 * n * q * (2 + 2 * nit) + 2.0 * n * q * (1 + (1 if err_on else 0))
        return flops / (FP32_MFMA_PEAK_TFLOPS * 1e12) * 1e3
    return (8.0 * n + 2.0 * payload_bytes) / (HBM_PEAK_GBS * 1e9) * 1e3


def host_cpu_info():
    """nproc, CPU model and socket count of this host (/proc/cpuinfo)."""
    model, sockets = "unknown", set()
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name") and model == "unknown":
                model = line.split(":", 1)[1].strip()
            elif line.startswith("physical id"):
                sockets.add(line.split(":", 1)[1].strip())
    except OSError:
        pass
    return os.cpu_count() or 1, model, max(1, len(sockets))


def cpu_baseline(x, direct, reps=5):
    """The reference's legacy OpenMP NF4 / NF4_DQ codec (nf4_impl.cpp:92-164,
    nf4_dq_impl.cpp:162-275, compiled from the reference's own sources into
    oracle/_ref) on the same matrix: compress and decompress timed
    separately, one warmup then the median of `reps`, with every host thread
    this job may use (OMP_NUM_THREADS, else nproc) and with one thread.  The
    thread count is set inside the library (omp_set_num_threads) and read
    back, so `cores` is what ran.  Falls back to the repository's C
    restatement (kind 'port') when that library is absent.  The reference
    has no CPU top-k, SVD or reconstruct."""
    import ctypes

    from oracle import oracle as O

    method = direct if direct != B.QUANT_NONE else B.NF4
    nproc, model, sockets = host_cpu_info()
    want = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or nproc
    ref_so = os.path.join(ROOT, "oracle", "_ref", "libref_nf4.so")
    # bounded sample: at most the headline matrix's bytes (the first rows)
    cap_rows = max(1, min(x.shape[0], (4096 * 11008) // x.shape[1]))
    sample = np.ascontiguousarray(x[:cap_rows], np.float32)
    n = sample.size
    nb, nc = (n + 63) // 64, (n + 1) // 2
    out = np.empty(n, np.float32)
    codes = np.empty(nc, np.uint8)
    P = ctypes.c_void_p
    if os.path.exists(ref_so):
        L = ctypes.CDLL(ref_so)
        kind = "reference"
        L.ref_set_threads.argtypes = [ctypes.c_int]
        L.ref_set_threads.restype = ctypes.c_int
        set_threads = L.ref_set_threads
        if method == B.NF4:
            L.ref_nf4_compress.argtypes = [P, ctypes.c_ulonglong, P, P]
            L.ref_nf4_decompress.argtypes = [P, P, ctypes.c_ulonglong, P]
            sc = np.empty(nb, np.float32)

            def comp():
                L.ref_nf4_compress(sample.ctypes.data, n, sc.ctypes.data, codes.ctypes.data)

            def decomp():
                L.ref_nf4_decompress(sc.ctypes.data, codes.ctypes.data, n, out.ctypes.data)
        else:
            L.ref_nf4dq_compress.argtypes = [P, ctypes.c_ulonglong, P, P, P]
            L.ref_nf4dq_decompress.argtypes = [ctypes.c_float, P, P, ctypes.c_ulonglong, P]
            sc = np.empty(nb, np.uint8)
            dq = np.zeros(1, np.float32)

            def comp():
                L.ref_nf4dq_compress(sample.ctypes.data, n, dq.ctypes.data, sc.ctypes.data, codes.ctypes.data)

            def decomp():
                L.ref_nf4dq_decompress(ctypes.c_float(dq[0]), sc.ctypes.data, codes.ctypes.data, n,
                                       out.ctypes.data)
    else:
        kind = "port"
        holder = {}
        set_threads = None

        def comp():
            holder["q"] = O.quant_compress(sample, method)

        def decomp():
            O.quant_decompress(holder["q"])

    def median_ms(fn):
        fn()
        ts = []
        for _ in range(reps):
            t0 = time.perf_counter()
            fn()
            ts.append((time.perf_counter() - t0) * 1e3)
        return float(np.median(ts))

    runs = {}
    for label, t in (("all", want), ("one", 1)):
        used = set_threads(t) if set_threads else int(os.environ.get("OMP_NUM_THREADS", "0") or nproc)
        cm = median_ms(comp)
        dm = median_ms(decomp)
        runs[label] = {"threads": used, "compress_ms": round(cm, 3), "decompress_ms": round(dm, 3),
                       "gbps_fp32_in": round(4 * n / ((cm + dm) * 1e-3) / 1e9, 3)}
    if set_threads:
        set_threads(want)
    label = "NF4" if method == B.NF4 else "NF4_DQ"
    a = runs["all"]
    return {"value": a["gbps_fp32_in"], "unit": "GB/s", "cores": a["threads"], "kind": kind,
            "sample": f"legacy {label} compress and decompress of "
                      f"{'the full' if cap_rows == x.shape[0] else f'the first {cap_rows} rows of the'} "
                      f"{x.shape[0]}x{x.shape[1]} matrix ({4 * n} bytes in), 1 warmup + median of {reps} each; "
                      f"the reference has no CPU top-k / SVD path",
            "compress_ms": a["compress_ms"], "decompress_ms": a["decompress_ms"],
            "one_thread": runs["one"], "nproc": nproc, "cpu_model": model, "sockets": sockets}


# The reference's legacy format benches (tests/quantization/test_*_impl.cpp):
# 5 arrays of 4 194 304 uniform[-10, 10] floats per method.
LEGACY_ARRAYS, LEGACY_N = 5, 4194304
LEGACY_NAMES = {0: "Q8_0", 1: "Q4_0", 2: "Q2_K", 3: "BF16", 4: "FP16", 5: "FP8", 6: "FP4", 7: "MXFP8",
                8: "MXFP4", 9: "NVFP4", 10: "NF4_DQ", 11: "NF4", 12: "Q2_K_FAST"}


def legacy_cpu_baseline(x, reps=3):
    """The reference's legacy dispatcher (quantization.cpp:125-476 and the
    eleven impl/*.cpp codecs, compiled from its own sources into
    oracle/_ref/libref_legacy.so) on one array of the workload per method:
    quantization_compress and quantization_decompress timed separately
    (1 warmup + mean of `reps`) with every host thread this job may use."""
    import ctypes

    so = os.path.join(ROOT, "oracle", "_ref", "libref_legacy.so")
    if not os.path.exists(so):
        return None
    L = ctypes.CDLL(so)
    L.ref_legacy_set_threads.argtypes = [ctypes.c_int]
    L.ref_legacy_set_threads.restype = ctypes.c_int
    P = ctypes.c_void_p
    D = ctypes.POINTER(ctypes.c_double)
    L.ref_legacy_roundtrip.argtypes = [ctypes.c_int, P, ctypes.c_ulonglong, P, ctypes.c_int, D, D]
    nproc, model, sockets = host_cpu_info()
    threads = L.ref_legacy_set_threads(int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or nproc)
    out = np.empty(x.size, np.float32)
    per, tot = {}, 0.0
    for m, name in LEGACY_NAMES.items():
        tc, td = ctypes.c_double(), ctypes.c_double()
        L.ref_legacy_roundtrip(m, x.ctypes.data, x.size, out.ctypes.data, 1, ctypes.byref(tc), ctypes.byref(td))
        assert L.ref_legacy_roundtrip(m, x.ctypes.data, x.size, out.ctypes.data, reps, ctypes.byref(tc),
                                      ctypes.byref(td)) == 0
        per[name] = {"compress_ms": round(tc.value * 1e3, 3), "decompress_ms": round(td.value * 1e3, 3)}
        tot += tc.value + td.value
    value = 4.0 * x.size * len(LEGACY_NAMES) / tot / 1e9
    return {"value": round(value, 3), "unit": "GB/s", "cores": threads, "kind": "reference",
            "sample": f"one array of {x.size} uniform[-10,10] floats per method, quantization_compress + "
                      f"quantization_decompress of the reference's legacy library, 1 warmup + mean of {reps}",
            "per_method": per, "nproc": nproc, "cpu_model": model, "sockets": sockets}


def legacy_bench(args):
    """Throughput of the legacy formats' device codecs (csrc/legacy.hip).

    A step encodes and decodes the reference benches' batch (5 arrays of
    4 194 304 uniform[-10, 10] floats, resident in HBM) with every one of the
    13 methods through bsq_legacy_encode_device / bsq_legacy_decode_device.
    `value` is FP32 input bytes over the timed steps' wall time.  Each
    method's encode and decode are also bracketed by HIP events: the roofline
    figure is algorithmic bytes (encode: 4n read + the payload written;
    decode: the payload read + 4n written) over that time, per method and
    over all methods."""
    L = B.lib()
    rng = np.random.default_rng(7)
    xs = rng.uniform(-10.0, 10.0, LEGACY_ARRAYS * LEGACY_N).astype(np.float32)
    dsrc = B.DeviceBuffer.from_array(xs)
    ddst = B.DeviceBuffer(xs.nbytes)
    sizes = {m: B.legacy_payload_bytes(m, LEGACY_N) for m in LEGACY_NAMES}
    pitch = (max(sizes.values()) + 255) // 256 * 256
    dimg = B.DeviceBuffer(pitch * LEGACY_ARRAYS)
    print(f"bench: legacy formats, {LEGACY_ARRAYS} x {LEGACY_N} floats", file=sys.stderr, flush=True)

    def run(m, a):
        src = dsrc.value + 4 * a * LEGACY_N
        img = dimg.value + pitch * a
        B.check(L.bsq_legacy_encode_device(m, src, LEGACY_N, img, None), "legacy encode")
        B.check(L.bsq_legacy_decode_device(m, img, LEGACY_N, ddst.value + 4 * a * LEGACY_N, None), "legacy decode")

    def step():
        for m in LEGACY_NAMES:
            for a in range(LEGACY_ARRAYS):
                run(m, a)

    for _ in range(args.warmup):
        step()
    B.device_synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    B.device_synchronize()
    dt = time.perf_counter() - t0
    ms_per_step = dt / args.steps * 1e3
    value = 4.0 * xs.size * len(LEGACY_NAMES) * args.steps / dt / 1e9

    # per-method encode / decode times with HIP events (same stream), and a
    # spot check of the last decode against the oracle's
    ev = [B.Event() for _ in range(3)]
    per, tot_bytes, tot_ms = {}, 0.0, 0.0
    reps = max(3, args.steps)
    for m, name in LEGACY_NAMES.items():
        enc = dec = 0.0
        for _ in range(reps):
            for a in range(LEGACY_ARRAYS):
                src = dsrc.value + 4 * a * LEGACY_N
                img = dimg.value + pitch * a
                ev[0].record()
                B.check(L.bsq_legacy_encode_device(m, src, LEGACY_N, img, None), "legacy encode")
                ev[1].record()
                B.check(L.bsq_legacy_decode_device(m, img, LEGACY_N, ddst.value + 4 * a * LEGACY_N, None), "decode")
                ev[2].record()
                B.check(L.bsq_stream_synchronize(None), "sync")
                enc += ev[0].elapsed_ms(ev[1])
                dec += ev[1].elapsed_ms(ev[2])
        launches = reps * LEGACY_ARRAYS
        enc, dec = enc / launches, dec / launches
        alg = 4.0 * LEGACY_N + sizes[m]
        per[name] = {"encode_us": round(enc * 1e3, 2), "decode_us": round(dec * 1e3, 2),
                     "alg_bytes": int(alg), "payload_bytes": sizes[m],
                     "encode_gbs": round(alg / (enc * 1e-3) / 1e9, 1), "decode_gbs": round(alg / (dec * 1e-3) / 1e9, 1),
                     "encode_frac": round(alg / (enc * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                     "decode_frac": round(alg / (dec * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
        tot_bytes += 2 * alg
        tot_ms += enc + dec
    achieved = tot_bytes / (tot_ms * 1e-3) / 1e9
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                "kernel": "legacy.hip encode + decode launches of all 13 methods (HIP events per call)",
                "avg_ms": round(tot_ms / (2 * len(LEGACY_NAMES)), 5), "per_method": per}
    line = {
        "metric": "legacy formats compress+decompress GB/s (FP32 in), 5 x 4194304 uniform[-10,10] per method",
        "value": round(value, 3), "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic",
        "config": {"workload": "legacy_formats", "arrays": LEGACY_ARRAYS, "elements": LEGACY_N,
                   "methods": list(LEGACY_NAMES.values()), "input": "device-resident"},
        "roofline": roofline,
    }
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = legacy_cpu_baseline(xs[:LEGACY_N].copy())
    print(json.dumps(line))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default="headline", choices=sorted(WORKLOADS))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--calibrate-copy", action="store_true")
    ap.add_argument("--lanes", type=int, default=4,
                    help="matrices in flight per step on independent runtime lanes (bsq_lanes_*), each on its own "
                         "stream; 1 = one matrix at a time through the process-global runtimes")
    ap.add_argument("--legacy", action="store_true",
                    help="measure the legacy formats' device codecs instead of the packed-object pipeline")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py: this build runs on one GPU only (a multi-GPU run would shard rows, with one "
              "all-reduce per NF4_DQ section and per power iteration; not built)", file=sys.stderr)
        sys.exit(2)
    if args.legacy:
        legacy_bench(args)
        return

    wl = WORKLOADS[args.workload]
    rows, cols, ro, rerr, svd, nit, uv, s, direct, gen, loc = wl
    x = make_input(rows, cols, gen)
    print(f"bench: workload={args.workload} {rows}x{cols} generated", file=sys.stderr, flush=True)
    B.compress_release()
    B.decompress_release()
    B.check(B.compress_initialize(rows, cols, ro, rerr, svd, nit, uv, s, direct, B.INPUT_DEVICE), "compress init")
    q = max(1, min(svd, rows, cols)) if svd >= 1 else -1
    B.check(B.decompress_initialize(rows, cols, ro, rerr, q, uv, s, direct), "decompress init")
    dsrc = B.DeviceBuffer.from_array(x)
    ddst = B.DeviceBuffer(x.nbytes)
    n = rows * cols
    stream = B.runtime_stream()

    def step():
        p = B.device_compress(dsrc)
        B.device_decompress(p, ddst, n)
        return p

    for _ in range(args.warmup):
        p = step()
    B.device_synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        p = step()
    B.device_synchronize()
    dt = time.perf_counter() - t0
    ms_per_step = dt / args.steps * 1e3
    value = 4.0 * n * args.steps / dt / 1e9
    print(f"bench: timed {args.steps} steps, {ms_per_step:.3f} ms/step", file=sys.stderr, flush=True)
    # the same steps again with every timed class bracketed by HIP events on
    # the runtime stream (each event record idles the queue for a few
    # microseconds, so these steps are kept out of `value`)
    B.kernel_timer_start()
    for _ in range(args.steps):
        p = step()
    B.device_synchronize()
    B.kernel_timer_stop()
    timers = {name: B.kernel_timer_read(cls) for name, cls in (
        ("reconstruct", B.TIMER_RECONSTRUCT), ("range_finder", B.TIMER_RANGE_FINDER),
        ("topk_outlier", B.TIMER_TOPK_OUTLIER), ("topk_error", B.TIMER_TOPK_ERROR),
        ("direct_encode", B.TIMER_DIRECT_ENCODE), ("direct_decode", B.TIMER_DIRECT_DECODE))}
    # correctness spot check of the last step against the input (reconstruction error)
    out = ddst.download(np.float32, n).reshape(rows, cols)
    rel = float(np.linalg.norm(out - x) / max(np.linalg.norm(x), 1e-30))

    # algorithmic work per launch of each timed class
    err_present = bool(p.header.flags & 4)
    ko = B.topk_num_columns(cols, ro) if ro > 0 else 0
    ke = B.topk_num_columns(cols, rerr) if rerr > 0 else 0
    sec = p.header.section_direct
    p_dir = sec.size - 48 if sec.storage == 2 else 0  # scales + codes of a quantised direct section
    # a quantised direct section with error correction on rows of a multiple
    # of 64 columns runs its encode and error top-k as one pass (timed as the
    # encode class; no error-class launches)
    fused = svd < 1 and ke > 0 and timers["topk_error"][1] == 0 and timers["direct_encode"][1] > 0
    alg = {"topk_outlier": 4 * n + 6 * rows * ko,
           "topk_error": 4 * n + p_dir + 6 * rows * ke,
           "direct_encode": 4 * n + p_dir + (6 * rows * ke if fused else 0),
           "direct_decode": p_dir + 6 * rows * (ko + (ke if err_present else 0)) + 4 * n}
    by_class = {}
    for name, (ms, cnt) in timers.items():
        if not cnt:
            continue
        avg = ms / cnt
        e = {"launches": cnt, "per_step": round(cnt / args.steps, 3), "avg_ms": round(avg, 5),
             "ms_per_step": round(ms / args.steps, 5)}
        if name in alg:
            gbs = alg[name] / (avg * 1e-3) / 1e9
            e.update({"alg_bytes": alg[name], "gbs": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4)})
        else:
            tf = 2.0 * n * q / (avg * 1e-3) / 1e12
            e.update({"alg_flops": 2.0 * n * q, "tflops": round(tf, 2), "frac_mfma": round(tf / FP32_MFMA_PEAK_TFLOPS, 4)})
        by_class[name] = e

    if svd >= 1:
        # the dominant kernel class: every GEMM over the m x n matrix (the
        # range finder's 2 + 2 it products and the reconstructions), each
        # 2 m n q flops, timed live with HIP events on the runtime's stream
        (rec_ms, rec_n), (rf_ms, rf_n) = timers["reconstruct"], timers["range_finder"]
        launches = rec_n + rf_n
        kms = (rec_ms + rf_ms) / max(launches, 1)
        kflops = 2.0 * rows * cols * q
        achieved = kflops / (kms * 1e-3) / 1e12
        traffic, tsrc = committed_traffic(args.workload, "gemm_mxn")
        roofline = {"bound": "mfma", "achieved": round(achieved, 2), "peak": FP32_MFMA_PEAK_TFLOPS,
                    "unit": "TFLOP/s", "frac": round(achieved / FP32_MFMA_PEAK_TFLOPS, 4),
                    "traffic": traffic, "traffic_source": tsrc,
                    "kernel": "the FP32-MFMA GEMMs over the m x n matrix: range finder A_w B (gemm_dma_kernel, "
                              "split-K + splitk_reduce_kernel) and A_w^T B (gemm_streamk_kernel + "
                              "streamk_reduce_kernel), reconstructions U diag(S) V^T (gemm_dma_kernel RECON on "
                              "the compress side, recon_q_kernel from the packed factors on the decompress side)",
                    "avg_ms": round(kms, 5), "launches": launches, "alg_flops": kflops, "by_class": by_class}
    else:
        hbm = {k: v for k, v in by_class.items() if k in alg}
        dom = max(hbm, key=lambda k: hbm[k]["ms_per_step"])
        d = hbm[dom]
        traffic, tsrc = committed_traffic(args.workload, dom)
        kernels = {"topk_outlier": "topk_reg_kernel (outlier separation)",
                   "topk_error": "topk_reg_kernel (error top-k of x - dequant)",
                   "direct_encode": ("topk_reg_kernel encode sources (NF4 / NF4_DQ encode and error top-k in "
                                     "one pass; + rows_gmax_kernel for NF4_DQ)" if fused else
                                     "quant_encode_kernel (+ rows_gmax_kernel for NF4_DQ)"),
                   "direct_decode": "quant_decode_rows_kernel / quant_decode_kernel"}
        roofline = {"bound": "hbm", "achieved": d["gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": d["frac_hbm"], "traffic": traffic, "traffic_source": tsrc,
                    "kernel": f"{dom}: {kernels[dom]}", "avg_ms": d["avg_ms"], "alg_bytes": alg[dom],
                    "by_class": by_class}

    t_roof = roofline_time_ms(rows, cols, svd, nit, q, rerr > 0, packed_payload_bytes(p, err_present))
    pipeline = {"t_roof_ms": round(t_roof, 4), "frac_of_roofline": round(t_roof / ms_per_step, 4)}

    host_step = None
    if loc == "host":
        # HOST input (BASELINE C5): the step includes the H2D copy of the
        # matrix from page-locked host memory into the runtime's input buffer
        hx = B.PinnedBuffer(n)
        hx.array[:] = x.ravel()
        for _ in range(2):
            hx.copy_to_device_async(dsrc, stream)
            step()
        B.device_synchronize()
        hk = max(3, args.steps // 2)
        t0 = time.perf_counter()
        for _ in range(hk):
            hx.copy_to_device_async(dsrc, stream)
            step()
        B.device_synchronize()
        hms = (time.perf_counter() - t0) / hk * 1e3
        t_link = 4.0 * n / 64e9 * 1e3
        host_step = {"value": round(4.0 * n / (hms * 1e-3) / 1e9, 3), "unit": "GB/s", "ms_per_step": round(hms, 4),
                     "steps": hk, "t_roof_ms": round(t_roof + t_link, 4),
                     "frac_of_roofline": round((t_roof + t_link) / hms, 4),
                     "what": "H2D of the FP32 matrix from pinned host memory (on the runtime stream) + device "
                             "compress + decompress; T_roof adds the matrix over a 64 GB/s host link"}
        hx.free()

    abi_gbs, abi_ms = abi_leg(x if loc == "host" else dsrc, ddst, n, wl)
    abi = {"value": round(abi_gbs, 3), "unit": "GB/s", "ms_per_step": round(abi_ms, 4),
           "what": "bitsqz_llm_compress + bitsqz_llm_decompress wall clock (payload D2H / H2D included"
                   + (", and the HOST input's H2D" if loc == "host" else "") + "), median of 5"}

    lanes = None
    if args.lanes > 1:
        # several matrices in flight: `args.lanes` independent compress +
        # decompress runtime pairs, each on its own stream, every lane a full
        # round trip of its own copy of the matrix per step
        L = B.lib()
        # the single runtime's streams are released first: a process has few
        # hardware queues, and each lane needs one of its own
        B.compress_release()
        B.decompress_release()
        B.check(L.bsq_lanes_initialize(args.lanes, rows, cols, ro, rerr, svd, nit, uv, s, direct), "lanes init")
        lsrc = [B.DeviceBuffer.from_array(x) for _ in range(args.lanes)]
        ldst = [B.DeviceBuffer(x.nbytes) for _ in range(args.lanes)]

        def lane_step():
            for i in range(args.lanes):
                B.check(L.bsq_lanes_roundtrip(i, lsrc[i].ptr, ldst[i].ptr), "lane round trip")

        for _ in range(args.warmup):
            lane_step()
        B.check(L.bsq_lanes_synchronize(), "lanes sync")
        t0 = time.perf_counter()
        for _ in range(args.steps):
            lane_step()
        B.check(L.bsq_lanes_synchronize(), "lanes sync")
        ldt = time.perf_counter() - t0
        same = all(d.download(np.float32, n).tobytes() == out.tobytes() for d in ldst)
        L.bsq_lanes_release()
        del lsrc, ldst
        if not same:
            raise RuntimeError("a lane's decode differs from the single runtime's")
        lanes = {"lanes": args.lanes, "ldt": ldt}
        print(f"bench: {args.lanes} lanes, {ldt / args.steps * 1e3:.3f} ms per step", file=sys.stderr, flush=True)

    if args.calibrate_copy:
        # known-size copy for rocprofv3 --pmc calibration (FETCH_SIZE / WRITE_SIZE per byte)
        stream = B.runtime_stream()  # the null stream once the lanes measurement released the runtimes
        for _ in range(3):
            B.check(B.lib().bsq_copy_kernel(dsrc.ptr, ddst.ptr, 4 * n, stream), "copy kernel")
        B.device_synchronize()
        print(f"bench: copy kernel calibration, {4 * n} bytes read + written per launch", file=sys.stderr)

    # single-lane figures: one matrix at a time through the process-global
    # runtimes (the reference ABI's model); with lanes, `value` and
    # `ms_per_step` are those of the lanes measurement (L matrices per step)
    single = {"value": round(value, 3), "unit": "GB/s", "ms_per_step": round(ms_per_step, 4),
              "frac_of_roofline": round(t_roof / ms_per_step, 4),
              "what": "one device-resident compress + decompress per step (bsq_device_compress / "
                      "bsq_device_decompress on the process-global runtimes)"}
    matrices = 1
    if lanes:
        matrices = lanes["lanes"]
        ms_per_step = lanes["ldt"] / args.steps * 1e3
        value = 4.0 * n * matrices * args.steps / lanes["ldt"] / 1e9
        pipeline = {"t_roof_ms": round(t_roof, 4), "ms_per_matrix": round(ms_per_step / matrices, 4),
                    "frac_of_roofline": round(t_roof * matrices / ms_per_step, 4)}
    line = {
        "metric": METRIC, "value": round(value, 3), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_per_step, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": args.workload, "rows": rows, "cols": cols, "outlier_topk_ratio": ro,
                   "error_correction_topk_ratio": rerr, "svd_ranks": svd, "svd_niters": nit,
                   "svd_uv_format": uv, "svd_s_format": s, "quantization_only_format": direct,
                   "input": "device-resident", "lanes": matrices, "matrices_per_step": matrices,
                   "rel_frobenius_error": round(rel, 6)},
        "roofline": roofline,
        "pipeline_roofline": pipeline,
        "single_lane": single,
        "abi_pcie_inclusive": abi,
    }
    if host_step:
        line["host_input_step"] = host_step
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(x, direct if svd < 1 else uv)
    B.compress_release()
    B.decompress_release()
    print(json.dumps(line))


if __name__ == "__main__":
    main()
