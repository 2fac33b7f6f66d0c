"""bsq_svd_lowrank_noalloc (the SVD entry point that allocates nothing,
include/bitsqz_llm_c.h) against bsq_svd_lowrank, the allocating entry point
with the same kernels and plan layout: the factors must be bit-identical, on
two calls in a row (the second with a smaller input, on the scratch array the
first one left behind), and a shape whose plan exceeds the fixed scratch
array must be rejected with an error."""
import numpy as np
import pytest

import bitsqz_amd as B

pytestmark = pytest.mark.gpu


def _svd(fn, A, q, it, R=None, seed=1241):
    m, n = A.shape
    k = max(1, min(q, m, n))
    dA = B.DeviceBuffer.from_array(np.ascontiguousarray(A, np.float32))
    dR = B.DeviceBuffer.from_array(np.ascontiguousarray(R, np.float32)) if R is not None else None
    dU, dS, dV = B.DeviceBuffer(m * k * 4), B.DeviceBuffer(k * 4), B.DeviceBuffer(n * k * 4)
    rc = getattr(B.lib(), fn)(dA.ptr, m, n, q, it, dR.ptr if dR else None, seed, dU.ptr, dS.ptr, dV.ptr, None)
    B.check(rc, fn)
    B.check(B.lib().bsq_stream_synchronize(None), "sync")
    return (dU.download(np.float32, m * k), dS.download(np.float32, k), dV.download(np.float32, n * k))


def _lowrank(m, n, r, decay, seed):
    rng = np.random.default_rng(seed)
    a = rng.standard_normal((m, r)).astype(np.float32) * (np.arange(1, r + 1, dtype=np.float32) ** -decay)
    return (a @ rng.standard_normal((r, n)).astype(np.float32) +
            np.float32(0.01) * rng.standard_normal((m, n)).astype(np.float32)).astype(np.float32)


def test_noalloc_matches_allocating_entry_point_on_two_calls():
    # first call: a larger plan (injected sketch); second: a smaller input and
    # rank on the same scratch array (built-in sketch)
    cases = [((1024, 2752, 128, 2), True), ((300, 500, 47, 2), False)]
    for (m, n, q, it), inject in cases:
        A = _lowrank(m, n, min(m, n, 256), 1.1, seed=q)
        R = np.random.default_rng(3).standard_normal((min(m, n), max(1, min(q, m, n)))) if inject else None
        ref = _svd("bsq_svd_lowrank", A, q, it, R)
        got = _svd("bsq_svd_lowrank_noalloc", A, q, it, R)
        for a, b, name in zip(got, ref, "USV"):
            assert a.tobytes() == b.tobytes(), f"{name} differs for {(m, n, q, it)}"
        assert np.all(np.isfinite(got[1])) and np.all(np.diff(got[1]) <= 0)


def test_noalloc_rejects_a_plan_above_its_scratch():
    # C5 (16384 x 14336, q = 512, 3 iterations) needs more than the fixed
    # array; real buffers of the right size are passed all the same
    m, n, q = 16384, 14336, 512
    dA = B.DeviceBuffer(m * n * 4)
    dA.zero()
    dU, dS, dV = B.DeviceBuffer(m * q * 4), B.DeviceBuffer(q * 4), B.DeviceBuffer(n * q * 4)
    rc = B.lib().bsq_svd_lowrank_noalloc(dA.ptr, m, n, q, 3, None, 1241, dU.ptr, dS.ptr, dV.ptr, None)
    assert rc == 1
    msg = B.lib().bsq_last_error().decode()
    assert "scratch" in msg and "268435456" in msg, msg
    B.check(B.lib().bsq_stream_synchronize(None), "sync")
    # the entry point still works afterwards
    A = _lowrank(200, 300, 40, 1.0, seed=5)
    ref = _svd("bsq_svd_lowrank", A, 16, 1)
    got = _svd("bsq_svd_lowrank_noalloc", A, 16, 1)
    assert all(a.tobytes() == b.tobytes() for a, b in zip(got, ref))


def _hip():
    import ctypes as C
    h = C.CDLL("libamdhip64.so")
    P = C.c_void_p
    for name, args in (("hipStreamCreate", [C.POINTER(P)]), ("hipStreamDestroy", [P]),
                       ("hipStreamSynchronize", [P]), ("hipStreamBeginCapture", [P, C.c_int]),
                       ("hipStreamEndCapture", [P, C.POINTER(P)]),
                       ("hipGraphInstantiate", [C.POINTER(P), P, P, P, C.c_size_t]),
                       ("hipGraphLaunch", [P, P]), ("hipGraphExecDestroy", [P]), ("hipGraphDestroy", [P])):
        getattr(h, name).restype = C.c_int
        getattr(h, name).argtypes = args
    return h


def test_noalloc_captured_in_a_graph_and_replayed():
    """The entry point's intended caller: one eager call (which looks up the
    scratch array's device address), then the same call captured into a HIP
    graph on a non-default stream, instantiated and replayed three times with
    eager work of the allocating entry point and host synchronisations
    between the replays; every replay's U, S, V equal the allocating entry
    point's bit for bit (the built-in sketch is deterministic)."""
    import ctypes as C
    h = _hip()
    m, n, q, it = 700, 1200, 64, 2
    A = _lowrank(m, n, 128, 1.0, seed=77)
    ref = _svd("bsq_svd_lowrank", A, q, it)
    dA = B.DeviceBuffer.from_array(A)
    k = q
    dU, dS, dV = B.DeviceBuffer(m * k * 4), B.DeviceBuffer(k * 4), B.DeviceBuffer(n * k * 4)
    s = C.c_void_p()
    assert h.hipStreamCreate(C.byref(s)) == 0
    call = lambda: B.lib().bsq_svd_lowrank_noalloc(dA.ptr, m, n, q, it, None, 1241, dU.ptr, dS.ptr, dV.ptr, s)
    graph, exe = C.c_void_p(), C.c_void_p()
    try:
        B.check(call(), "eager noalloc")
        assert h.hipStreamSynchronize(s) == 0
        assert h.hipStreamBeginCapture(s, 2) == 0  # relaxed capture mode
        rc = call()
        assert h.hipStreamEndCapture(s, C.byref(graph)) == 0
        B.check(rc, "captured noalloc")
        assert h.hipGraphInstantiate(C.byref(exe), graph, None, None, 0) == 0
        B2 = _lowrank(300, 500, 40, 1.2, seed=9)
        for rep in range(3):
            for buf in (dU, dS, dV):
                buf.zero()
            assert h.hipGraphLaunch(exe, s) == 0
            assert h.hipStreamSynchronize(s) == 0
            got = (dU.download(np.float32, m * k), dS.download(np.float32, k), dV.download(np.float32, n * k))
            for a, b, name in zip(got, ref, "USV"):
                assert a.tobytes() == b.tobytes(), f"replay {rep}: {name} differs"
            _svd("bsq_svd_lowrank", B2, 16, 1)  # eager work between the replays
    finally:
        if exe.value:
            h.hipGraphExecDestroy(exe)
        if graph.value:
            h.hipGraphDestroy(graph)
        h.hipStreamSynchronize(s)
        h.hipStreamDestroy(s)
