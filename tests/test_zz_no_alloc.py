"""dh_flash_bwd_noalloc (the flash backward over a fixed device array, for callers that cannot
allocate) against dh_flash_bwd on the same inputs: bit-identical outputs, fp32 and bf16, on
two calls in a row with the second one smaller, so stale scratch contents from the first call
cannot leak into the second; at shapes where dh_flash_bwd forms the fp32 dQ from a stored dS
(D = 64 or 128 over at least a round of 128-key tiles), equal to fp32 rounding.  Also the size limit,
the shared-buffer (aliased) cases, and a call recorded under HIP stream capture and replayed as
a graph."""
import ctypes

import numpy as np
import pytest

from _gpu import bf16_bits, flash_bwd, flash_fwd
from dreamcompiler_amd import hip

pytestmark = pytest.mark.gpu

DB = hip.DeviceBuffer


def _run_noalloc(Q, K, V, O_, dO, LSE, BH, S, D, causal, dtype, init=None, accumulate=False):
    dt = hip.BF16 if dtype == "bf16" else hip.F32
    np_t = np.uint16 if dtype == "bf16" else np.float32
    bufs = [DB.from_numpy(np.ascontiguousarray(x, np_t)) for x in (Q, K, V, O_, dO)]
    dL = DB.from_numpy(np.ascontiguousarray(LSE, np.float32))
    if init is None:
        grads = [DB.empty((BH, S * D), np.float32) for _ in range(3)]
    else:
        grads = [DB.from_numpy(np.ascontiguousarray(g, np.float32)) for g in init]
    st = hip.load().dh_flash_bwd_noalloc(dt, BH, S, D, 1.0 / np.sqrt(D), int(causal),
                                         *(b.ptr for b in bufs), dL.ptr,
                                         *(g.ptr for g in grads), int(accumulate))
    hip.check(st, "dh_flash_bwd_noalloc")
    out = tuple(g.numpy() for g in grads)
    for b in bufs + grads + [dL]:
        b.free()
    return out


def _case(BH, S, D, causal, dtype, seed):
    rng = np.random.default_rng(seed)
    Q, K, V, G = (rng.standard_normal((BH, S * D)).astype(np.float32) for _ in range(4))
    if dtype == "bf16":
        Q, K, V, G = (bf16_bits(x) for x in (Q, K, V, G))
    Of, lse = flash_fwd(Q, K, V, BH, S, D, causal, dtype=dtype)
    Oin = bf16_bits(Of) if dtype == "bf16" else Of
    return Q, K, V, Oin, G, lse


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_noalloc_matches_pool_version_on_two_calls(dtype):
    # the first call fills more scratch rows than the second one reads
    for BH, S, D, causal, seed in ((6, 777, 128, True, 1), (2, 130, 64, False, 2)):
        args = _case(BH, S, D, causal, dtype, seed)
        want = flash_bwd(*args, BH, S, D, causal, dtype=dtype)
        got = _run_noalloc(*args, BH, S, D, causal, dtype)
        for w, g in zip(want, got):
            assert np.array_equal(w, g), (BH, S, D, dtype)
        init = [np.random.default_rng(seed + 9).standard_normal((BH, S * D)).astype(np.float32)
                for _ in range(3)]
        want = flash_bwd(*args, BH, S, D, causal, dtype=dtype, accumulate=True, init=init)
        got = _run_noalloc(*args, BH, S, D, causal, dtype, init=init, accumulate=True)
        for w, g in zip(want, got):
            assert np.array_equal(w, g), (BH, S, D, dtype, "accumulate")


@pytest.mark.parametrize("BH,S,D,causal", [(64, 512, 128, True), (4, 8192, 128, True),
                                           (8, 4096, 128, False), (64, 1024, 64, False),
                                           (48, 1500, 64, True)])
def test_noalloc_fp32_where_the_pool_version_stores_ds(BH, S, D, causal):
    # D = 128 or 64 over at least a round of 128-key tiles: dh_flash_bwd writes scale dS to
    # pool memory and forms dQ as a GEMM on it; the no-alloc entry point recomputes dS in its
    # dQ launch.  dK and dV come from the same arithmetic either way (bit-identical); dQ agrees
    # to the fp32 bound.
    args = _case(BH, S, D, causal, "f32", 4)
    want = flash_bwd(*args, BH, S, D, causal, dtype="f32")
    got = _run_noalloc(*args, BH, S, D, causal, "f32")
    assert np.array_equal(want[1], got[1]) and np.array_equal(want[2], got[2])
    err = np.abs(want[0] - got[0]).max() / np.abs(want[0]).max()
    assert err <= 1e-5 * np.sqrt(S), err


def test_noalloc_rejects_sizes_beyond_its_scratch():
    BH, S, D = 1, 64, 32
    args = _case(BH, S, D, True, "f32", 3)
    bufs = [DB.from_numpy(np.ascontiguousarray(x, np.float32)) for x in args]
    grads = [DB.empty((BH, S * D), np.float32) for _ in range(3)]
    # BH * S = 2^20 + 1 rows: rejected by the size check before any pointer is used
    st = hip.load().dh_flash_bwd_noalloc(hip.F32, 1025, 1024, D, 1.0 / np.sqrt(D), 1,
                                         *(b.ptr for b in bufs), *(g.ptr for g in grads), 0)
    assert st == hip.DH_ERR_INVALID
    assert b"scratch" in hip.load().dh_last_error()
    for b in bufs + grads:
        b.free()


def _run_aliased(fn_name, Q, K, V, O_, dO, LSE, BH, S, D, causal, dtype, alias, init,
                 accumulate):
    """One backward with shared gradient buffers: alias "kv" passes one buffer as dK and dV,
    "qkv" one buffer as dQ, dK and dV (a tensor used as several of Q, K, V)."""
    dt = hip.BF16 if dtype == "bf16" else hip.F32
    np_t = np.uint16 if dtype == "bf16" else np.float32
    bufs = [DB.from_numpy(np.ascontiguousarray(x, np_t)) for x in (Q, K, V, O_, dO)]
    dL = DB.from_numpy(np.ascontiguousarray(LSE, np.float32))
    gq = DB.from_numpy(np.ascontiguousarray(init[0], np.float32))
    gkv = DB.from_numpy(np.ascontiguousarray(init[1], np.float32))
    ptrs = (gq.ptr, gkv.ptr, gkv.ptr) if alias == "kv" else (gq.ptr, gq.ptr, gq.ptr)
    st = getattr(hip.load(), fn_name)(dt, BH, S, D, 1.0 / np.sqrt(D), int(causal),
                                      *(b.ptr for b in bufs), dL.ptr, *ptrs, int(accumulate))
    hip.check(st, fn_name)
    out = (gq.numpy(), gkv.numpy())
    for b in bufs + [dL, gq, gkv]:
        b.free()
    return out


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("alias", ["kv", "qkv"])
@pytest.mark.parametrize("accumulate", [False, True])
def test_noalloc_aliased_gradients_match_pool_version(dtype, alias, accumulate):
    # bit for bit against dh_flash_bwd with the same aliasing; with accumulate = 0 the shared
    # buffer starts from non-zero garbage, which both must overwrite before summing into it
    for BH, S, D, causal, seed in ((4, 300, 64, True, 11), (2, 200, 128, False, 12)):
        args = _case(BH, S, D, causal, dtype, seed)
        rng = np.random.default_rng(seed + 5)
        init = [rng.standard_normal((BH, S * D)).astype(np.float32) for _ in range(2)]
        want = _run_aliased("dh_flash_bwd", *args, BH, S, D, causal, dtype, alias, init,
                            accumulate)
        got = _run_aliased("dh_flash_bwd_noalloc", *args, BH, S, D, causal, dtype, alias,
                           init, accumulate)
        for w, g in zip(want, got):
            assert np.array_equal(w, g), (BH, S, D, dtype, alias, accumulate)
        # and the sum itself: dQ + dK + dV (or dK + dV) of the separate-buffer call
        sep = flash_bwd(*args, BH, S, D, causal, dtype=dtype)
        ref = sep[1] + sep[2] if alias == "kv" else sep[0] + sep[1] + sep[2]
        if accumulate:
            ref = ref + init[1 if alias == "kv" else 0]
        cmp = got[1] if alias == "kv" else got[0]
        scale = np.abs(np.stack(sep)).sum(axis=0).max()
        assert np.abs(cmp - ref).max() <= 1e-5 * scale, (alias, accumulate)


def _hip_runtime():
    rt = ctypes.CDLL("libamdhip64.so")   # the HIP runtime libdream_hip.so is linked against
    for name, args in (("hipStreamCreate", [ctypes.POINTER(ctypes.c_void_p)]),
                       ("hipStreamDestroy", [ctypes.c_void_p]),
                       ("hipStreamSynchronize", [ctypes.c_void_p]),
                       ("hipStreamBeginCapture", [ctypes.c_void_p, ctypes.c_int]),
                       ("hipStreamEndCapture", [ctypes.c_void_p, ctypes.POINTER(ctypes.c_void_p)]),
                       ("hipGraphInstantiate", [ctypes.POINTER(ctypes.c_void_p), ctypes.c_void_p,
                                                ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t]),
                       ("hipGraphLaunch", [ctypes.c_void_p, ctypes.c_void_p]),
                       ("hipGraphExecDestroy", [ctypes.c_void_p]),
                       ("hipGraphDestroy", [ctypes.c_void_p])):
        f = getattr(rt, name)
        f.restype, f.argtypes = ctypes.c_int, args
    return rt


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_noalloc_under_stream_capture_replays(dtype):
    """A warm call (first-use set-up: scratch address, kernel attributes), then the same call
    recorded under global-mode stream capture -- which fails if anything in it allocates,
    synchronises or otherwise leaves the stream -- and the graph launched three times, the
    outputs overwritten with garbage by eager work between replays; every replay bit-identical
    to the uncaptured call."""
    BH, S, D, causal = 3, 260, 64, True
    args = _case(BH, S, D, causal, dtype, 21)
    want = flash_bwd(*args, BH, S, D, causal, dtype=dtype)
    R = _hip_runtime()
    lib = hip.load()
    dt = hip.BF16 if dtype == "bf16" else hip.F32
    np_t = np.uint16 if dtype == "bf16" else np.float32
    bufs = [DB.from_numpy(np.ascontiguousarray(x, np_t)) for x in args[:5]]
    dL = DB.from_numpy(np.ascontiguousarray(args[5], np.float32))
    grads = [DB.empty((BH, S * D), np.float32) for _ in range(3)]
    garbage = np.full((BH, S * D), 7.0, np.float32)
    call = lambda: lib.dh_flash_bwd_noalloc(dt, BH, S, D, 1.0 / np.sqrt(D), int(causal),  # noqa: E731
                                            *(b.ptr for b in bufs), dL.ptr,
                                            *(g.ptr for g in grads), 0)
    s = ctypes.c_void_p()
    assert R.hipStreamCreate(ctypes.byref(s)) == 0
    graph, exe = ctypes.c_void_p(), ctypes.c_void_p()
    try:
        hip.check(lib.dh_set_stream(s), "dh_set_stream")
        hip.check(call(), "warm call")
        assert R.hipStreamSynchronize(s) == 0
        for g, w in zip(grads, want):
            assert np.array_equal(g.numpy(), w)
        assert R.hipStreamBeginCapture(s, 0) == 0            # hipStreamCaptureModeGlobal
        st = call()
        assert R.hipStreamEndCapture(s, ctypes.byref(graph)) == 0
        hip.check(st, "dh_flash_bwd_noalloc under capture")
        assert R.hipGraphInstantiate(ctypes.byref(exe), graph, None, None, 0) == 0
        for _ in range(3):
            for g in grads:                                  # eager work between replays
                hip.check(lib.dh_memcpy_h2d(g.ptr, garbage.ctypes.data, garbage.nbytes),
                          "dh_memcpy_h2d")
            hip.sync()
            assert R.hipGraphLaunch(exe, s) == 0
            assert R.hipStreamSynchronize(s) == 0
            for g, w in zip(grads, want):
                assert np.array_equal(g.numpy(), w)
    finally:
        lib.dh_set_stream(None)
        if exe.value:
            R.hipGraphExecDestroy(exe)
        if graph.value:
            R.hipGraphDestroy(graph)
        R.hipStreamSynchronize(s)
        R.hipStreamDestroy(s)
        for b in bufs + grads + [dL]:
            b.free()
