"""dh_flash_bwd_noalloc (the flash backward over a fixed device array, for callers that cannot
allocate) against dh_flash_bwd on the same inputs: bit-identical outputs, fp32 and bf16, on
two calls in a row with the second one smaller, so stale scratch contents from the first call
cannot leak into the second.  Also the size limit and the shared-buffer (aliased) case."""
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
