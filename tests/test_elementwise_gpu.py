"""GPU parity of dh_binary / dh_unary (the runGPU / runGPUUnary replacement,
runtime/backend/gpu.inc:637-716) and of the elementwise builtins routed to them.

Checked against the fp64 oracle (orc_binary / orc_unary, pinned by the reference's golden
vectors in test_oracle.py) on the same inputs.  Tolerances:
  fp64: bit-exact for add sub mul div mod, the comparisons, and / or, min / max, relu, abs,
        logical not, floor / ceil / round, clip and sqrt (IEEE-exact or correctly rounded);
        <= 4 ulp of the result for atan2, pow, exp, log, sigmoid, tanh, sin, cos, tan, atan
        (device libm against the host's).
  fp32: bit-exact against numpy's float32 arithmetic for the exact ops; <= 4 fp32 ulp
        (+ 1e-30) against the fp64 oracle on the fp32 inputs for the transcendental ones.
"""
import os

import numpy as np
import pytest

import _oracle as O
from dreamcompiler_amd import hip, runtime as rt

pytestmark = pytest.mark.gpu
DB = hip.DeviceBuffer
GOLD = np.load(os.path.join(os.path.dirname(__file__), "golden", "ref_vectors.npz"))

EXACT_BIN = {"add", "sub", "mul", "div", "mod", "gt", "lt", "ge", "le", "eq", "ne", "and", "or",
             "min", "max"}
EXACT_UN = {"relu", "abs", "lnot", "floor", "ceil", "round", "clip", "sqrt"}


def strides(dims):
    """bcastStrides (gpu.inc:443-449) of a 4-dim shape."""
    d0, d1, d2, d3 = dims
    return [d1 * d2 * d3 if d0 > 1 else 0, d2 * d3 if d1 > 1 else 0, d3 if d2 > 1 else 0,
            1 if d3 > 1 else 0]


def run_binary(op, A, B, dtype=np.float64, c32=False):
    A, B = np.ascontiguousarray(A, dtype), np.ascontiguousarray(B, dtype)
    ad, bd = O.dims4(A.shape), O.dims4(B.shape)
    cd = np.maximum(ad, bd)
    n = int(np.prod(cd))
    dA, dB, dC = DB.from_numpy(A), DB.from_numpy(B), DB.empty((n,), dtype)
    d32 = DB.empty((n,), np.float32) if c32 else None
    try:
        hip.binary(op, hip._DT[np.dtype(dtype)], dA, A.size, strides(ad), dB, B.size,
                   strides(bd), dC, cd, d32)
        C = dC.numpy().reshape([int(x) for x in cd])
        return (C, d32.numpy().reshape(C.shape)) if c32 else C
    finally:
        for b in (dA, dB, dC, d32):
            if b is not None:
                b.free()


def run_unary(op, A, dtype=np.float64, lo=-0.5, hi=0.5, c32=False):
    A = np.ascontiguousarray(A, dtype)
    dA, dC = DB.from_numpy(A), DB.empty(A.shape, dtype)
    d32 = DB.empty(A.shape, np.float32) if c32 else None
    try:
        hip.unary(op, hip._DT[np.dtype(dtype)], dA, dC, A.size, lo, hi, d32)
        C = dC.numpy()
        return (C, d32.numpy()) if c32 else C
    finally:
        for b in (dA, dC, d32):
            if b is not None:
                b.free()


def ulps(got, want, dtype):
    """|got - want| in units of the last place of want (in dtype), inf where they differ in
    class (nan / inf)."""
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    sp = np.spacing(np.abs(want).astype(dtype)).astype(np.float64)
    d = np.abs(got - want)
    d[(got == want)] = 0.0
    return d / np.maximum(sp, np.finfo(dtype).tiny)


def check(op, got, want, dtype, exact):
    if exact:
        assert np.array_equal(got, want), (op, np.flatnonzero(got != want)[:5])
    else:
        assert ulps(got, want, dtype).max() <= 4, (op, ulps(got, want, dtype).max())


def inputs(shape_a, shape_b, seed, op):
    rng = np.random.default_rng(seed)
    A = np.round(rng.standard_normal(shape_a) * 2, 2)
    B = np.round(rng.standard_normal(shape_b) * 2, 2)
    B[B == 0] = 0.75
    if op == "pow":
        A = np.abs(A) + 0.25
    return A, B


SHAPES = [((1000003,), (1000003,)),             # contiguous vector path + scalar tail
          ((37, 129), (1, 129)),                # row broadcast
          ((37, 129), (37, 1)),                 # column broadcast
          ((37, 129), (1, 1)),                  # scalar
          ((1, 129), (37, 1)),                  # outer broadcast
          ((2, 3, 17, 5), (1, 3, 1, 5)),        # 4-D
          ((2, 1, 17, 1), (1, 3, 1, 5)),
          ((1, 1), (1, 1))]


@pytest.mark.parametrize("shapes", SHAPES, ids=lambda s: "x".join(map(str, s[0])) + "_" +
                         "x".join(map(str, s[1])))
def test_binary_f64_matches_oracle(shapes):
    for op in hip.BINOPS:
        A, B = inputs(*shapes, seed=len(op), op=op)
        want = O.binary(op, A, B)
        got = run_binary(op, A, B)
        check(op, got, want.reshape(got.shape), np.float64, op in EXACT_BIN)


@pytest.mark.parametrize("shapes", SHAPES[:6], ids=lambda s: "x".join(map(str, s[0])) + "_" +
                         "x".join(map(str, s[1])))
def test_binary_f32(shapes):
    for op in hip.BINOPS:
        A, B = inputs(*shapes, seed=len(op) + 1, op=op)
        A32, B32 = A.astype(np.float32), B.astype(np.float32)
        got = run_binary(op, A32, B32, np.float32)
        if op in EXACT_BIN:
            a, b = np.broadcast_arrays(A32.reshape(O.dims4(A.shape)), B32.reshape(O.dims4(B.shape)))
            one = lambda m: m.astype(np.float32)   # noqa: E731
            want = {"add": lambda: a + b, "sub": lambda: a - b, "mul": lambda: a * b,
                    "div": lambda: a / b, "mod": lambda: np.fmod(a, b),
                    "gt": lambda: one(a > b), "lt": lambda: one(a < b),
                    "ge": lambda: one(a >= b), "le": lambda: one(a <= b),
                    "eq": lambda: one(np.abs(a - b) < np.float32(1e-6)),
                    "ne": lambda: one(np.abs(a - b) >= np.float32(1e-6)),
                    "and": lambda: one((a > 0) & (b > 0)), "or": lambda: one((a > 0) | (b > 0)),
                    "min": lambda: np.where(a < b, a, b), "max": lambda: np.where(a > b, a, b),
                    }[op]()
            check(op, got.reshape(want.shape), want, np.float32, True)
        else:
            want = O.binary(op, A32, B32)
            check(op, got.reshape(want.shape), want, np.float32, False)


def test_binary_side_output_is_fp32_rounding():
    A, B = inputs((513, 77), (1, 77), 9, "mul")
    C, C32 = run_binary("mul", A, B, c32=True)
    assert np.array_equal(C32, C.astype(np.float32))
    C, C32 = run_binary("add", A.ravel(), A.ravel() * 3, c32=True)   # vector path
    assert np.array_equal(C32, C.astype(np.float32))


@pytest.mark.parametrize("dtype", [np.float64, np.float32])
@pytest.mark.parametrize("n", [1, 3, 1000001, 4 * 1048576 + 7])
def test_unary_matches_oracle(dtype, n):
    rng = np.random.default_rng(n)
    X = np.round(rng.standard_normal(n) * 3, 3).astype(dtype)
    X[: min(n, 6)] = np.array([0.0, -0.0, 0.5, -0.5, 2.5, -1.5], dtype)[: min(n, 6)]
    for op in hip.UNOPS:
        A = (np.abs(X) + dtype(0.1)) if op in ("log", "sqrt") else X
        got = run_unary(op, A, dtype)
        want = O.unary(op, A, -0.5, 0.5)
        if dtype == np.float32 and op in EXACT_UN:
            want = want.astype(np.float32)   # exact / correctly rounded: the fp32 rounding
        check(op, got, want, dtype, op in EXACT_UN)
    if dtype == np.float64:
        C, C32 = run_unary("tanh", X, dtype, c32=True)
        assert np.array_equal(C32, C.astype(np.float32))


def test_large_broadcast_grid_stride():
    # 4096 x 6145 row broadcast: 25.2M outputs, > 2^24, every work-group loops
    rng = np.random.default_rng(3)
    A, B = rng.standard_normal((4096, 6145)), rng.standard_normal((1, 6145))
    got = run_binary("sub", A, B)
    assert np.array_equal(got.reshape(A.shape), A - B)
    got = run_binary("div", B.T.copy(), A[:, :1].copy().T)   # (6145,1) / (1,4096) outer
    assert np.array_equal(got.reshape(6145, 4096), B.T / A[:, 0][None, :])


def test_binary_rejects_out_of_bounds_strides_and_bad_args():
    A = DB.from_numpy(np.zeros(12))
    C = DB.empty((12,), np.float64)
    try:
        with pytest.raises(hip.DreamHipError, match="strides reach"):
            hip.binary("add", hip.F64, A, 12, [4, 1, 0, 0], A, 8, [4, 1, 0, 0], C, [3, 4, 1, 1])
        with pytest.raises(hip.DreamHipError, match="unknown op"):
            hip.binary(17, hip.F64, A, 12, [0, 1, 0, 0], A, 12, [0, 1, 0, 0], C, [1, 12, 1, 1])
        with pytest.raises(hip.DreamHipError, match="dtype"):
            hip.binary("add", hip.BF16, A, 12, [0, 1, 0, 0], A, 12, [0, 1, 0, 0], C, [1, 12, 1, 1])
        with pytest.raises(hip.DreamHipError, match="C32"):
            hip.binary("add", hip.F32, A, 12, [0, 1, 0, 0], A, 12, [0, 1, 0, 0], C, [1, 12, 1, 1],
                       C)
        with pytest.raises(hip.DreamHipError, match="limit 2"):   # 2^31 outputs, host-side check
            hip.binary("add", hip.F64, A, 12, [0, 0, 0, 0], A, 12, [0, 0, 0, 0], C,
                       [1 << 16, 1 << 15, 1, 1])
        with pytest.raises(hip.DreamHipError, match="negative"):
            hip.binary("add", hip.F64, A, 12, [0, -1, 0, 0], A, 12, [0, 1, 0, 0], C, [1, 12, 1, 1])
        with pytest.raises(hip.DreamHipError, match="aligned"):
            hip.unary("exp", hip.F64, A.ptr + 8, C, 4)
        with pytest.raises(hip.DreamHipError, match="unknown op"):
            hip.unary(16, hip.F64, A, C, 4)
    finally:
        A.free()
        C.free()


# ----------------------------------------------------------------------------- builtins
@pytest.fixture
def gpu_elementwise(monkeypatch):
    """Every elementwise builtin on the GPU (the CPU-first bound moved to 0)."""
    monkeypatch.setenv("DREAM_ELEMWISE_CPU_MAX", "0")


def _gold_binary_input(op):
    X = GOLD["ew_X"]
    return np.abs(X) + 0.25 if op == "pow" else X


def test_builtins_on_gpu_match_reference_golden(gpu_elementwise):
    L = rt.load()
    G = GOLD["ew_G"]
    for op, fn in rt.BINARY.items():
        for r in ("same", "row", "col", "scalar"):
            key = f"ew_{op}_{r}"
            a, b = rt.tensor(_gold_binary_input(op)), rt.tensor(GOLD["ew_B_" + r])
            c = getattr(L, fn)(a, b)
            got = rt.read(c)
            check(op, got, GOLD[key + "_C"], np.float64, op in EXACT_BIN)
            if key + "_dA" in GOLD.files:
                # the backward runs on the host from the forward's values: exact where the
                # forward is, within the forward's few ulp for pow
                w = rt.tensor(G)
                L.backward(L.sum(L.tensor_mul(c, w)))
                for t, k in ((a, "_dA"), (b, "_dB")):
                    got, want = rt.read(t, grad=True), GOLD[key + k]
                    if op in EXACT_BIN:
                        assert np.array_equal(got, want), key + k
                    else:
                        assert np.abs(got - want).max() <= 1e-13 * np.abs(want).max(), key + k
                rt.release(w)
            rt.release(a, b, c)
    for op, fn in rt.UNARY.items():
        X = GOLD["ew_X"]
        A = np.abs(X) + 0.1 if op in ("log", "sqrt") else X * 3.0 \
            if op in ("lnot", "floor", "ceil", "round") else X
        a = rt.tensor(A)
        c = getattr(L, fn)(a)
        check(op, rt.read(c), GOLD[f"ew_u_{op}_C"], np.float64, op in EXACT_UN)
        if f"ew_u_{op}_dA" in GOLD.files:
            w = rt.tensor(G)
            L.backward(L.sum(L.tensor_mul(c, w)))
            want = GOLD[f"ew_u_{op}_dA"]
            assert np.abs(rt.read(a, grad=True) - want).max() <= 1e-13 * np.abs(want).max(), op
            rt.release(w)
        rt.release(a, c)


def test_large_builtin_takes_gpu_and_feeds_matmul():
    # 2048 x 2560 = 5.2M outputs: above the CPU-first bound with the default setting.  The
    # result's fp32 device copy is what the following matmul reads.
    L = rt.load()
    rng = np.random.default_rng(8)
    X, b = rng.standard_normal((2048, 2560)), rng.standard_normal((1, 2560))
    W = rng.standard_normal((2560, 64))
    x, bb, w = rt.tensor(X), rt.tensor(b), rt.tensor(W)
    h = L.relu(L.tensor_add(x, bb))
    H = rt.read(h)
    assert np.array_equal(H, np.maximum(X + b, 0.0))
    y = L.tensor_matmul(h, w)
    ref = O.gemm_ref_d(H.astype(np.float32).astype(np.float64), W.astype(np.float32).astype(np.float64))
    assert np.abs(rt.read(y) - ref).max() / np.abs(ref).max() <= 1e-5 * np.sqrt(2560)
    rt.release(x, bb, w, h, y)
