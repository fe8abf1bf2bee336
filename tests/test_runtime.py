"""Runtime builtins on the CPU: argument checks and error convention (no GPU work).

Mirrors tests/08_shape_mismatch.dream and the error rules of the reference
(runtime/ops/elementwise.inc:972-989): print "RUNTIME ERROR in matmul (@): ..." and
return a fresh 1x1 tensor; never exit.
"""
import numpy as np

from dreamcompiler_amd import runtime as rt


def test_shape_mismatch_error_and_1x1_result(capfd):
    L = rt.load()
    a, b = rt.tensor(np.ones((2, 3))), rt.tensor(np.ones((2, 3)))
    c = L.tensor_matmul(a, b)
    err = capfd.readouterr().err
    assert "RUNTIME ERROR in matmul (@): shape mismatch (2x3 @ 2x3)" in err
    assert (c.contents.d0, c.contents.d1, c.contents.size) == (1, 1, 1)
    rt.release(a, b, c)


def test_null_operand_error(capfd):
    L = rt.load()
    a = rt.tensor(np.ones((2, 2)))
    c = L.tensor_matmul(a, None)
    assert "null operand (right=null)" in capfd.readouterr().err
    assert c.contents.size == 1
    rt.release(a, c)


def test_fused_expressions_stay_on_cpu_branch():
    # Generated code asks dream_gpu_available() before JIT-ing OpenCL fused kernels
    # (src/AST.cpp:1053-1076); that path does not exist here, so it must answer 0.
    assert rt.load().dream_gpu_available() == 0


def test_attention_argument_check(capfd):
    L = rt.load()
    q = rt.tensor(np.ones((1, 10)))
    o = L.dream_flash_attention(q, q, q, rt.scalar(1), rt.scalar(4), rt.scalar(3), None)
    assert "Q/K/V must hold batch*seq*dk" in capfd.readouterr().err
    assert o.contents.size == 1


def test_host_builtins_and_refcounts():
    L = rt.load()
    L.dream_set_seed(rt.scalar(5))
    r1 = rt.read(L.dream_randn(rt.scalar(1), rt.scalar(512)))
    L.dream_set_seed(rt.scalar(5))
    r2 = rt.read(L.dream_randn(rt.scalar(1), rt.scalar(512)))
    assert np.array_equal(r1, r2) and r1.shape == (1, 512)
    o = L.ones(rt.scalar(2), rt.scalar(3))
    assert np.all(rt.read(o) == 1.0)
    s = L.sum(L.tensor_mul(o, o))
    assert rt.read(s)[0, 0] == 6.0
    L.backward(s)
    assert np.all(rt.read(o, grad=True) == 2.0)   # d/do sum(o*o) = 2o


def test_dropout_matches_reference_build():
    """dream_dropout (runtime/io/builtins.inc:151-163) and its backward (autograd.inc:472-482):
    the same fp32 uniform draws from the shared generator as the reference build, so the mask,
    the kept values x / keep and the gradient (1 / keep on kept elements) are bit-identical.
    Host-only: no GPU work."""
    import pytest
    import _ref_runtime
    if not _ref_runtime.available():
        pytest.skip("oracle/_ref not built (needs /root/reference)")
    R = _ref_runtime.RefRuntime()
    L = rt.load()
    X = np.random.default_rng(3).standard_normal((37, 53))
    out = []
    for lib, tensor, read in ((L, rt.tensor, rt.read), (R.L, R.tensor, R.read)):
        lib.dream_set_seed(lib.create_scalar(31337.0))
        x = tensor(X)
        d = lib.dream_dropout(x, lib.create_scalar(0.8))
        lib.backward(lib.sum(lib.tensor_mul(d, tensor(X))))   # upstream gradient X
        out.append((read(d), read(x, grad=True)))
    (d_ours, g_ours), (d_ref, g_ref) = out
    assert np.array_equal(d_ours, d_ref) and np.array_equal(g_ours, g_ref)
    kept = d_ref != 0
    assert 0.7 < kept.mean() < 0.9
    # x / keep (the -ffast-math build may form it as x * (1 / keep): one rounding apart)
    assert np.allclose(d_ref[kept], X[kept] / np.float64(np.float32(0.8)), rtol=4e-16, atol=0)


def test_host_pool_loops_match_numpy():
    """Host elementwise loops large enough to run on the runtime's worker pool (same-shape,
    scalar and broadcast operands, and a unary op), many times in a row: every element as
    numpy computes it (the split over threads cannot change any value)."""
    L = rt.load()
    rng = np.random.default_rng(7)
    A, B = rng.standard_normal((1500, 2000)), rng.standard_normal((1500, 2000))
    row, s = rng.standard_normal((1, 2000)), np.array([[2.5]])
    a, b, r, sc = rt.tensor(A), rt.tensor(B), rt.tensor(row), rt.tensor(s)
    for _ in range(20):
        for x, y, ref in ((a, b, A * B), (a, sc, A * 2.5), (a, r, A * row)):
            c = L.tensor_mul(x, y)
            assert np.array_equal(rt.read(c), ref)
            rt.release(c)
        c = L.dream_exp(a)
        assert np.allclose(rt.read(c), np.exp(A), rtol=4e-16, atol=0)
        rt.release(c)
    rt.release(a, b, r, sc)
