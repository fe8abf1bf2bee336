"""Elementwise builtins on the CPU side of the reference's CPU-first rule (outputs of at most
4194304 elements run on the host, runtime/backend/gpu.inc:640, 691): values and gradients
against the reference's golden vectors, error convention.  No GPU work."""
import os

import numpy as np
import pytest

from dreamcompiler_amd import hip, runtime as rt

GOLD = np.load(os.path.join(os.path.dirname(__file__), "golden", "ref_vectors.npz"))
NO_GRAD_UNARY = ("lnot", "floor", "ceil", "round")


def _unary_input(op):
    X = GOLD["ew_X"]
    return np.abs(X) + 0.1 if op in ("log", "sqrt") else X * 3.0 if op in NO_GRAD_UNARY else X


@pytest.mark.parametrize("op", list(rt.BINARY))
def test_binary_builtins_match_reference(op):
    L = rt.load()
    X = GOLD["ew_X"]
    A = np.abs(X) + 0.25 if op == "pow" else X
    for r in ("same", "row", "col", "scalar"):
        key = f"ew_{op}_{r}"
        a, b = rt.tensor(A), rt.tensor(GOLD["ew_B_" + r])
        c = getattr(L, rt.BINARY[op])(a, b)
        assert np.array_equal(rt.read(c), GOLD[key + "_C"]), key
        if key + "_dA" in GOLD.files:
            w = rt.tensor(GOLD["ew_G"])
            L.backward(L.sum(L.tensor_mul(c, w)))
            assert np.array_equal(rt.read(a, grad=True), GOLD[key + "_dA"]), key
            assert np.array_equal(rt.read(b, grad=True), GOLD[key + "_dB"]), key
            rt.release(w)
        rt.release(a, b, c)


@pytest.mark.parametrize("op", list(rt.UNARY))
def test_unary_builtins_match_reference(op):
    L = rt.load()
    a = rt.tensor(_unary_input(op))
    c = getattr(L, rt.UNARY[op])(a)
    assert np.array_equal(rt.read(c), GOLD[f"ew_u_{op}_C"]), op
    if op not in NO_GRAD_UNARY:
        w = rt.tensor(GOLD["ew_G"])
        L.backward(L.sum(L.tensor_mul(c, w)))
        assert np.array_equal(rt.read(a, grad=True), GOLD[f"ew_u_{op}_dA"]), op
        rt.release(w)
    rt.release(a, c)


def test_clip_and_pow_shapes():
    L = rt.load()
    X = GOLD["ew_X"]
    a = rt.tensor(X)
    c = L.dream_clip(a, rt.scalar(-0.5), rt.scalar(0.25))
    assert np.array_equal(rt.read(c), np.maximum(-0.5, np.minimum(0.25, X)))
    # pow's output is 2-D (max d0, max d1) and a 1x1 exponent broadcasts
    p = L.dream_pow(a, rt.scalar(2.0))
    assert (p.contents.d0, p.contents.d1) == X.shape
    assert np.array_equal(rt.read(p), X ** 2)
    rt.release(a, c, p)


def test_elementwise_errors(capfd):
    L = rt.load()
    a, b = rt.tensor(np.ones((3, 4))), rt.tensor(np.ones((2, 4)))
    c = L.tensor_sub(a, b)
    assert "RUNTIME ERROR in -: operands 3x4x1x1 and 2x4x1x1 do not broadcast" in capfd.readouterr().err
    assert c.contents.size == 1
    d = L.tensor_add(a, None)
    assert "RUNTIME ERROR in '+': null operand" in capfd.readouterr().err
    e = L.dream_exp(None)
    assert "RUNTIME ERROR in 'exp': null input" in capfd.readouterr().err
    assert d.contents.size == 1 and e.contents.size == 1
    rt.release(a, b, c, d, e)


def test_gpu_side_fails_loudly_without_a_device(capfd, monkeypatch):
    if hip.load().dh_available():
        pytest.skip("a GPU is present: the GPU tests cover this path")
    monkeypatch.setenv("DREAM_ELEMWISE_CPU_MAX", "0")
    L = rt.load()
    a = rt.tensor(np.ones((2, 2)))
    c = L.tensor_add(a, a)
    assert "RUNTIME ERROR in +: HIP backend unavailable" in capfd.readouterr().err
    assert c.contents.size == 1
    rt.release(a, c)


def test_34_minmax_program():
    # tests/34_minmax.dream: min(3, 5) = 3, max(3, 5) = 5 on scalars; max(ones, 2 ones) sends
    # the whole gradient of sum(c) to the larger operand (gb = 4).
    L = rt.load()
    lo, hi = L.dream_minimum(rt.scalar(3.0), rt.scalar(5.0)), L.dream_maximum(rt.scalar(3.0), rt.scalar(5.0))
    a = rt.tensor(np.ones((2, 2)))
    b = L.tensor_add(rt.tensor(np.ones((2, 2))), rt.tensor(np.ones((2, 2))))
    c = L.dream_maximum(a, b)
    L.backward(L.sum(c))
    assert rt.read(lo)[0, 0] == 3.0 and rt.read(hi)[0, 0] == 5.0
    assert rt.read(b, grad=True).sum() == 4.0 and rt.read(a, grad=True).sum() == 0.0
