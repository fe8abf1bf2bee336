"""GPU parity of dh_flash_fwd / dh_flash_bwd against the fp64 oracle.

Tolerances (normwise max relative error, max|x - x64| / max|x64|):
  fp32: <= 1e-5 * sqrt(S) for O, dQ, dK, dV (S = the longest contraction, keys);
        LSE absolute error <= 1e-5 * sqrt(S).
  bf16: <= 2e-2 against fp64 on the bf16-rounded (round-to-nearest-even) inputs.
The fp64 references are orc_attention / orc_attention_causal (runtime/nn/training.inc:
178-263), orc_flash_fwd (284-401) and their backward branches (autograd.inc:675-840).
"""
import numpy as np
import pytest

import _oracle as O
from _gpu import bf16_bits, bits_to_f32, flash_bwd, flash_fwd, maxrel
from dreamcompiler_amd import hip

pytestmark = pytest.mark.gpu


def inputs(BH, S, D, seed, scale=1.0, n=4):
    rng = np.random.default_rng(seed)
    return [(rng.standard_normal((BH, S * D)) * scale).astype(np.float32) for _ in range(n)]


def ref_lse(Q, K, BH, S, D, causal):
    return O.flash_lse(Q.astype(np.float64), K.astype(np.float64), BH, S, D, causal)


def test_c3_fp32_causal_b4_h6_s256_d64():
    # Config 3: B=4, H=6 -> 24 slices, S=256, D=64, Q,K,V ~ 0.5*N(0,1), scale 1/8, causal;
    # compared against the reference standard (attention_causal) and flash (Bc=64) paths.
    O.set_seed(3)
    BH, S, D = 24, 256, 64
    Q, K, V = (O.randn(BH, S * D) * 0.5 for _ in range(3))
    Q32, K32, V32 = (x.astype(np.float32) for x in (Q, K, V))
    got, lse = flash_fwd(Q32, K32, V32, BH, S, D, causal=True)
    tol = 1e-5 * np.sqrt(S)
    assert maxrel(got, O.attention(Q, K, V, BH, S, D, True)) <= tol
    assert maxrel(got, O.flash_fwd(Q, K, V, BH, S, D, 64)) <= tol
    assert np.abs(lse - ref_lse(Q32, K32, BH, S, D, True)).max() <= tol


@pytest.mark.parametrize("S", [1, 33, 100, 130, 257])
@pytest.mark.parametrize("D", [32, 64, 128])
@pytest.mark.parametrize("causal", [True, False])
def test_fp32_fwd_shapes(S, D, causal):
    BH = 3
    Q, K, V = inputs(BH, S, D, S * 7 + D + causal, n=3)
    got, lse = flash_fwd(Q, K, V, BH, S, D, causal)
    Q64, K64, V64 = (x.astype(np.float64) for x in (Q, K, V))
    ref = O.attention(Q64, K64, V64, BH, S, D, causal)
    tol = 1e-5 * np.sqrt(max(S, 1))
    assert maxrel(got, ref) <= tol
    assert np.abs(lse - ref_lse(Q, K, BH, S, D, causal)).max() <= tol
    if causal:   # row 0 attends only to key 0
        assert np.allclose(got.reshape(BH, S, D)[:, 0], V.reshape(BH, S, D)[:, 0], atol=1e-6)


@pytest.mark.parametrize("D", [32, 64, 128])
@pytest.mark.parametrize("causal", [True, False])
def test_fp32_fwd_wide_grid(D, causal):
    # 130 slices x 257 rows fill the chip with 128-row work-groups (the small-grid split
    # kernel covers the 3-slice shapes above); ragged last block, fp64 oracle.
    BH, S = 130, 257
    Q, K, V = inputs(BH, S, D, 1000 + D + causal, n=3)
    got, lse = flash_fwd(Q, K, V, BH, S, D, causal)
    Q64, K64, V64 = (x.astype(np.float64) for x in (Q, K, V))
    tol = 1e-5 * np.sqrt(S)
    assert maxrel(got, O.attention(Q64, K64, V64, BH, S, D, causal)) <= tol
    assert np.abs(lse - ref_lse(Q, K, BH, S, D, causal)).max() <= tol


@pytest.mark.parametrize("S", [1, 64, 100, 257, 520])
@pytest.mark.parametrize("D", [32, 64, 128])
@pytest.mark.parametrize("causal", [True, False])
def test_bf16_fwd_shapes(S, D, causal):
    BH = 2
    Q, K, V = (bf16_bits(x) for x in inputs(BH, S, D, S * 11 + D + causal, n=3))
    got, lse = flash_fwd(Q, K, V, BH, S, D, causal, dtype="bf16")
    Q64, K64, V64 = (bits_to_f32(x).astype(np.float64) for x in (Q, K, V))
    ref = O.attention(Q64, K64, V64, BH, S, D, causal)
    assert maxrel(got, ref) <= 2e-2
    assert np.abs(lse - O.flash_lse(Q64, K64, BH, S, D, causal)).max() <= 1e-3 * np.sqrt(D)


def _bwd_ref(Q, K, V, dO, BH, S, D, causal):
    args = [x.astype(np.float64) for x in (Q, K, V, dO)]
    return O.attention_bwd(*args, BH, S, D, causal)


@pytest.mark.parametrize("S", [1, 33, 100, 257])
@pytest.mark.parametrize("D", [32, 64, 128])
@pytest.mark.parametrize("causal", [True, False])
def test_fp32_bwd(S, D, causal):
    BH = 2
    Q, K, V, G = inputs(BH, S, D, S * 13 + D + causal)
    Of, lse = flash_fwd(Q, K, V, BH, S, D, causal)
    grads = flash_bwd(Q, K, V, Of, G, lse, BH, S, D, causal)
    refs = _bwd_ref(Q, K, V, G, BH, S, D, causal)
    tol = 1e-5 * np.sqrt(max(S, 1))
    for name, g, r in zip("QKV", grads, refs):
        if np.abs(r).max() < 1e-12:
            # S = 1: dS = P (dP - D) with D = dP exactly, so dQ = dK = 0 in exact
            # arithmetic; the GPU leaves fp32 rounding residue of the O(1) terms.
            assert np.abs(g).max() <= tol, name
        else:
            assert maxrel(g, r) <= tol, name
    if causal and S > 1:   # the reference's own flash backward agrees with the standard one
        fl = O.flash_bwd(*(x.astype(np.float64) for x in (Q, K, V, G)), BH, S, D)
        for g, r in zip(grads, fl):
            assert maxrel(g, r) <= tol


@pytest.mark.parametrize("S", [64, 100, 257])
@pytest.mark.parametrize("D", [32, 64, 128])
@pytest.mark.parametrize("causal", [True, False])
def test_bf16_bwd(S, D, causal):
    BH = 2
    Q, K, V, G = (bf16_bits(x) for x in inputs(BH, S, D, S * 17 + D + causal))
    Of, lse = flash_fwd(Q, K, V, BH, S, D, causal, dtype="bf16")
    grads = flash_bwd(Q, K, V, bf16_bits(Of), G, lse, BH, S, D, causal, dtype="bf16")
    refs = _bwd_ref(*(bits_to_f32(x) for x in (Q, K, V, G)), BH, S, D, causal)
    for name, g, r in zip("QKV", grads, refs):
        assert maxrel(g, r) <= 2e-2, name


def test_fwd_rejects_non_positive_scale():
    # The forward keeps its running max on raw scores, which needs scale > 0; the
    # reference always passes 1/sqrt(dk) (runtime/nn/training.inc:292).
    BH, S, D = 1, 64, 32
    bufs = [hip.DeviceBuffer.from_numpy(x) for x in inputs(BH, S, D, 3, n=3)]
    out = hip.DeviceBuffer.empty((BH, S * D), np.float32)
    lse = hip.DeviceBuffer.empty((BH, S), np.float32)
    for bad in (0.0, -0.125, float("inf"), float("nan")):
        st = hip.load().dh_flash_fwd(hip.F32, BH, S, D, bad, 1, *(b.ptr for b in bufs), out.ptr, lse.ptr)
        assert st == hip.DH_ERR_INVALID, bad
        assert b"scale" in hip.load().dh_last_error()


def test_bwd_accumulate_and_determinism():
    BH, S, D = 2, 130, 64
    Q, K, V, G = inputs(BH, S, D, 5)
    Of, lse = flash_fwd(Q, K, V, BH, S, D, True)
    g1 = flash_bwd(Q, K, V, Of, G, lse, BH, S, D, True)
    g2 = flash_bwd(Q, K, V, Of, G, lse, BH, S, D, True)
    for a, b in zip(g1, g2):
        assert np.array_equal(a, b)          # bit-identical run to run
    init = inputs(BH, S, D, 6, n=3)
    g3 = flash_bwd(Q, K, V, Of, G, lse, BH, S, D, True, accumulate=True, init=init)
    for a, b, c in zip(g3, g1, init):
        assert np.allclose(a, b + c, rtol=1e-6, atol=1e-6)


def test_c4_bf16_fwd_bwd_full_size():
    # Config 4: B=8 H=16 (128 slices) S=4096 D=128, Q,K,V,dO ~ N(0,1) rounded to bf16,
    # causal, fp32 accumulate / LSE.  One slice is checked element-wise against the fp64
    # oracle; every slice is checked through size-independent identities.
    BH, S, D = 128, 4096, 128
    rng = np.random.default_rng(4096)
    Q, K, V, G = (bf16_bits(rng.standard_normal((BH, S * D), dtype=np.float32)) for _ in range(4))
    Of, lse = flash_fwd(Q, K, V, BH, S, D, True, dtype="bf16")
    dQ, dK, dV = flash_bwd(Q, K, V, bf16_bits(Of), G, lse, BH, S, D, True, dtype="bf16")
    b = 77
    one = [bits_to_f32(x[b:b + 1]).astype(np.float64) for x in (Q, K, V, G)]
    assert maxrel(Of[b:b + 1], O.attention(*one[:3], 1, S, D, True)) <= 2e-2
    rQ, rK, rV = O.attention_bwd(*one, 1, S, D, True)
    assert maxrel(dQ[b:b + 1], rQ) <= 2e-2
    assert maxrel(dK[b:b + 1], rK) <= 2e-2
    assert maxrel(dV[b:b + 1], rV) <= 2e-2
    # identities for every slice: causal row 0 sees only key 0 -> O_0 = V_0;
    # rows of P sum to 1 -> sum_j dV_j = sum_i dO_i; rows of dS sum to 0 -> sum_j dK_j = 0.
    Vf, Gf = bits_to_f32(V).reshape(BH, S, D), bits_to_f32(G).reshape(BH, S, D)
    assert np.allclose(Of.reshape(BH, S, D)[:, 0], Vf[:, 0], atol=1e-2)
    sdv = dV.reshape(BH, S, D).sum(1, dtype=np.float64)
    sdo = Gf.sum(1, dtype=np.float64)
    assert np.abs(sdv - sdo).max() <= 2e-2 * np.abs(sdo).max()
    sdk = dK.reshape(BH, S, D).sum(1, dtype=np.float64)
    assert np.abs(sdk).max() <= 2e-2 * np.abs(dK).max() * np.sqrt(S)
    assert np.isfinite(dQ).all() and np.isfinite(lse).all()
