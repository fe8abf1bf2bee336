"""fp64 GEMM and attention on the GPU (dh_gemm_f64, dh_attention_f64_*) against the oracle.

dh_gemm_f64 sums every element in the reference dgemm's order (256-deep k blocks, each one
fused multiply-add chain), so NN with beta = 0 must equal orc_gemm_d -- itself bit-identical
to the reference's `@` (tests/test_oracle.py) -- bit for bit.  The other layouts, alpha, beta
and batches are checked against independent fp64 products at 1e-13 normwise; attention against
the oracle's standard attention (and its flash loop) at 1e-12, its backward at 1e-11.
"""
import numpy as np
import pytest

import _oracle as O
from dreamcompiler_amd import hip

pytestmark = pytest.mark.gpu
DB = hip.DeviceBuffer


def maxrel(a, b):
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-300))


def gemm64(A, B, transA=0, transB=0, beta=0.0, C0=None, alpha=1.0, pad=0):
    A, B = np.ascontiguousarray(A, np.float64), np.ascontiguousarray(B, np.float64)
    M = A.shape[1] if transA else A.shape[0]
    K = A.shape[0] if transA else A.shape[1]
    N = B.shape[0] if transB else B.shape[1]

    def padded(X):
        P = np.zeros((X.shape[0], X.shape[1] + pad))
        P[:, :X.shape[1]] = X
        return P

    Ap, Bp = padded(A), padded(B)
    Cp = padded(np.full((M, N), np.nan) if C0 is None else np.asarray(C0, np.float64))
    dA, dB, dC = DB.from_numpy(Ap), DB.from_numpy(Bp), DB.from_numpy(Cp)
    hip.gemm_f64(transA, transB, M, N, K, dA, Ap.shape[1], dB, Bp.shape[1], beta, dC,
                 Cp.shape[1], alpha=alpha)
    return dC.numpy((M, N + pad), np.float64)[:, :N]


# gemm_selftest's fp64 shapes (elementwise.inc:892-895), the config-2 products below the
# threshold, and K across the 256-deep block boundaries.
SHAPES = [(1, 1, 1), (1, 7, 1), (5, 1, 9), (3, 4, 5), (7, 13, 17), (31, 33, 37), (64, 64, 64),
          (65, 63, 66), (128, 100, 96), (200, 50, 300), (257, 129, 255), (4096, 257, 10),
          (100, 256, 70), (33, 257, 40), (70, 512, 33), (9, 1000, 130), (300, 2049, 7),
          (511, 300, 511),
          # grids of >= 512 tiles: one work-group runs all of K (the others split K at the
          # 256-deep blocks and sum the block sums in a second launch)
          (1024, 600, 512), (700, 513, 800)]


@pytest.mark.parametrize("M,K,N", SHAPES)
def test_gemm_f64_bit_identical_to_reference_order(M, K, N):
    rng = np.random.default_rng(M * 7919 + K * 31 + N)
    A, B = rng.uniform(-1, 1, (M, K)), rng.standard_normal((K, N))
    C = gemm64(A, B)
    ref = O.gemm_d(A, B)
    assert np.array_equal(C, ref), f"max diff {np.abs(C - ref).max():.3e}"
    assert maxrel(C, O.gemm_ref_d(A, B)) <= 1e-13


def test_gemm_f64_planted_order_is_distinguishable():
    # The bit-exact check has teeth: a single chain over all of K (no 256 blocks) rounds
    # differently from the reference's blocked order on long K.
    rng = np.random.default_rng(5)
    A, B = rng.standard_normal((40, 1500)), rng.standard_normal((1500, 30))
    single_chain = O.gemm_ref_d(A, B)
    assert not np.array_equal(single_chain, O.gemm_d(A, B))
    assert np.array_equal(gemm64(A, B), O.gemm_d(A, B))


@pytest.mark.parametrize("transA,transB", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("M,K,N", [(37, 300, 45), (64, 33, 96), (5, 700, 3)])
def test_gemm_f64_layouts_alpha_beta(transA, transB, M, K, N):
    rng = np.random.default_rng(M + K + N + 2 * transA + transB)
    A = rng.standard_normal((K, M) if transA else (M, K))
    B = rng.standard_normal((N, K) if transB else (K, N))
    C0 = rng.standard_normal((M, N))
    opA, opB = (A.T if transA else A), (B.T if transB else B)
    for alpha, beta in [(1.0, 0.0), (1.0, 1.0), (0.125, 1.0), (-2.0, 0.5)]:
        got = gemm64(A, B, transA, transB, beta=beta, C0=C0, alpha=alpha, pad=3)
        ref = alpha * (opA @ opB) + beta * C0
        assert maxrel(got, ref) <= 1e-13, (alpha, beta)
    # beta = 0 never reads C (C0 is NaN-filled by gemm64)
    assert np.isfinite(gemm64(A, B, transA, transB)).all()


def test_gemm_f64_batched_and_zero_k():
    rng = np.random.default_rng(11)
    Bt, M, K, N = 5, 19, 270, 23
    A, B = rng.standard_normal((Bt, M, K)), rng.standard_normal((Bt, K, N))
    dA, dB = DB.from_numpy(A), DB.from_numpy(B)
    dC = DB.empty((Bt, M, N), np.float64)
    hip.gemm_f64(0, 0, M, N, K, dA, K, dB, N, 0.0, dC, N, sA=M * K, sB=K * N, sC=M * N, batch=Bt)
    C = dC.numpy()
    for b in range(Bt):
        assert np.array_equal(C[b], O.gemm_d(A[b], B[b]))
    # shared B (stride 0)
    hip.gemm_f64(0, 0, M, N, K, dA, K, dB, N, 0.0, dC, N, sA=M * K, sB=0, sC=M * N, batch=Bt)
    C = dC.numpy()
    for b in range(Bt):
        assert np.array_equal(C[b], O.gemm_d(A[b], B[0]))
    # 520 members of one tile each: a grid of >= 512 work-groups, K not split
    Bt, M, K, N = 520, 19, 300, 23
    A, B = rng.standard_normal((Bt, M, K)), rng.standard_normal((Bt, K, N))
    dA, dB = DB.from_numpy(A), DB.from_numpy(B)
    dC = DB.empty((Bt, M, N), np.float64)
    hip.gemm_f64(0, 0, M, N, K, dA, K, dB, N, 0.0, dC, N, sA=M * K, sB=K * N, sC=M * N, batch=Bt)
    C = dC.numpy()
    for b in range(0, Bt, 37):
        assert np.array_equal(C[b], O.gemm_d(A[b], B[b]))
    # K = 0: C = beta * C
    C0 = rng.standard_normal((4, 6))
    assert np.array_equal(gemm64(np.zeros((4, 0)), np.zeros((0, 6)), beta=0.5, C0=C0), 0.5 * C0)
    assert np.array_equal(gemm64(np.zeros((4, 0)), np.zeros((0, 6))), np.zeros((4, 6)))


def test_gemm_f64_rejects_bad_arguments():
    d = DB.empty((4,), np.float64)
    L = hip.load()
    assert L.dh_gemm_f64(0, 0, -1, 2, 2, d.ptr, 2, d.ptr, 2, 0.0, d.ptr, 2) == hip.DH_ERR_INVALID
    assert L.dh_gemm_f64(0, 0, 2, 2, 2, d.ptr, 1, d.ptr, 2, 0.0, d.ptr, 2) == hip.DH_ERR_INVALID
    assert L.dh_gemm_f64(0, 0, 2, 2, 2, None, 2, d.ptr, 2, 0.0, d.ptr, 2) == hip.DH_ERR_INVALID
    assert L.dh_gemm_f64_ex(0, 0, 2, 2, 2, 1.0, d.ptr, 2, 4, d.ptr, 2, 4, 0.0, d.ptr, 2, 1,
                            2) == hip.DH_ERR_INVALID   # overlapping C members


def attn64(Q, K, V, B, S, D, causal, scale=None):
    scale = 1.0 / np.sqrt(D) if scale is None else scale
    dq, dk, dv = (DB.from_numpy(np.ascontiguousarray(x, np.float64)) for x in (Q, K, V))
    do = DB.empty((B, S * D), np.float64)
    hip.attention_f64_fwd(B, S, D, scale, causal, dq, dk, dv, do)
    return do.numpy()


def attn64_bwd(Q, K, V, G, B, S, D, causal, accumulate=False, init=None, alias=None):
    bufs = [DB.from_numpy(np.ascontiguousarray(x, np.float64)) for x in (Q, K, V, G)]
    if alias:
        g = DB.from_numpy(np.zeros((B, S * D)) if init is None else init)
        grads = [g, g, g]
    elif init is None:
        grads = [DB.empty((B, S * D), np.float64) for _ in range(3)]
    else:
        grads = [DB.from_numpy(np.ascontiguousarray(x, np.float64)) for x in init]
    hip.attention_f64_bwd(B, S, D, 1.0 / np.sqrt(D), causal, *bufs, *grads, int(accumulate))
    return tuple(g.numpy() for g in grads)


# the flash selftest's configurations (training.inc:411), head dims above 128, ragged S
ATTN = [(1, 64, 16), (1, 100, 24), (3, 1, 8), (2, 7, 5), (2, 130, 64), (1, 33, 160),
        (2, 70, 256), (1, 257, 200), (4, 48, 129)]


@pytest.mark.parametrize("B,S,D", ATTN)
@pytest.mark.parametrize("causal", [True, False])
def test_attention_f64_forward(B, S, D, causal):
    rng = np.random.default_rng(B * 1000 + S * 10 + D + causal)
    Q, K, V = (rng.standard_normal((B, S * D)) for _ in range(3))
    got = attn64(Q, K, V, B, S, D, causal)
    assert maxrel(got, O.attention(Q, K, V, B, S, D, causal)) <= 1e-12
    if causal:   # the reference's own fp64 flash loop (what flash_attention runs here)
        assert maxrel(got, O.flash_fwd(Q, K, V, B, S, D, 16)) <= 1e-12


def test_attention_f64_closed_forms():
    rng = np.random.default_rng(3)
    B, S, D = 2, 40, 136
    Q, V = rng.standard_normal((B, S * D)), rng.standard_normal((B, S * D))
    K = np.tile(rng.standard_normal((B, 1, D)), (1, S, 1)).reshape(B, S * D)
    # constant keys: causal output row i = mean of V rows 0..i; full = mean of all rows
    Vr = V.reshape(B, S, D)
    run_mean = np.cumsum(Vr, axis=1) / np.arange(1, S + 1)[None, :, None]
    assert maxrel(attn64(Q, K, V, B, S, D, True).reshape(B, S, D), run_mean) <= 1e-13
    full = np.broadcast_to(Vr.mean(axis=1, keepdims=True), Vr.shape)
    assert maxrel(attn64(Q, K, V, B, S, D, False).reshape(B, S, D), full) <= 1e-13
    # S = 1: O = V
    Q1, K1, V1 = (rng.standard_normal((3, D)) for _ in range(3))
    assert np.array_equal(attn64(Q1, K1, V1, 3, 1, D, True), V1)


@pytest.mark.parametrize("B,S,D", [(1, 4, 8), (1, 100, 24), (2, 33, 160), (3, 50, 64),
                                   (1, 129, 256)])
@pytest.mark.parametrize("causal", [True, False])
def test_attention_f64_backward(B, S, D, causal):
    rng = np.random.default_rng(S * D + B + causal)
    Q, K, V, G = (rng.standard_normal((B, S * D)) for _ in range(4))
    ref = O.attention_bwd(Q, K, V, G, B, S, D, causal)
    got = attn64_bwd(Q, K, V, G, B, S, D, causal)
    for g, r in zip(got, ref):
        assert maxrel(g, r) <= 1e-11
    init = [rng.standard_normal((B, S * D)) for _ in range(3)]
    acc = attn64_bwd(Q, K, V, G, B, S, D, causal, accumulate=True, init=init)
    for g, r, i in zip(acc, ref, init):
        assert maxrel(g, r + i) <= 1e-11


def test_attention_f64_backward_shared_gradient_buffer():
    # attention(q, q, q): one gradient buffer receives dQ + dK + dV (autograd.inc:693-728)
    rng = np.random.default_rng(8)
    B, S, D = 2, 20, 12
    Q, G = rng.standard_normal((B, S * D)), rng.standard_normal((B, S * D))
    ref = sum(O.attention_bwd(Q, Q, Q, G, B, S, D, True))
    got = attn64_bwd(Q, Q, Q, G, B, S, D, True, alias=True)[0]
    assert maxrel(got, ref) <= 1e-11
    init = rng.standard_normal((B, S * D))
    got = attn64_bwd(Q, Q, Q, G, B, S, D, True, accumulate=True, init=init, alias=True)[0]
    assert maxrel(got, ref + init) <= 1e-11


def test_attention_f64_chunks_over_slices():
    # S = 3000: one 72 MB score block per slice, so 3 slices run as one chunk of 3; S = 6000
    # gives 288 MB per slice, above the 256 MB budget: one slice at a time in blocks of 5592
    # query rows (and a last block of 408).  Checked on sampled rows of every slice.
    for B, S, D in [(3, 3000, 8), (2, 6000, 4)]:
        rng = np.random.default_rng(S)
        Q, K, V, G = (rng.standard_normal((B, S * D)) for _ in range(4))
        got = attn64(Q, K, V, B, S, D, True).reshape(B, S, D)
        rows = np.stack([rng.choice(S, 6, replace=False) for _ in range(B)]).astype(np.int32)
        Orow, _ = O.attention_rows(Q, K, V, G, rows, B, S, D, True)
        for b in range(B):
            assert maxrel(got[b, rows[b]], Orow[b]) <= 1e-12


@pytest.mark.parametrize("causal", [True, False])
def test_attention_f64_query_row_blocks(causal, monkeypatch):
    """Slices whose S x S scores exceed the score budget run in blocks of query rows (a
    rows x S buffer each), so no buffer exceeds the budget at any S.  The budget is lowered
    (DH_ATTN_F64_SCORE_BYTES, read at each call) to 100 rows x S x 8 bytes so small shapes take
    that path: blocks of 100 query rows and a ragged last block, forward and backward (fresh,
    accumulating, and one buffer for dQ, dK and dV) against the oracle."""
    B, S, D = 2, 330, 160
    monkeypatch.setenv("DH_ATTN_F64_SCORE_BYTES", str(100 * S * 8))
    rng = np.random.default_rng(330 + causal)
    Q, K, V, G = (rng.standard_normal((B, S * D)) for _ in range(4))
    assert maxrel(attn64(Q, K, V, B, S, D, causal), O.attention(Q, K, V, B, S, D, causal)) <= 1e-12
    ref = O.attention_bwd(Q, K, V, G, B, S, D, causal)
    for g, r in zip(attn64_bwd(Q, K, V, G, B, S, D, causal), ref):
        assert maxrel(g, r) <= 1e-11
    init = [rng.standard_normal((B, S * D)) for _ in range(3)]
    acc = attn64_bwd(Q, K, V, G, B, S, D, causal, accumulate=True, init=init)
    for g, r, i in zip(acc, ref, init):
        assert maxrel(g, r + i) <= 1e-11
    shared = sum(O.attention_bwd(Q, Q, Q, G, B, S, D, causal))
    assert maxrel(attn64_bwd(Q, Q, Q, G, B, S, D, causal, alias=True)[0], shared) <= 1e-11
