"""The Dream builtins of the hot path on the GPU, through libdream_rt.so.

Each test restates one of the reference's own tests (tests/*.dream) or selftests in Python
and adds parity against the fp64 oracle.  fp32 tolerance: normwise max relative error
<= 1e-5 * sqrt(K) (K = contraction length); bf16: <= 2e-2 on bf16-rounded inputs.
"""
import numpy as np
import pytest

import _oracle as O
from dreamcompiler_amd import runtime as rt

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def L():
    lib = rt.load()
    assert lib.dream_hip_available() == 1
    return lib


def maxrel(a, b):
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


def test_09_matmul_ones(L):
    c = L.tensor_matmul(L.ones(rt.scalar(2), rt.scalar(3)), L.ones(rt.scalar(3), rt.scalar(2)))
    assert np.array_equal(rt.read(c), np.full((2, 2), 3.0))        # prints "3 3"


def test_10_13_f32_matmul(L):
    a = L.dream_set_precision(L.ones(rt.scalar(2), rt.scalar(2)), 1)   # ones(2,2) as f32
    c = L.tensor_matmul(a, a)
    assert rt.read(L.sum(c))[0, 0] == 8.0                            # EXPECT: 8
    assert rt.read(c)[1, 0] == 2.0                                   # f32 result synced


def test_gpu_diagnose_256(L):
    # examples/gpu/gpu_diagnose.dream: sum(ones(256,256) @ ones(256,256)) = 16777216
    o = L.ones(rt.scalar(256), rt.scalar(256))
    assert rt.read(L.sum(L.tensor_matmul(o, o)))[0, 0] == 16777216.0


def test_c1_matmul_seed42(L):
    # config 1 through the builtin: set_seed(42); A = randn(1024,1024); B = randn(...); A @ B
    L.dream_set_seed(rt.scalar(42))
    A = L.dream_randn(rt.scalar(1024), rt.scalar(1024))
    B = L.dream_randn(rt.scalar(1024), rt.scalar(1024))
    O.set_seed(42)
    A_ref, B_ref = O.randn(1024, 1024), O.randn(1024, 1024)
    assert np.array_equal(rt.read(A), A_ref)                  # same reference RNG stream
    C = rt.read(L.tensor_matmul(A, B))
    assert maxrel(C, O.gemm_d(A_ref, B_ref)) <= 1e-5 * np.sqrt(1024)


def test_matmul_backward_matches_oracle(L):
    # gradcheck matmul entry (training.inc:3933-3941) and the C2 shapes: loss = sum((A@B)*W)
    for M, K, N in [(3, 4, 5), (4096, 784, 257), (257, 4096, 10)]:
        rng = np.random.default_rng(M + K + N)
        A, B, W = rng.standard_normal((M, K)), rng.standard_normal((K, N)), rng.standard_normal((M, N))
        a, b, w = rt.tensor(A), rt.tensor(B), rt.tensor(W)
        L.backward(L.sum(L.tensor_mul(L.tensor_matmul(a, b), w)))
        dA, dB = O.matmul_bwd(A, B, W)
        assert maxrel(rt.read(a, grad=True), dA) <= 1e-5 * np.sqrt(N)
        assert maxrel(rt.read(b, grad=True), dB) <= 1e-5 * np.sqrt(M)


def test_bf16_mode_matmul(L):
    L.dream_enable_fp16()
    try:
        rng = np.random.default_rng(1)
        A, B = rng.standard_normal((300, 520)), rng.standard_normal((520, 260))
        C = rt.read(L.tensor_matmul(rt.tensor(A), rt.tensor(B)))
        Ab = O.bf16_round(A.astype(np.float32)).astype(np.float64)
        Bb = O.bf16_round(B.astype(np.float32)).astype(np.float64)
        assert maxrel(C, Ab @ Bb) <= 2e-2
        assert maxrel(C, Ab @ Bb) <= 1e-5 * np.sqrt(520)
    finally:
        L.dream_disable_fp16()


def _attn(L, fn, Q, K, V, B, S, dk, blk=None):
    args = [rt.tensor(Q), rt.tensor(K), rt.tensor(V)]
    sc = [rt.scalar(B), rt.scalar(S), rt.scalar(dk)]
    out = fn(*args, *sc, rt.scalar(blk)) if blk is not None else fn(*args, *sc)
    return args, out


@pytest.mark.parametrize("B,S,dk", [(1, 100, 24), (2, 64, 16), (4, 130, 64), (2, 33, 128),
                                    (3, 70, 96)])
def test_attention_builtins_vs_golden_math(L, B, S, dk):
    rng = np.random.default_rng(B * S + dk)
    Q, K, V, W = (rng.standard_normal((B, S * dk)) for _ in range(4))
    tol = 1e-5 * np.sqrt(S)
    for fn, causal, kind in [(L.dream_flash_attention, True, "flash"),
                             (L.dream_attention_causal, True, "causal"),
                             (L.dream_attention, False, "plain")]:
        args, o = _attn(L, fn, Q, K, V, B, S, dk, 16 if kind == "flash" else None)
        assert maxrel(rt.read(o).reshape(B, -1), O.attention(Q, K, V, B, S, dk, causal)) <= tol
        L.backward(L.sum(L.tensor_mul(o, rt.tensor(W))))
        refs = O.attention_bwd(Q, K, V, W, B, S, dk, causal)
        for t, r in zip(args, refs):
            assert maxrel(rt.read(t, grad=True).reshape(B, -1), r) <= tol, kind


def test_26_flash_backward_matches_standard(L):
    # tests/26_flash_backward.dream: sum|dQ| of flash vs attention_causal, S=32, dk=16, Bc=8
    L.dream_set_seed(rt.scalar(5))
    Q, K, V = (L.dream_randn(rt.scalar(1), rt.scalar(512)) for _ in range(3))
    sc = lambda: [rt.scalar(1.0), rt.scalar(32.0), rt.scalar(16.0)]  # noqa: E731
    L.backward(L.sum(L.dream_attention_causal(Q, K, V, *sc())))
    g1 = np.abs(rt.read(Q, grad=True)).sum()
    for t in (Q, K, V):
        L.zero_grad(t)
    L.backward(L.sum(L.dream_flash_attention(Q, K, V, *sc(), rt.scalar(8.0))))
    g2 = np.abs(rt.read(Q, grad=True)).sum()
    assert abs(g1 - g2) < 1e-7                     # FLASH_BWD_MATCH
    q, k, v = (rt.read(t) for t in (Q, K, V))
    ref = np.abs(O.flash_bwd(q, k, v, np.ones_like(q), 1, 32, 16)[0]).sum()
    assert abs(g2 - ref) <= 1e-5 * np.sqrt(32) * ref


def test_18_25_selftests(L, capfd):
    assert rt.read(L.gpu_selftest())[0, 0] == 1.0
    assert rt.read(L.flash_attention_selftest())[0, 0] == 1.0
    assert rt.read(L.dream_gpu_warmup())[0, 0] > 0.0
    out = capfd.readouterr().out
    assert "GPU: 4/4 PASS" in out                  # tests/18_gpu.dream expects "GPU:"
    assert "FLASH_ATTN: 4/4 PASS" in out           # tests/25_flash_attention.dream


def test_determinism_16(L):
    # tests/16_determinism.dream: bit-exact repeat of matmul, attention and backward
    def run():
        L.dream_set_seed(rt.scalar(16))
        A, B = L.dream_randn(rt.scalar(300), rt.scalar(200)), L.dream_randn(rt.scalar(200), rt.scalar(257))
        C = L.tensor_matmul(A, B)
        Q, K, V = (L.dream_randn(rt.scalar(2), rt.scalar(130 * 64)) for _ in range(3))
        o = L.dream_flash_attention(Q, K, V, rt.scalar(2), rt.scalar(130), rt.scalar(64), None)
        L.backward(L.sum(L.tensor_mul(o, o)))
        return rt.read(C), rt.read(o), rt.read(Q, grad=True), rt.read(K, grad=True)
    for a, b in zip(run(), run()):
        assert np.array_equal(a, b)
