"""The Dream builtins of the hot path on the GPU, through libdream_rt.so.

Each test restates one of the reference's own tests (tests/*.dream) or selftests in Python
and adds parity against the fp64 oracle.  fp32 tolerance: normwise max relative error
<= 1e-5 * sqrt(K) (K = contraction length); bf16: <= 2e-2 on bf16-rounded inputs.
"""
import os

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
    # dream_enable_fp16 changes the reference's GPU branch only (elementwise.inc:1046-1071):
    # at or above the threshold `@` takes bf16 operands; below it stays the fp64 dgemm.
    L.dream_enable_fp16()
    try:
        rng = np.random.default_rng(1)
        A, B = rng.standard_normal((600, 520)), rng.standard_normal((520, 520))
        C = rt.read(L.tensor_matmul(rt.tensor(A), rt.tensor(B)))
        Ab = O.bf16_round(A.astype(np.float32)).astype(np.float64)
        Bb = O.bf16_round(B.astype(np.float32)).astype(np.float64)
        assert maxrel(C, Ab @ Bb) <= 2e-2
        assert maxrel(C, Ab @ Bb) <= 1e-5 * np.sqrt(520)
        C = rt.read(L.tensor_matmul(rt.tensor(A[:300]), rt.tensor(B[:, :260])))
        assert np.array_equal(C, O.gemm_d(A[:300], B[:, :260]))
    finally:
        L.dream_disable_fp16()


def _attn(L, fn, Q, K, V, B, S, dk, blk=None):
    args = [rt.tensor(Q), rt.tensor(K), rt.tensor(V)]
    sc = [rt.scalar(B), rt.scalar(S), rt.scalar(dk)]
    out = fn(*args, *sc, rt.scalar(blk)) if blk is not None else fn(*args, *sc)
    return args, out


# B*S*S below 262144 (fp64 path) and at or above it (the FlashAttention kernels, dk padded to
# 32 / 64 / 128 where needed)
@pytest.mark.parametrize("B,S,dk", [(1, 100, 24), (2, 64, 16), (4, 130, 64), (2, 33, 128),
                                    (3, 70, 96), (2, 400, 24), (1, 520, 96), (2, 384, 64),
                                    (1, 512, 128)])
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


@pytest.mark.timeout(600)
@pytest.mark.parametrize("bf16", [False, True])
def test_c4_flash_builtin_full_size(L, bf16):
    """Config 4 through the builtins: dream_flash_attention(Q, K, V, 128, 4096, 128, 64) on fp64
    host tensors (B8 x H16 slices), then backward(sum(O * W)), in the default precision (fp32
    FlashAttention kernels) and with dream_enable_fp16 (bf16 kernels; inputs and W pre-rounded
    to bf16 so the oracle sees the device's values).  O, dQ, dK, dV of 6 random slices in full
    against the fp64 oracle; on every slice causal row 0 of O = V_0 and sum_j dV_j = sum_i W_i
    (rows of P sum to one)."""
    B, S, dk = 128, 4096, 128
    rng = np.random.default_rng(44 + bf16)
    X = [rng.standard_normal((B, S * dk)) for _ in range(4)]
    if bf16:
        X = [O.bf16_round(x.astype(np.float32)).astype(np.float64) for x in X]
        L.dream_enable_fp16()
    try:
        Q, K, V, W = X
        args, o = _attn(L, L.dream_flash_attention, Q, K, V, B, S, dk, 64)
        Og = rt.read(o).reshape(B, S, dk)
        w = rt.tensor(W)
        m = L.tensor_mul(o, w)
        loss = L.sum(m)
        r = L.backward(loss)
        grads = [rt.read(t, grad=True).reshape(B, S, dk) for t in args]
        rt.release(r, loss, m, w, o, *args)
    finally:
        if bf16:
            L.dream_disable_fp16()
    tol = 2e-2 if bf16 else 1e-5 * np.sqrt(S)
    V3, W3 = V.reshape(B, S, dk), W.reshape(B, S, dk)
    assert np.allclose(Og[:, 0], V3[:, 0], rtol=0, atol=tol * np.abs(V3[:, 0]).max())
    dVsum, Wsum = grads[2].sum(axis=1), W3.sum(axis=1)
    assert np.abs(dVsum - Wsum).max() <= tol * np.abs(W3).sum(axis=1).max()
    sl = rng.choice(B, 6, replace=False)
    sub = lambda x: np.ascontiguousarray(x.reshape(B, S * dk)[sl])  # noqa: E731
    rO = O.attention(sub(Q), sub(K), sub(V), len(sl), S, dk, True).reshape(-1, S, dk)
    refs = [r.reshape(-1, S, dk) for r in
            O.attention_bwd(sub(Q), sub(K), sub(V), sub(W), len(sl), S, dk, True)]
    for i, b in enumerate(sl):
        assert maxrel(Og[b], rO[i]) <= tol, ("O", b)
        for name, g, r in zip(("dQ", "dK", "dV"), grads, refs):
            assert maxrel(g[b], r[i]) <= tol, (name, b)


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


def test_15_18_25_selftests(L, capfd):
    assert rt.read(L.gemm_selftest())[0, 0] == 1.0
    assert "GEMM: 17/17 PASS" in capfd.readouterr().out   # tests/15_gemm.dream
    assert rt.read(L.bf16_selftest())[0, 0] == 1.0
    assert "BF16_MIXED: 3/3 PASS" in capfd.readouterr().out   # tests/30_bf16.dream
    assert rt.read(L.gpu_selftest())[0, 0] == 1.0
    assert rt.read(L.flash_attention_selftest())[0, 0] == 1.0
    assert rt.read(L.dream_gpu_warmup())[0, 0] > 0.0
    out = capfd.readouterr().out
    assert "GPU: 4/4 PASS" in out                  # tests/18_gpu.dream expects "GPU:"
    assert "FLASH_ATTN: 4/4 PASS" in out           # tests/25_flash_attention.dream


def _run_16_determinism(lib, scalar, read):
    """One run_once() of tests/16_determinism.dream:6-16 through a runtime's builtins: returns
    loss[0] + sum(grad(W)) * 7.0 and the pieces it is made of."""
    A = lib.dream_randn(scalar(160), scalar(160))
    W = lib.dream_randn(scalar(160), scalar(160))
    h = lib.relu(lib.tensor_matmul(A, W))            # 160 x 160: the fp64 `@` (dgemm order)
    d = lib.dream_dropout(h, scalar(0.8))
    q = lib.dream_randn(scalar(1), scalar(128))
    at = lib.dream_attention(q, q, q, scalar(1.0), scalar(4.0), scalar(32.0))   # self-attention
    loss = lib.tensor_add(lib.sum(d), lib.tensor_mul(lib.sum(at), scalar(3.0)))
    lib.backward(loss)
    gW = read(W, grad=True)
    sW = read(lib.sum(lib.tensor_get_grad(W)))[0, 0]
    f = read(loss)[0, 0] + sW * 7.0
    return f, read(loss)[0, 0], gW, read(q, grad=True), read(at)


def test_determinism_16_as_written(L):
    """tests/16_determinism.dream replayed through the builtins as written: set_seed(31337);
    randn 160 x 160 `@` (below the GPU threshold: fp64 on the GPU in dgemm's order), relu,
    dropout(h, 0.8), randn(1, 128), attention(q, q, q, 1, 4, 32) (one tensor as Q, K and V, so
    its gradient is dQ + dK + dV), loss = sum(d) + sum(at) * 3, backward; twice, bit-identical
    (DETERMINISM: PASS).  Against the reference build's CPU runtime (oracle/_ref, when present)
    on the same program: the loss, grad(W) and grad(q) to 1e-12 (the fp64 products differ from
    the reference's loops only in summation order)."""
    runs = []
    for _ in range(2):
        L.dream_set_seed(rt.scalar(31337))
        runs.append(_run_16_determinism(L, rt.scalar, rt.read))
    f1, f2 = runs[0][0], runs[1][0]
    assert f1 - f2 == 0.0                                       # DETERMINISM: PASS
    for a, b in zip(runs[0][1:], runs[1][1:]):
        assert np.array_equal(a, b)
    import _ref_runtime
    if not _ref_runtime.available():
        pytest.skip("oracle/_ref not built: bit-exact repeat checked, reference values not")
    R = _ref_runtime.RefRuntime()
    R.L.dream_set_seed(R.scalar(31337))
    ref = _run_16_determinism(R.L, R.scalar, R.read)
    assert abs(runs[0][1] - ref[1]) <= 1e-12 * abs(ref[1])       # loss
    assert maxrel(runs[0][2], ref[2]) <= 1e-12                   # grad(W)
    assert maxrel(runs[0][3], ref[3]) <= 1e-12                   # grad(q) = dQ + dK + dV
    assert maxrel(runs[0][4], ref[4]) <= 1e-12                   # attention output
    assert abs(f1 - ref[0]) <= 1e-12 * (abs(ref[1]) + 7.0 * np.abs(ref[2]).sum())


def _shared_grad_err(g, parts):
    """Normwise error of a gradient that is a sum of terms, against the scale of the terms
    (the sum itself may cancel)."""
    ref = sum(parts)
    return float(np.abs(g - ref).max() / max(sum(np.abs(p) for p in parts).max(), 1e-30))


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("kind", ["flash", "causal", "plain"])
def test_self_attention_shared_gradient_buffers(L, kind, bf16):
    """attention(q, q, q) and attention(q, kv, kv) at a FlashAttention shape (B*S*S >= 262144,
    dk = 64) through the builtins and backward(sum(O * W)): the tensor passed as several
    operands receives the sum of their gradients, as the reference's "+=" into one grad buffer
    leaves it (autograd.inc:690-728, 779-840) -- the kernels' shared-gradient path reached
    through the runtime, in the default precision (fp32 kernels) and with dream_enable_fp16
    (bf16 kernels; inputs and W pre-rounded to bf16 so the oracle sees the device's values)."""
    B, S, dk = 2, 384, 64
    causal = kind != "plain"
    fn = {"flash": L.dream_flash_attention, "causal": L.dream_attention_causal,
          "plain": L.dream_attention}[kind]
    rng = np.random.default_rng(160 + 2 * bf16 + (kind == "plain"))
    X, KV, W = (rng.standard_normal((B, S * dk)) for _ in range(3))
    if bf16:
        X, KV, W = (O.bf16_round(a.astype(np.float32)).astype(np.float64) for a in (X, KV, W))
        L.dream_enable_fp16()
    tol = 2e-2 if bf16 else 1e-5 * np.sqrt(S)
    sc = lambda: ([rt.scalar(B), rt.scalar(S), rt.scalar(dk)]  # noqa: E731
                  + ([rt.scalar(64)] if kind == "flash" else []))
    try:
        # q as Q, K and V
        q, w = rt.tensor(X), rt.tensor(W)
        o = fn(q, q, q, *sc())
        assert maxrel(rt.read(o).reshape(B, -1), O.attention(X, X, X, B, S, dk, causal)) <= tol
        L.backward(L.sum(L.tensor_mul(o, w)))
        dQ, dK, dV = O.attention_bwd(X, X, X, W, B, S, dk, causal)
        assert _shared_grad_err(rt.read(q, grad=True).reshape(B, -1), (dQ, dK, dV)) <= tol
        # q as Q, kv as K and V
        q, kv = rt.tensor(X), rt.tensor(KV)
        o = fn(q, kv, kv, *sc())
        L.backward(L.sum(L.tensor_mul(o, w)))
        dQ, dK, dV = O.attention_bwd(X, KV, KV, W, B, S, dk, causal)
        assert maxrel(rt.read(q, grad=True).reshape(B, -1), dQ) <= tol
        assert _shared_grad_err(rt.read(kv, grad=True).reshape(B, -1), (dK, dV)) <= tol
    finally:
        if bf16:
            L.dream_disable_fp16()


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


# --------------------------------------------------------------------------- other GEMM callers

GOLD = np.load(os.path.join(os.path.dirname(__file__), "golden", "ref_vectors.npz"))


def _grads_through(L, out, G, *ins):
    """backward(sum(out * G)) through the runtime; returns the .grad of each input and of out."""
    L.backward(L.sum(L.tensor_mul(out, rt.tensor(G))))
    return tuple(rt.read(t, grad=True) for t in ins) + (rt.read(out, grad=True),)


@pytest.mark.parametrize("relu", [False, True])
def test_linear_against_reference_golden(L, relu):
    # The reference build's own dream_linear / dream_linear_relu and their backward
    # (tests/golden: X 9x13, W 11x13, b 1x11, upstream G 9x11), fp32 bound 1e-5 sqrt(K).
    X, W, b, G = (GOLD["linear_" + c] for c in "XWbG")
    key = "linear_relu" if relu else "linear"
    x, w, bb = rt.tensor(X), rt.tensor(W), rt.tensor(b)
    y = (L.dream_linear_relu if relu else L.dream_linear)(x, w, bb)
    assert maxrel(rt.read(y), GOLD[key + "_Y"]) <= 1e-5 * np.sqrt(13)
    dX, dW, db, dY = _grads_through(L, y, G, x, w, bb)
    assert maxrel(dX, GOLD[key + "_dX"]) <= 1e-5 * np.sqrt(11)
    assert maxrel(dW, GOLD[key + "_dW"]) <= 1e-5 * np.sqrt(9)
    assert maxrel(db, GOLD[key + "_db"]) <= 1e-5 * np.sqrt(9)
    assert maxrel(dY, GOLD[key + "_dY"]) <= 1e-6        # the node's own (masked) gradient


def test_linear_mlp_c2_against_oracle(L):
    # Config 2 through the fused builtins: h = linear_relu(X, W1^T, b1), y = linear(h, W2^T, b2),
    # loss = sum(y * G); every gradient against the fp64 oracle.
    rng = np.random.default_rng(2)
    X = rng.uniform(0, 1, (4096, 784))
    W1, W2 = rng.standard_normal((257, 784)) * np.sqrt(2 / 784), rng.standard_normal((10, 257)) * np.sqrt(2 / 257)
    b1, b2 = rng.standard_normal(257) * 0.1, rng.standard_normal(10) * 0.1
    G = rng.standard_normal((4096, 10))
    H = O.linear(X, W1, b1, relu=True)
    Y = O.linear(H, W2, b2)
    dY2, dH, dW2, db2 = O.linear_bwd(H, W2, Y, G)
    _, dX, dW1, db1 = O.linear_bwd(X, W1, H, dH, relu=True)
    x, w1, bb1, w2, bb2 = (rt.tensor(a) for a in (X, W1, b1, W2, b2))
    h = L.dream_linear_relu(x, w1, bb1)
    y = L.dream_linear(h, w2, bb2)
    assert maxrel(rt.read(h), H) <= 1e-5 * np.sqrt(784)
    assert maxrel(rt.read(y), Y) <= 1e-5 * np.sqrt(784)
    gx, gw1, gb1, gw2, gb2, _ = _grads_through(L, y, G, x, w1, bb1, w2, bb2)
    for got, ref, K in ((gx, dX, 257), (gw1, dW1, 4096), (gb1, db1, 4096), (gw2, dW2, 4096),
                        (gb2, db2, 4096)):
        assert maxrel(got.reshape(ref.shape), ref) <= 1e-5 * np.sqrt(K)


def test_bmm_against_reference_golden(L):
    A, B, G = GOLD["bmm_A"], GOLD["bmm_B"], GOLD["bmm_G"]
    a, b = rt.tensor(A), rt.tensor(B)
    c = L.dream_bmm(a, b, *(rt.scalar(v) for v in (3, 5, 7, 6)))
    assert maxrel(rt.read(c), GOLD["bmm_C"]) <= 1e-5 * np.sqrt(7)
    dA, dB, _ = _grads_through(L, c, G, a, b)
    assert maxrel(dA, GOLD["bmm_dA"]) <= 1e-5 * np.sqrt(6)
    assert maxrel(dB, GOLD["bmm_dB"]) <= 1e-5 * np.sqrt(5)


def test_bmm_size_mismatch_message(L, capfd):
    c = L.dream_bmm(rt.tensor(np.ones((2, 5))), rt.tensor(np.ones((2, 6))),
                    *(rt.scalar(v) for v in (2, 2, 3, 2)))
    assert rt.read(c).shape == (1, 1)
    assert "error: bmm size mismatch (a=10 need 12, b=12 need 12)" in capfd.readouterr().err


@pytest.mark.parametrize("op", ["softmax", "log_softmax", "layer_norm"])
def test_row_builtins_against_reference_golden(L, op):
    if op == "layer_norm":
        X, G, Yk, dk = GOLD["layer_norm_X"], GOLD["layer_norm_G"], "layer_norm_Y", "layer_norm_dX"
        fn = L.dream_layer_norm
    else:
        X, G = GOLD["softmax_X"], GOLD["softmax_G"]
        Yk, dk = (op + "_Y"), ("softmax_dX" if op == "softmax" else "log_softmax_dX")
        fn = L.dream_softmax if op == "softmax" else L.dream_log_softmax
    x = rt.tensor(X)
    y = fn(x)
    C = X.shape[1]
    assert np.abs(rt.read(y) - GOLD[Yk]).max() <= 1e-5 * np.sqrt(C) * max(1, np.abs(GOLD[Yk]).max())
    dX, _ = _grads_through(L, y, G, x)
    assert np.abs(dX - GOLD[dk]).max() <= 1e-5 * np.sqrt(C) * max(1, np.abs(GOLD[dk]).max())


def test_device_copy_follows_in_place_writes(L):
    # A's device copy is reused by the second product only while A is unchanged: an index
    # assignment (tensor_set_element_2d bumps the version) must be seen by the next `@`.
    # M*N = 512*512 is at the threshold, so these products run on the cached fp32 copies.
    rng = np.random.default_rng(3)
    A0, B0 = rng.standard_normal((512, 32)), rng.standard_normal((32, 512))
    a, b = rt.tensor(A0), rt.tensor(B0)
    c1 = rt.read(L.tensor_matmul(a, b))
    assert maxrel(c1, A0 @ B0) <= 1e-5 * np.sqrt(32)
    L.tensor_set_element_2d(a, rt.scalar(3), rt.scalar(5), rt.scalar(7.0))
    A1 = A0.copy()
    A1[3, 5] = 7.0
    c2 = rt.read(L.tensor_matmul(a, b))
    assert maxrel(c2, A1 @ B0) <= 1e-5 * np.sqrt(32)
    L.tensor_set_element(a, rt.scalar(-1), rt.tensor(np.arange(32.0)))   # last row
    A1[-1] = np.arange(32.0)
    c3 = rt.read(L.tensor_matmul(a, b))
    assert maxrel(c3, A1 @ B0) <= 1e-5 * np.sqrt(32)


def test_attention_device_copy_follows_in_place_writes(L):
    # Same for attention on the FlashAttention kernels (B*S*S = 262144): a write to Q and a
    # version bump must reach the next forward and backward.
    B, S, dk = 1, 512, 64
    rng = np.random.default_rng(12)
    Q0, K0, V0, G = (rng.standard_normal((B, S * dk)) for _ in range(4))
    q, k, v = (rt.tensor(x) for x in (Q0, K0, V0))
    sc = lambda: [rt.scalar(B), rt.scalar(S), rt.scalar(dk)]  # noqa: E731
    o1 = rt.read(L.dream_attention_causal(q, k, v, *sc()))
    assert maxrel(o1, O.attention(Q0, K0, V0, B, S, dk, True)) <= 1e-5 * np.sqrt(S)
    L.tensor_set_element_2d(q, rt.scalar(0), rt.scalar(dk * 300 + 5), rt.scalar(9.0))
    Q1 = Q0.copy()
    Q1[0, dk * 300 + 5] = 9.0
    o = L.dream_attention_causal(q, k, v, *sc())
    o2 = rt.read(o)
    assert maxrel(o2, O.attention(Q1, K0, V0, B, S, dk, True)) <= 1e-5 * np.sqrt(S)
    assert not np.allclose(o1, o2)
    gq = _grads_through(L, o, G, q)[0]
    assert maxrel(gq, O.attention_bwd(Q1, K0, V0, G, B, S, dk, True)[0]) <= 1e-5 * np.sqrt(S)


# ---------------------------------------------------------------- the reference's dispatch
@pytest.mark.parametrize("M,K,N", [(3, 4, 5), (200, 50, 300), (100, 1000, 100), (4096, 257, 10),
                                   (511, 513, 511), (1, 3000, 1)])
def test_matmul_below_threshold_is_the_reference_fp64(L, M, K, N):
    # M*N < 262144: the reference's `@` runs dream_gemm_d (elementwise.inc:1033-1040).  The
    # runtime's fp64 GEMM sums in the same order, so `@` returns the reference's values bit
    # for bit (O.gemm_d is bit-identical to the reference build, tests/test_oracle.py), and
    # its backward is the fp64 one of autograd.inc:91-125.
    rng = np.random.default_rng(M + 3 * K + 7 * N)
    A, B, W = rng.standard_normal((M, K)), rng.uniform(-1, 1, (K, N)), rng.standard_normal((M, N))
    a, b = rt.tensor(A), rt.tensor(B)
    c = L.tensor_matmul(a, b)
    assert np.array_equal(rt.read(c), O.gemm_d(A, B))
    ga, gb, _ = _grads_through(L, c, W, a, b)
    dA, dB = O.matmul_bwd(A, B, W)
    assert maxrel(ga, dA) <= 1e-13
    assert maxrel(gb, dB) <= 1e-13


def test_matmul_threshold_and_f32_operands_take_fp32(L):
    # M*N = 262144 reaches the threshold: the fp32 matrix-core GEMM (the reference's GPU
    # branch); `as f32` operands take the fp32 GEMM at any size (elementwise.inc:1000-1017).
    rng = np.random.default_rng(21)
    A, B = rng.standard_normal((512, 300)), rng.standard_normal((300, 512))
    C = rt.read(L.tensor_matmul(rt.tensor(A), rt.tensor(B)))
    ref = O.gemm_d(A, B)
    assert maxrel(C, ref) <= 1e-5 * np.sqrt(300)
    assert not np.array_equal(C, ref)
    a, b = rt.tensor(A[:20, :30]), rt.tensor(B[:30, :20])
    L.dream_set_precision(a, 1)
    L.dream_set_precision(b, 1)
    C = rt.read(L.tensor_matmul(a, b))
    ref = O.gemm_d(A[:20, :30].astype(np.float32), B[:30, :20].astype(np.float32))
    assert maxrel(C, ref) <= 1e-5 * np.sqrt(30)
    assert not np.array_equal(C, ref)


def _gc_run(L, fwd, leaves, W):
    """The reference's gradcheck harness (training.inc:3856-3907): analytic gradients from
    backward(sum(y * w)); numerical ones by central differences with eps = 1e-6 max(1, |x|),
    written straight into each leaf's data as the reference writes them.  Returns max_rel."""
    for t in leaves:
        L.zero_grad(t)
    w = rt.tensor(W)
    y = fwd()
    L.backward(L.sum(L.tensor_mul(y, w)))
    ana = [rt.read(t, grad=True).ravel().copy() for t in leaves]

    def num_loss():
        yy = fwd()
        s = float(np.dot(rt.read(yy).ravel(), W.ravel()))
        rt.release(yy)
        return s

    max_rel, ana_abs, num_abs = 0.0, 0.0, 0.0
    for t, g in zip(leaves, ana):
        data = np.ctypeslib.as_array(t.contents.data, shape=(t.contents.size,))
        for i in range(t.contents.size):
            orig = data[i]
            eps = 1e-6 * max(1.0, abs(orig))
            data[i] = orig + eps
            lp = num_loss()
            data[i] = orig - eps
            lm = num_loss()
            data[i] = orig
            gnum = (lp - lm) / (2 * eps)
            ana_abs, num_abs = max(ana_abs, abs(g[i])), max(num_abs, abs(gnum))
            max_rel = max(max_rel, abs(gnum - g[i]) / max(abs(gnum), abs(g[i]), 1e-6))
    assert ana_abs > 1e-12 or num_abs > 1e-12     # the reference's degenerate guard
    return max_rel


def test_14_gradcheck_matmul_attention_entries(L):
    # tests/14_gradcheck.dream's entries on the hot path, replayed through this runtime with
    # the reference's harness, shapes, ranges and tolerance 1e-4: matmul 3x4 @ 4x5
    # (training.inc:3933-3941), attention and attn_causal on Q, K, V of 1 x (4*8)
    # (4180-4193, 4240-4252); flash_attention on the same shape as well.
    rng = np.random.default_rng(20260706)
    A, B = rng.uniform(-1, 1, (3, 4)), rng.uniform(-1, 1, (4, 5))
    a, b = rt.tensor(A), rt.tensor(B)
    mr = _gc_run(L, lambda: L.tensor_matmul(a, b), [a, b], rng.uniform(-1, 1, (3, 5)))
    assert mr < 1e-4, f"matmul max_rel {mr:.2e}"
    Q, K, V, W = (rng.uniform(-1, 1, (1, 32)) for _ in range(4))
    q, k, v = rt.tensor(Q), rt.tensor(K), rt.tensor(V)
    sc = lambda: [rt.scalar(1), rt.scalar(4), rt.scalar(8)]  # noqa: E731
    for name, fwd in [("attention", lambda: L.dream_attention(q, k, v, *sc())),
                      ("attn_causal", lambda: L.dream_attention_causal(q, k, v, *sc())),
                      ("flash", lambda: L.dream_flash_attention(q, k, v, *sc(), rt.scalar(2)))]:
        mr = _gc_run(L, fwd, [q, k, v], W)
        assert mr < 1e-4, f"{name} max_rel {mr:.2e}"


@pytest.mark.parametrize("B,S,dk", [(1, 40, 160), (2, 300, 256), (2, 400, 144)])
def test_attention_builtins_head_dim_above_128(L, B, S, dk):
    # dk > 128 is outside the reference's GPU rule (training.inc:336): all three builtins run
    # in fp64, forward and backward, whatever B*S*S is.
    rng = np.random.default_rng(B * S * dk)
    Q, K, V, W = (rng.standard_normal((B, S * dk)) for _ in range(4))
    for fn, causal, blk in [(L.dream_flash_attention, True, 64),
                            (L.dream_attention_causal, True, None),
                            (L.dream_attention, False, None)]:
        args, o = _attn(L, fn, Q, K, V, B, S, dk, blk)
        assert maxrel(rt.read(o).reshape(B, -1), O.attention(Q, K, V, B, S, dk, causal)) <= 1e-12
        L.backward(L.sum(L.tensor_mul(o, rt.tensor(W))))
        for t, r in zip(args, O.attention_bwd(Q, K, V, W, B, S, dk, causal)):
            assert maxrel(rt.read(t, grad=True).reshape(B, -1), r) <= 1e-11


def test_chained_gpu_graph_with_host_ops_gradients(L):
    # Gradients between GPU ops stay on the device; host ops in the middle (mul, add) must
    # see them.  loss = sum(layer_norm(softmax(((a*s) @ W) + c)) * G) against oracle/numpy.
    # The product is 512 x 512 (at the threshold), so it runs on the device copies too.
    rng = np.random.default_rng(4)
    A, S, W, Cb, G = (rng.standard_normal(sh) for sh in ((512, 24), (512, 24), (24, 512),
                                                         (512, 512), (512, 512)))
    a, s, w, cb = (rt.tensor(x) for x in (A, S, W, Cb))
    h = L.tensor_mul(a, s)
    p = L.tensor_matmul(h, w)
    q = L.tensor_add(p, cb)
    r = L.dream_softmax(q)
    y = L.dream_layer_norm(r)
    ga, gs, gw, gc, _ = _grads_through(L, y, G, a, s, w, cb)
    H = A * S
    Q = H @ W + Cb
    R = O.softmax_rows(Q)
    Y = O.layer_norm(R)
    gR = O.layer_norm_bwd(R, Y, G)
    gQ = O.softmax_bwd(R, gR)
    gW = H.T @ gQ
    gH = gQ @ W.T
    for got, ref in ((gw, gW), (gc, gQ), (ga, gH * S), (gs, gH * A)):
        assert maxrel(got, ref) <= 1e-4
