"""Pins the CPU oracle (oracle/dream_oracle.cpp) before anything is checked against it.

Three kinds of evidence, chosen so that a dropped term, a wrong sign or index or a
transposed operand fails at least one check:
  1. golden vectors written by the reference runtime itself (tests/golden/);
  2. the reference build in oracle/_ref/, called on fresh inputs (skipped where the
     reference tree was not available to build it, e.g. on the GPU box);
  3. mathematics: closed forms, special cases, independent numpy/scipy/torch
     computations and central finite differences.
Runs on the CPU only.
"""
import os

import numpy as np
import pytest
import scipy.special as sps

import _oracle as O
import _ref_runtime

GOLD = np.load(os.path.join(os.path.dirname(__file__), "golden", "ref_vectors.npz"))


def rel(a, b):
    return float(np.abs(np.asarray(a) - np.asarray(b)).max() / max(np.abs(b).max(), 1e-300))


@pytest.fixture(scope="module", autouse=True)
def _oracle_built():
    O.lib()


# --------------------------------------------------------------------------- golden
def test_rng_matches_reference_stream():
    O.set_seed(42)
    assert np.array_equal(O.randn(4, 250), GOLD["rng_randn_s42"])
    O.set_seed(7)
    assert np.array_equal(O.kaiming(16, 10), GOLD["rng_kaiming_s7_16x10"])


def _mt19937_raw(seed, n):
    """n raw 32-bit outputs of an independent mt19937: numpy's legacy RandomState seeds an
    integer with init_genrand, the seeding of std::mt19937(seed)."""
    return np.random.RandomState(seed)._bit_generator.random_raw(n).astype(np.uint64)


def _round_f32(v):
    """Exact rational v rounded to the nearest float32 (ties to even)."""
    from fractions import Fraction
    c = np.float32(float(v))
    best = None
    for x in (np.nextafter(c, np.float32(-np.inf)), c, np.nextafter(c, np.float32(np.inf))):
        d = abs(Fraction(float(x)) - v)
        key = (d, int(np.float32(x).view(np.uint32)) & 1)
        if best is None or key < best[0]:
            best = (key, x)
    return np.float32(best[1])


@pytest.mark.parametrize("lo,hi", [(0.0, 1.0), (-1.0, 1.0), (0.1, 10.0), (-2.5, 0.3)])
def test_uniform_draws_follow_generate_canonical(lo, hi):
    """orc_uniform / orc_uniform_f32 are std::uniform_real_distribution over the reference's
    mt19937 (elementwise.inc:897, builtins.inc:158-160).  Restated independently: libstdc++'s
    generate_canonical<T, digits> takes ceil(digits / 32) raw words, sum_i w_i 2^(32 i) / 2^(32 k)
    (1.0 clamped to the largest value below it), then a + (b - a) r, fused into one rounding
    by the reference's -ffast-math -mfma build.  Bit-exact on 2000 draws per seed."""
    from fractions import Fraction
    for seed in (1, 42, 20260707):
        n = 2000
        O.set_seed(seed)
        got = O.uniform(n, lo, hi)
        w = _mt19937_raw(seed, 2 * n)
        r = (w[0::2].astype(np.float64) + w[1::2].astype(np.float64) * 2.0 ** 32) / 2.0 ** 64
        r = np.where(r >= 1.0, np.nextafter(1.0, 0.0), r)
        want = np.array([float(Fraction(x) * Fraction(hi - lo) + Fraction(lo)) for x in r])
        assert np.array_equal(got, want), seed
        # one word per float draw (24 digits <= 32)
        lo32, hi32 = np.float32(lo), np.float32(hi)
        O.set_seed(seed)
        got32 = O.uniform_f32(n, lo32, hi32)
        w = _mt19937_raw(seed, n)
        r32 = w.astype(np.float32) / np.float32(2.0 ** 32)
        r32 = np.where(r32 >= 1, np.nextafter(np.float32(1), np.float32(0)), r32)
        span = Fraction(float(hi32 - lo32))
        want32 = np.array([_round_f32(Fraction(float(x)) * span + Fraction(float(lo32)))
                           for x in r32], np.float32)
        assert np.array_equal(got32, want32), seed


def test_uniform_draws_range_and_moments():
    """10^6 draws: inside [lo, hi), mean and variance of U(lo, hi) within 5 sigma, and a
    planted mistake (one word per double draw) breaks the bit-exact restatement."""
    O.set_seed(7)
    u = O.uniform(10 ** 6, -1.0, 3.0)
    assert u.min() >= -1.0 and u.max() < 3.0
    n, mu, var = u.size, 1.0, 16.0 / 12.0
    assert abs(u.mean() - mu) < 5 * np.sqrt(var / n)
    assert abs(u.var() - var) < 5 * np.sqrt((16.0 ** 2 / 80.0 - var ** 2) / n)
    O.set_seed(7)
    one_word = _mt19937_raw(7, 8).astype(np.float64)[:8] / 2.0 ** 32 * 4.0 - 1.0
    assert not np.array_equal(O.uniform(8, -1.0, 3.0), one_word)


@pytest.mark.parametrize("shape", [(65, 63, 66), (33, 300, 35), (1, 7, 1), (5, 1, 9)])
def test_gemm_d_golden(shape):
    key = "gemm_d_%dx%dx%d" % shape
    A, B, C = GOLD[key + "_A"], GOLD[key + "_B"], GOLD[key + "_C"]
    assert rel(O.gemm_d(A, B), C) <= 1e-12
    assert rel(O.gemm_ref_d(A, B), C) <= 1e-11   # the reference's own selftest gate


@pytest.mark.parametrize("shape", [(33, 31, 35), (40, 300, 37)])
def test_gemm_f32_golden(shape):
    key = "gemm_f32_%dx%dx%d" % shape
    A, B, C = GOLD[key + "_A"], GOLD[key + "_B"], GOLD[key + "_C"]
    got = O.gemm_f32(A.astype(np.float32), B.astype(np.float32))
    assert rel(got, C) <= 1e-6


def test_matmul_bwd_golden():
    k = "mmbwd_65x63x66"
    dA, dB = O.matmul_bwd(GOLD[k + "_A"], GOLD[k + "_B"], GOLD[k + "_W"])
    assert rel(dA, GOLD[k + "_dA"]) <= 1e-12
    assert rel(dB, GOLD[k + "_dB"]) <= 1e-12


ATTN_CASES = [("attn_B1_S100_dk24_Bc16", 1, 100, 24, 16), ("attn_B2_S64_dk16_Bc8", 2, 64, 16, 8)]


@pytest.mark.parametrize("key,B,S,dk,Bc", ATTN_CASES)
def test_attention_family_golden(key, B, S, dk, Bc):
    Q, K, V, W = (GOLD[f"{key}_{c}"] for c in "QKVW")
    assert rel(O.attention(Q, K, V, B, S, dk, False), GOLD[key + "_plain_O"]) <= 1e-12
    assert rel(O.attention(Q, K, V, B, S, dk, True), GOLD[key + "_causal_O"]) <= 1e-12
    assert rel(O.flash_fwd(Q, K, V, B, S, dk, Bc), GOLD[key + "_flash_O"]) <= 1e-12
    grads = {
        "plain": O.attention_bwd(Q, K, V, W, B, S, dk, False),
        "causal": O.attention_bwd(Q, K, V, W, B, S, dk, True),
        "flash": O.flash_bwd(Q, K, V, W, B, S, dk),
    }
    for kind, g in grads.items():
        for i, c in enumerate("QKV"):
            assert rel(g[i], GOLD[f"{key}_{kind}_d{c}"]) <= 1e-12, (kind, c)


def test_softmax_golden():
    X = GOLD["softmax_X"]
    assert rel(O.softmax_rows(X), GOLD["softmax_Y"]) <= 1e-14
    assert rel(O.log_softmax_rows(X), GOLD["log_softmax_Y"]) <= 1e-14


# --------------------------------------------------------------------------- mathematics
def test_gemm_closed_forms():
    # all-ones M x K @ K x N is exactly K everywhere (tests/09, 10, 13; gpu_diagnose 256^2).
    for M, K, N in [(2, 3, 2), (256, 256, 256), (7, 300, 5)]:
        C = O.gemm_d(np.ones((M, K)), np.ones((K, N)))
        assert np.all(C == K)
        assert np.all(O.gemm_f32(np.ones((M, K)), np.ones((K, N))) == K)
    A = np.random.default_rng(1).standard_normal((37, 41))
    assert np.array_equal(O.gemm_ref_d(A, np.eye(41)), A)
    assert np.array_equal(O.gemm_d(np.eye(37), A), A)


def test_gemm_against_independent_numpy():
    rng = np.random.default_rng(2)
    for M, K, N in [(65, 63, 66), (130, 513, 67), (1, 1, 1), (9, 1000, 3)]:
        A, B = rng.standard_normal((M, K)), rng.standard_normal((K, N))
        ref = A @ B
        assert rel(O.gemm_ref_d(A, B), ref) <= 1e-13
        assert rel(O.gemm_d(A, B), ref) <= 1e-13
        assert rel(O.gemm_f32(A, B), A.astype(np.float32).astype(np.float64)
                   @ B.astype(np.float32).astype(np.float64)) <= 2e-6 * np.sqrt(K)


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_gemm_general_transposes_and_beta(ta, tb):
    rng = np.random.default_rng(3 + 2 * ta + tb)
    M, N, K = 23, 17, 29
    A = rng.standard_normal((K, M) if ta else (M, K))
    B = rng.standard_normal((N, K) if tb else (K, N))
    C0 = rng.standard_normal((M, N))
    opA = A.T if ta else A
    opB = B.T if tb else B
    for beta in (0.0, 1.0, -0.5):
        got = O.gemm_general_d(ta, tb, A, B, beta, C0)
        assert rel(got, opA @ opB + beta * C0) <= 1e-13
    # beta = 0 must ignore C, even NaN
    got = O.gemm_general_d(ta, tb, A, B, 0.0, np.full((M, N), np.nan))
    assert np.isfinite(got).all()


def test_matmul_bwd_is_nt_tn_and_accumulates():
    rng = np.random.default_rng(4)
    A, B, dY = rng.standard_normal((13, 7)), rng.standard_normal((7, 11)), rng.standard_normal((13, 11))
    dA0, dB0 = rng.standard_normal((13, 7)), rng.standard_normal((7, 11))
    dA, dB = O.matmul_bwd(A, B, dY, dA0, dB0)
    assert rel(dA, dA0 + dY @ B.T) <= 1e-13
    assert rel(dB, dB0 + A.T @ dY) <= 1e-13


def _fd_grad(f, X, eps=1e-6):
    g = np.zeros_like(X)
    flat, gf = X.reshape(-1), g.reshape(-1)
    for i in range(flat.size):
        h = eps * max(1.0, abs(flat[i]))
        old = flat[i]
        flat[i] = old + h
        fp = f()
        flat[i] = old - h
        fm = f()
        flat[i] = old
        gf[i] = (fp - fm) / (2 * h)
    return g


@pytest.mark.parametrize("causal", [False, True])
def test_attention_bwd_finite_differences(causal):
    # gradcheck pattern of training.inc:3856-3907: loss = sum(O * W) with random W.
    rng = np.random.default_rng(5)
    B, S, dk = 2, 5, 3
    Q, K, V, W = (rng.standard_normal((B, S * dk)) for _ in range(4))
    loss = lambda: float((O.attention(Q, K, V, B, S, dk, causal) * W).sum())  # noqa: E731
    dQ, dK, dV = O.attention_bwd(Q, K, V, W, B, S, dk, causal)
    for X, g in ((Q, dQ), (K, dK), (V, dV)):
        assert rel(g, _fd_grad(loss, X)) <= 1e-6
    if causal:
        fQ, fK, fV = O.flash_bwd(Q, K, V, W, B, S, dk)
        for a, b in ((fQ, dQ), (fK, dK), (fV, dV)):
            assert rel(a, b) <= 1e-12


def test_flash_special_cases():
    rng = np.random.default_rng(6)
    # S = 1: the only key is the query's own -> O = V.
    Q, K, V = (rng.standard_normal((3, 8)) for _ in range(3))
    assert rel(O.flash_fwd(Q, K, V, 3, 1, 8), V) <= 1e-15
    # Constant keys: uniform weights over j <= i -> causal running mean of V.
    S, dk = 37, 4
    Q = rng.standard_normal((1, S * dk))
    K = np.tile(rng.standard_normal(dk), S)[None, :]
    V = rng.standard_normal((1, S * dk))
    Vm = V.reshape(S, dk)
    mean = np.cumsum(Vm, axis=0) / np.arange(1, S + 1)[:, None]
    for Bc in (1, 5, 64):
        assert rel(O.flash_fwd(Q, K, V, 1, S, dk, Bc).reshape(S, dk), mean) <= 1e-13
    # flash == standard causal at the reference's own selftest gate (1e-9).
    for S, dk, Bc in [(64, 16, 8), (64, 16, 16), (128, 32, 32), (100, 24, 16)]:
        Q, K, V = (rng.standard_normal((1, S * dk)) for _ in range(3))
        assert rel(O.flash_fwd(Q, K, V, 1, S, dk, Bc), O.attention(Q, K, V, 1, S, dk, True)) < 1e-9


def test_attention_against_independent_numpy():
    rng = np.random.default_rng(7)
    B, S, dk = 3, 19, 6
    Q, K, V = (rng.standard_normal((B, S * dk)) for _ in range(3))
    for causal in (False, True):
        q, k, v = (x.reshape(B, S, dk) for x in (Q, K, V))
        s = q @ k.transpose(0, 2, 1) / np.sqrt(dk)
        if causal:
            s = np.where(np.tril(np.ones((S, S), bool)), s, -np.inf)
        ref = (sps.softmax(s, axis=-1) @ v).reshape(B, S * dk)
        assert rel(O.attention(Q, K, V, B, S, dk, causal), ref) <= 1e-13
        lse = sps.logsumexp(s, axis=-1)
        assert rel(O.flash_lse(Q, K, B, S, dk, causal), lse) <= 1e-13


@pytest.mark.parametrize("causal", [True, False])
def test_attention_rows_are_rows_of_the_full_oracle(causal):
    """orc_attention_rows (the row-sampled check of full-size attention) against the rows of
    orc_attention(_causal) and of orc_attention_bwd's dQ, both pinned above, on ragged
    shapes with random row choices per slice (incl. row 0 and row S - 1)."""
    rng = np.random.default_rng(11 + causal)
    for B, S, dk in ((3, 37, 16), (2, 130, 64)):
        Q, K, V, G = (rng.standard_normal((B, S * dk)) for _ in range(4))
        rows = np.stack([np.r_[0, S - 1, rng.choice(np.arange(1, S - 1), 5, replace=False)]
                         for _ in range(B)])
        Orow, dQrow = O.attention_rows(Q, K, V, G, rows, B, S, dk, causal)
        Of = O.attention(Q, K, V, B, S, dk, causal).reshape(B, S, dk)
        dQf = O.attention_bwd(Q, K, V, G, B, S, dk, causal)[0].reshape(B, S, dk)
        for b in range(B):
            assert rel(Orow[b], Of[b, rows[b]]) <= 1e-13
            assert rel(dQrow[b], dQf[b, rows[b]]) <= 1e-12
    # a planted wrong mask (non-causal rows where causal ones were asked) is caught
    if causal:
        Orow_nc, _ = O.attention_rows(Q, K, V, G, rows, B, S, dk, False)
        assert rel(Orow_nc[:, 2:], Of[np.arange(B)[:, None], rows][:, 2:]) > 1e-3


def test_attention_bwd_invariants():
    # sum_j dS_ij = 0 per row  <=>  sum over keys of dK contributions is consistent;
    # checked through the identity D_i = dO_i . O_i = sum_j P_ij dP_ij.
    rng = np.random.default_rng(8)
    B, S, dk = 1, 9, 4
    Q, K, V, dO = (rng.standard_normal((B, S * dk)) for _ in range(4))
    O_ = O.attention(Q, K, V, B, S, dk, True).reshape(S, dk)
    q, k, v, do = (x.reshape(S, dk) for x in (Q, K, V, dO))
    s = np.where(np.tril(np.ones((S, S), bool)), q @ k.T / np.sqrt(dk), -np.inf)
    P = sps.softmax(s, axis=-1)
    dP = do @ v.T
    assert np.allclose((do * O_).sum(1), (P * dP).sum(1), rtol=1e-12, atol=1e-12)
    # shifting every key by the same vector c adds q_i . c to a whole score row, which
    # the row softmax removes: O is unchanged.
    K2 = (k + rng.standard_normal(dk)[None, :]).reshape(1, -1)
    assert rel(O.attention(Q, K2, V, B, S, dk, True).reshape(S, dk), O_) <= 1e-13


def test_softmax_math():
    rng = np.random.default_rng(9)
    X = rng.standard_normal((11, 257)) * 5
    Y = O.softmax_rows(X)
    assert np.allclose(Y.sum(1), 1.0, atol=1e-14)
    assert rel(Y, sps.softmax(X, axis=1)) <= 1e-14
    assert rel(O.softmax_rows(X + 3.0), Y) <= 1e-13          # shift invariance
    assert rel(O.log_softmax_rows(X), sps.log_softmax(X, axis=1)) <= 1e-14


def test_bf16_round_to_nearest_even():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(10)
    x = np.concatenate([
        rng.standard_normal(100000).astype(np.float32) * np.float32(10) ** rng.integers(
            -30, 30, 100000).astype(np.float32),
        np.array([0.0, -0.0, 1.0, -1.0, 3.4e38, 1e-40, -1e-40], np.float32),
        # exact ties: 1 + 2^-8 (even below), 1 + 3*2^-8 (even above)
        np.array([1.00390625, 1.01171875, -1.00390625], np.float32),
    ])
    x = x[np.isfinite(x)]
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(O.bf16_bits(x), ref)
    assert O.to_bf16(1.00390625) == 1.0
    assert O.to_bf16(1.01171875) == 1.015625


def test_planted_mistakes_are_caught():
    """Mutations of the oracle's outputs that a plausible bug would produce fail the gates."""
    k = "attn_B1_S100_dk24_Bc16"
    Q, K, V, W = (GOLD[f"{k}_{c}"] for c in "QKVW")
    good = O.flash_fwd(Q, K, V, 1, 100, 24, 16)
    # dropped scale (1/sqrt(dk) missing) -> reference mismatch
    bad = O.flash_fwd(Q * np.sqrt(24), K, V, 1, 100, 24, 16)
    assert rel(good, GOLD[k + "_flash_O"]) <= 1e-12 and rel(bad, GOLD[k + "_flash_O"]) > 1e-3
    # swapped Q and K -> mismatch
    assert rel(O.flash_fwd(K, Q, V, 1, 100, 24, 16), GOLD[k + "_flash_O"]) > 1e-3
    # non-causal instead of causal -> mismatch
    assert rel(O.attention(Q, K, V, 1, 100, 24, False), GOLD[k + "_flash_O"]) > 1e-3
    # transposed B in the GEMM -> mismatch
    g = "gemm_d_65x63x66"
    A, B = GOLD[g + "_A"], GOLD[g + "_B"]
    assert rel(O.gemm_d(A, B[::-1]), GOLD[g + "_C"]) > 1e-3


# --------------------------------------------------------------------------- reference build
needs_ref = pytest.mark.skipif(not _ref_runtime.available(),
                               reason="oracle/_ref not built (no reference tree on this host)")


@pytest.fixture(scope="module")
def ref():
    return _ref_runtime.RefRuntime()


@needs_ref
@pytest.mark.parametrize("shape", [(257, 129, 255), (64, 64, 64), (7, 13, 17), (300, 200, 257)])
def test_gemm_against_reference_build(ref, shape):
    M, K, N = shape
    rng = np.random.default_rng(M * 7 + K)
    A, B = rng.standard_normal((M, K)), rng.standard_normal((K, N))
    assert rel(O.gemm_d(A, B), ref.matmul(A, B)) <= 1e-12
    assert rel(O.gemm_f32(A, B), ref.matmul(A, B, f32=True)) <= 1e-6


@needs_ref
def test_flash_against_reference_build(ref):
    rng = np.random.default_rng(12)
    B, S, dk, Bc = 2, 130, 32, 64
    Q, K, V, W = (rng.standard_normal((B, S * dk)) for _ in range(4))
    assert rel(O.flash_fwd(Q, K, V, B, S, dk, Bc), ref.attention("flash", Q, K, V, B, S, dk, Bc)) <= 1e-12
    got = O.flash_bwd(Q, K, V, W, B, S, dk)
    want = ref.attention_grads("flash", Q, K, V, W, B, S, dk, Bc)
    for a, b in zip(got, want):
        assert rel(a, b) <= 1e-12


# --------------------------------------------------------------------------- row ops, linear, bmm
def _fd_sumgrad(f, X, W, h=1e-6):
    """Central differences of sum(f(X) * W) with respect to every entry of X."""
    g = np.zeros_like(X)
    for idx in np.ndindex(X.shape):
        Xp, Xm = X.copy(), X.copy()
        Xp[idx] += h
        Xm[idx] -= h
        g[idx] = ((f(Xp) * W).sum() - (f(Xm) * W).sum()) / (2 * h)
    return g


def test_row_ops_golden():
    X, G = GOLD["softmax_X"], GOLD["softmax_G"]
    assert rel(O.softmax_bwd(O.softmax_rows(X), G), GOLD["softmax_dX"]) <= 1e-12
    assert rel(O.log_softmax_bwd(X, G), GOLD["log_softmax_dX"]) <= 1e-12
    LX, LG = GOLD["layer_norm_X"], GOLD["layer_norm_G"]
    Y = O.layer_norm(LX)
    assert rel(Y, GOLD["layer_norm_Y"]) <= 1e-12
    assert rel(O.layer_norm_bwd(LX, Y, LG), GOLD["layer_norm_dX"]) <= 1e-12


def test_row_ops_math():
    rng = np.random.default_rng(31)
    X, W = rng.standard_normal((4, 9)) * 2, rng.standard_normal((4, 9))
    # backward = finite differences of the forward (independent of the closed forms)
    assert rel(O.softmax_bwd(O.softmax_rows(X), W), _fd_sumgrad(O.softmax_rows, X, W)) <= 1e-7
    assert rel(O.log_softmax_bwd(X, W), _fd_sumgrad(O.log_softmax_rows, X, W)) <= 1e-7
    assert rel(O.layer_norm_bwd(X, O.layer_norm(X), W), _fd_sumgrad(O.layer_norm, X, W)) <= 1e-6
    # layer norm: rows have mean 0 and variance var / (var + eps); affine invariance
    Xl = rng.standard_normal((6, 300)) * 4 + 2
    Y = O.layer_norm(Xl)
    var = Xl.var(axis=1)
    assert np.abs(Y.mean(1)).max() <= 1e-13
    assert rel(Y.var(axis=1), var / (var + 1e-5)) <= 1e-12
    assert rel(O.layer_norm(Xl * 3 - 7), O.layer_norm(Xl)) <= 1e-5   # eps breaks exactness
    # softmax backward rows sum to zero; log_softmax backward of a constant gradient too
    assert np.abs(O.softmax_bwd(O.softmax_rows(X), W).sum(1)).max() <= 1e-14
    assert np.abs(O.log_softmax_bwd(X, np.ones_like(X)).sum(1)).max() <= 1e-13
    # "+=" semantics
    base = rng.standard_normal(X.shape)
    assert rel(O.softmax_bwd(O.softmax_rows(X), W, base),
               base + O.softmax_bwd(O.softmax_rows(X), W)) <= 1e-14


def test_linear_golden():
    X, W, b, G = (GOLD["linear_" + c] for c in "XWbG")
    for relu, key in ((False, "linear"), (True, "linear_relu")):
        Y = O.linear(X, W, b, relu)
        assert rel(Y, GOLD[key + "_Y"]) <= 1e-12
        dY, dX, dW, db = O.linear_bwd(X, W, Y, G, relu)
        for got, name in ((dY, "dY"), (dX, "dX"), (dW, "dW"), (db.reshape(1, -1), "db")):
            assert rel(got, GOLD[f"{key}_{name}"]) <= 1e-12, name


def test_linear_math():
    rng = np.random.default_rng(32)
    X, W, b = rng.standard_normal((6, 5)), rng.standard_normal((4, 5)), rng.standard_normal(4)
    Y = O.linear(X, W, b)
    assert rel(Y, X @ W.T + b) <= 1e-14                                   # independent numpy
    assert rel(O.linear(X, W, b, relu=True), np.maximum(X @ W.T + b, 0)) <= 1e-14
    G = rng.standard_normal(Y.shape)
    for relu in (False, True):
        dY, dX, dW, db = O.linear_bwd(X, W, O.linear(X, W, b, relu), G, relu)
        f = lambda x: O.linear(x, W, b, relu)   # noqa: E731
        assert rel(dX, _fd_sumgrad(f, X, G)) <= 1e-6
        assert rel(dW, _fd_sumgrad(lambda w: O.linear(X, w, b, relu), W, G)) <= 1e-6
        assert rel(db, _fd_sumgrad(lambda bb: O.linear(X, W, bb, relu), b, G)) <= 1e-6


def test_bmm_golden_and_math():
    A, B, G = GOLD["bmm_A"], GOLD["bmm_B"], GOLD["bmm_G"]
    assert rel(O.bmm(A, B, 3, 5, 7, 6), GOLD["bmm_C"]) <= 1e-12
    gA, gB = O.bmm_bwd(A, B, G, 3, 5, 7, 6)
    assert rel(gA, GOLD["bmm_dA"]) <= 1e-12 and rel(gB, GOLD["bmm_dB"]) <= 1e-12
    # independent numpy batched product, and its adjoint identities
    A3, B3, G3 = A.reshape(3, 5, 7), B.reshape(3, 7, 6), G.reshape(3, 5, 6)
    assert rel(O.bmm(A, B, 3, 5, 7, 6).reshape(3, 5, 6), A3 @ B3) <= 1e-14
    assert rel(gA.reshape(3, 5, 7), G3 @ B3.transpose(0, 2, 1)) <= 1e-14
    assert rel(gB.reshape(3, 7, 6), A3.transpose(0, 2, 1) @ G3) <= 1e-14


def test_planted_mistakes_in_new_rows_are_caught():
    # log_softmax backward with the softmax form (wrong formula) -> golden mismatch
    X, G = GOLD["softmax_X"], GOLD["softmax_G"]
    assert rel(O.softmax_bwd(O.log_softmax_rows(X), G), GOLD["log_softmax_dX"]) > 1e-3
    # linear with W instead of W^T (square case would hide it: use the transposed shape)
    X, W, b = GOLD["linear_X"], GOLD["linear_W"], GOLD["linear_b"]
    assert rel(O.linear(X, W, np.zeros_like(b)), GOLD["linear_Y"]) > 1e-3   # dropped bias
    # bmm operands of different batches paired (batch index off by one)
    A, B = GOLD["bmm_A"], GOLD["bmm_B"]
    assert rel(O.bmm(A, np.roll(B, 1, axis=0), 3, 5, 7, 6), GOLD["bmm_C"]) > 1e-3


@needs_ref
def test_new_rows_against_reference_build(ref):
    rng = np.random.default_rng(33)
    X, W = rng.standard_normal((17, 129)) * 2, rng.standard_normal((17, 129))
    assert rel(O.softmax_bwd(O.softmax_rows(X), W), ref.softmax_grads(X, W)) <= 1e-12
    assert rel(O.log_softmax_bwd(X, W), ref.softmax_grads(X, W, log=True)) <= 1e-12
    assert rel(O.layer_norm(X), ref.layer_norm(X)) <= 1e-12
    assert rel(O.layer_norm_bwd(X, O.layer_norm(X), W), ref.layer_norm_grads(X, W)) <= 1e-12
    Xl, Wl, bl = rng.standard_normal((40, 33)), rng.standard_normal((21, 33)), rng.standard_normal((1, 21))
    Gl = rng.standard_normal((40, 21))
    for relu in (False, True):
        Y = O.linear(Xl, Wl, bl, relu)
        assert rel(Y, ref.linear(Xl, Wl, bl, relu)) <= 1e-12
        got = O.linear_bwd(Xl, Wl, Y, Gl, relu)
        dX, dW, db, dY = ref.linear_grads(Xl, Wl, bl, Gl, relu)
        for a, b in zip(got, (dY, dX, dW, db.ravel())):
            assert rel(a, b) <= 1e-12


def test_conv2d_golden_and_finite_differences():
    X, Kn, b, G = (GOLD["conv_" + c] for c in "XKbG")
    dims = (2, 3, 7, 6, 4, 3, 2)
    assert rel(O.conv2d(X, Kn, b, *dims), GOLD["conv_Y"]) <= 1e-12
    gX, gK = O.conv2d_bwd(X, Kn, G, *dims)
    assert rel(gX, GOLD["conv_dX"]) <= 1e-12 and rel(gK, GOLD["conv_dK"]) <= 1e-12
    assert rel(O.conv2d(X, Kn, b, *dims, 1, 2), GOLD["conv_padded_Y"]) <= 1e-12
    # finite differences of the forward, valid and padded / strided (the padded backward has
    # no reference counterpart that computes it correctly)
    rng = np.random.default_rng(34)
    for pad, stride in ((0, 1), (1, 2), (2, 1)):
        N, Cin, H, W, Cout, KH, KW = 2, 2, 5, 4, 3, 3, 2
        X = rng.standard_normal((N, Cin * H * W))
        Kn = rng.standard_normal((Cout, Cin * KH * KW))
        OH, OW = O.conv_out(H, W, KH, KW, pad, stride)
        G = rng.standard_normal((N, Cout * OH * OW))
        dims = (N, Cin, H, W, Cout, KH, KW, pad, stride)
        gX, gK = O.conv2d_bwd(X, Kn, G, *dims)
        assert rel(gX, _fd_sumgrad(lambda x: O.conv2d(x, Kn, None, *dims), X, G)) <= 1e-6
        assert rel(gK, _fd_sumgrad(lambda k: O.conv2d(X, k, None, *dims), Kn, G)) <= 1e-6
    # a 1x1 kernel is a per-pixel matmul over channels
    X = rng.standard_normal((3, 4 * 9))
    Kn = rng.standard_normal((5, 4))
    Y = O.conv2d(X, Kn, None, 3, 4, 3, 3, 5, 1, 1)
    ref = np.einsum("oc,ncp->nop", Kn, X.reshape(3, 4, 9)).reshape(3, 45)
    assert rel(Y, ref) <= 1e-14


# --------------------------------------------------------------------------- elementwise
EW_RIGHTS = ("same", "row", "col", "scalar")
EW_GRAD_OPS = ("add", "sub", "mul", "div", "min", "max", "pow")
EW_NO_GRAD_UNARY = ("lnot", "floor", "ceil", "round")


def _ew_base(op):
    X = GOLD["ew_X"]
    return np.abs(X) + 0.25 if op == "pow" else X


def _ew_unary_input(op):
    X = GOLD["ew_X"]
    return np.abs(X) + 0.1 if op in ("log", "sqrt") else X * 3.0 if op in EW_NO_GRAD_UNARY else X


def _np_binary(op, A, B):
    """Independent numpy statement of each op under numpy's own broadcasting."""
    one = lambda m: m.astype(np.float64)   # noqa: E731
    return {
        "add": lambda: A + B, "sub": lambda: A - B, "mul": lambda: A * B, "div": lambda: A / B,
        "mod": lambda: np.fmod(A, B), "gt": lambda: one(A > B), "lt": lambda: one(A < B),
        "ge": lambda: one(A >= B), "le": lambda: one(A <= B),
        "eq": lambda: one(np.abs(A - B) < 1e-6), "ne": lambda: one(np.abs(A - B) >= 1e-6),
        "and": lambda: one((A > 0) & (B > 0)), "or": lambda: one((A > 0) | (B > 0)),
        "atan2": lambda: np.arctan2(A, B), "pow": lambda: np.power(A, B),
        "min": lambda: np.where(A < B, A, B), "max": lambda: np.where(A > B, A, B),
    }[op]()


def _np_unary(op, A, lo=-0.5, hi=0.5):
    return {
        "relu": lambda: np.where(A > 0, A, 0.0), "exp": lambda: np.exp(A),
        "log": lambda: np.log(A), "sqrt": lambda: np.sqrt(A), "abs": lambda: np.abs(A),
        "sigmoid": lambda: 1 / (1 + np.exp(-A)), "tanh": lambda: np.tanh(A),
        "lnot": lambda: (A == 0).astype(np.float64), "sin": lambda: np.sin(A),
        "cos": lambda: np.cos(A), "tan": lambda: np.tan(A), "atan": lambda: np.arctan(A),
        "floor": lambda: np.floor(A), "ceil": lambda: np.ceil(A),
        "round": lambda: np.where(A >= 0, np.floor(A + 0.5), -np.floor(-A + 0.5)),
        "clip": lambda: np.maximum(lo, np.minimum(hi, A)),
    }[op]()


@pytest.mark.parametrize("op", O.BINOPS)
def test_binary_golden(op):
    A, G = _ew_base(op), GOLD["ew_G"]
    for r in EW_RIGHTS:
        key, B = f"ew_{op}_{r}", GOLD["ew_B_" + r]
        C = O.binary(op, A, B)[:, :, 0, 0]
        assert rel(C, GOLD[key + "_C"]) <= 1e-15, (op, r)
        if op in EW_GRAD_OPS:
            gA, gB = O.binary_bwd(op, A, B, C, G)
            assert rel(gA, GOLD[key + "_dA"]) <= 1e-14, (op, r)
            assert rel(gB, GOLD[key + "_dB"]) <= 1e-14, (op, r)


@pytest.mark.parametrize("op", O.UNOPS[:-1])
def test_unary_golden(op):
    A = _ew_unary_input(op)
    C = O.unary(op, A)
    assert rel(C, GOLD[f"ew_u_{op}_C"]) <= 1e-15
    if op not in EW_NO_GRAD_UNARY:
        assert rel(O.unary_bwd(op, A, C, GOLD["ew_G"]), GOLD[f"ew_u_{op}_dA"]) <= 1e-15


@pytest.mark.parametrize("shapes", [((2, 3, 4, 5), (1, 3, 1, 5)), ((2, 1, 4, 1), (1, 3, 1, 5)),
                                    ((3, 4, 5, 6), (3, 4, 5, 6)), ((1, 1, 1, 7), (4, 3, 2, 1)),
                                    ((5, 2, 1, 3), (1, 1, 1, 1))])
def test_binary_broadcast_against_numpy(shapes):
    # 4-D broadcasts (the golden vectors only reach 2-D): numpy's broadcasting is an
    # independent statement of the bcastStrides rule on compatible shapes.
    rng = np.random.default_rng(sum(map(sum, shapes)))
    # one decimal: many equal pairs for eq / ne / min / max, no zero divisors
    A, B = (np.round(rng.standard_normal(s), 1) for s in shapes)
    B[B == 0] = 0.5
    for op in O.BINOPS:
        a = np.abs(A) + 0.25 if op == "pow" else A
        want = _np_binary(op, a, B)
        got = O.binary(op, a, B)
        assert got.shape == want.shape
        assert rel(got, want) <= 4e-16 or np.array_equal(got, want), op


def test_unary_against_numpy():
    rng = np.random.default_rng(5)
    X = rng.standard_normal(1000) * 3
    X[:8] = [0.0, -0.0, 0.5, -0.5, 1.5, -2.5, 2.0, -1e-300]
    for op in O.UNOPS:
        A = np.abs(X) + 0.1 if op in ("log", "sqrt") else X
        assert rel(O.unary(op, A, -0.5, 0.5), _np_unary(op, A)) <= 4e-16, op


def test_elementwise_backward_finite_differences():
    rng = np.random.default_rng(6)
    A, B, G = rng.standard_normal((4, 5)), rng.standard_normal((4, 5)), rng.standard_normal((4, 5))
    B += np.sign(B) * 0.5   # away from 0 for div, away from A for min / max
    for op in ("add", "sub", "mul", "div", "pow", "min", "max"):
        a = np.abs(A) + 0.5 if op == "pow" else A
        f = lambda x, y: O.binary(op, x, y).reshape(4, 5)   # noqa: E731
        gA, gB = O.binary_bwd(op, a, B, f(a, B), G)
        assert rel(gA, _fd_sumgrad(lambda x: f(x, B), a, G)) <= 1e-6, op
        assert rel(gB, _fd_sumgrad(lambda y: f(a, y), B, G)) <= 1e-6, op
    for op in ("relu", "exp", "log", "sqrt", "abs", "sigmoid", "tanh", "sin", "cos", "tan", "atan"):
        X = np.abs(A) + 0.2 if op in ("log", "sqrt") else A * 0.7
        gX = O.unary_bwd(op, X, O.unary(op, X), G)
        assert rel(gX, _fd_sumgrad(lambda x: O.unary(op, x), X, G)) <= 1e-6, op


def test_elementwise_planted_mistakes_are_caught():
    A, B, G = GOLD["ew_X"], GOLD["ew_B_col"], GOLD["ew_G"]
    # sub's backward with the rhs sign flipped
    gA, gB = O.binary_bwd("add", A, B, O.binary("sub", A, B), G)
    assert rel(gB, GOLD["ew_sub_col_dB"]) > 1e-3
    # a column operand read by the flat index modulo its size (the backward's rule) in the forward
    modular = A + B.ravel()[np.arange(A.size) % B.size].reshape(A.shape)
    assert rel(modular, GOLD["ew_add_col_C"]) > 1e-3
    # the forward's broadcast strides used in the backward (the reference uses j % size)
    assert rel(G.sum(axis=1, keepdims=True), GOLD["ew_add_col_dB"]) > 1e-3


@needs_ref
def test_elementwise_against_reference_build(ref):
    rng = np.random.default_rng(35)
    A, G = rng.standard_normal((13, 21)), rng.standard_normal((13, 21))
    for B in (rng.standard_normal((13, 21)), rng.standard_normal((1, 21)),
              rng.standard_normal((13, 1))):
        for op in O.BINOPS:
            a = np.abs(A) + 0.25 if op == "pow" else A
            if op in EW_GRAD_OPS:
                C, dA, dB = ref.binary(op, a, B, G)
                gA, gB = O.binary_bwd(op, a, B, C, G)
                assert rel(gA, dA) <= 1e-14 and rel(gB, dB) <= 1e-14, op
            else:
                C = ref.binary(op, a, B)
            assert rel(O.binary(op, a, B)[:, :, 0, 0], C) <= 1e-15, op
