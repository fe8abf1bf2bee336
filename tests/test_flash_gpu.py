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


@pytest.mark.parametrize("BH,S,D", [(2, 1040, 32), (2, 1040, 64), (2, 1040, 128), (1, 17, 128),
                                    (3, 2000, 64), (8, 2048, 32), (40, 512, 128), (96, 256, 64)])
@pytest.mark.parametrize("causal", [True, False])
def test_fp32_fwd_small_grid_key_chunks(BH, S, D, causal):
    # Small grids take 16-row work-groups whose 8 waves split the key range in 16- or 32-key
    # chunks: S = 1040 and 2000 give each wave several chunks (online rescaling across them,
    # the next chunk's loads in flight) and a ragged last chunk whose V rows past S read zeros
    # through the buffer range; S = 17 a single partial chunk; (8, 2048, 32), (40, 512, 128) and
    # (96, 256, 64) grids of half to three quarters of a round of 128-row tiles, which take
    # this kernel when causal (non-causal: the tiled kernels).  fp64 oracle, and for causal
    # grids row 0 is V's row 0.
    Q, K, V = inputs(BH, S, D, 3000 + S + D + causal, scale=0.5, n=3)
    got, lse = flash_fwd(Q, K, V, BH, S, D, causal)
    Q64, K64, V64 = (x.astype(np.float64) for x in (Q, K, V))
    tol = 1e-5 * np.sqrt(S)
    assert maxrel(got, O.attention(Q64, K64, V64, BH, S, D, causal)) <= tol
    assert np.abs(lse - ref_lse(Q, K, BH, S, D, causal)).max() <= tol
    if causal:
        assert np.allclose(got.reshape(BH, S, D)[:, 0], V.reshape(BH, S, D)[:, 0], atol=1e-6)


@pytest.mark.parametrize("BH,S", [(130, 257), (64, 520), (300, 1), (256, 3)])
@pytest.mark.parametrize("D", [32, 64, 128])
@pytest.mark.parametrize("causal", [True, False])
def test_fp32_fwd_wide_grid(BH, S, D, causal):
    # Grids that fill the chip (the small-grid 16-row kernel covers the 3-slice shapes above):
    # 130 slices x 257 rows take 256-row work-groups on 8 waves (a one-row last tile), 64 x 520
    # causal 128-row work-groups on 4 waves (its 256-row grid, 192, is short of one round of
    # the CUs; non-causal takes 8 waves from 5/8 of a round); many one- and three-row slices
    # take the 8-wave kernel with a single, mostly padding stage; ragged last blocks, fp64
    # oracle.
    Q, K, V = inputs(BH, S, D, 1000 + D + causal, n=3)
    got, lse = flash_fwd(Q, K, V, BH, S, D, causal)
    Q64, K64, V64 = (x.astype(np.float64) for x in (Q, K, V))
    tol = 1e-5 * np.sqrt(S)
    assert maxrel(got, O.attention(Q64, K64, V64, BH, S, D, causal)) <= tol
    assert np.abs(lse - ref_lse(Q, K, BH, S, D, causal)).max() <= tol


@pytest.mark.parametrize("BH,S", [(130, 257), (64, 520), (300, 2), (256, 3), (64, 256), (32, 256),
                                  (200, 20)])
@pytest.mark.parametrize("D", [32, 64, 128])
@pytest.mark.parametrize("causal", [True, False])
def test_fp32_bwd_wide_grid(BH, S, D, causal):
    # Grids that fill the chip: 130 x 257 takes the dQ launch on 256-query tiles (8 waves, a
    # one-row last tile), 64 x 520 on 128-query tiles (4 waves), many two- and three-row
    # slices the 8-wave launch with one mostly padding stage; 64 x 256 and 32 x 256 at
    # D = 128 the smaller work-groups of both launches (dK/dV on 4 and 2 waves, dQ on 2 and 1),
    # as grids short of a round take them (except where the small-grid 16-row kernels do:
    # 64 x 256 and 32 x 256 at D <= 64, causal ones at D = 128, and causal 256 x 3 at D <= 64);
    # 200 x 20 non-causal at D = 128 the 1-wave work-groups of both.  The whole tensor meets the
    # normwise bar; each slice, so that a misplaced tile cannot hide behind the others,
    # meets it relative to the size of the terms it sums (for two keys dQ_1 is
    # scale P10 P11 (dP10 - dP11)(K0 - K1), which cancellation can make far smaller than
    # the fp32 rounding of dP and D).
    Q, K, V, G = inputs(BH, S, D, 2000 + D + causal)
    Of, lse = flash_fwd(Q, K, V, BH, S, D, causal)
    grads = flash_bwd(Q, K, V, Of, G, lse, BH, S, D, causal)
    refs = _bwd_ref(Q, K, V, G, BH, S, D, causal)
    mags = _bwd_term_size(Q, K, V, G, BH, S, D, causal)
    tol = 1e-5 * np.sqrt(S)
    for name, g, r, m in zip("QKV", grads, refs, mags):
        assert maxrel(g, r) <= tol, name
        err = np.abs(g.reshape(BH, S, D) - r.reshape(BH, S, D)).max(axis=(1, 2))
        worst = int(np.argmax(err / (tol * m.max(axis=(1, 2)))))
        assert err[worst] <= tol * m[worst].max(), (name, worst)


@pytest.mark.parametrize("BH,S,D,causal", [(8, 4096, 128, True), (16, 2048, 128, False),
                                           (13, 2558, 128, True), (24, 1500, 64, True),
                                           (20, 1700, 64, False)])
def test_fp32_bwd_stored_ds_few_slices(BH, S, D, causal):
    """Grids of a round of 128-key dK/dV work-groups over few, long slices: that launch
    stores scale dS and dQ comes from one GEMM launch over all T = ceil(S / 128) query tiles of
    every slice, heaviest first -- 32, 16, 20, 12 and 14 tiles here, so tile t's dS rows (keys
    up to 128 (t + 1) causal, all 128 T otherwise) sit far into each slice's scratch; S = 2558,
    1500 and 1700 leave a ragged last tile (at D = 64 the GEMM's second 64-row block of it is
    short or empty), and S = 2558 rows whose length is not a multiple of 4 (the GEMM's
    scalar-load form).  Every slice of all three gradients against the fp64 oracle."""
    Q, K, V, G = inputs(BH, S, D, 9100 + S + causal)
    Of, lse = flash_fwd(Q, K, V, BH, S, D, causal)
    grads = flash_bwd(Q, K, V, Of, G, lse, BH, S, D, causal)
    refs = _bwd_ref(Q, K, V, G, BH, S, D, causal)
    tol = 1e-5 * np.sqrt(S)
    for name, g, r in zip("QKV", grads, refs):
        for b in range(BH):
            assert maxrel(g.reshape(BH, S, D)[b], r.reshape(BH, S, D)[b]) <= tol, (name, b)


_CHUNK_SCRIPT = r"""
import hashlib, sys
sys.path.insert(0, {tests!r})
sys.path.insert(0, {root!r})
import numpy as np
from _gpu import flash_bwd, flash_fwd
for BH, S, causal in ((512, 128, True), (600, 100, False), (384, 200, True), (769, 64, True)):
    rng = np.random.default_rng(BH + S)
    Q, K, V, G = (rng.standard_normal((BH, S * 128)).astype(np.float32) for _ in range(4))
    O, lse = flash_fwd(Q, K, V, BH, S, 128, causal)
    init = [rng.standard_normal((BH, S * 128)).astype(np.float32) for _ in range(3)]
    for acc in (False, True):
        g = flash_bwd(Q, K, V, O, G, lse, BH, S, 128, causal, accumulate=acc,
                      init=init if acc else None)
        print(BH, S, int(causal), int(acc), *(hashlib.sha1(x.tobytes()).hexdigest()[:16] for x in g),
              flush=True)
"""


def test_fp32_bwd_stored_ds_slice_chunks():
    """The stored-dS backward in chunks of slices, as a scratch cap below the whole run forces
    (the cap is read once per process, so each setting runs in a child process): with a 24 MB
    cap these shapes split into 2 equal, 2 equal, 3 equal and 3 unequal chunks (257, 256, 256),
    each a round of 128-key tiles.  Every slice does the same work in any chunk, so dQ, dK and
    dV, plain and accumulated, are bit-identical to the one-chunk run.  With the stored dS off,
    dK and dV are again identical (the same dK/dV arithmetic) while dQ, recomputed by the other
    launch, differs in rounding -- which shows the chunked runs took the stored-dS path."""
    import os
    import subprocess
    import sys
    here = os.path.dirname(os.path.abspath(__file__))
    code = _CHUNK_SCRIPT.format(tests=here, root=os.path.dirname(here))

    def run(env):
        r = subprocess.run([sys.executable, "-c", code], env={**os.environ, **env},
                           capture_output=True, text=True, timeout=110)
        assert r.returncode == 0, r.stdout + r.stderr
        lines = r.stdout.split("\n")
        lines = [l.split() for l in lines if l.strip()]
        assert len(lines) == 8, r.stdout
        return lines

    one = run({})
    chunked = run({"DH_FLASH_BWD_F32_DS_CAP": str(24 << 20)})
    off = run({"DH_FLASH_BWD_F32_DS": "0"})
    assert chunked == one
    for a, b in zip(one, off):
        assert a[:4] == b[:4] and a[5:] == b[5:], (a, b)   # dK, dV
        assert a[4] != b[4], a                              # dQ


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


@pytest.mark.parametrize("BH,S,causal", [(520, 257, True), (520, 257, False), (516, 130, True),
                                         (1601, 130, False), (1544, 257, False)])
@pytest.mark.parametrize("D", [32, 64, 128])
def test_bf16_fwd_wide_grid(BH, S, D, causal):
    # Wide grids: 520 slices x 257 rows in the XCD-grouped slice order with a one-row last
    # tile, 516 x 130 in rank-major order (4-wave work-groups); non-causal grids past six
    # rounds of the CUs take the 8-wave ones: 1601 x 130 (rank-major) and 1544 x 257
    # (grouped).  Against fp64 slice by slice: every slice up to 520, else the first and last
    # 32 and 32 others drawn at random (the oracle's cost).
    Q, K, V = (bf16_bits(x) for x in inputs(BH, S, D, 5000 + D + causal, n=3))
    got, lse = flash_fwd(Q, K, V, BH, S, D, causal, dtype="bf16")
    if BH <= 520:
        sl = np.arange(BH)
    else:
        rng = np.random.default_rng(BH + D)
        mid = rng.choice(np.arange(32, BH - 32), 32, replace=False)
        sl = np.concatenate([np.arange(32), np.sort(mid), np.arange(BH - 32, BH)])
    n = len(sl)
    Q64, K64, V64 = (bits_to_f32(x).reshape(BH, S * D)[sl].astype(np.float64) for x in (Q, K, V))
    ref = O.attention(Q64, K64, V64, n, S, D, causal).reshape(n, S, D)
    g3 = got.reshape(BH, S, D)[sl]
    for b in range(n):
        assert maxrel(g3[b], ref[b]) <= 2e-2, int(sl[b])
    lse_ref = O.flash_lse(Q64, K64, n, S, D, causal)
    assert np.abs(lse.reshape(BH, S)[sl] - lse_ref.reshape(n, S)).max() <= 1e-3 * np.sqrt(D)


def _bwd_ref(Q, K, V, dO, BH, S, D, causal):
    args = [x.astype(np.float64) for x in (Q, K, V, dO)]
    return O.attention_bwd(*args, BH, S, D, causal)


def _bwd_term_size(Q, K, V, dO, BH, S, D, causal):
    """fp64 sizes of the terms each gradient element sums, per (slice, row, column):
    dQ: scale |P| (|dP| + |Dv|) |K|, dK: scale (|P| (|dP| + |Dv|))^T |Q|, dV: P^T |dO|, with
    Dv_i = sum_j P_ij dP_ij.  fp32 rounding of dP and Dv errs in proportion to these, not to
    the (possibly cancelled) gradient itself; they bound it from above, never define it."""
    q, k, v, g = (x.astype(np.float64).reshape(BH, S, D) for x in (Q, K, V, dO))
    sc = 1.0 / np.sqrt(D)
    s = q @ k.transpose(0, 2, 1) * sc
    if causal:
        s = np.where(np.tril(np.ones((S, S), dtype=bool)), s, -np.inf)
    p = np.exp(s - s.max(axis=-1, keepdims=True))
    p /= p.sum(axis=-1, keepdims=True)
    dp = g @ v.transpose(0, 2, 1)
    t = p * (np.abs(dp) + np.abs((p * dp).sum(axis=-1, keepdims=True)))
    return (sc * (t @ np.abs(k)), sc * (t.transpose(0, 2, 1) @ np.abs(q)),
            p.transpose(0, 2, 1) @ np.abs(g))


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


@pytest.mark.parametrize("BH,S,D,causal", [(2, 1040, 32, True), (2, 1040, 64, False),
                                           (3, 600, 64, True), (16, 300, 32, False),
                                           (20, 2048, 32, True), (2, 1040, 128, False),
                                           (4, 600, 128, True)])
def test_fp32_bwd_small_grid_chunks(BH, S, D, causal):
    # Grids short of a round of 128-row tiles take the 16-key (dK/dV) and 16-query
    # (dQ) work-groups whose 8 waves split the other dimension in 16-row chunks: several
    # chunks per wave, ragged last chunks (operand rows past S read as zeros through the
    # buffer range), and (20, 2048, 32) causal, which takes them because S >= 2048 with up to
    # two rounds of 128-row tiles.  Whole tensor against the fp64 standard backward; for the
    # shorter shapes each slice also against the size of the terms it sums.
    Q, K, V, G = inputs(BH, S, D, 4000 + S + D + causal)
    Of, lse = flash_fwd(Q, K, V, BH, S, D, causal)
    grads = flash_bwd(Q, K, V, Of, G, lse, BH, S, D, causal)
    refs = _bwd_ref(Q, K, V, G, BH, S, D, causal)
    tol = 1e-5 * np.sqrt(S)
    for name, g, r in zip("QKV", grads, refs):
        assert maxrel(g, r) <= tol, name
    if S <= 1040:
        mags = _bwd_term_size(Q, K, V, G, BH, S, D, causal)
        for name, g, r, m in zip("QKV", grads, refs, mags):
            err = np.abs(g.reshape(BH, S, D) - r.reshape(BH, S, D)).max(axis=(1, 2))
            assert (err <= tol * m.max(axis=(1, 2))).all(), name


@pytest.mark.parametrize("S", [1, 33, 64, 100, 257])
@pytest.mark.parametrize("D", [32, 64, 128])
@pytest.mark.parametrize("causal", [True, False])
def test_bf16_bwd(S, D, causal):
    BH = 2
    Q, K, V, G = (bf16_bits(x) for x in inputs(BH, S, D, S * 17 + D + causal))
    Of, lse = flash_fwd(Q, K, V, BH, S, D, causal, dtype="bf16")
    grads = flash_bwd(Q, K, V, bf16_bits(Of), G, lse, BH, S, D, causal, dtype="bf16")
    refs = _bwd_ref(*(bits_to_f32(x) for x in (Q, K, V, G)), BH, S, D, causal)
    for name, g, r in zip("QKV", grads, refs):
        if np.abs(r).max() < 1e-12:
            # S = 1: dS = P (dP - Dvec) with Dvec = dP exactly, so dQ = dK = 0; the GPU keeps
            # fp32 rounding residue of the O(1) terms dP and Dvec.
            assert np.abs(g).max() <= 2e-2, name
        else:
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


def _aliased_bwd(Q, K, V, O_, dO, LSE, BH, S, D, causal, dtype, pattern, accumulate, init):
    """dh_flash_bwd with gradient buffers shared as one tensor passed twice or three times:
    pattern "qqq" (dQ = dK = dV) or "qkk" (dK = dV).  Returns the distinct buffers."""
    scale = 1.0 / np.sqrt(D)
    dt = hip.BF16 if dtype == "bf16" else hip.F32
    np_t = np.uint16 if dtype == "bf16" else np.float32
    bufs = [hip.DeviceBuffer.from_numpy(np.ascontiguousarray(x, np_t)) for x in (Q, K, V, O_, dO)]
    dL = hip.DeviceBuffer.from_numpy(np.ascontiguousarray(LSE, np.float32))
    g = [hip.DeviceBuffer.from_numpy(np.ascontiguousarray(x, np.float32)) for x in init]
    if pattern == "qqq":
        hip.flash_bwd(dt, BH, S, D, scale, causal, *bufs, dL, g[0], g[0], g[0], int(accumulate))
        return (g[0].numpy(),)
    hip.flash_bwd(dt, BH, S, D, scale, causal, *bufs, dL, g[0], g[1], g[1], int(accumulate))
    return g[0].numpy(), g[1].numpy()


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("pattern", ["qqq", "qkk"])
@pytest.mark.parametrize("accumulate", [False, True])
@pytest.mark.parametrize("BH,S,D", [(3, 200, 64), (128, 256, 128)])
def test_bwd_aliased_gradient_buffers(dtype, pattern, accumulate, BH, S, D):
    """attention(q, q, q) and attention(q, kv, kv): one tensor's gradient buffer is passed as
    two or three of dQ, dK, dV and must receive the sum of the gradients aimed at it (the
    reference adds each input's gradient in turn, autograd.inc:693-728).  fp32: 3 x 200 takes
    the small-grid 16-row kernels, 128 x 256 at D = 128 (a round of 128-row tiles) the tiled
    ones."""
    causal = True
    x, kv, G, i0, i1 = inputs(BH, S, D, 91 + accumulate + 2 * (pattern == "qkk"), n=5)
    if dtype == "bf16":
        x, kv, G = bf16_bits(x), bf16_bits(kv), bf16_bits(G)
    Q, K, V = (x, x, x) if pattern == "qqq" else (x, kv, kv)
    Of, lse = flash_fwd(Q, K, V, BH, S, D, causal, dtype=dtype)
    Oin = bf16_bits(Of) if dtype == "bf16" else Of
    init = [i0, i1] if accumulate else [np.zeros_like(i0), np.zeros_like(i0)]
    got = _aliased_bwd(Q, K, V, Oin, G, lse, BH, S, D, causal, dtype, pattern, accumulate, init)
    up = (lambda a: bits_to_f32(a)) if dtype == "bf16" else (lambda a: a)
    rQ, rK, rV = _bwd_ref(up(Q), up(K), up(V), up(G), BH, S, D, causal)
    want = (rQ + rK + rV,) if pattern == "qqq" else (rQ, rK + rV)
    tol = 2e-2 if dtype == "bf16" else 1e-5 * np.sqrt(S)
    for g, w, base in zip(got, want, init):
        assert maxrel(g - base, w) <= tol
    # separate buffers give the same sums
    sep = flash_bwd(Q, K, V, Oin, G, lse, BH, S, D, causal, dtype=dtype)
    both = (sep[0] + sep[1] + sep[2],) if pattern == "qqq" else (sep[0], sep[1] + sep[2])
    for g, w, base in zip(got, both, init):
        assert np.allclose(g - base, w, rtol=1e-5, atol=1e-5 * np.abs(w).max())


def test_bwd_rejects_partially_overlapping_gradients():
    BH, S, D = 1, 64, 32
    Q, K, V, G = inputs(BH, S, D, 8)
    Of, lse = flash_fwd(Q, K, V, BH, S, D, True)
    bufs = [hip.DeviceBuffer.from_numpy(x) for x in (Q, K, V, Of, G)]
    dL = hip.DeviceBuffer.from_numpy(lse)
    big = hip.DeviceBuffer.empty((2, S * D), np.float32)
    other = hip.DeviceBuffer.empty((BH, S * D), np.float32)
    st = hip.load().dh_flash_bwd(hip.F32, BH, S, D, 1 / np.sqrt(D), 1, *(b.ptr for b in bufs),
                                 dL.ptr, other.ptr, big.ptr, big.ptr + 256, 0)
    assert st == hip.DH_ERR_INVALID
    assert b"overlap" in hip.load().dh_last_error()


@pytest.mark.parametrize("BH", [8, 40])
@pytest.mark.parametrize("causal", [True, False])
def test_bf16_fwd_bwd_grouped_slice_order(BH, causal):
    """BH % 8 == 0 takes the forward's XCD-grouped slice order (groups of 4 slices, BH = 40
    ends on a short group); ragged S = 520 against the block sizes.  Every slice, every
    output, compared in full with the fp64 oracle."""
    S, D = 520, 128
    Q, K, V, G = (bf16_bits(x) for x in inputs(BH, S, D, 4000 + BH + causal))
    Of, lse = flash_fwd(Q, K, V, BH, S, D, causal, dtype="bf16")
    grads = flash_bwd(Q, K, V, bf16_bits(Of), G, lse, BH, S, D, causal, dtype="bf16")
    Q64, K64, V64, G64 = (bits_to_f32(x).astype(np.float64) for x in (Q, K, V, G))
    ref = O.attention(Q64, K64, V64, BH, S, D, causal).reshape(BH, S, D)
    refs = [r.reshape(BH, S, D) for r in _bwd_ref(Q64, K64, V64, G64, BH, S, D, causal)]
    for b in range(BH):   # per slice, so a misplaced slice cannot hide behind the others
        assert maxrel(Of.reshape(BH, S, D)[b], ref[b]) <= 2e-2, b
        for name, g, r in zip("QKV", grads, refs):
            assert maxrel(g.reshape(BH, S, D)[b], r[b]) <= 2e-2, (name, b)
    lse_ref = O.flash_lse(Q64, K64, BH, S, D, causal)
    assert np.abs(lse - lse_ref).max() <= 1e-3 * np.sqrt(D)


@pytest.mark.parametrize("BH,S,D", [(8, 300, 128), (8, 512, 128), (16, 1000, 64), (40, 1024, 32),
                                    (72, 2048, 128), (24, 767, 64)])
def test_bf16_causal_fwd_bwd_grouped_even_tiles(BH, S, D):
    """Causal bf16 with BH % 8 == 0 (the XCD-grouped slice order, 4 slices per group; BH = 72
    and 40 end on a short group) at q-tile counts from 2 to 8, S = 300, 1000, 767 leaving the
    last tile ragged, every head dim.  Every slice and row in full against the fp64 oracle,
    O and LSE, and the backward run on that O and LSE; a second run is bit-identical."""
    Q, K, V, G = (bf16_bits(x) for x in inputs(BH, S, D, 5000 + BH + S + D))
    Of, lse = flash_fwd(Q, K, V, BH, S, D, True, dtype="bf16")
    Q64, K64, V64, G64 = (bits_to_f32(x).astype(np.float64) for x in (Q, K, V, G))
    ref = O.attention(Q64, K64, V64, BH, S, D, True).reshape(BH, S, D)
    for b in range(BH):
        assert maxrel(Of.reshape(BH, S, D)[b], ref[b]) <= 2e-2, b
    assert np.abs(lse - O.flash_lse(Q64, K64, BH, S, D, True)).max() <= 1e-3 * np.sqrt(D)
    if S <= 1024:
        grads = flash_bwd(Q, K, V, bf16_bits(Of), G, lse, BH, S, D, True, dtype="bf16")
        refs = [r.reshape(BH, S, D) for r in _bwd_ref(Q64, K64, V64, G64, BH, S, D, True)]
        for name, g, r in zip("QKV", grads, refs):
            for b in range(BH):
                assert maxrel(g.reshape(BH, S, D)[b], r[b]) <= 2e-2, (name, b)
    # bit-identical on a second run (the schedule is static)
    again, _ = flash_fwd(Q, K, V, BH, S, D, True, dtype="bf16")
    assert np.array_equal(again, Of)


@pytest.mark.parametrize("BH,S,D", [(31, 300, 128), (33, 520, 64), (63, 200, 32)])
@pytest.mark.parametrize("causal", [True, False])
def test_bf16_padded_slice_grid(BH, S, D, causal):
    """BH not a multiple of 8 but large enough that slices are still grouped by XCD: the grid
    is padded to 8 ceil(BH / 8) slices and the work-groups past an XCD's last slice do
    nothing.  Every slice in full against the fp64 oracle (a slice computed twice or not at
    all would show), forward, LSE and backward."""
    Q, K, V, G = (bf16_bits(x) for x in inputs(BH, S, D, 7000 + BH + S + causal))
    Of, lse = flash_fwd(Q, K, V, BH, S, D, causal, dtype="bf16")
    grads = flash_bwd(Q, K, V, bf16_bits(Of), G, lse, BH, S, D, causal, dtype="bf16")
    Q64, K64, V64, G64 = (bits_to_f32(x).astype(np.float64) for x in (Q, K, V, G))
    ref = O.attention(Q64, K64, V64, BH, S, D, causal).reshape(BH, S, D)
    refs = [r.reshape(BH, S, D) for r in _bwd_ref(Q64, K64, V64, G64, BH, S, D, causal)]
    for b in range(BH):
        assert maxrel(Of.reshape(BH, S, D)[b], ref[b]) <= 2e-2, b
        for name, g, r in zip("QKV", grads, refs):
            assert maxrel(g.reshape(BH, S, D)[b], r[b]) <= 2e-2, (name, b)
    assert np.abs(lse - O.flash_lse(Q64, K64, BH, S, D, causal)).max() <= 1e-3 * np.sqrt(D)


@pytest.mark.parametrize("causal", [True, False])
def test_bf16_bwd_wide_grid(causal):
    """88 slices x 520 rows at D = 128: a dQ grid of 264 256-query tiles, the band that keeps
    8-wave dQ work-groups (other shapes take 4-wave ones).  12 slices (the first and last 4, 4
    drawn at random) in full against the fp64 oracle."""
    BH, S, D = 88, 520, 128
    Q, K, V, G = (bf16_bits(x) for x in inputs(BH, S, D, 6000 + causal))
    Of, lse = flash_fwd(Q, K, V, BH, S, D, causal, dtype="bf16")
    grads = flash_bwd(Q, K, V, bf16_bits(Of), G, lse, BH, S, D, causal, dtype="bf16")
    rng = np.random.default_rng(88 + causal)
    sl = np.concatenate([np.arange(4), np.sort(rng.choice(np.arange(4, BH - 4), 4, replace=False)),
                         np.arange(BH - 4, BH)])
    n = len(sl)
    Q64, K64, V64, G64 = (bits_to_f32(x).reshape(BH, S * D)[sl].astype(np.float64)
                          for x in (Q, K, V, G))
    refs = [r.reshape(n, S, D) for r in _bwd_ref(Q64, K64, V64, G64, n, S, D, causal)]
    for name, g, r in zip("QKV", grads, refs):
        g3 = g.reshape(BH, S, D)[sl]
        for b in range(n):
            assert maxrel(g3[b], r[b]) <= 2e-2, (name, int(sl[b]))


@pytest.mark.timeout(600)
def test_c4_bf16_fwd_bwd_full_size():
    """Config 4: B=8 H=16 (128 slices) S=4096 D=128, Q,K,V,dO ~ N(0,1) rounded to bf16,
    causal, fp32 accumulate / LSE.  Every slice of O, dQ, dK, dV is compared in full with the
    fp64 oracle (standard causal attention and its backward, slices in parallel on the host),
    each slice on its own so that a misplaced or skipped slice cannot hide behind the others;
    LSE of every row against the oracle's log-sum-exp.  Causal row 0 of O equals V_0."""
    BH, S, D = 128, 4096, 128
    rng = np.random.default_rng(4096)
    Q, K, V, G = (bf16_bits(rng.standard_normal((BH, S * D), dtype=np.float32)) for _ in range(4))
    Of, lse = flash_fwd(Q, K, V, BH, S, D, True, dtype="bf16")
    dQ, dK, dV = flash_bwd(Q, K, V, bf16_bits(Of), G, lse, BH, S, D, True, dtype="bf16")
    Q64, K64, V64, G64 = (bits_to_f32(x).astype(np.float64) for x in (Q, K, V, G))
    got = [x.reshape(BH, S, D) for x in (Of, dQ, dK, dV)]
    rO = O.attention(Q64, K64, V64, BH, S, D, True).reshape(BH, S, D)
    assert np.allclose(got[0][:, 0], V64.reshape(BH, S, D)[:, 0], atol=1e-2)
    for b in range(BH):
        assert maxrel(got[0][b], rO[b]) <= 2e-2, ("O", b)
    del rO
    lse_ref = O.flash_lse(Q64, K64, BH, S, D, True)
    assert np.abs(lse - lse_ref).max() <= 1e-3 * np.sqrt(D)
    refs = [r.reshape(BH, S, D) for r in O.attention_bwd(Q64, K64, V64, G64, BH, S, D, True)]
    for name, g, r in zip(("dQ", "dK", "dV"), got[1:], refs):
        for b in range(BH):
            assert maxrel(g[b], r[b]) <= 2e-2, (name, b)
