"""GPU parity of dh_gemm_f32 / dh_gemm_bf16 against the fp64 oracle.

Tolerances (stated per the contract of the north star):
  fp32: max_ij |C - C64| / max_ij |C64| <= 1e-5 * sqrt(K), where C64 is the fp64 oracle
        on the same fp64 inputs the fp32 operands were rounded from; the per-element
        form |C - C64|_ij <= 1e-5 * sqrt(K) * (|A| |B|)_ij is checked as well.
  bf16: max_ij |C - C64| / max_ij |C64| <= 2e-2, C64 = fp64 oracle on the bf16-rounded
        (round-to-nearest-even) inputs.
  The reference's own gates are also applied where they exist: gpu_selftest's
  absolute sqrt(K) * 1e-4 (elementwise.inc:840-846) and gemm_selftest's f32 2e-4.
"""
import numpy as np
import pytest

import _oracle as O
from _gpu import bf16_bits, bits_to_f32, elementwise_ratio, gemm, maxrel
from dreamcompiler_amd import hip

pytestmark = pytest.mark.gpu


def f32(x):
    return np.asarray(x, np.float32)


def check_f32(got, A64, B64, K, transA=False, transB=False, beta=0.0, C0=None):
    ref = O.gemm_general_d(transA, transB, A64, B64, beta, C0)
    tol = 1e-5 * np.sqrt(max(K, 1))
    e1 = maxrel(got, ref)
    assert e1 <= tol, f"maxrel {e1:.3e} > {tol:.3e}"
    if not beta:
        opA = np.abs(A64.T if transA else A64)
        opB = np.abs(B64.T if transB else B64)
        e2 = elementwise_ratio(got, ref, opA, opB)
        assert e2 <= tol, f"per-element {e2:.3e} > {tol:.3e}"
    return e1


def test_c1_fp32_1024_seed42():
    # Config 1: set_seed(42); A = randn(1024,1024); B = randn(1024,1024); C = A @ B.
    O.set_seed(42)
    A, B = O.randn(1024, 1024), O.randn(1024, 1024)
    got = gemm(f32(A), f32(B))
    ref = O.gemm_d(A, B)                      # the reference's fp64 `@`
    assert maxrel(got, ref) <= 1e-5 * np.sqrt(1024)
    assert np.abs(got - ref).max() < np.sqrt(1024) * 1e-4   # gpu_selftest gate


@pytest.mark.parametrize("shape", [
    (1, 1, 1), (1, 7, 1), (5, 1, 9), (3, 4, 5), (7, 13, 17), (31, 33, 37), (64, 64, 64),
    (65, 63, 66), (128, 100, 96), (200, 50, 300), (257, 129, 255),          # gemm_selftest
    (32, 32, 32), (33, 31, 35), (256, 128, 256), (300, 200, 257), (100, 100, 100),
    (1, 64, 1), (65, 1, 63),                                                 # kernel-sim shapes
    (256, 128, 256), (300, 200, 257), (512, 64, 300),                        # gpu_selftest
])
def test_fp32_adversarial_shapes(shape):
    M, K, N = shape
    rng = np.random.default_rng(M * 1000 + K * 10 + N)
    A, B = rng.uniform(-1, 1, (M, K)), rng.uniform(-1, 1, (K, N))
    A, B = f32(A).astype(np.float64), f32(B).astype(np.float64)
    got = gemm(f32(A), f32(B))
    check_f32(got, A, B, K)
    assert np.abs(got - O.gemm_ref_d(A, B)).max() < np.sqrt(K) * 1e-4


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("beta", [0.0, 1.0, -0.5])
@pytest.mark.parametrize("ldpad", [0, 3, 4])
def test_fp32_transposes_beta_strides(ta, tb, beta, ldpad):
    M, N, K = 131, 67, 259
    rng = np.random.default_rng(17 + ta + 2 * tb + int(4 * beta) + ldpad)
    A = f32(rng.standard_normal((K, M) if ta else (M, K))).astype(np.float64)
    B = f32(rng.standard_normal((N, K) if tb else (K, N))).astype(np.float64)
    C0 = f32(rng.standard_normal((M, N))).astype(np.float64)
    got = gemm(f32(A), f32(B), bool(ta), bool(tb), beta, f32(C0), ldpad=ldpad)
    check_f32(got, A, B, K, ta, tb, beta, C0)


def test_fp32_closed_forms_and_degenerate_shapes():
    # ones(256,256) @ ones(256,256): every element is 256, sum 16777216 (gpu_diagnose).
    C = gemm(np.ones((256, 256), np.float32), np.ones((256, 256), np.float32))
    assert np.all(C == 256) and C.sum(dtype=np.float64) == 16777216
    C = gemm(np.ones((2, 3), np.float32), np.ones((3, 2), np.float32))   # tests/09: "3 3"
    assert np.all(C == 3)
    # K = 0: C = beta * C
    C0 = np.arange(12, dtype=np.float32).reshape(3, 4)
    got = gemm(np.zeros((3, 0), np.float32), np.zeros((0, 4), np.float32), beta=2.0, C0=C0)
    assert np.array_equal(got, 2 * C0)
    # beta = 0 ignores NaN already in C
    got = gemm(np.ones((5, 6), np.float32), np.ones((6, 7), np.float32), beta=0.0,
               C0=np.full((5, 7), np.nan, np.float32))
    assert np.all(got == 6)


def _mlp_tensors():
    # Config 2: X[4096x784] ~ U(0,1), W1 = kaiming_init(784, 257), W2 = kaiming_init(257, 10)
    # (Dream's kaiming_init(r, c) draws N(0, sqrt(2/c)), builtins.inc:511-519); upstream
    # gradients N(0,1); all from the reference RNG stream, seed 1234.
    O.set_seed(1234)
    X = O.uniform(4096 * 784, 0.0, 1.0).reshape(4096, 784)
    W1, W2 = O.kaiming(784, 257), O.kaiming(257, 10)
    dY = O.randn(4096, 10)
    H = np.maximum(O.gemm_d(f32(X).astype(np.float64), f32(W1).astype(np.float64)), 0.0)
    dZ1 = O.randn(4096, 257)
    return [f32(t).astype(np.float64) for t in (X, W1, W2, dY, H, dZ1)]


def test_c2_mlp_forward_backward_set():
    X, W1, W2, dY, H, dZ1 = _mlp_tensors()
    cases = [
        ("X@W1", X, W1, 0, 0, 784),
        ("H@W2", H, W2, 0, 0, 257),
        ("dW1=X^T dZ1", X, dZ1, 1, 0, 4096),
        ("dX=dZ1 W1^T", dZ1, W1, 0, 1, 257),
        ("dW2=H^T dY", H, dY, 1, 0, 4096),
        ("dH=dY W2^T", dY, W2, 0, 1, 10),
    ]
    for name, A, B, ta, tb, K in cases:
        got = gemm(f32(A), f32(B), bool(ta), bool(tb))
        check_f32(got, A, B, K, ta, tb)


def _rowcol_sums_check(got, A64, B64, tol):
    """Full-size property: row sums of C equal A @ (B 1) and column sums (1^T A) B."""
    r_ref = A64 @ B64.sum(axis=1)
    c_ref = A64.sum(axis=0) @ B64
    r = got.sum(axis=1, dtype=np.float64)
    c = got.sum(axis=0, dtype=np.float64)
    assert np.abs(r - r_ref).max() <= tol * max(np.abs(r_ref).max(), 1.0)
    assert np.abs(c - c_ref).max() <= tol * max(np.abs(c_ref).max(), 1.0)


def test_c5_fp32_4096_full_size():
    rng = np.random.default_rng(4096)
    A = rng.standard_normal((4096, 4096), dtype=np.float32)
    B = rng.standard_normal((4096, 4096), dtype=np.float32)
    got = gemm(A, B)
    A64, B64 = A.astype(np.float64), B.astype(np.float64)
    rows = np.sort(rng.choice(4096, 48, replace=False))
    ref = O.gemm_d(A64[rows], B64)
    assert maxrel(got[rows], ref) <= 1e-5 * np.sqrt(4096)
    _rowcol_sums_check(got, A64, B64, 1e-5)


@pytest.mark.parametrize("shape", [(1024, 1024, 1024), (257, 129, 255), (65, 63, 66),
                                   (300, 200, 257), (1, 64, 1), (520, 8192, 264)])
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0)])
def test_bf16_parity(shape, ta, tb):
    M, K, N = shape
    rng = np.random.default_rng(M + K + N + 7 * ta + 13 * tb)
    A = rng.standard_normal((K, M) if ta else (M, K), dtype=np.float32)
    B = rng.standard_normal((N, K) if tb else (K, N), dtype=np.float32)
    Ab, Bb = bf16_bits(A), bf16_bits(B)
    got = gemm(Ab, Bb, bool(ta), bool(tb), dtype="bf16")
    ref = O.gemm_general_d(ta, tb, bits_to_f32(Ab).astype(np.float64),
                           bits_to_f32(Bb).astype(np.float64))
    assert maxrel(got, ref) <= 2e-2
    # fp32 accumulation of exact bf16 products is far tighter than the contract:
    assert maxrel(got, ref) <= 1e-5 * np.sqrt(K)


def test_bf16_beta_and_padding():
    M, N, K = 200, 136, 264
    rng = np.random.default_rng(99)
    A, B = rng.standard_normal((M, K), dtype=np.float32), rng.standard_normal((K, N), dtype=np.float32)
    C0 = rng.standard_normal((M, N), dtype=np.float32)
    for ldpad in (0, 3, 8):
        Ab, Bb = bf16_bits(A), bf16_bits(B)
        got = gemm(Ab, Bb, beta=1.0, C0=C0, dtype="bf16", ldpad=ldpad)
        ref = O.gemm_general_d(0, 0, bits_to_f32(Ab).astype(np.float64),
                               bits_to_f32(Bb).astype(np.float64), 1.0, C0.astype(np.float64))
        assert maxrel(got, ref) <= 1e-5 * np.sqrt(K)


def test_c5_bf16_8192_full_size():
    # Config 5: A, B 8192^2 ~ N(0,1) rounded to bf16 (RNE), fp32 accumulate and output.
    rng = np.random.default_rng(8192)
    Ab = bf16_bits(rng.standard_normal((8192, 8192), dtype=np.float32))
    Bb = bf16_bits(rng.standard_normal((8192, 8192), dtype=np.float32))
    got = gemm(Ab, Bb, dtype="bf16")
    A64 = bits_to_f32(Ab).astype(np.float64)
    B64 = bits_to_f32(Bb).astype(np.float64)
    rows = np.sort(rng.choice(8192, 24, replace=False))
    ref = O.gemm_d(A64[rows], B64)
    assert maxrel(got[rows], ref) <= 2e-2
    assert maxrel(got[rows], ref) <= 1e-5 * np.sqrt(8192)
    _rowcol_sums_check(got, A64, B64, 1e-5)


# 1..10 stages of 32 k.  Default forms: 8 waves, NN and NT with a k-contiguous A in double
# stages of 64 k (so odd stage counts, 1, 3, 5, end on half a pair), TN and TT in 32-k stages.
# The other forms, reachable through DH_GEMM_BF16_WAVES / DH_GEMM_BF16_DEEP8, are covered by
# test_bf16_fast_path_knob_variants.
@pytest.mark.parametrize("K", [32, 64, 96, 160, 256, 320])
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_bf16_tile_aligned_fast_path(K, ta, tb):
    # M = N = 4096 gives 256 tiles of 256 x 256, the direct-to-LDS path.
    M = N = 4096
    rng = np.random.default_rng(K + 10 * ta + 20 * tb)
    A = bf16_bits(rng.standard_normal((K, M) if ta else (M, K), dtype=np.float32))
    B = bf16_bits(rng.standard_normal((N, K) if tb else (K, N), dtype=np.float32))
    C0 = rng.standard_normal((M, N), dtype=np.float32)
    got = gemm(A, B, bool(ta), bool(tb), beta=0.5, C0=C0, dtype="bf16")
    A64, B64 = bits_to_f32(A).astype(np.float64), bits_to_f32(B).astype(np.float64)
    opA = A64.T if ta else A64
    opB = B64.T if tb else B64
    rows = np.sort(rng.choice(M, 64, replace=False))
    ref = opA[rows] @ opB + 0.5 * C0[rows].astype(np.float64)
    assert maxrel(got[rows], ref) <= 1e-5 * np.sqrt(K)
    _rowcol_sums_check(got - 0.5 * C0, A64.T if ta else A64, B64.T if tb else B64, 1e-5)


@pytest.mark.parametrize("ldcpad", [1, 2, 4])
@pytest.mark.parametrize("beta", [0.0, -0.5])
def test_bf16_fast_path_c_strides(ldcpad, beta):
    # Fast-path operands (lda, ldb multiples of 8) with C rows that are not 16-byte
    # aligned (ldc = N + 1, N + 2) take the per-element store form; ldc = N + 4 the
    # 16-byte form at a padded stride.
    M = N = 4096
    K = 64
    rng = np.random.default_rng(ldcpad + 100 * (beta != 0))
    A = bf16_bits(rng.standard_normal((M, K), dtype=np.float32))
    B = bf16_bits(rng.standard_normal((K, N), dtype=np.float32))
    C0 = rng.standard_normal((M, N), dtype=np.float32)
    got = gemm(A, B, beta=beta, C0=C0, dtype="bf16", ldpad=8, ldcpad=ldcpad)
    A64, B64 = bits_to_f32(A).astype(np.float64), bits_to_f32(B).astype(np.float64)
    rows = np.sort(rng.choice(M, 64, replace=False))
    ref = A64[rows] @ B64 + beta * C0[rows].astype(np.float64)
    assert maxrel(got[rows], ref) <= 1e-5 * np.sqrt(K)


_VARIANT_SCRIPT = r"""
import sys, numpy as np
sys.path[:0] = [{tests!r}, {root!r}]
from _gpu import bf16_bits, bits_to_f32, gemm, maxrel
for K in (32, 96, 160, 320):
    for ta, tb in [(0, 0), (0, 1), (1, 0), (1, 1)]:
        M = N = 4096
        rng = np.random.default_rng(7 + K + 10 * ta + 20 * tb)
        A = bf16_bits(rng.standard_normal((K, M) if ta else (M, K), dtype=np.float32))
        B = bf16_bits(rng.standard_normal((N, K) if tb else (K, N), dtype=np.float32))
        got = gemm(A, B, bool(ta), bool(tb), dtype="bf16")
        A64, B64 = bits_to_f32(A).astype(np.float64), bits_to_f32(B).astype(np.float64)
        opA, opB = (A64.T if ta else A64), (B64.T if tb else B64)
        rows = np.sort(rng.choice(M, 64, replace=False))
        e = maxrel(got[rows], opA[rows] @ opB)
        # every column, through its sum: (1^T C) = (1^T opA) opB
        c_ref = opA.sum(axis=0) @ opB
        cs = np.abs(got.sum(axis=0, dtype=np.float64) - c_ref).max() / np.abs(c_ref).max()
        print("variant", K, ta, tb, e, cs, flush=True)
        assert e <= 1e-5 * np.sqrt(K), e
        assert cs <= 1e-5, cs
"""


# The fast path's form is chosen once per process from the environment, so each runs in a
# child process of its own: 8 waves set explicitly (the default), 4 waves for all four layouts
# (NN and NT with 64-k A stages), and 8 waves with 32-k A stages for NN and NT
# (DH_GEMM_BF16_DEEP8=0), each over odd and even stage counts.
@pytest.mark.parametrize("env", [{"DH_GEMM_BF16_WAVES": "8"}, {"DH_GEMM_BF16_WAVES": "4"},
                                 {"DH_GEMM_BF16_DEEP8": "0"}],
                         ids=["waves8", "waves4", "deep8_off"])
def test_bf16_fast_path_knob_variants(env):
    import os
    import subprocess
    import sys
    here = os.path.dirname(os.path.abspath(__file__))
    code = _VARIANT_SCRIPT.format(tests=here, root=os.path.dirname(here))
    r = subprocess.run([sys.executable, "-c", code], env={**os.environ, **env},
                       capture_output=True, text=True, timeout=110)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.count("variant") == 16, r.stdout

_OCC4_SCRIPT = r"""
import hashlib, sys
sys.path[:0] = [{tests!r}, {root!r}]
from test_gemm_gpu import _ex
for ta, tb in [(0, 0), (0, 1), (1, 0), (1, 1)]:
    got, _ = _ex("f32", ta, tb, 1, 4096, 4096, 520, beta=0.5, bias=True, relu=True, seed=ta + 2 * tb)
    print("single", ta, tb, hashlib.sha1(got.tobytes()).hexdigest()[:16], flush=True)
got, _ = _ex("f32", 0, 0, 40, 512, 640, 300, beta=0.0, bias=True, seed=7)
print("batched", hashlib.sha1(got.tobytes()).hexdigest()[:16], flush=True)
"""


def test_fp32_four_wave_form_is_bit_identical():
    """One-pass fp32 grids of at least four 128 x 128 tiles per CU take the four-wave form of
    the tile kernel (same tile body, held to 128 registers so that four work-groups share a
    CU).  Every layout at 4096 x 4096 (1024 tiles) with beta, bias and ReLU, and a batched grid
    (40 x 20 tiles), against the default form (DH_GEMM_F32_OCC4=0), bit for bit: the
    arithmetic and its order are the same.  The switch is read once per process, so each form
    runs in a child process."""
    import os
    import subprocess
    import sys
    here = os.path.dirname(os.path.abspath(__file__))
    code = _OCC4_SCRIPT.format(tests=here, root=os.path.dirname(here))

    def run(env):
        r = subprocess.run([sys.executable, "-c", code], env={**os.environ, **env},
                           capture_output=True, text=True, timeout=110)
        assert r.returncode == 0, r.stdout + r.stderr
        lines = [l for l in r.stdout.split("\n") if l.strip()]
        assert len(lines) == 5, r.stdout
        return lines

    assert run({}) == run({"DH_GEMM_F32_OCC4": "0"})


def _ex(dtype, ta, tb, Bt, M, N, K, beta=0.0, bias=True, relu=False, share=None, seed=0,
        row_bias=False):
    """Run dh_gemm_*_ex on random inputs; returns (got, ref) as (Bt, M, N) arrays."""
    rng = np.random.default_rng(seed)
    shA = (K, M) if ta else (M, K)
    shB = (N, K) if tb else (K, N)
    A = rng.standard_normal((1 if share == "A" else Bt,) + shA).astype(np.float32)
    B = rng.standard_normal((1 if share == "B" else Bt,) + shB).astype(np.float32)
    C0 = rng.standard_normal((Bt, M, N)).astype(np.float32)
    b = rng.standard_normal(M if row_bias else N).astype(np.float32) if bias else None
    if dtype == "bf16":
        A, B = bf16_bits(A), bf16_bits(B)
        A64, B64 = bits_to_f32(A).astype(np.float64), bits_to_f32(B).astype(np.float64)
    else:
        A64, B64 = A.astype(np.float64), B.astype(np.float64)
    opA = np.swapaxes(A64, 1, 2) if ta else A64
    opB = np.swapaxes(B64, 1, 2) if tb else B64
    ref = np.matmul(opA, opB) + beta * C0.astype(np.float64)
    if bias:
        ref = ref + (b.astype(np.float64)[:, None] if row_bias else b.astype(np.float64))
    if relu:
        ref = np.maximum(ref, 0.0)
    DB = hip.DeviceBuffer
    dA, dB, dC = DB.from_numpy(A), DB.from_numpy(B), DB.from_numpy(C0)
    dbias = DB.from_numpy(b) if bias else None
    sA = 0 if share == "A" else shA[0] * shA[1]
    sB = 0 if share == "B" else shB[0] * shB[1]
    hip.gemm_ex(dtype, ta, tb, M, N, K, dA, shA[1], sA, dB, shB[1], sB, beta, dC, N, M * N, Bt,
                dbias, relu, row_bias)
    got = dC.numpy()
    for x in (dA, dB, dC, dbias):
        if x is not None:
            x.free()
    return got, ref



@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("relu", [False, True])
def test_gemm_ex_batched_bias_relu(dtype, ta, tb, relu):
    Bt, M, N, K = 3, 70, 50, 33
    got, ref = _ex(dtype, ta, tb, Bt, M, N, K, beta=0.5, relu=relu, seed=ta + 2 * tb + 4 * relu)
    tol = (1e-5 * np.sqrt(K)) if dtype == "f32" else 2e-2
    assert maxrel(got, ref) <= tol


@pytest.mark.parametrize("share", ["A", "B"])
def test_gemm_ex_shared_operand(share):
    got, ref = _ex("f32", 0, 0, 4, 40, 36, 20, share=share, seed=7)
    assert maxrel(got, ref) <= 1e-5 * np.sqrt(20)


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1)])
@pytest.mark.parametrize("relu", [False, True])
def test_gemm_ex_bf16_fast_path_batched(ta, tb, relu):
    # 16 members of 1024 x 1024 = 256 tiles of 256 x 256: the direct-to-LDS fast path with
    # gridDim.y batches, the bias / ReLU epilogue form.
    Bt, M, N, K = 16, 1024, 1024, 64
    got, ref = _ex("bf16", ta, tb, Bt, M, N, K, relu=relu, seed=40 + ta + 2 * relu)
    assert maxrel(got, ref) <= 1e-5 * np.sqrt(K)      # exact bf16 products, fp32 sums


def test_gemm_ex_rejects_overlapping_batches():
    DB = hip.DeviceBuffer
    a, b, c = DB(4 * 64), DB(4 * 64), DB(4 * 64)
    with pytest.raises(hip.DreamHipError):
        hip.gemm_ex("f32", 0, 0, 4, 4, 4, a, 4, 16, b, 4, 16, 0.0, c, 4, 8, 2)
    with pytest.raises(hip.DreamHipError):
        hip.gemm_ex("bf16", 0, 0, 4, 4, 4, a, 4, -16, b, 4, 16, 0.0, c, 4, 16, 2)


def test_linear_reference_golden_vectors():
    # Y = X W^T + b (NT with the bias epilogue), and with ReLU, against the reference build's
    # own dream_linear / dream_linear_relu outputs.
    import os
    G = np.load(os.path.join(os.path.dirname(__file__), "golden", "ref_vectors.npz"))
    X, W, b = (G["linear_" + c].astype(np.float32) for c in "XWb")
    N_, K_ = X.shape
    O_ = W.shape[0]
    DB = hip.DeviceBuffer
    for relu, key in ((False, "linear_Y"), (True, "linear_relu_Y")):
        dX, dW, db, dY = DB.from_numpy(X), DB.from_numpy(W), DB.from_numpy(b.ravel()), \
            DB.empty((N_, O_), np.float32)
        hip.gemm_ex("f32", 0, 1, N_, O_, K_, dX, K_, 0, dW, K_, 0, 0.0, dY, O_, 0, 1, db, relu)
        assert maxrel(dY.numpy(), G[key]) <= 1e-5 * np.sqrt(K_)


@pytest.mark.parametrize("M,N,K", [(40, 33, 5000), (300, 200, 2048), (784, 257, 4096), (257, 10, 4096)])
@pytest.mark.parametrize("ta,tb", [(0, 0), (1, 0), (0, 1), (1, 1)])
def test_fp32_split_k_skinny_long_k(M, N, K, ta, tb):
    # Few output tiles and a long contraction take the split-K path (K chunks as gridDim.y
    # members, a ragged last chunk of its own, an ordered reduction with beta / bias / ReLU).
    got, ref = _ex("f32", ta, tb, 1, M, N, K, beta=0.5, relu=bool(ta), seed=M + K + ta)
    assert maxrel(got, ref) <= 1e-5 * np.sqrt(K)


def test_fp32_split_k_bit_identical_reruns():
    a, _ = _ex("f32", 1, 0, 1, 784, 257, 4096, seed=3)
    b, _ = _ex("f32", 1, 0, 1, 784, 257, 4096, seed=3)
    assert np.array_equal(a, b)


@pytest.mark.parametrize("Bt,M,N,K", [(3, 40, 300, 70), (2, 300, 50, 129), (1, 64, 4096, 576),
                                      (1, 4096, 10, 784), (4, 1, 513, 33), (1, 64, 40000, 40),
                                      (1, 40000, 48, 40)])
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("row_bias", [False, True])
def test_fp32_narrow_tiles(Bt, M, N, K, ta, tb, row_bias):
    # M <= 64 takes 64 x 256 work-group tiles, N <= 64 256 x 64 -- or 64 x 64 when those grids
    # are small (the first five shapes); the last two keep the wide tiles.  Batched, split-K
    # and the epilogue with either bias orientation go through the same shapes.
    got, ref = _ex("f32", ta, tb, Bt, M, N, K, beta=0.25, relu=row_bias, row_bias=row_bias,
                   seed=M + N + K + ta + 2 * tb)
    assert maxrel(got, ref) <= 1e-5 * np.sqrt(K)


@pytest.mark.parametrize("Bt,M,N,K", [(1, 1024, 1024, 1024), (1, 1000, 777, 100), (2, 520, 700, 33),
                                      (1, 4096, 257, 784), (1, 700, 900, 7), (1, 784, 257, 4096),
                                      (1, 300, 200, 2048)])
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_fp32_64x64_tiles(Bt, M, N, K, ta, tb):
    # Products whose 128 x 128 grid is under one tile per CU run on 64 x 64 tiles (one 32 x 32
    # MFMA block per wave): config 1, ragged edges, batched, config 2's first layer, a single
    # k-slice (K = 7), and split-K grids whose 128-wide tiles would be mostly padding (config
    # 2's dW1, 784 x 257 with K = 4096; 300 x 200); beta and a per-column bias with ReLU
    # through the epilogue (the split-K reduce applies it).
    got, ref = _ex("f32", ta, tb, Bt, M, N, K, beta=0.5, relu=True, seed=M + N + K + ta + 2 * tb)
    assert maxrel(got, ref) <= 1e-5 * np.sqrt(K)


@pytest.mark.parametrize("Bt,M,N,K", [(1, 1000, 1000, 300), (1, 999, 1001, 257), (2, 512, 900, 512),
                                      (1, 1024, 960, 1000), (1, 1000, 1000, 256), (1, 960, 1000, 1300)])
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("row_bias", [False, True])
def test_fp32_64x64_two_waves_per_simd(Bt, M, N, K, ta, tb, row_bias):
    # At most one 64 x 64 tile per CU (256 on MI355X) and K >= 256: the 8-wave kernel, two
    # waves per 32 x 32 block splitting each 32-wide k-slice and reducing through LDS.
    # Ragged M / N, K not a multiple of 32 (300, 1000) or of 4 (257: scalar loads), batched,
    # all layouts, beta and either bias orientation with ReLU.  K = 256, 512, 1000 and 1300
    # (8, 16, 32 and 41 slices) keep four slices in flight, 1300 with three zero slices in its
    # last group of four; the others two.
    got, ref = _ex("f32", ta, tb, Bt, M, N, K, beta=0.5, relu=True, row_bias=row_bias,
                   seed=M + N + K + ta + 2 * tb + row_bias)
    assert maxrel(got, ref) <= 1e-5 * np.sqrt(K)


# A 128 x 128 grid a few tiles past whole rounds of the CUs: the output is cut into whole
# rounds and a tail strip of tile rows (or columns, the 2000 x 4200 case) whose K is split into
# chunks with an ordered reduction.  Ragged strips (4100: 132 rows; 4200: 104 columns), K not a
# multiple of 4 (scalar loads), all layouts, beta and either bias orientation with ReLU.
SPLIT_TAIL_F32 = [(3000, 3000, 1024), (2000, 4200, 1100), (4100, 4100, 1027)]


@pytest.mark.parametrize("M,N,K", SPLIT_TAIL_F32)
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("row_bias", [False, True])
def test_fp32_split_tail(M, N, K, ta, tb, row_bias):
    got, ref = _ex("f32", ta, tb, 1, M, N, K, beta=0.5, relu=row_bias, row_bias=row_bias,
                   seed=M + N + K + ta + 2 * tb + row_bias)
    assert maxrel(got, ref) <= 1e-5 * np.sqrt(K)


def test_fp32_split_tail_bit_identical_reruns():
    a, _ = _ex("f32", 0, 0, 1, 3000, 3000, 1024, seed=5)
    b, _ = _ex("f32", 0, 0, 1, 3000, 3000, 1024, seed=5)
    assert np.array_equal(a, b)


# Skinny products (a side <= 16): config 2's H W2 (4096 x 10, K 257), dW2 = H^T dY (257 x 10,
# K 4096, split over work-groups) and dH = dY W2^T (4096 x 257, K 10); M <= 16 (operands
# swapped, C written transposed); tails of every side; K = 0.
SKINNY = [(4096, 10, 257), (257, 10, 4096), (4096, 257, 10), (10, 4096, 257), (16, 16, 16),
          (1, 1, 1), (17, 5, 3), (5, 1000, 3000), (3000, 7, 64), (33, 2, 65), (2, 33, 1000),
          (300, 16, 17), (1, 513, 33)]


@pytest.mark.parametrize("M,N,K", SKINNY)
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_fp32_skinny_products(M, N, K, ta, tb):
    got, ref = _ex("f32", ta, tb, 1, M, N, K, beta=0.0, seed=M + 3 * N + 7 * K + ta + 2 * tb)
    assert maxrel(got, ref) <= 1e-5 * np.sqrt(K)
    rng = np.random.default_rng(M + N + K)
    A = rng.standard_normal((K, M) if ta else (M, K))
    B = rng.standard_normal((N, K) if tb else (K, N))
    check_f32(gemm(f32(A), f32(B), bool(ta), bool(tb)), A.astype(np.float32).astype(np.float64),
              B.astype(np.float32).astype(np.float64), K, bool(ta), bool(tb))


@pytest.mark.parametrize("M,N,K", [(4096, 10, 257), (257, 10, 4096), (4096, 257, 10),
                                   (10, 300, 700), (7, 9, 2000)])
@pytest.mark.parametrize("relu,row_bias", [(False, False), (True, False), (True, True)])
def test_fp32_skinny_epilogue(M, N, K, relu, row_bias):
    got, ref = _ex("f32", 0, 0, 1, M, N, K, beta=-0.5, relu=relu, row_bias=row_bias,
                   seed=M + N + K + relu)
    assert maxrel(got, ref) <= 1e-5 * np.sqrt(K)


def test_fp32_skinny_k_zero_and_reruns():
    C0 = np.arange(30, dtype=np.float32).reshape(10, 3)
    got = gemm(np.zeros((10, 0), np.float32), np.zeros((0, 3), np.float32), beta=0.5, C0=C0)
    assert np.array_equal(got, 0.5 * C0)
    a, _ = _ex("f32", 1, 0, 1, 257, 10, 4096, seed=5)
    b, _ = _ex("f32", 1, 0, 1, 257, 10, 4096, seed=5)
    assert np.array_equal(a, b)


def test_fp32_skinny_split_k_many_launches():
    # K split over work-groups with pooled partials added in a fixed order: 150 launches
    # alternating two shapes with different block counts (the pool hands the partial buffers
    # back and forth); every result must equal the first one bit for bit and the oracle
    # within the fp32 bound.
    rng = np.random.default_rng(77)
    shapes = [(1, 0, 257, 10, 4096), (0, 1, 7, 600, 3000)]
    DB = hip.DeviceBuffer
    runs = []
    for ta, tb, M, N, K in shapes:
        A = rng.standard_normal((K, M) if ta else (M, K)).astype(np.float32)
        B = rng.standard_normal((N, K) if tb else (K, N)).astype(np.float32)
        ref = O.gemm_general_d(ta, tb, A.astype(np.float64), B.astype(np.float64))
        runs.append((ta, tb, M, N, K, DB.from_numpy(A), DB.from_numpy(B), DB.empty((M, N), np.float32),
                     A.shape[1], B.shape[1], ref))
    first = [None, None]
    for it in range(150):
        x = it % 2
        ta, tb, M, N, K, dA, dB, dC, lda, ldb, ref = runs[x]
        hip.gemm_f32(ta, tb, M, N, K, dA, lda, dB, ldb, 0.0, dC, N)
        got = dC.numpy()
        if first[x] is None:
            first[x] = got
            assert maxrel(got, ref) <= 1e-5 * np.sqrt(K)
        else:
            assert np.array_equal(got, first[x]), f"launch {it}"


# Ragged shapes on the direct-to-LDS bf16 path (at least one round of 256 x 256 tiles): edge
# tiles for M, N; the last K % 32 on the general kernel; unaligned leading dimensions copied to
# aligned rows first.
RAGGED = [(4000, 4000, 256), (4000, 4000, 300), (4095, 4097, 100), (3900, 4352, 33),
          (4352, 3841, 1000)]


@pytest.mark.parametrize("M,N,K", RAGGED)
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_bf16_ragged_fast_path(M, N, K, ta, tb):
    rng = np.random.default_rng(M + 3 * N + 7 * K + 11 * ta + 13 * tb)
    A = bf16_bits(rng.standard_normal((K, M) if ta else (M, K), dtype=np.float32))
    B = bf16_bits(rng.standard_normal((N, K) if tb else (K, N), dtype=np.float32))
    C0 = rng.standard_normal((M, N), dtype=np.float32)
    got = gemm(A, B, bool(ta), bool(tb), beta=-0.5, C0=C0, dtype="bf16")
    A64, B64 = bits_to_f32(A).astype(np.float64), bits_to_f32(B).astype(np.float64)
    opA, opB = (A64.T if ta else A64), (B64.T if tb else B64)
    rows = np.sort(np.concatenate([rng.choice(M, 40, replace=False), [0, M - 1]]))
    ref = opA[rows] @ opB - 0.5 * C0[rows].astype(np.float64)
    assert maxrel(got[rows], ref) <= 1e-5 * np.sqrt(K)
    # every element, through the row and column sums (the edge tiles included)
    _rowcol_sums_check(got + 0.5 * C0, opA, opB, 1e-5)


@pytest.mark.parametrize("ldpad", [1, 3, 4])
@pytest.mark.parametrize("ta,tb", [(0, 0), (1, 1)])
def test_bf16_unaligned_rows_take_aligned_copies(ldpad, ta, tb):
    # leading dimensions that are not multiples of 8 elements (rows not 16-byte aligned)
    M, N, K = 4100, 4000, 264
    rng = np.random.default_rng(ldpad + 5 * ta)
    A = bf16_bits(rng.standard_normal((K, M) if ta else (M, K), dtype=np.float32))
    B = bf16_bits(rng.standard_normal((N, K) if tb else (K, N), dtype=np.float32))
    got = gemm(A, B, bool(ta), bool(tb), dtype="bf16", ldpad=ldpad, ldcpad=0)
    A64, B64 = bits_to_f32(A).astype(np.float64), bits_to_f32(B).astype(np.float64)
    opA, opB = (A64.T if ta else A64), (B64.T if tb else B64)
    rows = np.sort(rng.choice(M, 40, replace=False))
    assert maxrel(got[rows], opA[rows] @ opB) <= 1e-5 * np.sqrt(K)
    _rowcol_sums_check(got, opA, opB, 1e-5)


@pytest.mark.parametrize("relu", [False, True])
def test_bf16_ragged_epilogue_bias_relu(relu):
    # column bias and ReLU on ragged edge tiles, and applied once when K has a tail
    for M, N, K in ((4000, 4000, 300), (4095, 4097, 256)):
        got, ref = _ex("bf16", 0, 1, 1, M, N, K, beta=0.25, bias=True, relu=relu, seed=M + K)
        assert maxrel(got, ref) <= 1e-5 * np.sqrt(K)


def test_bf16_ragged_k_tail_keeps_nonfinite_values_in_their_row():
    # A NaN in the last column of A row i and an Inf in row i+1: only C rows i and i+1 may be
    # non-finite (the k-tail of row i must not read row i+1's values, nor the reverse).
    M, N, K = 4000, 4000, 300
    rng = np.random.default_rng(5)
    Af = rng.standard_normal((M, K), dtype=np.float32)
    Af[1000, K - 1] = np.nan
    Af[1001, 0] = np.inf
    A = bf16_bits(Af)
    B = bf16_bits(rng.standard_normal((K, N), dtype=np.float32))
    got = gemm(A, B, dtype="bf16")
    bad = np.where(~np.isfinite(got).all(axis=1))[0]
    assert set(bad.tolist()) == {1000, 1001}
    ok = np.isfinite(got).all(axis=1)
    A64, B64 = bits_to_f32(A).astype(np.float64), bits_to_f32(B).astype(np.float64)
    rows = np.where(ok)[0][::97]
    assert maxrel(got[rows], A64[rows] @ B64) <= 1e-5 * np.sqrt(K)


# The 128 x 128 direct-to-LDS path: shapes whose 256 x 256 tiles do not make one round of
# the CUs.  1..5 stages of 32 k (ring fill and drain), K tails, ragged edge tiles, a grid
# of more than two tiles per CU (3000^2), one-tile and one-row products, and split K (at most
# half the CUs' worth of tiles and K >= 2048: 784 x 257 x 4096, 512^2 x 8192, 300 x 200 x 2048,
# 1000 x 700 x 2100, chunks whose last one takes the rest of K); every element against fp64
# on the bf16-rounded inputs.
MID = [(2048, 2048, 2048), (128, 128, 32), (256, 384, 64), (129, 255, 96), (300, 200, 128),
       (1000, 1900, 160), (2000, 1900, 1000), (3000, 3000, 500), (1, 64, 64), (70, 1, 33),
       (4096, 10, 257), (784, 257, 4096), (512, 512, 8192), (300, 200, 2048), (1000, 700, 2100)]


@pytest.mark.parametrize("M,N,K", MID)
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_bf16_mid_path(M, N, K, ta, tb):
    rng = np.random.default_rng(M + 5 * N + 9 * K + 11 * ta + 13 * tb)
    A = bf16_bits(rng.standard_normal((K, M) if ta else (M, K), dtype=np.float32))
    B = bf16_bits(rng.standard_normal((N, K) if tb else (K, N), dtype=np.float32))
    C0 = rng.standard_normal((M, N), dtype=np.float32)
    got = gemm(A, B, bool(ta), bool(tb), beta=0.75, C0=C0, dtype="bf16")
    A64, B64 = bits_to_f32(A).astype(np.float64), bits_to_f32(B).astype(np.float64)
    opA, opB = (A64.T if ta else A64), (B64.T if tb else B64)
    ref = opA @ opB + 0.75 * C0.astype(np.float64)
    assert maxrel(got, ref) <= 1e-5 * np.sqrt(K)


@pytest.mark.parametrize("Bt,M,N,K", [(3, 500, 300, 200), (2, 1024, 1024, 97), (1, 256, 384, 4099)])
@pytest.mark.parametrize("ta,tb", [(0, 0), (1, 1)])
@pytest.mark.parametrize("relu,row_bias", [(False, False), (True, False), (True, True)])
def test_bf16_mid_path_batched_epilogue(Bt, M, N, K, ta, tb, relu, row_bias):
    got, ref = _ex("bf16", ta, tb, Bt, M, N, K, beta=-0.5, bias=True, relu=relu,
                   seed=Bt + M + K, row_bias=row_bias)
    assert maxrel(got, ref) <= 1e-5 * np.sqrt(K)


def test_bf16_mid_path_k_tail_keeps_nonfinite_values_in_their_row():
    M, N, K = 1000, 900, 300
    rng = np.random.default_rng(6)
    Af = rng.standard_normal((M, K), dtype=np.float32)
    Af[500, K - 1] = np.nan
    Af[501, 0] = np.inf
    A = bf16_bits(Af)
    B = bf16_bits(rng.standard_normal((K, N), dtype=np.float32))
    got = gemm(A, B, dtype="bf16")
    bad = np.where(~np.isfinite(got).all(axis=1))[0]
    assert set(bad.tolist()) == {500, 501}
    ok = np.isfinite(got).all(axis=1)
    A64, B64 = bits_to_f32(A).astype(np.float64), bits_to_f32(B).astype(np.float64)
    assert maxrel(got[ok], A64[ok] @ B64) <= 1e-5 * np.sqrt(K)


# Between half a round and a round of 256 x 256 tiles the fast kernel runs a partial round
# (144, 224 and 225 tiles here), at the boundary (128 tiles) the 128 x 128 path.
@pytest.mark.parametrize("M,N,K", [(3000, 3000, 300), (3500, 4000, 96), (3840, 3840, 33),
                                   (2048, 4096, 160)])
@pytest.mark.parametrize("ta,tb", [(0, 0), (1, 1)])
def test_bf16_partial_round_of_256_tiles(M, N, K, ta, tb):
    rng = np.random.default_rng(M + N + K + ta)
    A = bf16_bits(rng.standard_normal((K, M) if ta else (M, K), dtype=np.float32))
    B = bf16_bits(rng.standard_normal((N, K) if tb else (K, N), dtype=np.float32))
    C0 = rng.standard_normal((M, N), dtype=np.float32)
    got = gemm(A, B, bool(ta), bool(tb), beta=0.5, C0=C0, dtype="bf16")
    A64, B64 = bits_to_f32(A).astype(np.float64), bits_to_f32(B).astype(np.float64)
    opA, opB = (A64.T if ta else A64), (B64.T if tb else B64)
    rows = np.sort(np.concatenate([rng.choice(M, 40, replace=False), [0, M - 1]]))
    assert maxrel(got[rows], opA[rows] @ opB + 0.5 * C0[rows].astype(np.float64)) <= 1e-5 * np.sqrt(K)
    _rowcol_sums_check(got - 0.5 * C0, opA, opB, 1e-5)


# More than a round of 256 x 256 tiles with a last round of at most half the CUs and K >= 4096:
# the full rounds, then the tail tiles split into K chunks (last chunk with the rest, K % 32
# tails included) reduced in order with the epilogue.  Every element through the row and column
# sums.
SPLIT_TAIL = [(4352, 4352, 4352), (4300, 4400, 4100), (4608, 4096, 4096)]


@pytest.mark.parametrize("M,N,K", SPLIT_TAIL)
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_bf16_split_tail_round(M, N, K, ta, tb):
    rng = np.random.default_rng(M + 3 * N + K + 5 * ta + 7 * tb)
    A = bf16_bits(rng.standard_normal((K, M) if ta else (M, K), dtype=np.float32))
    B = bf16_bits(rng.standard_normal((N, K) if tb else (K, N), dtype=np.float32))
    C0 = rng.standard_normal((M, N), dtype=np.float32)
    got = gemm(A, B, bool(ta), bool(tb), beta=-0.25, C0=C0, dtype="bf16")
    A64, B64 = bits_to_f32(A).astype(np.float64), bits_to_f32(B).astype(np.float64)
    opA, opB = (A64.T if ta else A64), (B64.T if tb else B64)
    rows = np.sort(np.concatenate([rng.choice(M, 48, replace=False), [0, M - 1]]))
    ref = opA[rows] @ opB - 0.25 * C0[rows].astype(np.float64)
    assert maxrel(got[rows], ref) <= 1e-5 * np.sqrt(K)
    _rowcol_sums_check(got + 0.25 * C0, opA, opB, 1e-5)


@pytest.mark.parametrize("relu,row_bias", [(False, False), (True, False), (True, True)])
def test_bf16_split_tail_epilogue_and_reruns(relu, row_bias):
    got, ref = _ex("bf16", 0, 1, 1, 4300, 4400, 4100, beta=0.5, bias=True, relu=relu,
                   seed=11, row_bias=row_bias)
    assert maxrel(got, ref) <= 1e-5 * np.sqrt(4100)
    again, _ = _ex("bf16", 0, 1, 1, 4300, 4400, 4100, beta=0.5, bias=True, relu=relu,
                   seed=11, row_bias=row_bias)
    assert np.array_equal(got, again)


def test_bf16_mid_split_k_is_deterministic():
    # the partials are added in a fixed order: reruns are bit-identical
    rng = np.random.default_rng(17)
    A = bf16_bits(rng.standard_normal((600, 5000), dtype=np.float32))
    B = bf16_bits(rng.standard_normal((5000, 500), dtype=np.float32))
    first = gemm(A, B, dtype="bf16")
    for _ in range(3):
        assert np.array_equal(gemm(A, B, dtype="bf16"), first)


_MID_OFF_SCRIPT = r"""
import sys, numpy as np
sys.path[:0] = [{tests!r}, {root!r}]
from _gpu import bf16_bits, bits_to_f32, gemm, maxrel
for M, N, K in [(2048, 2048, 2048), (129, 255, 96), (1000, 1900, 160)]:
    for ta, tb in [(0, 0), (0, 1), (1, 0), (1, 1)]:
        rng = np.random.default_rng(M + N + K + ta + 2 * tb)
        A = bf16_bits(rng.standard_normal((K, M) if ta else (M, K), dtype=np.float32))
        B = bf16_bits(rng.standard_normal((N, K) if tb else (K, N), dtype=np.float32))
        got = gemm(A, B, bool(ta), bool(tb), dtype="bf16")
        A64, B64 = bits_to_f32(A).astype(np.float64), bits_to_f32(B).astype(np.float64)
        e = maxrel(got, (A64.T if ta else A64) @ (B64.T if tb else B64))
        print("general", M, N, K, ta, tb, e, flush=True)
        assert e <= 1e-5 * np.sqrt(K), e
"""


def test_bf16_mid_shapes_on_the_general_kernel():
    # DH_GEMM_BF16_MID=0 (read once per process): the same shapes on the register-staged
    # general kernel, which still serves K < 32 and operands past 4 GB.
    import os
    import subprocess
    import sys
    here = os.path.dirname(os.path.abspath(__file__))
    code = _MID_OFF_SCRIPT.format(tests=here, root=os.path.dirname(here))
    r = subprocess.run([sys.executable, "-c", code], env={**os.environ, "DH_GEMM_BF16_MID": "0"},
                       capture_output=True, text=True, timeout=110)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.count("general") == 12, r.stdout
