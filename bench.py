#!/usr/bin/env python3
"""Benchmark of the Dream dense-tensor hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME] [--no-cpu]

A "step" is one launch of the hot-path kernel over one batch of synthetic input that is
already resident in HBM.  The headline workload (`value`) is config 5 of the contract:
bf16 GEMM C = A @ B, M = N = K = 8192, A, B ~ N(0,1) rounded to bf16, fp32 accumulate and
output.  The same run also times fp32 GEMM 4096^3 (the fp32 MFMA figure of config 5), the
causal FlashAttention forward and backward of config 4 (B8 H16 S4096 D128 bf16), config 3
(fp32 causal flash B4 H6 S256 D64), the config 2 MLP GEMM set and the fp64 paths (`@` below
the dispatch threshold, attention with dk = 256); they are reported under "metrics".
Prints two JSON lines: {"bench_detail": ...} with every figure, then the result line (the
contract's keys, the north-star figures, parity verdicts; a few KB).  With --only, just the
result line.

Timing: HIP events recorded on the library stream (the stream every kernel here is
launched on) around K back-to-back launches, after W warm-up launches, with a stream
synchronisation on both sides.  ms_per_step is the mean launch duration.  Every workload's
inputs are staged in HBM before the first one is timed, and the workloads run back to back
(fp32 GEMM 4096^3 first, then the headline), so none but the first starts from an idle chip.
The two PCIe-inclusive runtime steps (config 2 and config 4 through the Dream builtins on
host fp64 tensors) run last, after 20 s of idle.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

from dreamcompiler_amd import hip  # noqa: E402

DB = hip.DeviceBuffer
PEAK = {"bf16": 2516.6, "fp32": 157.3, "fp64": 78.6}   # dense TFLOP/s, MI355X (256 CU x 2.4 GHz)
HBM_PEAK_GBS = 8000.0


def _bf16_dev(rng, shape):
    x = DB.from_numpy(rng.standard_normal(shape, dtype=np.float32))
    out = DB.empty(shape, np.uint16)
    hip.convert(out, hip.BF16, x, hip.F32, int(np.prod(shape)))
    hip.sync()
    x.free()
    return out


def _time(fn, steps, warmup):
    for _ in range(warmup):
        fn()
    hip.sync()
    t0 = time.perf_counter()
    with hip.Timer() as t:
        for _ in range(steps):
            fn()
    wall = time.perf_counter() - t0
    return t.ms / steps, wall


# --------------------------------------------------------------------------- workloads
def gemm_workload(dtype, M, N, K, seed=0):
    rng = np.random.default_rng(seed)
    if dtype == "bf16":
        A, B = _bf16_dev(rng, (M, K)), _bf16_dev(rng, (K, N))
        fn_ = hip.gemm_bf16
        in_bytes = 2
    else:
        A = DB.from_numpy(rng.standard_normal((M, K), dtype=np.float32))
        B = DB.from_numpy(rng.standard_normal((K, N), dtype=np.float32))
        fn_ = hip.gemm_f32
        in_bytes = 4
    C = DB.empty((M, N), np.float32)

    def step():
        fn_(0, 0, M, N, K, A, K, B, N, 0.0, C, N)

    flops = 2.0 * M * N * K
    alg_bytes = (M * K + K * N) * in_bytes + M * N * 4
    return step, flops, alg_bytes, [A, B, C]


def gemm_f64_workload(M, N, K, seed=11):
    """fp64 `@` below the dispatch threshold (M*N < 262144): dh_gemm_f64, the reference's
    dgemm summation order (bit-identical results), on the fp64 VALU."""
    rng = np.random.default_rng(seed)
    A, B = DB.from_numpy(rng.standard_normal((M, K))), DB.from_numpy(rng.standard_normal((K, N)))
    C = DB.empty((M, N), np.float64)

    def step():
        hip.gemm_f64(0, 0, M, N, K, A, K, B, N, 0.0, C, N)
    return step, 2.0 * M * N * K, 8.0 * (M * K + K * N + M * N), [A, B, C]


def attention_f64_workload(BH, S, D, causal, backward=False, seed=12):
    """fp64 attention outside the flash rule (here dk > 128): dh_attention_f64_fwd / _bwd,
    the standard form on fp64 GEMMs with the S x S scores in HBM.  FLOPs: the products
    (forward 4 S^2 D per slice, backward 8 S^2 D), all S^2 scores computed even when causal."""
    rng = np.random.default_rng(seed)
    Q, K, V, G = (DB.from_numpy(rng.standard_normal((BH, S * D)) * 0.5) for _ in range(4))
    O = DB.empty((BH, S * D), np.float64)
    sc = 1.0 / np.sqrt(D)
    if not backward:
        def step():
            hip.attention_f64_fwd(BH, S, D, sc, causal, Q, K, V, O)
        return step, 4.0 * BH * S * S * D, 8.0 * 4 * BH * S * D, [Q, K, V, G, O]
    dQ, dK, dV = (DB.empty((BH, S * D), np.float64) for _ in range(3))

    def step():
        hip.attention_f64_bwd(BH, S, D, sc, causal, Q, K, V, G, dQ, dK, dV, 0)
    return step, 8.0 * BH * S * S * D, 8.0 * 7 * BH * S * D, [Q, K, V, G, O, dQ, dK, dV]


def flash_workload(dtype, BH, S, D, causal, backward=False, seed=1):
    rng = np.random.default_rng(seed)
    np_t = np.uint16 if dtype == "bf16" else np.float32
    dt = hip.BF16 if dtype == "bf16" else hip.F32
    elt = 2 if dtype == "bf16" else 4
    if dtype == "bf16":
        Q, K, V, G = (_bf16_dev(rng, (BH, S * D)) for _ in range(4))
    else:
        Q, K, V, G = (DB.from_numpy(rng.standard_normal((BH, S * D), dtype=np.float32) * 0.5)
                      for _ in range(4))
    O = DB.empty((BH, S * D), np_t)
    L = DB.empty((BH, S), np.float32)
    scale = 1.0 / np.sqrt(D)
    hip.flash_fwd(dt, BH, S, D, scale, causal, Q, K, V, O, L)
    fwd_flops = 4.0 * BH * D * S * (S + 1) / 2 if causal else 4.0 * BH * D * S * S
    bufs = [Q, K, V, G, O, L]
    if not backward:
        def step():
            hip.flash_fwd(dt, BH, S, D, scale, causal, Q, K, V, O, L)
        return step, fwd_flops, 4 * BH * S * D * elt + 4 * BH * S, bufs
    dQ, dK, dV = (DB.empty((BH, S * D), np.float32) for _ in range(3))
    bufs += [dQ, dK, dV]

    def step():
        hip.flash_bwd(dt, BH, S, D, scale, causal, Q, K, V, O, G, L, dQ, dK, dV, 0)
    # FlashAttention-2 convention: backward = 2.5 x forward FLOPs (5 S^2 D products).
    return step, 2.5 * fwd_flops, 5 * BH * S * D * elt + 3 * BH * S * D * 4 + 8 * BH * S, bufs


def rows_workload(op, R, C, seed=4):
    """Row-wise ops (HBM-bound): algorithmic bytes = every input read once + the output written
    once (fp32)."""
    rng = np.random.default_rng(seed)
    X = DB.from_numpy(rng.standard_normal((R, C), dtype=np.float32))
    Y, G, GX = (DB.empty((R, C), np.float32) for _ in range(3))
    hip.row_softmax(X, Y, R, C)
    G2 = DB.from_numpy(rng.standard_normal((R, C), dtype=np.float32))
    n = 4.0 * R * C
    if op == "softmax_fwd":
        step, byts = (lambda: hip.row_softmax(X, Y, R, C)), 2 * n
    elif op == "softmax_bwd":
        step, byts = (lambda: hip.row_softmax_bwd(Y, G2, GX, R, C)), 3 * n
    elif op == "layer_norm_fwd":
        step, byts = (lambda: hip.layer_norm(X, Y, R, C)), 2 * n
    else:   # layer_norm_bwd: X, Y, dY read, dX written
        hip.layer_norm(X, Y, R, C)
        step, byts = (lambda: hip.layer_norm_bwd(X, Y, G2, GX, R, C)), 4 * n
    return step, 0.0, byts, [X, Y, G, GX, G2]


def elementwise_workload(op, shape_a, shape_b=None, seed=10):
    """Elementwise op in fp64 (Dream's number type; HBM-bound): dh_binary over broadcast
    strides or dh_unary.  Algorithmic bytes = every operand read once + C written once."""
    rng = np.random.default_rng(seed)
    A = DB.from_numpy(rng.standard_normal(shape_a))
    n = int(np.prod(shape_a))
    C = DB.empty((n,), np.float64)
    if shape_b is None:
        return (lambda: hip.unary(op, hip.F64, A, C, n)), 0.0, 16.0 * n, [A, C]
    B = DB.from_numpy(rng.standard_normal(shape_b))
    da, db = [*shape_a, 1, 1][:4], [*shape_b, 1, 1][:4]
    sa = [da[1] * da[2] * da[3] if da[0] > 1 else 0, da[2] * da[3] if da[1] > 1 else 0,
          da[3] if da[2] > 1 else 0, 1 if da[3] > 1 else 0]
    sb = [db[1] * db[2] * db[3] if db[0] > 1 else 0, db[2] * db[3] if db[1] > 1 else 0,
          db[3] if db[2] > 1 else 0, 1 if db[3] > 1 else 0]
    nb = int(np.prod(shape_b))

    def step():
        hip.binary(op, hip.F64, A, n, sa, B, nb, sb, C, da)
    return step, 0.0, 8.0 * (2 * n + nb), [A, B, C]


def linear_workload(N, IN, OUT, relu=True, seed=6):
    """Fused linear layer Y = relu(X W^T + b) (dream_linear_relu) as one GEMM with the bias /
    ReLU epilogue, fp32."""
    rng = np.random.default_rng(seed)
    X = DB.from_numpy(rng.uniform(0, 1, (N, IN)).astype(np.float32))
    W = DB.from_numpy((rng.standard_normal((OUT, IN)) * np.sqrt(2 / IN)).astype(np.float32))
    b = DB.from_numpy(rng.standard_normal(OUT).astype(np.float32))
    Y = DB.empty((N, OUT), np.float32)

    def step():
        hip.gemm_ex("f32", 0, 1, N, OUT, IN, X, IN, 0, W, IN, 0, 0.0, Y, OUT, 0, 1, b, relu)
    return step, 2.0 * N * IN * OUT, 4.0 * (N * IN + OUT * IN + OUT + N * OUT), [X, W, b, Y]


def bmm_workload(Bt, M, N, K, seed=7):
    """dream_bmm as one batched fp32 GEMM launch (gridDim.y = batch member)."""
    rng = np.random.default_rng(seed)
    A = DB.from_numpy(rng.standard_normal((Bt, M * K), dtype=np.float32))
    B = DB.from_numpy(rng.standard_normal((Bt, K * N), dtype=np.float32))
    C = DB.empty((Bt, M * N), np.float32)

    def step():
        hip.gemm_ex("f32", 0, 0, M, N, K, A, K, M * K, B, N, K * N, 0.0, C, N, M * N, Bt)
    return step, 2.0 * Bt * M * N * K, 4.0 * Bt * (M * K + K * N + M * N), [A, B, C]


def conv_workload(N, Cin, H, W, Cout, KH, KW, pad, stride, seed=9):
    """dream_conv2d's device work: one implicit-GEMM launch (dh_conv2d_fwd: the im2col matrix
    gathered inside the GEMM's operand loader, never stored) with the per-channel bias, fp32.
    Algorithmic bytes: input, kernel, bias read and output written once."""
    rng = np.random.default_rng(seed)
    OH, OW = (H + 2 * pad - KH) // stride + 1, (W + 2 * pad - KW) // stride + 1
    K, P = Cin * KH * KW, OH * OW
    X = DB.from_numpy(rng.standard_normal((N, Cin * H * W), dtype=np.float32))
    Kn = DB.from_numpy((rng.standard_normal((Cout, K)) * 0.05).astype(np.float32))
    b = DB.from_numpy(rng.standard_normal(Cout).astype(np.float32))
    Y = DB.empty((N, Cout * P), np.float32)

    def step():
        hip.conv2d_fwd(X, Kn, b, Y, N, Cin, H, W, Cout, KH, KW, pad, stride)
    flops = 2.0 * N * Cout * P * K
    return step, flops, 4.0 * (N * Cin * H * W + Cout * K + Cout + N * Cout * P), [X, Kn, b, Y]


def conv_bwd_workload(N, Cin, H, W, Cout, KH, KW, pad, stride, seed=10):
    """dream_conv2d's backward as the runtime issues it (autograd.inc:507-535 over all images
    at once): gK += sum_n go_n col_n^T as one implicit GEMM (dh_conv2d_bwd_filter: col gathered
    in the loader, partials over the (image, position) contraction reduced in order), and
    gX += col2im(K^T go') as one implicit-GEMM convolution of go with the flipped kernel
    (dh_conv2d_bwd_data, stride 1).  FLOPs: the two products; algorithmic bytes: go, X, K read,
    gK and gX read and written once."""
    rng = np.random.default_rng(seed)
    OH, OW = (H + 2 * pad - KH) // stride + 1, (W + 2 * pad - KW) // stride + 1
    K, P = Cin * KH * KW, OH * OW
    NP = N * P
    X = DB.from_numpy(rng.standard_normal((N, Cin * H * W), dtype=np.float32))
    Kn = DB.from_numpy((rng.standard_normal((Cout, K)) * 0.05).astype(np.float32))
    go = DB.from_numpy(rng.standard_normal((N, Cout * P), dtype=np.float32))
    gK, gX = DB.from_numpy(np.zeros((Cout, K), np.float32)), \
        DB.from_numpy(np.zeros((N, Cin * H * W), np.float32))

    def step():
        hip.conv2d_bwd_filter(go, X, gK, N, Cin, H, W, Cout, KH, KW, pad, stride, accumulate=True)
        hip.conv2d_bwd_data(go, Kn, gX, N, Cin, H, W, Cout, KH, KW, pad, stride, accumulate=True)
    flops = 4.0 * Cout * K * NP
    alg = 4.0 * (N * Cout * P + N * Cin * H * W + Cout * K) + 8.0 * (Cout * K + N * Cin * H * W)
    return step, flops, alg, [X, Kn, go, gK, gX]


WORKLOADS = {
    # name: (builder, kwargs, precision for the peak, description)
    "gemm_bf16_8192": (gemm_workload, dict(dtype="bf16", M=8192, N=8192, K=8192), "bf16",
                       "bf16 GEMM C=A@B M=N=K=8192, fp32 accumulate/output (config 5)"),
    "gemm_fp32_4096": (gemm_workload, dict(dtype="fp32", M=4096, N=4096, K=4096), "fp32",
                       "fp32 GEMM 4096^3 (config 5, fp32 MFMA figure)"),
    "gemm_fp32_1024": (gemm_workload, dict(dtype="fp32", M=1024, N=1024, K=1024), "fp32",
                       "fp32 GEMM 1024^3 (config 1)"),
    "flash_fwd_c4": (flash_workload, dict(dtype="bf16", BH=128, S=4096, D=128, causal=True),
                     "bf16", "causal FlashAttention fwd B8 H16 S4096 D128 bf16 (config 4)"),
    "flash_bwd_c4": (flash_workload, dict(dtype="bf16", BH=128, S=4096, D=128, causal=True,
                                          backward=True), "bf16",
                     "causal FlashAttention bwd B8 H16 S4096 D128 bf16 (config 4)"),
    "flash_fwd_c4_fp32": (flash_workload, dict(dtype="fp32", BH=128, S=4096, D=128, causal=True),
                          "fp32", "causal FlashAttention fwd B8 H16 S4096 D128 fp32 (the default "
                                  "precision's kernels at config 4's shape)"),
    "flash_bwd_c4_fp32": (flash_workload, dict(dtype="fp32", BH=128, S=4096, D=128, causal=True,
                                               backward=True), "fp32",
                          "causal FlashAttention bwd B8 H16 S4096 D128 fp32"),
    "flash_fwd_c3": (flash_workload, dict(dtype="fp32", BH=24, S=256, D=64, causal=True),
                     "fp32", "causal FlashAttention fwd B4 H6 S256 D64 fp32 (config 3)"),
    "gemm_f64_511": (gemm_f64_workload, dict(M=511, N=511, K=511), "fp64",
                     "fp64 `@` 511^3 (below the dispatch threshold: the reference's dgemm "
                     "order, bit-identical)"),
    "gemm_f64_256x1024_k4096": (gemm_f64_workload, dict(M=256, N=1023, K=4096), "fp64",
                                "fp64 `@` 256 x 4096 @ 4096 x 1023 (below the threshold, long K)"),
    "attention_f64_d256_fwd": (attention_f64_workload, dict(BH=16, S=1024, D=256, causal=True),
                               "fp64", "causal attention fwd B2 H8 S1024 dk=256 in fp64 "
                                       "(outside the flash rule)"),
    "attention_f64_d256_bwd": (attention_f64_workload, dict(BH=16, S=1024, D=256, causal=True,
                                                            backward=True), "fp64",
                               "causal attention bwd B2 H8 S1024 dk=256 in fp64"),
    "linear_relu_c2": (linear_workload, dict(N=4096, IN=784, OUT=257), "fp32",
                       "fused linear_relu X[4096x784] W[257x784]^T + b (config 2 layer 1), fp32"),
    "bmm_64x512": (bmm_workload, dict(Bt=64, M=512, N=512, K=512), "fp32",
                   "dream_bmm 64 x (512x512 @ 512x512) fp32, one batched launch"),
    "conv2d_resnet_64x56x56": (conv_workload, dict(N=64, Cin=64, H=56, W=56, Cout=64, KH=3, KW=3,
                                                   pad=1, stride=1), "fp32",
                               "conv2d 64 x 64ch 56x56, 64 out ch, 3x3 pad 1 (implicit GEMM), fp32"),
    "conv2d_bwd_resnet_64x56x56": (conv_bwd_workload, dict(N=64, Cin=64, H=56, W=56, Cout=64, KH=3,
                                                           KW=3, pad=1, stride=1), "fp32",
                                   "conv2d backward, same layer: implicit-GEMM kernel and "
                                   "data gradients, fp32"),
    "softmax_fwd_16384x1024": (rows_workload, dict(op="softmax_fwd", R=16384, C=1024), "hbm",
                               "row softmax 16384 x 1024 fp32 (HBM-bound)"),
    "softmax_bwd_16384x1024": (rows_workload, dict(op="softmax_bwd", R=16384, C=1024), "hbm",
                               "row softmax backward 16384 x 1024 fp32 (HBM-bound)"),
    "layer_norm_fwd_16384x1024": (rows_workload, dict(op="layer_norm_fwd", R=16384, C=1024),
                                  "hbm", "row layer norm 16384 x 1024 fp32 (HBM-bound)"),
    "layer_norm_bwd_16384x1024": (rows_workload, dict(op="layer_norm_bwd", R=16384, C=1024),
                                  "hbm", "row layer norm backward 16384 x 1024 fp32 (HBM-bound)"),
    "ew_add_f64_4096x4096": (elementwise_workload, dict(op="add", shape_a=(4096, 4096),
                                                        shape_b=(4096, 4096)), "hbm",
                             "elementwise A + B, 4096 x 4096 fp64 (runGPU, HBM-bound)"),
    "ew_mul_rowbcast_f64_4096x4096": (elementwise_workload,
                                      dict(op="mul", shape_a=(4096, 4096), shape_b=(1, 4096)),
                                      "hbm", "elementwise A * b, 4096 x 4096 fp64 with a broadcast "
                                             "row (runGPU strides, HBM-bound)"),
    "ew_sigmoid_f64_4096x4096": (elementwise_workload,
                                 dict(op="sigmoid", shape_a=(4096, 4096)), "hbm",
                                 "elementwise sigmoid, 4096 x 4096 fp64 (runGPUUnary, HBM-bound)"),
}

# Timed first, in this order (see main): the fp32 GEMM absorbs the chip's start-up transient.
NORTH_STAR_ORDER = ["gemm_fp32_4096", "gemm_bf16_8192", "flash_fwd_c4", "flash_bwd_c4"]

MLP_SHAPES = [  # config 2: (name, transA, transB, M, N, K)
    ("X@W1", 0, 0, 4096, 257, 784), ("H@W2", 0, 0, 4096, 10, 257),
    ("dW1=X^T.dZ1", 1, 0, 784, 257, 4096), ("dX=dZ1.W1^T", 0, 1, 4096, 784, 257),
    ("dW2=H^T.dY", 1, 0, 257, 10, 4096), ("dH=dY.W2^T", 0, 1, 4096, 257, 10),
]


def mlp_metrics(steps, warmup):
    rng = np.random.default_rng(2)
    out, tot_ms, tot_flops = {}, 0.0, 0.0
    staged = []   # every shape's operands in HBM before the first is timed (no idle gaps)
    for name, ta, tb, M, N, K in MLP_SHAPES:
        staged.append((DB.from_numpy(rng.standard_normal((K, M) if ta else (M, K), dtype=np.float32)),
                       DB.from_numpy(rng.standard_normal((N, K) if tb else (K, N), dtype=np.float32)),
                       DB.empty((M, N), np.float32)))
    hip.sync()
    for (name, ta, tb, M, N, K), (A, B, C) in zip(MLP_SHAPES, staged):
        lda, ldb = (M if ta else K), (K if tb else N)
        ms, _ = _time(lambda: hip.gemm_f32(ta, tb, M, N, K, A, lda, B, ldb, 0.0, C, N),
                      steps, warmup)
        fl = 2.0 * M * N * K
        byts = 4.0 * (M * K + K * N + M * N)
        out[name] = {"ms": round(ms, 5), "gflops": round(fl / ms / 1e6, 1),
                     "gbs": round(byts / ms / 1e6, 1)}
        tot_ms += ms
        tot_flops += fl
        for b in (A, B, C):
            b.free()
    out["total"] = {"ms": round(tot_ms, 4), "gflops": round(tot_flops / tot_ms / 1e6, 1)}
    return out


def _mlp_c2_inputs(seed=8):
    rng = np.random.default_rng(seed)
    return (rng.uniform(0, 1, (4096, 784)), rng.standard_normal((257, 784)) * np.sqrt(2 / 784),
            rng.standard_normal((1, 257)) * 0.1, rng.standard_normal((10, 257)) * np.sqrt(2 / 257),
            rng.standard_normal((1, 10)) * 0.1, rng.standard_normal((4096, 10)))


def _mlp_c2_program(L, tensor, X, W1, b1, W2, b2, G):
    """One config-2 training step as a .dream program would issue it: h = linear_relu(X, W1, b1),
    y = linear(h, W2, b2), loss = sum(log_softmax(y) * G), backward(loss).  Returns a step
    function (the graph of each step is released after its backward)."""
    x, w1, bb1, w2, bb2, g = (tensor(a) for a in (X, W1, b1, W2, b2, G))

    def step():
        h = L.dream_linear_relu(x, w1, bb1)
        y = L.dream_linear(h, w2, bb2)
        lp = L.dream_log_softmax(y)
        m = L.tensor_mul(lp, g)
        loss = L.sum(m)
        r = L.backward(loss)
        for t in (r, loss, m, lp, y, h):
            L.tensor_decref(t)
        for t in (x, w1, bb1, w2, bb2):
            L.tensor_decref(L.zero_grad(t))
    return step


def runtime_mlp_metrics(steps=10, warmup=3):
    """Config 2 end to end through the Dream builtins (libdream_rt): host fp64 tensors in and
    out, so PCIe staging is inside the time; the weights' and inputs' device copies persist
    across steps (their versions do not change), the activations and gradients stay on the
    device between the GPU ops of one step."""
    from dreamcompiler_amd import runtime as rt
    step = _mlp_c2_program(rt.load(), rt.tensor, *_mlp_c2_inputs())
    for _ in range(warmup):
        step()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    ms = (time.perf_counter() - t0) * 1000.0 / steps
    flops = 3 * 2.0 * 4096 * (784 * 257 + 257 * 10)
    return {"ms_per_step": round(ms, 3), "gflops": round(flops / ms / 1e6, 1),
            "desc": "config 2 fwd+bwd step through dream_linear_relu / dream_linear / "
                    "dream_log_softmax / backward on fp64 host tensors (PCIe-inclusive), "
                    "no optimizer update"}


def runtime_flash_c4_metrics(steps=3, warmup=1):
    """Config 4 end to end through the Dream builtins with dream_enable_fp16: O =
    dream_flash_attention(Q, K, V, 128, 4096, 128, 64) on fp64 host tensors, then
    backward(sum(O * W)) -- PCIe-inclusive (Q, K, V, W in; O and the three gradients, 537 MB
    each in fp64, out every step).  Device copies of the unchanged inputs persist across
    steps, as they would in a training loop."""
    from dreamcompiler_amd import runtime as rt
    L = rt.load()
    B, S, dk = 128, 4096, 128
    rng = np.random.default_rng(13)
    ts = [rt.tensor(rng.standard_normal((B, S * dk)) * 0.5) for _ in range(4)]
    sc = [rt.scalar(v) for v in (B, S, dk, 64)]
    L.dream_enable_fp16()
    try:
        def step():
            o = L.dream_flash_attention(ts[0], ts[1], ts[2], *sc)
            m = L.tensor_mul(o, ts[3])
            loss = L.sum(m)
            r = L.backward(loss)
            rt.release(r, loss, m, o)
            for t in ts[:3]:
                L.tensor_decref(L.zero_grad(t))
        for _ in range(warmup):
            step()
        t0 = time.perf_counter()
        for _ in range(steps):
            step()
        ms = (time.perf_counter() - t0) * 1000.0 / steps
    finally:
        L.dream_disable_fp16()
        rt.release(*ts, *sc)
    return {"ms_per_step": round(ms, 2),
            "desc": "config 4 causal flash fwd + backward(sum(O*W)) through dream_flash_attention / "
                    "backward on fp64 host tensors, bf16 mode (PCIe-inclusive)"}


# --------------------------------------------------------------------------- CPU baseline
def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _maxrel(got, ref):
    return float(np.abs(got - ref).max() / max(float(np.abs(ref).max()), 1e-300))


def parity_checks():
    """Parity of every contract config on the GPU, checked on the CPU (part of the CPU leg):
    the GPU result against an fp64 reference on the same inputs -- numpy's fp64 products for
    the GEMMs, fp64 softmax attention for config 3, the CPU restatement of the reference
    (oracle, sampled rows) for config 4 -- as the normwise max relative error beside the
    contract's bound (fp32 1e-5 sqrt(K), bf16 2e-2)."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    out = {}

    def rec(name, err, tol, sample):
        out[name] = {"gpu_maxrel": float(f"{err:.3e}"), "tol": float(f"{tol:.3e}"),
                     "ok": bool(err <= tol), "sample": sample}

    def gemm_gpu(dtype, A, B, ta=0, tb=0):
        M = A.shape[1] if ta else A.shape[0]
        K = A.shape[0] if ta else A.shape[1]
        N = B.shape[0] if tb else B.shape[1]
        dA, dB, dC = DB.from_numpy(A), DB.from_numpy(B), DB.empty((M, N), np.float32)
        fn = hip.gemm_bf16 if dtype == "bf16" else hip.gemm_f32
        fn(ta, tb, M, N, K, dA, A.shape[1], dB, B.shape[1], 0.0, dC, N)
        C = dC.numpy()
        for b in (dA, dB, dC):
            b.free()
        return C

    def bf16(x):
        u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
        return (((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFFFFFF) >> 16).astype(np.uint16)

    def unbf16(b):
        return (b.astype(np.uint32) << 16).view(np.float32)

    rng = np.random.default_rng(42)
    # config 1: fp32 1024^3, full product
    A, B = (rng.standard_normal((1024, 1024), dtype=np.float32) for _ in range(2))
    rec("C1_fp32_1024", _maxrel(gemm_gpu("f32", A, B), A.astype(np.float64) @ B.astype(np.float64)),
        1e-5 * np.sqrt(1024), "full 1024 x 1024")
    # config 2: the six products of the MLP set, full
    worst, wtol = 0.0, 1.0
    for name, ta, tb, M, N, K in MLP_SHAPES:
        A = rng.standard_normal((K, M) if ta else (M, K), dtype=np.float32)
        B = rng.standard_normal((N, K) if tb else (K, N), dtype=np.float32)
        ref = (A.T if ta else A).astype(np.float64) @ (B.T if tb else B).astype(np.float64)
        e, t = _maxrel(gemm_gpu("f32", A, B, ta, tb), ref), 1e-5 * np.sqrt(K)
        if e / t > worst / wtol:
            worst, wtol = e, t
    rec("C2_mlp_set", worst, wtol, "six products in full; the one nearest its bound")
    # config 5: bf16 8192^3 and fp32 4096^3 on sampled rows
    for name, dtype, n, rows in (("C5_bf16_8192", "bf16", 8192, 16), ("C5_fp32_4096", "f32", 4096, 32)):
        A, B = (rng.standard_normal((n, n), dtype=np.float32) for _ in range(2))
        if dtype == "bf16":
            A, B = bf16(A), bf16(B)
            A64, B64 = unbf16(A).astype(np.float64), unbf16(B).astype(np.float64)
        else:
            A64, B64 = A.astype(np.float64), B.astype(np.float64)
        C = gemm_gpu(dtype, A, B)
        idx = rng.choice(n, rows, replace=False)
        rec(name, _maxrel(C[idx], A64[idx] @ B64), 2e-2 if dtype == "bf16" else 1e-5 * np.sqrt(n),
            f"{rows} random rows of {n}, all columns (fp64 on the {'bf16-rounded ' if dtype == 'bf16' else ''}inputs)")
        del A, B, A64, B64, C
    # config 3: fp32 causal flash B4 H6 S256 D64, full, against fp64 softmax attention
    BH, S, D = 24, 256, 64
    Q, K, V = (rng.standard_normal((BH, S * D), dtype=np.float32) * np.float32(0.5) for _ in range(3))
    dq, dk, dv = (DB.from_numpy(x) for x in (Q, K, V))
    dO, dL = DB.empty((BH, S * D), np.float32), DB.empty((BH, S), np.float32)
    hip.flash_fwd(hip.F32, BH, S, D, 1.0 / np.sqrt(D), True, dq, dk, dv, dO, dL)
    Og = dO.numpy().reshape(BH, S, D)
    q, k, v = (x.astype(np.float64).reshape(BH, S, D) for x in (Q, K, V))
    s = np.einsum("bid,bjd->bij", q, k) / np.sqrt(D)
    s = np.where(np.tril(np.ones((S, S), bool))[None], s, -np.inf)
    p = np.exp(s - s.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    rec("C3_flash_fp32", _maxrel(Og, np.einsum("bij,bjd->bid", p, v)), 1e-5 * np.sqrt(S), "full")
    # config 4: bf16 causal flash fwd + bwd at full size; O and dQ of 4 rows in each of 16
    # slices from the CPU restatement (oracle attention_rows), fp64 on the bf16-rounded inputs
    import _oracle  # noqa: E402  (test infrastructure: the checker of the CPU leg)
    BH, S, D = 128, 4096, 128
    Qb, Kb, Vb, Gb = (bf16(rng.standard_normal((BH, S * D), dtype=np.float32)) for _ in range(4))
    bufs = [DB.from_numpy(x) for x in (Qb, Kb, Vb, Gb)]
    dO, dL = DB.empty((BH, S * D), np.uint16), DB.empty((BH, S), np.float32)
    grads = [DB.empty((BH, S * D), np.float32) for _ in range(3)]
    sc = 1.0 / np.sqrt(D)
    hip.flash_fwd(hip.BF16, BH, S, D, sc, True, bufs[0], bufs[1], bufs[2], dO, dL)
    hip.flash_bwd(hip.BF16, BH, S, D, sc, True, bufs[0], bufs[1], bufs[2], dO, bufs[3], dL,
                  grads[0], grads[1], grads[2], 0)
    Og = unbf16(dO.numpy()).reshape(BH, S, D)
    dQg = grads[0].numpy().reshape(BH, S, D)
    sl = rng.choice(BH, 16, replace=False)
    rows = np.stack([rng.choice(S, 4, replace=False) for _ in sl]).astype(np.int32)
    f64 = [unbf16(x[sl]).astype(np.float64) for x in (Qb, Kb, Vb, Gb)]
    Oref, dQref = _oracle.attention_rows(*f64, rows, len(sl), S, D, True)
    rec("C4_flash_bf16_fwd_O", _maxrel(np.stack([Og[b][r] for b, r in zip(sl, rows)]), Oref), 2e-2,
        "4 random rows in each of 16 random slices")
    rec("C4_flash_bf16_bwd_dQ", _maxrel(np.stack([dQg[b][r] for b, r in zip(sl, rows)]), dQref), 2e-2,
        "4 random rows in each of 16 random slices")
    for b in bufs + grads + [dO, dL, dq, dk, dv]:
        b.free()
    hip.load().dh_pool_release()
    return out


def cpu_baseline_gemm(n=8192, rows=8192, reps=3):
    """The reference's CPU `@` on fp32 operands (`as f32` -> dream_gemm_f32, blocked 8x16
    AVX2 kernel, OpenMP over 128-row blocks, runtime/ops/elementwise.inc:689-738) on a
    bounded sample of the workload: `rows` rows of A times the full 8192 x 8192 B.
    There is no bf16 CPU path in the reference; fp32 is its closest `@`."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    rng = np.random.default_rng(3)
    A = rng.standard_normal((rows, n)).astype(np.float32).astype(np.float64)
    B = rng.standard_normal((n, n)).astype(np.float32).astype(np.float64)
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    import _ref_runtime  # noqa: E402  (test infrastructure: the CPU comparison only)
    if _ref_runtime.available():
        R = _ref_runtime.RefRuntime()
        kind = "reference"
        run = lambda: R.matmul(A, B, f32=True)  # noqa: E731
    else:
        import _oracle  # noqa: E402
        kind = "port"
        A32, B32 = A.astype(np.float32), B.astype(np.float32)
        run = lambda: _oracle.gemm_f32(A32, B32)  # noqa: E731
    best, C = 1e30, None
    for _ in range(reps):
        t0 = time.perf_counter()
        C = run()
        best = min(best, time.perf_counter() - t0)
    gflops = 2.0 * rows * n * n / best / 1e9
    idx = rng.choice(rows, 16, replace=False)   # the CPU result's own error, sampled rows
    err = _maxrel(np.asarray(C, np.float64)[idx], A[idx] @ B)
    return {"value": round(gflops, 2), "unit": "GFLOP/s", "cores": threads, "kind": kind,
            "cpu_model": cpu_model(),
            "cpu_maxrel": float(f"{err:.3e}"),
            "sample": f"fp32 `@` (as f32) {rows}x{n} @ {n}x{n} (rows {rows}/{n} of the "
                      f"workload), best of {reps}, {best:.2f} s, OMP threads {threads}; "
                      f"cpu_maxrel: 16 random rows against fp64"}


def cpu_baseline_flash(S=4096, D=128, slices=32):
    """The reference's CPU flash_attention forward (fp64, single-threaded,
    runtime/nn/training.inc:366-399) on `slices` of the 128 (batch x head) slices of
    config 4; slices are independent and equal in work, so the rate scales exactly."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import _ref_runtime  # noqa: E402
    rng = np.random.default_rng(5)
    Q, K, V = (rng.standard_normal((slices, S * D)) for _ in range(3))
    if _ref_runtime.available():
        R = _ref_runtime.RefRuntime()
        kind = "reference"
        t0 = time.perf_counter()
        R.attention("flash", Q, K, V, slices, S, D, 64)
    else:
        import _oracle  # noqa: E402
        kind = "port"
        t0 = time.perf_counter()
        _oracle.flash_fwd(Q, K, V, slices, S, D, 64)
    dt = time.perf_counter() - t0
    flops = 4.0 * slices * D * S * (S + 1) / 2
    return {"value": round(flops / dt / 1e9, 3), "unit": "GFLOP/s", "cores": 1, "kind": kind,
            "sample": f"{slices} of 128 slices, S={S} D={D}, fp64, {dt:.1f} s"}


def cpu_baseline_mlp(steps=2):
    """The same config-2 step on the reference's own CPU runtime (oracle/_ref): its fused
    linear (elementwise.inc:1432-1516), log_softmax and backward (autograd.inc:156-233), OpenMP
    over the host's OMP_NUM_THREADS."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import _ref_runtime  # noqa: E402  (test infrastructure: the CPU comparison only)
    if not _ref_runtime.available():
        return {"error": "oracle/_ref not built"}
    R = _ref_runtime.RefRuntime()
    step = _mlp_c2_program(R.L, R.tensor, *_mlp_c2_inputs())
    step()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    ms = (time.perf_counter() - t0) * 1000.0 / steps
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    return {"ms_per_step": round(ms, 2), "cores": threads, "kind": "reference",
            "sample": f"{steps} steps after 1 warm-up"}


def cpu_baseline_workloads(gpu_ms):
    """The reference's own CPU path (oracle/_ref) timed on each secondary workload's shape, or
    on a stated sample of it: ms per full workload (sampled runs scaled by the exact work
    ratio), beside the GPU's ms.  fp64 (Dream's type) on the host's OMP_NUM_THREADS where the
    reference uses OpenMP, single-threaded where it does not."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import _ref_runtime  # noqa: E402  (test infrastructure: the CPU comparison only)
    if not _ref_runtime.available():
        return {"error": "oracle/_ref not built"}
    R = _ref_runtime.RefRuntime()
    L = R.L
    rng = np.random.default_rng(12)
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    out = {}

    def timed(fn, reps=1):
        fn()   # warm-up (page-in, OpenMP pool)
        t0 = time.perf_counter()
        for _ in range(reps):
            fn()
        return (time.perf_counter() - t0) * 1000.0 / reps

    def record(name, ms_sample, scale, sample, cores=threads):
        ms = ms_sample * scale
        g = gpu_ms.get(name)
        out[name] = {"value": round(ms, 3), "unit": "ms", "cores": cores, "kind": "reference",
                     "sample": sample, "gpu_ms": g,
                     "gpu_speedup": round(ms / g, 1) if g else None}

    # row ops at 16384 x 1024: forward builtins, and the backward of backward(sum(Y * G))
    X, G = rng.standard_normal((16384, 1024)), rng.standard_normal((16384, 1024))
    x, g = R.tensor(X), R.tensor(G)
    for name, fn in (("softmax_fwd_16384x1024", L.dream_softmax),
                     ("layer_norm_fwd_16384x1024", L.dream_layer_norm)):
        record(name, timed(lambda: L.tensor_decref(fn(x))), 1, "full shape, fp64", 1)
    # backward(Y) on the op's own output runs exactly that op's backward branch (upstream
    # gradient of ones: the same work as any other upstream)
    for name, fn in (("softmax_bwd_16384x1024", L.dream_softmax),
                     ("layer_norm_bwd_16384x1024", L.dream_layer_norm)):
        y = fn(x)
        record(name, timed(lambda: L.backward(y)), 1, "full shape, fp64; backward(Y) of the op", 1)
    # elementwise at 4096 x 4096 (runCPUBinary / runCPUUnary, OpenMP on the same-shape path)
    A, B, b = rng.standard_normal((4096, 4096)), rng.standard_normal((4096, 4096)), \
        rng.standard_normal((1, 4096))
    a, bb, brow = R.tensor(A), R.tensor(B), R.tensor(b)
    record("ew_add_f64_4096x4096", timed(lambda: L.tensor_decref(L.tensor_add(a, bb)), 3), 1,
           "full shape, fp64")
    record("ew_mul_rowbcast_f64_4096x4096",
           timed(lambda: L.tensor_decref(L.tensor_mul(a, brow)), 3), 1,
           "full shape, fp64 (the broadcast loop is single-threaded)", 1)
    record("ew_sigmoid_f64_4096x4096", timed(lambda: L.tensor_decref(L.dream_sigmoid(a)), 3), 1,
           "full shape, fp64")
    # fused linear_relu of config 2's first layer
    Xl = rng.uniform(0, 1, (4096, 784))
    Wl, bl = rng.standard_normal((257, 784)) * np.sqrt(2 / 784), rng.standard_normal((1, 257))
    xl, wl, bl_ = R.tensor(Xl), R.tensor(Wl), R.tensor(bl)
    record("linear_relu_c2", timed(lambda: L.tensor_decref(L.dream_linear_relu(xl, wl, bl_)), 3),
           1, "full shape, fp64")
    # bmm 64 x 512^3: 4 of the 64 batch members (the reference's loop is the same per member)
    nb = 2
    Ab, Bb = rng.standard_normal((nb, 512 * 512)), rng.standard_normal((nb, 512 * 512))
    ab, bbm = R.tensor(Ab), R.tensor(Bb)
    sc = [R.scalar(v) for v in (nb, 512, 512, 512)]
    record("bmm_64x512", timed(lambda: L.tensor_decref(L.dream_bmm(ab, bbm, *sc))), 64 / nb,
           f"{nb} of 64 batch members, fp64, scaled by 64/{nb}", 1)
    # conv2d 64 x 64ch 56x56 -> 64ch 3x3 pad 1: 8 of the 64 images (per-image host loop)
    ni = 4
    Xc = rng.standard_normal((ni, 64 * 56 * 56))
    Kc, bc = rng.standard_normal((64, 64 * 9)) * 0.05, rng.standard_normal((1, 64))
    xc, kc, bcc = R.tensor(Xc), R.tensor(Kc), R.tensor(bc)
    scc = [R.scalar(v) for v in (56, 56, 3, 3, 1, 1)]
    record("conv2d_resnet_64x56x56",
           timed(lambda: L.tensor_decref(L.dream_conv2d_padded(xc, kc, bcc, *scc))), 64 / ni,
           f"{ni} of 64 images, fp64, scaled by 64/{ni}")
    # its backward: backward(Y) on the conv output runs the conv branch only (autograd.inc:507-535)
    yc = L.dream_conv2d_padded(xc, kc, bcc, *scc)
    t0 = time.perf_counter()
    L.backward(yc)
    record("conv2d_bwd_resnet_64x56x56", (time.perf_counter() - t0) * 1000.0, 64 / ni,
           f"{ni} of 64 images, fp64, backward(Y) of the conv, scaled by 64/{ni}")
    # fp64 `@` below the threshold: the reference's dgemm on the full shapes
    for name, (M, N, K) in (("gemm_f64_511", (511, 511, 511)),
                            ("gemm_f64_256x1024_k4096", (256, 1023, 4096))):
        Ag, Bg = rng.standard_normal((M, K)), rng.standard_normal((K, N))
        ag, bg = R.tensor(Ag), R.tensor(Bg)
        record(name, timed(lambda: L.tensor_decref(L.tensor_matmul(ag, bg))), 1,
               "full shape, fp64 dgemm")
    # causal attention, dk = 256 (fp64 on the reference's CPU for every shape): 1 of the 16
    # slices, forward, and backward(O) of the attention node
    q6, k6, v6 = (R.tensor(rng.standard_normal((1, 1024 * 256)) * 0.5) for _ in range(3))
    sc6 = [R.scalar(v) for v in (1, 1024, 256)]
    record("attention_f64_d256_fwd",
           timed(lambda: L.tensor_decref(L.dream_attention_causal(q6, k6, v6, *sc6))), 16,
           "1 of 16 slices, S=1024 dk=256, fp64, scaled by 16", 1)
    o6 = L.dream_attention_causal(q6, k6, v6, *sc6)
    t0 = time.perf_counter()
    L.backward(o6)
    record("attention_f64_d256_bwd", (time.perf_counter() - t0) * 1000.0, 16,
           "1 of 16 slices, S=1024 dk=256, fp64, backward(O) only, scaled by 16", 1)
    # config 3 flash forward (fp64, single-threaded) on the whole config
    Q3, K3, V3 = (rng.standard_normal((24, 256 * 64)) * 0.5 for _ in range(3))
    record("flash_fwd_c3", timed(lambda: R.attention("flash", Q3, K3, V3, 24, 256, 64, 64)), 1,
           "full config, fp64", 1)
    # config 4 flash backward: 1 of the 128 slices (fp64, single-threaded), backward(O) only
    ns = 1
    q4, k4, v4 = (R.tensor(rng.standard_normal((ns, 4096 * 128))) for _ in range(3))
    o4 = L.dream_flash_attention(q4, k4, v4, *(R.scalar(v) for v in (ns, 4096, 128, 64)))
    t0 = time.perf_counter()
    L.backward(o4)
    bwd_ms = (time.perf_counter() - t0) * 1000.0
    record("flash_bwd_c4", bwd_ms, 128 / ns,
           f"{ns} of 128 slices, S=4096 D=128, fp64, backward(O) only, scaled by 128/{ns}", 1)
    return out


# --------------------------------------------------------------------------- main
def load_traffic():
    """HBM bytes per launch measured with rocprofv3 --pmc (FETCH_SIZE, WRITE_SIZE), scaled
    by the copy-kernel calibration factor, read from the committed summaries
    profiles/<workload>_traffic.md (their "Total HBM traffic per launch ... N bytes" line),
    so the figure is the one the summary states and nothing is kept twice."""
    import re
    out = {}
    d = os.path.join(ROOT, "profiles")
    if not os.path.isdir(d):
        return out
    for fn in sorted(os.listdir(d)):
        if not fn.endswith("_traffic.md"):
            continue
        with open(os.path.join(d, fn)) as f:
            txt = f.read()
        m = re.search(r"Total HBM traffic per launch[^:]*:\s*([0-9.]+e[+-]?[0-9]+) bytes", txt)
        r = re.search(r"\(ratio ([0-9.]+)\)", txt)
        if m:
            out[fn[:-len("_traffic.md")]] = {
                "bytes_per_launch": int(float(m.group(1))),
                "ratio_to_algorithmic": float(r.group(1)) if r else None,
                "source": "profiles/" + fn}
    return out


def prepare(name):
    """Inputs of one workload generated on the host and staged in HBM (untimed)."""
    builder, kw, _, _ = WORKLOADS[name]
    return builder(**kw)


def measure(name, steps, warmup, prepared=None):
    _, _, prec, desc = WORKLOADS[name]
    step, flops, alg_bytes, bufs = prepared or prepare(name)
    ms, wall = _time(step, steps, warmup)
    gbs = alg_bytes / ms / 1e6
    if prec == "hbm":
        res = {"workload": name, "desc": desc, "ms": round(ms, 5), "gbs": round(gbs, 1),
               "frac_peak": round(gbs / HBM_PEAK_GBS, 4), "peak_gbs": HBM_PEAK_GBS,
               "alg_bytes": alg_bytes, "wall_s": round(wall, 4)}
    else:
        tflops = flops / ms / 1e9
        res = {"workload": name, "desc": desc, "ms": round(ms, 5), "tflops": round(tflops, 2),
               "frac_peak": round(tflops / PEAK[prec], 4), "peak_tflops": PEAK[prec],
               "gbs": round(gbs, 1), "alg_bytes": alg_bytes, "wall_s": round(wall, 4)}
    traffic = load_traffic().get(name)
    if traffic:
        res["hbm_bytes_measured"] = traffic["bytes_per_launch"]
    for b in bufs:
        b.free()
    hip.load().dh_pool_release()
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=30)
    ap.add_argument("--workload", default="gemm_bf16_8192", choices=sorted(WORKLOADS))
    ap.add_argument("--only", action="store_true",
                    help="time only --workload (for profiling runs); no extra metrics")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--vendor", action="store_true",
                    help="only time the vendor libraries: hipBLASLt through torch.mm on the "
                         "headline shape (bf16 8192^3, fp32 out) after the same kind of idle gap "
                         "the bench has before its launches, then config 4's causal attention "
                         "forward and backward through torch's scaled_dot_product_attention "
                         "backends, under the same --warmup / --steps")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run 5 plain device copies of 1 GiB (dh_convert F32->F32), the "
                         "known-size reference for rocprof FETCH_SIZE / WRITE_SIZE")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); "
              "multi-GPU sharding is a design note, not a measured path.", file=sys.stderr)
        sys.exit(2)
    if args.vendor:   # before this library loads: torch brings its own HIP runtime
        import torch
        n = 8192
        a = torch.randn(n, n, device="cuda").to(torch.bfloat16)
        b = torch.randn(n, n, device="cuda").to(torch.bfloat16)
        torch.cuda.synchronize()
        time.sleep(2.0)   # the GPU idles while bench.py generates its inputs on the host
        for _ in range(args.warmup):
            torch.mm(a, b, out_dtype=torch.float32)
        torch.cuda.synchronize()
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0.record()
        for _ in range(args.steps):
            torch.mm(a, b, out_dtype=torch.float32)
        t1.record()
        torch.cuda.synchronize()
        ms = t0.elapsed_time(t1) / args.steps
        out = {"vendor": "hipBLASLt via torch.mm, bf16 8192^3, fp32 out",
               "warmup": args.warmup, "steps": args.steps, "ms": round(ms, 5),
               "tflops": round(2.0 * n ** 3 / ms / 1e9, 1)}
        del a, b
        # config 4 through torch's scaled_dot_product_attention, each backend it offers here
        import torch.nn.functional as F
        from torch.nn.attention import SDPBackend, sdpa_kernel
        Bt, H, S, D = 8, 16, 4096, 128
        q, k, v = (torch.randn(Bt, H, S, D, device="cuda", dtype=torch.bfloat16,
                               requires_grad=True) for _ in range(3))
        g = torch.randn(Bt, H, S, D, device="cuda", dtype=torch.bfloat16)
        fwd_flops = 4.0 * Bt * H * D * S * (S + 1) / 2

        def timed(fn, steps):
            for _ in range(args.warmup):
                fn()
            torch.cuda.synchronize()
            t0.record()
            for _ in range(steps):
                fn()
            t1.record()
            torch.cuda.synchronize()
            return t0.elapsed_time(t1) / steps

        attn = {}
        for name, be in (("flash", SDPBackend.FLASH_ATTENTION),
                         ("efficient", SDPBackend.EFFICIENT_ATTENTION)):
            try:
                with sdpa_kernel(be):
                    f_ms = timed(lambda: F.scaled_dot_product_attention(q, k, v, is_causal=True),
                                 args.steps)
                    o = F.scaled_dot_product_attention(q, k, v, is_causal=True)

                    def bwd():
                        q.grad = k.grad = v.grad = None
                        o.backward(g, retain_graph=True)
                    b_ms = timed(bwd, max(5, args.steps // 2))
                attn[name] = {"fwd_ms": round(f_ms, 4), "fwd_tflops": round(fwd_flops / f_ms / 1e9, 1),
                              "bwd_ms": round(b_ms, 4),
                              "bwd_tflops": round(2.5 * fwd_flops / b_ms / 1e9, 1)}
            except Exception as e:  # a backend this torch build does not offer
                attn[name] = {"error": repr(e)[:200]}
        out["sdpa_c4_causal_bf16"] = attn
        print(json.dumps(out), flush=True)
        return

    if not hip.available():
        raise SystemExit("bench.py: no usable HIP device: " + hip.load().dh_last_error().decode())

    if args.copy_calibration:
        n = (1 << 30) // 4
        src, dst = DB(n * 4), DB(n * 4)
        src.fill_zero()
        for _ in range(5):
            hip.convert(dst, hip.F32, src, hip.F32, n)
        hip.sync()
        print(json.dumps({"copy_calibration_bytes": n * 4, "copies": 5}), flush=True)
        return

    info = hip.device_info()
    metrics = {}
    if args.only:
        head = measure(args.workload, args.steps, args.warmup)
    else:
        # The north-star workloads are staged in HBM first and then timed back to back, each
        # with its own W warm-up and K timed launches.  Generating an input on the host takes
        # seconds, and after such an idle gap the chip's first ~30 launches run in a
        # power-management transient (per-launch trace: bf16 GEMM 8192^3 0.90, 0.86, 1.06,
        # 1.07, ... back to 0.84 ms by launch 30; launched right after another workload it
        # runs 0.83-0.84 ms from the first launch).  So no timed workload follows an idle
        # gap except the first, the fp32 GEMM, which takes the transient.  The other
        # workloads follow in the same way (all inputs together take a few GB of HBM).
        # The two runtime steps (host fp64 tensors, PCIe copies inside the time) come last,
        # after 20 s of idle: after heavy GPU work the platform's power management leaves
        # device-to-host copies slow for seconds (config-2 step 2.3 ms right after the fp32
        # flash backward at config 4's shape, then 1.7 / 1.6 / 1.4 ms after 1 / 3 / 10 s of
        # idle; its kernels unchanged, rocprofv3 copy trace 62 -> 135 us per copy).  Timed
        # first instead, they left the bf16 GEMM's 5-launch protocol 2% slower.
        order = NORTH_STAR_ORDER + [n for n in WORKLOADS if n not in NORTH_STAR_ORDER]
        staged = {n: prepare(n) for n in order}
        hip.sync()
        for name in order:
            metrics[name] = measure(name, args.steps, args.warmup, staged.pop(name))
        head = metrics.pop(args.workload)
        metrics["mlp_c2"] = mlp_metrics(max(5, args.steps), 3)
        hip.sync()
        time.sleep(20.0)
        metrics["runtime_mlp_c2_step"] = runtime_mlp_metrics()
        metrics["runtime_flash_c4_step"] = runtime_flash_c4_metrics()

    traffic = load_traffic().get(args.workload)
    prec = WORKLOADS[args.workload][2]
    if prec == "hbm":   # a memory-bound workload chosen with --workload (profiling runs)
        roofline = {"bound": "hbm", "achieved": head["gbs"], "peak": HBM_PEAK_GBS,
                    "unit": "GB/s", "frac": head["frac_peak"],
                    "traffic": traffic["bytes_per_launch"] if traffic else None}
    else:
        roofline = {"bound": "mfma", "achieved": head["tflops"], "peak": PEAK[prec],
                    "unit": "TFLOP/s", "frac": head["frac_peak"],
                    "traffic": traffic["bytes_per_launch"] if traffic else None}
    if roofline["traffic"] and traffic.get("ratio_to_algorithmic"):
        roofline["traffic_note"] = (
            f"{traffic['ratio_to_algorithmic']}x the algorithmic bytes ({traffic['source']})")
    line = {
        "metric": "GEMM GFLOP/s fp32 4096^3 / bf16 8192^3; FlashAttn fwd TFLOP/s; % MFMA peak",
        "value": round(head["gbs"] if prec == "hbm" else head["tflops"] * 1000.0, 1),
        "unit": "GB/s" if prec == "hbm" else "GFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["ms"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": ("bf16" if prec == "bf16" else
                  "f64" if prec == "fp64" or args.workload.startswith("ew_") else "f32"),
        "data": "synthetic N(0,1) inputs (numpy PCG64, seeded), resident in HBM",
        "config": {"workload": head["desc"], "name": args.workload},
        "roofline": roofline,
    }
    detail = {"metrics": metrics, "device": info}
    if not args.no_cpu and not args.only:
        try:
            if args.workload.startswith("flash"):
                line["cpu_baseline"] = cpu_baseline_flash()
            else:
                line["cpu_baseline"] = cpu_baseline_gemm()
            detail["cpu_baseline_flash_fwd_c4"] = cpu_baseline_flash()
            detail["cpu_baseline_runtime_mlp_c2_step"] = cpu_baseline_mlp()
            detail["cpu_baseline_workloads"] = cpu_baseline_workloads(
                {k: v["ms"] for k, v in metrics.items() if isinstance(v, dict) and "ms" in v})
            detail["parity"] = parity_checks()
        except Exception as e:  # the CPU comparison must not hide the GPU result
            line["cpu_baseline"] = {"error": repr(e)}
    if not args.only:
        # Every figure first, on its own line; the result line below stays short (a few KB)
        # so that a reader keeping only the end of stdout still has all of it.
        print(json.dumps({"bench_detail": detail}), flush=True)
        line.update(summary_fields(head, metrics, detail))
    print(json.dumps(line), flush=True)


def summary_fields(head, metrics, detail):
    """The compact part of the result line: the three north-star figures (bf16 GEMM 8192^3,
    fp32 GEMM 4096^3, causal FA forward of config 4) plus the FA backward, each as ms and
    fraction of its peak; the config-2 products and the two runtime steps; the parity
    verdicts; the CPU rates."""
    allm = dict(metrics)
    allm[head["workload"]] = head

    def fig(name):
        m = allm.get(name)
        if not m:
            return None
        r = {"ms": m["ms"], "frac_peak": m["frac_peak"]}
        r["tflops" if "tflops" in m else "gbs"] = m.get("tflops", m.get("gbs"))
        return r
    out = {"north_star": {n: fig(n) for n in ("gemm_bf16_8192", "gemm_fp32_4096",
                                              "flash_fwd_c4", "flash_bwd_c4")},
           "secondary": {n: fig(n) for n in ("gemm_fp32_1024", "flash_fwd_c3",
                                             "flash_fwd_c4_fp32", "flash_bwd_c4_fp32")}}
    mlp = metrics.get("mlp_c2")
    if mlp:
        out["mlp_c2_us"] = {k: round(v["ms"] * 1000.0, 2) for k, v in mlp.items()}
    for k in ("runtime_mlp_c2_step", "runtime_flash_c4_step"):
        if k in metrics:
            out[k + "_ms"] = metrics[k]["ms_per_step"]
    par = detail.get("parity")
    if isinstance(par, dict):
        out["parity"] = {k: {"maxrel": v.get("gpu_maxrel"), "tol": v.get("tol"), "ok": v.get("ok")}
                         for k, v in par.items() if isinstance(v, dict)}
        out["parity_all_ok"] = all(v.get("ok") for v in par.values() if isinstance(v, dict))
    cpu = {}
    fl = detail.get("cpu_baseline_flash_fwd_c4")
    if isinstance(fl, dict) and "value" in fl:
        cpu["flash_fwd_c4_gflops"] = fl["value"]
    ml = detail.get("cpu_baseline_runtime_mlp_c2_step")
    if isinstance(ml, dict) and "ms_per_step" in ml:
        cpu["runtime_mlp_c2_step_ms"] = ml["ms_per_step"]
    if cpu:
        out["cpu_other"] = cpu
    return out


if __name__ == "__main__":
    main()
