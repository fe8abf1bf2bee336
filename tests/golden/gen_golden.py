"""Write tests/golden/ref_vectors.npz from the reference runtime built from source.

Run in a container that has the reference tree (it builds oracle/_ref/ first):

    make -C oracle ref && python tests/golden/gen_golden.py

Every input is drawn by the reference's own RNG (set_seed + randn, elementwise.inc:35-54)
and every output comes from the reference builtins through their C ABI:
tensor_matmul (CPU dgemm / f32 fgemm), backward through "matmul", dream_attention,
dream_attention_causal, dream_flash_attention and their backward branches,
dream_softmax, dream_log_softmax, dream_layer_norm, dream_linear(_relu), dream_bmm,
dream_conv2d(_padded) and their backward branches, the elementwise builtins (tensor_add ...
dream_maximum, dream_pow, relu ... dream_round) and their backward branches,
dream_kaiming_init.  The file holds data
only (inputs and expected outputs, fp64).
"""
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
from _ref_runtime import BINARY as R_BINARY, UNARY as R_UNARY, RefRuntime  # noqa: E402

OUT = os.path.join(HERE, "ref_vectors.npz")


def main():
    R = RefRuntime()
    v = {}
    manifest = {}

    # RNG: set_seed(42); randn(4, 250) and set_seed(7); kaiming_init(16, 10).
    R.set_seed(42)
    v["rng_randn_s42"] = R.randn(4, 250)
    R.set_seed(7)
    v["rng_kaiming_s7_16x10"] = R.kaiming(16, 10)
    manifest["rng"] = "randn(4,250) after set_seed(42); kaiming_init(16,10) after set_seed(7)"

    # fp64 dgemm via tensor_matmul.  K=300 crosses the KC=256 slice; M*K*N >= 262144
    # takes the OpenMP branch.
    R.set_seed(20260707)
    for (M, K, N) in [(65, 63, 66), (33, 300, 35), (1, 7, 1), (5, 1, 9)]:
        A, B = R.randn(M, K), R.randn(K, N)
        key = f"gemm_d_{M}x{K}x{N}"
        v[key + "_A"], v[key + "_B"], v[key + "_C"] = A, B, R.matmul(A, B)
    manifest["gemm_d"] = "set_seed(20260707); per shape A=randn(M,K), B=randn(K,N); C=A@B (fp64)"

    # fp32 fgemm via `as f32` operands.
    for (M, K, N) in [(33, 31, 35), (40, 300, 37)]:
        A, B = R.randn(M, K), R.randn(K, N)
        key = f"gemm_f32_{M}x{K}x{N}"
        v[key + "_A"], v[key + "_B"], v[key + "_C"] = A, B, R.matmul(A, B, f32=True)
    manifest["gemm_f32"] = "continuing the stream: A,B randn; C = (A as f32) @ (B as f32)"

    # matmul backward with a random upstream gradient W: backward(sum((A@B) * W)).
    for (M, K, N) in [(65, 63, 66)]:
        A, B, W = R.randn(M, K), R.randn(K, N), R.randn(M, N)
        dA, dB = R.matmul_grads(A, B, W)
        key = f"mmbwd_{M}x{K}x{N}"
        v[key + "_A"], v[key + "_B"], v[key + "_W"] = A, B, W
        v[key + "_dA"], v[key + "_dB"] = dA, dB
    manifest["matmul_bwd"] = "A,B,W randn; dA,dB from backward(sum((A@B)*W))"

    # Attention family.  One slice, S=100 (ragged against Bc=16 forward and the
    # fixed Bc=64 backward), dk=24; plus S=64, dk=16, Bc=8.
    R.set_seed(20260709)
    for (B, S, dk, Bc) in [(1, 100, 24, 16), (2, 64, 16, 8)]:
        Q, K, V, W = (R.randn(B, S * dk) for _ in range(4))
        key = f"attn_B{B}_S{S}_dk{dk}_Bc{Bc}"
        v[key + "_Q"], v[key + "_K"], v[key + "_V"], v[key + "_W"] = Q, K, V, W
        for kind in ("plain", "causal", "flash"):
            v[f"{key}_{kind}_O"] = R.attention(kind, Q, K, V, B, S, dk, Bc)
            dQ, dK, dV = R.attention_grads(kind, Q, K, V, W, B, S, dk, Bc)
            v[f"{key}_{kind}_dQ"], v[f"{key}_{kind}_dK"], v[f"{key}_{kind}_dV"] = dQ, dK, dV
    manifest["attention"] = ("set_seed(20260709); Q,K,V,W = randn(B, S*dk); O from "
                             "attention / attention_causal / flash_attention(Bc); grads from "
                             "backward(sum(O*W))")

    R.set_seed(11)
    X = R.randn(7, 33)
    v["softmax_X"], v["softmax_Y"], v["log_softmax_Y"] = X, R.softmax(X), R.softmax(X, log=True)
    manifest["softmax"] = "set_seed(11); X=randn(7,33); softmax(X), log_softmax(X)"

    # Row ops, linear layers and bmm with their backward (upstream gradient W through
    # backward(sum(Y * W))).
    R.set_seed(13)
    G = R.randn(7, 33)
    v["softmax_G"] = G
    v["softmax_dX"] = R.softmax_grads(X, G)
    v["log_softmax_dX"] = R.softmax_grads(X, G, log=True)
    LX, LG = R.randn(6, 50) * 3.0 + 1.5, R.randn(6, 50)
    v["layer_norm_X"], v["layer_norm_G"] = LX, LG
    v["layer_norm_Y"], v["layer_norm_dX"] = R.layer_norm(LX), R.layer_norm_grads(LX, LG)
    manifest["rows"] = ("set_seed(13); G=randn(7,33) on softmax_X: dX of softmax / log_softmax; "
                        "layer_norm_X = 3*randn(6,50)+1.5, G=randn(6,50): Y and dX")
    LinX, LinW, Linb, LinG = R.randn(9, 13), R.randn(11, 13), R.randn(1, 11), R.randn(9, 11)
    v["linear_X"], v["linear_W"], v["linear_b"], v["linear_G"] = LinX, LinW, Linb, LinG
    for relu in (False, True):
        key = "linear_relu" if relu else "linear"
        v[key + "_Y"] = R.linear(LinX, LinW, Linb, relu)
        dX, dW, db, dY = R.linear_grads(LinX, LinW, Linb, LinG, relu)
        v[key + "_dX"], v[key + "_dW"], v[key + "_db"], v[key + "_dY"] = dX, dW, db, dY
    manifest["linear"] = ("X=randn(9,13), W=randn(11,13) (out x in), b=randn(1,11), "
                          "G=randn(9,11); Y of linear / linear_relu; dX, dW, db and the node's "
                          "own grad dY (ReLU-masked in place) after backward(sum(Y*G))")
    BA, BB, BG = R.randn(3, 5 * 7), R.randn(3, 7 * 6), R.randn(3, 5 * 6)
    v["bmm_A"], v["bmm_B"], v["bmm_G"] = BA, BB, BG
    v["bmm_C"] = R.bmm(BA, BB, 3, 5, 7, 6)
    v["bmm_dA"], v["bmm_dB"] = R.bmm(BA, BB, 3, 5, 7, 6, grads_W=BG)
    manifest["bmm"] = "A=randn(3,35), B=randn(3,42), G=randn(3,30); bmm(B=3,M=5,K=7,N=6), grads"

    # conv2d: N=2, Cin=3, H=7, W=6, Cout=4, KH=3, KW=2 (valid: OH=5, OW=5) with bias, and the
    # padded / strided forward (pad 1, stride 2: OH=4, OW=4).
    CX, CK, Cb = R.randn(2, 3 * 7 * 6), R.randn(4, 3 * 3 * 2), R.randn(1, 4)
    CG = R.randn(2, 4 * 5 * 5)
    v["conv_X"], v["conv_K"], v["conv_b"], v["conv_G"] = CX, CK, Cb, CG
    v["conv_Y"] = R.conv2d(CX, CK, Cb, 7, 6, 3, 2)
    v["conv_dX"], v["conv_dK"] = R.conv2d(CX, CK, Cb, 7, 6, 3, 2, G=CG)
    v["conv_padded_Y"] = R.conv2d(CX, CK, Cb, 7, 6, 3, 2, pad=1, stride=2)
    manifest["conv2d"] = ("X=randn(2,126) (N=2, Cin=3, 7x6), K=randn(4,18) (Cout=4, 3x2), "
                          "b=randn(1,4), G=randn(2,100); conv2d Y, dX, dK of backward(sum(Y*G)); "
                          "conv2d_padded(pad=1, stride=2) Y")

    # Elementwise builtins: every binary op on a same-shape, a row (1 x C), a column (R x 1)
    # and a scalar (1 x 1) right operand, with the backward of the ops that have one; every
    # unary op with its backward.  Half of E's entries copy X's so eq / ne see both answers.
    R.set_seed(17)
    EX, EY, EG = R.randn(6, 9), R.randn(6, 9), R.randn(6, 9)
    EY[:, ::2] = EX[:, ::2]
    rights = {"same": EY, "row": R.randn(1, 9), "col": R.randn(6, 1), "scalar": R.randn(1, 1)}
    v["ew_X"], v["ew_G"] = EX, EG
    for name, Bx in rights.items():
        v["ew_B_" + name] = Bx
    grad_ops = ("add", "sub", "mul", "div", "min", "max", "pow")
    for op in R_BINARY:
        for name, Bx in rights.items():
            A = np.abs(EX) + 0.25 if op == "pow" else EX
            key = f"ew_{op}_{name}"
            if op in grad_ops:
                v[key + "_C"], v[key + "_dA"], v[key + "_dB"] = R.binary(op, A, Bx, EG)
            else:
                v[key + "_C"] = R.binary(op, A, Bx)
    no_grad = ("lnot", "floor", "ceil", "round")
    for op in R_UNARY:
        A = np.abs(EX) + 0.1 if op in ("log", "sqrt") else EX * 3.0 if op in no_grad else EX
        key = f"ew_u_{op}"
        if op in no_grad:
            v[key + "_C"] = R.unary(op, A)
        else:
            v[key + "_C"], v[key + "_dA"] = R.unary(op, A, EG)
    manifest["elementwise"] = ("set_seed(17); X, Y, G = randn(6,9), Y[:, ::2] = X[:, ::2]; right "
                               "operands same=Y, row=randn(1,9), col=randn(6,1), "
                               "scalar=randn(1,1); C = op(X, B) (pow: |X|+0.25 as base), "
                               "dA/dB of backward(sum(C*G)); unary on X (log, sqrt: |X|+0.1; "
                               "lnot/floor/ceil/round: 3X) with dA")

    np.savez_compressed(OUT, **v)
    manifest["file"] = os.path.basename(OUT)
    manifest["arrays"] = {k: list(a.shape) for k, a in v.items()}
    with open(os.path.join(HERE, "manifest.json"), "w") as f:
        json.dump(manifest, f, indent=1, sort_keys=True)
    print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes, {len(v)} arrays)")


if __name__ == "__main__":
    main()
