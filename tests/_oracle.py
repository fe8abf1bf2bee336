"""ctypes wrapper around oracle/liboracle.so (the CPU restatement of the reference path).

Test infrastructure: imported only by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg.  Every function returns fresh numpy arrays and never touches the GPU.
"""
import ctypes
import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(ROOT, "oracle", "liboracle.so")

_dp = ctypes.POINTER(ctypes.c_double)
_fp = ctypes.POINTER(ctypes.c_float)
_u16p = ctypes.POINTER(ctypes.c_uint16)
_i = ctypes.c_int
_ll = ctypes.c_longlong
_ip = ctypes.POINTER(ctypes.c_int)

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise FileNotFoundError(f"{LIB_PATH} missing: run `make -C oracle`")
        L = ctypes.CDLL(LIB_PATH)
        sig = {
            "orc_set_seed": [ctypes.c_uint],
            "orc_randn": [_dp, _ll],
            "orc_uniform": [_dp, _ll, ctypes.c_double, ctypes.c_double],
            "orc_uniform_f32": [_fp, _ll, ctypes.c_float, ctypes.c_float],
            "orc_kaiming": [_dp, _i, _i],
            "orc_gemm_ref_d": [_dp, _dp, _dp, _i, _i, _i],
            "orc_gemm_d": [_dp, _dp, _dp, _i, _i, _i],
            "orc_gemm_f32": [_fp, _fp, _fp, _i, _i, _i],
            "orc_gemm_general_d": [_i, _i, _i, _i, _i, _dp, _i, _dp, _i, ctypes.c_double, _dp, _i],
            "orc_matmul_bwd": [_dp, _dp, _dp, _dp, _dp, _i, _i, _i],
            "orc_attention": [_dp, _dp, _dp, _dp, _i, _i, _i],
            "orc_attention_causal": [_dp, _dp, _dp, _dp, _i, _i, _i],
            "orc_flash_fwd": [_dp, _dp, _dp, _dp, _i, _i, _i, _i],
            "orc_attention_bwd": [_dp] * 7 + [_i, _i, _i, _i],
            "orc_flash_bwd": [_dp] * 7 + [_i, _i, _i],
            "orc_attention_rows": [_dp, _dp, _dp, _dp, _ip, _i, _dp, _dp, _i, _i, _i, _i],
            "orc_flash_lse": [_dp, _dp, _dp, _i, _i, _i, _i],
            "orc_softmax_rows": [_dp, _dp, _i, _i],
            "orc_log_softmax_rows": [_dp, _dp, _i, _i],
            "orc_softmax_bwd": [_dp, _dp, _dp, _i, _i],
            "orc_log_softmax_bwd": [_dp, _dp, _dp, _i, _i],
            "orc_layer_norm": [_dp, _dp, _i, _i],
            "orc_layer_norm_bwd": [_dp, _dp, _dp, _dp, _i, _i],
            "orc_linear": [_dp, _dp, _dp, _dp, _i, _i, _i, _i],
            "orc_linear_bwd": [_dp] * 7 + [_i, _i, _i, _i],
            "orc_bmm": [_dp, _dp, _dp, _i, _i, _i, _i],
            "orc_bmm_bwd": [_dp] * 5 + [_i, _i, _i, _i],
            "orc_conv2d": [_dp] * 4 + [_i] * 9,
            "orc_conv2d_bwd": [_dp] * 5 + [_i] * 9,
            "orc_binary": [_i, _dp, _ip, _dp, _ip, _dp, _ip],
            "orc_unary": [_i, _dp, _dp, _ll, ctypes.c_double, ctypes.c_double],
            "orc_binary_bwd": [_i, _dp, _ll, _dp, _ll, _dp, _dp, _ll, _dp, _dp],
            "orc_unary_bwd": [_i, _dp, _dp, _dp, _dp, _ll],
            "orc_to_bf16": [ctypes.c_float],
            "orc_bf16_bits": [_fp, _u16p, _ll],
        }
        for name, args in sig.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = None
        L.orc_to_bf16.restype = ctypes.c_float
        _lib = L
    return _lib


def _d(a):
    return np.ascontiguousarray(a, dtype=np.float64)


def _ptr(a, t=_dp):
    return a.ctypes.data_as(t)


# --- RNG ---------------------------------------------------------------------
def set_seed(seed):
    lib().orc_set_seed(int(seed))


def randn(*shape):
    out = np.empty(int(np.prod(shape)), np.float64)
    lib().orc_randn(_ptr(out), out.size)
    return out.reshape(shape)


def uniform(n, lo, hi):
    out = np.empty(int(n), np.float64)
    lib().orc_uniform(_ptr(out), out.size, lo, hi)
    return out


def uniform_f32(n, lo, hi):
    out = np.empty(int(n), np.float32)
    lib().orc_uniform_f32(_ptr(out, _fp), out.size, lo, hi)
    return out


def kaiming(rows, cols):
    out = np.empty((rows, cols), np.float64)
    lib().orc_kaiming(_ptr(out), rows, cols)
    return out


# --- GEMM ----------------------------------------------------------------------
def gemm_ref_d(A, B):
    A, B = _d(A), _d(B)
    M, K = A.shape
    N = B.shape[1]
    C = np.empty((M, N), np.float64)
    lib().orc_gemm_ref_d(_ptr(A), _ptr(B), _ptr(C), M, K, N)
    return C


def gemm_d(A, B):
    A, B = _d(A), _d(B)
    M, K = A.shape
    N = B.shape[1]
    C = np.empty((M, N), np.float64)
    lib().orc_gemm_d(_ptr(A), _ptr(B), _ptr(C), M, K, N)
    return C


def gemm_f32(A, B):
    A = np.ascontiguousarray(A, np.float32)
    B = np.ascontiguousarray(B, np.float32)
    M, K = A.shape
    N = B.shape[1]
    C = np.empty((M, N), np.float32)
    lib().orc_gemm_f32(_ptr(A, _fp), _ptr(B, _fp), _ptr(C, _fp), M, K, N)
    return C


def gemm_general_d(transA, transB, A, B, beta=0.0, C=None):
    """C = op(A) @ op(B) + beta*C in fp64; A/B given in their stored layout."""
    A, B = _d(A), _d(B)
    M = A.shape[1] if transA else A.shape[0]
    K = A.shape[0] if transA else A.shape[1]
    N = B.shape[0] if transB else B.shape[1]
    out = np.zeros((M, N), np.float64) if C is None else _d(C).copy()
    lib().orc_gemm_general_d(int(transA), int(transB), M, N, K, _ptr(A), A.shape[1],
                             _ptr(B), B.shape[1], float(beta), _ptr(out), N)
    return out


def matmul_bwd(A, B, dY, dA=None, dB=None):
    A, B, dY = _d(A), _d(B), _d(dY)
    M, K = A.shape
    N = B.shape[1]
    dA = np.zeros((M, K)) if dA is None else _d(dA).copy()
    dB = np.zeros((K, N)) if dB is None else _d(dB).copy()
    lib().orc_matmul_bwd(_ptr(A), _ptr(B), _ptr(dY), _ptr(dA), _ptr(dB), M, K, N)
    return dA, dB


# --- attention (layout (B, S*dk)) ----------------------------------------------
def _qkv(Q, K, V):
    return _d(Q), _d(K), _d(V)


def attention(Q, K, V, B, S, dk, causal):
    Q, K, V = _qkv(Q, K, V)
    O = np.empty_like(Q)
    fn = lib().orc_attention_causal if causal else lib().orc_attention
    fn(_ptr(Q), _ptr(K), _ptr(V), _ptr(O), B, S, dk)
    return O


def flash_fwd(Q, K, V, B, S, dk, Bc=64):
    Q, K, V = _qkv(Q, K, V)
    O = np.empty_like(Q)
    lib().orc_flash_fwd(_ptr(Q), _ptr(K), _ptr(V), _ptr(O), B, S, dk, Bc)
    return O


def attention_bwd(Q, K, V, dO, B, S, dk, causal):
    Q, K, V = _qkv(Q, K, V)
    dO = _d(dO)
    dQ, dK, dV = np.zeros_like(Q), np.zeros_like(Q), np.zeros_like(Q)
    lib().orc_attention_bwd(_ptr(Q), _ptr(K), _ptr(V), _ptr(dO), _ptr(dQ), _ptr(dK), _ptr(dV),
                            B, S, dk, int(causal))
    return dQ, dK, dV


def attention_rows(Q, K, V, dO, rows, B, S, dk, causal):
    """O and dQ of the query rows rows[b] (an int array of shape (B, n)) of every slice:
    returns two (B, n, dk) arrays."""
    Q, K, V = _qkv(Q, K, V)
    dO = _d(dO)
    rows = np.ascontiguousarray(rows, np.int32)
    n = rows.shape[1]
    Orow, dQrow = np.zeros((B, n, dk)), np.zeros((B, n, dk))
    lib().orc_attention_rows(_ptr(Q), _ptr(K), _ptr(V), _ptr(dO),
                             rows.ctypes.data_as(_ip), n, _ptr(Orow), _ptr(dQrow), B, S, dk,
                             int(causal))
    return Orow, dQrow


def flash_bwd(Q, K, V, dO, B, S, dk):
    Q, K, V = _qkv(Q, K, V)
    dO = _d(dO)
    dQ, dK, dV = np.zeros_like(Q), np.zeros_like(Q), np.zeros_like(Q)
    lib().orc_flash_bwd(_ptr(Q), _ptr(K), _ptr(V), _ptr(dO), _ptr(dQ), _ptr(dK), _ptr(dV),
                        B, S, dk)
    return dQ, dK, dV


def flash_lse(Q, K, B, S, dk, causal=True):
    Q, K = _d(Q), _d(K)
    lse = np.empty(B * S, np.float64)
    lib().orc_flash_lse(_ptr(Q), _ptr(K), _ptr(lse), B, S, dk, int(causal))
    return lse.reshape(B, S)


# --- row reductions / bf16 -----------------------------------------------------
def softmax_rows(X):
    X = _d(X)
    Y = np.empty_like(X)
    lib().orc_softmax_rows(_ptr(X), _ptr(Y), X.shape[0], X.size // X.shape[0])
    return Y


def log_softmax_rows(X):
    X = _d(X)
    Y = np.empty_like(X)
    lib().orc_log_softmax_rows(_ptr(X), _ptr(Y), X.shape[0], X.size // X.shape[0])
    return Y


def _rows(X):
    R = X.shape[0] if X.ndim > 1 else 1
    return R, X.size // R


def softmax_bwd(Y, G, GX=None):
    """gx += y (g - sum(g y)) per row (softmax backward from its output)."""
    Y, G = _d(Y), _d(G)
    GX = np.zeros_like(Y) if GX is None else _d(GX).copy()
    lib().orc_softmax_bwd(_ptr(Y), _ptr(G), _ptr(GX), *_rows(Y))
    return GX


def log_softmax_bwd(X, G, GX=None):
    """gx += g - softmax(x) sum(g) per row (log_softmax backward from its input)."""
    X, G = _d(X), _d(G)
    GX = np.zeros_like(X) if GX is None else _d(GX).copy()
    lib().orc_log_softmax_bwd(_ptr(X), _ptr(G), _ptr(GX), *_rows(X))
    return GX


def layer_norm(X):
    X = _d(X)
    Y = np.empty_like(X)
    lib().orc_layer_norm(_ptr(X), _ptr(Y), *_rows(X))
    return Y


def layer_norm_bwd(X, Y, DY, GX=None):
    X, Y, DY = _d(X), _d(Y), _d(DY)
    GX = np.zeros_like(X) if GX is None else _d(GX).copy()
    lib().orc_layer_norm_bwd(_ptr(X), _ptr(Y), _ptr(DY), _ptr(GX), *_rows(X))
    return GX


def linear(X, W, b, relu=False):
    """Y = X W^T + b (W is out x in), optionally ReLU."""
    X, W, b = _d(X), _d(W), _d(b).ravel()
    Y = np.empty((X.shape[0], W.shape[0]), np.float64)
    lib().orc_linear(_ptr(X), _ptr(W), _ptr(b), _ptr(Y), X.shape[0], X.shape[1], W.shape[0],
                     int(relu))
    return Y


def linear_bwd(X, W, Y, dY, relu=False):
    """Returns (dY after the ReLU mask, dX, dW, db), accumulated from zero."""
    X, W, Y = _d(X), _d(W), _d(Y)
    dY = _d(dY).copy()
    dX, dW, db = np.zeros_like(X), np.zeros_like(W), np.zeros(W.shape[0], np.float64)
    lib().orc_linear_bwd(_ptr(X), _ptr(W), _ptr(Y), _ptr(dY), _ptr(dX), _ptr(dW), _ptr(db),
                         X.shape[0], X.shape[1], W.shape[0], int(relu))
    return dY, dX, dW, db


def bmm(A, B, Bt, M, K, N):
    A, B = _d(A), _d(B)
    C = np.empty((Bt, M * N), np.float64)
    lib().orc_bmm(_ptr(A), _ptr(B), _ptr(C), Bt, M, K, N)
    return C


def bmm_bwd(A, B, G, Bt, M, K, N):
    A, B, G = _d(A), _d(B), _d(G)
    gA, gB = np.zeros((Bt, M * K), np.float64), np.zeros((Bt, K * N), np.float64)
    lib().orc_bmm_bwd(_ptr(A), _ptr(B), _ptr(G), _ptr(gA), _ptr(gB), Bt, M, K, N)
    return gA, gB


def conv_out(H, W, KH, KW, pad=0, stride=1):
    return (H + 2 * pad - KH) // stride + 1, (W + 2 * pad - KW) // stride + 1


def conv2d(X, Kn, bias, N, Cin, H, W, Cout, KH, KW, pad=0, stride=1):
    """X (N, Cin*H*W), Kn (Cout, Cin*KH*KW), bias (Cout) or None -> (N, Cout*OH*OW)."""
    OH, OW = conv_out(H, W, KH, KW, pad, stride)
    X, Kn = _d(X), _d(Kn)
    b = None if bias is None else _d(bias).ravel()
    Y = np.empty((N, Cout * OH * OW), np.float64)
    lib().orc_conv2d(_ptr(X), _ptr(Kn), None if b is None else _ptr(b), _ptr(Y), N, Cin, H, W,
                     Cout, KH, KW, pad, stride)
    return Y


def conv2d_bwd(X, Kn, G, N, Cin, H, W, Cout, KH, KW, pad=0, stride=1):
    X, Kn, G = _d(X), _d(Kn), _d(G)
    gX, gK = np.zeros_like(X), np.zeros_like(Kn)
    lib().orc_conv2d_bwd(_ptr(X), _ptr(Kn), _ptr(G), _ptr(gX), _ptr(gK), N, Cin, H, W, Cout, KH,
                         KW, pad, stride)
    return gX, gK


# Elementwise op codes: the reference's BinopCode / UnopCode order (gpu.inc:455-460, 571-577).
BINOPS = ["add", "sub", "mul", "div", "mod", "gt", "lt", "ge", "le", "eq", "ne", "and", "or",
          "atan2", "pow", "min", "max"]
UNOPS = ["relu", "exp", "log", "sqrt", "abs", "sigmoid", "tanh", "lnot", "sin", "cos", "tan",
         "atan", "floor", "ceil", "round", "clip"]


def dims4(shape):
    """A Dream tensor's (d0, d1, d2, d3) for a numpy shape of up to 4 dims."""
    d = list(shape) + [1] * (4 - len(shape))
    return np.array(d, np.int32)


def _code(op, table):
    return op if isinstance(op, (int, np.integer)) else table.index(op)


def binary(op, A, B, c_shape=None):
    """runCPUBinary on Dream shapes: C's dims are the per-dim max of A's and B's."""
    A, B = _d(A), _d(B)
    ad, bd = dims4(A.shape), dims4(B.shape)
    cd = np.maximum(ad, bd).astype(np.int32) if c_shape is None else dims4(c_shape)
    C = np.empty(int(np.prod(cd)), np.float64)
    lib().orc_binary(_code(op, BINOPS), _ptr(A), _ptr(ad, _ip), _ptr(B), _ptr(bd, _ip), _ptr(C),
                     _ptr(cd, _ip))
    return C.reshape([int(x) for x in cd])


def unary(op, A, lo=0.0, hi=0.0):
    A = _d(A)
    C = np.empty_like(A)
    lib().orc_unary(_code(op, UNOPS), _ptr(A), _ptr(C), A.size, lo, hi)
    return C


def binary_bwd(op, A, B, Y, G):
    """(gA, gB) of the reference's backward branch for one node (fresh zero accumulators)."""
    A, B, Y, G = _d(A), _d(B), _d(Y), _d(G)
    gA, gB = np.zeros_like(A), np.zeros_like(B)
    lib().orc_binary_bwd(_code(op, BINOPS), _ptr(A), A.size, _ptr(B), B.size, _ptr(Y), _ptr(G),
                         G.size, _ptr(gA), _ptr(gB))
    return gA, gB


def unary_bwd(op, X, Y, G):
    X, Y, G = _d(X), _d(Y), _d(G)
    GX = np.zeros_like(X)
    lib().orc_unary_bwd(_code(op, UNOPS), _ptr(X), _ptr(Y), _ptr(G), _ptr(GX), X.size)
    return GX


def to_bf16(x):
    return lib().orc_to_bf16(float(x))


def bf16_bits(x):
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().orc_bf16_bits(_ptr(x, _fp), _ptr(out, _u16p), x.size)
    return out


def bf16_round(x):
    """fp32 values rounded to bf16 (returned as fp32) by the reference's rule."""
    bits = bf16_bits(x).astype(np.uint32) << 16
    return bits.view(np.float32)
