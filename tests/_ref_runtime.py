"""ctypes driver for the reference runtime built from source into oracle/_ref/.

Test infrastructure.  The reference's builtins are extern "C" and take/return
`Tensor*`; only the IR-visible fields 0-6 (data, grad, size, d0..d3) are read
here, exactly what compiled .dream programs read (runtime/runtime.h:49-55).
Used to write tests/golden/ fixtures and to cross-check the oracle where the
reference build is present.  The GPU box has no reference tree; tests that need
this driver skip when the library is missing.
"""
import ctypes
import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(ROOT, "oracle", "_ref", "libdreamref.so")


class _TensorHead(ctypes.Structure):
    _fields_ = [
        ("data", ctypes.POINTER(ctypes.c_double)),
        ("grad", ctypes.POINTER(ctypes.c_double)),
        ("size", ctypes.c_int),
        ("d0", ctypes.c_int),
        ("d1", ctypes.c_int),
        ("d2", ctypes.c_int),
        ("d3", ctypes.c_int),
    ]


_TP = ctypes.POINTER(_TensorHead)


# Elementwise builtins by op name (elementwise.inc:290-311, 320-327; math_extra.inc:1-10;
# builtins.inc:85-87; dream_pow, elementwise.inc:1254).
BINARY = {"add": "tensor_add", "sub": "tensor_sub", "mul": "tensor_mul", "div": "tensor_div",
          "mod": "tensor_mod", "gt": "tensor_gt", "lt": "tensor_lt", "ge": "tensor_ge",
          "le": "tensor_le", "eq": "tensor_eq", "ne": "tensor_ne", "and": "tensor_and",
          "or": "tensor_or", "atan2": "dream_atan2", "pow": "dream_pow", "min": "dream_minimum",
          "max": "dream_maximum"}
UNARY = {"relu": "relu", "exp": "dream_exp", "log": "dream_log", "sqrt": "dream_sqrt",
         "abs": "dream_abs", "sigmoid": "dream_sigmoid", "tanh": "dream_tanh",
         "lnot": "dream_logical_not", "sin": "dream_sin", "cos": "dream_cos", "tan": "dream_tan",
         "atan": "dream_atan", "floor": "dream_floor", "ceil": "dream_ceil",
         "round": "dream_round"}


def available():
    return os.path.exists(LIB_PATH)


class RefRuntime:
    def __init__(self, path=LIB_PATH):
        L = ctypes.CDLL(path)
        for name, nargs in [("alloc_tensor", None), ("create_scalar", None),
                            ("tensor_matmul", 2), ("tensor_mul", 2), ("sum", 1),
                            ("backward", 1), ("dream_flash_attention", 7),
                            ("dream_attention", 6), ("dream_attention_causal", 6),
                            ("dream_softmax", 1), ("dream_log_softmax", 1),
                            ("dream_layer_norm", 1), ("dream_linear", 3),
                            ("dream_linear_relu", 3), ("dream_bmm", 6),
                            ("dream_set_seed", 1), ("dream_randn", 2), ("dream_dropout", 2),
                            ("tensor_get_grad", 1),
                            ("dream_kaiming_init", 2), ("gemm_selftest", 0),
                            ("flash_attention_selftest", 0), ("tensor_decref", 1),
                            ("zero_grad", 1), ("dream_conv2d", 7),
                            ("dream_conv2d_padded", 9), ("dream_clip", 3),
                            *[(n, 2) for n in BINARY.values()],
                            *[(n, 1) for n in UNARY.values()]]:
            fn = getattr(L, name)
            fn.restype = _TP
            if nargs is not None:
                fn.argtypes = [_TP] * nargs
        L.alloc_tensor.argtypes = [ctypes.c_int] * 4
        L.create_scalar.argtypes = [ctypes.c_double]
        L.dream_set_precision.restype = _TP
        L.dream_set_precision.argtypes = [_TP, ctypes.c_int]
        self.L = L

    # -- tensors -------------------------------------------------------------
    def tensor(self, arr):
        arr = np.ascontiguousarray(arr, np.float64)
        d0, d1 = (arr.shape + (1,))[:2] if arr.ndim == 1 else arr.shape[:2]
        if arr.ndim == 1:
            d0, d1 = 1, arr.shape[0]
        t = self.L.alloc_tensor(int(d0), int(d1), 1, 1)
        ctypes.memmove(t.contents.data, arr.ctypes.data, arr.nbytes)
        return t

    def scalar(self, v):
        return self.L.create_scalar(float(v))

    @staticmethod
    def read(t, grad=False):
        h = t.contents
        ptr = h.grad if grad else h.data
        out = np.ctypeslib.as_array(ptr, shape=(h.size,)).copy()
        return out.reshape(h.d0, h.size // max(h.d0, 1))

    # -- builtins ------------------------------------------------------------
    def set_seed(self, s):
        self.L.dream_set_seed(self.scalar(s))

    def randn(self, r, c):
        return self.read(self.L.dream_randn(self.scalar(r), self.scalar(c)))

    def kaiming(self, r, c):
        return self.read(self.L.dream_kaiming_init(self.scalar(r), self.scalar(c)))

    def matmul(self, A, B, f32=False):
        a, b = self.tensor(A), self.tensor(B)
        if f32:
            self.L.dream_set_precision(a, 1)
            self.L.dream_set_precision(b, 1)
        return self.read(self.L.tensor_matmul(a, b))

    def matmul_grads(self, A, B, W):
        """backward(sum(A@B * W)) -> (A.grad, B.grad); the matmul node sees dY = W."""
        a, b, w = self.tensor(A), self.tensor(B), self.tensor(W)
        y = self.L.tensor_matmul(a, b)
        self.L.backward(self.L.sum(self.L.tensor_mul(y, w)))
        return self.read(a, grad=True), self.read(b, grad=True)

    def _attn(self, kind, Q, K, V, B, S, dk, Bc):
        q, k, v = self.tensor(Q), self.tensor(K), self.tensor(V)
        sc = [self.scalar(B), self.scalar(S), self.scalar(dk)]
        if kind == "flash":
            o = self.L.dream_flash_attention(q, k, v, *sc, self.scalar(Bc))
        elif kind == "causal":
            o = self.L.dream_attention_causal(q, k, v, *sc)
        else:
            o = self.L.dream_attention(q, k, v, *sc)
        return (q, k, v), o

    def attention(self, kind, Q, K, V, B, S, dk, Bc=64):
        return self.read(self._attn(kind, Q, K, V, B, S, dk, Bc)[1])

    def attention_grads(self, kind, Q, K, V, W, B, S, dk, Bc=64):
        """backward(sum(O * W)) -> (dQ, dK, dV) through the named attention node."""
        (q, k, v), o = self._attn(kind, Q, K, V, B, S, dk, Bc)
        w = self.tensor(W)
        self.L.backward(self.L.sum(self.L.tensor_mul(o, w)))
        return tuple(self.read(t, grad=True) for t in (q, k, v))

    def softmax(self, X, log=False):
        fn = self.L.dream_log_softmax if log else self.L.dream_softmax
        return self.read(fn(self.tensor(X)))

    def _grads(self, out, W, *ins):
        """backward(sum(out * W)) -> the .grad of each input tensor and of out."""
        w = self.tensor(W)
        self.L.backward(self.L.sum(self.L.tensor_mul(out, w)))
        return tuple(self.read(t, grad=True) for t in ins) + (self.read(out, grad=True),)

    def softmax_grads(self, X, W, log=False):
        x = self.tensor(X)
        y = (self.L.dream_log_softmax if log else self.L.dream_softmax)(x)
        return self._grads(y, W, x)[0]

    def layer_norm(self, X):
        return self.read(self.L.dream_layer_norm(self.tensor(X)))

    def layer_norm_grads(self, X, W):
        x = self.tensor(X)
        return self._grads(self.L.dream_layer_norm(x), W, x)[0]

    def linear(self, X, Wt, b, relu=False):
        fn = self.L.dream_linear_relu if relu else self.L.dream_linear
        return self.read(fn(self.tensor(X), self.tensor(Wt), self.tensor(b)))

    def linear_grads(self, X, Wt, b, G, relu=False):
        """(dX, dW, db, dY of the node after backward) for backward(sum(Y * G))."""
        fn = self.L.dream_linear_relu if relu else self.L.dream_linear
        x, w, bb = self.tensor(X), self.tensor(Wt), self.tensor(b)
        return self._grads(fn(x, w, bb), G, x, w, bb)

    def bmm(self, A, B, Bt, M, K, N, grads_W=None):
        a, b = self.tensor(A), self.tensor(B)
        c = self.L.dream_bmm(a, b, *(self.scalar(v) for v in (Bt, M, K, N)))
        if grads_W is None:
            return self.read(c)
        return self._grads(c, grads_W, a, b)[:2]

    def conv2d(self, X, Kn, bias, H, W, KH, KW, G=None, pad=None, stride=None):
        """dream_conv2d (or dream_conv2d_padded when pad/stride are given); with G also the
        gradients (dX, dK) of backward(sum(Y * G))."""
        x, k = self.tensor(X), self.tensor(Kn)
        b = self.tensor(bias) if bias is not None else None
        sc = [self.scalar(v) for v in (H, W, KH, KW)]
        if pad is None:
            y = self.L.dream_conv2d(x, k, b, *sc)
        else:
            y = self.L.dream_conv2d_padded(x, k, b, *sc, self.scalar(pad), self.scalar(stride))
        if G is None:
            return self.read(y)
        return self._grads(y, G, x, k)[:2]

    def binary(self, op, A, B, W=None):
        """The builtin's output for 2-D A, B; with W also (A.grad, B.grad) of
        backward(sum(C * W))."""
        a, b = self.tensor(A), self.tensor(B)
        c = getattr(self.L, BINARY[op])(a, b)
        if W is None:
            return self.read(c)
        return self.read(c), *self._grads(c, W, a, b)[:2]

    def unary(self, op, A, W=None):
        a = self.tensor(A)
        c = getattr(self.L, UNARY[op])(a)
        if W is None:
            return self.read(c)
        return self.read(c), self._grads(c, W, a)[0]

    def clip(self, A, lo, hi):
        return self.read(self.L.dream_clip(self.tensor(A), self.scalar(lo), self.scalar(hi)))
