"""ctypes binding of libdream_rt.so (include/dream_rt.h): the Dream builtins of the hot path.

Only the IR-visible Tensor fields 0-6 (data, grad, size, d0..d3) are read from Python,
exactly what compiled .dream programs read.  Every builtin returns a +1 reference; the
helpers here release what they create.
"""
import ctypes
import os

import numpy as np

from . import hip

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "lib", "libdream_rt.so")


class TensorHead(ctypes.Structure):
    _fields_ = [("data", ctypes.POINTER(ctypes.c_double)),
                ("grad", ctypes.POINTER(ctypes.c_double)),
                ("size", ctypes.c_int), ("d0", ctypes.c_int), ("d1", ctypes.c_int),
                ("d2", ctypes.c_int), ("d3", ctypes.c_int)]


TP = ctypes.POINTER(TensorHead)
_SIGS = {
    "alloc_tensor": [ctypes.c_int] * 4, "create_scalar": [ctypes.c_double],
    "tensor_incref": [TP], "tensor_decref": [TP], "ones": [TP, TP],
    "dream_set_seed": [TP], "dream_randn": [TP, TP], "sum": [TP], "dream_dropout": [TP, TP],
    "tensor_add": [TP, TP], "tensor_mul": [TP, TP], "tensor_get_grad": [TP],
    "zero_grad": [TP], "dream_set_precision": [TP, ctypes.c_int], "dream_to_float32": [TP],
    "dream_enable_fp16": [], "dream_disable_fp16": [], "tensor_matmul": [TP, TP],
    "dream_flash_attention": [TP] * 7, "dream_attention": [TP] * 6,
    "dream_attention_causal": [TP] * 6, "backward": [TP], "gpu_selftest": [],
    "dream_gpu_warmup": [], "flash_attention_selftest": [], "gemm_selftest": [],
    "bf16_selftest": [],
    "dream_linear": [TP] * 3, "dream_linear_relu": [TP] * 3, "linear": [TP] * 3,
    "linear_relu": [TP] * 3, "dream_bmm": [TP] * 6, "dream_softmax": [TP],
    "dream_log_softmax": [TP], "dream_layer_norm": [TP], "tensor_set_element": [TP] * 3,
    "tensor_set_element_2d": [TP] * 4, "dream_conv2d": [TP] * 7, "dream_conv2d_padded": [TP] * 9,
    "dream_clip": [TP] * 3,
}
# Elementwise builtins by op name (include/dream_rt.h).
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
_SIGS.update({n: [TP, TP] for n in BINARY.values()})
_SIGS.update({n: [TP] for n in UNARY.values()})

_lib = None


def load():
    global _lib
    if _lib is None:
        hip.load()   # the backend first, so its failure message is the one raised
        if not os.path.exists(LIB_PATH):
            raise hip.DreamHipError(f"{LIB_PATH} is missing: run `python -m dreamcompiler_amd.build`")
        L = ctypes.CDLL(LIB_PATH)
        for name, args in _SIGS.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = TP
        L.dream_gpu_available.restype = ctypes.c_int
        L.dream_hip_available.restype = ctypes.c_int
        _lib = L
    return _lib


def tensor(arr):
    """New runtime tensor holding a copy of a 1-D or 2-D array (fp64)."""
    arr = np.ascontiguousarray(arr, np.float64)
    if arr.ndim == 1:
        arr = arr[None, :]
    t = load().alloc_tensor(arr.shape[0], arr.shape[1], 1, 1)
    ctypes.memmove(t.contents.data, arr.ctypes.data, arr.nbytes)
    return t


def scalar(v):
    return load().create_scalar(float(v))


def read(t, grad=False):
    h = t.contents
    ptr = h.grad if grad else h.data
    out = np.ctypeslib.as_array(ptr, shape=(h.size,)).copy()
    return out.reshape(h.d0, h.size // max(h.d0, 1))


def release(*ts):
    for t in ts:
        if t:
            load().tensor_decref(t)
