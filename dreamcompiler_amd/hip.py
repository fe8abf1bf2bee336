"""ctypes binding of libdream_hip.so (include/dream_hip.h) plus a small device-buffer type.

The product path: every call goes to the HIP library.  There is no CPU fallback;
if the library is missing or no GPU is usable the calls raise.
"""
import ctypes
import os

import numpy as np

PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG, "lib", "libdream_hip.so")

DH_OK, DH_ERR_NO_DEVICE, DH_ERR_INVALID, DH_ERR_OOM, DH_ERR_HIP, DH_ERR_UNSUPPORTED = range(6)
F32, BF16, F64 = 0, 1, 2
_DT = {np.dtype(np.float32): F32, np.dtype(np.uint16): BF16, np.dtype(np.float64): F64}

_vp = ctypes.c_void_p
_i = ctypes.c_int
_f = ctypes.c_float
_sz = ctypes.c_size_t
_ll = ctypes.c_longlong
_d = ctypes.c_double

# name: (restype, argtypes) -- mirrors include/dream_hip.h
_SIGS = {
    "dh_init": (_i, []),
    "dh_available": (_i, []),
    "dh_device_info": (_i, [ctypes.c_char_p, _i, ctypes.POINTER(_i), ctypes.POINTER(_i),
                            ctypes.POINTER(_i), ctypes.POINTER(ctypes.c_longlong)]),
    "dh_last_error": (ctypes.c_char_p, []),
    "dh_dispatch_threshold": (_sz, []),
    "dh_matmul_eligible": (_i, [_i, _i]),
    "dh_flash_eligible": (_i, [_i, _i, _i]),
    "dh_malloc": (_vp, [_sz]),
    "dh_free": (_i, [_vp]),
    "dh_pool_release": (_i, []),
    "dh_host_alloc": (_vp, [_sz]),
    "dh_host_free": (_i, [_vp]),
    "dh_memcpy_h2d": (_i, [_vp, _vp, _sz]),
    "dh_memcpy_d2h": (_i, [_vp, _vp, _sz]),
    "dh_memcpy_d2h_async": (_i, [_vp, _vp, _sz]),
    "dh_event_create": (_vp, []),
    "dh_event_record": (_i, [_vp]),
    "dh_event_wait": (_i, [_vp]),
    "dh_event_destroy": (_i, [_vp]),
    "dh_memcpy_d2d": (_i, [_vp, _vp, _sz]),
    "dh_memset": (_i, [_vp, _i, _sz]),
    "dh_sync": (_i, []),
    "dh_get_stream": (_vp, []),
    "dh_set_stream": (_i, [_vp]),
    "dh_timer_start": (_i, []),
    "dh_timer_stop": (_i, [ctypes.POINTER(_f)]),
    "dh_convert": (_i, [_vp, _i, _vp, _i, _sz]),
    "dh_axpy": (_i, [_vp, _vp, _f, _sz]),
    "dh_gemm_f32": (_i, [_i, _i, _i, _i, _i, _vp, _i, _vp, _i, _f, _vp, _i]),
    "dh_gemm_bf16": (_i, [_i, _i, _i, _i, _i, _vp, _i, _vp, _i, _f, _vp, _i]),
    "dh_gemm_f32_ex": (_i, [_i, _i, _i, _i, _i, _vp, _i, _ll, _vp, _i, _ll, _f, _vp, _i, _ll,
                            _i, _vp, _i]),
    "dh_gemm_bf16_ex": (_i, [_i, _i, _i, _i, _i, _vp, _i, _ll, _vp, _i, _ll, _f, _vp, _i, _ll,
                             _i, _vp, _i]),
    "dh_gemm_f64": (_i, [_i, _i, _i, _i, _i, _vp, _i, _vp, _i, _d, _vp, _i]),
    "dh_gemm_f64_ex": (_i, [_i, _i, _i, _i, _i, _d, _vp, _i, _ll, _vp, _i, _ll, _d, _vp, _i, _ll,
                            _i]),
    "dh_attention_f64_fwd": (_i, [_i, _i, _i, _d, _i, _vp, _vp, _vp, _vp]),
    "dh_attention_f64_bwd": (_i, [_i, _i, _i, _d, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i]),
    "dh_flash_fwd": (_i, [_i, _i, _i, _i, _f, _i, _vp, _vp, _vp, _vp, _vp]),
    "dh_flash_bwd": (_i, [_i, _i, _i, _i, _f, _i, _vp, _vp, _vp, _vp, _vp, _vp,
                          _vp, _vp, _vp, _i]),
    "dh_flash_bwd_noalloc": (_i, [_i, _i, _i, _i, _f, _i, _vp, _vp, _vp, _vp, _vp, _vp,
                                  _vp, _vp, _vp, _i]),
    "dh_row_softmax": (_i, [_vp, _vp, _i, _i, _i]),
    "dh_row_softmax_bwd": (_i, [_vp, _vp, _vp, _i, _i, _i, _i]),
    "dh_layer_norm": (_i, [_vp, _vp, _i, _i]),
    "dh_layer_norm_bwd": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i]),
    "dh_linear_bias_grad": (_i, [_vp, _vp, _vp, _i, _i, _i, _i]),
    "dh_im2col": (_i, [_vp, _vp] + [_i] * 8),
    "dh_col2im": (_i, [_vp, _vp] + [_i] * 9),
    "dh_nct_to_cnt": (_i, [_vp, _vp, _i, _i, _sz]),
    "dh_conv2d_fwd": (_i, [_vp, _vp, _vp, _vp] + [_i] * 9),
    "dh_conv2d_bwd_data": (_i, [_vp, _vp, _vp] + [_i] * 10),
    "dh_conv2d_bwd_filter": (_i, [_vp, _vp, _vp] + [_i] * 10),
    "dh_binary": (_i, [_i, _i, _vp, _sz, ctypes.POINTER(_i), _vp, _sz, ctypes.POINTER(_i), _vp,
                       ctypes.POINTER(_i), _vp]),
    "dh_unary": (_i, [_i, _i, _vp, _vp, _sz, ctypes.c_double, ctypes.c_double, _vp]),
}

EXPORTED = tuple(_SIGS)
_lib = None


class DreamHipError(RuntimeError):
    pass


def load():
    """Load libdream_hip.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise DreamHipError(
                f"{LIB_PATH} is missing: build it with `python -m dreamcompiler_amd.build`")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(status, what="dream_hip"):
    if status != DH_OK:
        msg = load().dh_last_error().decode(errors="replace")
        raise DreamHipError(f"{what} failed with status {status}: {msg}")


def available():
    return load().dh_available() == 1


def device_info():
    L = load()
    name = ctypes.create_string_buffer(256)
    cus, xcds, clk = _i(), _i(), _i()
    hbm = ctypes.c_longlong()
    check(L.dh_device_info(name, 256, ctypes.byref(cus), ctypes.byref(xcds),
                           ctypes.byref(clk), ctypes.byref(hbm)), "dh_device_info")
    return {"name": name.value.decode(), "cus": cus.value, "xcds": xcds.value,
            "sclk_mhz": clk.value, "hbm_bytes": hbm.value}


def sync():
    check(load().dh_sync(), "dh_sync")


class DeviceBuffer:
    """A device allocation from the library pool, with numpy upload/download."""

    def __init__(self, nbytes):
        self.nbytes = int(nbytes)
        self.ptr = load().dh_malloc(max(self.nbytes, 1))
        if not self.ptr:
            check(DH_ERR_OOM, f"dh_malloc({self.nbytes})")

    @classmethod
    def from_numpy(cls, arr):
        arr = np.ascontiguousarray(arr)
        buf = cls(arr.nbytes)
        buf.dtype, buf.shape = arr.dtype, arr.shape
        check(load().dh_memcpy_h2d(buf.ptr, arr.ctypes.data, arr.nbytes), "dh_memcpy_h2d")
        sync()
        return buf

    @classmethod
    def empty(cls, shape, dtype):
        dtype = np.dtype(dtype)
        buf = cls(int(np.prod(shape)) * dtype.itemsize)
        buf.dtype, buf.shape = dtype, tuple(shape)
        return buf

    def numpy(self, shape=None, dtype=None):
        dtype = np.dtype(dtype or self.dtype)
        shape = tuple(shape or self.shape)
        out = np.empty(shape, dtype)
        assert out.nbytes <= self.nbytes
        check(load().dh_memcpy_d2h(out.ctypes.data, self.ptr, out.nbytes), "dh_memcpy_d2h")
        return out

    def fill_zero(self):
        check(load().dh_memset(self.ptr, 0, self.nbytes), "dh_memset")

    def free(self):
        if self.ptr:
            load().dh_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def _p(x):
    return x.ptr if isinstance(x, DeviceBuffer) else x


def convert(dst, dst_type, src, src_type, n):
    check(load().dh_convert(_p(dst), dst_type, _p(src), src_type, int(n)), "dh_convert")


def axpy(y, x, alpha, n):
    check(load().dh_axpy(_p(y), _p(x), float(alpha), int(n)), "dh_axpy")


def gemm_f32(transA, transB, M, N, K, A, lda, B, ldb, beta, C, ldc):
    check(load().dh_gemm_f32(int(transA), int(transB), M, N, K, _p(A), lda, _p(B), ldb,
                             float(beta), _p(C), ldc), "dh_gemm_f32")


def gemm_bf16(transA, transB, M, N, K, A, lda, B, ldb, beta, C, ldc):
    check(load().dh_gemm_bf16(int(transA), int(transB), M, N, K, _p(A), lda, _p(B), ldb,
                              float(beta), _p(C), ldc), "dh_gemm_bf16")


EPI_RELU, EPI_ROW_BIAS = 1, 2


def gemm_ex(dtype, transA, transB, M, N, K, A, lda, sA, B, ldb, sB, beta, C, ldc, sC, batch=1,
            bias=None, relu=False, row_bias=False):
    """dh_gemm_{f32,bf16}_ex: batched GEMM with the bias (by column, or by row) + ReLU
    epilogue."""
    fn = load().dh_gemm_bf16_ex if dtype == "bf16" else load().dh_gemm_f32_ex
    epi = (EPI_RELU if relu else 0) | (EPI_ROW_BIAS if row_bias else 0)
    check(fn(int(transA), int(transB), M, N, K, _p(A), lda, int(sA), _p(B), ldb, int(sB),
             float(beta), _p(C), ldc, int(sC), int(batch), _p(bias) if bias is not None else None,
             epi), f"dh_gemm_{dtype}_ex")


def gemm_f64(transA, transB, M, N, K, A, lda, B, ldb, beta, C, ldc, alpha=1.0, sA=0, sB=0,
             sC=0, batch=1):
    """dh_gemm_f64_ex: fp64 GEMM in the reference dgemm's summation order."""
    check(load().dh_gemm_f64_ex(int(transA), int(transB), M, N, K, float(alpha), _p(A), lda,
                                int(sA), _p(B), ldb, int(sB), float(beta), _p(C), ldc, int(sC),
                                int(batch)), "dh_gemm_f64_ex")


def attention_f64_fwd(BH, S, D, scale, causal, Q, K, V, O):
    check(load().dh_attention_f64_fwd(BH, S, D, float(scale), int(causal), _p(Q), _p(K), _p(V),
                                      _p(O)), "dh_attention_f64_fwd")


def attention_f64_bwd(BH, S, D, scale, causal, Q, K, V, dO, dQ, dK, dV, accumulate):
    check(load().dh_attention_f64_bwd(BH, S, D, float(scale), int(causal), _p(Q), _p(K), _p(V),
                                      _p(dO), _p(dQ), _p(dK), _p(dV), int(accumulate)),
          "dh_attention_f64_bwd")


def flash_fwd(dtype, BH, S, D, scale, causal, Q, K, V, O, LSE):
    check(load().dh_flash_fwd(dtype, BH, S, D, float(scale), int(causal), _p(Q), _p(K),
                              _p(V), _p(O), _p(LSE)), "dh_flash_fwd")


def flash_bwd(dtype, BH, S, D, scale, causal, Q, K, V, O, dO, LSE, dQ, dK, dV, accumulate):
    check(load().dh_flash_bwd(dtype, BH, S, D, float(scale), int(causal), _p(Q), _p(K),
                              _p(V), _p(O), _p(dO), _p(LSE), _p(dQ), _p(dK), _p(dV),
                              int(accumulate)), "dh_flash_bwd")


def row_softmax(X, Y, R, C, log=False):
    check(load().dh_row_softmax(_p(X), _p(Y), R, C, int(log)), "dh_row_softmax")


def row_softmax_bwd(Y, G, GX, R, C, log=False, accumulate=False):
    check(load().dh_row_softmax_bwd(_p(Y), _p(G), _p(GX), R, C, int(log), int(accumulate)),
          "dh_row_softmax_bwd")


def layer_norm(X, Y, R, C):
    check(load().dh_layer_norm(_p(X), _p(Y), R, C), "dh_layer_norm")


def linear_bias_grad(Y, dY, db, N, out, relu=False, accumulate=False):
    check(load().dh_linear_bias_grad(_p(Y) if Y is not None else None, _p(dY), _p(db), N, out,
                                     int(relu), int(accumulate)), "dh_linear_bias_grad")


def im2col(X, col, N, Cin, H, W, KH, KW, pad=0, stride=1):
    check(load().dh_im2col(_p(X), _p(col), N, Cin, H, W, KH, KW, pad, stride), "dh_im2col")


def col2im(dcol, dX, N, Cin, H, W, KH, KW, pad=0, stride=1, accumulate=False):
    check(load().dh_col2im(_p(dcol), _p(dX), N, Cin, H, W, KH, KW, pad, stride, int(accumulate)),
          "dh_col2im")


def conv2d_fwd(X, Kn, bias, Y, N, Cin, H, W, Cout, KH, KW, pad=0, stride=1):
    check(load().dh_conv2d_fwd(_p(X), _p(Kn), _p(bias), _p(Y), N, Cin, H, W, Cout, KH, KW, pad,
                               stride), "dh_conv2d_fwd")


def conv2d_bwd_data(dY, Kn, dX, N, Cin, H, W, Cout, KH, KW, pad=0, stride=1, accumulate=False):
    check(load().dh_conv2d_bwd_data(_p(dY), _p(Kn), _p(dX), N, Cin, H, W, Cout, KH, KW, pad,
                                    stride, int(accumulate)), "dh_conv2d_bwd_data")


def conv2d_bwd_filter(dY, X, dK, N, Cin, H, W, Cout, KH, KW, pad=0, stride=1, accumulate=False):
    check(load().dh_conv2d_bwd_filter(_p(dY), _p(X), _p(dK), N, Cin, H, W, Cout, KH, KW, pad,
                                      stride, int(accumulate)), "dh_conv2d_bwd_filter")


def nct_to_cnt(src, dst, N, C, T):
    check(load().dh_nct_to_cnt(_p(src), _p(dst), N, C, int(T)), "dh_nct_to_cnt")


# Elementwise op codes (include/dream_hip.h, the reference's BinopCode / UnopCode order).
BINOPS = ["add", "sub", "mul", "div", "mod", "gt", "lt", "ge", "le", "eq", "ne", "and", "or",
          "atan2", "pow", "min", "max"]
UNOPS = ["relu", "exp", "log", "sqrt", "abs", "sigmoid", "tanh", "lnot", "sin", "cos", "tan",
         "atan", "floor", "ceil", "round", "clip"]


def _i4(v):
    return (_i * 4)(*[int(x) for x in v])


def binary(op, dtype, A, a_len, a_strides, B, b_len, b_strides, C, c_dims, C32=None):
    """dh_binary: op is a name of BINOPS or its code; strides / dims are 4 ints each."""
    code = BINOPS.index(op) if isinstance(op, str) else int(op)
    check(load().dh_binary(code, int(dtype), _p(A), int(a_len), _i4(a_strides), _p(B),
                           int(b_len), _i4(b_strides), _p(C), _i4(c_dims), _p(C32)),
          "dh_binary")


def unary(op, dtype, A, C, n, lo=0.0, hi=0.0, C32=None):
    code = UNOPS.index(op) if isinstance(op, str) else int(op)
    check(load().dh_unary(code, int(dtype), _p(A), _p(C), int(n), float(lo), float(hi), _p(C32)),
          "dh_unary")


def layer_norm_bwd(X, Y, DY, GX, R, C, accumulate=False):
    check(load().dh_layer_norm_bwd(_p(X), _p(Y), _p(DY), _p(GX), R, C, int(accumulate)),
          "dh_layer_norm_bwd")


class Timer:
    """HIP events on the library stream (the stream every kernel here runs on)."""

    def __enter__(self):
        check(load().dh_timer_start(), "dh_timer_start")
        return self

    def __exit__(self, *exc):
        ms = _f()
        check(load().dh_timer_stop(ctypes.byref(ms)), "dh_timer_stop")
        self.ms = ms.value
        return False
