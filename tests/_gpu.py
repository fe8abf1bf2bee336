"""Helpers for the GPU parity tests: run the HIP entry points on numpy inputs.

All device work goes through dreamcompiler_amd.hip (the C ABI); there is no other path.
"""
import numpy as np

from dreamcompiler_amd import hip

DB = hip.DeviceBuffer


def bf16_bits(x):
    """fp32 -> bf16 bits by the round-to-nearest-even rule (numpy, host side)."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFFFFFF
    return (u >> 16).astype(np.uint16)


def bits_to_f32(b):
    return (np.asarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


def gemm(A, B, transA=False, transB=False, beta=0.0, C0=None, dtype="f32", ldpad=0,
         ldcpad=None):
    """Run dh_gemm_{f32,bf16} on host arrays given in their stored layout.

    A, B: fp32 arrays (stored layout), or uint16 bf16 bits for dtype="bf16".
    ldpad: extra columns of padding on every stored matrix (exercises lda > K etc.).
    ldcpad: padding of C alone when given (overrides ldpad for C).
    """
    M = A.shape[1] if transA else A.shape[0]
    K = A.shape[0] if transA else A.shape[1]
    N = B.shape[0] if transB else B.shape[1]
    np_t = np.uint16 if dtype == "bf16" else np.float32

    def padded(X, t, pad):
        X = np.ascontiguousarray(X, t)
        if not pad:
            return X
        P = np.zeros((X.shape[0], X.shape[1] + pad), t)
        P[:, :X.shape[1]] = X
        return P

    cpad = ldpad if ldcpad is None else ldcpad
    Ap, Bp = padded(A, np_t, ldpad), padded(B, np_t, ldpad)
    Cp = padded(np.zeros((M, N), np.float32) if C0 is None else C0, np.float32, cpad)
    dA, dB, dC = DB.from_numpy(Ap), DB.from_numpy(Bp), DB.from_numpy(Cp)
    fn = hip.gemm_bf16 if dtype == "bf16" else hip.gemm_f32
    fn(transA, transB, M, N, K, dA, Ap.shape[1], dB, Bp.shape[1], beta, dC, Cp.shape[1])
    out = dC.numpy((M, N + cpad), np.float32)[:, :N]
    for b in (dA, dB, dC):
        b.free()
    return out


def maxrel(got, ref):
    """max_ij |got - ref| / max_ij |ref| (the normwise max relative error)."""
    return float(np.abs(got - ref).max() / max(np.abs(ref).max(), 1e-30))


def elementwise_ratio(got, ref, absA, absB):
    """max_ij |got - ref| / (|A| |B|)_ij: error against the per-element product scale."""
    scale = absA @ absB
    return float((np.abs(got - ref) / np.maximum(scale, 1e-30)).max())


def flash_fwd(Q, K, V, BH, S, D, causal=True, dtype="f32", scale=None):
    """dh_flash_fwd on host arrays of shape (BH, S*D).  Q/K/V fp32 (dtype f32) or bf16
    bits (dtype bf16).  Returns (O as fp32, LSE)."""
    scale = 1.0 / np.sqrt(D) if scale is None else scale
    dt = hip.BF16 if dtype == "bf16" else hip.F32
    np_t = np.uint16 if dtype == "bf16" else np.float32
    dQ, dK, dV = (DB.from_numpy(np.ascontiguousarray(x, np_t)) for x in (Q, K, V))
    dO_ = DB.empty((BH, S * D), np_t)
    dL = DB.empty((BH, S), np.float32)
    hip.flash_fwd(dt, BH, S, D, scale, causal, dQ, dK, dV, dO_, dL)
    O = dO_.numpy()
    O = bits_to_f32(O) if dtype == "bf16" else O
    return O, dL.numpy()


def flash_bwd(Q, K, V, O, dO, LSE, BH, S, D, causal=True, dtype="f32", scale=None,
              accumulate=False, init=None):
    """dh_flash_bwd; O/dO in the input dtype (bf16 bits for bf16).  Returns fp32 grads."""
    scale = 1.0 / np.sqrt(D) if scale is None else scale
    dt = hip.BF16 if dtype == "bf16" else hip.F32
    np_t = np.uint16 if dtype == "bf16" else np.float32
    bufs = [DB.from_numpy(np.ascontiguousarray(x, np_t)) for x in (Q, K, V, O, dO)]
    dL = DB.from_numpy(np.ascontiguousarray(LSE, np.float32))
    if init is None:
        grads = [DB.empty((BH, S * D), np.float32) for _ in range(3)]
    else:
        grads = [DB.from_numpy(np.ascontiguousarray(g, np.float32)) for g in init]
    hip.flash_bwd(dt, BH, S, D, scale, causal, *bufs, dL, *grads, int(accumulate))
    return tuple(g.numpy() for g in grads)
