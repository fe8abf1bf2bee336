"""GPU parity of conv2d: the data-movement kernels (dh_im2col, dh_col2im, dh_nct_to_cnt), the
implicit-GEMM forward (dh_conv2d_fwd), data gradient (dh_conv2d_bwd_data) and kernel gradient
(dh_conv2d_bwd_filter), and the dream_conv2d / dream_conv2d_padded builtins with their
backward.

Tolerances: im2col and the permute are copies (bit-exact); col2im sums at most KH*KW values per
element (fp32 vs fp64 numpy: 1e-6 relative).  The builtins (fp32 on the GPU) against the fp64
oracle and the reference build's golden vectors: normwise max relative error <= 1e-5 * sqrt(L)
with L the contraction length of the product (Cin*KH*KW forward, N*OH*OW for dK, Cout for dX).
"""
import os

import numpy as np
import pytest

import _oracle as O
from dreamcompiler_amd import hip
from dreamcompiler_amd import runtime as rt

pytestmark = pytest.mark.gpu
DB = hip.DeviceBuffer
GOLD = np.load(os.path.join(os.path.dirname(__file__), "golden", "ref_vectors.npz"))


def maxrel(a, b):
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


def np_im2col(X, N, Cin, H, W, KH, KW, pad, stride):
    OH, OW = O.conv_out(H, W, KH, KW, pad, stride)
    Xp = np.zeros((N, Cin, H + 2 * pad, W + 2 * pad), X.dtype)
    Xp[:, :, pad:pad + H, pad:pad + W] = X.reshape(N, Cin, H, W)
    col = np.empty((Cin, KH, KW, N, OH, OW), X.dtype)
    for kh in range(KH):
        for kw in range(KW):
            col[:, kh, kw] = Xp[:, :, kh:kh + stride * OH:stride, kw:kw + stride * OW:stride].transpose(1, 0, 2, 3)
    return col.reshape(Cin * KH * KW, N * OH * OW)


@pytest.mark.parametrize("shape", [(2, 3, 7, 6, 3, 2, 0, 1), (3, 4, 9, 8, 3, 3, 1, 2),
                                   (1, 2, 5, 5, 5, 5, 2, 1), (2, 1, 11, 7, 1, 1, 0, 3)])
def test_im2col_col2im_permute(shape):
    N, Cin, H, W, KH, KW, pad, stride = shape
    OH, OW = O.conv_out(H, W, KH, KW, pad, stride)
    rng = np.random.default_rng(sum(shape))
    X = rng.standard_normal((N, Cin * H * W)).astype(np.float32)
    ref = np_im2col(X, N, Cin, H, W, KH, KW, pad, stride)
    dX, dcol = DB.from_numpy(X), DB.empty(ref.shape, np.float32)
    hip.im2col(dX, dcol, N, Cin, H, W, KH, KW, pad, stride)
    assert np.array_equal(dcol.numpy(), ref)
    # col2im is the adjoint of im2col: <im2col(X), C> = <X, col2im(C)>, and its sums match the
    # explicit scatter of numpy
    C = rng.standard_normal(ref.shape).astype(np.float32)
    dC, dG = DB.from_numpy(C), DB.empty(X.shape, np.float32)
    hip.col2im(dC, dG, N, Cin, H, W, KH, KW, pad, stride)
    G = dG.numpy()
    scatter = np.zeros((N, Cin, H + 2 * pad, W + 2 * pad))
    C6 = C.astype(np.float64).reshape(Cin, KH, KW, N, OH, OW)
    for kh in range(KH):
        for kw in range(KW):
            scatter[:, :, kh:kh + stride * OH:stride, kw:kw + stride * OW:stride] += C6[:, kh, kw].transpose(1, 0, 2, 3)
    want = scatter[:, :, pad:pad + H, pad:pad + W].reshape(X.shape)
    assert maxrel(G, want) <= 1e-6
    base = rng.standard_normal(X.shape).astype(np.float32)
    dB_ = DB.from_numpy(base)
    hip.col2im(dC, dB_, N, Cin, H, W, KH, KW, pad, stride, accumulate=True)
    assert maxrel(dB_.numpy(), base + want) <= 1e-6
    # channel-first permute of an (N, C, T) gradient
    T = OH * OW
    Y = rng.standard_normal((N, 5, T)).astype(np.float32)
    dY, dP = DB.from_numpy(Y), DB.empty((5, N * T), np.float32)
    hip.nct_to_cnt(dY, dP, N, 5, T)
    assert np.array_equal(dP.numpy(), Y.transpose(1, 0, 2).reshape(5, N * T))


@pytest.mark.parametrize("shape", [
    (2, 3, 7, 6, 4, 3, 2, 0, 1),        # golden-vector geometry, Cout <= 64 (64 x 64 tiles)
    (3, 5, 9, 8, 70, 3, 3, 1, 2),       # Cout > 64: 128 x 128 tiles, padded and strided
    (1, 2, 5, 5, 1, 5, 5, 2, 1),        # window as large as the padded input, one channel out
    (2, 16, 23, 17, 33, 3, 1, 1, 1),    # ragged positions, a K = 48 contraction
    (4, 7, 15, 15, 65, 1, 1, 0, 1),     # 1x1 kernel: R = Cin = 7 (a single k-slice)
    (2, 64, 20, 20, 64, 3, 3, 1, 1),    # R = 576, as in the ResNet-like bench layer
    (8, 16, 30, 30, 96, 3, 3, 1, 1),    # Cout > 64 on a small grid: 64 x 64 tiles
])
def test_conv2d_fwd_implicit_gemm_against_oracle(shape):
    # dh_conv2d_fwd against the fp64 oracle (orc_conv2d, pinned by the reference's golden
    # vectors) and against the stored im2col + GEMM path; bias and no bias.
    N, Cin, H, W, Cout, KH, KW, pad, stride = shape
    OH, OW = O.conv_out(H, W, KH, KW, pad, stride)
    rng = np.random.default_rng(sum(shape))
    X = rng.standard_normal((N, Cin * H * W)).astype(np.float32)
    Kn = rng.standard_normal((Cout, Cin * KH * KW)).astype(np.float32)
    b = rng.standard_normal(Cout).astype(np.float32)
    dX, dK, db = DB.from_numpy(X), DB.from_numpy(Kn), DB.from_numpy(b)
    dY = DB.empty((N, Cout * OH * OW), np.float32)
    try:
        for bias in (db, None):
            hip.conv2d_fwd(dX, dK, bias, dY, N, Cin, H, W, Cout, KH, KW, pad, stride)
            got = dY.numpy()
            ref = O.conv2d(X.astype(np.float64), Kn.astype(np.float64),
                           None if bias is None else b.astype(np.float64), N, Cin, H, W, Cout,
                           KH, KW, pad, stride)
            assert maxrel(got, ref) <= 1e-5 * np.sqrt(Cin * KH * KW), (shape, bias is None)
    finally:
        for t in (dX, dK, db, dY):
            t.free()


def test_conv2d_fwd_rejects_bad_shapes():
    d = DB.empty((64,), np.float32)
    try:
        with pytest.raises(hip.DreamHipError, match="kernel larger"):
            hip.conv2d_fwd(d, d, None, d, 1, 1, 2, 2, 1, 5, 5, 0, 1)
        with pytest.raises(hip.DreamHipError, match="invalid shape"):
            hip.conv2d_fwd(d, d, None, d, 1, 1, 2, 2, 1, 1, 1, 0, 0)
    finally:
        d.free()


@pytest.mark.parametrize("shape", [
    # N, Cin, H, W, Cout, KH, KW, pad
    (2, 3, 7, 6, 4, 3, 2, 0),       # valid conv, KH != KW
    (3, 5, 9, 8, 6, 3, 3, 1),       # 'same' padding
    (1, 2, 5, 5, 3, 5, 5, 4),       # pad = KH - 1 (the largest handled): a full correlation
    (2, 4, 11, 7, 2, 5, 3, 2),      # KH != KW with pad = KW - 1, the largest both allow
    (4, 7, 15, 15, 65, 1, 1, 0),    # 1x1 kernel, Cout = 65 (a partial k-slice of Cout KH KW)
    (2, 64, 20, 20, 64, 3, 3, 1),   # the bench layer's channels
    (2, 96, 12, 12, 32, 3, 3, 1),   # Cin = 96 > 64 output rows of the data-gradient GEMM
])
def test_conv2d_bwd_data_against_oracle(shape):
    # dh_conv2d_bwd_data (dX as the convolution of dY with the flipped, channel-swapped kernel)
    # against the fp64 oracle's conv backward (orc_conv2d_bwd, pinned by the reference's golden
    # vectors and finite differences) and against the stored dcol + col2im path; overwrite and
    # accumulate.
    N, Cin, H, W, Cout, KH, KW, pad = shape
    OH, OW = O.conv_out(H, W, KH, KW, pad, 1)
    rng = np.random.default_rng(sum(shape) + 7)
    X = rng.standard_normal((N, Cin * H * W)).astype(np.float32)
    Kn = rng.standard_normal((Cout, Cin * KH * KW)).astype(np.float32)
    G = rng.standard_normal((N, Cout * OH * OW)).astype(np.float32)
    X0 = rng.standard_normal((N, Cin * H * W)).astype(np.float32)
    rX, _ = O.conv2d_bwd(X.astype(np.float64), Kn.astype(np.float64), G.astype(np.float64),
                         N, Cin, H, W, Cout, KH, KW, pad, 1)
    dG, dK, dX = DB.from_numpy(G), DB.from_numpy(Kn), DB.from_numpy(X0)
    try:
        tol = 1e-5 * np.sqrt(Cout * KH * KW)
        hip.conv2d_bwd_data(dG, dK, dX, N, Cin, H, W, Cout, KH, KW, pad, 1)
        got = dX.numpy()
        assert maxrel(got, rX) <= tol, shape
        hip.conv2d_bwd_data(dG, dK, dX, N, Cin, H, W, Cout, KH, KW, pad, 1, accumulate=True)
        assert maxrel(dX.numpy(), 2 * rX) <= tol, shape
    finally:
        for t in (dG, dK, dX):
            t.free()


@pytest.mark.parametrize("shape", [
    # N, Cin, H, W, Cout, KH, KW, pad, stride
    (2, 3, 7, 6, 4, 3, 2, 0, 1),       # P = 20: one partial slice per image
    (3, 5, 9, 8, 6, 3, 3, 1, 2),       # strided, P = 20
    (1, 2, 5, 5, 3, 5, 5, 2, 1),       # one image
    (2, 1, 11, 7, 1, 1, 1, 0, 3),      # 1x1 taps, stride 3, P = 12
    (5, 4, 13, 13, 130, 3, 3, 2, 3),   # Cout > 64: 128 x 128 tiles; P = 25 (not a multiple of 4)
    (16, 64, 14, 14, 64, 3, 3, 1, 1),  # the bench layer's channels: many chunks over 16 images
    (64, 3, 8, 8, 8, 3, 3, 1, 1),      # a long contraction over 64 small images
])
def test_conv2d_bwd_filter_against_oracle(shape):
    # dh_conv2d_bwd_filter (implicit GEMM over the (image, position) contraction, col
    # gathered in the loader) against the fp64 oracle's kernel gradient (orc_conv2d_bwd,
    # pinned by the reference's golden vectors and finite differences); overwrite, accumulate,
    # and bit-identical reruns.
    N, Cin, H, W, Cout, KH, KW, pad, stride = shape
    OH, OW = O.conv_out(H, W, KH, KW, pad, stride)
    rng = np.random.default_rng(sum(shape) + 11)
    X = rng.standard_normal((N, Cin * H * W)).astype(np.float32)
    Kn = rng.standard_normal((Cout, Cin * KH * KW)).astype(np.float32)
    G = rng.standard_normal((N, Cout * OH * OW)).astype(np.float32)
    _, rK = O.conv2d_bwd(X.astype(np.float64), Kn.astype(np.float64), G.astype(np.float64),
                         N, Cin, H, W, Cout, KH, KW, pad, stride)
    K0 = rng.standard_normal((Cout, Cin * KH * KW)).astype(np.float32)
    dG, dX, dK = DB.from_numpy(G), DB.from_numpy(X), DB.from_numpy(K0)
    try:
        tol = 1e-5 * np.sqrt(N * OH * OW)
        hip.conv2d_bwd_filter(dG, dX, dK, N, Cin, H, W, Cout, KH, KW, pad, stride)
        got = dK.numpy()
        assert maxrel(got, rK) <= tol, shape
        hip.conv2d_bwd_filter(dG, dX, dK, N, Cin, H, W, Cout, KH, KW, pad, stride)
        assert np.array_equal(dK.numpy(), got), shape
        hip.conv2d_bwd_filter(dG, dX, dK, N, Cin, H, W, Cout, KH, KW, pad, stride, accumulate=True)
        assert maxrel(dK.numpy(), 2 * rK) <= tol, shape
    finally:
        for t in (dG, dX, dK):
            t.free()


def test_conv2d_bwd_filter_empty_batch_and_rejects():
    K0 = np.arange(2 * 9, dtype=np.float32).reshape(2, 9)
    d, dK = DB.empty((4096,), np.float32), DB.from_numpy(K0)
    try:
        # N = 0: an empty sum -- dK unchanged with accumulate, zeros without
        hip.conv2d_bwd_filter(d, d, dK, 0, 1, 8, 8, 2, 3, 3, 1, 1, accumulate=True)
        assert np.array_equal(dK.numpy(), K0)
        hip.conv2d_bwd_filter(d, d, dK, 0, 1, 8, 8, 2, 3, 3, 1, 1)
        assert not dK.numpy().any()
        with pytest.raises(hip.DreamHipError, match="kernel larger"):
            hip.conv2d_bwd_filter(d, d, d, 1, 1, 2, 2, 1, 5, 5, 0, 1)
        with pytest.raises(hip.DreamHipError, match="invalid shape"):
            hip.conv2d_bwd_filter(d, d, d, 1, 1, 8, 8, 1, 3, 3, 0, 0)
        with pytest.raises(hip.DreamHipError, match="null pointer"):
            hip.conv2d_bwd_filter(None, d, d, 1, 1, 8, 8, 1, 3, 3, 0, 1)
    finally:
        d.free()
        dK.free()


def test_conv2d_bwd_data_rejects():
    d = DB.empty((4096,), np.float32)
    try:
        with pytest.raises(hip.DreamHipError, match="stride 2"):
            hip.conv2d_bwd_data(d, d, d, 1, 1, 8, 8, 1, 3, 3, 1, 2)
        with pytest.raises(hip.DreamHipError, match="pad 3"):
            hip.conv2d_bwd_data(d, d, d, 1, 1, 8, 8, 1, 3, 3, 3, 1)
        with pytest.raises(hip.DreamHipError, match="pad 2"):
            hip.conv2d_bwd_data(d, d, d, 1, 1, 8, 8, 1, 5, 2, 2, 1)   # pad > KW - 1
        with pytest.raises(hip.DreamHipError, match="kernel larger"):
            hip.conv2d_bwd_data(d, d, d, 1, 1, 2, 2, 1, 5, 5, 0, 1)
        with pytest.raises(hip.DreamHipError, match="invalid shape"):
            hip.conv2d_bwd_data(d, d, d, 1, 0, 8, 8, 1, 3, 3, 0, 1)
        with pytest.raises(hip.DreamHipError, match="null pointer"):
            hip.conv2d_bwd_data(None, d, d, 1, 1, 8, 8, 1, 3, 3, 0, 1)
    finally:
        d.free()


@pytest.fixture(scope="module")
def L():
    return rt.load()


def _conv(L, X, Kn, b, H, W, KH, KW, pad=None, stride=None):
    x, k = rt.tensor(X), rt.tensor(Kn)
    bb = rt.tensor(b) if b is not None else None
    sc = [rt.scalar(v) for v in (H, W, KH, KW)]
    if pad is None:
        y = L.dream_conv2d(x, k, bb, *sc)
    else:
        y = L.dream_conv2d_padded(x, k, bb, *sc, rt.scalar(pad), rt.scalar(stride))
    return x, k, y


def _grads(L, y, G, *ins):
    L.backward(L.sum(L.tensor_mul(y, rt.tensor(G))))
    return [rt.read(t, grad=True) for t in ins]


def test_conv2d_against_reference_golden(L):
    X, Kn, b, G = (GOLD["conv_" + c] for c in "XKbG")
    x, k, y = _conv(L, X, Kn, b, 7, 6, 3, 2)
    assert maxrel(rt.read(y), GOLD["conv_Y"]) <= 1e-5 * np.sqrt(18)
    gX, gK = _grads(L, y, G, x, k)
    assert maxrel(gX, GOLD["conv_dX"]) <= 1e-5 * np.sqrt(4)
    assert maxrel(gK, GOLD["conv_dK"]) <= 1e-5 * np.sqrt(50)
    _, _, yp = _conv(L, X, Kn, b, 7, 6, 3, 2, pad=1, stride=2)
    assert maxrel(rt.read(yp), GOLD["conv_padded_Y"]) <= 1e-5 * np.sqrt(18)


@pytest.mark.parametrize("pad,stride", [(0, 1), (1, 1), (1, 2), (2, 3)])
def test_conv2d_layer_shape_against_oracle(L, pad, stride):
    # A CNN layer: N=8, Cin=16, 32x32, Cout=32, 3x3 (valid and padded / strided), forward and
    # both gradients.  The padded backward is the exact gradient (pinned by finite differences
    # in tests/test_oracle.py), not the reference node's.
    N, Cin, H, W, Cout, KH, KW = 8, 16, 32, 32, 32, 3, 3
    rng = np.random.default_rng(pad * 10 + stride)
    X = rng.standard_normal((N, Cin * H * W))
    Kn = rng.standard_normal((Cout, Cin * KH * KW)) * 0.1
    b = rng.standard_normal((1, Cout))
    OH, OW = O.conv_out(H, W, KH, KW, pad, stride)
    G = rng.standard_normal((N, Cout * OH * OW))
    args = (N, Cin, H, W, Cout, KH, KW, pad, stride)
    x, k, y = _conv(L, X, Kn, b, H, W, KH, KW, *(() if (pad, stride) == (0, 1) else (pad, stride)))
    assert maxrel(rt.read(y), O.conv2d(X, Kn, b, *args)) <= 1e-5 * np.sqrt(Cin * KH * KW)
    gX, gK = _grads(L, y, G, x, k)
    rX, rK = O.conv2d_bwd(X, Kn, G, *args)
    assert maxrel(gX, rX) <= 1e-5 * np.sqrt(Cout * KH * KW)
    assert maxrel(gK, rK) <= 1e-5 * np.sqrt(N * OH * OW)


def test_conv2d_short_bias_and_errors(L, capfd):
    # A bias with fewer values than output channels covers only its first channels
    # (conv.inc:5-10); a kernel larger than the input is the reference's error.
    rng = np.random.default_rng(9)
    X, Kn, b = rng.standard_normal((2, 2 * 25)), rng.standard_normal((3, 2 * 4)), np.array([[1.0, -2.0]])
    _, _, y = _conv(L, X, Kn, b, 5, 5, 2, 2)
    want = O.conv2d(X, Kn, np.array([1.0, -2.0, 0.0]), 2, 2, 5, 5, 3, 2, 2)
    assert maxrel(rt.read(y), want) <= 1e-5 * np.sqrt(8)
    _, _, e = _conv(L, X, Kn, None, 5, 5, 6, 2)
    assert rt.read(e).shape == (1, 1)
    assert "error: conv2d kernel larger than input" in capfd.readouterr().err
