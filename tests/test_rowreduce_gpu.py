"""GPU parity of dh_convert (bit-exact) and the row-wise ops (fp32 vs the fp64 oracle).

Row ops: dh_row_softmax (softmax / log_softmax), dh_row_softmax_bwd, dh_layer_norm,
dh_layer_norm_bwd.  Tolerance: max |got - ref| <= 1e-5 * sqrt(C) * max(1, max |ref|) against the
fp64 oracle on the same fp32 inputs (C = row length, the reduction length); the reference's
own golden vectors are checked at the same bound.  Shapes cover every kernel form: segments
of 4, 16 and 64 lanes with 4-value and 1-value chunks (C % 4 == 0 or not) and the streaming
long-row kernels (C > 1024), plus accumulate on and off.
"""
import os

import numpy as np
import pytest

import _oracle as O
from dreamcompiler_amd import hip

pytestmark = pytest.mark.gpu
DB = hip.DeviceBuffer


def _convert(src, src_t, dst_t, dst_np):
    d_src = DB.from_numpy(src)
    d_dst = DB.empty(src.shape, dst_np)
    hip.convert(d_dst, dst_t, d_src, src_t, src.size)
    return d_dst.numpy()


def test_convert_bit_exact():
    rng = np.random.default_rng(1)
    x64 = np.concatenate([rng.standard_normal(100003) * 10.0 ** rng.integers(-20, 20, 100003),
                          [0.0, -0.0, 1.0, 1.00390625, 1.01171875, -1.00390625]])
    got32 = _convert(x64, hip.F64, hip.F32, np.float32)
    assert np.array_equal(got32.view(np.uint32), x64.astype(np.float32).view(np.uint32))
    # fp64 -> fp32 -> bf16, the reference's dream_to_bf16 of the HostBuf value
    gotb = _convert(x64, hip.F64, hip.BF16, np.uint16)
    assert np.array_equal(gotb, O.bf16_bits(x64.astype(np.float32)))
    gotb2 = _convert(x64.astype(np.float32), hip.F32, hip.BF16, np.uint16)
    assert np.array_equal(gotb2, gotb)
    back = _convert(gotb, hip.BF16, hip.F32, np.float32)
    assert np.array_equal(back, O.bf16_round(x64.astype(np.float32)))
    back64 = _convert(got32, hip.F32, hip.F64, np.float64)
    assert np.array_equal(back64, got32.astype(np.float64))


@pytest.mark.parametrize("R,C", [(1, 1), (5, 7), (100, 64), (33, 65), (7, 1000), (3, 4097)])
@pytest.mark.parametrize("log", [False, True])
def test_row_softmax(R, C, log):
    rng = np.random.default_rng(R * 7 + C)
    X = (rng.standard_normal((R, C)) * 4).astype(np.float32)
    dX, dY = DB.from_numpy(X), DB.empty((R, C), np.float32)
    hip.row_softmax(dX, dY, R, C, log)
    Y = dY.numpy()
    X64 = X.astype(np.float64)
    ref = O.log_softmax_rows(X64) if log else O.softmax_rows(X64)
    if log:
        assert np.abs(Y - ref).max() <= 1e-5 * max(1.0, np.abs(ref).max())
    else:
        assert np.abs(Y - ref).max() <= 1e-6
        assert np.allclose(Y.sum(1), 1.0, atol=1e-5)


GOLD = np.load(os.path.join(os.path.dirname(__file__), "golden", "ref_vectors.npz"))
SHAPES = [(1, 1), (3, 10), (37, 33), (64, 64), (19, 100), (50, 256), (9, 257), (8, 1000),
          (5, 1024), (4, 1025), (3, 4096), (2, 5001)]


def _tol(ref, C):
    return 1e-5 * np.sqrt(C) * max(1.0, float(np.abs(ref).max()))


def _run(fn, ins, out_shape, *args, init=None):
    bufs = [DB.from_numpy(np.ascontiguousarray(x, np.float32)) for x in ins]
    out = DB.from_numpy(np.ascontiguousarray(init, np.float32)) if init is not None \
        else DB.empty(out_shape, np.float32)
    fn(*bufs, out, *args)
    return out.numpy()


@pytest.mark.parametrize("R,C", SHAPES)
@pytest.mark.parametrize("log", [False, True])
def test_row_softmax_bwd(R, C, log):
    rng = np.random.default_rng(R * 11 + C + log)
    X = (rng.standard_normal((R, C)) * 3).astype(np.float32)
    G = rng.standard_normal((R, C)).astype(np.float32)
    X64 = X.astype(np.float64)
    Y64 = O.log_softmax_rows(X64) if log else O.softmax_rows(X64)
    Y = Y64.astype(np.float32)          # the forward output the backward is given
    if log:
        ref = O.log_softmax_bwd(X64, G.astype(np.float64))
    else:
        ref = O.softmax_bwd(Y.astype(np.float64), G.astype(np.float64))
    got = _run(lambda y, g, gx: hip.row_softmax_bwd(y, g, gx, R, C, log), (Y, G), (R, C))
    assert np.abs(got - ref).max() <= _tol(ref, C)
    base = rng.standard_normal((R, C)).astype(np.float32)
    got2 = _run(lambda y, g, gx: hip.row_softmax_bwd(y, g, gx, R, C, log, accumulate=True),
                (Y, G), (R, C), init=base)
    assert np.abs(got2 - (base + ref)).max() <= _tol(base + ref, C)


@pytest.mark.parametrize("R,C", SHAPES)
def test_layer_norm_fwd_bwd(R, C):
    rng = np.random.default_rng(R * 13 + C)
    X = (rng.standard_normal((R, C)) * 3 + 1.5).astype(np.float32)
    DY = rng.standard_normal((R, C)).astype(np.float32)
    X64 = X.astype(np.float64)
    ref = O.layer_norm(X64)
    Y = _run(lambda x, y: hip.layer_norm(x, y, R, C), (X,), (R, C))
    assert np.abs(Y - ref).max() <= _tol(ref, C)
    gref = O.layer_norm_bwd(X64, ref, DY.astype(np.float64))
    got = _run(lambda x, y, dy, gx: hip.layer_norm_bwd(x, y, dy, gx, R, C), (X, ref, DY), (R, C))
    assert np.abs(got - gref).max() <= _tol(gref, C)
    base = rng.standard_normal((R, C)).astype(np.float32)
    got2 = _run(lambda x, y, dy, gx: hip.layer_norm_bwd(x, y, dy, gx, R, C, accumulate=True),
                (X, ref, DY), (R, C), init=base)
    assert np.abs(got2 - (base + gref)).max() <= _tol(base + gref, C)


def test_row_ops_reference_golden_vectors():
    X, G = GOLD["softmax_X"], GOLD["softmax_G"]
    R, C = X.shape
    Y = _run(lambda x, y: hip.row_softmax(x, y, R, C, False), (X,), (R, C))
    assert np.abs(Y - GOLD["softmax_Y"]).max() <= _tol(GOLD["softmax_Y"], C)
    LY = _run(lambda x, y: hip.row_softmax(x, y, R, C, True), (X,), (R, C))
    assert np.abs(LY - GOLD["log_softmax_Y"]).max() <= _tol(GOLD["log_softmax_Y"], C)
    dX = _run(lambda y, g, gx: hip.row_softmax_bwd(y, g, gx, R, C, False), (Y, G), (R, C))
    assert np.abs(dX - GOLD["softmax_dX"]).max() <= _tol(GOLD["softmax_dX"], C)
    dXl = _run(lambda y, g, gx: hip.row_softmax_bwd(y, g, gx, R, C, True), (LY, G), (R, C))
    assert np.abs(dXl - GOLD["log_softmax_dX"]).max() <= _tol(GOLD["log_softmax_dX"], C)
    LX, LG = GOLD["layer_norm_X"], GOLD["layer_norm_G"]
    R, C = LX.shape
    LNY = _run(lambda x, y: hip.layer_norm(x, y, R, C), (LX,), (R, C))
    assert np.abs(LNY - GOLD["layer_norm_Y"]).max() <= _tol(GOLD["layer_norm_Y"], C)
    LdX = _run(lambda x, y, dy, gx: hip.layer_norm_bwd(x, y, dy, gx, R, C), (LX, LNY, LG), (R, C))
    assert np.abs(LdX - GOLD["layer_norm_dX"]).max() <= _tol(GOLD["layer_norm_dX"], C)


def test_row_ops_large_rows_count():
    # Many short rows (the segment kernels' multi-row work-groups with a ragged last group)
    # and the properties that hold at any size: softmax rows sum to 1, layer-norm rows have
    # mean 0, softmax backward rows sum to 0.
    R, C = 100003, 20
    rng = np.random.default_rng(5)
    X = rng.standard_normal((R, C)).astype(np.float32)
    Y = _run(lambda x, y: hip.row_softmax(x, y, R, C, False), (X,), (R, C))
    assert np.abs(Y.sum(1) - 1).max() <= 1e-5
    N = _run(lambda x, y: hip.layer_norm(x, y, R, C), (X,), (R, C))
    assert np.abs(N.mean(1)).max() <= 1e-5
    G = rng.standard_normal((R, C)).astype(np.float32)
    dX = _run(lambda y, g, gx: hip.row_softmax_bwd(y, g, gx, R, C, False), (Y, G), (R, C))
    assert np.abs(dX.sum(1)).max() <= 1e-5
