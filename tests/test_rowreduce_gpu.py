"""GPU parity of dh_convert (bit-exact) and dh_row_softmax (fp32 vs the fp64 oracle)."""
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
