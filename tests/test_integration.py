"""The reference runtime with the HIP backend bound in (oracle/_ref/libdreamref_hip.so, built
by `make -C oracle ref-hip` from the reference's own sources, the insertion-only hooks of
dreamcompiler_amd/integration/reference_hooks.patch and dream_hip_binding.inc).

CPU (no device): every hooked builtin -- `@` above and below the dispatch threshold, the
`as f32` product, flash_attention and the backward through both nodes -- prints the binding's
"warning: HIP backend unavailable (...) -- using CPU" once and returns exactly the plain
reference build's values (its CPU path runs unchanged).

GPU: the same program on the hooks' HIP path, without the warning: `@` below the threshold
bit-identical to the reference's dgemm (dh_gemm_f64 sums in its order), above it and in
flash_attention within the fp32 bounds (1e-5 sqrt(K), 1e-5 sqrt(S)) against the reference's
fp64 values, and bf16 mode (dream_enable_fp16) within 2e-2.

Each program runs in a child process of its own: the patched runtime and the plain one
export the same symbols.
"""
import json
import os
import subprocess
import sys

import numpy as np
import pytest

import _ref_runtime

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
HIP_REF = os.path.join(ROOT, "oracle", "_ref", "libdreamref_hip.so")

# The program: inputs from a seeded numpy generator, outputs to an .npz.
_PROGRAM = r"""
import sys, ctypes, numpy as np
sys.path[:0] = [{tests!r}]
import _ref_runtime
R = _ref_runtime.RefRuntime({lib!r})
L = R.L
if {fp16}:
    L.dream_enable_fp16.restype = _ref_runtime._TP
    L.dream_enable_fp16()
rng = np.random.default_rng(2027)
out = {{}}
A, B = rng.standard_normal((600, 520)), rng.standard_normal((520, 520))   # M*N >= 262144
W = rng.standard_normal((600, 520))
out["mm_big"] = R.matmul(A, B)
out["mm_big_dA"], out["mm_big_dB"] = R.matmul_grads(A, B, W)
a, b = rng.standard_normal((100, 300)), rng.standard_normal((300, 90))     # below it
w = rng.standard_normal((100, 90))
out["mm_small"] = R.matmul(a, b)
out["mm_small_dA"], out["mm_small_dB"] = R.matmul_grads(a, b, w)
F1, F2 = rng.standard_normal((300, 520)), rng.standard_normal((520, 880))
out["mm_f32"] = R.matmul(F1, F2, f32=True)
Bt, S, dk = 2, 384, 48                                                     # flash rule, dk padded
Q, K, V, G = (rng.standard_normal((Bt, S * dk)) for _ in range(4))
out["fa_O"] = R.attention("flash", Q, K, V, Bt, S, dk)
out["fa_dQ"], out["fa_dK"], out["fa_dV"] = R.attention_grads("flash", Q, K, V, G, Bt, S, dk)
q = rng.standard_normal((Bt, S * dk))                                      # q as Q, K and V
qt = R.tensor(q)
o = L.dream_flash_attention(qt, qt, qt, R.scalar(Bt), R.scalar(S), R.scalar(dk), R.scalar(64))
L.backward(L.sum(L.tensor_mul(o, R.tensor(G))))
out["fa_self_dq"] = R.read(qt, grad=True)
np.savez({path!r}, **out)
print("PROGRAM_DONE", flush=True)
"""


def _run(lib, path, fp16=False, env=None):
    code = _PROGRAM.format(tests=HERE, lib=lib, path=str(path), fp16=bool(fp16))
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=600,
                       env={**os.environ, **(env or {})})
    assert r.returncode == 0 and "PROGRAM_DONE" in r.stdout, r.stdout[-2000:] + r.stderr[-4000:]
    return dict(np.load(path)), r.stderr


def _need_builds():
    if not (_ref_runtime.available() and os.path.exists(HIP_REF)):
        pytest.skip("oracle/_ref/libdreamref(_hip).so not built (needs /root/reference)")


def test_binding_without_device_falls_back_to_reference_cpu(tmp_path):
    _need_builds()
    got, err = _run(HIP_REF, tmp_path / "hip.npz", env={"HIP_VISIBLE_DEVICES": "-1"})
    if "HIP backend unavailable" not in err:
        pytest.skip("a HIP device is visible: the fallback is exercised on machines without one")
    assert err.count("warning: HIP backend unavailable") == 1, err[-2000:]
    assert "-- using CPU" in err
    ref, _ = _run(_ref_runtime.LIB_PATH, tmp_path / "ref.npz")
    for k in ref:
        assert np.array_equal(got[k], ref[k]), k


def _err(a, b):
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-300))


@pytest.mark.gpu
@pytest.mark.parametrize("fp16", [False, True])
def test_binding_on_gpu_matches_reference(tmp_path, fp16):
    _need_builds()
    got, err = _run(HIP_REF, tmp_path / "hip.npz", fp16=fp16)
    assert "using CPU" not in err, err[-2000:]
    ref, _ = _run(_ref_runtime.LIB_PATH, tmp_path / "ref.npz", fp16=fp16)
    # below the threshold: the fp64 GEMM in dgemm's order, the reference's values exactly
    assert np.array_equal(got["mm_small"], ref["mm_small"])
    # its backward in fp64 (summation order of a GEMM, not of the reference's loops)
    for k in ("mm_small_dA", "mm_small_dB"):
        assert _err(got[k], ref[k]) <= 1e-13, k
    f32 = 2e-2 if fp16 else None
    bounds = {"mm_big": f32 or 1e-5 * np.sqrt(520), "mm_big_dA": f32 or 1e-5 * np.sqrt(520),
              "mm_big_dB": f32 or 1e-5 * np.sqrt(600), "mm_f32": 1e-5 * np.sqrt(520),
              "fa_O": f32 or 1e-5 * np.sqrt(384), "fa_dQ": f32 or 1e-5 * np.sqrt(384),
              "fa_dK": f32 or 1e-5 * np.sqrt(384), "fa_dV": f32 or 1e-5 * np.sqrt(384),
              "fa_self_dq": f32 or 1e-5 * np.sqrt(384)}
    report = {k: _err(got[k], ref[k]) for k in bounds}
    print(json.dumps(report))
    for k, tol in bounds.items():
        assert report[k] <= tol, (k, report[k], tol)
