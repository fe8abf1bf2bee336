"""The C-ABI libraries load and export every symbol their headers declare (CPU only;
no kernel is launched here)."""
import ctypes
import os
import re
import subprocess
import sys

import pytest

from dreamcompiler_amd import hip

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
DECL = re.compile(r"^[A-Za-z_][\w\s\*]*?\b((?:dh|dream|tensor)_\w+|backward|gpu_selftest|"
                  r"flash_attention_selftest|alloc_tensor|create_scalar|sum|ones|relu)\s*\(", re.M)


def declared(header):
    text = open(os.path.join(ROOT, "include", header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    return sorted(set(DECL.findall(text)))


def test_hip_library_exports_every_declared_symbol():
    L = hip.load()
    names = declared("dream_hip.h")
    assert len(names) >= 25
    for n in names:
        assert hasattr(L, n), f"libdream_hip.so does not export {n}"
    # the Python binding covers exactly the header
    assert sorted(hip.EXPORTED) == names


def test_runtime_library_exports_every_declared_symbol():
    path = os.path.join(ROOT, "dreamcompiler_amd", "lib", "libdream_rt.so")
    if not os.path.exists(os.path.join(ROOT, "include", "dream_rt.h")):
        pytest.skip("runtime header not present")
    L = ctypes.CDLL(path)
    for n in declared("dream_rt.h"):
        assert hasattr(L, n), f"libdream_rt.so does not export {n}"


def _policy(env):
    code = ("from dreamcompiler_amd import hip; L = hip.load(); "
            "print(L.dh_dispatch_threshold(), L.dh_matmul_eligible(512, 512), "
            "L.dh_matmul_eligible(511, 512), L.dh_flash_eligible(1, 512, 64), "
            "L.dh_flash_eligible(1, 511, 64), L.dh_flash_eligible(4, 512, 256))")
    out = subprocess.run([sys.executable, "-c", code], env={**os.environ, **env}, cwd=ROOT,
                         capture_output=True, text=True, check=True).stdout.split()
    return [int(x) for x in out]


def test_dispatch_policy_matches_reference():
    # gpu.inc:293-307 (threshold 262144, env override), elementwise.inc:1033,
    # training.inc:308/336 (B*S*S >= 262144 and dk <= 128).
    env = {k: v for k, v in os.environ.items() if k != "DREAM_GPU_THRESHOLD"}
    env.pop("DREAM_GPU_THRESHOLD", None)
    assert _policy({"DREAM_GPU_THRESHOLD": ""}) == [262144, 1, 0, 1, 0, 0]
    assert _policy({"DREAM_GPU_THRESHOLD": "0"})[:3] == [0, 1, 1]
    assert _policy({"DREAM_GPU_THRESHOLD": "1000000"})[:3] == [1000000, 0, 0]
    assert _policy({"DREAM_GPU_THRESHOLD": "junk"})[0] == 262144
