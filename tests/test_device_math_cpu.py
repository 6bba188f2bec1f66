"""The device-side integer helpers (heatvit_amd/csrc/hv_device.h), built for
the host and checked against the CPU oracle: exhaustive GELU with the
reciprocal estimate perturbed, the 32-bit softmax path, and the int32
LayerNorm normalisation on random and degenerate rows."""

import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HIPCC = Path("/opt/rocm/bin/hipcc")


@pytest.mark.skipif(not HIPCC.exists() or shutil.which("gcc") is None, reason="needs hipcc and gcc")
def test_device_math_matches_oracle(tmp_path):
    obj = tmp_path / "hv_oracle.o"
    subprocess.run(["gcc", "-O2", "-c", "-o", str(obj), str(ROOT / "oracle" / "hv_oracle.c")], check=True)
    exe = tmp_path / "check_device_math"
    r = subprocess.run([str(HIPCC), "-O2", "-std=c++17", "-I", str(ROOT / "heatvit_amd" / "csrc"),
                        "-I", str(ROOT / "include"), "-I", str(ROOT / "oracle"), "-o", str(exe),
                        str(ROOT / "tests" / "device_math" / "check_device_math.cpp"),
                        "-x", "none", str(obj)], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    out = subprocess.run([str(exe), "60000"], capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stdout[-2000:]
    assert "gelu_bad=0 softmax_bad=0 layernorm_bad=0" in out.stdout
