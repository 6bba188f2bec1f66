"""The CPU code under AddressSanitizer and UndefinedBehaviorSanitizer (any
finding aborts the run):

* the oracle (oracle/hv_oracle.c built by `make liboracle_san.so`) through
  the oracle's own test files -- the reference's vectors, the golden
  composite fixtures and the reference's seeded e2e model -- in a child
  process with libasan preloaded;
* the host build of the device integer helpers (hv_device.h: GELU,
  softmax, LayerNorm limb split) against the oracle, both instrumented.
"""

import os
import shutil
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HIPCC = Path("/opt/rocm/bin/hipcc")
CLANG = Path("/opt/rocm/llvm/bin/clang")
SAN_ENV = {"ASAN_OPTIONS": "detect_leaks=0:abort_on_error=1",
           "UBSAN_OPTIONS": "print_stacktrace=1:halt_on_error=1"}


def _gcc_runtime(name):
    r = subprocess.run(["gcc", f"-print-file-name={name}"], capture_output=True, text=True)
    p = Path(r.stdout.strip())
    return p if p.is_absolute() and p.exists() else None


@pytest.mark.skipif(shutil.which("gcc") is None or shutil.which("make") is None,
                    reason="needs gcc and make")
def test_oracle_suites_under_asan_ubsan():
    asan = _gcc_runtime("libasan.so")
    if asan is None:
        pytest.skip("gcc's libasan is not installed")
    subprocess.run(["make", "-s", "-B", "liboracle_san.so"], cwd=ROOT / "oracle", check=True)
    env = dict(os.environ, **SAN_ENV, LD_PRELOAD=str(asan),
               HEATVIT_ORACLE_LIB=str(ROOT / "oracle" / "liboracle_san.so"))
    # the two 32-image forwards are left out (the seeded e2e model and the
    # single-image full model cover the same code)
    cmd = [sys.executable, "-m", "pytest", "-q", "-x", "-p", "no:cacheprovider",
           "tests/test_oracle_units.py", "tests/test_oracle_composite.py",
           "tests/test_ref_vectors_cpu.py", "tests/test_real_weights_cpu.py",
           "-k", "not pruned_model_matches and not pruned_batch_logits"]
    r = subprocess.run(cmd, cwd=ROOT, env=env, capture_output=True, text=True, timeout=900)
    tail = (r.stdout + r.stderr)[-3000:]
    assert r.returncode == 0, tail
    assert "passed" in r.stdout and "failed" not in r.stdout, tail


@pytest.mark.skipif(not HIPCC.exists() or not CLANG.exists(), reason="needs hipcc")
def test_device_math_under_asan_ubsan(tmp_path):
    san = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all"]
    obj = tmp_path / "hv_oracle.o"
    subprocess.run([str(CLANG), "-O1", "-g", *san, "-c", "-o", str(obj),
                    str(ROOT / "oracle" / "hv_oracle.c")], check=True)
    exe = tmp_path / "check_device_math_san"
    host_san = []
    for f in san:  # host code only: GPU code is never built with a sanitizer here
        host_san += ["-Xarch_host", f]
    r = subprocess.run([str(HIPCC), "-O1", "-g", "-std=c++17", *host_san,
                        "-I", str(ROOT / "heatvit_amd" / "csrc"), "-I", str(ROOT / "include"),
                        "-I", str(ROOT / "oracle"), "-o", str(exe),
                        str(ROOT / "tests" / "device_math" / "check_device_math.cpp"),
                        "-x", "none", str(obj)], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    out = subprocess.run([str(exe), "60000"], capture_output=True, text=True, timeout=600,
                         env=dict(os.environ, **SAN_ENV))
    assert out.returncode == 0, (out.stdout + out.stderr)[-2000:]
    assert "gelu_bad=0 softmax_bad=0 layernorm_bad=0" in out.stdout
