"""Builds libheatvit_hip.so (gfx950) from heatvit_amd/csrc with hipcc.

Every .hip file is compiled to an object in parallel, then linked into one
shared library next to this file.  Run `python -m heatvit_amd.build`.
"""

import hashlib
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
LIB = HERE / "libheatvit_hip.so"
OBJ = HERE / "_obj"
ARCH = os.environ.get("HEATVIT_ARCH", "gfx950")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-Wall",
    "-Wno-unused-function", "-Wno-unused-variable",
    # Packed FP32 instructions are kept out of every code object.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA accumulators in ordinary VGPRs: the epilogues then read them
    # without a v_accvgpr_read per element (and need fewer registers).
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    "-I", str(HERE.parent / "include"), "-I", str(OBJ),
]


def _compile(src):
    obj = OBJ / (src.stem + ".o")
    cmd = [HIPCC, *FLAGS, "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    errs = "\n".join(l for l in (r.stderr or "").splitlines()
                     if "packed-fp32-ops" not in l)
    return src.name, r.returncode, errs, obj


def _gelu_tables():
    """Writes _obj/gelu_lut.inc with gen_gelu_lut.py unless the file was
    made by the same generator source (its SHA-256 on the first line)."""
    gen = CSRC / "gen_gelu_lut.py"
    out = OBJ / "gelu_lut.inc"
    tag = "// generator " + hashlib.sha256(gen.read_bytes()).hexdigest() + "\n"
    if out.exists() and out.read_text().startswith(tag):
        return
    tmp = out.with_suffix(".tmp")
    subprocess.run([sys.executable, str(gen), str(tmp)], check=True)
    out.write_text(tag + tmp.read_text())
    tmp.unlink()


def build(verbose=True):
    OBJ.mkdir(exist_ok=True)
    _gelu_tables()
    sources = sorted(CSRC.glob("*.hip"))
    with ThreadPoolExecutor(max_workers=min(8, len(sources))) as ex:
        results = list(ex.map(_compile, sources))
    failed = False
    for name, rc, errs, _ in results:
        if errs.strip() and verbose:
            print(f"[{name}]\n{errs}", file=sys.stderr)
        failed |= rc != 0
    if failed:
        raise RuntimeError("HIP compilation failed")
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp),
           *[str(o) for *_, o in results]]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("link failed:\n" + r.stderr)
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build()
