"""CPU-side checks of the HIP library and host layer: every symbol the
C header declares is exported, the weight packing is a lossless
permutation, parameter validation raises the reference's exception types,
and the synthetic generator is stable."""

import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

from heatvit_amd import synth
from heatvit_amd.device import pack_mfma32, unpack_mfma32
from heatvit_amd.params import MhsaParams, check_scale_exps

ROOT = Path(__file__).resolve().parents[1]
LIB = ROOT / "heatvit_amd" / "libheatvit_hip.so"


def _declared():
    text = (ROOT / "include" / "heatvit_hip.h").read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(hv_\w+)\(", text, re.M)))


@pytest.mark.skipif(not LIB.exists(), reason="library not built")
def test_library_exports_every_declared_symbol():
    names = _declared()
    assert len(names) >= 14
    lib = ctypes.CDLL(str(LIB))
    for n in names:
        assert hasattr(lib, n), n
    from heatvit_amd import _lib
    assert sorted(_lib.exported_symbols()) == names


def test_mfma32_packing_roundtrip_and_layout():
    rng = np.random.default_rng(1)
    for k, n in ((192, 576), (768, 192), (192, 1000), (32, 5)):
        w = rng.integers(-128, 128, (k, n)).astype(np.int8)
        p = pack_mfma32(w)
        assert p.size == -(-n // 32) * 32 * k
        assert np.array_equal(unpack_mfma32(p, k, n), w)
        # element (k, n) sits at tile (n/32, k/32), lane r(n%32) + 32*((k%32)/16),
        # byte k%16, with r(c) = 8*((c%16)/4) + 4*(c/16) + c%4 (include/heatvit_hip.h)
        for kk, nn in ((0, 0), (k - 1, n - 1), (17, min(33, n - 1)), (40 % k, min(21, n - 1))):
            c = nn % 32
            tile = (nn // 32) * (k // 32) + kk // 32
            lane = 8 * ((c % 16) // 4) + 4 * (c // 16) + c % 4 + 32 * ((kk % 32) // 16)
            assert p[tile * 1024 + lane * 16 + kk % 16] == w[kk, nn]
    # MFMA 32x32 result layout: lane l, element i is operand row
    # 8*(i//4) + 4*(l//32) + i%4; with this packing that row carries output
    # channel 16*(l//32) + i, so each lane ends with 16 contiguous channels.
    w = np.arange(32, dtype=np.int8)[None, :].repeat(32, 0)  # W[k][n] = n
    tile = pack_mfma32(w).reshape(64, 16)
    for lane in range(64):
        for i in range(16):
            row = 8 * (i // 4) + 4 * (lane // 32) + i % 4
            assert tile[row, 0] == 16 * (lane // 32) + i
    with pytest.raises(ValueError):
        pack_mfma32(np.zeros((17, 4), np.int8))


def test_params_validation_mirrors_reference():
    with pytest.raises(ValueError):
        MhsaParams(ln_gamma=[0] * 191, ln_beta=[0] * 192, wqkv=np.zeros((192, 576)),
                   bqkv=[0] * 576, wproj=np.zeros((192, 192)), bproj=[0] * 192)
    with pytest.raises(TypeError):
        MhsaParams(ln_gamma=[0.5] * 192, ln_beta=[0] * 192, wqkv=np.zeros((192, 576), int),
                   bqkv=[0] * 576, wproj=np.zeros((192, 192), int), bproj=[0] * 192)
    with pytest.raises(ValueError):
        MhsaParams(ln_gamma=[128] * 192, ln_beta=[0] * 192, wqkv=np.zeros((192, 576), int),
                   bqkv=[0] * 576, wproj=np.zeros((192, 192), int), bproj=[0] * 192)
    _, bp = synth.block_workload()
    check_scale_exps(bp)
    from dataclasses import replace
    with pytest.raises(ValueError):
        check_scale_exps(replace(bp, mhsa=replace(bp.mhsa, wqkv_scale_exp=40)))


def test_synthetic_generator_is_stable():
    # Digests pinned when the golden fixtures were written.
    import golden_io as gio
    meta, _ = gio.load("block")
    x, _ = synth.block_workload()
    assert gio.digest(x, np.int8) == meta["input_sha256"]
    w = synth.normal_i8(1, "t", (100000,))
    assert abs(float(w.astype(np.float64).std()) - 40.0) < 1.0
    assert abs(float(w.mean())) < 0.5
    u = synth.uniform_i8(1, "u", (100000,))
    assert u.min() == -128 and u.max() == 127
    for _ in range(3):
        e = synth._Exps(5, "p")("x")
        assert -12 <= e <= -4


def test_calibration_targets_recorded():
    cal = synth.load_calibration()
    assert abs(cal["selector"]["kept_fraction"] - 0.45) < 0.01
    means = [np.mean(c) for c in cal["pruned"]["calibration_token_counts"]]
    assert [round(m) for m in means] == list(synth.TOKEN_TARGETS)


def _abi_kind(t):
    """ctypes argtype reduced to what the C ABI sees: any pointer is a pointer."""
    if t is ctypes.c_void_p or (isinstance(t, type) and issubclass(t, ctypes._Pointer)):
        return "ptr"
    return ctypes.sizeof(t), t.__name__.replace("c_int32", "c_int")


def test_integration_example_matches_binding():
    """The ctypes example of INTEGRATION.md declares the argtypes that
    heatvit_amd._lib declares, and its call passes as many arguments as
    include/heatvit_hip.h's prototype has."""
    from heatvit_amd import _lib

    text = (ROOT / "INTEGRATION.md").read_text()
    block = text.split("### ctypes binding", 1)[1].split("```python", 1)[1].split("```", 1)[0]
    stmts = re.findall(r"^(lib\.hv_\w+\.(?:argtypes|restype) = (?:.*\\\n)*.*)$", block, re.M)
    assert any("hv_model_forward.argtypes" in s for s in stmts)

    class Fn:
        pass

    class Lib:
        def __getattr__(self, name):
            f = Fn()
            setattr(self, name, f)
            return f

    doc, ref = Lib(), Lib()
    for s in stmts:
        exec(s, {"ctypes": ctypes, "lib": doc})
    _lib._declare(ref)
    for name, fn in vars(doc).items():
        want = getattr(ref, name)
        if hasattr(fn, "argtypes"):
            assert [_abi_kind(t) for t in fn.argtypes] == \
                [_abi_kind(t) for t in want.argtypes], name
        if hasattr(fn, "restype"):
            assert fn.restype is want.restype, name

    header = (ROOT / "include" / "heatvit_hip.h").read_text()
    proto = re.search(r"int hv_model_forward\(([^)]*)\);", header).group(1)
    n_params = len(proto.split(","))
    assert n_params == len(doc.hv_model_forward.argtypes)
    call = re.search(r"lib\.hv_model_forward\((.*?)\)\n", block, re.S).group(1)
    depth, args = 0, 1
    for ch in call:
        depth += ch == "("
        depth -= ch == ")"
        args += ch == "," and depth == 0
    assert args == n_params
