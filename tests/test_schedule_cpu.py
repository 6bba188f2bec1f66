"""Descriptor front end on the CPU: hv_schedule_compile (host code) on the
reference's committed ROM, on the ROM the reference's generator builds for
this build's synthetic model (tests/golden/e2e_rom.mem), on the engine's
error-injection ROMs, and on mutated ROMs."""

import ctypes as C
import hashlib
import json
from pathlib import Path

import numpy as np
import pytest

import memory_image as mi
from heatvit_amd import _lib, synth
from heatvit_amd.schedule import read_rom

HERE = Path(__file__).resolve().parent
COMMITTED = HERE / "fixtures" / "descriptors" / "heatvit_descriptors.mem"
OURS = HERE / "golden" / "e2e_rom.mem"
META = json.loads((HERE / "golden" / "e2e.json").read_text())


@pytest.fixture(scope="module")
def L():
    if not _lib.LIB_PATH.exists():
        pytest.skip("libheatvit_hip.so not built")
    lib = C.CDLL(str(_lib.LIB_PATH))
    _lib._declare(lib)
    return lib


def compile_words(L, words):
    words = np.ascontiguousarray(words, np.uint8)
    s = _lib.Schedule()
    rc = L.hv_schedule_compile(words.ctypes.data, len(words), C.byref(s))
    return rc, L.hv_last_error_class(), s


def offsets(s):
    out = {n: getattr(s, n) for n in ("patch_w", "patch_b", "cls", "pos", "final_gamma",
                                      "final_beta", "head_w", "head_b")}
    for b in range(12):
        for n in _lib.SCHEDULE_BLOCK_TENSORS:
            out[f"b{b + 1}_{n}"] = getattr(s.blocks[b], n)
    for i in range(3):
        for n in _lib.SCHEDULE_SELECTOR_TENSORS:
            out[f"s{i + 1}_{n}"] = getattr(s.selectors[i], n)
    return out


def set_field(word, lsb, width, value):
    """Rewrites bits [lsb, lsb+width) of a little-endian 320-bit word."""
    v = int.from_bytes(bytes(word), "little")
    v = (v & ~(((1 << width) - 1) << lsb)) | ((value & ((1 << width) - 1)) << lsb)
    word[:] = np.frombuffer(v.to_bytes(40, "little"), np.uint8)


def test_committed_rom_compiles_to_the_reference_memory_map(L):
    assert hashlib.sha256(COMMITTED.read_bytes()).hexdigest() == META["committed_rom_sha256"]
    rc, cls, s = compile_words(L, read_rom(COMMITTED))
    assert rc == 0 and cls == 0, L.hv_last_error()
    assert offsets(s) == {k: v for k, v in META["weight_map"].items()}
    assert s.weight_bytes <= META["weight_bytes"]
    m = s.model
    assert m.n_selectors == 3 and list(m.selector_blocks) == [4, 7, 10]
    # the synthetic ROM's uniform scales (generate_descriptors.py:68-72)
    assert (m.patch.image_exp, m.patch.tokens_exp, m.final_ln_out_exp) == (-7, -7, -7)
    assert all(b.gamma1_exp == -6 and b.score_exp == -17 and b.prob_exp == -8
               for b in m.blocks)


def test_generated_rom_carries_the_model_exponents(L):
    params = synth.pruned_params()
    rc, cls, s = compile_words(L, read_rom(OURS))
    assert rc == 0, L.hv_last_error()
    assert offsets(s) == META["weight_map"]
    m, p = s.model, params
    assert (m.patch.image_exp, m.patch.weight_exp, m.patch.activation_exp, m.patch.tokens_exp,
            m.patch.cls_exp, m.patch.pos_exp) == (
        p.patch.image_scale_exp, p.patch.weight_scale_exp, p.patch.activation_scale_exp,
        p.patch.tokens_scale_exp, p.patch.cls_scale_exp, p.patch.pos_scale_exp)
    for e, bp in zip(m.blocks, p.blocks):
        mh, f = bp.mhsa, bp.ffn
        assert [getattr(e, n) for n in _lib.BLOCK_EXPS] == [
            mh.x_scale_exp, mh.gamma1_scale_exp, mh.beta1_scale_exp, mh.ln1_out_scale_exp,
            mh.wqkv_scale_exp, mh.qkv_out_scale_exp, mh.score_scale_exp, mh.prob_scale_exp,
            mh.context_out_scale_exp, mh.wproj_scale_exp, mh.msa_out_scale_exp, f.x_scale_exp,
            f.gamma2_scale_exp, f.beta2_scale_exp, f.ln2_out_scale_exp, f.w1_scale_exp,
            f.hidden_out_scale_exp, f.w2_scale_exp, f.ffn_out_scale_exp, f.out_scale_exp]
    for e, sp in zip(m.selectors, p.selectors):
        assert [getattr(e, n) for n in _lib.SELECTOR_EXPS] == [
            sp.in_scale_exp, sp.local_w_scale_exp, sp.local_out_scale_exp,
            sp.concat_out_scale_exp, sp.score_w1_scale_exp, sp.score_w2_scale_exp,
            sp.score_w3_scale_exp, sp.h1_out_scale_exp, sp.h2_out_scale_exp,
            sp.logits_out_scale_exp, sp.stats_out_scale_exp, sp.hw_w1_scale_exp,
            sp.hw_hidden_out_scale_exp, sp.hw_w2_scale_exp]
    assert (m.final_gamma_exp, m.final_beta_exp, m.final_ln_out_exp, m.head_w_exp) == (
        p.final_gamma_scale_exp, p.final_beta_scale_exp, p.final_ln_out_scale_exp,
        p.head_w_scale_exp)
    # the weight region at the compiled offsets is the reference's serialize_weights
    region = mi.weight_region(params, s)
    assert len(region) == META["weights_len"]
    assert hashlib.sha256(region).hexdigest() == META["weights_sha256"]


@pytest.mark.parametrize("name,cls", [("err1_opcode", _lib.HV_ERR_OPCODE),
                                      ("err2_dimension", _lib.HV_ERR_DIMENSION),
                                      ("err3_address", _lib.HV_ERR_ADDRESS)])
def test_error_roms_get_the_engine_code(L, name, cls):
    rc, got, _ = compile_words(L, read_rom(HERE / "golden" / "e2e_errors" / f"{name}.mem"))
    assert rc == _lib.HV_EVALUE and got == cls, L.hv_last_error()


def test_injection_roms_are_not_a_heatvit_schedule(L):
    """The other injection ROMs are legal descriptors whose faults the
    engine's bench forces at run time; as schedules they are rejected."""
    for f in sorted((HERE / "golden" / "e2e_errors").glob("*.mem")):
        rc, cls, _ = compile_words(L, read_rom(f))
        assert rc == _lib.HV_EVALUE and cls in (_lib.HV_ERR_OPCODE, _lib.HV_ERR_DIMENSION,
                                                _lib.HV_ERR_ADDRESS), f.name


def test_mutated_roms(L):
    base = read_rom(OURS).copy()

    def expect(mutate, cls):
        w = base.copy()
        mutate(w)
        rc, got, _ = compile_words(L, w)
        assert rc == _lib.HV_EVALUE and got == cls, L.hv_last_error()

    expect(lambda w: set_field(w[7], 312, 8, 0x5A), _lib.HV_ERR_OPCODE)       # opcode
    expect(lambda w: set_field(w[7], 0, 4, 1), _lib.HV_ERR_DIMENSION)         # reserved
    expect(lambda w: set_field(w[7], 288 + 22, 2, 1), _lib.HV_ERR_DIMENSION)  # flag 22
    expect(lambda w: set_field(w[7], 288 + 8, 3, 7), _lib.HV_ERR_DIMENSION)   # post-op 7
    expect(lambda w: set_field(w[4], 204, 32, 0x1004), _lib.HV_ERR_ADDRESS)   # src0 offset
    expect(lambda w: set_field(w[4], 70, 6, 5), _lib.HV_ERR_DIMENSION)        # QKV s0 chain
    expect(lambda w: set_field(w[3], 256, 16, 64), _lib.HV_ERR_DIMENSION)     # LN over 64
    # weight GEMMs (patch 1, QKV 4, proj 10, selector-1 local 42, its score
    # layer 3 47, head-weight 50) with transposed or swapped operands, an
    # unsigned activation or an int32 output; the classifier without int32
    for idx in (1, 4, 10, 42, 47, 50):
        for flag in (0, 4, 7, 18):
            expect(lambda w: set_field(w[idx], 288 + flag, 1, 1), _lib.HV_ERR_DIMENSION)
    expect(lambda w: set_field(w[len(w) - 2], 288 + 7, 1, 0), _lib.HV_ERR_DIMENSION)
    rc, cls, _ = compile_words(L, base[:150])                                  # truncated
    assert rc == _lib.HV_EVALUE and cls == _lib.HV_ERR_OPCODE
    rc, cls, _ = compile_words(L, np.concatenate([base, base[-1:]]))          # after FINISH
    assert rc == _lib.HV_EVALUE and cls == _lib.HV_ERR_DIMENSION
    w = base.copy()
    set_field(w[1], 288 + 12, 1, 1)  # patch weights from the scratch region
    rc, cls, _ = compile_words(L, w)
    assert rc == _lib.HV_EVALUE and cls == _lib.HV_ERR_ADDRESS
