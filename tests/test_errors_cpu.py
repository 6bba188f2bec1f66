"""Error and warning parity without a GPU.

Host validation: every failing entry point returns the golden model's
exception class as its status and records the reference engine's error code
(heatvit_pkg.sv:109-118; docs/heatvit.md:751-763) -- the CPU-forcible half of
sim/tb/tb_heatvit_errors.sv.  These calls fail before any HIP call, so they
run here.  Warnings: the oracle's per-forward warning bits on parameter sets
that force each of the engine's three warnings (tests/warning_cases.py).
"""

import ctypes as C

import numpy as np
import pytest

import warning_cases as wc
from heatvit_amd import _lib, synth


@pytest.fixture(scope="module")
def L():
    if not _lib.LIB_PATH.exists():
        pytest.skip("libheatvit_hip.so not built")
    lib = C.CDLL(str(_lib.LIB_PATH))
    _lib._declare(lib)
    return lib


def _expect(L, rc, status, cls):
    assert rc == status, (rc, L.hv_last_error())
    assert L.hv_last_error_class() == cls, L.hv_last_error()
    assert L.hv_last_error()


def test_error_codes_match_the_engine(L):
    assert (_lib.HV_ERR_OPCODE, _lib.HV_ERR_DIMENSION, _lib.HV_ERR_ADDRESS,
            _lib.HV_ERR_TOKEN_COUNT, _lib.HV_ERR_MEMORY_PROTOCOL, _lib.HV_ERR_SOFTMAX_ZERO_SUM,
            _lib.HV_ERR_BUSY_START) == (1, 2, 3, 4, 5, 6, 7)
    assert (_lib.HV_WARN_HEAD_DEN_ZERO, _lib.HV_WARN_PACKAGE_DEN_ZERO,
            _lib.HV_WARN_LN_NEGATIVE_VARIANCE) == (1, 2, 4)


def test_primitive_and_layernorm_validation(L):
    buf = (C.c_int64 * 4)()
    _expect(L, L.hv_eval_primitive(7, buf, buf, 4, 0, 0, 0, None), _lib.HV_EVALUE,
            _lib.HV_ERR_OPCODE)
    _expect(L, L.hv_eval_primitive(_lib.HV_PRIM_REQUANT, buf, buf, 4, 0, 0, 64, None),
            _lib.HV_EVALUE, _lib.HV_ERR_DIMENSION)
    rows = (C.c_int8 * 192)()
    # layernorm input scale outside [-32, 0] (nonlinear.py:150-151)
    _expect(L, L.hv_layernorm_i8(rows, rows, rows, rows, 1, None, 1, -6, -7, -7, None, None),
            _lib.HV_EVALUE, _lib.HV_ERR_DIMENSION)
    _expect(L, L.hv_layernorm_i8(rows, rows, rows, rows, 1, None, -33, -6, -7, -7, None, None),
            _lib.HV_EVALUE, _lib.HV_ERR_DIMENSION)


def test_gemm_validation(L):
    a = (C.c_int8 * 4096)()
    d = _lib.GemmDesc(a=C.addressof(a), b_packed=C.addressof(a), c=C.addressof(a), m=1, n=32,
                      k=32, lda=32, ldc=32, epilogue=9)
    _expect(L, L.hv_gemm_i8(None, None), _lib.HV_EVALUE, _lib.HV_ERR_ADDRESS)
    _expect(L, L.hv_gemm_i8(C.byref(d), None), _lib.HV_EVALUE, _lib.HV_ERR_OPCODE)
    d.epilogue = _lib.HV_EPI_RESIDUAL
    _expect(L, L.hv_gemm_i8(C.byref(d), None), _lib.HV_EVALUE, _lib.HV_ERR_ADDRESS)
    d.epilogue = _lib.HV_EPI_I8
    d.k = 48  # K must be a positive multiple of 32
    _expect(L, L.hv_gemm_i8(C.byref(d), None), _lib.HV_EVALUE, _lib.HV_ERR_DIMENSION)
    d.k, d.n = 32, 0
    _expect(L, L.hv_gemm_i8(C.byref(d), None), _lib.HV_EVALUE, _lib.HV_ERR_DIMENSION)
    d.n, d.lda = 32, 40  # rows must stay 16-byte aligned
    _expect(L, L.hv_gemm_i8(C.byref(d), None), _lib.HV_EVALUE, _lib.HV_ERR_ADDRESS)
    d.lda, d.k = 131104, 131104  # int32 accumulator bound (gemm.py:116-117)
    _expect(L, L.hv_gemm_i8(C.byref(d), None), _lib.HV_EOVERFLOW, _lib.HV_ERR_DIMENSION)
    # unsigned A: K <= 65536 (255 * 128 * K < 2^31), whole rows only
    d.a_mode = _lib.HV_A_ROWS | _lib.HV_A_UNSIGNED
    d.lda, d.k = 65568, 65568
    _expect(L, L.hv_gemm_i8(C.byref(d), None), _lib.HV_EOVERFLOW, _lib.HV_ERR_DIMENSION)
    d.lda, d.k = 32, 32
    d.a_mode = _lib.HV_A_GATHER | _lib.HV_A_UNSIGNED
    d.a_rows = C.addressof(a)
    _expect(L, L.hv_gemm_i8(C.byref(d), None), _lib.HV_EVALUE, _lib.HV_ERR_OPCODE)


def test_block_selector_model_validation(L):
    blk = _lib.BlockDev()
    x = (C.c_int8 * 256)()
    off = (C.c_int32 * 2)(0, 1)
    _expect(L, L.hv_block_forward(None, x, off, 1, 1, x, None, None, None, x, 256, None),
            _lib.HV_EVALUE, _lib.HV_ERR_ADDRESS)
    _expect(L, L.hv_block_forward(C.byref(blk), x, off, 0, 1, x, None, None, None, x, 256,
                                  None), _lib.HV_EVALUE, _lib.HV_ERR_DIMENSION)
    blk.x_exp = 40  # scale exponent outside [-32, 31] (descriptor.py:186-188)
    _expect(L, L.hv_block_forward(C.byref(blk), x, off, 1, 1, x, None, None, None, x, 256,
                                  None), _lib.HV_EVALUE, _lib.HV_ERR_DIMENSION)
    blk.x_exp = 1  # a LayerNorm input scale above 0
    _expect(L, L.hv_block_forward(C.byref(blk), x, off, 1, 1, x, None, None, None, x, 256,
                                  None), _lib.HV_EVALUE, _lib.HV_ERR_DIMENSION)
    blk.x_exp = -7
    _expect(L, L.hv_block_forward(C.byref(blk), x, off, 1, 1, x, None, None, None, x, 256,
                                  None), _lib.HV_EVALUE, _lib.HV_ERR_ADDRESS)  # workspace
    sel = _lib.SelectorDev()
    _expect(L, L.hv_selector_forward(C.byref(sel), x, off, None, 1, x, None, x, off, off, off,
                                     None, x, 256, None), _lib.HV_EVALUE, _lib.HV_ERR_ADDRESS)
    _expect(L, L.hv_selector_finalize(x, off, None, None, 1, x, off, x, off, off, None),
            _lib.HV_EVALUE, _lib.HV_ERR_ADDRESS)
    m = _lib.ModelDev()
    logits = (C.c_int32 * 1000)()
    _expect(L, L.hv_model_forward(None, x, 1, logits, None, None, None, None, None, x, 256,
                                  None), _lib.HV_EVALUE, _lib.HV_ERR_ADDRESS)
    _expect(L, L.hv_model_forward(C.byref(m), x, 0, logits, None, None, None, None, None, x, 256,
                                  None), _lib.HV_EVALUE, _lib.HV_ERR_DIMENSION)
    m.n_selectors = 4
    _expect(L, L.hv_model_forward(C.byref(m), x, 1, logits, None, None, None, None, None, x, 256,
                                  None), _lib.HV_EVALUE, _lib.HV_ERR_DIMENSION)
    m.n_selectors = 3
    _expect(L, L.hv_model_forward(C.byref(m), x, 1, logits, None, None, None, None, None, x, 256,
                                  None), _lib.HV_EVALUE, _lib.HV_ERR_ADDRESS)  # workspace
    _expect(L, L.hv_model_forward(C.byref(m), x, 1 << 20, logits, None, None, None, None, None,
                                  x, 256, None), _lib.HV_EVALUE, _lib.HV_ERR_DIMENSION)
    # the _ex entries refuse option bits they do not know, and otherwise
    # validate as the plain entries do
    for entry in (L.hv_model_forward_ex, L.hv_model_forward_f32_ex):
        _expect(L, entry(C.byref(m), x, 1, logits, None, None, None, None, None, x, 256, 2, None),
                _lib.HV_EVALUE, _lib.HV_ERR_OPCODE)
        _expect(L, entry(C.byref(m), x, 1, logits, None, None, None, None, None, x, 256,
                         _lib.HV_FWD_PIPELINED, None), _lib.HV_EVALUE, _lib.HV_ERR_ADDRESS)


def test_success_clears_the_error_class(L):
    _expect(L, L.hv_gemm_i8(None, None), _lib.HV_EVALUE, _lib.HV_ERR_ADDRESS)
    assert L.hv_profile_read(None, None, 0) == _lib.HV_OK
    assert L.hv_last_error_class() == _lib.HV_ERR_NONE and L.hv_last_error() == b""


# ------------------------------------------------------------------ warnings


def test_oracle_ln_negative_variance_reaches_the_forward(oracle):
    imgs, params = synth.pruned_workload(2)
    p = wc.ln_negative_variance_model(synth.unpruned_control(params))
    _, ck = oracle.transformer_block(np.tile(wc.LN_NEG_ROW, (5, 1)), p.blocks[0])
    assert ck["warnings"] == oracle.WARN_LN_NEGATIVE_VARIANCE
    _, _, status, warnings = oracle.model_infer_batch(imgs, p, threads=2)
    assert not status.any() and warnings.tolist() == [oracle.WARN_LN_NEGATIVE_VARIANCE] * 2
    # the unmodified forward raises no warning
    _, _, _, warnings = oracle.model_infer_batch(imgs, params, threads=2)
    assert not warnings.any()


def test_oracle_selector_warnings_reach_the_forward(oracle):
    imgs, params = synth.pruned_workload(2)
    head = wc.with_selector(params, 0, wc.head_den_zero_selector)
    pkg = wc.with_selector(params, 2, wc.package_den_zero_selector)
    both = wc.with_selector(pkg, 1, wc.head_den_zero_selector)
    for p, want in ((head, oracle.WARN_HEAD_DEN_ZERO), (pkg, oracle.WARN_PACKAGE_DEN_ZERO),
                    (both, oracle.WARN_HEAD_DEN_ZERO | oracle.WARN_PACKAGE_DEN_ZERO)):
        _, counts, status, warnings = oracle.model_infer_batch(imgs, p, threads=2)
        assert not status.any() and warnings.tolist() == [want] * 2, (want, warnings)
        _, _, summary, w = oracle.model_infer(imgs[0], p, checkpoints=False)
        assert w == want and w == np.bitwise_or.reduce([s["warnings"] for s in summary])
    # every candidate of the last selector pruned: CLS + package remain
    assert counts[:, 3].tolist() == [2, 2]
