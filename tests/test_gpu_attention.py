"""GPU parity of the attention core entry point (hv_attention_i8: score,
softmax_attention, P.V and head_concat of transformer.mhsa,
transformer.py:228-266) against the golden block fixture and the CPU
oracle's mhsa checkpoints, bit-exact."""

import dataclasses

import numpy as np
import pytest

import golden_io as gio
from heatvit_amd import synth

pytestmark = pytest.mark.gpu


def _exps(m):
    return m.qkv_out_scale_exp, m.score_scale_exp, m.prob_scale_exp, m.context_out_scale_exp


def test_attention_matches_golden_block(oracle):
    from heatvit_amd.ops import attention
    meta, _ = gio.load("block")
    x, bp = synth.block_workload()
    _, ck = oracle.transformer_block(x, bp)
    assert gio.digest(ck["fused_qkv"], gio.BLOCK_DTYPES["fused_qkv"]) == \
        meta["checkpoints"]["fused_qkv"]
    [(score, prob, concat)] = attention([ck["fused_qkv"]], *_exps(bp.mhsa))
    for key, got in (("score", score), ("prob", prob), ("concat", concat)):
        assert gio.digest(got, gio.BLOCK_DTYPES[key]) == meta["checkpoints"][key], key


def peaky_qkv(rng, n):
    """fused_qkv [n][576] whose keys repeat the queries with per-row
    magnitudes from 1 to 127: attention rows range from flat to one-hot."""
    mag = rng.integers(1, 128, (n, 1))
    q = (rng.integers(-128, 128, (n, 192)) * mag // 128).astype(np.int8)
    k = q.copy()
    flip = rng.random((n, 192)) < 0.2
    k[flip] = rng.integers(-128, 128, flip.sum())
    v = rng.integers(-128, 128, (n, 192)).astype(np.int8)
    return np.concatenate([q, k, v], axis=1)


EXPS = [
    (-4, -11, -8, -4),   # the block fixture's exponents (score = 2*qkv - 3)
    (-4, -6, -8, -4),    # q16 by a left shift (score_exp + 13 > 0)
    (-4, -31, -8, -4),   # q16 rounds 18 bits away; rows flatten
    (-7, -17, -8, -12),  # context requant by a left shift
    (-4, -11, -8, 20),   # context shift beyond the int32 rounding range
    (-2, 10, -8, -4),    # score requant drops bits before the q16 step
]


@pytest.mark.parametrize("exps", EXPS)
def test_attention_ragged_vs_oracle(oracle, exps):
    from heatvit_amd.ops import attention
    rng = np.random.default_rng(11)
    lens = [197, 1, 63, 64, 65, 2, 150, 16, 17]
    qkvs = [peaky_qkv(rng, n) for n in lens]
    got = attention(qkvs, *exps)
    for i, (qkv, (score, prob, concat)) in enumerate(zip(qkvs, got)):
        want = oracle.attention(qkv, *exps)
        assert np.array_equal(score, want[0]), i
        assert np.array_equal(prob, want[1]), i
        assert np.array_equal(concat, want[2]), i


def test_attention_reports_bad_token_counts():
    import torch
    from heatvit_amd import _lib
    L = _lib.lib()
    qkv = torch.zeros((300, 576), dtype=torch.int8, device="cuda")
    ctx = torch.zeros((300, 192), dtype=torch.int8, device="cuda")
    # image 0: 197 rows; image 1: no rows; image 2: 198 rows (too many)
    off = torch.tensor([0, 197, 197, 395], dtype=torch.int32, device="cuda")
    status = torch.full((4,), 99, dtype=torch.int32, device="cuda")
    rc = L.hv_attention_i8(qkv.data_ptr(), off.data_ptr(), 3, 300, ctx.data_ptr(), None, None,
                           -4, -11, -8, -4, status.data_ptr(),
                           torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    torch.cuda.synchronize()
    assert status[:3].tolist() == [0, _lib.HV_ERR_TOKEN_COUNT, _lib.HV_ERR_TOKEN_COUNT]
    # image 1: 123 rows, ending past the 300-row buffer
    off = torch.tensor([0, 197, 320], dtype=torch.int32, device="cuda")
    rc = L.hv_attention_i8(qkv.data_ptr(), off.data_ptr(), 2, 300, ctx.data_ptr(), None, None,
                           -4, -11, -8, -4, status.data_ptr(),
                           torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    torch.cuda.synchronize()
    assert status[:2].tolist() == [0, _lib.HV_ERR_TOKEN_COUNT]


def test_attention_rejects_bad_arguments():
    import torch
    from heatvit_amd import _lib
    L = _lib.lib()
    qkv = torch.zeros((16, 576), dtype=torch.int8, device="cuda")
    ctx = torch.zeros((16, 192), dtype=torch.int8, device="cuda")
    off = torch.tensor([0, 16], dtype=torch.int32, device="cuda")
    s = torch.cuda.current_stream().cuda_stream
    rc = L.hv_attention_i8(qkv.data_ptr(), off.data_ptr(), 1, 16, ctx.data_ptr(), None, None,
                           -4, 40, -8, -4, None, s)
    assert rc == _lib.HV_EVALUE and L.hv_last_error_class() == _lib.HV_ERR_DIMENSION
    rc = L.hv_attention_i8(qkv.data_ptr() + 4, off.data_ptr(), 1, 15, ctx.data_ptr(), None,
                           None, -4, -11, -8, -4, None, s)
    assert rc == _lib.HV_EVALUE and L.hv_last_error_class() == _lib.HV_ERR_ADDRESS
    with pytest.raises(ValueError):
        from heatvit_amd.ops import attention
        attention([np.zeros((198, 576), np.int8)], -4, -11, -8, -4)
