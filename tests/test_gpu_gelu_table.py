"""GPU parity of the FFN GELU post-op step tables: requant(gelu(q), -16,
so - 16, 8) read from the tables equals the evaluated post-op for every q
of the 24-bit Q8.16 domain and every table (so in [3, 12]), and the
evaluated post-op equals the oracle (nonlinear.gelu, fixed.requant) on a
spread of the domain."""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _prim(op, x, so):
    import torch
    from heatvit_amd import _lib
    out = torch.empty_like(x)
    _lib.check(_lib.lib().hv_eval_primitive(op, x.data_ptr(), out.data_ptr(), x.numel(), so, 0,
                                            0, torch.cuda.current_stream().cuda_stream),
               "gelu post")
    return out


def test_tables_match_post_op_on_whole_domain():
    import torch
    from heatvit_amd import _lib
    q = torch.arange(-(1 << 23), 1 << 23, dtype=torch.int64, device="cuda")
    for so in _lib.GELU_TABLE_SO:
        exact = _prim(_lib.HV_PRIM_GELU_POST, q, so)
        table = _prim(_lib.HV_PRIM_GELU_TABLE, q, so)
        bad = (exact != table).nonzero()
        assert bad.numel() == 0, (so, q[bad[:5, 0]].tolist())


@pytest.mark.parametrize("so", [3, 7, 12, 0, -5, 20])
def test_post_op_matches_oracle(oracle, so):
    from heatvit_amd.ops import gelu_post
    rng = np.random.default_rng(so + 40)
    q = np.concatenate([np.arange(-70000, 70000, 7), rng.integers(-(1 << 23), 1 << 23, 20000),
                        [-(1 << 23), (1 << 23) - 1, -1, 0, 1, 1 << 30, -(1 << 40)]]).astype(np.int64)
    qs = np.clip(q, -(1 << 23), (1 << 23) - 1)
    want = oracle.requant_array(oracle.gelu_array(qs), -16, so - 16, 8)
    assert np.array_equal(gelu_post(q, so), want)
    if 3 <= so <= 12:
        assert np.array_equal(gelu_post(q, so, table=True), want)


def test_table_range_is_checked():
    from heatvit_amd import _lib
    from heatvit_amd.ops import gelu_post
    with pytest.raises(ValueError):
        gelu_post([0, 1], 2, table=True)
    with pytest.raises(ValueError):
        gelu_post([0, 1], 13, table=True)
    assert _lib.lib().hv_last_error_class() == _lib.HV_ERR_DIMENSION


@pytest.mark.parametrize("src", [-14, -19])
def test_ffn_gemm_gelu_every_table(oracle, src):
    # The FFN1 shape (K = 192, N = 768) through the GEMM's GELU epilogue for
    # every output shift with a step table (so = dst + 16 in [3, 12], one-
    # and three-change tables) and the evaluated neighbours (so = 2, 13);
    # src = -14 shifts the product left, -19 right.
    from heatvit_amd import ops
    rng = np.random.default_rng(-src)
    m, k, n = 300, 192, 768
    a = rng.integers(-128, 128, (m, k))
    a[::7] //= 64                      # rows whose q stays near zero
    w = rng.integers(-128, 128, (k, n))
    bias = rng.integers(-(1 << 18), 1 << 18, n)
    acc = oracle.gemm(a, w, bias)
    q = oracle.requant_array(acc, src, -16, 24)
    y = oracle.gelu_array(q).astype(np.int64)
    for dst in range(-14, -2):
        want = oracle.requant_array(y, -16, dst, 8)
        got = ops.gemm_writeback(a, w, bias, src, dst, 8, epilogue="gelu")
        assert np.array_equal(got, want), (src, dst)
