"""GPU parity of the composite stages: the HIP transformer block, token
selector, patch embedding and full model against the reference golden
model's fixtures (tests/golden) and the CPU oracle, bit-exact."""

import numpy as np
import pytest

import golden_io as gio
from heatvit_amd import synth

pytestmark = pytest.mark.gpu


def _block_ck_digests(ck):
    return {k: gio.digest(v, gio.BLOCK_DTYPES[k]) for k, v in ck.items()
            if k in gio.BLOCK_DTYPES}


def test_block_matches_golden():
    from heatvit_amd.transformer import transformer_block
    meta, arrays = gio.load("block")
    x, bp = synth.block_workload()
    z, ck = transformer_block(x, bp)
    assert np.array_equal(z, arrays["z"])
    got = _block_ck_digests(ck)
    bad = [k for k, v in meta["checkpoints"].items() if got.get(k) != v]
    assert not bad, bad


def test_block_ragged_batch_vs_oracle(oracle):
    from heatvit_amd.transformer import transformer_block_batch
    x, bp = synth.block_workload()
    rng = np.random.default_rng(3)
    lens = [197, 100, 17, 1, 64, 2, 197, 45]
    xs = [rng.integers(-128, 128, (n, 192)).astype(np.int8) for n in lens]
    xs[0] = x
    zs, cks = transformer_block_batch(xs, bp, checkpoints=True)
    for i, xi in enumerate(xs):
        z, ck = oracle.transformer_block(xi, bp)
        assert np.array_equal(zs[i], z), i
        for k in ("ln1", "fused_qkv", "score", "prob", "msa", "y", "ln2", "hidden", "ffn_out",
                  "qkv", "context", "concat"):
            assert np.array_equal(cks[i][k], ck[k]), (i, k)


@pytest.mark.parametrize("wide", ["b1", "b2", "both"])
def test_fused_ffn_wide_biases_and_ragged_rows_vs_oracle(oracle, wide):
    """Without checkpoints the block's FFN runs as one fused kernel (hidden
    rows in LDS); an FFN1 or FFN2 bias beyond the int32 epilogue bound sends
    that phase to the exact 64-bit forms, and ragged images leave partial
    64-row blocks."""
    import dataclasses
    from heatvit_amd.transformer import transformer_block_batch
    _, bp = synth.block_workload()
    b1 = np.asarray(bp.ffn.b1).astype(np.int64).copy()
    b2 = np.asarray(bp.ffn.b2).astype(np.int64).copy()
    if wide in ("b1", "both"):
        b1[5] = (1 << 31) - 1
        b1[300:310] = -(1 << 31)
        b1[700] = (1 << 30)
    if wide in ("b2", "both"):
        b2[0] = -(1 << 31)
        b2[191] = (1 << 31) - 1
        b2[77] = -(1 << 30)
    bp = dataclasses.replace(bp, ffn=dataclasses.replace(bp.ffn, b1=b1, b2=b2))
    rng = np.random.default_rng(8)
    lens = [197, 63, 1, 65, 130, 197, 7]
    xs = [rng.integers(-128, 128, (n, 192)).astype(np.int8) for n in lens]
    zs = transformer_block_batch(xs, bp)
    for i, x in enumerate(xs):
        z, _ = oracle.transformer_block(x, bp, checkpoints=False)
        assert np.array_equal(zs[i], z), i


@pytest.mark.parametrize("blk,tail", [(0, 0), (5, 1), (10, 2)])
def test_fused_ffn_split_last_blocks_vs_oracle(oracle, blk, tail):
    """A block over 32,768 rows or more runs the fused FFN in 64-row blocks
    whose last few, beyond whole rounds of one block per CU, are split into
    32-row blocks (the second row tile's steps skipped): 168 images of 197
    rows are 33,096 rows, 512 whole blocks and 11 halves, the last of 8 rows;
    `tail` trims the last images so the final half ends mid-tile."""
    from heatvit_amd.transformer import transformer_block_batch
    _, params = synth.throughput_workload(1)
    bp = params.blocks[blk]
    rng = np.random.default_rng(40 + blk)
    lens = [197] * 168
    if tail == 1:
        lens[-1] = 150  # 33,049 rows: 512 whole blocks, 9 halves, the last of 25 rows
    elif tail == 2:
        lens[-1:] = [1, 30, 64]  # 32,994 rows: 8 halves, the last of 2 rows
    xs = [rng.integers(-128, 128, (n, 192)).astype(np.int8) for n in lens]
    assert sum(lens) >= 32768
    zs = transformer_block_batch(xs, bp)
    for i, x in enumerate(xs):
        z, _ = oracle.transformer_block(x, bp, checkpoints=False)
        assert np.array_equal(zs[i], z), (blk, i, len(x))


def test_fused_ffn_split_blocks_past_the_live_rows_vs_oracle(oracle):
    """The row capacity sizes the launch (33,096 rows: 512 whole blocks and
    11 halves) while the batch's offsets hold 32,900 live rows: the fifth
    half keeps 4 live rows, the last six exit before any work, and the rows
    past the live count are never written."""
    import torch
    from heatvit_amd import _lib
    from heatvit_amd.device import DeviceBlock
    _, params = synth.throughput_workload(1)
    bp = params.blocks[3]
    rng = np.random.default_rng(77)
    lens = [197] * 167 + [1]
    live, cap = sum(lens), 33096
    assert live == 32900
    xs = [rng.integers(-128, 128, (n, 192)).astype(np.int8) for n in lens]
    x = np.concatenate(xs + [rng.integers(-128, 128, (cap - live, 192)).astype(np.int8)])
    offsets = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    L = _lib.lib()
    db = DeviceBlock(bp)
    xd = torch.from_numpy(x).cuda()
    off = torch.from_numpy(offsets).cuda()
    z = torch.full((cap, 192), 55, dtype=torch.int8, device="cuda")
    ws = torch.empty(L.hv_block_workspace_bytes(len(lens), cap), dtype=torch.uint8, device="cuda")
    _lib.check(L.hv_block_forward(db.struct, xd.data_ptr(), off.data_ptr(), len(lens), cap,
                                  z.data_ptr(), None, None, None, ws.data_ptr(), ws.numel(),
                                  torch.cuda.current_stream().cuda_stream), "block")
    zs = z.cpu().numpy()
    assert (zs[live:] == 55).all()
    for i, xi in enumerate(xs):
        want, _ = oracle.transformer_block(xi, bp, checkpoints=False)
        assert np.array_equal(zs[offsets[i]:offsets[i + 1]], want), (i, len(xi))


# Ragged token counts of a pruned stage: partial 32-row tiles and 64-row
# FFN blocks, images of one and two key tiles, many small images; 32 images,
# so the attention kernel runs the QKV GEMM.
RAGGED_LENS = [1, 2, 16, 17, 31, 32, 33, 48, 63, 64, 65, 100, 128, 129, 150, 197] + [3] * 16


def _ragged_batch(rng, lens=RAGGED_LENS):
    return [rng.integers(-128, 128, (n, 192)).astype(np.int8) for n in lens]


@pytest.mark.parametrize("blk", range(12))
def test_block_every_model_block_ragged_vs_oracle(oracle, blk):
    """Every block of the 256-image workload's model (its requant
    directions, attention modes and GELU tables differ) over a ragged batch
    of mostly small images, against the oracle."""
    from heatvit_amd.transformer import transformer_block_batch
    _, params = synth.throughput_workload(1)
    bp = params.blocks[blk]
    xs = _ragged_batch(np.random.default_rng(100 + blk))
    zs = transformer_block_batch(xs, bp)
    for i, x in enumerate(xs):
        z, _ = oracle.transformer_block(x, bp, checkpoints=False)
        assert np.array_equal(zs[i], z), (blk, i, len(x))


def _block_launches(xs, bp, checkpoints):
    """Block forward with kernel-class profiling: outputs and launches per class."""
    from heatvit_amd import _lib
    from heatvit_amd.transformer import transformer_block_batch
    L = _lib.lib()
    L.hv_profile_enable(1)
    try:
        out = transformer_block_batch(xs, bp, checkpoints=checkpoints)
        ms = np.zeros(len(_lib.PROF_CLASSES), np.float32)
        n = np.zeros(len(_lib.PROF_CLASSES), np.int32)
        _lib.check(L.hv_profile_read(ms.ctypes.data, n.ctypes.data, len(ms)), "profile")
    finally:
        L.hv_profile_enable(0)
    return out, dict(zip(_lib.PROF_CLASSES, n.tolist()))


def test_block_ln2_inside_fused_ffn_vs_oracle(oracle):
    """Without checkpoints the QKV GEMM runs inside the attention kernel (32
    images or more) and the attention projection and LayerNorm 2 inside the
    fused FFN kernel (y and the LN2 rows pass through LDS): one LayerNorm
    launch per block (LN1), one attention and one FFN launch.  A batch of 8
    keeps the QKV launch.  With checkpoints QKV, the projection and LN2 have
    launches of their own, which write the fused_qkv, y and ln2 checkpoints,
    and FFN1 / FFN2 run as two GEMMs (the hidden checkpoint).  All match the
    oracle over ragged images (partial 32-row tiles and 64-row blocks)."""
    _, bp = synth.block_workload()
    xs = _ragged_batch(np.random.default_rng(21))
    zs, n = _block_launches(xs, bp, False)
    assert n["layernorm"] == 1 and n["ffn"] == 1 and n["gemm_proj"] == 0, n
    assert n["gemm_ffn1"] == 0 and n["gemm_ffn2"] == 0, n
    assert n["gemm_qkv"] == 0 and n["attention"] == 1, n
    zs8, n8 = _block_launches(xs[8:16], bp, False)
    assert n8["gemm_qkv"] == 1 and n8["attention"] == 1 and n8["ffn"] == 1, n8
    for i, x in enumerate(xs[8:16]):
        assert np.array_equal(zs8[i], zs[8 + i]), i
    (zs_ck, cks), n_ck = _block_launches(xs, bp, True)
    assert n_ck["layernorm"] == 2 and n_ck["ffn"] == 0 and n_ck["gemm_proj"] == 1, n_ck
    assert n_ck["gemm_qkv"] == 1, n_ck
    for i, x in enumerate(xs):
        z, ck = oracle.transformer_block(x, bp, checkpoints=True)
        assert np.array_equal(zs[i], z), (i, len(x))
        assert np.array_equal(zs_ck[i], z), (i, len(x))
        assert np.array_equal(cks[i]["ln2"], ck["ln2"]), (i, len(x))
        assert np.array_equal(cks[i]["y"], ck["y"]), (i, len(x))
        assert np.array_equal(cks[i]["fused_qkv"], ck["fused_qkv"]), (i, len(x))


@pytest.mark.parametrize("msa_exp,ffn_x_exp,dirs", [(-7, -11, 0), (-13, -12, 1), (-7, -12, 2),
                                                    (-11, -12, 3)])
def test_block_projection_requant_directions_in_ffn_kernel_vs_oracle(oracle, msa_exp,
                                                                     ffn_x_exp, dirs):
    """The projection inside the fused FFN kernel with each pair of requant
    directions (bit 0: the product's requant shifts left, msa_out at or
    below context_out + wproj; bit 1: the residual align-add's output shift
    is not positive), over 32 ragged images without checkpoints: no
    projection launch, and z equal to the oracle's."""
    import dataclasses
    _, bp = synth.block_workload()
    m, f = bp.mhsa, bp.ffn
    shift_a = msa_exp - (m.context_out_scale_exp + m.wproj_scale_exp)
    os_ = ffn_x_exp - min(m.x_scale_exp, msa_exp)
    assert (shift_a <= 0) + 2 * (os_ <= 0) == dirs
    bp = dataclasses.replace(bp, mhsa=dataclasses.replace(m, msa_out_scale_exp=msa_exp),
                             ffn=dataclasses.replace(f, x_scale_exp=ffn_x_exp))
    xs = _ragged_batch(np.random.default_rng(40 + dirs))
    zs, n = _block_launches(xs, bp, False)
    assert n["gemm_proj"] == 0 and n["ffn"] == 1 and n["layernorm"] == 1, n
    for i, x in enumerate(xs):
        z, _ = oracle.transformer_block(x, bp, checkpoints=False)
        assert np.array_equal(zs[i], z), (i, len(x))


@pytest.mark.parametrize("qkv_exp,score_exp", [(-9, -21), (-4, -11), (-9, -7), (-19, -30)])
def test_block_attention_with_qkv_in_kernel_exponents_vs_oracle(oracle, qkv_exp, score_exp):
    """The QKV GEMM inside the attention kernel over 32 ragged images without
    checkpoints, under the score paths of the int32 Q8.16 conversion (a
    right shift, a plain saturation, the general two-step form) and a QKV
    requant that shifts left (the last case): no QKV launch, z equal to the
    oracle's."""
    import dataclasses
    _, bp = synth.block_workload()
    bp = dataclasses.replace(bp, mhsa=dataclasses.replace(
        bp.mhsa, qkv_out_scale_exp=qkv_exp, score_scale_exp=score_exp))
    xs = _ragged_batch(np.random.default_rng(60 - qkv_exp))
    zs, n = _block_launches(xs, bp, False)
    assert n["gemm_qkv"] == 0 and n["attention"] == 1, n
    for i, x in enumerate(xs):
        z, _ = oracle.transformer_block(x, bp, checkpoints=False)
        assert np.array_equal(zs[i], z), (i, len(x))


def test_block_wide_biases_all_gemms_vs_oracle(oracle):
    """Biases beyond the int32 epilogue bounds in all four GEMMs send their
    tiles to the exact 64-bit forms (the projection's inside the fused FFN
    kernel, as the block runs without checkpoints)."""
    import dataclasses
    from heatvit_amd.transformer import transformer_block_batch
    _, bp = synth.block_workload()
    f = lambda v: np.asarray(v).astype(np.int64).copy()
    bqkv, bproj, b1, b2 = f(bp.mhsa.bqkv), f(bp.mhsa.bproj), f(bp.ffn.b1), f(bp.ffn.b2)
    bqkv[[0, 200, 575]] = [(1 << 31) - 1, -(1 << 31), 1 << 30]
    bproj[[3, 191]] = [-(1 << 31), (1 << 31) - 1]
    b1[[5, 300, 767]] = [(1 << 31) - 1, -(1 << 31), -(1 << 30)]
    b2[[0, 100]] = [-(1 << 31), (1 << 31) - 1]
    bp = dataclasses.replace(bp, mhsa=dataclasses.replace(bp.mhsa, bqkv=bqkv, bproj=bproj),
                             ffn=dataclasses.replace(bp.ffn, b1=b1, b2=b2))
    xs = _ragged_batch(np.random.default_rng(9))
    zs = transformer_block_batch(xs, bp)
    for i, x in enumerate(xs):
        z, _ = oracle.transformer_block(x, bp, checkpoints=False)
        assert np.array_equal(zs[i], z), (i, len(x))


def test_selector_matches_golden():
    from heatvit_amd.selector import token_selector_batch
    meta, arrays = gio.load("selector")
    tokens, sp = synth.selector_workload()
    res = token_selector_batch(list(tokens), [False] * len(tokens), sp)
    for i, (r, want) in enumerate(zip(res, meta["results"])):
        assert r.token_count == want["token_count"], i
        assert r.kept_normal_count == want["kept_normal_count"], i
        assert r.pruned_normal_count == want["pruned_normal_count"], i
        assert r.warnings == want["warnings"], i
        assert int(r.package_present) == want["package_present"], i
        assert gio.digest(r.tokens, np.int8) == want["tokens_sha256"], i
        assert gio.digest(r.local, np.int8) == want["local_sha256"], i
        assert gio.digest(r.global_features, np.int8) == want["global_sha256"], i
        assert gio.digest(r.head_scores, "<i4") == want["head_scores_sha256"], i
        assert gio.digest(r.head_stats, np.int8) == want["head_stats_sha256"], i
        assert gio.digest(r.head_weights, "<i4") == want["head_weights_sha256"], i
        assert np.array_equal(r.fused_scores, arrays["fused"][i]), i
        if r.package_present:
            assert np.array_equal(r.tokens[-1], arrays["package"][i]), i
        assert np.array_equal(r.kept_index, np.nonzero(arrays["fused"][i] >= 32768)[0])


def test_selector_ragged_with_packages_vs_oracle(oracle):
    from heatvit_amd.selector import token_selector_batch
    tokens, sp = synth.selector_workload()
    rng = np.random.default_rng(4)
    lens = [197, 3, 2, 90, 45, 150, 33]
    flags = [False, True, False, True, True, False, True]
    sets = [tokens[i][:n] if i % 2 == 0 else rng.integers(-128, 128, (n, 192)).astype(np.int8)
            for i, n in enumerate(lens)]
    res = token_selector_batch(sets, flags, sp)
    for i, (t, f) in enumerate(zip(sets, flags)):
        want = oracle.token_selector(t, f, sp)
        r = res[i]
        assert np.array_equal(r.tokens, want["tokens"]), i
        assert np.array_equal(r.fused_scores, want["fused_scores"]), i
        assert np.array_equal(r.kept_index, want["kept_index"]), i
        assert (r.token_count, r.warnings, r.pruned_normal_count) == \
            (want["token_count"], want["warnings"], want["pruned_normal_count"]), i


def test_patch_embedding_vs_golden_and_oracle(oracle):
    from heatvit_amd.transformer import patch_embedding
    meta, _ = gio.load("full")
    img, params = synth.full_workload()
    x = patch_embedding(img[0], params.patch)
    assert gio.digest(x, np.int8) == meta["checkpoints"][0]["patch"]
    imgs, pp = synth.pruned_workload(5)
    xb = patch_embedding(imgs, pp.patch, batch=True)
    for i in range(5):
        assert np.array_equal(xb[i], oracle.patch_embedding(imgs[i], pp.patch))


def _check_model_golden(which, images, params, count):
    from heatvit_amd.model import HeatViTModel
    meta, arrays = gio.load(which)
    m = HeatViTModel()
    res = m.infer_batch(images[:count], params, checkpoints=True)
    for i in range(count):
        assert np.array_equal(res.logits[i], arrays["logits"][i]), i
        got = gio.model_checkpoint_digests(res.checkpoints[i])
        bad = [k for k, v in meta["checkpoints"][i].items() if got.get(k) != v]
        assert not bad, (i, bad)
        rows = meta["rows"][i]
        if params.selectors:
            want = [rows["block_01"], rows["block_04"], rows["block_07"], rows["block_10"]]
            assert res.token_counts[i].tolist() == want, i
    return res


def test_full_model_matches_golden():
    img, params = synth.full_workload()
    _check_model_golden("full", img, params, 1)


def test_infer_single_image_api():
    from heatvit_amd.model import HeatViTModel
    meta, arrays = gio.load("pruned")
    imgs, params = synth.pruned_workload(2)
    r = HeatViTModel().infer(imgs[1].reshape(-1), params)
    assert list(r.logits) == arrays["logits"][1].tolist()
    assert r.output_scale_exp == -14
    assert gio.model_checkpoint_digests(r.checkpoints) == meta["checkpoints"][1]
    for s, want in zip(r.selector_summary, meta["selector_summary"][1]):
        assert s == want


def test_pruned_model_matches_golden():
    imgs, params = synth.pruned_workload()
    _check_model_golden("pruned", imgs, params, len(imgs))


def test_throughput_batch_vs_oracle_and_deterministic(oracle):
    from heatvit_amd.model import HeatViTModel
    imgs, params = synth.throughput_workload()
    m = HeatViTModel()
    r1 = m.infer_batch(imgs, params)
    r2 = m.infer_batch(imgs, params)
    assert np.array_equal(r1.logits, r2.logits) and np.array_equal(r1.token_counts,
                                                                   r2.token_counts)
    logits, counts, status, warnings = oracle.model_infer_batch(imgs, params)
    assert not status.any()
    assert np.array_equal(r1.logits, logits)
    assert np.array_equal(r1.warnings, warnings)
    assert np.array_equal(r1.token_counts, counts)
    # batch invariance: a sub-batch reproduces the same rows
    r3 = m.infer_batch(imgs[100:103], params)
    assert np.array_equal(r3.logits, r1.logits[100:103])


def test_model_split_ffn_blocks_at_200_images_vs_oracle(oracle):
    """200 images: stage 0's 39,400 rows are 616 blocks of 64 rows on 256
    CUs, 104 past two per CU, so the fused FFN runs 512 whole blocks and 208
    of 32 rows (the last of 8 rows), with and without the next LayerNorm 1."""
    from heatvit_amd.model import HeatViTModel
    imgs, params = synth.throughput_workload(200)
    r = HeatViTModel().infer_batch(imgs, params)
    logits, counts, status, warnings = oracle.model_infer_batch(imgs, params)
    assert not status.any()
    assert np.array_equal(r.logits, logits)
    assert np.array_equal(r.token_counts, counts)
    assert np.array_equal(r.warnings, warnings)


def test_unpruned_control_vs_oracle(oracle):
    from heatvit_amd.model import HeatViTModel
    imgs, params = synth.throughput_workload()  # all 256 images of the control
    ctrl = synth.unpruned_control(params)
    r = HeatViTModel().infer_batch(imgs, ctrl)
    logits, counts, status, warnings = oracle.model_infer_batch(imgs, ctrl)
    assert not status.any()
    assert np.array_equal(r.warnings, warnings)
    assert np.array_equal(r.logits, logits)
    assert (r.token_counts == 197).all()


def test_pipeline_slots_match_engine():
    """Batches in flight on several streams (heatvit_amd.model.Pipeline)
    give exactly Engine.forward's outputs, including after slots are reused
    and for inputs produced on the caller's stream just before submit."""
    import torch
    from heatvit_amd.model import Engine, Pipeline
    imgs, params = synth.throughput_workload(40)
    src = torch.from_numpy(np.ascontiguousarray(imgs.reshape(40, -1))).cuda()
    eng = Engine(params, 16)
    cuts = [(0, 16), (16, 23), (23, 39), (5, 14), (24, 40), (0, 1)]
    want = []
    for a, b in cuts:
        lg, tc, st, wn = eng.forward(src[a:b].clone())
        want.append((lg.cpu().numpy(), tc.cpu().numpy(), st.cpu().numpy(), wn.cpu().numpy()))
    pipe = Pipeline(eng.model, 16, depth=3)
    for start in (0, 3):
        tickets = [pipe.submit(src[a:b].clone()) for a, b in cuts[start:start + 3]]
        for k, t in enumerate(tickets):
            got = [x.cpu().numpy() for x in t.synchronize()]
            for g, w in zip(got, want[start + k]):
                assert np.array_equal(g, w)
    pipe.synchronize()


@pytest.mark.parametrize("pruned", [True, False])
def test_model_chains_layernorm1_through_ffn_kernels(oracle, pruned):
    """Each block's FFN kernel also writes the next block's LayerNorm 1 unless
    a selector changes the rows in between, and block 12's the final
    LayerNorm, so the LayerNorm launches are block 1's and one after each
    selector; logits, token counts and warnings match the oracle."""
    from heatvit_amd import _lib
    from heatvit_amd.model import HeatViTModel
    imgs, params = synth.pruned_workload(6)
    if not pruned:
        params = synth.unpruned_control(params)
    L = _lib.lib()
    m = HeatViTModel()
    L.hv_profile_enable(1)
    try:
        r = m.infer_batch(imgs, params)
        ms = np.zeros(len(_lib.PROF_CLASSES), np.float32)
        n = np.zeros(len(_lib.PROF_CLASSES), np.int32)
        _lib.check(L.hv_profile_read(ms.ctypes.data, n.ctypes.data, len(ms)), "profile")
    finally:
        L.hv_profile_enable(0)
    n = dict(zip(_lib.PROF_CLASSES, n.tolist()))
    assert n["layernorm"] == 1 + len(params.selectors) and n["ffn"] == 12, n
    logits, counts, status, warnings = oracle.model_infer_batch(imgs, params)
    assert not status.any()
    assert np.array_equal(r.logits, logits)
    assert np.array_equal(r.warnings, warnings)
    if pruned:
        assert np.array_equal(r.token_counts, counts)


def test_model_layernorm_fallbacks_vs_oracle(oracle):
    """Blocks whose LayerNorm leaves the int32 form (beta 17 binary places
    below gamma, so gamma no longer sits at the common exponent): block 2's
    LayerNorm 1 then runs as a launch of the general kernel (block 1's FFN
    kernel does not write it), block 5's LayerNorm 2 runs outside its FFN
    kernel, which then writes no LayerNorm 1 for block 6 either, and the
    final LayerNorm, so changed, runs as a launch after block 12; the other
    blocks stay fused.  The LayerNorm launch count follows, and logits,
    token counts and warnings match the oracle."""
    import dataclasses
    from heatvit_amd import _lib
    from heatvit_amd.model import HeatViTModel
    imgs, params = synth.pruned_workload(6)
    blocks = list(params.blocks)
    m1, f4 = blocks[1].mhsa, blocks[4].ffn
    blocks[1] = dataclasses.replace(
        blocks[1], mhsa=dataclasses.replace(m1, beta1_scale_exp=m1.gamma1_scale_exp - 17))
    blocks[4] = dataclasses.replace(
        blocks[4], ffn=dataclasses.replace(f4, beta2_scale_exp=f4.gamma2_scale_exp - 17))
    p = dataclasses.replace(params, blocks=tuple(blocks),
                            final_beta_scale_exp=params.final_gamma_scale_exp - 17)
    L = _lib.lib()
    L.hv_profile_enable(1)
    try:
        r = HeatViTModel().infer_batch(imgs, p)
        ms = np.zeros(len(_lib.PROF_CLASSES), np.float32)
        n = np.zeros(len(_lib.PROF_CLASSES), np.int32)
        _lib.check(L.hv_profile_read(ms.ctypes.data, n.ctypes.data, len(ms)), "profile")
    finally:
        L.hv_profile_enable(0)
    n = dict(zip(_lib.PROF_CLASSES, n.tolist()))
    # blocks 1, 4, 7, 10 and the final one; block 2's LN1, block 5's LN2, block 6's LN1
    # block 5's projection runs as its own launch too (it feeds LayerNorm 2)
    assert n["layernorm"] == 5 + 3 and n["ffn"] == 12 and n["gemm_proj"] == 1, n
    logits, counts, status, warnings = oracle.model_infer_batch(imgs, p)
    assert not status.any()
    assert np.array_equal(r.logits, logits)
    assert np.array_equal(r.token_counts, counts)
    assert np.array_equal(r.warnings, warnings)


def test_model_projection_and_qkv_outside_fused_kernels_vs_oracle(oracle):
    """A block whose residual align-add after the attention projection needs
    the exact epilogue (the projection's output 22 binary places below x,
    beyond the int32 form's 21) runs the projection as a launch of its own
    and its FFN kernel reads y from memory, still with LayerNorm 2 inside;
    a block whose QKV requant shifts left by 10 (no int32 bias bound left)
    runs the QKV GEMM as a launch of its own and its attention kernel reads
    Q, K, V from memory.  The other blocks keep the projection in their FFN
    kernels and the QKV GEMM in their attention kernels.  Logits, token
    counts and warnings match the oracle."""
    import dataclasses
    from heatvit_amd import _lib
    from heatvit_amd.model import HeatViTModel
    imgs, params = synth.pruned_workload(32)
    blocks = list(params.blocks)
    m7, m9 = blocks[7].mhsa, blocks[9].mhsa
    blocks[7] = dataclasses.replace(
        blocks[7], mhsa=dataclasses.replace(m7, msa_out_scale_exp=m7.x_scale_exp - 22))
    blocks[9] = dataclasses.replace(blocks[9], mhsa=dataclasses.replace(
        m9, qkv_out_scale_exp=m9.ln1_out_scale_exp + m9.wqkv_scale_exp - 10))
    p = dataclasses.replace(params, blocks=tuple(blocks))
    L = _lib.lib()
    L.hv_profile_enable(1)
    try:
        r = HeatViTModel().infer_batch(imgs, p)
        ms = np.zeros(len(_lib.PROF_CLASSES), np.float32)
        n = np.zeros(len(_lib.PROF_CLASSES), np.int32)
        _lib.check(L.hv_profile_read(ms.ctypes.data, n.ctypes.data, len(ms)), "profile")
    finally:
        L.hv_profile_enable(0)
    n = dict(zip(_lib.PROF_CLASSES, n.tolist()))
    assert n["gemm_proj"] == 1 and n["ffn"] == 12, n
    assert n["gemm_qkv"] == 1 and n["attention"] == 12, n
    assert n["layernorm"] == 1 + len(params.selectors), n
    logits, counts, status, warnings = oracle.model_infer_batch(imgs, p)
    assert not status.any()
    assert np.array_equal(r.logits, logits)
    assert np.array_equal(r.token_counts, counts)
    assert np.array_equal(r.warnings, warnings)
