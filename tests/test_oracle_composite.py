"""Pins the oracle's composite stages (transformer_block, token_selector,
patch embedding + full model) against golden fixtures produced by the
reference's own golden model on the seeded workloads, plus structural
identities of the reference (verification/tests/test_transformer.py,
test_selector.py, test_model.py)."""

import numpy as np
import pytest

import golden_io as gio
from heatvit_amd import synth


def test_block_matches_golden(oracle):
    meta, arrays = gio.load("block")
    x, bp = synth.block_workload()
    assert gio.digest(x, np.int8) == meta["input_sha256"]
    z, ck = oracle.transformer_block(x, bp)
    ck["z"] = z
    assert np.array_equal(z, arrays["z"])
    for k, want in meta["checkpoints"].items():
        assert gio.digest(ck[k], gio.BLOCK_DTYPES[k]) == want, k


def test_block_residual_identities(oracle):
    # y = align_add(x, msa) and z = align_add(y, ffn_out) element-wise, and the
    # score checkpoint is an independent int64 recompute of Q K^T << shift
    # (test_transformer.py:234-337 style).
    x, bp = synth.block_workload()
    z, ck = oracle.transformer_block(x, bp)
    m, f = bp.mhsa, bp.ffn
    n = len(x)
    q = ck["fused_qkv"][:, 0:192].astype(np.int64)
    k = ck["fused_qkv"][:, 192:384].astype(np.int64)
    for h in range(3):
        acc = q[:, h * 64:(h + 1) * 64] @ k[:, h * 64:(h + 1) * 64].T
        shift = m.score_scale_exp - 2 * m.qkv_out_scale_exp
        want = np.clip(acc * (1 << -shift) if shift <= 0 else acc, -(1 << 31), (1 << 31) - 1)
        if shift <= 0:
            assert np.array_equal(ck["score"][h], want)
    # prob rows of the attention softmax sum to about 256 (UQ0.8)
    sums = ck["prob"].astype(np.int64).sum(axis=2)
    assert sums.max() <= 256 + n and sums.min() >= 256 - n
    for r in range(0, n, 37):
        for c in range(0, 192, 11):
            ce = min(m.x_scale_exp, m.msa_out_scale_exp)
            s = (int(x[r, c]) << (m.x_scale_exp - ce)) + (int(ck["msa"][r, c]) << (m.msa_out_scale_exp - ce))
            assert ck["y"][r, c] == oracle.requant(s, ce, f.x_scale_exp, 8)
            ce = min(f.x_scale_exp, f.ffn_out_scale_exp)
            s = (int(ck["y"][r, c]) << (f.x_scale_exp - ce)) + \
                (int(ck["ffn_out"][r, c]) << (f.ffn_out_scale_exp - ce))
            assert z[r, c] == oracle.requant(s, ce, f.out_scale_exp, 8)


@pytest.mark.skipif(not gio.available("selector"), reason="selector fixture not generated")
@pytest.mark.parametrize("exps", [None, dict(score_scale_exp=-6), dict(score_scale_exp=-31),
                                  dict(qkv_out_scale_exp=-7, context_out_scale_exp=-12),
                                  dict(context_out_scale_exp=20)])
def test_attention_core_matches_block(oracle, exps):
    # The composed attention (score GEMM, q16, softmax rows, P.V) gives the
    # block's score / prob / concat checkpoints, and at the fixture's own
    # exponents the golden digests.
    import dataclasses
    meta, _ = gio.load("block")
    x, bp = synth.block_workload()
    if exps:
        bp = dataclasses.replace(bp, mhsa=dataclasses.replace(bp.mhsa, **exps))
    rng = np.random.default_rng(4)
    for xi in (x, rng.integers(-128, 128, (37, 192)).astype(np.int8)):
        _, ck = oracle.transformer_block(xi, bp)
        m = bp.mhsa
        got = oracle.attention(ck["fused_qkv"], m.qkv_out_scale_exp, m.score_scale_exp,
                               m.prob_scale_exp, m.context_out_scale_exp)
        for key, arr in zip(("score", "prob", "concat"), got):
            assert np.array_equal(arr, ck[key]), key
            if exps is None and xi is x:
                assert gio.digest(arr, gio.BLOCK_DTYPES[key]) == meta["checkpoints"][key], key


def test_selector_matches_golden(oracle):
    meta, arrays = gio.load("selector")
    tokens, sp = synth.selector_workload()
    assert gio.digest(tokens, np.int8) == meta["input_sha256"]
    for i, want in enumerate(meta["results"]):
        r = oracle.token_selector(tokens[i], False, sp)
        for key in ("token_count", "kept_normal_count", "pruned_normal_count", "warnings"):
            assert r[key] == want[key], (i, key)
        assert int(r["package_present"]) == want["package_present"]
        assert gio.digest(r["tokens"], np.int8) == want["tokens_sha256"], i
        assert gio.digest(r["local"], np.int8) == want["local_sha256"], i
        assert gio.digest(r["global_features"], np.int8) == want["global_sha256"], i
        assert gio.digest(r["head_scores"], "<i4") == want["head_scores_sha256"], i
        assert gio.digest(r["head_stats"], np.int8) == want["head_stats_sha256"], i
        assert gio.digest(r["head_weights"], "<i4") == want["head_weights_sha256"], i
        assert np.array_equal(r["fused_scores"], arrays["fused"][i])
        if r["package_present"]:
            assert np.array_equal(r["tokens"][-1], arrays["package"][i])
        kept = np.nonzero(arrays["fused"][i] >= 32768)[0]
        assert np.array_equal(r["kept_index"], kept)


def test_selector_incoming_package_and_manual_finalize(oracle):
    # test_selector.py:256-306: output equals a manual finalize on the fused
    # scores, with and without an incoming package.
    tokens, sp = synth.selector_workload()
    t = tokens[0][:40]
    r = oracle.token_selector(t, False, sp)
    out, _, st = oracle.finalize_tokens(t[0], t[1:], None, r["fused_scores"])
    assert np.array_equal(out, r["tokens"])
    r = oracle.token_selector(t, True, sp)
    out, _, st = oracle.finalize_tokens(t[0], t[1:-1], t[-1], r["fused_scores"])
    assert np.array_equal(out, r["tokens"]) and st.package_present


def _check_model(oracle, which, images, params, count=None):
    meta, arrays = gio.load(which)
    count = len(images) if count is None else count
    for i in range(count):
        assert gio.digest(images[i], np.int8) == meta["input_sha256"][i]
        logits, cks, summary, warnings = oracle.model_infer(images[i], params)
        assert warnings == 0
        assert np.array_equal(logits, arrays["logits"][i]), i
        got = gio.model_checkpoint_digests(cks)
        assert got == meta["checkpoints"][i], (i, [k for k in got if got[k] != meta["checkpoints"][i].get(k)])
        for s, want in zip(summary, meta["selector_summary"][i]):
            assert s["token_count"] == want["output_tokens"]
            assert s["kept_normal"] == want["kept_normal"]
            assert s["pruned_normal"] == want["pruned_normal"]
            assert s["package_present"] == want["package_present"]


@pytest.mark.skipif(not gio.available("full"), reason="full fixture not generated")
def test_full_model_matches_golden(oracle):
    img, params = synth.full_workload()
    _check_model(oracle, "full", img, params)


@pytest.mark.skipif(not gio.available("pruned"), reason="pruned fixture not generated")
def test_pruned_model_matches_golden(oracle):
    imgs, params = synth.pruned_workload()
    _check_model(oracle, "pruned", imgs, params, count=8)


@pytest.mark.skipif(not gio.available("pruned"), reason="pruned fixture not generated")
def test_pruned_batch_logits_and_counts(oracle):
    meta, arrays = gio.load("pruned")
    imgs, params = synth.pruned_workload()
    logits, counts, status, warnings = oracle.model_infer_batch(imgs, params)
    assert not warnings.any()
    assert not status.any()
    assert np.array_equal(logits, arrays["logits"])
    want = [[r["block_01"], r["block_04"], r["block_07"], r["block_10"]] for r in meta["rows"]]
    assert counts.tolist() == want
