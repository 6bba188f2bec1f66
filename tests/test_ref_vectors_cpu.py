"""The reference's own seeded workloads on the CPU oracle.

* The synthetic end-to-end model (weights.build_params, seed 20260815): the
  parameters heatvit_amd.ref_synth draws equal, tensor by tensor, what the
  reference's build_params produced (tests/golden/ref_e2e.json, written by
  tests/golden/make_ref_e2e.py); the calibration driven by the oracle picks
  the same attempts, reaches the reference's committed token counts
  197 -> 100 -> 55 -> 28 with a package at every selector
  (sim/generated/e2e_tb_config.sv:18-20), and the oracle forward gives the
  golden logits and checkpoints.
* The full selector bench case (tools/generate_selector_vectors.py, seed
  20260815): 193 output tokens with a package
  (sim/generated/selector_tb_config.sv:44-45).
"""

import json
from pathlib import Path

import numpy as np
import pytest

import golden_io as gio
import selector_vectors as sv
from heatvit_amd import ref_synth
from heatvit_amd.params import HeatViTParams

GOLDEN = json.loads((Path(__file__).resolve().parent / "golden" / "ref_e2e.json").read_text())
E2E_COUNTS = [197, 100, 55, 28]  # sim/generated/e2e_tb_config.sv:18-20


def test_det_image_is_the_reference_image():
    assert gio.digest(ref_synth.det_image(), np.int8) == GOLDEN["image_sha256"]


def oracle_build(oracle):
    """ref_synth.build_params with the oracle running every stage."""
    base = ref_synth.base_params()
    x = oracle.patch_embedding(ref_synth.det_image(), base.patch)
    pkg, summary, chosen, counts, stage = False, [], [], [197], 0
    for blk in range(1, 13):
        if blk in ref_synth.SELECTOR_BLOCKS:
            stage += 1
            sb = base.selectors[stage - 1]
            h2 = oracle.token_selector(x, pkg, sb)["h2"]
            for att in ref_synth.score_layer_attempts(stage, h2):
                p = ref_synth.with_score_layer(sb, att)
                r = oracle.token_selector(x, pkg, p, checkpoints=False)
                if ref_synth.accepted(r["kept_normal_count"], r["pruned_normal_count"]):
                    break
            summary.append((att.attempt, att.median, r["token_count"]))
            chosen.append(p)
            x, pkg = r["tokens"], r["package_present"]
            counts.append(r["token_count"])
        x, _ = oracle.transformer_block(x, base.blocks[blk - 1], checkpoints=False)
    params = HeatViTParams(patch=base.patch, blocks=base.blocks, selectors=tuple(chosen),
                           final_gamma=base.final_gamma, final_beta=base.final_beta,
                           head_w=base.head_w, head_b=base.head_b)
    return params, summary, counts


@pytest.fixture(scope="module")
def built(oracle):
    return oracle_build(oracle)


def test_reference_e2e_model_on_the_oracle(oracle, built):
    params, summary, counts = built
    assert counts == E2E_COUNTS == GOLDEN["token_counts"]
    want = [(s["attempt"], s["median_logit_diff"], s["output_tokens"]) for s in GOLDEN["summary"]]
    assert summary == want
    got = gio.param_digests(params)
    bad = [k for k, v in GOLDEN["params"].items() if got.get(k) != v]
    assert not bad and len(got) == len(GOLDEN["params"]), bad
    logits, cks, summ, _ = oracle.model_infer(ref_synth.det_image(), params)
    assert logits.tolist() == GOLDEN["logits"]
    assert gio.model_checkpoint_digests(cks) == GOLDEN["checkpoints"]
    assert [s["token_count"] for s in summ] == E2E_COUNTS[1:]
    assert all(s["package_present"] for s in summ)


def test_base_draws_match_before_calibration(built):
    """The ordinary tensors alone (every selector's calibrated w3/b3 aside)
    pin the draw order; a shifted stream would change all of them."""
    base = ref_synth.base_params()
    got = gio.param_digests(built[0])
    assert gio.digest(base.head_w, np.int8) == GOLDEN["params"]["head_w"] == got["head_w"]
    assert gio.digest(base.selectors[2].score.w1, np.int8) == GOLDEN["params"]["selector3.w1"]


def test_reference_selector_bench_case_on_the_oracle(oracle):
    def run(tokens, pkg, p):
        r = oracle.token_selector(tokens, pkg, p, checkpoints=False)
        return r["token_count"], r["kept_normal_count"], r["pruned_normal_count"], \
            r["package_present"]
    _, (count, kept, pruned, pkg), steps = sv.calibrate(run)
    assert count == sv.NEXT_TOKEN_COUNT and pkg
    assert count == 1 + kept + 1 and pruned >= 2
