"""The reference's own seeded workloads on the GPU, bit-exact:

* heatvit_amd.ref_synth.build_params on the reference's e2e image builds,
  with every stage and calibration run on the GPU, exactly the parameters
  the reference's weights.build_params produced (tests/golden/ref_e2e.json)
  and its committed token counts 197 -> 100 -> 55 -> 28
  (sim/generated/e2e_tb_config.sv:18-20); HeatViTModel.infer then gives the
  golden logits and all 18 checkpoints.
* The reference's committed descriptor ROM (rtl/generated/
  heatvit_descriptors.mem, copied to tests/fixtures/descriptors) run through
  hv_schedule on the weight region of that model gives the same.
* The full selector bench case: 193 tokens with a package
  (sim/generated/selector_tb_config.sv:44-45).
"""

import json
from pathlib import Path

import numpy as np
import pytest

import golden_io as gio
import memory_image as mi
import selector_vectors as sv
from heatvit_amd import ref_synth

pytestmark = pytest.mark.gpu
HERE = Path(__file__).resolve().parent
GOLDEN = json.loads((HERE / "golden" / "ref_e2e.json").read_text())
ROM = HERE / "fixtures" / "descriptors" / "heatvit_descriptors.mem"


@pytest.fixture(scope="module")
def built():
    print("ref_synth.build_params on the GPU", flush=True)
    return ref_synth.build_params(ref_synth.det_image())


def test_build_params_on_gpu_matches_reference(built):
    params, summary, counts = built
    assert counts == [197, 100, 55, 28] == GOLDEN["token_counts"]
    assert summary == GOLDEN["summary"]
    got = gio.param_digests(params)
    bad = [k for k, v in GOLDEN["params"].items() if got.get(k) != v]
    assert not bad and len(got) == len(GOLDEN["params"]), bad


def test_reference_e2e_forward_matches_golden(built):
    from heatvit_amd.model import HeatViTModel
    params = built[0]
    r = HeatViTModel().infer(ref_synth.det_image(), params)
    assert list(r.logits) == GOLDEN["logits"]
    assert r.output_scale_exp == GOLDEN["output_scale_exp"]
    assert gio.model_checkpoint_digests(r.checkpoints) == GOLDEN["checkpoints"]
    assert [dict(s) for s in r.selector_summary] == GOLDEN["selector_summary"]


def test_committed_rom_runs_the_reference_model(built):
    from heatvit_amd.schedule import compile_rom, read_rom, run
    words = read_rom(ROM)
    region = mi.weight_region(built[0], compile_rom(words))
    logits, cks, counts = run(words, region, ref_synth.det_image()[None])
    assert logits[0].tolist() == GOLDEN["logits"]
    assert counts[0].tolist() == GOLDEN["token_counts"]
    got = {name: np.frombuffer(v[0], np.int8) for name, v in cks.items() if v[0]}
    got["logits"] = logits[0]
    assert gio.model_checkpoint_digests(got) == GOLDEN["checkpoints"]


def test_reference_selector_bench_case_on_gpu():
    from heatvit_amd.selector import token_selector_batch

    def run(tokens, pkg, p):
        r = token_selector_batch([tokens], [pkg], p)[0]
        return r.token_count, r.kept_normal_count, r.pruned_normal_count, r.package_present
    _, (count, kept, pruned, pkg), _ = sv.calibrate(run)
    assert count == sv.NEXT_TOKEN_COUNT and pkg
