"""Real-weight parameters and the per-tensor scale table on the CPU.

tests/golden/real.json holds what the reference's own real-weight tools
produced on the stand-in model of tests/real_weights.py (see
tests/golden/make_real.py): the HeatViTParams of
p2_export_weights.golden_params_from_real, the quantised images of
real_image_list, and the logits/token counts of the accuracy engine
(p2_sim.forward_image with pruning, p2_sim_ivit.forward_batch_cfg without).
"""

import json
from pathlib import Path

import numpy as np
import pytest

import real_weights as rw
from heatvit_amd import scale_table as st
from heatvit_amd.real_params import (golden_params_from_real, merge_selector_scales,
                                     quantize_bias, quantize_int8)

FIXTURE = Path(__file__).resolve().parent / "golden" / "real.json"


@pytest.fixture(scope="module")
def real():
    fx = json.loads(FIXTURE.read_text())
    floats, table, payload, imgs, _ = rw.make(fx["images"])
    return fx, floats, table, payload, imgs


def test_scale_table_schema_and_validation(tmp_path):
    assert len(st.WEIGHT_NAMES) == 3 + 12 * 8 + 3 * 6 + 3 == 120
    assert len(st.ACTIVATION_NAMES) == 4 + 12 * 9 + 3 * 7 + 1 == 134
    t = st.ScaleTable({n: -7 for n in st.WEIGHT_NAMES}, {n: -6 for n in st.ACTIVATION_NAMES})
    t.validate()
    t.save(tmp_path / "t.json")
    doc = json.loads((tmp_path / "t.json").read_text())
    assert list(doc) == ["weights", "activations"] and list(doc["weights"]) == sorted(doc["weights"])
    u = st.ScaleTable.load(tmp_path / "t.json").validate()
    assert u.weights == t.weights and u.activations == t.activations
    for mutate, msg in ((lambda x: x.weights.pop("b7_w1"), "missing weight"),
                        (lambda x: x.activations.pop("s2_h1_out"), "missing activation"),
                        (lambda x: x.weights.__setitem__("b13_w1", -7), "unknown weight"),
                        (lambda x: x.weights.__setitem__("head_w", 32), "outside"),
                        (lambda x: x.activations.__setitem__("input", -33), "outside"),
                        (lambda x: x.weights.__setitem__("cls", True), "integer"),
                        (lambda x: x.weights.__setitem__("cls", -7.0), "integer")):
        bad = st.ScaleTable(t.weights, t.activations)
        mutate(bad)
        with pytest.raises(ValueError, match=msg):
            bad.validate()
    with pytest.raises(KeyError):
        t.weight_exp("nope")
    (tmp_path / "bad.json").write_text("[1]")
    with pytest.raises(ValueError):
        st.ScaleTable.load(tmp_path / "bad.json")


def test_quantizers_round_half_even_and_saturate():
    x = np.array([0.5, 1.5, 2.5, -0.5, -1.5, 300.0, -300.0, 127.49, -128.5], np.float32)
    assert quantize_int8(x, 0).tolist() == [0, 2, 2, 0, -2, 127, -128, 127, -128]
    assert quantize_int8(x * 4, 2).tolist() == quantize_int8(x, 0).tolist()
    b = np.array([2.5, 3.5, 2.0 ** 40, -(2.0 ** 40)], np.float64)
    assert quantize_bias(b, 0).tolist() == [2, 4, 2 ** 31 - 1, -2 ** 31]


def test_params_from_real_match_the_reference(real):
    fx, floats, table, payload, _ = real
    assert table.weights == fx["table"]["weights"]
    assert table.activations == fx["table"]["activations"]
    got = rw.param_digests(golden_params_from_real(floats, table, payload))
    assert {k: got.get(k) for k in fx["params"]} == fx["params"]


def test_merge_selector_scales(real):
    _, _, table, payload, _ = real
    t = st.ScaleTable(dict(table.weights), dict(table.activations))
    pay = dict(payload, weight_exps={str(s): {"local_w": -9, "hw_w2": -3} for s in (1, 2, 3)},
               sel_acts={str(s): {"h1_out": -2} for s in (1, 2, 3)})
    merge_selector_scales(t, pay)
    assert t.weights["s2_local_w"] == -9 and t.weights["s3_hw_w2"] == -3
    assert t.activations["s1_h1_out"] == -2
    p = golden_params_from_real(*real[1:2], t, payload)
    assert p.selectors[1].local_w_scale_exp == -9 and p.selectors[0].h1_out_scale_exp == -2


def test_oracle_reproduces_the_reference_accuracy_engine(real, oracle):
    """The accuracy engine's outputs equal the golden model's (the oracle)
    on the same parameters: pruned per image, and unpruned."""
    fx, floats, table, payload, imgs = real
    p = golden_params_from_real(floats, table, payload)
    q = np.stack([oracle.quantize_image(im, table.activation_exp("input")) for im in imgs])
    assert [rw.digest(x, np.int8) for x in q] == fx["image_sha256"]
    logits, counts, status, _ = oracle.model_infer_batch(q, p, threads=4)
    assert not status.any()
    for i, want in enumerate(fx["forward_image"]):
        assert logits[i].tolist() == want["logits"], i
        assert counts[i].tolist() == want["token_counts"], i
    from heatvit_amd import synth
    logits, _, _, _ = oracle.model_infer_batch(q, synth.unpruned_control(p), threads=4)
    assert logits.tolist() == fx["forward_batch_unpruned"]["logits"]
