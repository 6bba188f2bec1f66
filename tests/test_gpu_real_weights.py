"""The reference's accuracy engine on the GPU: real-weight parameters from
the scale table, float CHW images, pruning batched on the device, against
the reference's own outputs (tests/golden/real.json, written by
tests/golden/make_real.py)."""

import json
from pathlib import Path

import numpy as np
import pytest

import real_weights as rw

pytestmark = pytest.mark.gpu
FIXTURE = Path(__file__).resolve().parent / "golden" / "real.json"


def test_forward_batch_matches_the_reference_accuracy_engine():
    from heatvit_amd.model import HeatViTModel
    from heatvit_amd.real_params import golden_params_from_real
    fx = json.loads(FIXTURE.read_text())
    floats, table, payload, imgs, _ = rw.make(fx["images"])
    p = golden_params_from_real(floats, table, payload)
    m = HeatViTModel()
    logits, counts, exp = m.forward_batch(imgs, p)
    assert exp == fx["forward_image"][0]["logits_scale_exp"]
    for i, want in enumerate(fx["forward_image"]):
        assert logits[i].tolist() == want["logits"], i
        assert counts[i].tolist() == want["token_counts"], i
    logits, counts, _ = m.forward_batch(imgs, p, prune=False)
    assert logits.tolist() == fx["forward_batch_unpruned"]["logits"]
    assert (counts == 197).all()
