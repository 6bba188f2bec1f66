"""GPU image front end against the oracle: float CHW images quantised to
int8 NHWC and to patch rows (hv_quantize_images), and the whole forward from
float images (hv_model_forward_f32) against the oracle's model on the
oracle-quantised images."""

import numpy as np
import pytest
import torch

from heatvit_amd import synth
from test_image_cpu import special_images

pytestmark = pytest.mark.gpu


def test_quantize_images_vs_oracle(oracle):
    from heatvit_amd.image import quantize_images, real_image_list
    rng = np.random.default_rng(21)
    for exp in (-7, -5, 0, -32, 31):
        print(f"quantize exp {exp}", flush=True)
        imgs = special_images(rng, 3, exp)
        imgs[1, 2, 100, 100] = np.nan
        dev = torch.from_numpy(imgs).cuda()
        nhwc = quantize_images(dev, exp).cpu().numpy()
        rows = quantize_images(dev, exp, layout="patches").cpu().numpy().reshape(3, 196, 768)
        for b in range(3):
            want = oracle.quantize_image(imgs[b], exp)
            assert np.array_equal(nhwc[b], want), (exp, b)
            assert np.array_equal(rows[b], oracle.patchify(want)), (exp, b)
    assert real_image_list(imgs[0], -32) == [int(v) for v in oracle.quantize_image(imgs[0], -32)]


def test_model_forward_from_float_images(oracle):
    from heatvit_amd.model import HeatViTModel
    _, params = synth.pruned_workload(1)
    exp = params.patch.image_scale_exp
    rng = np.random.default_rng(22)
    imgs = rng.normal(0, 2.0 ** (exp + 6), (6, 3, 224, 224)).astype(np.float32)
    q = np.stack([oracle.quantize_image(im, exp) for im in imgs])
    m = HeatViTModel()
    r = m.infer_float_batch(imgs, params)
    logits, counts, status, warnings = oracle.model_infer_batch(q, params, threads=4)
    assert not status.any()
    assert np.array_equal(r.logits, logits)
    assert np.array_equal(r.token_counts, counts)
    assert np.array_equal(r.warnings, warnings)
    r8 = m.infer_batch(q, params, checkpoints=True)
    rf = m.infer_float_batch(imgs, params, checkpoints=True)
    for a, b in zip(r8.checkpoints, rf.checkpoints):
        assert a.keys() == b.keys() and all(np.array_equal(a[k], b[k]) for k in a)
