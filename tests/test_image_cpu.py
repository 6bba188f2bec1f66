"""Image front end on the CPU: the oracle's quantiser and patchify against
the reference's own torch expressions for them (tools/p2/
p2_export_weights.py:246-251 and p2_sim.py:536-543), which are library
routines (torch.round ties-to-even, clamp, permute/reshape) rather than a
restatement."""

import numpy as np
import torch


def special_images(rng, count, exp):
    """Float CHW images with ties, out-of-range values, infinities, signed
    zeros and subnormal quotients mixed into normal pixels."""
    imgs = rng.normal(0, 2.0 ** (exp + 6), (count, 3, 224, 224)).astype(np.float32)
    flat = imgs.reshape(count, -1)
    step = np.float32(2.0 ** exp)
    n = flat.shape[1]
    for b in range(count):
        idx = rng.choice(n, 4000, replace=False)
        k = rng.integers(-140, 140, 1000).astype(np.float32)
        flat[b, idx[:1000]] = (k + np.float32(0.5)) * step         # exact ties
        flat[b, idx[1000:1100]] = np.float32(np.inf)
        flat[b, idx[1100:1200]] = np.float32(-np.inf)
        flat[b, idx[1200:1300]] = np.float32(-0.0)
        flat[b, idx[1300:1400]] = rng.normal(0, 1e30, 100).astype(np.float32)
        flat[b, idx[1400:1500]] = (rng.normal(0, 1, 100) * 1e-38).astype(np.float32)
        flat[b, idx[1500:1600]] = np.nextafter((k[:100] + np.float32(0.5)) * step,
                                               np.float32(np.inf))
    return imgs


def torch_reference(chw, exp):
    q = torch.clamp(torch.round(torch.from_numpy(chw) / (2.0 ** exp)), -128, 127).to(torch.int8)
    return q.permute(1, 2, 0).reshape(-1).numpy()


def test_quantize_image_matches_the_torch_expression(oracle):
    rng = np.random.default_rng(7)
    for exp in (-7, -5, 0, -32, 31, 3):
        imgs = special_images(rng, 2, exp)
        for img in imgs:
            assert np.array_equal(oracle.quantize_image(img, exp), torch_reference(img, exp)), exp


def test_quantize_nan_is_zero(oracle):
    img = np.zeros((3, 224, 224), np.float32)
    img[1, 5, 7] = np.nan
    img[0, 0, 0] = 3.0
    q = oracle.quantize_image(img, -1)
    assert q[(5 * 224 + 7) * 3 + 1] == 0 and q[0] == 6


def test_patchify_matches_the_torch_expression(oracle):
    rng = np.random.default_rng(8)
    img = rng.integers(-128, 128, 224 * 224 * 3).astype(np.int8)
    want = torch.from_numpy(img).reshape(224, 224, 3).reshape(14, 16, 14, 16, 3) \
        .permute(0, 2, 1, 3, 4).reshape(196, 768).numpy()
    assert np.array_equal(oracle.patchify(img), want)
