"""The Python boundary takes parameter objects shaped like the reference's
own dataclasses (field names of verification/heatvit_ref model.py:24-47,
transformer.py:51-398, selector.py:111-222): the GPU results equal those for
this package's containers, bit for bit."""

import numpy as np
import pytest

from heatvit_amd import synth
from test_params_cpu import standin

pytestmark = pytest.mark.gpu


def test_model_block_selector_accept_reference_shaped_params():
    from heatvit_amd.model import HeatViTModel
    from heatvit_amd.selector import token_selector
    from heatvit_amd.transformer import patch_embedding, transformer_block
    imgs, params = synth.pruned_workload(2)
    like = standin(params)
    a = HeatViTModel().infer_batch(imgs, params)
    b = HeatViTModel().infer_batch(imgs, like)
    assert np.array_equal(a.logits, b.logits)
    assert np.array_equal(a.token_counts, b.token_counts)
    r = HeatViTModel().infer(imgs[0].reshape(-1), like)
    assert list(r.logits) == a.logits[0].tolist()
    x = patch_embedding(imgs[0], like.patch)
    assert np.array_equal(x, patch_embedding(imgs[0], params.patch))
    z1, _ = transformer_block(x, params.blocks[0])
    z2, _ = transformer_block(x, like.blocks[0])
    assert np.array_equal(z1, z2)
    s1 = token_selector(z1, False, params.selectors[0])
    s2 = token_selector(z1, False, like.selectors[0])
    assert np.array_equal(s1.tokens, s2.tokens) and np.array_equal(s1.fused_scores,
                                                                   s2.fused_scores)
