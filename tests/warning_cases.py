"""Parameter sets that drive the engine's three warning bits through a whole
forward (heatvit_pkg.sv:120-122; the reference's error bench forces the same
conditions one stage at a time, sim/tb/tb_heatvit_errors.sv cases 8-10).

* LayerNorm negative variance: the reference's row [127]*95 + [90]*97 at
  x_scale -23 clamps its variance (verification/tests/test_nonlinear.py:
  157-163).  With zero patch weights and bias, a zero CLS and every position
  row equal to that row (position exponent = token exponent), each token row
  is exactly the row, and block 1 reads it at x_scale -23.
* Head denominator zero: a head-weight MLP whose second layer is zero with a
  bias far below zero saturates every head weight's PLAN sigmoid to 0.
* Package denominator zero: the score MLP's last bias saturates the two
  logits at +127 / -128 and a logit scale of 2^0 makes their softmax keep
  score exactly 0, so every candidate is pruned with zero total weight.  Only
  the last selector may prune everything: an earlier one would leave the next
  selector a package without a normal candidate (selector.py:448-449).
"""

import dataclasses

import numpy as np

LN_NEG_ROW = np.array([127] * 95 + [90] * 97, np.int8)
LN_NEG_X_EXP = -23


def ln_negative_variance_block(bp):
    """Copy of block params `bp` whose LN1 reads its input at x_scale -23."""
    return dataclasses.replace(bp, mhsa=dataclasses.replace(bp.mhsa, x_scale_exp=LN_NEG_X_EXP))


def ln_negative_variance_model(params):
    """Copy of `params` whose block 1 LN1 sees LN_NEG_ROW on every token."""
    p = params.patch
    patch = dataclasses.replace(
        p, patch_weight=np.zeros_like(np.asarray(p.patch_weight)),
        patch_bias=np.zeros_like(np.asarray(p.patch_bias)),
        cls=np.zeros_like(np.asarray(p.cls)), pos=np.tile(LN_NEG_ROW, (197, 1)),
        pos_scale_exp=p.tokens_scale_exp)
    blocks = (ln_negative_variance_block(params.blocks[0]), *params.blocks[1:])
    return dataclasses.replace(params, patch=patch, blocks=blocks)


def head_den_zero_selector(sp):
    hw = sp.head_weight
    head_weight = dataclasses.replace(hw, w2=np.zeros_like(np.asarray(hw.w2)),
                                      b2=np.full(3, -(1 << 30), np.int32))
    return dataclasses.replace(sp, head_weight=head_weight)


def package_den_zero_selector(sp):
    sc = sp.score
    b3 = np.tile(np.array([1 << 30, -(1 << 30)], np.int32), (3, 1))
    score = dataclasses.replace(sc, w3=np.zeros_like(np.asarray(sc.w3)), b3=b3)
    return dataclasses.replace(sp, score=score, logits_out_scale_exp=0)


def with_selector(params, index, make):
    sels = list(params.selectors)
    sels[index] = make(sels[index])
    return dataclasses.replace(params, selectors=tuple(sels))
