"""Calibrates the synthetic workloads' selector keep-logit biases with the
CPU oracle and writes heatvit_amd/data/calibration.json.

  selector workload: one bias b (every head's b3[h][1]) so that about 45 % of
      all candidates over the 64 token sets clear the 0.5 keep threshold.
  pruned workload: biases for the selectors before blocks 4, 7 and 10, fixed
      one stage at a time, so that the mean token count after each stage over
      the first 8 images lands nearest to 88, 45 and 32.

The keep score rises with b (monotone up to integer rounding), so a shared
bias is first bisected on [-2^30, 2^30].  Saturated int8 logits leave each
head with only a few distinct keep scores, so the count moves in coarse
jumps; per-head biases are then refined by coordinate descent in steps of one
logit LSB (2^(logits_out - h2_out - score_w3) bias units), which interleaves
the three heads' levels in the fused score.  Run:
    python tests/golden/calibrate.py
"""

import json
import sys
from dataclasses import replace
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from heatvit_amd import synth  # noqa: E402
from oracle import oracle  # noqa: E402

CAL_IMAGES = 8


def _bisect(measure, target, lo=-(1 << 30), hi=(1 << 30)):
    """Integer b minimising |measure(b) - target| for non-decreasing measure."""
    best = None
    while lo <= hi:
        mid = (lo + hi) // 2
        val = measure(mid)
        if best is None or abs(val - target) < abs(best[1] - target):
            best = (mid, val)
        if val < target:
            lo = mid + 1
        elif val > target:
            hi = mid - 1
        else:
            break
    return best


def _with_bias(sp, bias):
    b3 = np.array(sp.score.b3).copy()
    b3[:, 1] = np.broadcast_to(np.asarray(bias, np.int64), (3,))
    return replace(sp, score=replace(sp.score, b3=b3))


def _refine_per_head(sp, measure, target, bias, rounds=2, steps=48):
    """Coordinate descent on the three per-head biases around `bias`."""
    lsb = 1 << max(0, sp.logits_out_scale_exp - sp.h2_out_scale_exp - sp.score_w3_scale_exp)
    biases = [int(bias)] * 3
    best = measure(biases)
    for _ in range(rounds):
        for h in range(3):
            for k in range(-steps, steps + 1):
                trial = list(biases)
                trial[h] = int(bias) + k * lsb
                val = measure(trial)
                if abs(val - target) < abs(best - target):
                    best, biases = val, trial
    return biases, best


EXP_DRAWS = 16


def _pick_draw(make, xs, pkgs):
    """Exponent draw whose fused keep scores take the most distinct values
    (mean over the calibration inputs)."""
    best = None
    for draw in range(EXP_DRAWS):
        sp = make(draw)
        div = np.mean([len(np.unique(oracle.token_selector(x, pk, sp, True)["fused_scores"]))
                       for x, pk in zip(xs, pkgs)])
        if best is None or div > best[1]:
            best = (draw, div)
    return best


def calibrate_selector():
    tokens, _ = synth.selector_workload(keep_bias=0, exp_draw=0)
    draw, div = _pick_draw(lambda d: synth.selector_workload(keep_bias=0, exp_draw=d)[1],
                           tokens[:8], [False] * 8)
    print(f"selector: exp_draw={draw} distinct fused scores={div:.1f}")
    _, sp = synth.selector_workload(keep_bias=0, exp_draw=draw)
    total = tokens.shape[0] * (tokens.shape[1] - 1)

    def kept_fraction(bias):
        p = _with_bias(sp, bias)
        kept = sum(oracle.token_selector(t, False, p, checkpoints=False)["kept_normal_count"]
                   for t in tokens)
        return kept / total

    bias, frac = _bisect(kept_fraction, synth.SELECTOR_KEEP_FRACTION)
    biases, frac = _refine_per_head(sp, kept_fraction, synth.SELECTOR_KEEP_FRACTION, bias)
    print(f"selector: keep_bias={biases} kept_fraction={frac:.4f}")
    return {"keep_bias": biases, "exp_draw": draw, "kept_fraction": frac}


def calibrate_pruned():
    imgs = synth.images(synth.WORKLOAD_SEED["pruned"], CAL_IMAGES)
    params = synth.pruned_params(keep_biases=(0, 0, 0), exp_draws=(0, 0, 0))
    seed = synth.WORKLOAD_SEED["pruned"]
    biases, draws = [0, 0, 0], [0, 0, 0]
    xs = [oracle.patch_embedding(img, params.patch) for img in imgs]
    pkgs = [False] * len(xs)
    counts = []
    block = 1
    for stage, sel_block in enumerate(params.selector_blocks):
        while block < sel_block:
            xs = [oracle.transformer_block(x, params.blocks[block - 1], False)[0] for x in xs]
            block += 1
        in_exp = params.selectors[stage].in_scale_exp
        draw, div = _pick_draw(
            lambda d, st=stage, ie=in_exp: synth.make_selector(seed, st + 1, ie, 0, d), xs, pkgs)
        draws[stage] = draw
        base = synth.make_selector(seed, stage + 1, in_exp, 0, draw)
        print(f"pruned stage {stage + 1}: exp_draw={draw} distinct fused scores={div:.1f}")

        def mean_tokens(bias, base=base, xs=xs, pkgs=pkgs):
            p = _with_bias(base, bias)
            return float(np.mean([oracle.token_selector(x, pk, p, False)["token_count"]
                                  for x, pk in zip(xs, pkgs)]))

        bias, mean = _bisect(mean_tokens, synth.TOKEN_TARGETS[stage])
        bias, mean = _refine_per_head(base, mean_tokens, synth.TOKEN_TARGETS[stage], bias)
        biases[stage] = bias
        p = _with_bias(base, bias)
        res = [oracle.token_selector(x, pk, p, False) for x, pk in zip(xs, pkgs)]
        xs = [r["tokens"] for r in res]
        pkgs = [r["package_present"] for r in res]
        counts.append([int(r["token_count"]) for r in res])
        print(f"pruned stage {stage + 1}: keep_bias={bias} mean_tokens={mean:.2f} "
              f"counts={counts[-1]}")
    return {"keep_biases": biases, "exp_draws": draws, "calibration_images": CAL_IMAGES,
            "calibration_token_counts": counts}


def main():
    out = {"selector": calibrate_selector(), "pruned": calibrate_pruned()}
    synth.CALIBRATION_FILE.parent.mkdir(parents=True, exist_ok=True)
    synth.CALIBRATION_FILE.write_text(json.dumps(out, indent=2) + "\n")
    print("wrote", synth.CALIBRATION_FILE)


if __name__ == "__main__":
    main()
