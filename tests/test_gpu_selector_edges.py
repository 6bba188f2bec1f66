"""GPU selector at the edges of its parameter and input ranges, against the
CPU oracle, bit-exact:

* every selector bias tensor at the int32 limits (selector.py:370-389 adds
  biases in int64, gemm.py:118-119), so the int32 fast paths must hand over
  to the exact forms;
* the three GELU layers' output exponents over a range of post-op shifts
  (so = exponent + 16: 3, 12, 13, 14 and the left shift -4), each layer
  on its own;
* hv_selector_finalize given Q0.16 scores outside [0, 65536]: the golden
  finalize raises ValueError (selector._q016), the device path rejects that
  image (state token count -1) and leaves the others untouched.
"""

import dataclasses

import numpy as np
import pytest

from heatvit_amd import synth

pytestmark = pytest.mark.gpu

I32_MAX, I32_MIN = (1 << 31) - 1, -(1 << 31)
BIAS_FIELDS = (("local", "b"), ("score", "b1"), ("score", "b2"), ("score", "b3"),
               ("head_weight", "b1"), ("head_weight", "b2"))


def _with_bias(sp, part, name, fill):
    sub = getattr(sp, part)
    old = np.asarray(getattr(sub, name))
    return dataclasses.replace(sp, **{part: dataclasses.replace(sub, **{name: fill(old.shape)})})


def _fills():
    yield "max", lambda shape: np.full(shape, I32_MAX, np.int64)
    yield "min", lambda shape: np.full(shape, I32_MIN, np.int64)
    yield "zero", lambda shape: np.zeros(shape, np.int64)
    # alternating limits: lanes of one wavefront take different paths
    yield "alt", lambda shape: np.where(np.arange(int(np.prod(shape))).reshape(shape) % 2,
                                        I32_MAX, I32_MIN)


@pytest.mark.parametrize("part,name", BIAS_FIELDS)
def test_selector_extreme_biases_vs_oracle(oracle, part, name):
    from heatvit_amd.selector import token_selector_batch
    tokens, sp = synth.selector_workload()
    sets = [tokens[0], tokens[1][:40], tokens[2][:3]]
    flags = [False, True, False]
    for tag, fill in _fills():
        p = _with_bias(sp, part, name, fill)
        print(f"selector bias {part}.{name} = {tag}", flush=True)
        res = token_selector_batch(sets, flags, p)
        for i, (t, f) in enumerate(zip(sets, flags)):
            want = oracle.token_selector(t, f, p)
            r = res[i]
            for k in ("local", "global_features", "head_scores", "head_stats", "head_weights",
                      "fused_scores"):
                assert np.array_equal(getattr(r, k), want[k]), (tag, i, k)
            assert np.array_equal(r.tokens, want["tokens"]), (tag, i)
            assert np.array_equal(r.kept_index, want["kept_index"]), (tag, i)
            assert (r.token_count, r.warnings, r.pruned_normal_count) == \
                (want["token_count"], want["warnings"], want["pruned_normal_count"]), (tag, i)


@pytest.mark.parametrize("field", ["local_out_scale_exp", "h1_out_scale_exp",
                                   "h2_out_scale_exp"])
def test_selector_gelu_table_range_vs_oracle(oracle, field):
    from heatvit_amd.selector import token_selector_batch
    tokens, sp = synth.selector_workload()
    sets = [tokens[0], tokens[1][:40], tokens[2][:3]]
    flags = [False, True, False]
    for e in (-13, -4, -3, -2, -20):
        p = dataclasses.replace(sp, **{field: e})
        print(f"selector {field} = {e}", flush=True)
        res = token_selector_batch(sets, flags, p)
        for i, (t, f) in enumerate(zip(sets, flags)):
            want = oracle.token_selector(t, f, p)
            r = res[i]
            for k in ("local", "h2", "head_scores", "fused_scores"):
                assert np.array_equal(getattr(r, k), want[k]), (e, i, k)
            assert np.array_equal(r.tokens, want["tokens"]), (e, i)
            assert r.token_count == want["token_count"], (e, i)


@pytest.mark.parametrize("bad", [65537, -1, I32_MAX, I32_MIN])
def test_finalize_rejects_out_of_range_scores(oracle, bad):
    import torch

    from heatvit_amd import _lib
    rng = np.random.default_rng(11)
    lens, flags = [40, 30, 12], [0, 1, 0]
    sets = [rng.integers(-128, 128, (n, 192)).astype(np.int8) for n in lens]
    scores = [rng.integers(0, 65537, n - 1).astype(np.int32) for n in lens]
    scores[1][7] = bad
    offsets = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    fused = np.zeros((3, 196), np.int32)
    for i, s in enumerate(scores):
        fused[i, :len(s)] = s
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    tok, off, pkg, fz = dev(np.concatenate(sets)), dev(offsets), dev(np.uint8(flags)), dev(fused)
    out = torch.zeros((sum(lens) + 3, 192), dtype=torch.int8, device="cuda")
    out_off = torch.zeros(4, dtype=torch.int32, device="cuda")
    pkg_out = torch.zeros(3, dtype=torch.uint8, device="cuda")
    kept = torch.zeros((3, 196), dtype=torch.int32, device="cuda")
    state = torch.zeros((3, 5), dtype=torch.int32, device="cuda")
    _lib.check(_lib.lib().hv_selector_finalize(
        tok.data_ptr(), off.data_ptr(), pkg.data_ptr(), fz.data_ptr(), 3, out.data_ptr(),
        out_off.data_ptr(), pkg_out.data_ptr(), kept.data_ptr(), state.data_ptr(),
        torch.cuda.current_stream().cuda_stream), "finalize")
    st, o, out = state.cpu().numpy(), out_off.cpu().numpy(), out.cpu().numpy()
    assert st[1, 0] == -1 and int(pkg_out[1]) == 0
    assert o[2] - o[1] == 0
    for i in (0, 2):
        t = sets[i]
        inc = t[-1] if flags[i] else None
        normal = t[1:-1] if flags[i] else t[1:]
        want, want_kept, wst = oracle.finalize_tokens(t[0], normal, inc, scores[i])
        assert st[i, 0] == wst.token_count
        assert np.array_equal(out[o[i]:o[i + 1]], want), i
        assert np.array_equal(kept.cpu().numpy()[i, :st[i, 2]], want_kept), i


def test_selector_1024_images_vs_oracle(oracle):
    """hv_selector_forward over 1,024 ragged token sets (2 to 197 tokens,
    every eighth with an incoming package, some near the keep threshold's
    edges) against the oracle: every image's output offset sums the counts
    of all images before it, so every image's rows must land at the right
    place."""
    from heatvit_amd.selector import token_selector_batch
    tokens, sp = synth.selector_workload()
    rng = np.random.default_rng(1024)
    sets, flags = [], []
    for i in range(1024):
        n = int(rng.integers(2, 198)) if i % 5 else 197
        f = i % 8 == 3 and n >= 3
        base = tokens[i % len(tokens)]
        t = base[:n].copy()
        if i % 3 == 1:  # fresh rows so images differ beyond the 64 base sets
            t[1:] = rng.integers(-128, 128, (n - 1, 192), dtype=np.int16).astype(np.int8)
        sets.append(t)
        flags.append(f)
    print("selector 1024 images", flush=True)
    res = token_selector_batch(sets, flags, sp)
    kept_total = 0
    for i, (t, f) in enumerate(zip(sets, flags)):
        want = oracle.token_selector(t, f, sp, checkpoints=False)
        r = res[i]
        assert r.token_count == want["token_count"], i
        assert np.array_equal(r.tokens, want["tokens"]), i
        assert np.array_equal(r.kept_index, want["kept_index"]), i
        assert r.warnings == want["warnings"], i
        kept_total += r.kept_normal_count
    assert 0 < kept_total < sum(len(t) - 1 for t in sets)
