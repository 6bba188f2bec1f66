"""hv_selector_forward_noalloc: the selector forward with its scratch in the
library's fixed device array instead of a caller workspace.  Two calls in a
row (the second on a smaller batch, so stale scratch from the first would
show) must equal hv_selector_forward on a caller workspace bit for bit; so
must a call at the largest batch the fixed array takes and a call captured
into a HIP graph and replayed; a batch beyond the fixed maximum is refused
before any launch."""

import numpy as np
import pytest

from heatvit_amd import _lib, synth

pytestmark = pytest.mark.gpu


def _run(L, entry, ds, sets, flags, ws=None):
    import torch
    b = len(sets)
    lens = [len(t) for t in sets]
    off = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    tin, offs, pkg = dev(np.concatenate(sets)), dev(off), dev(np.uint8(flags))
    out = dict(tok=torch.full((int(off[-1]) + b, 192), 7, dtype=torch.int8, device="cuda"),
               off=torch.full((b + 1,), -5, dtype=torch.int32, device="cuda"),
               pkg=torch.full((b,), 9, dtype=torch.uint8, device="cuda"),
               fused=torch.full((b, 196), -3, dtype=torch.int32, device="cuda"),
               kept=torch.full((b, 196), -9, dtype=torch.int32, device="cuda"),
               state=torch.full((b, 5), -7, dtype=torch.int32, device="cuda"))
    ck_bufs = dict(local=torch.zeros((b, 3, 196, 32), dtype=torch.int8, device="cuda"),
                   global_=torch.zeros((b, 3, 32), dtype=torch.int8, device="cuda"),
                   head_scores=torch.zeros((b, 3, 196), dtype=torch.int32, device="cuda"),
                   head_stats=torch.zeros((b, 196, 3), dtype=torch.int8, device="cuda"),
                   head_weights=torch.zeros((b, 196, 3), dtype=torch.int32, device="cuda"))
    ck = _lib.SelectorCkpt(*[ck_bufs[k].data_ptr() for k in (
        "local", "global_", "head_scores", "head_stats", "head_weights")])
    args = [ds.struct, tin.data_ptr(), offs.data_ptr(), pkg.data_ptr(), b, out["tok"].data_ptr(),
            out["off"].data_ptr(), out["pkg"].data_ptr(), out["fused"].data_ptr(),
            out["kept"].data_ptr(), out["state"].data_ptr(), ck]
    s = torch.cuda.current_stream().cuda_stream
    if ws is None:
        rc = entry(*args, s)
    else:
        rc = entry(*args, ws.data_ptr(), ws.numel(), s)
    _lib.check(rc, "selector")
    torch.cuda.synchronize()
    res = {k: v.cpu().numpy() for k, v in out.items()}
    res.update({k: v.cpu().numpy() for k, v in ck_bufs.items()})
    return res


def test_noalloc_selector_matches_workspace_entry():
    import torch
    from heatvit_amd.device import DeviceSelector
    L = _lib.lib()
    tokens, sp = synth.selector_workload()
    ds = DeviceSelector(sp)
    rng = np.random.default_rng(21)
    calls = [
        ([tokens[i] for i in range(40)] + [tokens[40][:90], tokens[41][:3]],
         [False] * 40 + [True, False]),
        ([tokens[50][:120], rng.integers(-128, 128, (33, 192)).astype(np.int8), tokens[51]],
         [True, False, True]),
    ]
    for sets, flags in calls:
        print(f"noalloc selector: batch {len(sets)}", flush=True)
        ws = torch.empty(L.hv_selector_workspace_bytes(len(sets)), dtype=torch.uint8,
                         device="cuda")
        want = _run(L, L.hv_selector_forward, ds, sets, flags, ws)
        got = _run(L, L.hv_selector_forward_noalloc, ds, sets, flags)
        for k in want:
            assert np.array_equal(got[k], want[k]), (len(sets), k)
        assert (got["state"][:, 0] > 0).all()


def test_noalloc_selector_refuses_oversized_batch():
    from heatvit_amd.device import DeviceSelector
    L = _lib.lib()
    _, sp = synth.selector_workload()
    ds = DeviceSelector(sp)
    b = _lib.HV_SELECTOR_NOALLOC_MAX_BATCH + 1
    rc = L.hv_selector_forward_noalloc(ds.struct, None, None, None, b, None, None, None, None,
                                       None, None, None, None)
    assert rc == _lib.HV_EVALUE
    assert L.hv_last_error_class() == _lib.HV_ERR_DIMENSION
    assert b"exceeds" in L.hv_last_error()


def _sets(tokens, count, seed):
    rng = np.random.default_rng(seed)
    sets = [tokens[i % len(tokens)][:int(rng.integers(3, 198))] for i in range(count)]
    flags = [i % 7 == 2 for i in range(count)]
    return sets, flags


def test_noalloc_selector_at_max_batch():
    import torch
    from heatvit_amd.device import DeviceSelector
    L = _lib.lib()
    tokens, sp = synth.selector_workload()
    ds = DeviceSelector(sp)
    sets, flags = _sets(tokens, _lib.HV_SELECTOR_NOALLOC_MAX_BATCH, 5)
    print(f"noalloc selector: batch {len(sets)}", flush=True)
    ws = torch.empty(L.hv_selector_workspace_bytes(len(sets)), dtype=torch.uint8, device="cuda")
    want = _run(L, L.hv_selector_forward, ds, sets, flags, ws)
    got = _run(L, L.hv_selector_forward_noalloc, ds, sets, flags)
    for k in want:
        assert np.array_equal(got[k], want[k]), k
    assert (got["state"][:, 0] > 0).all()


def test_noalloc_selector_in_hip_graph():
    """One call outside capture (it finds the device's copy of the fixed
    array), then the same call captured into a graph: three replays, with
    the outputs overwritten and other selector work run eagerly between
    them, each equal to the workspace entry's outputs."""
    import torch
    from heatvit_amd.device import DeviceSelector
    L = _lib.lib()
    tokens, sp = synth.selector_workload()
    ds = DeviceSelector(sp)
    sets, flags = _sets(tokens, 24, 6)
    b = len(sets)
    ws = torch.empty(L.hv_selector_workspace_bytes(b), dtype=torch.uint8, device="cuda")
    want = _run(L, L.hv_selector_forward, ds, sets, flags, ws)
    lens = [len(t) for t in sets]
    off = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    tin, offs, pkg = dev(np.concatenate(sets)), dev(off), dev(np.uint8(flags))
    out = dict(tok=torch.empty((int(off[-1]) + b, 192), dtype=torch.int8, device="cuda"),
               off=torch.empty((b + 1,), dtype=torch.int32, device="cuda"),
               pkg=torch.empty((b,), dtype=torch.uint8, device="cuda"),
               fused=torch.empty((b, 196), dtype=torch.int32, device="cuda"),
               kept=torch.empty((b, 196), dtype=torch.int32, device="cuda"),
               state=torch.empty((b, 5), dtype=torch.int32, device="cuda"))

    def call():
        return L.hv_selector_forward_noalloc(
            ds.struct, tin.data_ptr(), offs.data_ptr(), pkg.data_ptr(), b,
            out["tok"].data_ptr(), out["off"].data_ptr(), out["pkg"].data_ptr(),
            out["fused"].data_ptr(), out["kept"].data_ptr(), out["state"].data_ptr(), None,
            torch.cuda.current_stream().cuda_stream)

    def check(tag):
        torch.cuda.synchronize()
        n = int(want["off"][-1])
        got = {k: v.cpu().numpy() for k, v in out.items()}
        assert np.array_equal(got["off"], want["off"]), tag
        assert np.array_equal(got["tok"][:n], want["tok"][:n]), tag
        for k in ("pkg", "fused", "kept", "state"):
            # fused scores past each image's candidates are not written
            if k == "fused":
                for i, c in enumerate(lens):
                    assert np.array_equal(got[k][i, :c - 1], want[k][i, :c - 1]), (tag, i)
            else:
                assert np.array_equal(got[k], want[k]), (tag, k)

    _lib.check(call(), "selector noalloc")
    check("eager")
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        _lib.check(call(), "selector noalloc (capture)")
    other_sets, other_flags = _sets(tokens, 9, 7)
    for rep in range(3):
        for v in out.values():
            v.fill_(-1 - rep)
        _run(L, L.hv_selector_forward_noalloc, ds, other_sets, other_flags)
        print(f"noalloc selector graph replay {rep}", flush=True)
        g.replay()
        check(f"replay {rep}")
