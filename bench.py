#!/usr/bin/env python3
"""Throughput of HeatViT-T's integer inference path on one MI355X.

Workload: the pruned HeatViT-T (selectors before blocks 4/7/10 calibrated to
the 197 -> 88 -> 45 -> 32 token budget) over a batch of 256 seeded synthetic
224x224x3 int8 images (heatvit_amd.synth, "throughput" workload).  One step
is one full forward of the batch: patch embedding, 12 blocks, 3 token
selectors with stream compaction, final LayerNorm and the 1000-class head,
with the images already resident in HBM.  Every output is bit-exact with
the reference's golden model (tests/test_gpu_composite.py).

`value` is the throughput with --streams batches in flight (default 4),
each on its own HIP stream with its own workspace (heatvit_amd.model.Pipeline):
the timed region holds exactly --steps forwards of 256 images, and the GPU
overlaps one batch's latency-bound stages with another batch's GEMMs.  HIP
maps streams onto GPU_MAX_HW_QUEUES hardware queues per process (4 by
default); with fewer queues than streams plus the default one, batches share
a queue and serialise, so the bench asks the runtime for --hw-queues (8)
before it starts.  The
same line reports one batch at a time (the per-batch latency), and checks
that every pipeline slot's logits equal the single-stream forward's.

Prints one JSON line (rank 0) with the images/s figure, the roofline of the
dominant kernel class (HIP start/stop events recorded by each kernel's own
dispatch on the launch stream, over a second pass of the same steps), the
GEMM-phase int8 MFMA utilisation, the unpruned control's images/s, the CPU
oracle's throughput on a bounded sample of the same workload, and
`bit_exact`: the 256-image logits and token counts of the pruned batch and
of the unpruned control, compared with the CPU oracle on the same inputs
(the process exits with status 1 when they differ).  `configs` times the
smaller workloads (one block, the unpruned model on one image, the selector
over 64 token sets, the pruned model over 32 images), each checked against
the oracle, and `softmax_standalone` the integer softmax over the attention's
3*197 rows per image of the batch.

    python bench.py [--gpus 1] [--steps 20] [--warmup 5]
"""

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

MI355X_INT8_TOPS = 5000.0   # dense int8 MFMA, TOPS
MI355X_HBM_GBS = 8000.0     # HBM3E, GB/s
MI355X_VALU_GINST = 614.4   # 256 CUs x 1 wavefront VALU instruction / cycle x 2.4 GHz
METRIC = "images/sec (batch 256, pruned HeatViT-T, 1 MI355X); % int8 MFMA peak; bit-exact"


def class_work(counts, params, batch):
    """Algorithmic int8 ops (2 x MACs) and minimal HBM bytes per kernel class
    for one forward, from the per-image token counts [B][4].  Per-unit
    figures: QKV 2*192*576, proj 2*192*192, FFN1 2*192*768, FFN2 2*768*192
    ops per token; attention 2*384*N^2 per image; patch 2*768*192 per
    patch; head 2*192*1000 per image; selector 2*13938 per candidate.  The
    attention kernel computes its head's Q, K and V itself (the LayerNorm 1
    rows in, the context rows out: 384 B per token, with the QKV ops); where
    the QKV GEMM runs as its own launch instead (fewer than 32 images),
    `launched_work` moves those ops back to it.  The fused FFN kernel runs
    the attention projection and its residual (the context rows and x in
    once; y stays on the CU), LayerNorm 2, FFN1,
    FFN2 and writes the block output and, when the next block follows
    without a selector in between, that block's LayerNorm 1 (block 12: the
    final LayerNorm): 576 B per token plus 192 B for those blocks; the
    LayerNorm class is then each stage's first LayerNorm 1.  Only the
    classes a run launches are reported."""
    counts = np.asarray(counts, np.int64)
    stage_of_block = []
    s = 0
    for b in range(1, 13):
        if s < len(params.selector_blocks) and params.selector_blocks[s] == b:
            s += 1
        stage_of_block.append(s)
    ops = dict.fromkeys(("patch", "layernorm", "gemm_qkv", "attention", "gemm_proj",
                         "gemm_ffn1", "gemm_ffn2", "ffn", "selector", "head"), 0)
    hbm = dict(ops)
    for b, st in enumerate(stage_of_block, start=1):
        n = counts[:, st]
        t = int(n.sum())
        chained = b == 12 or (b + 1) not in params.selector_blocks
        stage_first = b == 1 or b in params.selector_blocks
        ops["gemm_qkv"] += 2 * 192 * 576 * t
        ops["gemm_proj"] += 2 * 192 * 192 * t
        ops["gemm_ffn1"] += 2 * 192 * 768 * t
        ops["gemm_ffn2"] += 2 * 768 * 192 * t
        # attention with each head's Q, K, V from its own GEMM: LayerNorm 1
        # rows in, context rows out
        ops["attention"] += 2 * 192 * 576 * t + int((2 * 384 * n * n).sum())
        hbm["gemm_qkv"] += (192 + 576) * t
        hbm["gemm_proj"] += (192 + 192 + 192) * t
        hbm["gemm_ffn1"] += (192 + 768) * t
        hbm["gemm_ffn2"] += (768 + 192 + 192) * t
        # fused FFN: context rows and x in, block output (and the next
        # LayerNorm 1) out
        ops["ffn"] += (2 * 192 * 192 + 2 * 2 * 192 * 768) * t
        hbm["ffn"] += (192 + 192 + 192 + (192 if chained else 0)) * t
        hbm["attention"] += (192 + 192) * t
        if stage_first:
            hbm["layernorm"] += 2 * 192 * t
    for s in range(len(params.selectors)):
        c = counts[:, s] - 1
        ops["selector"] += int(2 * 13938 * c.sum())
        hbm["selector"] += int((192 * counts[:, s] + 192 * counts[:, s + 1]).sum())
    ops["patch"] = 2 * 768 * 192 * 196 * batch
    hbm["patch"] = 150528 * batch + 197 * 192 * batch
    ops["head"] = 2 * 192 * 1000 * batch
    hbm["head"] = 192 * batch + 4000 * batch
    return ops, hbm


def launched_work(ops, hbm, launched):
    """The per-class work of the classes a run launched.  When the QKV GEMM
    ran as its own launch, the attention kernel read the fused QKV rows
    (576 B per token) instead of computing them: its QKV ops belong to the
    GEMM class only, and its bytes are 768 B per token (QKV rows in, context
    out) instead of 384."""
    ops, hbm = dict(ops), dict(hbm)
    if "gemm_qkv" in launched and ops.get("attention"):
        ops["attention"] -= ops["gemm_qkv"]
        hbm["attention"] = hbm["attention"] * 2
    return ({n: v for n, v in ops.items() if n in launched},
            {n: v for n, v in hbm.items() if n in launched})


def oracle_model(images, params, threads):
    """The CPU oracle over a batch: (logits, token counts, status, seconds)."""
    from oracle import oracle
    t0 = time.perf_counter()
    logits, counts, status, _ = oracle.model_infer_batch(images, params, threads=threads)
    return logits, counts, status, time.perf_counter() - t0


def roof(ops, nbytes, ms):
    """Roofline entry of one kernel class: the binding roof is the one its
    arithmetic intensity (int8 ops per algorithmic HBM byte) selects against
    the ridge point peak_ops / peak_bytes = 625 ops/B; the other roof's
    fraction is reported beside it."""
    t = ms * 1e-3
    tops = ops / t / 1e12 if ops else 0.0
    gbs = nbytes / t / 1e9 if nbytes else 0.0
    ridge = MI355X_INT8_TOPS * 1e12 / (MI355X_HBM_GBS * 1e9)
    intensity = ops / nbytes if nbytes else float("inf")
    if intensity >= ridge:
        r = {"bound": "mfma", "achieved": round(tops, 2), "peak": MI355X_INT8_TOPS,
             "unit": "TFLOP/s", "frac": round(tops / MI355X_INT8_TOPS, 4),
             "hbm_frac": round(gbs / MI355X_HBM_GBS, 4)}
    else:
        r = {"bound": "hbm", "achieved": round(gbs, 1), "peak": MI355X_HBM_GBS, "unit": "GB/s",
             "frac": round(gbs / MI355X_HBM_GBS, 4),
             "mfma_frac": round(tops / MI355X_INT8_TOPS, 4)}
    r["ops_per_byte"] = round(intensity, 1) if nbytes else None
    return r


def reference_cpu():
    """The reference's own golden model (verification/heatvit_ref,
    HeatViTModel.infer) on the 32 images of the pruned workload, timed when
    the fixture tests/golden/pruned.json was written: one image per process,
    eight processes on the eight cores of the development container.  Not
    measured on the GPU box's host, so it is labelled and kept apart from
    cpu_baseline."""
    f = ROOT / "tests" / "golden" / "pruned.json"
    if not f.exists():
        return None
    secs = json.loads(f.read_text())["golden_seconds"]
    per_image = float(np.mean(secs))
    return {"seconds_per_image": round(per_image, 2),
            "images_per_s": round(8 / per_image, 4), "cores": 8, "same_box": False,
            "sample": f"golden model HeatViTModel.infer on {len(secs)} pruned images "
                      "(197->88->45->32), one per process in an 8-process pool on the "
                      "8-core development container, from tests/golden/pruned.json"}


def _sync_time(fn, warmup, steps):
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        fn()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) * 1e3 / steps


def _class_ms(L, fn, steps):
    """Per-class kernel milliseconds per call of fn (dispatch-recorded events)."""
    from heatvit_amd import _lib
    L.hv_profile_enable(1)
    for _ in range(steps):
        fn()
    ms = np.zeros(len(_lib.PROF_CLASSES), np.float32)
    launches = np.zeros(len(_lib.PROF_CLASSES), np.int32)
    _lib.check(L.hv_profile_read(ms.ctypes.data, launches.ctypes.data, len(ms)), "profile")
    L.hv_profile_enable(0)
    return {n: float(ms[i]) / steps for i, n in enumerate(_lib.PROF_CLASSES) if launches[i]}


GEMM_CLASSES = ("patch", "gemm_qkv", "attention", "gemm_proj", "gemm_ffn1", "gemm_ffn2", "ffn",
                "head")


def _summary(cls_ms, ops, hbm, batch, ms, exact, cpu_s):
    # classes the run launched (the fused FFN's work also has entries under
    # the separate FFN1 / FFN2 GEMMs, which then do not launch)
    ops, hbm = launched_work(ops, hbm, cls_ms)
    gemm_ms = sum(cls_ms.get(n, 0.0) for n in GEMM_CLASSES)
    gemm_ops = sum(ops.get(n, 0) for n in GEMM_CLASSES if n in cls_ms)
    line = {"images_per_s": round(batch / (ms * 1e-3), 1), "ms_per_forward": round(ms, 4),
            "bit_exact": exact,
            "cpu_oracle_images_per_s": round(batch / cpu_s, 2) if cpu_s else None}
    if gemm_ms:
        line["gemm_phase_frac_int8_peak"] = round(
            gemm_ops / (gemm_ms * 1e-3) / 1e12 / MI355X_INT8_TOPS, 4)
    for name in ("layernorm", "selector"):
        if cls_ms.get(name) and hbm.get(name):
            gbs = hbm[name] / (cls_ms[name] * 1e-3) / 1e9
            line[f"{name}_gbs"] = round(gbs, 1)
            line[f"{name}_hbm_frac"] = round(gbs / MI355X_HBM_GBS, 4)
    return line


def config_lines(args, L):
    """The smaller workloads, one forward at a time on the current stream,
    each compared with the CPU oracle: one block over 197 tokens, the
    unpruned model on one image, the selector over 64 token sets of 197, the
    pruned model over 32 images."""
    import torch

    from heatvit_amd import _lib, synth
    from heatvit_amd.device import DeviceBlock, DeviceSelector
    from heatvit_amd.model import Engine
    from oracle import oracle

    def stream():
        return torch.cuda.current_stream().cuda_stream

    def dev(a):
        return torch.from_numpy(np.ascontiguousarray(a)).cuda()

    threads = min(16, os.cpu_count() or 1)
    out = {}

    x, bp = synth.block_workload()
    db = DeviceBlock(bp)
    xd, off = dev(x), dev(np.array([0, 197], np.int32))
    z = torch.empty((197, 192), dtype=torch.int8, device="cuda")
    ws = torch.empty(L.hv_block_workspace_bytes(1, 197), dtype=torch.uint8, device="cuda")

    def block():
        _lib.check(L.hv_block_forward(db.struct, xd.data_ptr(), off.data_ptr(), 1, 197,
                                      z.data_ptr(), None, None, None, ws.data_ptr(), ws.numel(),
                                      stream()), "block")
    ms = _sync_time(block, args.warmup, args.steps)
    t0 = time.perf_counter()
    want, _ = oracle.transformer_block(x, bp, checkpoints=False)
    cpu_s = time.perf_counter() - t0
    n = 197
    ops = {"gemm_qkv": 2 * 192 * 576 * n, "gemm_proj": 2 * 192 * 192 * n,
           "gemm_ffn1": 2 * 192 * 768 * n, "gemm_ffn2": 2 * 768 * 192 * n,
           "ffn": (2 * 192 * 192 + 2 * 2 * 192 * 768) * n,
           "attention": 2 * 192 * 576 * n + 2 * 384 * n * n}
    # one LayerNorm launch (LayerNorm 1; LayerNorm 2 runs inside the fused
    # FFN kernel)
    hbm = {"layernorm": 2 * 192 * n, "attention": 384 * n}
    out["c0_block_b1"] = _summary(_class_ms(L, block, args.steps), ops, hbm, 1, ms,
                                  bool(np.array_equal(z.cpu().numpy(), want)), cpu_s)

    for key, (imgs, params) in (("c1_full_unpruned_b1", synth.full_workload()),
                                ("c3_pruned_b32", synth.pruned_workload())):
        b = len(imgs)
        eng = Engine(params, b)
        idev = dev(imgs.reshape(b, -1))
        ms = _sync_time(lambda: eng.forward(idev), args.warmup, args.steps)
        logits = eng.logits[:b].cpu().numpy()
        counts = eng.token_counts[:b].cpu().numpy()
        o_logits, o_counts, o_status, cpu_s = oracle_model(imgs, params, threads)
        exact = bool(not o_status.any() and np.array_equal(logits, o_logits) and
                     np.array_equal(counts, o_counts))
        ops, hbm = class_work(counts, params, b)
        out[key] = _summary(_class_ms(L, lambda: eng.forward(idev), args.steps), ops, hbm, b,
                            ms, exact, cpu_s)
        if params.selectors:
            out[key]["mean_tokens_per_stage"] = counts.mean(axis=0).round(2).tolist()
        del eng

    tokens, sp = synth.selector_workload()
    b = len(tokens)
    ds = DeviceSelector(sp)
    tin = dev(tokens.reshape(-1, 192))
    offs = dev(np.arange(b + 1, dtype=np.int32) * 197)
    pkg = torch.zeros(b, dtype=torch.uint8, device="cuda")
    o_tok = torch.empty((b * 198, 192), dtype=torch.int8, device="cuda")
    o_off = torch.empty(b + 1, dtype=torch.int32, device="cuda")
    o_pkg = torch.empty(b, dtype=torch.uint8, device="cuda")
    fused = torch.empty((b, 196), dtype=torch.int32, device="cuda")
    kept = torch.empty((b, 196), dtype=torch.int32, device="cuda")
    state = torch.empty((b, 5), dtype=torch.int32, device="cuda")
    sws = torch.empty(L.hv_selector_workspace_bytes(b), dtype=torch.uint8, device="cuda")

    def selector():
        _lib.check(L.hv_selector_forward(ds.struct, tin.data_ptr(), offs.data_ptr(),
                                         pkg.data_ptr(), b, o_tok.data_ptr(), o_off.data_ptr(),
                                         o_pkg.data_ptr(), fused.data_ptr(), kept.data_ptr(),
                                         state.data_ptr(), None, sws.data_ptr(), sws.numel(),
                                         stream()), "selector")
    ms = _sync_time(selector, args.warmup, args.steps)
    got_tok, got_off, st = o_tok.cpu().numpy(), o_off.cpu().numpy(), state.cpu().numpy()
    exact, cpu_s = True, 0.0
    for i in range(b):
        t0 = time.perf_counter()
        w = oracle.token_selector(tokens[i], False, sp, checkpoints=False)
        cpu_s += time.perf_counter() - t0
        exact = exact and st[i, 0] == w["token_count"] and \
            np.array_equal(got_tok[got_off[i]:got_off[i + 1]], w["tokens"])
    n_out = int(st[:, 0].sum())
    ops = {"selector": 2 * 13938 * 196 * b}
    hbm = {"selector": 192 * 197 * b + 192 * n_out}
    out["c2_selector_b64"] = _summary(_class_ms(L, selector, args.steps), ops, hbm, b, ms,
                                      bool(exact), cpu_s)
    out["c2_selector_b64"]["mean_tokens_out"] = round(n_out / b, 2)
    return out


def softmax_standalone(args, L):
    """hv_softmax_rows over the attention's rows of one batch at stage 0:
    3 heads x 197 query rows of 197 q16 scores per image (int32 in, UQ0.8
    out: 5 bytes per element), checked against the oracle on 256 rows."""
    import torch

    from heatvit_amd import _lib
    from oracle import oracle
    rows = 3 * 197 * args.batch
    g = torch.Generator(device="cuda")
    g.manual_seed(20260815)
    x = torch.randint(-(1 << 18), 1 << 18, (rows * 197,), dtype=torch.int32, device="cuda",
                      generator=g)
    off = torch.arange(rows + 1, dtype=torch.int32, device="cuda") * 197
    att = torch.empty(rows * 197, dtype=torch.uint8, device="cuda")

    def run():
        _lib.check(L.hv_softmax_rows(x.data_ptr(), off.data_ptr(), rows, att.data_ptr(), None,
                                     torch.cuda.current_stream().cuda_stream), "softmax")
    ms = _sync_time(run, args.warmup, args.steps)
    xs, got = x.view(rows, 197).cpu().numpy(), att.view(rows, 197).cpu().numpy()
    pick = np.random.default_rng(7).choice(rows, 256, replace=False)
    exact = all(np.array_equal(got[r], oracle.softmax_attention(xs[r])) for r in pick)
    nbytes = rows * 197 * 5
    gbs = nbytes / (ms * 1e-3) / 1e9
    return {"workload": f"{rows} rows of 197 int32 scores (3 x 197 per image, batch "
                        f"{args.batch}) -> UQ0.8", "ms": round(ms, 4), "gbs": round(gbs, 1),
            "hbm_frac": round(gbs / MI355X_HBM_GBS, 4), "bit_exact_sample": bool(exact)}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--batch", type=int, default=256)
    ap.add_argument("--streams", type=int, default=4,
                    help="batches in flight, each on its own HIP stream (1: one at a time)")
    ap.add_argument("--control-streams", type=int, default=3,
                    help="batches in flight for the unpruned control (its best: its "
                         "stage-0 work fills the GPU with fewer)")
    ap.add_argument("--hw-queues", type=int, default=8,
                    help="HIP hardware queues per process (GPU_MAX_HW_QUEUES, at most 32), "
                         "set before the runtime starts; 0 leaves the environment's value")
    ap.add_argument("--cpu-passes", type=int, default=30,
                    help="most passes of the CPU oracle over the whole batch (0 skips it)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="the CPU oracle stops after the first pass that ends past this time")
    ap.add_argument("--no-control", action="store_true", help="skip the unpruned control")
    ap.add_argument("--no-float", action="store_true",
                    help="skip the float-image front-end measurement")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the per-config lines and the standalone softmax")
    ap.add_argument("--sustained-seconds", type=float, default=5.0,
                    help="length of the sustained pipelined run reported beside `value` "
                         "(0 skips it)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="first run three 64 MiB device-to-device copies (the reference "
                         "kernel for scaling HBM counters in a profiler run)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one MI355X: the whole batch runs on a single GPU (images are "
              "independent, so more GPUs would each take a share of the batch in a process of "
              "their own). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    if args.hw_queues:
        # before anything initialises HIP (torch and the library load below)
        os.environ["GPU_MAX_HW_QUEUES"] = str(min(max(args.hw_queues, 1), 32))

    import torch

    from heatvit_amd import _lib, synth
    from heatvit_amd.model import Engine, Pipeline

    if args.copy_calibration:
        src = torch.randint(-128, 127, (64 << 20,), dtype=torch.int8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    images, params = synth.throughput_workload(args.batch)
    dev = torch.from_numpy(np.ascontiguousarray(images.reshape(args.batch, -1))).cuda()
    eng = Engine(params, args.batch)

    def timed(step, steps):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            step(dev)
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) * 1e3 / steps

    # One batch at a time on one stream: the per-batch latency.
    for _ in range(args.warmup):
        eng.forward(dev)
    latency_ms = timed(eng.forward, args.steps)
    counts = eng.token_counts[:args.batch].cpu().numpy()
    ref_logits = eng.logits[:args.batch].clone()
    # Throughput: batches are independent, so `streams` of them are kept in
    # flight on their own streams (every step is still one full forward of
    # a 256-image batch; the timed region holds exactly `steps` of them).
    pipe_equal = None
    if args.streams > 1:
        pipe = Pipeline(eng.model, args.batch, depth=args.streams)
        for _ in range(max(args.warmup, args.streams)):
            pipe.submit(dev)
        wall_ms = timed(pipe.submit, args.steps)
        pipe_equal = all(bool(torch.equal(e.logits[:args.batch], ref_logits))
                         for e in pipe.engines)
        del pipe
    else:
        wall_ms = latency_ms
    value = args.batch / (wall_ms / 1e3)

    # Sustained: the same pipelined forwards back to back for a few seconds,
    # so clocks reach steady state; reported beside `value`, never as it.
    sustained = None
    if args.sustained_seconds > 0:
        spipe = Pipeline(eng.model, args.batch, depth=max(args.streams, 1)) \
            if args.streams > 1 else None
        step = spipe.submit if spipe else eng.forward
        per = max(1, int(args.sustained_seconds * 1e3 / max(wall_ms, 1e-3)))
        s_ms = timed(step, per)
        sustained = {"value": round(args.batch / (s_ms / 1e3), 1), "ms_per_step": round(s_ms, 4),
                     "steps": per, "seconds": round(per * s_ms / 1e3, 2),
                     "batches_in_flight": max(args.streams, 1)}
        if spipe:
            sustained["logits_equal"] = all(bool(torch.equal(e.logits[:args.batch], ref_logits))
                                            for e in spipe.engines)
            del spipe

    # Second pass over the same steps; every kernel carries start/stop HIP
    # events recorded by its dispatch (kept out of the timed region above).
    L = _lib.lib()
    L.hv_profile_enable(1)
    for _ in range(args.steps):
        eng.forward(dev)
    ms = np.zeros(len(_lib.PROF_CLASSES), np.float32)
    launches = np.zeros(len(_lib.PROF_CLASSES), np.int32)
    _lib.check(L.hv_profile_read(ms.ctypes.data, launches.ctypes.data, len(ms)), "profile")
    L.hv_profile_enable(0)
    ops, hbm = launched_work(*class_work(counts, params, args.batch),
                             {n for i, n in enumerate(_lib.PROF_CLASSES) if launches[i]})
    per_class = {}
    for i, name in enumerate(_lib.PROF_CLASSES):
        if launches[i] == 0:
            continue
        t = float(ms[i]) / args.steps
        entry = {"ms_per_step": round(t, 4), "launches_per_step": int(launches[i]) // args.steps,
                 "avg_launch_us": round(1e3 * float(ms[i]) / int(launches[i]), 2)}
        if ops.get(name):
            entry["tops"] = round(ops[name] / (t * 1e-3) / 1e12, 2)
        if hbm.get(name):
            entry["gbs"] = round(hbm[name] / (t * 1e-3) / 1e9, 1)
        per_class[name] = entry
    gemm_names = GEMM_CLASSES
    gemm_ms = sum(per_class[n]["ms_per_step"] for n in gemm_names if n in per_class)
    gemm_ops = sum(ops[n] for n in gemm_names if n in per_class)
    gemm_tops = gemm_ops / (gemm_ms * 1e-3) / 1e12
    dom = max(per_class, key=lambda n: per_class[n]["ms_per_step"])
    d = per_class[dom]
    roofline = roof(ops.get(dom, 0), hbm.get(dom, 0), d["ms_per_step"])
    for name, entry in per_class.items():
        if ops.get(name) or hbm.get(name):
            r = roof(ops.get(name, 0), hbm.get(name, 0), entry["ms_per_step"])
            entry["bound"], entry["frac"] = r["bound"], r["frac"]
    roofline["kernel"] = dom
    roofline["avg_launch_us"] = d["avg_launch_us"]
    traffic_file = ROOT / "profiles" / f"traffic_{dom}.json"
    roofline["traffic"] = None
    if traffic_file.exists():
        roofline["traffic"] = json.loads(traffic_file.read_text()).get("bytes_per_launch")
    # Instruction-issue bound of the dominant kernel: its wavefront VALU
    # instructions per launch (rocprofv3 SQ_INSTS_VALU, same workload) over
    # the launch time, against 256 CUs x 1 wavefront instruction per cycle.
    valu_file = ROOT / "profiles" / f"valu_{dom}.json"
    if valu_file.exists():
        insts = json.loads(valu_file.read_text())["valu_insts_per_launch"]
        rate = insts / (d["avg_launch_us"] * 1e-6) / 1e9
        roofline["valu"] = {"insts_per_launch": insts, "achieved": round(rate, 1),
                            "peak": MI355X_VALU_GINST, "unit": "G wavefront-instr/s",
                            "frac": round(rate / MI355X_VALU_GINST, 4)}

    control = None
    ctrl_logits = None
    if not args.no_control:
        ctrl = Engine(synth.unpruned_control(params), args.batch)
        for _ in range(max(1, args.warmup // 2)):
            ctrl.forward(dev)
        ctrl_logits = ctrl.logits[:args.batch].cpu().numpy()
        c_lat = timed(ctrl.forward, args.steps)
        c_wall = c_lat
        cs = args.control_streams
        if cs > 1:
            cpipe = Pipeline(ctrl.model, args.batch, depth=cs)
            for _ in range(max(1, args.warmup // 2, cs)):
                cpipe.submit(dev)
            c_wall = timed(cpipe.submit, args.steps)
            del cpipe
        control = {"workload": "unpruned HeatViT-T (same weights, no selectors), batch "
                               f"{args.batch}, {cs} in flight",
                   "value": round(args.batch / (c_wall / 1e3), 1),
                   "ms_per_step": round(c_wall, 4),
                   "one_at_a_time": round(args.batch / (c_lat / 1e3), 1)}
        del ctrl

    float_fe = None
    if not args.no_float:
        # The same images as preprocessed float CHW (q * 2^image_exp), which the
        # front end quantises back to exactly q on its way into the patch rows.
        exp = params.patch.image_scale_exp
        fdev = dev.view(args.batch, 224, 224, 3).permute(0, 3, 1, 2).float().mul_(2.0 ** exp) \
            .contiguous()
        def timed_float(steps):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(steps):
                eng.forward(fdev)
            torch.cuda.synchronize()
            return (time.perf_counter() - t0) * 1e3 / steps

        for _ in range(args.warmup):
            eng.forward(fdev)
        f_wall = timed_float(args.steps)
        same = bool(torch.equal(eng.logits[:args.batch], ref_logits))
        L.hv_profile_enable(1)
        eng.forward(fdev)
        _lib.check(L.hv_profile_read(ms.ctypes.data, launches.ctypes.data, len(ms)), "profile")
        L.hv_profile_enable(0)
        fe_ms = float(ms[_lib.PROF_CLASSES.index("patch")])
        fe_bytes = args.batch * (224 * 224 * 3 * 5) + hbm["patch"]
        float_fe = {"workload": f"the same {args.batch} images as float32 CHW, quantised on the "
                                "device into the patch rows", "value": round(args.batch / (f_wall / 1e3), 1),
                    "ms_per_step": round(f_wall, 4), "logits_equal_int8_path": same,
                    "front_end_ms": round(fe_ms, 4),
                    "front_end_gbs": round(fe_bytes / (fe_ms * 1e-3) / 1e9, 1)}
        del fdev

    configs = None if args.no_configs else config_lines(args, L)
    softmax = None if args.no_configs else softmax_standalone(args, L)

    # Bit-exactness of the timed outputs against the CPU oracle on the same
    # images: the pruned batch (its first pass is also the CPU baseline's
    # first pass) and the unpruned control.
    threads = min(16, os.cpu_count() or 1)
    gpu_logits = ref_logits.cpu().numpy()
    o_logits, o_counts, o_status, dt = oracle_model(images, params, threads)
    bit_exact = {"pruned": bool(not o_status.any() and np.array_equal(o_logits, gpu_logits)
                                and np.array_equal(o_counts, counts))}
    if ctrl_logits is not None:
        c_logits, c_counts, c_status, _ = oracle_model(images, synth.unpruned_control(params),
                                                       threads)
        bit_exact["unpruned_control"] = bool(not c_status.any() and
                                             np.array_equal(c_logits, ctrl_logits))
    cpu = None
    if args.cpu_passes > 0:
        secs, passes = dt, 1
        while passes < args.cpu_passes and secs < args.cpu_seconds:
            dt = oracle_model(images, params, threads)[3]
            secs += dt
            passes += 1
        n = passes * args.batch
        cpu = {"value": round(n / secs, 2), "unit": "images/s", "cores": threads, "kind": "port",
               "sample": f"CPU oracle (oracle/hv_oracle.c, OpenMP, {threads} threads) over the "
                         f"same {args.batch}-image workload, {passes} passes, "
                         f"{secs:.1f} s wall"}

    mean_tokens = counts.mean(axis=0).round(2).tolist()
    line = {
        "metric": METRIC, "value": round(value, 1), "unit": "images/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(wall_ms, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int8",
        "data": "synthetic (seeded int8 images and weights, heatvit_amd.synth)",
        "config": {"workload": f"pruned HeatViT-T throughput: batches of {args.batch} images "
                               "224x224x3 int8, selectors before blocks 4/7/10 "
                               "(197->88->45->32 budget)",
                   "global_batch": args.batch, "batches_in_flight": args.streams,
                   "hw_queues": int(os.environ.get("GPU_MAX_HW_QUEUES", "4")),
                   "mean_tokens_per_stage": mean_tokens},
        "one_batch_at_a_time": {"value": round(args.batch / (latency_ms / 1e3), 1),
                                "ms_per_batch": round(latency_ms, 4)},
        "pipelined_logits_equal": pipe_equal,
        "bit_exact": all(bit_exact.values()) and pipe_equal is not False,
        "bit_exact_checks": bit_exact,
        "roofline": roofline,
        "gemm_phase": {"tops": round(gemm_tops, 1), "frac_int8_peak": round(gemm_tops / MI355X_INT8_TOPS, 4),
                       "ms_per_step": round(gemm_ms, 4)},
        "kernels": per_class,
        "control": control,
        "float_images": float_fe,
        "configs": configs,
        "softmax_standalone": softmax,
        "cpu_baseline": cpu,
        "reference_cpu": reference_cpu(),
        "sustained": sustained,
    }
    print(json.dumps(line))
    if not line["bit_exact"] or (configs and not all(c["bit_exact"] for c in configs.values())):
        print("bench.py: GPU outputs differ from the CPU oracle", file=sys.stderr)
        sys.exit(1)


if __name__ == "__main__":
    main()
