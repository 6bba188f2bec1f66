#!/usr/bin/env python3
"""Throughput of HeatViT-T's integer inference path on one MI355X.

Workload: the pruned HeatViT-T (selectors before blocks 4/7/10 calibrated to
the 197 -> 88 -> 45 -> 32 token budget) over a batch of 256 seeded synthetic
224x224x3 int8 images (heatvit_amd.synth, "throughput" workload).  One step
is one full forward of the batch: patch embedding, 12 blocks, 3 token
selectors with stream compaction, final LayerNorm and the 1000-class head,
with the images already resident in HBM.  Every output is bit-exact with
the reference's golden model (tests/test_gpu_composite.py).

`value` is the throughput with --streams batches in flight (default 3),
each on its own HIP stream with its own workspace (heatvit_amd.model.Pipeline):
the timed region holds exactly --steps forwards of 256 images, and the GPU
overlaps one batch's latency-bound stages with another batch's GEMMs.  The
same line reports one batch at a time (the per-batch latency), and checks
that every pipeline slot's logits equal the single-stream forward's.

Prints one JSON line (rank 0) with the images/s figure, the roofline of the
dominant kernel class (HIP start/stop events recorded by each kernel's own
dispatch on the launch stream, over a second pass of the same steps), the GEMM-phase int8 MFMA utilisation, the unpruned
control's images/s and the CPU oracle's throughput on a bounded sample of
the same workload.

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
    ops per token; attention 2*384*N^2 per image; patch 2*768*192 per patch;
    head 2*192*1000 per image; selector 2*13938 per candidate."""
    counts = np.asarray(counts, np.int64)
    stage_of_block = []
    s = 0
    for b in range(1, 13):
        if s < len(params.selector_blocks) and params.selector_blocks[s] == b:
            s += 1
        stage_of_block.append(s)
    ops = dict.fromkeys(("patch", "layernorm", "gemm_qkv", "attention", "gemm_proj",
                         "gemm_ffn1", "gemm_ffn2", "selector", "head"), 0)
    hbm = dict(ops)
    for st in stage_of_block:
        n = counts[:, st]
        t = int(n.sum())
        ops["gemm_qkv"] += 2 * 192 * 576 * t
        ops["gemm_proj"] += 2 * 192 * 192 * t
        ops["gemm_ffn1"] += 2 * 192 * 768 * t
        ops["gemm_ffn2"] += 2 * 768 * 192 * t
        ops["attention"] += int((2 * 384 * n * n).sum())
        hbm["gemm_qkv"] += (192 + 576) * t
        hbm["gemm_proj"] += (192 + 192 + 192) * t
        hbm["gemm_ffn1"] += (192 + 768) * t
        hbm["gemm_ffn2"] += (768 + 192 + 192) * t
        hbm["attention"] += (576 + 192) * t
        hbm["layernorm"] += 2 * 2 * 192 * t
    for s in range(len(params.selectors)):
        c = counts[:, s] - 1
        ops["selector"] += int(2 * 13938 * c.sum())
        hbm["selector"] += int((192 * counts[:, s] + 192 * counts[:, s + 1]).sum())
    ops["patch"] = 2 * 768 * 192 * 196 * batch
    hbm["patch"] = 150528 * batch + 197 * 192 * batch
    ops["head"] = 2 * 192 * 1000 * batch
    hbm["layernorm"] += 2 * 192 * int(counts[:, len(params.selectors)].sum())
    hbm["head"] = 192 * batch + 4000 * batch
    return ops, hbm


def cpu_baseline(images, params, threads):
    from oracle import oracle
    t0 = time.perf_counter()
    _, _, status, _ = oracle.model_infer_batch(images, params, threads=threads)
    dt = time.perf_counter() - t0
    assert not status.any()
    return len(images) / dt, dt


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--batch", type=int, default=256)
    ap.add_argument("--streams", type=int, default=3,
                    help="batches in flight, each on its own HIP stream (1: one at a time)")
    ap.add_argument("--cpu-passes", type=int, default=30,
                    help="most passes of the CPU oracle over the whole batch (0 skips it)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="the CPU oracle stops after the first pass that ends past this time")
    ap.add_argument("--no-control", action="store_true", help="skip the unpruned control")
    ap.add_argument("--no-float", action="store_true",
                    help="skip the float-image front-end measurement")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="first run three 64 MiB device-to-device copies (the reference "
                         "kernel for scaling HBM counters in a profiler run)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one MI355X: this build runs the whole batch on a single GPU "
              "(images are independent; see DESIGN.md for how the path would shard). "
              "Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

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
    ops, hbm = class_work(counts, params, args.batch)
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
    gemm_names = ("patch", "gemm_qkv", "attention", "gemm_proj", "gemm_ffn1", "gemm_ffn2", "head")
    gemm_ms = sum(per_class[n]["ms_per_step"] for n in gemm_names if n in per_class)
    gemm_ops = sum(ops[n] for n in gemm_names)
    gemm_tops = gemm_ops / (gemm_ms * 1e-3) / 1e12
    dom = max(per_class, key=lambda n: per_class[n]["ms_per_step"])
    d = per_class[dom]
    if dom in gemm_names:
        achieved = ops[dom] / (d["ms_per_step"] * 1e-3) / 1e12
        roofline = {"bound": "mfma", "achieved": round(achieved, 2), "peak": MI355X_INT8_TOPS,
                    "unit": "TFLOP/s", "frac": round(achieved / MI355X_INT8_TOPS, 4)}
    else:
        achieved = hbm[dom] / (d["ms_per_step"] * 1e-3) / 1e9
        roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": MI355X_HBM_GBS,
                    "unit": "GB/s", "frac": round(achieved / MI355X_HBM_GBS, 4)}
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
    if not args.no_control:
        ctrl = Engine(synth.unpruned_control(params), args.batch)
        for _ in range(max(1, args.warmup // 2)):
            ctrl.forward(dev)
        c_lat = timed(ctrl.forward, args.steps)
        c_wall = c_lat
        if args.streams > 1:
            cpipe = Pipeline(ctrl.model, args.batch, depth=args.streams)
            for _ in range(max(1, args.warmup // 2, args.streams)):
                cpipe.submit(dev)
            c_wall = timed(cpipe.submit, args.steps)
            del cpipe
        control = {"workload": "unpruned HeatViT-T (same weights, no selectors), batch "
                               f"{args.batch}, {args.streams} in flight",
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

    cpu = None
    if args.cpu_passes > 0:
        threads = min(16, os.cpu_count() or 1)
        secs, passes = 0.0, 0
        while passes < args.cpu_passes and (passes == 0 or secs < args.cpu_seconds):
            _, dt = cpu_baseline(images, params, threads)
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
                   "mean_tokens_per_stage": mean_tokens},
        "one_batch_at_a_time": {"value": round(args.batch / (latency_ms / 1e3), 1),
                                "ms_per_batch": round(latency_ms, 4)},
        "pipelined_logits_equal": pipe_equal,
        "roofline": roofline,
        "gemm_phase": {"tops": round(gemm_tops, 1), "frac_int8_peak": round(gemm_tops / MI355X_INT8_TOPS, 4),
                       "ms_per_step": round(gemm_ms, 4)},
        "kernels": per_class,
        "control": control,
        "float_images": float_fe,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
