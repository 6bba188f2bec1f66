"""Descriptor front end: the reference engine's ROM and memory image on the GPU.

The reference's end-to-end bench (tb_heatvit_e2e) loads a descriptor ROM
(rtl/generated/heatvit_descriptors.mem) and a vector directory written by
tools/generate_e2e_vectors.py: input.mem / weights.mem region images (one
64-bit little-endian beat per line), checkpoints/<name>.mem with the 18
golden checkpoints, and manifest.json (region sizes, checkpoint byte
counts).  Here the ROM is compiled (hv_schedule_compile: validation with the
engine's error codes, HeatViT-T sequence, scale chain, weight offsets), the
weight region is repacked on the device (hv_schedule_bind) and the forward
runs batched (hv_model_forward), with every checkpoint captured:

    python -m heatvit_amd.schedule --vectors build/vectors/e2e \\
        --rom rtl/generated/heatvit_descriptors.mem
"""

import argparse
import ctypes as C
import json
import sys
from pathlib import Path

import numpy as np
import torch

from . import _lib

CHECKPOINT_SLOTS = (["patch"] + [f"selector_{i:02d}" for i in range(1, 4)] +
                    [f"block_{i:02d}" for i in range(1, 13)] + ["final_ln"])


def read_rom(path):
    """Descriptor ROM text (one 320-bit word per line, 80 hex digits, most
    significant first) -> uint8 [n][40], little-endian words."""
    words = [int(line, 16) for line in Path(path).read_text().split()]
    if any(w >> 320 for w in words):
        raise ValueError("descriptor wider than 320 bits")
    return np.frombuffer(b"".join(w.to_bytes(_lib.HV_DESC_WORD_BYTES, "little") for w in words),
                         np.uint8).reshape(-1, _lib.HV_DESC_WORD_BYTES)


def read_mem(path, valid_bytes=None):
    """Region image (one 64-bit little-endian beat per line) -> bytes,
    trimmed to `valid_bytes` when given."""
    data = b"".join(int(line, 16).to_bytes(8, "little") for line in Path(path).read_text().split())
    return data if valid_bytes is None else data[:valid_bytes]


def compile_rom(words):
    """hv_schedule for a ROM (uint8 [n][40]); raises with the engine's error
    code (`error_class`) when the engine would reject it."""
    L = _lib.lib()
    words = np.ascontiguousarray(words, np.uint8)
    sched = _lib.Schedule()
    _lib.check(L.hv_schedule_compile(words.ctypes.data, len(words), C.byref(sched)),
               "schedule compile")
    return sched


class ScheduledModel:
    """Device weights of a compiled ROM: the weight region repacked into
    the kernels' layouts; usable wherever a DeviceModel is (Engine)."""

    def __init__(self, sched, weights, device="cuda"):
        L = _lib.lib()
        self.device = torch.device(device)
        self.schedule = sched
        region = weights if isinstance(weights, torch.Tensor) else \
            torch.from_numpy(np.frombuffer(bytes(weights), np.uint8).copy())
        region = region.to(self.device)
        self.packed = torch.empty(L.hv_schedule_packed_bytes(C.byref(sched)), dtype=torch.uint8,
                                  device=self.device)
        self.struct = _lib.ModelDev()
        _lib.check(L.hv_schedule_bind(C.byref(sched), region.data_ptr(), region.numel(),
                                      self.packed.data_ptr(), self.packed.numel(),
                                      C.byref(self.struct),
                                      torch.cuda.current_stream(self.device).cuda_stream),
                   "schedule bind")
        torch.cuda.current_stream(self.device).synchronize()  # region may be freed after this


def run(rom_words, weights, images):
    """Runs the compiled ROM over `images` (input regions, [B][150528]
    int8).  Returns (logits [B][1000] int32, {checkpoint: [B] list of
    bytes}, token_counts [B][4])."""
    from .model import Engine
    sched = compile_rom(rom_words)
    model = ScheduledModel(sched, weights)
    imgs = torch.from_numpy(np.array(images, np.int8).reshape(-1, 150528)).cuda()
    b = imgs.shape[0]
    eng = Engine(model, b)
    ck = torch.zeros((b, 17, 197, 192), dtype=torch.int8, device="cuda")
    rows = torch.zeros((b, 17), dtype=torch.int32, device="cuda")
    logits, counts, _, _ = eng.forward(imgs, ck, rows)
    ck, rows = ck.cpu().numpy(), rows.cpu().numpy()
    cks = {name: [ck[i, s, :rows[i, s]].tobytes() for i in range(b)]
           for s, name in enumerate(CHECKPOINT_SLOTS)}
    return logits.cpu().numpy().copy(), cks, counts.cpu().numpy().copy()


def run_vectors(vector_dir, rom_path):
    """One e2e vector directory: returns {checkpoint name: matches} with the
    logits included, compared byte for byte with checkpoints/<name>.mem."""
    d = Path(vector_dir)
    manifest = json.loads((d / "manifest.json").read_text())
    regions = manifest["regions"]
    image = read_mem(d / "input.mem", regions["input"]["valid_bytes"])
    weights = read_mem(d / "weights.mem", regions["weight"]["valid_bytes"])
    logits, cks, _ = run(read_rom(rom_path), weights, np.frombuffer(image, np.int8))
    cks["logits"] = [logits[0].astype("<i4").tobytes()]
    result = {}
    for entry in manifest["checkpoints"]:
        want = read_mem(d / "checkpoints" / f"{entry['name']}.mem", entry["bytes"])
        result[entry["name"]] = cks[entry["name"]][0] == want
    return result


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--vectors", required=True, help="e2e vector directory")
    ap.add_argument("--rom", required=True, help="descriptor ROM (.mem)")
    args = ap.parse_args(argv)
    result = run_vectors(args.vectors, args.rom)
    for name, ok in result.items():
        print(f"{name:12s} {'match' if ok else 'MISMATCH'}")
    passed = all(result.values())
    print("TEST_PASS" if passed else "TEST_FAIL")
    return 0 if passed else 1


if __name__ == "__main__":
    sys.exit(main())
