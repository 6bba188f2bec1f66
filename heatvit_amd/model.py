"""Full HeatViT-T inference on the GPU.

HeatViTModel.infer keeps the golden model's signature and result
(model.py:49-123): logits (1000 int32 at LOGIT_SCALE_EXP = -14), the
18 checkpoints (patch, selector_NN, block_NN, final_ln, logits) and the
selector summary, plus the engine's warning bits of the forward
(WARN_HEAD_DEN_ZERO | WARN_PACKAGE_DEN_ZERO | WARN_LN_NEGATIVE_VARIANCE,
heatvit_pkg.sv:120-122), which the golden model computes and drops.
HeatViTModel.infer_batch and Engine run many images per launch sequence;
pruned images keep ragged token counts on the device.
"""

import dataclasses
from dataclasses import dataclass

import numpy as np
import torch

from . import _lib
from .device import DeviceModel
from .image import float_images
from .params import HeatViTParams, coerce

LOGIT_SCALE_EXP = -14
WARN_HEAD_DEN_ZERO, WARN_PACKAGE_DEN_ZERO, WARN_LN_NEGATIVE_VARIANCE = 1, 2, 4
IMAGE_BYTES = 224 * 224 * 3
CKPT_NAMES = (["patch"] + [f"selector_{i:02d}" for i in range(1, 4)] +
              [f"block_{i:02d}" for i in range(1, 13)] + ["final_ln"])


@dataclass(frozen=True)
class ModelResult:
    logits: tuple
    output_scale_exp: int
    checkpoints: dict
    selector_summary: tuple
    warnings: int = 0          # engine warning bits of the forward


@dataclass(frozen=True)
class BatchResult:
    logits: np.ndarray         # [B][1000] int32 at output_scale_exp
    output_scale_exp: int
    token_counts: np.ndarray   # [B][4]: rows entering block 1 and after each selector
    selector_state: np.ndarray  # [n_selectors][B][5]: count, package, kept, pruned, warnings
    warnings: np.ndarray = None  # [B] engine warning bits of each image's forward
    checkpoints: list = None   # per image dict when requested


class Engine:
    """Device-resident model plus a reusable workspace for batches of up to
    `max_batch` images.  `forward(images)` takes a device int8 tensor
    [B][150528] and enqueues the whole forward on the current stream; it
    returns device views (logits, token_counts, selector state, warnings).
    `pipelined`: other forwards run on the GPU at the same time (Pipeline's
    slots), so the kernels keep the launch shapes that suit a shared GPU
    (HV_FWD_PIPELINED); the outputs are the same either way."""

    def __init__(self, params, max_batch, device="cuda", pipelined=False):
        self.options = _lib.HV_FWD_PIPELINED if pipelined else 0
        # a DeviceModel, a compiled-ROM model (heatvit_amd.schedule), or params
        self.model = params if hasattr(params, "struct") else DeviceModel(params, device)
        self.max_batch = int(max_batch)
        L = _lib.lib()
        dev = self.model.device
        self.workspace = torch.empty(L.hv_model_workspace_bytes(self.max_batch),
                                     dtype=torch.uint8, device=dev)
        self.logits = torch.empty((self.max_batch, 1000), dtype=torch.int32, device=dev)
        self.token_counts = torch.empty((self.max_batch, 4), dtype=torch.int32, device=dev)
        self.state = torch.zeros((3, self.max_batch, 5), dtype=torch.int32, device=dev)
        self.warnings = torch.zeros(self.max_batch, dtype=torch.int32, device=dev)

    def forward(self, images, ckpt=None, ckpt_rows=None):
        """images: int8 NHWC [B][150528], or float32 CHW [B][3][224][224]
        quantised on the device at the patch's image_scale_exp."""
        b = images.shape[0]
        if b > self.max_batch:
            raise ValueError(f"batch {b} exceeds the engine's {self.max_batch}")
        if images.dtype == torch.float32:
            if not images.is_contiguous() or tuple(images.shape[1:]) != (3, 224, 224):
                raise ValueError("float images must be a contiguous tensor [B][3][224][224]")
            entry = _lib.lib().hv_model_forward_f32_ex
        elif images.dtype != torch.int8 or not images.is_contiguous() or \
                images.numel() != b * IMAGE_BYTES:
            raise ValueError("images must be a contiguous int8 device tensor [B][150528]")
        else:
            entry = _lib.lib().hv_model_forward_ex
        state = self.state[:, :b] if b == self.max_batch else \
            torch.zeros((3, b, 5), dtype=torch.int32, device=images.device)
        _lib.check(entry(
            self.model.struct, images.data_ptr(), b, self.logits.data_ptr(),
            self.token_counts.data_ptr(), state.data_ptr(), self.warnings.data_ptr(),
            None if ckpt is None else ckpt.data_ptr(),
            None if ckpt_rows is None else ckpt_rows.data_ptr(),
            self.workspace.data_ptr(), self.workspace.numel(), self.options,
            torch.cuda.current_stream(images.device).cuda_stream), "model forward")
        return self.logits[:b], self.token_counts[:b], state, self.warnings[:b]


@dataclass(frozen=True)
class Ticket:
    """One submitted batch: device views of its outputs (logits,
    token_counts, selector state, warnings), the event recorded after its
    forward and the stream it runs on."""
    outputs: tuple
    done: torch.cuda.Event
    stream: torch.cuda.Stream

    def wait(self):
        """Orders the caller's current stream after this batch's forward."""
        torch.cuda.current_stream(self.stream.device).wait_event(self.done)
        return self.outputs

    def synchronize(self):
        """Blocks the host until this batch's forward has finished."""
        self.done.synchronize()
        return self.outputs


class Pipeline:
    """Up to `depth` batches in flight at once, each slot with its own
    workspace and outputs on its own HIP stream (default priority), over one
    shared device model.  Forwards of different batches are independent, so
    the GPU overlaps one batch's latency-bound stages (the small pruned
    blocks, the selectors) with another batch's wide GEMMs.

    submit(images) enqueues a forward after the work already queued on the
    caller's current stream (so the images and any reads of the slot's
    previous outputs queued there come first) and returns a Ticket.  A
    ticket's outputs stay valid until `depth` later submissions reuse its
    slot; readers on other streams must order themselves after
    `ticket.done`.  Every slot computes exactly what Engine.forward does."""

    def __init__(self, params, max_batch, depth=3, device="cuda"):
        if depth < 1:
            raise ValueError("pipeline depth must be at least 1")
        model = params if hasattr(params, "struct") else DeviceModel(params, device)
        self.model = model
        self.engines = [Engine(model, max_batch, device, pipelined=depth > 1)
                        for _ in range(depth)]
        self.streams = [torch.cuda.Stream(device=model.device) for _ in range(depth)]
        self._next = 0

    @property
    def depth(self):
        return len(self.engines)

    def submit(self, images, ckpt=None, ckpt_rows=None):
        i = self._next
        self._next = (i + 1) % len(self.engines)
        s = self.streams[i]
        s.wait_stream(torch.cuda.current_stream(images.device))
        with torch.cuda.stream(s):
            outputs = self.engines[i].forward(images, ckpt, ckpt_rows)
        images.record_stream(s)
        done = torch.cuda.Event()
        done.record(s)
        return Ticket(outputs, done, s)

    def synchronize(self):
        for s in self.streams:
            s.synchronize()


def _images(images):
    a = np.asarray(images.cpu().numpy() if isinstance(images, torch.Tensor) else images)
    if a.dtype.kind == "f":
        raise TypeError("images must hold integers")
    a = a.reshape(-1, IMAGE_BYTES)
    if a.size and (a.min() < -128 or a.max() > 127):
        raise ValueError("image outside int8")
    return np.ascontiguousarray(a, np.int8)


class HeatViTModel:
    """Integer HeatViT-T inference (model.py:70) on one MI355X."""

    def __init__(self):
        self._cache = None

    def _engine(self, params, batch):
        # params: HeatViTParams, or the reference's own HeatViTParams (or any
        # object with its field names), converted once per params object
        if (self._cache is None or self._cache[0] is not params or
                self._cache[1].max_batch < batch):
            self._cache = (params, Engine(coerce(params, HeatViTParams), batch))
        return self._cache[1]

    def infer_batch(self, images, params, checkpoints=False):
        return self._run(torch.from_numpy(_images(images)).cuda(), params, checkpoints)

    def infer_float_batch(self, images, params, checkpoints=False):
        """Forward from preprocessed float CHW images ([B][3][224][224]),
        quantised on the device at params.patch.image_scale_exp
        (p2_sim.forward_image's front end, tools/p2/p2_sim.py:536-543)."""
        return self._run(float_images(images), params, checkpoints)

    def _run(self, dev, params, checkpoints):
        b = dev.shape[0]
        eng = self._engine(params, b)
        ck = ck_rows = None
        if checkpoints:
            ck = torch.zeros((b, 17, 197, 192), dtype=torch.int8, device="cuda")
            ck_rows = torch.zeros((b, 17), dtype=torch.int32, device="cuda")
        logits, counts, state, warnings = eng.forward(dev, ck, ck_rows)
        n_sel = len(params.selectors)
        state = state.cpu().numpy()[:n_sel]
        if (state[:, :, 0] < 0).any():
            e = ValueError("selector input invalid for some image (too few tokens)")
            e.error_class = _lib.HV_ERR_TOKEN_COUNT
            raise e
        cks = None
        if checkpoints:
            ck, ck_rows = ck.cpu().numpy(), ck_rows.cpu().numpy()
            lg = logits.cpu().numpy()
            cks = []
            for i in range(b):
                d = {name: ck[i, s, :ck_rows[i, s]].copy()
                     for s, name in enumerate(CKPT_NAMES) if ck_rows[i, s]}
                d["logits"] = lg[i].copy()
                cks.append(d)
        return BatchResult(logits=logits.cpu().numpy().copy(), output_scale_exp=LOGIT_SCALE_EXP,
                           token_counts=counts.cpu().numpy().copy(), selector_state=state.copy(),
                           warnings=warnings.cpu().numpy().copy(), checkpoints=cks)

    def forward_batch(self, images, params, prune=True):
        """The reference's accuracy engine (p2_sim.forward_image per image,
        tools/p2/p2_sim.py:527-;  p2_sim_ivit.forward_batch_cfg without
        pruning, tools/p2/p2_sim_ivit.py:563-624) over a batch of float CHW
        images: returns (logits [B][1000] int32, token_counts [B][4],
        LOGIT_SCALE_EXP).  prune=False skips the selectors."""
        if not prune:
            params = dataclasses.replace(coerce(params, HeatViTParams), selectors=(),
                                         selector_blocks=())
        r = self.infer_float_batch(images, params)
        return r.logits, r.token_counts, LOGIT_SCALE_EXP

    def infer(self, image, params):
        """HeatViTModel.infer (model.py:73): one image, all checkpoints."""
        res = self.infer_batch(_images(image)[:1], params, checkpoints=True)
        summary = []
        counts = res.token_counts[0]
        prev = 197
        for s in range(len(params.selectors)):
            st = res.selector_state[s, 0]
            summary.append({"input_tokens": int(prev), "output_tokens": int(st[0]),
                            "kept_normal": int(st[2]), "pruned_normal": int(st[3]),
                            "package_present": int(st[1])})
            prev = int(counts[s + 1])
        return ModelResult(logits=tuple(int(v) for v in res.logits[0]),
                           output_scale_exp=LOGIT_SCALE_EXP, checkpoints=res.checkpoints[0],
                           selector_summary=tuple(summary), warnings=int(res.warnings[0]))
