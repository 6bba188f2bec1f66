"""Token selector on the GPU with the golden model's result type.

  token_selector(tokens, package_present, SelectorParams)   selector.py:503-563
  token_selector_batch(token_sets, package_flags, params)   ragged batch

The result carries the reference's SelectorResult fields (selector.py:
235-250) plus `kept_index`, the candidate index of every kept normal token.
"""

from dataclasses import dataclass, field

import numpy as np
import torch

from . import _lib
from .device import DeviceSelector

WARN_HEAD_DEN_ZERO = 1 << 0
WARN_PACKAGE_DEN_ZERO = 1 << 1
KEEP_THRESHOLD = 32768
Q016_ONE = 65536
MAX_CANDIDATES = 196


@dataclass(frozen=True)
class SelectorResult:
    tokens: np.ndarray = field(default_factory=lambda: np.zeros((0, 192), np.int8))
    token_count: int = 0
    package_present: bool = False
    kept_normal_count: int = 0
    pruned_normal_count: int = 0
    warnings: int = 0
    local: np.ndarray = None
    global_features: np.ndarray = None
    head_scores: np.ndarray = None
    head_stats: np.ndarray = None
    head_weights: np.ndarray = None
    fused_scores: np.ndarray = None
    kept_index: np.ndarray = None
    h2: np.ndarray = None  # [3][C][16] second score-MLP layer (selector.py:307-335)


def _stream():
    return torch.cuda.current_stream().cuda_stream


def token_selector_batch(token_sets, package_flags, params):
    if isinstance(params, DeviceSelector):
        dev = params
    else:
        dev = DeviceSelector(params)
    sets = []
    for t in token_sets:
        a = np.asarray(t.cpu().numpy() if isinstance(t, torch.Tensor) else t)
        if a.dtype.kind == "f":
            raise TypeError("tokens must hold integers")
        if a.ndim != 2 or a.shape[1] != 192 or len(a) < 2:
            raise ValueError("selector input needs CLS plus at least one candidate")
        if len(a) > MAX_CANDIDATES + 1:
            raise ValueError("at most 197 tokens per image")
        if a.min() < -128 or a.max() > 127:
            raise ValueError("tokens outside int8")
        sets.append(np.ascontiguousarray(a, np.int8))
    b = len(sets)
    flags = np.asarray([bool(f) for f in package_flags], np.uint8)
    if len(flags) != b:
        raise ValueError("one package flag per token set")
    for a, f in zip(sets, flags):
        if f and len(a) < 3:
            raise ValueError("incoming package requires at least one candidate")
    lens = [len(a) for a in sets]
    offsets = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    dev_in = torch.from_numpy(np.concatenate(sets)).cuda()
    off = torch.from_numpy(offsets).cuda()
    pkg_in = torch.from_numpy(flags).cuda()
    t = int(offsets[-1])
    out = torch.empty((t + b, 192), dtype=torch.int8, device="cuda")
    out_off = torch.empty(b + 1, dtype=torch.int32, device="cuda")
    pkg_out = torch.empty(b, dtype=torch.uint8, device="cuda")
    fused = torch.zeros((b, MAX_CANDIDATES), dtype=torch.int32, device="cuda")
    kept = torch.empty((b, MAX_CANDIDATES), dtype=torch.int32, device="cuda")
    state = torch.empty((b, 5), dtype=torch.int32, device="cuda")
    ck_bufs = dict(local=torch.zeros((b, 3, MAX_CANDIDATES, 32), dtype=torch.int8, device="cuda"),
                   global_=torch.zeros((b, 3, 32), dtype=torch.int8, device="cuda"),
                   head_scores=torch.zeros((b, 3, MAX_CANDIDATES), dtype=torch.int32,
                                           device="cuda"),
                   head_stats=torch.zeros((b, MAX_CANDIDATES, 3), dtype=torch.int8,
                                          device="cuda"),
                   head_weights=torch.zeros((b, MAX_CANDIDATES, 3), dtype=torch.int32,
                                            device="cuda"),
                   h2=torch.zeros((b, 3, MAX_CANDIDATES, 16), dtype=torch.int8, device="cuda"))
    ck = _lib.SelectorCkpt(*[ck_bufs[k].data_ptr() for k in (
        "local", "global_", "head_scores", "head_stats", "head_weights", "h2")])
    L = _lib.lib()
    ws = torch.empty(max(1, L.hv_selector_workspace_bytes(b)), dtype=torch.uint8, device="cuda")
    _lib.check(L.hv_selector_forward(dev.struct, dev_in.data_ptr(), off.data_ptr(),
                                     pkg_in.data_ptr(), b, out.data_ptr(), out_off.data_ptr(),
                                     pkg_out.data_ptr(), fused.data_ptr(), kept.data_ptr(),
                                     state.data_ptr(), ck, ws.data_ptr(), ws.numel(), _stream()),
               "token_selector")
    out, out_off = out.cpu().numpy(), out_off.cpu().numpy()
    fused, kept, state = fused.cpu().numpy(), kept.cpu().numpy(), state.cpu().numpy()
    host = {k: v.cpu().numpy() for k, v in ck_bufs.items()}
    results = []
    for i in range(b):
        c = lens[i] - 1
        if state[i, 0] < 0:
            raise ValueError(f"token set {i}: invalid selector input")
        results.append(SelectorResult(
            tokens=out[out_off[i]:out_off[i + 1]].copy(), token_count=int(state[i, 0]),
            package_present=bool(state[i, 1]), kept_normal_count=int(state[i, 2]),
            pruned_normal_count=int(state[i, 3]), warnings=int(state[i, 4]),
            local=host["local"][i, :, :c].copy(), global_features=host["global_"][i].copy(),
            head_scores=host["head_scores"][i, :, :c].copy(),
            head_stats=host["head_stats"][i, :c].copy(),
            head_weights=host["head_weights"][i, :c].copy(),
            fused_scores=fused[i, :c].copy(), kept_index=kept[i, :state[i, 2]].copy(),
            h2=host["h2"][i, :, :c].copy()))
    return results


def token_selector(tokens, package_present, params):
    """selector.token_selector (selector.py:503) on the GPU."""
    return token_selector_batch([tokens], [package_present], params)[0]


@dataclass(frozen=True)
class FinalizeResult:
    tokens: np.ndarray
    package_present: bool = False
    kept_normal_count: int = 0
    pruned_normal_count: int = 0
    warnings: int = 0
    kept_index: np.ndarray = None


def finalize_tokens(cls, normal, incoming_package, scores):
    """selector.finalize_tokens (selector.py:421) on the GPU for 192-wide
    tokens: stable keep of scores >= 32768, package accumulation."""
    cls = np.asarray(cls, np.int64).reshape(-1)
    if cls.size != 192:
        raise ValueError("the HIP finalize handles 192-channel tokens")
    normal = np.asarray(normal, np.int64).reshape(-1, 192)
    scores = np.asarray(scores, np.int64).reshape(-1)
    if scores.size and (scores.min() < 0 or scores.max() > Q016_ONE):
        raise ValueError("scores outside Q0.16 [0, 65536]")
    pkg = incoming_package is not None
    if pkg and len(normal) == 0:
        raise ValueError("incoming package requires at least one candidate")
    if len(scores) != len(normal) + pkg:
        raise ValueError("scores length must match normal candidates")
    rows = [cls[None], normal] + ([np.asarray(incoming_package, np.int64).reshape(1, 192)]
                                  if pkg else [])
    tokens = np.concatenate(rows)
    if tokens.min() < -128 or tokens.max() > 127:
        raise ValueError("tokens outside int8")
    n = len(tokens)
    if n - 1 > MAX_CANDIDATES:
        raise ValueError("at most 196 candidates")
    dev = torch.from_numpy(np.ascontiguousarray(tokens, np.int8)).cuda()
    off = torch.tensor([0, n], dtype=torch.int32, device="cuda")
    pkg_in = torch.tensor([int(pkg)], dtype=torch.uint8, device="cuda")
    fused = torch.zeros((1, MAX_CANDIDATES), dtype=torch.int32, device="cuda")
    fused[0, :len(scores)] = torch.from_numpy(scores.astype(np.int32))
    out = torch.empty((n + 1, 192), dtype=torch.int8, device="cuda")
    out_off = torch.empty(2, dtype=torch.int32, device="cuda")
    pkg_out = torch.empty(1, dtype=torch.uint8, device="cuda")
    kept = torch.empty((1, MAX_CANDIDATES), dtype=torch.int32, device="cuda")
    state = torch.empty((1, 5), dtype=torch.int32, device="cuda")
    _lib.check(_lib.lib().hv_selector_finalize(
        dev.data_ptr(), off.data_ptr(), pkg_in.data_ptr(), fused.data_ptr(), 1, out.data_ptr(),
        out_off.data_ptr(), pkg_out.data_ptr(), kept.data_ptr(), state.data_ptr(), _stream()),
        "finalize_tokens")
    st = state.cpu().numpy()[0]
    if st[0] < 0:
        raise ValueError("invalid finalize input")
    o = out_off.cpu().numpy()
    return FinalizeResult(tokens=out.cpu().numpy()[o[0]:o[1]].copy(),
                          package_present=bool(st[1]), kept_normal_count=int(st[2]),
                          pruned_normal_count=int(st[3]), warnings=int(st[4]),
                          kept_index=kept.cpu().numpy()[0, :st[2]].copy())
