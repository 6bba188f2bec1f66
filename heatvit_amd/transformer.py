"""Transformer stages on the GPU, with the golden model's signatures.

  patch_embedding(image, PatchParams)      transformer.py:104-145
  transformer_block(x, BlockParams)        transformer.py:401-431
  transformer_block_batch(xs, BlockParams) the same over a ragged batch

Activations travel as packed rows [T][192] with per-image offsets; a
block's checkpoints use the reference's keys (transformer.py:274-283,
378-383, 428-431).
"""

import numpy as np
import torch

from . import _lib
from .device import DeviceBlock, _Holder, _patch_struct
from .params import PatchParams, check_scale_exps, coerce


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _rows_i8(name, x):
    if isinstance(x, torch.Tensor):
        x = x.cpu().numpy()
    a = np.asarray(x)
    if a.dtype.kind == "f":
        raise TypeError(f"{name} must hold integers")
    if a.ndim != 2 or a.shape[1] != 192:
        raise ValueError(f"{name} must be [N][192]")
    if a.size and (a.min() < -128 or a.max() > 127):
        raise ValueError(f"{name} outside int8")
    return np.ascontiguousarray(a, np.int8)


def patch_embedding(image, params, *, batch=False):
    """NHWC image(s) -> [197][192] int8 at tokens_scale_exp.  With
    batch=True, `image` is [B][224*224*3] (or [B][224][224][3]) and the
    result is [B][197][192]."""
    params = coerce(params, PatchParams)
    check_scale_exps(params)
    if (params.width, params.height, params.patch) != (224, 224, 16):
        raise ValueError("the HIP patch embedding handles 224x224x3 images with 16x16 patches")
    img = np.asarray(image)
    if img.dtype.kind == "f":
        raise TypeError("image must hold integers")
    img = img.reshape((-1, 224 * 224 * 3) if batch else (1, 224 * 224 * 3))
    if img.size and (img.min() < -128 or img.max() > 127):
        raise ValueError("image outside int8")
    h = _Holder("cuda")
    st = _patch_struct(params, h)
    dev = torch.from_numpy(np.ascontiguousarray(img, np.int8)).cuda()
    out = torch.empty((len(img), 197, 192), dtype=torch.int8, device="cuda")
    _lib.check(_lib.lib().hv_patch_embedding(st, dev.data_ptr(), len(img), out.data_ptr(),
                                             _stream()), "patch_embedding")
    res = out.cpu().numpy()
    return res if batch else res[0]


CHECKPOINT_KEYS = ("ln1", "fused_qkv", "qkv", "score", "prob", "context", "concat", "msa", "y",
                   "ln2", "hidden", "ffn_out", "z")


def transformer_block_batch(xs, params, checkpoints=False, warnings=False):
    """Runs one block over a ragged batch (each x is [N_i][192], N_i <= 197).
    Returns the list of z arrays, plus per-image checkpoint dicts when asked,
    plus (warnings=True) the per-image warning bits [B] int32
    (WARN_LN_NEGATIVE_VARIANCE when LN1 or LN2 clamped a row's variance)."""
    if isinstance(params, DeviceBlock):
        dev = params
    else:
        dev = DeviceBlock(params)
    xs = [_rows_i8("x", x) for x in xs]
    lens = [len(x) for x in xs]
    if not xs or any(n < 1 or n > 197 for n in lens):
        raise ValueError("each image needs 1..197 token rows")
    b = len(xs)
    offsets = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    t = int(offsets[-1])
    x = torch.from_numpy(np.concatenate(xs)).cuda()
    off = torch.from_numpy(offsets).cuda()
    z = torch.empty((t, 192), dtype=torch.int8, device="cuda")
    status = torch.empty(b, dtype=torch.int32, device="cuda")
    warn = torch.empty(b, dtype=torch.int32, device="cuda")
    L = _lib.lib()
    ws = torch.empty(L.hv_block_workspace_bytes(b, t), dtype=torch.uint8, device="cuda")
    ck = None
    bufs = {}
    if checkpoints:
        bufs = dict(ln1=(t, 192), fused_qkv=(t, 576), concat=(t, 192), msa=(t, 192),
                    y=(t, 192), ln2=(t, 192), hidden=(t, 768), ffn_out=(t, 192))
        bufs = {k: torch.empty(s, dtype=torch.int8, device="cuda") for k, s in bufs.items()}
        bufs["score"] = torch.zeros((b, 3, 197, 197), dtype=torch.int32, device="cuda")
        bufs["prob"] = torch.zeros((b, 3, 197, 197), dtype=torch.uint8, device="cuda")
        ck = _lib.BlockCkpt(*[bufs[k].data_ptr() for k in (
            "ln1", "fused_qkv", "concat", "msa", "y", "ln2", "hidden", "ffn_out", "score",
            "prob")])
    _lib.check(L.hv_block_forward(dev.struct, x.data_ptr(), off.data_ptr(), b, t, z.data_ptr(),
                                  ck, status.data_ptr(), warn.data_ptr(), ws.data_ptr(),
                                  ws.numel(), _stream()), "transformer_block")
    if status.any():
        e = ValueError("transformer_block: token count outside [1, 197]")
        e.error_class = _lib.HV_ERR_TOKEN_COUNT
        raise e
    zs = z.cpu().numpy()
    outs = [zs[offsets[i]:offsets[i + 1]] for i in range(b)]
    tail = (warn.cpu().numpy(),) if warnings else ()
    if not checkpoints:
        return (outs, *tail) if tail else outs
    host = {k: v.cpu().numpy() for k, v in bufs.items()}
    per_image = []
    for i in range(b):
        lo, hi, n = offsets[i], offsets[i + 1], lens[i]
        d = {k: host[k][lo:hi] for k in ("ln1", "fused_qkv", "concat", "msa", "y", "ln2",
                                        "hidden", "ffn_out")}
        d["score"] = host["score"][i, :, :n, :n]
        d["prob"] = host["prob"][i, :, :n, :n]
        d["qkv"] = d["fused_qkv"].reshape(n, 3, 3, 64).transpose(1, 2, 0, 3)
        d["context"] = d["concat"].reshape(n, 3, 64).transpose(1, 0, 2)
        d["z"] = outs[i]
        per_image.append(d)
    return (outs, per_image, *tail)


def transformer_block(x, params):
    """transformer_block (transformer.py:401): returns (z, checkpoints)."""
    outs, cks = transformer_block_batch([x], params, checkpoints=True)
    return outs[0], cks[0]
