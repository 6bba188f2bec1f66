"""Image front end on the GPU.

  real_image_list(img_float, table)    p2_export_weights.real_image_list
                                       (tools/p2/p2_export_weights.py:246-251)
  quantize_images(images, input_exp)   the same over a batch, as device tensors

Preprocessed float images (CHW [3][224][224], or a batch [B][3][224][224])
become int8 at the input exponent: q = clamp(round_half_even(x / 2^exp),
-128, 127), flat NHWC (the golden model's image) or, with
layout="patches", the patch matrix [B*196][768] of layout.patchify.
HeatViTModel.infer_float_batch runs the whole forward from float images.
"""

import numpy as np
import torch

from . import _lib

LAYOUTS = {"nhwc": 0, "patches": 1}


def _input_exp(table):
    """An int exponent, or a scale table with activation_exp("input")."""
    if hasattr(table, "activation_exp"):
        table = table.activation_exp("input")
    if isinstance(table, bool) or not isinstance(table, (int, np.integer)):
        raise TypeError("input exponent must be an integer or a scale table")
    if not -32 <= int(table) <= 31:
        raise ValueError("input scale exponent outside [-32, 31]")
    return int(table)


def float_images(images):
    """A contiguous float32 CUDA tensor [B][3][224][224] (copies as needed)."""
    t = images if isinstance(images, torch.Tensor) else torch.from_numpy(np.asarray(images))
    if not t.dtype.is_floating_point:
        raise TypeError("images must be floating point (preprocessed CHW)")
    if t.dim() == 3:
        t = t.unsqueeze(0)
    if t.dim() != 4 or tuple(t.shape[1:]) != (3, 224, 224):
        raise ValueError("images must be [3][224][224] or [B][3][224][224]")
    return t.to(device="cuda", dtype=torch.float32).contiguous()


def quantize_images(images, input_exp, layout="nhwc"):
    """Device int8 tensor: [B][150528] NHWC, or [B*196][768] patch rows."""
    exp = _input_exp(input_exp)
    if layout not in LAYOUTS:
        raise ValueError(f"layout must be one of {tuple(LAYOUTS)}")
    x = float_images(images)
    b = x.shape[0]
    shape = (b, 224 * 224 * 3) if layout == "nhwc" else (b * 196, 768)
    out = torch.empty(shape, dtype=torch.int8, device=x.device)
    _lib.check(_lib.lib().hv_quantize_images(x.data_ptr(), b, exp, LAYOUTS[layout],
                                             out.data_ptr(),
                                             torch.cuda.current_stream(x.device).cuda_stream),
               "quantize_images")
    return out


def real_image_list(img_float, table):
    """One preprocessed float CHW image -> flat NHWC int8 list at the
    table's input exponent (or an explicit exponent)."""
    q = quantize_images(img_float, table)
    if q.shape[0] != 1:
        raise ValueError("real_image_list takes one image")
    return [int(v) for v in q[0].cpu().numpy()]
