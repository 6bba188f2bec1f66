"""GPU element-wise and row-wise primitives, mirroring the golden model's
fixed.py / nonlinear.py / gemm.py functions on whole arrays.

  requant, round_shift_away      fixed.py:15-45
  gelu, plan_sigmoid             nonlinear.py:60-95
  softmax_attention/_selector    nonlinear.py:109-133 (ragged batches of rows)
  layernorm_rows                 nonlinear.py:136-186
  attention                      mhsa's attention core (transformer.py:228-266)
  gemm_writeback                 gemm.gemm_numpy + gemm_writeback (gemm.py:93-139)

Inputs are array-likes on the host or torch tensors on the GPU; results
come back as numpy arrays.  Every call runs the HIP kernels.
"""

import numpy as np
import torch

from . import _lib
from .device import pack_mfma32


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _to_dev(arr, dtype):
    if isinstance(arr, torch.Tensor):
        return arr.to(device="cuda", dtype=dtype).contiguous()
    np_dtype = {torch.int8: np.int8, torch.int32: np.int32, torch.int64: np.int64,
                torch.uint8: np.uint8}[dtype]
    a = np.asarray(arr)
    if a.dtype.kind == "f":
        raise TypeError("integer inputs required, got floats")
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np_dtype)).cuda()


def _prim(op, values, a=0, b=0, c=0):
    x = _to_dev(values, torch.int64).reshape(-1)
    out = torch.empty_like(x)
    _lib.check(_lib.lib().hv_eval_primitive(op, x.data_ptr(), out.data_ptr(), x.numel(), a, b,
                                            c, _stream()), "primitive")
    return out.cpu().numpy().reshape(np.shape(values))


def requant(values, src_exp, dst_exp, bits):
    """fixed.requant over an int64 array (|value| < 2^62, bits <= 63)."""
    return _prim(_lib.HV_PRIM_REQUANT, values, src_exp, dst_exp, bits)


def round_shift_away(values, shift):
    return _prim(_lib.HV_PRIM_RSA, values, shift)


def gelu(values):
    """nonlinear.gelu over 24-bit signed Q8.16 inputs."""
    v = np.asarray(values)
    if v.size and (v.min() < -(1 << 23) or v.max() >= (1 << 23)):
        raise ValueError("gelu inputs must be 24-bit signed Q8.16")
    return _prim(_lib.HV_PRIM_GELU, values)


def gelu_post(values, so, table=False):
    """requant(gelu(q), -16, so - 16, 8), the FFN GELU post-op, over Q8.16
    values (saturated to 24 bits); table=True reads the step tables the
    FFN GEMM uses (so in [3, 12])."""
    return _prim(_lib.HV_PRIM_GELU_TABLE if table else _lib.HV_PRIM_GELU_POST, values, so)


def plan_sigmoid(values):
    return _prim(_lib.HV_PRIM_PLAN, values)


def softmax_rows(rows):
    """Both softmax narrowings for a list of rows (each <= 256 long):
    returns (attention UQ0.8 rows, selector Q0.16 rows)."""
    lens = [len(r) for r in rows]
    if any(n == 0 for n in lens):
        raise ValueError("softmax row must not be empty")
    if any(n > 256 for n in lens):
        raise ValueError("softmax rows longer than 256 are not supported")
    offsets = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    flat = np.concatenate([np.asarray(r, np.int64) for r in rows])
    if flat.min() < -(1 << 31) or flat.max() >= (1 << 31):
        raise ValueError("softmax inputs must fit int32")
    x = _to_dev(flat, torch.int32)
    off = _to_dev(offsets, torch.int32)
    att = torch.empty(len(flat), dtype=torch.uint8, device="cuda")
    sel = torch.empty(len(flat), dtype=torch.int32, device="cuda")
    _lib.check(_lib.lib().hv_softmax_rows(x.data_ptr(), off.data_ptr(), len(rows),
                                          att.data_ptr(), sel.data_ptr(), _stream()), "softmax")
    att, sel = att.cpu().numpy(), sel.cpu().numpy()
    return ([att[offsets[i]:offsets[i + 1]] for i in range(len(rows))],
            [sel[offsets[i]:offsets[i + 1]] for i in range(len(rows))])


def softmax_attention(row):
    return softmax_rows([row])[0][0]


def softmax_selector(row):
    return softmax_rows([row])[1][0]


def layernorm_rows(x, gamma, beta, x_scale, gamma_scale, beta_scale, out_scale):
    """nonlinear.layernorm on every row of x [R][192]; returns
    (outputs [R][192] int8, negative_variance [R] bool)."""
    x = np.asarray(x)
    if x.ndim != 2 or x.shape[1] != 192:
        raise ValueError("layernorm rows must have exactly 192 channels")
    xd = _to_dev(x, torch.int8)
    g = _to_dev(gamma, torch.int8)
    b = _to_dev(beta, torch.int8)
    y = torch.empty_like(xd)
    neg = torch.zeros(len(x), dtype=torch.uint8, device="cuda")
    _lib.check(_lib.lib().hv_layernorm_i8(xd.data_ptr(), g.data_ptr(), b.data_ptr(),
                                          y.data_ptr(), len(x), None, x_scale, gamma_scale,
                                          beta_scale, out_scale, neg.data_ptr(), _stream()),
               "layernorm")
    return y.cpu().numpy(), neg.cpu().numpy().astype(bool)


def attention(fused_qkv, qkv_exp, score_exp, prob_exp, context_exp):
    """The attention core of transformer.mhsa (transformer.py:228-266) for
    a batch of images: fused_qkv is one [N][576] int8 array per image (Q,
    K, V column blocks, heads of 64).  Returns one (score [3][N][N] int32,
    prob [3][N][N] uint8, concat [N][192] int8) per image, the `score`,
    `prob` and `concat` checkpoints of mhsa."""
    mats = [np.asarray(q) for q in fused_qkv]
    if not mats:
        return []
    for q in mats:
        if q.ndim != 2 or q.shape[1] != 576:
            raise ValueError("fused_qkv rows must have 576 channels")
        if not 1 <= len(q) <= 197:
            raise ValueError(f"token count {len(q)} outside [1, 197]")
    lens = [len(q) for q in mats]
    offsets = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    qkv = _to_dev(np.concatenate(mats), torch.int8)
    off = _to_dev(offsets, torch.int32)
    b, rows = len(mats), int(offsets[-1])
    ctx = torch.empty((rows, 192), dtype=torch.int8, device="cuda")
    score = torch.zeros((b, 3, 197, 197), dtype=torch.int32, device="cuda")
    prob = torch.zeros((b, 3, 197, 197), dtype=torch.uint8, device="cuda")
    status = torch.zeros(b, dtype=torch.int32, device="cuda")
    _lib.check(_lib.lib().hv_attention_i8(qkv.data_ptr(), off.data_ptr(), b, rows, ctx.data_ptr(),
                                          score.data_ptr(), prob.data_ptr(), qkv_exp, score_exp,
                                          prob_exp, context_exp, status.data_ptr(), _stream()),
               "attention")
    if status.any():
        raise ValueError("attention: token count outside [1, 197]")
    ctx, score, prob = ctx.cpu().numpy(), score.cpu().numpy(), prob.cpu().numpy()
    return [(score[i, :, :n, :n], prob[i, :, :n, :n], ctx[offsets[i]:offsets[i + 1]])
            for i, n in enumerate(lens)]


def gemm_writeback(a, w, bias, src_exp, dst_exp, output_bits, *, epilogue=None, mid_exp=0,
                   residual=None, res_exp=0, a_rows=None, a_unsigned=False):
    """requant(A W + bias) as gemm_writeback(gemm_numpy(...)) computes it,
    on the MFMA GEMM.  A [M][K] int8 (uint8 with a_unsigned, gemm.py:93-114),
    W [K][N] int8 (row-major, reference layout), bias [N] int32 or None.  K
    is zero-padded to a multiple of 32.  `epilogue` selects the fused
    variants ('gelu', 'residual')."""
    a = np.asarray(a)
    w = np.asarray(w)
    m, k = a.shape
    if w.shape[0] != k:
        raise ValueError(f"K mismatch: a has {k}, b has {w.shape[0]}")
    lo, hi = (0, 255) if a_unsigned else (-128, 127)
    if a.size and (a.min() < lo or a.max() > hi):
        raise ValueError(f"A values must lie in [{lo}, {hi}]")
    if a_unsigned and a_rows is not None:
        raise ValueError("unsigned A takes whole rows (no a_rows)")
    n = w.shape[1]
    kp = -(-k // 32) * 32
    ap = np.zeros((m, kp), np.uint8 if a_unsigned else np.int8)
    ap[:, :k] = a
    ap = ap.view(np.int8)
    wp = np.zeros((kp, n), np.int8)
    wp[:k] = w
    ad = _to_dev(ap, torch.int8)
    wd = _to_dev(pack_mfma32(wp), torch.int8)
    bd = None if bias is None else _to_dev(bias, torch.int32)
    epi = {None: _lib.HV_EPI_I32 if output_bits == 32 else _lib.HV_EPI_I8,
           "gelu": _lib.HV_EPI_GELU, "residual": _lib.HV_EPI_RESIDUAL}[epilogue]
    if epilogue is None and output_bits not in (8, 32):
        raise ValueError("output_bits must be 8 or 32")
    c = torch.empty((m, n), dtype=torch.int32 if epi == _lib.HV_EPI_I32 else torch.int8,
                    device="cuda")
    rd = None if residual is None else _to_dev(residual, torch.int8)
    rows = None if a_rows is None else _to_dev(a_rows, torch.int32)
    d = _lib.GemmDesc()
    d.a, d.b_packed, d.c = ad.data_ptr(), wd.data_ptr(), c.data_ptr()
    d.bias = None if bd is None else bd.data_ptr()
    d.residual = None if rd is None else rd.data_ptr()
    d.a_rows = None if rows is None else rows.data_ptr()
    d.m, d.n, d.k, d.lda, d.ldc, d.ldr = (len(rows) if rows is not None else m), n, kp, kp, n, n
    d.a_mode = _lib.HV_A_GATHER if rows is not None else _lib.HV_A_ROWS
    if a_unsigned:
        d.a_mode |= _lib.HV_A_UNSIGNED
    d.epilogue = epi
    d.src_exp, d.dst_exp, d.mid_exp, d.res_exp = src_exp, dst_exp, mid_exp, res_exp
    if rows is not None:
        c = torch.empty((len(rows), n), dtype=c.dtype, device="cuda")
        d.c = c.data_ptr()
    _lib.check(_lib.lib().hv_gemm_i8(d, _stream()), "gemm")
    return c.cpu().numpy()
