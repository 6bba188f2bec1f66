"""Immutable HeatViT-T parameter containers.

Field names, shapes, defaults and validation errors follow the reference's
golden-model dataclasses so callers can pass the same keyword arguments:
  PatchParams        verification/heatvit_ref/transformer.py:51-93
  MhsaParams         verification/heatvit_ref/transformer.py:148-198
  FfnParams          verification/heatvit_ref/transformer.py:287-325
  BlockParams        verification/heatvit_ref/transformer.py:387-398
  Selector*Params    verification/heatvit_ref/selector.py:111-222
  HeatViTParams      verification/heatvit_ref/model.py:24-47

Tensors are stored as read-only numpy arrays (int8 weights in row-major
[K][N], int32 biases) instead of nested tuples; nested lists/tuples and
arrays are both accepted.  Floats raise TypeError, out-of-range values and
wrong shapes raise ValueError, as in the reference.
"""

from dataclasses import MISSING, dataclass, field, fields

import numpy as np

INT8 = (-128, 127)
INT32 = (-(1 << 31), (1 << 31) - 1)


def _as_int_array(name, value, shape, lo, hi, dtype):
    if isinstance(value, float):
        raise TypeError(f"{name} must be an integer tensor, got float")
    arr = np.asarray(value)
    if arr.dtype.kind == "f":
        raise TypeError(f"{name} must hold integers, got floats")
    if arr.dtype.kind == "O":
        for v in arr.reshape(-1):
            if isinstance(v, float):
                raise TypeError(f"{name} must hold integers, got floats")
        arr = arr.astype(np.int64)
    if arr.dtype.kind not in "iub":
        raise TypeError(f"{name} must hold integers")
    if tuple(arr.shape) != tuple(shape):
        raise ValueError(f"{name} must have shape {tuple(shape)}, got {tuple(arr.shape)}")
    if arr.size and (int(arr.min()) < lo or int(arr.max()) > hi):
        raise ValueError(f"{name} has values outside [{lo}, {hi}]")
    out = np.ascontiguousarray(arr, dtype=dtype)
    out.setflags(write=False)
    return out


def _i8(name, value, *shape):
    return _as_int_array(name, value, shape, *INT8, np.int8)


def _i32(name, value, *shape):
    return _as_int_array(name, value, shape, *INT32, np.int32)


def _check_exps(obj):
    for f in fields(obj):
        if f.name.endswith("_exp"):
            v = getattr(obj, f.name)
            if isinstance(v, float):
                raise TypeError(f"{f.name} must be an integer")
            if not isinstance(v, (int, np.integer)):
                raise TypeError(f"{f.name} must be an integer")
            object.__setattr__(obj, f.name, int(v))


@dataclass(frozen=True)
class PatchParams:
    patch_weight: object = ()
    patch_bias: object = ()
    cls: object = ()
    pos: object = ()
    width: int = 224
    height: int = 224
    patch: int = 16
    embed_dim: int = 192
    tokens: int = 197
    image_scale_exp: int = -7
    weight_scale_exp: int = -7
    activation_scale_exp: int = -7
    tokens_scale_exp: int = -7
    cls_scale_exp: int = -7
    pos_scale_exp: int = -7

    def __post_init__(self):
        if self.embed_dim != 192:
            raise ValueError("embed_dim must be 192")
        if self.tokens != 197:
            raise ValueError("tokens must be 197")
        if self.width % self.patch or self.height % self.patch:
            raise ValueError("image size must be a multiple of patch")
        if (self.width // self.patch) * (self.height // self.patch) + 1 != self.tokens:
            raise ValueError("tokens must be num_patches + 1")
        kdim = self.patch * self.patch * 3
        object.__setattr__(self, "patch_weight", _i8("patch_weight", self.patch_weight, kdim, 192))
        object.__setattr__(self, "patch_bias", _i32("patch_bias", self.patch_bias, 192))
        object.__setattr__(self, "cls", _i8("cls", self.cls, 192))
        object.__setattr__(self, "pos", _i8("pos", self.pos, self.tokens, 192))
        _check_exps(self)


@dataclass(frozen=True)
class MhsaParams:
    ln_gamma: object = ()
    ln_beta: object = ()
    wqkv: object = ()
    bqkv: object = ()
    wproj: object = ()
    bproj: object = ()
    embed_dim: int = 192
    heads: int = 3
    head_dim: int = 64
    x_scale_exp: int = -7
    gamma1_scale_exp: int = -6
    beta1_scale_exp: int = -7
    ln1_out_scale_exp: int = -7
    wqkv_scale_exp: int = -7
    qkv_out_scale_exp: int = -7
    score_scale_exp: int = -17
    prob_scale_exp: int = -8
    context_out_scale_exp: int = -7
    wproj_scale_exp: int = -7
    msa_out_scale_exp: int = -7

    def __post_init__(self):
        if (self.embed_dim, self.heads, self.head_dim) != (192, 3, 64):
            raise ValueError("MHSA dims must be 192/3/64")
        object.__setattr__(self, "ln_gamma", _i8("ln_gamma", self.ln_gamma, 192))
        object.__setattr__(self, "ln_beta", _i8("ln_beta", self.ln_beta, 192))
        object.__setattr__(self, "wqkv", _i8("wqkv", self.wqkv, 192, 576))
        object.__setattr__(self, "bqkv", _i32("bqkv", self.bqkv, 576))
        object.__setattr__(self, "wproj", _i8("wproj", self.wproj, 192, 192))
        object.__setattr__(self, "bproj", _i32("bproj", self.bproj, 192))
        _check_exps(self)


@dataclass(frozen=True)
class FfnParams:
    ln_gamma: object = ()
    ln_beta: object = ()
    w1: object = ()
    b1: object = ()
    w2: object = ()
    b2: object = ()
    embed_dim: int = 192
    ffn_dim: int = 768
    x_scale_exp: int = -7
    gamma2_scale_exp: int = -6
    beta2_scale_exp: int = -7
    ln2_out_scale_exp: int = -7
    w1_scale_exp: int = -7
    hidden_out_scale_exp: int = -7
    w2_scale_exp: int = -7
    ffn_out_scale_exp: int = -7
    out_scale_exp: int = -7

    def __post_init__(self):
        if (self.embed_dim, self.ffn_dim) != (192, 768):
            raise ValueError("FFN dims must be 192/768")
        object.__setattr__(self, "ln_gamma", _i8("ln_gamma", self.ln_gamma, 192))
        object.__setattr__(self, "ln_beta", _i8("ln_beta", self.ln_beta, 192))
        object.__setattr__(self, "w1", _i8("w1", self.w1, 192, 768))
        object.__setattr__(self, "b1", _i32("b1", self.b1, 768))
        object.__setattr__(self, "w2", _i8("w2", self.w2, 768, 192))
        object.__setattr__(self, "b2", _i32("b2", self.b2, 192))
        _check_exps(self)


@dataclass(frozen=True)
class BlockParams:
    mhsa: MhsaParams
    ffn: FfnParams

    def __post_init__(self):
        if not isinstance(self.mhsa, MhsaParams):
            raise TypeError("mhsa must be MhsaParams")
        if not isinstance(self.ffn, FfnParams):
            raise TypeError("ffn must be FfnParams")


@dataclass(frozen=True)
class SelectorLocalParams:
    w: object = ()  # [3][64][32] int8
    b: object = ()  # [3][32] int32

    def __post_init__(self):
        object.__setattr__(self, "w", _i8("local w", self.w, 3, 64, 32))
        object.__setattr__(self, "b", _i32("local b", self.b, 3, 32))


@dataclass(frozen=True)
class SelectorScoreParams:
    w1: object = ()  # [3][64][32]
    b1: object = ()  # [3][32]
    w2: object = ()  # [3][32][16]
    b2: object = ()  # [3][16]
    w3: object = ()  # [3][16][2]
    b3: object = ()  # [3][2]

    def __post_init__(self):
        object.__setattr__(self, "w1", _i8("score w1", self.w1, 3, 64, 32))
        object.__setattr__(self, "b1", _i32("score b1", self.b1, 3, 32))
        object.__setattr__(self, "w2", _i8("score w2", self.w2, 3, 32, 16))
        object.__setattr__(self, "b2", _i32("score b2", self.b2, 3, 16))
        object.__setattr__(self, "w3", _i8("score w3", self.w3, 3, 16, 2))
        object.__setattr__(self, "b3", _i32("score b3", self.b3, 3, 2))


@dataclass(frozen=True)
class SelectorHeadWeightParams:
    w1: object = ()  # [3][3]
    b1: object = ()  # [3]
    w2: object = ()  # [3][3]
    b2: object = ()  # [3]

    def __post_init__(self):
        object.__setattr__(self, "w1", _i8("head w1", self.w1, 3, 3))
        object.__setattr__(self, "b1", _i32("head b1", self.b1, 3))
        object.__setattr__(self, "w2", _i8("head w2", self.w2, 3, 3))
        object.__setattr__(self, "b2", _i32("head b2", self.b2, 3))


@dataclass(frozen=True)
class SelectorParams:
    local: SelectorLocalParams
    score: SelectorScoreParams
    head_weight: SelectorHeadWeightParams
    heads: int = 3
    head_dim: int = 64
    local_dim: int = 32
    activation_scale_exp: int = -7
    weight_scale_exp: int = -7
    logits_scale_exp: int = -7
    in_scale_exp: int = -7
    local_w_scale_exp: int = -7
    local_out_scale_exp: int = -7
    concat_out_scale_exp: int = -7
    score_w1_scale_exp: int = -7
    score_w2_scale_exp: int = -7
    score_w3_scale_exp: int = -7
    h1_out_scale_exp: int = -7
    h2_out_scale_exp: int = -7
    logits_out_scale_exp: int = -7
    stats_out_scale_exp: int = -7
    hw_w1_scale_exp: int = -7
    hw_hidden_out_scale_exp: int = -7
    hw_w2_scale_exp: int = -7

    def __post_init__(self):
        if (self.heads, self.head_dim, self.local_dim) != (3, 64, 32):
            raise ValueError("selector dims must be 3 heads / 64 / 32")
        if not isinstance(self.local, SelectorLocalParams):
            raise TypeError("local must be SelectorLocalParams")
        if not isinstance(self.score, SelectorScoreParams):
            raise TypeError("score must be SelectorScoreParams")
        if not isinstance(self.head_weight, SelectorHeadWeightParams):
            raise TypeError("head_weight must be SelectorHeadWeightParams")
        _check_exps(self)


@dataclass(frozen=True)
class HeatViTParams:
    patch: PatchParams
    blocks: tuple
    selectors: tuple
    final_gamma: object
    final_beta: object
    head_w: object
    head_b: object
    final_gamma_scale_exp: int = -6
    final_beta_scale_exp: int = -7
    final_ln_out_scale_exp: int = -7
    head_w_scale_exp: int = -7
    selector_blocks: tuple = (4, 7, 10)

    def __post_init__(self):
        if len(self.blocks) != 12:
            raise ValueError("HeatViT-T needs exactly 12 blocks")
        if len(self.selectors) != len(self.selector_blocks):
            raise ValueError("selector count must match selector_blocks")
        if len(self.selector_blocks) > 3:
            raise ValueError("at most three selectors are supported")
        object.__setattr__(self, "blocks", tuple(self.blocks))
        object.__setattr__(self, "selectors", tuple(self.selectors))
        object.__setattr__(self, "selector_blocks", tuple(int(b) for b in self.selector_blocks))
        if list(self.selector_blocks) != sorted(set(self.selector_blocks)) or any(
                b < 1 or b > 12 for b in self.selector_blocks):
            raise ValueError("selector_blocks must be increasing block numbers in 1..12")
        object.__setattr__(self, "final_gamma", _i8("final_gamma", self.final_gamma, 192))
        object.__setattr__(self, "final_beta", _i8("final_beta", self.final_beta, 192))
        object.__setattr__(self, "head_w", _i8("head_w", self.head_w, 192, 1000))
        object.__setattr__(self, "head_b", _i32("head_b", self.head_b, 1000))
        _check_exps(self)


# Container-valued fields, per container class.
_NESTED = {
    (HeatViTParams, "patch"): lambda v: coerce(v, PatchParams),
    (HeatViTParams, "blocks"): lambda v: tuple(coerce(b, BlockParams) for b in v),
    (HeatViTParams, "selectors"): lambda v: tuple(coerce(s, SelectorParams) for s in v),
    (BlockParams, "mhsa"): lambda v: coerce(v, MhsaParams),
    (BlockParams, "ffn"): lambda v: coerce(v, FfnParams),
    (SelectorParams, "local"): lambda v: coerce(v, SelectorLocalParams),
    (SelectorParams, "score"): lambda v: coerce(v, SelectorScoreParams),
    (SelectorParams, "head_weight"): lambda v: coerce(v, SelectorHeadWeightParams),
}


def coerce(obj, cls):
    """`obj` as an instance of `cls` (one of the containers above).

    An instance is returned unchanged.  Any other object is rebuilt from its
    attributes of the same names -- the reference's own frozen dataclasses
    (model.py:24-47, transformer.py:51-398, selector.py:111-222) or any
    stand-in with those fields -- with nested containers converted alike and
    every value validated as for a direct construction.  A missing field
    that has no default raises TypeError."""
    if isinstance(obj, cls):
        return obj
    kwargs = {}
    for f in fields(cls):
        if not hasattr(obj, f.name):
            if f.default is MISSING and f.default_factory is MISSING:
                raise TypeError(f"{type(obj).__name__} lacks field {f.name!r} of {cls.__name__}")
            continue
        v = getattr(obj, f.name)
        conv = _NESTED.get((cls, f.name))
        kwargs[f.name] = conv(v) if conv else v
    return cls(**kwargs)


SCALE_EXP_RANGE = (-32, 31)


def check_scale_exps(obj):
    """Raise ValueError when any *_scale_exp is outside the 6-bit signed
    range [-32, 31] (descriptor.py:53-62)."""
    stack = [obj]
    while stack:
        o = stack.pop()
        if isinstance(o, (tuple, list)):
            stack.extend(o)
            continue
        if not hasattr(o, "__dataclass_fields__"):
            continue
        for f in fields(o):
            v = getattr(o, f.name)
            if f.name.endswith("_exp"):
                if not SCALE_EXP_RANGE[0] <= v <= SCALE_EXP_RANGE[1]:
                    raise ValueError(f"{type(o).__name__}.{f.name}={v} outside [-32, 31]")
            elif hasattr(v, "__dataclass_fields__") or isinstance(v, (tuple, list)):
                stack.append(v)


__all__ = [
    "PatchParams", "MhsaParams", "FfnParams", "BlockParams", "SelectorLocalParams",
    "SelectorScoreParams", "SelectorHeadWeightParams", "SelectorParams", "HeatViTParams",
    "check_scale_exps", "coerce", "field",
]
