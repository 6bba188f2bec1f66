"""Parameter objects shaped like the reference's (verification/heatvit_ref
model.py:24-47, transformer.py:51-398, selector.py:111-222) are accepted
wherever this package takes parameters: params.coerce rebuilds them field
by field.  The stand-ins here are plain namedtuples holding nested tuples of
Python ints, the reference dataclasses' own value types."""

import collections
import dataclasses

import numpy as np
import pytest

from heatvit_amd import params as P
from heatvit_amd import synth


def _tuples(v):
    if isinstance(v, np.ndarray):
        return v.tolist() if v.ndim == 0 else tuple(_tuples(x) for x in v)
    if isinstance(v, (list, tuple)):
        return tuple(_tuples(x) for x in v)
    if isinstance(v, np.integer):
        return int(v)
    return v


def standin(obj):
    """A namedtuple with the same field names as the dataclass `obj`,
    nested containers converted alike."""
    if dataclasses.is_dataclass(obj):
        names = [f.name for f in dataclasses.fields(obj)]
        cls = collections.namedtuple(type(obj).__name__ + "Like", names)
        return cls(*[standin(getattr(obj, n)) for n in names])
    if isinstance(obj, tuple) and obj and dataclasses.is_dataclass(obj[0]):
        return tuple(standin(x) for x in obj)
    return _tuples(obj)


def _assert_same(a, b, path="params"):
    assert type(a) is type(b), path
    for f in dataclasses.fields(a):
        x, y = getattr(a, f.name), getattr(b, f.name)
        p = f"{path}.{f.name}"
        if dataclasses.is_dataclass(x):
            _assert_same(x, y, p)
        elif isinstance(x, tuple) and x and dataclasses.is_dataclass(x[0]):
            assert len(x) == len(y), p
            for i, (u, v) in enumerate(zip(x, y)):
                _assert_same(u, v, f"{p}[{i}]")
        elif isinstance(x, np.ndarray):
            assert x.dtype == y.dtype and np.array_equal(x, y), p
        else:
            assert x == y, p


def test_model_params_from_reference_shaped_object():
    _, params = synth.pruned_workload(1)
    ref_like = standin(params)
    assert not isinstance(ref_like, P.HeatViTParams)
    got = P.coerce(ref_like, P.HeatViTParams)
    _assert_same(got, params)
    assert P.coerce(params, P.HeatViTParams) is params


def test_block_and_selector_params_from_reference_shaped_objects():
    _, bp = synth.block_workload()
    _assert_same(P.coerce(standin(bp), P.BlockParams), bp)
    _, sp = synth.selector_workload()
    _assert_same(P.coerce(standin(sp), P.SelectorParams), sp)


def test_defaults_fill_missing_optional_fields():
    _, sp = synth.selector_workload()
    full = standin(sp)
    short = collections.namedtuple("S", "local score head_weight")(
        full.local, full.score, full.head_weight)
    got = P.coerce(short, P.SelectorParams)
    assert got.in_scale_exp == -7 and got.heads == 3


def test_missing_required_field_and_bad_values_raise():
    _, bp = synth.block_workload()
    like = standin(bp)
    with pytest.raises(TypeError, match="mhsa"):
        P.coerce(collections.namedtuple("B", "ffn")(like.ffn), P.BlockParams)
    with pytest.raises(TypeError):
        P.coerce([1, 2, 3], P.BlockParams)
    bad = like._replace(mhsa=like.mhsa._replace(wqkv=((300,) * 576,) * 192))
    with pytest.raises(ValueError, match="wqkv"):
        P.coerce(bad, P.BlockParams)
    flt = like._replace(ffn=like.ffn._replace(b1=(0.5,) * 768))
    with pytest.raises(TypeError):
        P.coerce(flt, P.BlockParams)
