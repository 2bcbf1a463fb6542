"""Range / ParamRange (elastic_megatron/resharding/util.py:49-214) against numpy slicing."""

import numpy as np
import pytest
from hypothesis import given, settings
from hypothesis import strategies as st

from elasticmegatron_amd.resharding.util import ParamRange, Range


def test_range_basics():
    r = Range(4, 10)
    assert r.size == len(r) == 6 and not r.is_normalized
    assert r.normalize() == Range(0, 6)
    assert r.normalize(2) == Range(2, 8)
    with pytest.raises(AssertionError):
        r.normalize(5)
    assert r.chunk(3) == [Range(4, 6), Range(6, 8), Range(8, 10)]
    with pytest.raises(AssertionError):
        r.chunk(4)
    assert r.is_contain(Range(5, 10)) and not r.is_contain(Range(3, 5))
    assert Range(0, 6).get_sub_range_slices(Range(0, 6)) == (slice(None),)
    assert Range(0, 6).get_sub_range_slices(Range(2, 4)) == (slice(2, 4),)
    assert r.intersect(Range(8, 20)) == Range(8, 10) and r.intersect(Range(10, 12)) is None


@given(st.integers(1, 40), st.integers(1, 40), st.integers(1, 4), st.integers(0, 1))
@settings(max_examples=60, deadline=None)
def test_param_range_chunk_is_numpy_split(rows, cols, split, dim):
    shape = (rows * split, cols) if dim == 0 else (rows, cols * split)
    x = np.arange(shape[0] * shape[1]).reshape(shape)
    whole = ParamRange(param_shape=shape)
    for piece, ref in zip(whole.chunk(split, dim), np.split(x, split, axis=dim)):
        assert np.array_equal(x[whole.get_sub_range_slices(piece)], ref)
        assert whole.is_contain(piece) == (dim if split > 1 else -1)
        assert piece.size == ref.size


def test_param_range_contain_requires_one_dim():
    a = ParamRange(ranges=[Range(0, 8), Range(0, 8)])
    assert a.is_contain(ParamRange(ranges=[Range(0, 4), Range(0, 8)])) == 0
    assert a.is_contain(ParamRange(ranges=[Range(0, 4), Range(0, 4)])) == -1
    assert a.is_contain(ParamRange(ranges=[Range(0, 8)])) == -1
    assert a == ParamRange(param_shape=(8, 8)) and hash(a) == hash(ParamRange(param_shape=(8, 8)))
    assert a.normalize([0, 0]) == a
    assert ParamRange(ranges=[Range(2, 4)]).normalize([2]) == ParamRange(param_shape=(2,))


def test_param_range_contain_scans_dimensions_in_order():
    """util.py:154-172: the first dimension whose range contains the other's decides, unless a
    later dimension differs as well; an equal box is not a sub-box."""
    a = ParamRange(param_shape=(8, 8))
    assert a.is_contain(ParamRange(ranges=[Range(0, 8), Range(2, 6)])) == 1
    assert a.is_contain(a) == -1
    # Dimension 0 differs without containment, dimension 1 is contained: dimension 1.
    assert a.is_contain(ParamRange(ranges=[Range(4, 12), Range(0, 4)])) == 1
    # Dimension 0 contained, dimension 1 differs as well: not a sub-box.
    assert a.is_contain(ParamRange(ranges=[Range(0, 4), Range(4, 12)])) == -1
    assert a.is_contain(ParamRange(ranges=[Range(4, 12), Range(4, 12)])) == -1
    with pytest.raises(AssertionError):
        a.get_sub_range_slices(ParamRange(ranges=[Range(0, 4), Range(0, 4)]))
    with pytest.raises(AssertionError):
        ParamRange(ranges=[Range(1, 8), Range(0, 8)]).get_sub_range_slices(a)
    with pytest.raises(AssertionError):
        ParamRange(param_shape=(2, 2, 2))


def test_ranges_are_values():
    import copy
    import pickle

    r = ParamRange(ranges=[Range(2, 6), Range(0, 3)])
    assert pickle.loads(pickle.dumps(r)) == r and copy.deepcopy(r) == r
    assert {r: 1}[ParamRange(ranges=[Range(2, 6), Range(0, 3)])] == 1
    assert r.size == 12 and r.to_shape() == (4, 3) and not r.is_normalized
    assert r.normalize([2, 0]) == ParamRange(param_shape=(4, 3))
    with pytest.raises(AttributeError):
        r.dims = 3
    with pytest.raises(Exception):
        Range(0, 4).start = 1
    assert Range(3, 3).chunk(2) == [Range(3, 3), Range(3, 3)]
    assert Range(0, 4) != (0, 4)
