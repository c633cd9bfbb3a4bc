"""The NF4-fused linears' host cache (no GPU): a weight's descriptor and the descriptor arrays of
a grouping are built once per weight version, and rebuilt when anything they point into
changes or the grouping holds other QuantState objects."""

import torch

from claudemaxing_amd import nf4
from claudemaxing_amd.nf4_linear import _descriptor, _weights


def _weight(seed, rows=64, cols=128):
    g = torch.Generator().manual_seed(seed)
    return nf4.quantize_nf4(torch.randn(rows, cols, generator=g) * 0.02, 64, True)


def test_descriptor_is_reused_for_the_same_weight_version():
    packed, state = _weight(0)
    d1, _ = _descriptor(packed, state)
    d2, _ = _descriptor(packed, state)
    assert d1 is d2
    state.absmax.add_(0)  # an in-place write bumps the version: the descriptor is rebuilt
    d3, _ = _descriptor(packed, state)
    assert d3 is not d1
    assert (d3.packed, d3.absmax, d3.rows, d3.cols) == (d1.packed, d1.absmax, d1.rows, d1.cols)


def test_descriptor_follows_the_tensors_it_points_into():
    packed, state = _weight(1)
    d1, _ = _descriptor(packed, state)
    other = packed.clone()
    d2, _ = _descriptor(other, state)
    assert d2.packed == other.data_ptr() != d1.packed
    state.absmax = state.absmax.clone()
    d3, _ = _descriptor(other, state)
    assert d3.absmax == state.absmax.data_ptr() != d1.absmax


def test_weight_arrays_are_per_grouping_and_per_state_object():
    (p0, s0), (p1, s1) = _weight(2), _weight(3)
    a = _weights([(p0, s0), (p1, s1)])
    assert _weights([(p0, s0), (p1, s1)]) is a
    b = _weights([(p0, s0)])
    assert b is not a and len(b[0]) == 1 and len(a[0]) == 2
    assert [d.packed for d in a[0]] == [p0.data_ptr(), p1.data_ptr()]
    # a different QuantState object over the same tensors is a different weight for the cache
    s1b = nf4.QuantState(**{f: getattr(s1, f) for f in s1.__dataclass_fields__})
    c = _weights([(p0, s0), (p1, s1b)])
    assert c is not a
    assert [d.packed for d in c[0]] == [d.packed for d in a[0]]
