"""The grouped-expansion registry of claudemaxing_amd/expand.py on the host (no GPU): an
expansion left for a weight is handed out once, only in fp16, and dropped with its device's
entries; a weight with no recorded group gets no backward group; a layer without NF4
projections is left alone."""

import torch

from claudemaxing_amd import expand


def test_take_hands_an_expansion_out_once():
    packed = torch.zeros(8, dtype=torch.uint8)
    w = torch.ones(2, 2, dtype=torch.float16)
    expand._READY[packed.device.index] = {packed.data_ptr(): w}
    try:
        assert expand.take(packed, torch.float32) is None  # another dtype: not this expansion
        assert expand.take(packed, torch.float16) is w
        assert expand.take(packed, torch.float16) is None  # once
    finally:
        expand.drop(packed.device)


def test_take_pair_and_drop():
    gate, up = torch.zeros(8, dtype=torch.uint8), torch.zeros(8, dtype=torch.uint8)

    class Proj:
        def __init__(self, packed):
            self.packed = packed

    w2 = torch.ones(4, 2, dtype=torch.float16)
    key = ("pair", gate.data_ptr(), up.data_ptr())
    expand._READY[gate.device.index] = {key: w2}
    assert expand.take_pair(Proj(up), Proj(gate)) is None  # the order matters: [Wg; Wu]
    expand.drop(gate.device)
    assert expand.take_pair(Proj(gate), Proj(up)) is None  # dropped
    expand._READY[gate.device.index] = {key: w2}
    assert expand.take_pair(Proj(gate), Proj(up)) is w2
    expand.drop(gate.device)


def test_no_group_without_a_recorded_layer():
    packed = torch.zeros(8, dtype=torch.uint8)
    assert expand.backward_group(packed, torch.float16) is None


def test_layer_without_nf4_projections_is_left_alone():
    layer = torch.nn.Module()
    layer.self_attn = torch.nn.Module()
    layer.self_attn.o_proj = torch.nn.Linear(4, 4)
    layer.mlp = torch.nn.Module()
    for name in ("gate_proj", "up_proj", "down_proj"):
        setattr(layer.mlp, name, torch.nn.Linear(4, 4))
    hidden = torch.zeros(1, 3, 4)
    expand.expand_layer(layer, hidden)
    assert not expand._READY.get(hidden.device.index)
