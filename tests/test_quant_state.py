"""bitsandbytes' serialized QuantState (claudemaxing_amd.nf4.QuantState.as_dict / from_dict)
and NF4Linear's state dict in Linear4bit's key layout, on the CPU.

bitsandbytes is absent here, so parity with its own serialized bytes is unpinned; these tests
hold the writer and the reader to the documented layout separately (a dict built by hand in
that layout loads; as_dict writes exactly those keys and JSON fields) and check the round trip
through a safetensors file, field by field."""

import json

import pytest
import torch

from claudemaxing_amd.nf4 import QuantState, quantize_nf4
from claudemaxing_amd.nf4_linear import NF4Linear


def _same_state(a, b):
    assert tuple(a.shape) == tuple(b.shape) and a.blocksize == b.blocksize
    assert a.quant_type == b.quant_type and a.dtype == b.dtype
    assert torch.equal(a.absmax, b.absmax) and torch.equal(a.code, b.code)
    assert a.nested == b.nested
    if a.nested:
        assert torch.equal(a.offset, b.offset) and a.offset.dtype == torch.float32
        assert torch.equal(a.state2.absmax, b.state2.absmax)
        assert torch.equal(a.state2.code, b.state2.code)
        assert a.state2.blocksize == b.state2.blocksize and a.state2.dtype == b.state2.dtype


def test_packed_layout_keys_and_fields():
    w = torch.randn(384, 256).half()
    _, st = quantize_nf4(w)
    d = st.as_dict(packed=True)
    assert set(d) == {"absmax", "quant_map", "nested_absmax", "nested_quant_map",
                      "quant_state.bitsandbytes__nf4"}
    blob = d["quant_state.bitsandbytes__nf4"]
    assert blob.dtype == torch.uint8 and blob.dim() == 1
    fields = json.loads(bytes(blob.tolist()).decode("utf-8"))
    assert fields == {"quant_type": "nf4", "blocksize": 64, "dtype": "float16",
                      "shape": [384, 256], "nested_blocksize": 256, "nested_dtype": "float32",
                      "nested_offset": float(st.offset)}
    assert d["absmax"].dtype == torch.uint8 and d["nested_absmax"].dtype == torch.float32
    plain = st.as_dict()
    assert plain["shape"] == (384, 256) and plain["nested_offset"] == float(st.offset)


def test_round_trip_through_safetensors(tmp_path):
    from safetensors.torch import load_file, save_file

    w = torch.randn(512, 192)
    packed, st = quantize_nf4(w)
    d = {"layer.weight": packed.clone()}
    d.update({"layer.weight." + k: v.contiguous() for k, v in st.as_dict(packed=True).items()})
    path = tmp_path / "nf4.safetensors"
    save_file(d, str(path))
    back = load_file(str(path))
    lin = NF4Linear.from_state_dict(back, prefix="layer.")
    assert torch.equal(lin.packed, packed)
    _same_state(lin.quant_state, st)


def test_hand_built_dict_loads():
    """A state in the documented layout, written without as_dict."""
    absmax8 = torch.randint(0, 256, (8,), dtype=torch.uint8)
    code = torch.linspace(-1, 1, 16)
    code2 = torch.linspace(-1, 1, 256)
    absmax2 = torch.rand(1)
    fields = {"quant_type": "nf4", "blocksize": 64, "dtype": "bfloat16", "shape": [8, 64],
              "nested_blocksize": 256, "nested_dtype": "float32", "nested_offset": 0.125}
    blob = torch.tensor(list(json.dumps(fields).encode()), dtype=torch.uint8)
    st = QuantState.from_dict({"absmax": absmax8, "quant_map": code, "nested_absmax": absmax2,
                               "nested_quant_map": code2,
                               "quant_state.bitsandbytes__nf4": blob})
    assert st.shape == torch.Size([8, 64]) and st.dtype == torch.bfloat16 and st.nested
    assert st.offset.item() == 0.125 and st.state2.blocksize == 256
    assert torch.equal(st.absmax, absmax8) and torch.equal(st.state2.code, code2)
    # not double-quantized: fp32 absmax, no nested fields
    st1 = QuantState.from_dict({"absmax": torch.rand(8), "quant_map": code, "quant_type": "nf4",
                                "blocksize": 64, "dtype": "float16", "shape": (8, 64)})
    assert not st1.nested and st1.offset is None


def test_nf4linear_state_dict_round_trip():
    w, b = torch.randn(128, 64), torch.randn(128)
    a = NF4Linear.from_weight(w, bias=b)
    sd = a.state_dict()
    assert set(sd) == {"weight", "bias", "weight.absmax", "weight.quant_map",
                       "weight.nested_absmax", "weight.nested_quant_map",
                       "weight.quant_state.bitsandbytes__nf4"}
    assert sd["weight"].shape == (128 * 64 // 2, 1)
    c = NF4Linear.from_weight(torch.zeros(128, 64), bias=torch.zeros(128))
    c.load_state_dict(sd)
    assert torch.equal(c.packed, a.packed) and torch.equal(c.bias, b)
    _same_state(c.quant_state, a.quant_state)


def test_errors():
    with pytest.raises(ValueError, match="missing"):
        QuantState.from_dict({"absmax": torch.zeros(1)})
    a = NF4Linear.from_weight(torch.randn(64, 64))
    other = NF4Linear.from_weight(torch.randn(128, 64)).state_dict()
    with pytest.raises(RuntimeError, match="shape"):
        a.load_state_dict(other)
