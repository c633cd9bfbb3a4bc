"""A decoder layer's NF4 expansions issued as one launch (claudemaxing_amd/expand.py) against
one launch per weight: a 2-layer Qwen2.5-1.5B-shaped training step (1276 packed tokens, LoRA
dropout on with the same draws in both runs, so q/k/v take the fused NF4QKV block as in the
training step) gives the same loss and LoRA gradients bit for bit, each layer expands its o,
gate, up and down weights in one launch forward and one backward, and no single-weight
expansion is left."""

import pytest
import torch

from claudemaxing_amd import _lib, expand, qlora_step
from tests.conftest import banner

pytestmark = pytest.mark.gpu


def _loss_and_grads(model, batch):
    model.zero_grad(set_to_none=True)
    model.__dict__[qlora_step._REQUEST_ATTR] = True
    with torch.autocast("cuda", dtype=torch.float16):
        out = model(**batch, use_cache=False)
    model.__dict__.pop(qlora_step._REQUEST_ATTR, None)
    out.loss.backward()
    grads = {n: p.grad.detach().clone() for n, p in model.named_parameters() if p.requires_grad}
    return out.loss.detach().clone(), grads


def _bits(a, b, what):
    assert a.dtype == b.dtype and a.shape == b.shape, what
    assert torch.equal(a.view(torch.int32) if a.dtype == torch.float32 else a,
                       b.view(torch.int32) if b.dtype == torch.float32 else b), what


def test_grouped_expansions_equal_single_ones(dev, monkeypatch):
    banner("grouped NF4 expansions: 2-layer step, grouped vs one launch per weight")
    model = qlora_step.build_model(dev, seed=0, num_hidden_layers=2)
    g = torch.Generator(device=dev).manual_seed(1)
    for n, p in model.named_parameters():
        if "lora_B" in n:
            p.data = torch.randn(p.shape, generator=g, device=dev) * 0.02
    batch, _ = qlora_step.make_batch(dev, seed=0)
    calls = []
    real = _lib.call

    def counting(name, *args):
        if name.startswith("cm_nf4_dequant"):
            calls.append(name)
        return real(name, *args)

    monkeypatch.setattr(_lib, "call", counting)
    torch.manual_seed(5)
    loss1, grads1 = _loss_and_grads(model, batch)
    torch.cuda.synchronize()
    # per layer: the forward's group (o, gate, up, down) and the backward's
    assert calls == ["cm_nf4_dequant_group"] * 4, calls
    assert not expand._READY.get(dev.index), "expansions left over after the step"

    calls.clear()
    monkeypatch.setattr(expand, "expand_layer", lambda layer, hidden: None)
    monkeypatch.setattr(expand, "backward_group", lambda packed, dtype: None)
    torch.manual_seed(5)
    loss2, grads2 = _loss_and_grads(model, batch)
    torch.cuda.synchronize()
    # without the layer's grouping: o and down one launch each way, gate + up (the MLP's merged
    # weight) one two-weight launch each way
    assert calls.count("cm_nf4_dequant") == 8, calls
    assert calls.count("cm_nf4_dequant_group") == 4, calls
    _bits(loss1, loss2, "loss")
    assert grads1.keys() == grads2.keys() and len(grads1) == 8
    for n in grads1:
        _bits(grads1[n], grads2[n], n)
