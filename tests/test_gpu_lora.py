"""LoRA mask pack/unpack on the GPU against the oracle (bit-exact), and LoRABranch against the
plain peft computation under fp16 autocast."""

import numpy as np
import pytest
import torch

from claudemaxing_amd import lora as L
from oracle import lora as O
from tests.conftest import banner
from tests.helpers import assert_bits_equal

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n", [8, 3 * 37 * 64, 1152 * 1536, 1000 * 8 + 8])
@pytest.mark.parametrize("x_dtype", [torch.float32, torch.float16])
def test_pack_unpack_match_oracle(n, x_dtype, dev):
    banner(f"lora pack/unpack n={n} {x_dtype}")
    g = torch.Generator().manual_seed(n)
    x = torch.randn(n, generator=g).to(x_dtype)
    keep = torch.rand(n, generator=g) > 0.05
    g16 = torch.randn(n, generator=g).to(torch.float16)
    scale = 1.0 / (1.0 - 0.05)
    xd, bits = L._pack(x.to(dev), keep.to(dev), scale)
    rxd, rbits = O.pack(x.numpy(), keep.numpy(), scale)
    assert_bits_equal(xd, torch.from_numpy(rxd), "xd")
    assert torch.equal(bits.cpu(), torch.from_numpy(rbits))
    x16 = x.to(torch.float16)
    xd2, dx = L._unpack(x16.to(dev), bits, g16.to(dev), scale, torch.float32)
    uxd, udx = O.unpack(x16.numpy(), rbits, g16.numpy(), scale, np.float32)
    assert_bits_equal(xd2, torch.from_numpy(uxd), "unpack xd")
    assert_bits_equal(dx, torch.from_numpy(udx), "unpack dx")


def test_known_answer_closed_forms(dev):
    """tests_local/test_lora.py:24-33."""
    banner("lora known answer")
    g = torch.Generator().manual_seed(0)
    x16 = torch.randn(3, 37, 64, generator=g).half().to(dev)
    mask = (torch.rand(3, 37, 64, generator=g) > 0.3).to(dev)
    xd, bits = L._pack(x16, mask, 1.25)
    assert torch.equal(xd, torch.where(mask, (x16.float() * 1.25).half(), 0))
    gg = torch.randn(x16.shape, generator=g).half().to(dev)
    xd2, dx = L._unpack(x16, bits, gg, 1.25, torch.float32)
    assert torch.equal(xd2, xd)
    assert torch.equal(dx, torch.where(mask, gg.float() * 1.25, 0))


def test_lora_branch_matches_plain_computation(dev):
    banner("lora branch vs plain")
    torch.manual_seed(0)
    base = torch.nn.Linear(256, 128, bias=False).to(dev).requires_grad_(False)
    layer = L.LoRALinear(base, r=16, alpha=32, dropout=0.05).to(dev)
    with torch.no_grad():
        layer.lora_B.weight.normal_(0, 0.1)
    layer.train()
    x = torch.randn(4, 50, 256, device=dev)

    def run(use_branch):
        for p in layer.parameters():
            p.grad = None
        xx = x.clone().requires_grad_(True)
        torch.manual_seed(7)
        with torch.autocast("cuda", dtype=torch.float16):
            if use_branch:
                out = layer(xx)
            else:
                out = base(xx) + layer.lora_B(layer.lora_A(torch.nn.functional.dropout(
                    xx, 0.05, True))) * layer.scaling
        (out.float() * torch.linspace(-1, 1, out.shape[-1], device=dev)).sum().backward()
        return out.detach(), xx.grad, layer.lora_A.weight.grad.clone(), \
            layer.lora_B.weight.grad.clone()

    ref = run(False)
    ours = run(True)
    assert ours[0].dtype == ref[0].dtype
    assert torch.equal(ours[0], ref[0])  # forward bit-identical (same mask, same fp16 GEMMs)
    rel = lambda a, b: ((a.float() - b.float()).norm() / b.float().norm()).item()  # noqa: E731
    assert rel(ours[1], ref[1]) < 2e-3
    assert rel(ours[2], ref[2]) < 5e-3 and rel(ours[3], ref[3]) < 5e-3
