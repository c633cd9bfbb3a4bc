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


@pytest.mark.parametrize("dx_dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("in_off,dx_off", [(0, 0), (1, 0), (0, 1), (0, 2), (4, 4)])
def test_unpack_gradient_dtypes_and_misaligned_buffers(dx_dtype, in_off, dx_off, dev):
    """cm_lora_unpack called directly on buffers that start in_off / dx_off elements into their
    storage (2-, 4- and 8-byte offsets take the element-wise path), over whole workgroups and a
    ragged tail, for every gradient dtype."""
    from claudemaxing_amd import _lib

    n = 4096 * 3 + 8 * 37
    banner(f"lora unpack dx={dx_dtype} offsets x/g/xd {in_off} dx {dx_off}")
    g = torch.Generator().manual_seed(11 + 3 * in_off + dx_off)
    x16 = torch.randn(n, generator=g).half()
    g16 = torch.randn(n, generator=g).half()
    bits = torch.randint(0, 256, (n // 8,), generator=g, dtype=torch.uint8)
    scale = 1.0 / 0.9

    def placed(dtype, off, src=None):
        buf = torch.zeros(n + off, dtype=dtype, device=dev)[off:]
        return buf.copy_(src) if src is not None else buf

    xs, gs = placed(torch.float16, in_off, x16), placed(torch.float16, in_off, g16)
    xd, dx = placed(torch.float16, in_off), placed(dx_dtype, dx_off)
    bd = bits.to(dev)
    _lib.call("cm_lora_unpack", xs.data_ptr(), bd.data_ptr(), gs.data_ptr(), xd.data_ptr(),
              dx.data_ptr(), _lib.dtype_code(dx_dtype), n, scale, _lib.stream(xs.device))
    uxd, udx = O.unpack(x16.numpy(), bits.numpy(), g16.numpy(), scale, np.float32)
    assert_bits_equal(xd, torch.from_numpy(uxd), "unpack xd")
    # the gradient is formed in fp32 and rounded once to its dtype (round to nearest even)
    assert_bits_equal(dx, torch.from_numpy(udx).to(dx_dtype), "unpack dx")


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
