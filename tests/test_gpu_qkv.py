"""NF4QKV (the q/k/v projections as one NF4-fused GEMM each way) against the three separate
layers it replaces (LoRALinear over NF4Linear for q and v, NF4Linear for k), both held against an
fp32 evaluation with the same dropout masks."""

import types

import pytest
import torch

from claudemaxing_amd.lora import LoRALinear
from claudemaxing_amd.nf4_linear import NF4Linear
from claudemaxing_amd.qkv import NF4QKV, _fused_layout, fused_qkv
from tests.conftest import banner
from tests.helpers import assert_close
from tests.test_gpu_nf4 import oracle_of

pytestmark = pytest.mark.gpu


def make_block(dev, h=1536, nq=1536, nkv=256, seed=0):
    g = torch.Generator().manual_seed(seed)

    def nf4(n):
        w = torch.randn(n, h, generator=g) * 0.02
        b = torch.randn(n, generator=g) * 0.1
        return NF4Linear.from_weight(w, bias=b)

    q, k, v = LoRALinear(nf4(nq)), nf4(nkv), LoRALinear(nf4(nkv))
    for lo in (q, v):  # a trained adapter: B nonzero, so both adapter products count
        with torch.no_grad():
            lo.lora_A.weight.copy_(torch.randn(lo.lora_A.weight.shape, generator=g) * 0.05)
            lo.lora_B.weight.copy_(torch.randn(lo.lora_B.weight.shape, generator=g) * 0.05)
    block = types.SimpleNamespace(q_proj=q.to(dev).train(), k_proj=k.to(dev),
                                  v_proj=v.to(dev).train())
    return block


def run(block, x, grads, fused, seed):
    torch.manual_seed(seed)
    xx = x.detach().clone().requires_grad_(True)
    with torch.autocast("cuda", dtype=torch.float16):
        if fused:
            q, k, v = fused_qkv(block, xx)
        else:
            q, k, v = block.q_proj(xx), block.k_proj(xx), block.v_proj(xx)
    loss = sum((o.float() * gr).sum() for o, gr in zip((q, k, v), grads))
    params = [block.q_proj.lora_A.weight, block.q_proj.lora_B.weight,
              block.v_proj.lora_A.weight, block.v_proj.lora_B.weight]
    for p in params:
        p.grad = None
    loss.backward()
    return [q.float(), k.float(), v.float(), xx.grad] + [p.grad.clone() for p in params]


def reference(block, x, grads, seed):
    """fp32 evaluation with the same dropout masks (the same generator draws, in q, v order),
    the fp16-rounded input and the NF4 weights expanded by the oracle."""
    torch.manual_seed(seed)
    masks = [torch.native_dropout(x, block.q_proj.p, True)[1] for _ in range(2)]
    xx = x.detach().half().float().requires_grad_(True)
    outs, params = [], []
    for layer, mask in ((block.q_proj, masks[0]), (block.k_proj, None), (block.v_proj, masks[1])):
        base = layer.base_layer if mask is not None else layer
        w = oracle_of(base.packed.cpu(), base.quant_state.to("cpu"), torch.float16).float()
        y = xx @ w.to(x.device).t() + base.bias.half().float()
        if mask is not None:
            a = layer.lora_A.weight.detach().clone().requires_grad_(True)
            b = layer.lora_B.weight.detach().clone().requires_grad_(True)
            xd = xx * mask / (1 - layer.p)
            y = y + (xd @ a.t()) @ b.t() * layer.scaling
            params += [a, b]
        outs.append(y)
    loss = sum((o * gr).sum() for o, gr in zip(outs, grads))
    loss.backward()
    return [o.detach() for o in outs] + [xx.grad] + [p.grad for p in params]


@pytest.mark.parametrize("tokens,h,nq,nkv", [(1276, 1536, 1536, 256), (37, 1536, 1536, 256),
                                             (300, 896, 896, 128), (300, 2048, 2048, 256)],
                         ids=["1.5B-1276", "1.5B-37", "0.5B-300", "3B-300"])
def test_fused_qkv_matches_separate_layers(tokens, h, nq, nkv, dev):
    banner(f"NF4QKV tokens={tokens} hidden={h} q={nq} kv={nkv}")
    block = make_block(dev, h=h, nq=nq, nkv=nkv)
    x = torch.randn(1, tokens, h, device=dev)
    assert _fused_layout(block, x.requires_grad_(True)) is False  # outside fp16 autocast
    with torch.autocast("cuda", dtype=torch.float16):
        assert _fused_layout(block, x)
    grads = [torch.randn(1, tokens, n, device=dev) for n in (nq, nkv, nkv)]
    fused = run(block, x, grads, True, 7)
    sep = run(block, x, grads, False, 7)
    ref = reference(block, x, grads, 7)
    names = ["q", "k", "v", "dx", "dA_q", "dB_q", "dA_v", "dB_v"]
    for name, f, s, r in zip(names, fused, sep, ref):
        # both within fp16 tolerance of the fp32 evaluation, the fused one no worse than 2x the
        # separate layers' error (plus a small floor for outputs the two round alike)
        assert_close(f, r, 1e-2, f"{name} fused vs fp32")
        ef = (f - r).abs().max().item()
        es = (s - r).abs().max().item()
        assert ef <= 2 * es + 2e-3 * r.abs().max().item(), (name, ef, es)
