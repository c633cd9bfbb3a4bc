"""The decoder layer's residual adds inside its RMSNorms: cm_rmsnorm_add_fwd / cm_rmsnorm_bwd_res
through AddNorm and NormPass, and the patched Qwen2DecoderLayer. Each output and gradient must be
the bits of the unfused computation with the same norm kernels -- torch's fp32 add, autograd's
sum of a tensor's two gradients, torch's fp16 cast of that sum -- since every add is the same
single fp32 rounding. Shapes cover the full-row kernels (hidden 1536 and 2048) and the general
kernels with the separate add / gradient kernels (896, 3584, 100 columns, and a weight with
tiny-|w| columns, which the full-row path does not take)."""

import pytest
import torch

from claudemaxing_amd import qlora_step
from claudemaxing_amd.rmsnorm import (MIN_ABS_WEIGHT, add_norm, fp16_grad_copy_of, norm_pass,
                                      rmsnorm)
from tests.conftest import banner

pytestmark = pytest.mark.gpu

EPS = 1e-6
SHAPES = [(1193, 1536), (64, 2048), (37, 896), (50, 3584), (5, 100)]


def _weight(dev, cols, kind, seed):
    g = torch.Generator(device="cpu").manual_seed(seed)
    w = 1.0 + 0.1 * torch.randn(cols, generator=g)
    if kind == "tiny":  # three columns below the tiny-|w| threshold
        w[[0, cols // 2, cols - 1]] = MIN_ABS_WEIGHT / 4
    if kind == "fp16":
        return w.half().to(dev)
    w = w.to(dev)
    return w.requires_grad_(kind == "trainable")


def _same(a, b, what):
    assert a.dtype == b.dtype and a.shape == b.shape, what
    assert torch.equal(a, b), f"{what}: max diff {(a.float() - b.float()).abs().max().item():.3e}"


@pytest.mark.parametrize("rows,cols", SHAPES)
@pytest.mark.parametrize("x_dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("kind", ["frozen", "trainable", "tiny", "fp16"])
def test_add_norm_equals_unfused(dev, rows, cols, x_dtype, kind):
    banner(f"add_norm: [{rows},{cols}] x {x_dtype} weight {kind}")
    g = torch.Generator(device="cpu").manual_seed(rows * 7 + cols)
    r = torch.randn(rows, cols, generator=g).to(dev).requires_grad_(True)
    x = (2 * torch.randn(rows, cols, generator=g)).to(dev, x_dtype).requires_grad_(True)
    w = _weight(dev, cols, kind, cols)
    gy = torch.randn(rows, cols, generator=g).to(dev)
    gh = torch.randn(rows, cols, generator=g).to(dev)
    wants = (r, x, w) if w.requires_grad else (r, x)

    y1, h1 = add_norm(r, x, w, EPS)
    d1 = torch.autograd.grad((y1, h1), wants, (gy, gh))
    h2 = r + x
    y2 = rmsnorm(h2, w, EPS)
    d2 = torch.autograd.grad((y2, h2), wants, (gy, gh))
    torch.cuda.synchronize()
    _same(h1, h2, "h")
    _same(y1, y2, "y")
    for a, b, name in zip(d1, d2, ("d residual", "dx", "dw")):
        _same(a, b, name)


def test_add_norm_fp16_gradient_copy(dev):
    """The fp32 input gradient's fp16 copy is its .to(fp16), handed out once and only for it."""
    banner("add_norm: fp16 copy of the input gradient")
    g = torch.Generator(device="cpu").manual_seed(5)
    r = torch.randn(300, 1536, generator=g).to(dev).requires_grad_(True)
    x = torch.randn(300, 1536, generator=g).to(dev).requires_grad_(True)
    w = _weight(dev, 1536, "frozen", 1)
    y, h = add_norm(r, x, w, EPS)
    dr, dx = torch.autograd.grad((y, h), (r, x), (torch.randn_like(y), torch.randn_like(h)))
    assert fp16_grad_copy_of(dx.clone()) is None  # other bytes
    copy = fp16_grad_copy_of(dx)
    assert copy is not None and copy.dtype == torch.float16
    _same(copy, dx.to(torch.float16), "fp16 copy")
    assert fp16_grad_copy_of(dx) is None  # handed out once


@pytest.mark.parametrize("rows,cols", [(1193, 1536), (37, 896), (50, 3584)])
@pytest.mark.parametrize("x_dtype", [torch.float32, torch.float16])
@pytest.mark.parametrize("kind", ["frozen", "trainable", "tiny"])
def test_norm_pass_equals_unfused(dev, rows, cols, x_dtype, kind):
    banner(f"norm_pass: [{rows},{cols}] x {x_dtype} weight {kind}")
    g = torch.Generator(device="cpu").manual_seed(rows + cols)
    x = torch.randn(rows, cols, generator=g).to(dev, x_dtype).requires_grad_(True)
    w = _weight(dev, cols, kind, 3)
    gy = torch.randn(rows, cols, generator=g).to(dev)
    gp = torch.randn(rows, cols, generator=g).to(dev, x_dtype)
    wants = (x, w) if w.requires_grad else (x,)
    y1, p1 = norm_pass(x, w, EPS)
    d1 = torch.autograd.grad((y1, p1), wants, (gy, gp))
    y2 = rmsnorm(x, w, EPS)
    d2 = torch.autograd.grad((y2, x.view_as(x)), wants, (gy, gp))
    torch.cuda.synchronize()
    _same(y1, y2, "y")
    assert p1.data_ptr() == x.data_ptr()
    for a, b, name in zip(d1, d2, ("dx", "dw")):
        _same(a, b, name)
    # an unused bypass: the norm's gradient alone
    (d3,) = torch.autograd.grad(norm_pass(x, w, EPS)[0], (x,), gy)
    (d4,) = torch.autograd.grad(rmsnorm(x, w, EPS), (x,), gy)
    _same(d3, d4, "dx without the bypass")


def _loss_and_grads(model, batch):
    model.zero_grad(set_to_none=True)
    model.__dict__[qlora_step._REQUEST_ATTR] = True
    with torch.autocast("cuda", dtype=torch.float16):
        out = model(**batch, use_cache=False)
    model.__dict__.pop(qlora_step._REQUEST_ATTR, None)
    out.loss.backward()
    grads = {n: p.grad.detach().clone() for n, p in model.named_parameters() if p.requires_grad}
    return out.loss.detach().clone(), grads


def test_patched_layer_equals_unfused_step(dev, monkeypatch):
    """A fused training forward + backward of a 2-layer Qwen2.5-1.5B-shaped model (dropout off)
    with and without the decoder-layer patch: the same loss and LoRA gradients, bit for bit; the
    patched run took the fused norms in both layers."""
    banner("decoder residual patch: 2-layer step, patched vs unpatched layer")
    from transformers.models.qwen2 import modeling_qwen2 as mq

    from claudemaxing_amd import decoder as D

    calls = []
    for name in ("norm_pass", "add_norm"):
        fn = getattr(D, name)
        monkeypatch.setattr(D, name, lambda *a, _fn=fn, _n=name: (calls.append(_n), _fn(*a))[1])

    model = qlora_step.build_model(dev, seed=0, dropout=0.0, num_hidden_layers=2)
    g = torch.Generator(device=dev).manual_seed(1)
    for n, p in model.named_parameters():
        if "lora_B" in n:
            p.data = torch.randn(p.shape, generator=g, device=dev) * 0.02
    batch, _ = qlora_step.make_batch(dev, seed=3)
    patched = mq.Qwen2DecoderLayer.forward
    assert getattr(patched, "_cm_patch", None) == "decoder_residual"
    from claudemaxing_amd import gemm

    adds = []
    real = gemm.gemm_f32

    def counting(*pairs, out=None, residual=None):
        adds.append(residual is not None)
        return real(*pairs, out=out, residual=residual)

    monkeypatch.setattr(gemm, "gemm_f32", counting)
    from claudemaxing_amd import nf4_linear
    monkeypatch.setattr(nf4_linear, "gemm_f32", counting)
    loss1, grads1 = _loss_and_grads(model, batch)
    assert calls == ["norm_pass", "add_norm"] * 2
    assert adds.count(True) == 2  # each layer's last residual added by its down projection
    mq.Qwen2DecoderLayer.forward = patched._original
    try:
        loss2, grads2 = _loss_and_grads(model, batch)
    finally:
        mq.Qwen2DecoderLayer.forward = patched
    torch.cuda.synchronize()
    _same(loss1, loss2, "loss")
    assert grads1.keys() == grads2.keys() and len(grads1) == 8
    for n in grads1:
        _same(grads1[n], grads2[n], n)


def test_fused_rope_step_equals_separate_rope(dev, monkeypatch):
    """The training step with the rotary embedding inside the native attention and with RoPE's
    own launches (qkv.FUSE_ROPE off): the same loss and LoRA gradients, bit for bit; the fused
    run took the fused attention in both layers."""
    banner("fused rope attention: 2-layer step, fused vs separate RoPE")
    from claudemaxing_amd import attention as A
    from claudemaxing_amd import qkv

    # LoRA dropout on (the fused q/k/v block's layout), the same draws in both runs
    model = qlora_step.build_model(dev, seed=0, num_hidden_layers=2)
    g = torch.Generator(device=dev).manual_seed(1)
    for n, p in model.named_parameters():
        if "lora_B" in n:
            p.data = torch.randn(p.shape, generator=g, device=dev) * 0.02
    batch, _ = qlora_step.make_batch(dev, seed=3)
    fused = []
    real = A.packed_causal_attention

    def counting(*args, **kwargs):
        fused.append(kwargs.get("cos") is not None)
        return real(*args, **kwargs)

    monkeypatch.setattr(A, "packed_causal_attention", counting)
    monkeypatch.setattr(qkv, "FUSE_ROPE", True)
    torch.manual_seed(5)
    loss1, grads1 = _loss_and_grads(model, batch)
    assert fused == [True, True], fused
    monkeypatch.setattr(qkv, "FUSE_ROPE", False)
    fused.clear()
    torch.manual_seed(5)
    loss2, grads2 = _loss_and_grads(model, batch)
    assert fused == [False, False], fused
    torch.cuda.synchronize()
    _same(loss1, loss2, "loss")
    for n in grads1:
        _same(grads1[n], grads2[n], n)
