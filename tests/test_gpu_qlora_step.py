"""The QLoRA step on the GPU: it runs and trains, and its fused path (packed tokens, the kernel
set's RMSNorm/RoPE/SwiGLU/head) gives the loss and LoRA gradients of the stock transformers
model on the same weights (padded batch, full fp16 logits, transformers' causal-LM loss).
Tolerances are the fp16-level ones of the kernel tests: the two paths round differently at every
layer (tol 2e-3 on the loss, 2e-2 relative to the largest entry on the gradients)."""

import pytest
import torch

from claudemaxing_amd import qlora_step
from tests.conftest import banner

TWO_LAYERS = dict(num_hidden_layers=2)


@pytest.mark.gpu
def test_step_runs_and_trains(dev):
    banner("qlora step: 2 layers, 3 steps")
    model = qlora_step.build_model(dev, seed=0, **TWO_LAYERS)
    batch, _ = qlora_step.make_batch(dev, seed=0)
    opt = qlora_step.make_optimizer(model)
    scaler = torch.amp.GradScaler("cuda")
    b_before = [p.detach().clone() for n, p in model.named_parameters() if "lora_B" in n]
    losses = [float(qlora_step.train_step(model, opt, scaler, batch)) for _ in range(3)]
    torch.cuda.synchronize()
    assert all(torch.isfinite(torch.tensor(losses)))
    assert 9.0 < losses[0] < 14.0  # ~ln(151936) for a random model
    b_after = [p.detach() for n, p in model.named_parameters() if "lora_B" in n]
    assert any(not torch.equal(a, b) for a, b in zip(b_before, b_after))


def _loss_and_grads(model, batch, fused, autocast=True):
    model.zero_grad(set_to_none=True)
    if fused:
        model.__dict__[qlora_step._REQUEST_ATTR] = True
    with torch.autocast("cuda", dtype=torch.float16, enabled=autocast):
        out = model(**batch, use_cache=False)
    model.__dict__.pop(qlora_step._REQUEST_ATTR, None)
    out.loss.backward()
    grads = {n: p.grad.detach().float().clone() for n, p in model.named_parameters()
             if p.requires_grad}
    return float(out.loss.detach()), grads


@pytest.mark.gpu
def test_fused_step_matches_stock(dev):
    """Both fp16 paths against the fp32 evaluation of the same model (stock code, no autocast,
    NF4 weights expanded to fp32): the fused path must be about as close as the stock fp16 path
    (within 2x its error, or within tol)."""
    banner("qlora step: fused vs stock transformers vs fp32, 2 layers")
    from claudemaxing_amd.nf4_linear import NF4Linear

    model = qlora_step.build_model(dev, seed=0, dropout=0.0, **TWO_LAYERS)
    g = torch.Generator(device=dev).manual_seed(1)
    for n, p in model.named_parameters():
        if "lora_B" in n:  # nonzero, so the LoRA branch changes the forward
            p.data = torch.randn(p.shape, generator=g, device=dev) * 0.02
    batch, _ = qlora_step.make_batch(dev, seed=3)
    loss_f, grads_f = _loss_and_grads(model, batch, True)
    with qlora_step.unpatched():
        loss_s, grads_s = _loss_and_grads(model, batch, False)
        nf4 = [m for m in model.modules() if isinstance(m, NF4Linear)]
        for m in nf4:
            m.compute_dtype = torch.float32
        # the fused step stored the tied weight in fp16 (lossless); fp32 products need fp32
        emb = model.get_input_embeddings()
        assert emb.weight.dtype == torch.float16
        w16 = emb.weight.data
        emb.weight.data = w16.float()
        try:
            loss_r, grads_r = _loss_and_grads(model, batch, False, autocast=False)
        finally:
            emb.weight.data = w16
            for m in nf4:
                m.compute_dtype = torch.float16
    report = [f"loss: fp32 {loss_r:.6f}, stock fp16 {loss_s:.6f}, fused fp16 {loss_f:.6f}"]
    assert grads_f.keys() == grads_s.keys() == grads_r.keys() and len(grads_r) == 8
    worst = []
    for n, ref in grads_r.items():
        scale = float(ref.abs().max())
        assert scale > 0, n
        e_s = float((grads_s[n] - ref).abs().max()) / scale
        e_f = float((grads_f[n] - ref).abs().max()) / scale
        report.append(f"{n}: max|g| {scale:.3e}  stock fp16 err {e_s:.2e}  fused err {e_f:.2e}")
        worst.append((n, e_f, e_s))
    print("\n".join(report), flush=True)
    d_s, d_f = abs(loss_s - loss_r), abs(loss_f - loss_r)
    assert d_f <= max(2e-3 * abs(loss_r), 2 * d_s), report[0]
    for n, e_f, e_s in worst:
        assert e_f <= max(2e-2, 2 * e_s), (n, e_f, e_s)


@pytest.mark.gpu
def test_graphed_step_matches_eager(dev):
    """Three steps replayed from the HIP graph against three eager steps of an identical model
    (dropout off, so both draw no random numbers): the same loss and the same LoRA weights after
    every step. The optimizer step between replays is eager work, and each step ends with a
    device sync, as the graph tests of this platform require."""
    banner("qlora step: graphed vs eager, 2 layers, 3 steps")
    runs = []
    for graphed in (False, True):
        model = qlora_step.build_model(dev, seed=0, dropout=0.0, **TWO_LAYERS)
        batch, _ = qlora_step.make_batch(dev, seed=4)
        opt = qlora_step.make_optimizer(model)
        scaler = torch.amp.GradScaler("cuda")
        if graphed:
            gstep = qlora_step.GraphedStep(model, opt, scaler, batch)
            step = gstep.step
        else:
            def step():
                return qlora_step.train_step(model, opt, scaler, batch)
        trace = []
        for _ in range(3):
            loss = float(step())
            torch.cuda.synchronize()
            trace.append((loss, [p.detach().clone() for p in qlora_step.lora_parameters(model)]))
        runs.append(trace)
    for (le, pe), (lg, pg) in zip(*runs):
        assert le == lg, (le, lg)
        for a, b in zip(pe, pg):
            assert torch.equal(a, b)


@pytest.mark.gpu
def test_graphed_step_trains_with_dropout(dev):
    banner("qlora step: graphed with dropout, 2 layers, 4 steps")
    model = qlora_step.build_model(dev, seed=0, **TWO_LAYERS)
    batch, _ = qlora_step.make_batch(dev, seed=0)
    opt = qlora_step.make_optimizer(model)
    gstep = qlora_step.GraphedStep(model, opt, torch.amp.GradScaler("cuda"), batch)
    b0 = [p.detach().clone() for n, p in model.named_parameters() if "lora_B" in n]
    losses = [float(gstep.step()) for _ in range(4)]
    torch.cuda.synchronize()
    assert all(9.0 < x < 14.0 for x in losses)
    assert len(set(losses)) > 1  # fresh dropout masks and updated weights every replay
    b1 = [p.detach() for n, p in model.named_parameters() if "lora_B" in n]
    assert any(not torch.equal(a, b) for a, b in zip(b0, b1))
    gstep.load(qlora_step.make_batch(dev, seed=0)[0])  # same packed shape: accepted
    with pytest.raises(ValueError):
        gstep.load(qlora_step.make_batch(dev, seed=1)[0])  # other lengths: a new capture
