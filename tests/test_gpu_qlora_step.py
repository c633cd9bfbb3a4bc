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


# Two-layer models of the Qwen2.5 shapes: 1.5B (the benchmark's), 0.5B, 3B, and 7B, whose head
# weight is not tied to the embedding.
SHAPES = {
    "1.5B": TWO_LAYERS,
    "0.5B": dict(TWO_LAYERS, hidden_size=896, intermediate_size=4864, num_attention_heads=14,
                 num_key_value_heads=2),
    "3B": dict(TWO_LAYERS, hidden_size=2048, intermediate_size=11008, num_attention_heads=16,
               num_key_value_heads=2),
    "7B": dict(TWO_LAYERS, hidden_size=3584, intermediate_size=18944, num_attention_heads=28,
               num_key_value_heads=4, tie_word_embeddings=False),
}


@pytest.mark.gpu
@pytest.mark.parametrize("shape", list(SHAPES))
def test_fused_step_matches_stock(dev, shape):
    """Both fp16 paths against the fp32 evaluation of the same model (stock code, no autocast,
    NF4 weights expanded to fp32): the fused path must be about as close as the stock fp16 path
    (within 2x its error, or within tol)."""
    banner(f"qlora step: fused vs stock transformers vs fp32, 2 layers, Qwen2.5-{shape} shape")
    from claudemaxing_amd.nf4_linear import NF4Linear

    model = qlora_step.build_model(dev, seed=0, dropout=0.0, **SHAPES[shape])
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
        tied = model.config.tie_word_embeddings
        assert emb.weight.dtype == (torch.float16 if tied else torch.float32)
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
def test_graph_captures_do_not_accumulate_memory(dev):
    """A new GraphedStep per batch (packed shapes change every step in SFT) keeps the HBM in use
    flat: every capture warms up and records on the one side stream of the device, so torch's
    per-stream BLAS workspaces are made once, and each graph's pool is released with the graph.
    Five captures after the first two may not raise the allocated bytes by more than 4 MiB."""
    banner("qlora step: 7 graph captures over distinct batches, 2 layers")
    model = qlora_step.build_model(dev, seed=0, **TWO_LAYERS)
    opt = qlora_step.make_optimizer(model)
    scaler = torch.amp.GradScaler("cuda")
    held = []
    for i in range(7):
        batch, _ = qlora_step.make_batch(dev, seed=100 + i)
        float(qlora_step.GraphedStep(model, opt, scaler, batch, warmup=1).step())
        torch.cuda.synchronize()
        held.append(torch.cuda.memory_allocated())
    assert held[-1] - held[1] <= 4 << 20, [h / 2 ** 20 for h in held]


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


@pytest.mark.gpu
def test_full_depth_step_trains(dev):
    """Config 5 at its stated size: 28 layers of the Qwen2.5-1.5B shape, NF4 base weights, LoRA
    r16 / alpha 32 on q/v, fp16 autocast + GradScaler + AdamW, batch 4 with lengths U[64, 512]
    packed. Over 4 steps on one batch (dropout off, so the steps differ only by the updates) the
    loss starts near ln(151936) and goes down, the LoRA weights move, TRL's metrics are sane, and
    the peak HBM is reported."""
    import math

    banner("qlora step: 28 layers, 4 steps")
    model = qlora_step.build_model(dev, seed=0, dropout=0.0)
    assert len(model.model.layers) == 28
    batch, lengths = qlora_step.make_batch(dev, seed=0)
    opt = qlora_step.make_optimizer(model)
    scaler = torch.amp.GradScaler("cuda")
    b_before = [p.detach().clone() for n, p in model.named_parameters() if "lora_B" in n]
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats()
    losses, metrics = [], []
    for _ in range(4):
        m = {}
        losses.append(float(qlora_step.train_step(model, opt, scaler, batch, metrics=m)))
        metrics.append(m)
    torch.cuda.synchronize()
    peak = torch.cuda.max_memory_allocated() / 2 ** 30
    print(f"28 layers, {int(lengths.sum())} tokens: losses {losses}; peak allocated "
          f"{peak:.2f} GiB, reserved {torch.cuda.max_memory_reserved() / 2 ** 30:.2f} GiB; "
          f"metrics {metrics[0]}", flush=True)
    assert all(math.isfinite(x) for x in losses)
    assert abs(losses[0] - math.log(151936)) < 1.5
    assert losses[-1] < losses[0]
    b_after = [p.detach() for n, p in model.named_parameters() if "lora_B" in n]
    assert len(b_after) == 56 and any(not torch.equal(a, b) for a, b in zip(b_before, b_after))
    for m in metrics:
        assert m["num_tokens"] == int(lengths.sum())
        assert 0 < m["entropy"] <= math.log(151936) + 1e-3
        assert 0.0 <= m["mean_token_accuracy"] <= 1.0
    assert peak < 16.0


def _predicted_batch(model, dev, seed):
    """A config-5 batch whose labels are mostly the model's own greedy prediction of the next
    token (70%, the rest random), so that token accuracy and entropy are not trivial numbers
    (tests_local/test_lm_head_trainer.py builds its rows the same way)."""
    batch, _ = qlora_step.make_batch(dev, seed=seed)
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.float16), qlora_step.unpatched():
        logits = model(input_ids=batch["input_ids"], attention_mask=batch["attention_mask"],
                       use_cache=False).logits
    pred = logits.argmax(-1)
    g = torch.Generator(device=dev).manual_seed(100 + seed)
    take = torch.rand(pred.shape, generator=g, device=dev) < 0.7
    labels = batch["labels"].clone()
    labels[:, 1:] = torch.where(take[:, :-1], pred[:, :-1], labels[:, 1:])
    labels[batch["attention_mask"] == 0] = -100
    batch["labels"] = labels
    return batch


def _stock_step(model, opt, scaler, batch):
    """The unpatched transformers step with TRL's metrics evaluated on its fp16 logits."""
    import torch.nn.functional as F

    with torch.autocast("cuda", dtype=torch.float16):
        out = model(**batch, use_cache=False)
    with torch.no_grad():
        z = out.logits.float()
        logp = F.log_softmax(z, -1)
        ent = -(logp.exp() * logp).sum(-1)
        mask = batch["attention_mask"]
        lab = batch["labels"][:, 1:]
        hit = (z[:, :-1].argmax(-1) == lab) & (lab != -100)
        m = dict(entropy=float((ent * mask).sum() / mask.sum()), num_tokens=int(mask.sum()),
                 mean_token_accuracy=float(hit.sum() / (lab != -100).sum()))
        del z, logp, ent
    scaler.scale(out.loss).backward()
    scaler.step(opt)
    scaler.update()
    opt.zero_grad(set_to_none=True)
    return float(out.loss.detach()), m


@pytest.mark.gpu
def test_training_curve_matches_stock(dev):
    """8 training steps on 8 different batches, fused path against the stock transformers path
    from identical weights, by the reference's end-to-end rules (tests_local/
    test_lm_head_trainer.py:164-188): num_tokens identical every step; first-step loss within
    1%; mean relative gap of the loss, entropy and token-accuracy curves within 3%. Dropout is off
    so that both runs see the same computation (the two paths draw their masks differently)."""
    banner("qlora step: 8-step curve, fused vs stock, 2 layers")
    runs = []
    for fused in (True, False):
        model = qlora_step.build_model(dev, seed=0, dropout=0.0, **TWO_LAYERS)
        if fused:
            batches = [_predicted_batch(model, dev, s) for s in range(8)]
        opt = qlora_step.make_optimizer(model)
        scaler = torch.amp.GradScaler("cuda")
        curve = []
        for b in batches:
            if fused:
                m = {}
                loss = float(qlora_step.train_step(model, opt, scaler, b, metrics=m))
            else:
                with qlora_step.unpatched():
                    loss, m = _stock_step(model, opt, scaler, b)
            curve.append(dict(loss=loss, **m))
        torch.cuda.synchronize()
        runs.append(curve)
        del model, opt
        torch.cuda.empty_cache()
    fused_c, stock_c = runs

    def gap(key):
        return sum(abs(f[key] - s[key]) / max(abs(s[key]), 1e-12)
                   for f, s in zip(fused_c, stock_c)) / len(stock_c)

    for f, s in zip(fused_c, stock_c):
        print(f"  loss {s['loss']:.5f} / {f['loss']:.5f}   entropy {s['entropy']:.4f} / "
              f"{f['entropy']:.4f}   acc {s['mean_token_accuracy']:.4f} / "
              f"{f['mean_token_accuracy']:.4f}   tokens {s['num_tokens']}", flush=True)
    gaps = {k: gap(k) for k in ("loss", "entropy", "mean_token_accuracy")}
    first = abs(fused_c[0]["loss"] - stock_c[0]["loss"]) / abs(stock_c[0]["loss"])
    print(f"first-step loss gap {first:.4%}; mean gaps {gaps}", flush=True)
    assert [f["num_tokens"] for f in fused_c] == [s["num_tokens"] for s in stock_c]
    assert first <= 0.01
    assert all(v <= 0.03 for v in gaps.values()), gaps
    assert 0.2 < stock_c[0]["mean_token_accuracy"] < 0.95  # the labels are learnable, not noise


def _eager_metrics(model, batch):
    """TRL's three metrics of the eager fused forward on `batch` (packed without a bucket)."""
    from claudemaxing_amd.lm_head_loss import _STEP_ATTR, trl_metrics

    model.__dict__[qlora_step._REQUEST_ATTR] = True
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.float16):
        model(**batch, use_cache=False)
    model.__dict__.pop(qlora_step._REQUEST_ATTR, None)
    return trl_metrics(model.__dict__.pop(_STEP_ATTR), batch)


def _eager_scaled(model, batch, bucket, scale):
    """Loss and LoRA gradients of the eager fused step on `batch` (packed to `bucket`, or without
    filler when None), backpropagated at the loss scale `scale` as the GradScaler does and then
    unscaled (a power of two: exact): small fp16 gradients keep their precision, as in
    training."""
    from claudemaxing_amd.lm_head_loss import _pack_batch, _packed_forward

    model.zero_grad(set_to_none=True)
    kwargs = dict(input_ids=batch["input_ids"], attention_mask=batch["attention_mask"],
                  use_cache=False)
    packed = _pack_batch(model, kwargs, batch["labels"], bucket=bucket)
    with torch.autocast("cuda", dtype=torch.float16):
        out = _packed_forward(model, dict(use_cache=False), packed)
    (out.loss * scale).backward()
    return float(out.loss.detach()), [p.grad.detach().float() / scale
                                      for p in qlora_step.lora_parameters(model)]


@pytest.mark.gpu
def test_bucketed_graph_matches_eager_unpadded(dev):
    """One graph captured for a 256-token bucket replays five distinct batches of that bucket
    (each packed with a filler row of ignored labels up to the bucket, its rows loaded into the
    attention's device image), dropout off:
      * each replay gives the bits of the eager step on the same bucketed packing (loss and
        every LoRA gradient): loading a batch into the graph is exact;
      * against the eager step on the batch packed without filler, the loss agrees to 1e-4
        relative and the gradients to 2e-2 of their largest entry (the filler changes the token
        count, so GEMM routes, tilings and split-K slicing, and with them fp32 summation orders
        and fp16 rounding points, as between the fused and the stock step), and TRL's metrics
        agree, num_tokens exactly (the batch's own token count).
    Then batches of two other buckets run through BucketedGraphSteps (one shared pool, one
    capture per bucket)."""
    banner("qlora step: bucketed graph vs eager, 2 layers, 5 batches")
    model = qlora_step.build_model(dev, seed=0, dropout=0.0, **TWO_LAYERS)
    params = qlora_step.lora_parameters(model)
    names = [n for n, p in model.named_parameters() if p.requires_grad]
    opt = torch.optim.SGD(params, lr=0.0)  # the weights stay put between comparisons
    scaler = torch.amp.GradScaler("cuda")
    bucket, batches, total0 = 256, [], None
    for seed in range(100, 600):
        b, lengths = qlora_step.make_batch(dev, seed=seed)
        total = -(-int(lengths.sum()) // bucket) * bucket
        total0 = total0 or total
        if total == total0:
            batches.append((b, int(lengths.sum())))
        if len(batches) == 5:
            break
    assert len(batches) == 5
    gstep = qlora_step.GraphedStep(model, opt, scaler, batches[0][0], warmup=2, bucket=bucket)
    assert gstep.packed.ids.shape[1] == total0
    for i, (b, n_real) in enumerate(batches):
        if i:
            gstep.load(b)
        m = {}
        g_loss = float(gstep.step(m, b))
        torch.cuda.synchronize()
        g_grads = [p.grad.detach().float().clone() for p in params]  # unscaled by the step
        scale = float(scaler.get_scale())
        k_loss, k_grads = _eager_scaled(model, b, bucket, scale)
        assert g_loss == k_loss, (i, g_loss, k_loss)
        for name, gg, kg in zip(names, g_grads, k_grads):
            assert torch.equal(gg, kg), (i, name)
        e_loss, e_grads = _eager_scaled(model, b, None, scale)
        e_m = _eager_metrics(model, b)
        assert abs(g_loss - e_loss) <= 1e-4 * abs(e_loss), (i, g_loss, e_loss)
        for name, gg, eg in zip(names, g_grads, e_grads):
            err = float((gg - eg).abs().max())
            assert err <= 2e-2 * float(eg.abs().max()), (i, name, err)
        assert m["num_tokens"] == e_m["num_tokens"] == n_real
        assert abs(m["entropy"] - e_m["entropy"]) <= 1e-4 * abs(e_m["entropy"]), (m, e_m)
        labelled = int((b["labels"][:, 1:] != -100).sum())
        assert abs(m["mean_token_accuracy"] - e_m["mean_token_accuracy"]) <= 1.0 / labelled
    runner = qlora_step.BucketedGraphSteps(model, opt, scaler, bucket=bucket)
    seen = set()
    for seed in range(600, 900):
        b, lengths = qlora_step.make_batch(dev, seed=seed)
        total = -(-int(lengths.sum()) // bucket) * bucket
        if total == total0 or (len(seen) == 2 and total not in seen):
            continue
        seen.add(total)
        loss = float(runner.step(b, metrics={}))
        torch.cuda.synchronize()
        assert torch.isfinite(torch.tensor(loss))
        if len(seen) == 2 and seed >= 640:
            break
    assert len(seen) == 2
    assert sorted(runner.graphs) == sorted(seen) and len(runner.capture_ms) == 2
