"""One QLoRA training step of a Qwen2.5-1.5B-shaped model on one GPU, on this kernel set.

The reference measures its kernels inside a Soup/TRL SFT run of Qwen2.5-1.5B-Instruct
(task/task.yaml: 4-bit quantization, LoRA r=16 / alpha=32, lr 2e-4, batch 4, max_length 512)
driven by harness/_train.py, which times each trainer step between two
`torch.cuda.synchronize()` calls (_train.py:145-157). The trainer step is fp16 autocast +
GradScaler, AdamW on the LoRA parameters, and TRL's compute_loss asking the causal LM for the
fused head (solution/lm_head_loss.py:475-512), which packs the pad tokens out (300-363).

This module builds the same step without the network and without bitsandbytes/peft/TRL:

* `build_model`: transformers' Qwen2ForCausalLM from a local config (random init), every
  linear of the decoder stored as NF4 (`NF4Linear`, blocksize 64 with double-quantized absmax;
  o_proj and down_proj hand their output to the fp32 residual stream in fp32),
  LoRA (`LoRALinear`, fp32 parameters, dropout 0.05) on q_proj and v_proj, everything else
  frozen, tied fp32 embedding (fp16 values, as a checkpoint loaded in fp16 and upcast; the fused
  head then stores it in fp16), and the kernel set's patches applied (`apply()`);
* `make_batch`: 4 rows with token lengths uniform in [64, 512], right-padded, labels = ids with
  -100 at the pads;
* `train_step`: the fused-head request TRL's compute_loss makes, the forward under fp16 autocast,
  the scaled backward, the AdamW step through the GradScaler, zeroed gradients.

`unpatched()` restores the stock transformers code paths for the duration of a `with` block,
so the same model can be run through both (the parity test of the step).
"""

import contextlib
import threading
import time

import torch

from . import apply
from .attention import packed_rows
from .embedding import shrink_tied_embedding
from .lm_head_loss import (_REQUEST_ATTR, _STEP_ATTR, HeadTerms, _pack_batch, _packed_forward,
                           head_metrics_from_logits, trl_metrics)
from .lora import LoRALinear
from .nf4_linear import NF4Linear

# Qwen2.5-1.5B (config.json of Qwen/Qwen2.5-1.5B-Instruct, restated).
QWEN25_1P5B = dict(vocab_size=151936, hidden_size=1536, intermediate_size=8960,
                   num_hidden_layers=28, num_attention_heads=12, num_key_value_heads=2,
                   max_position_embeddings=32768, rope_theta=1000000.0, rms_norm_eps=1e-6,
                   tie_word_embeddings=True, hidden_act="silu", attention_dropout=0.0,
                   use_sliding_window=False, initializer_range=0.02)

LORA_TARGETS = ("q_proj", "v_proj")
# linears whose output is added to the fp32 residual stream: they hand over fp32
RESIDUAL_OUTPUTS = ("o_proj", "down_proj")
NF4_TARGETS = (("self_attn", ("q_proj", "k_proj", "v_proj", "o_proj")),
               ("mlp", ("gate_proj", "up_proj", "down_proj")))


def qwen2_config(**overrides):
    from transformers import Qwen2Config

    cfg = Qwen2Config(**{**QWEN25_1P5B, **overrides})
    cfg._attn_implementation = "sdpa"
    return cfg


def build_model(device, seed=0, r=16, alpha=32, dropout=0.05, patch=True, **overrides):
    """The QLoRA model: random-init Qwen2 weights (seeded), NF4 decoder linears, LoRA on q/v.

    transformers' Qwen2ForCausalLM is built on the meta device and materialized part by part:
    the embedding (tied to the head), the final norm and the rotary table, then one decoder layer
    at a time, whose fp32 linears exist on `device` only until they are stored as NF4. The
    device's peak during the build is then the embedding, one fp32 layer and the NF4 layers
    so far (~1.8 GB at the 1.5B shape), where building the whole fp32 model first took 6.8 GB
    and left its NF4 layers scattered over 2 GB of cached, unreleasable segments. Weights are
    drawn as transformers' _init_weights draws them (linears and embedding N(0,
    initializer_range), zero biases, unit norm weights) and rounded to fp16 values, as a
    checkpoint loaded in fp16 and upcast for k-bit training."""
    from transformers import Qwen2ForCausalLM
    from transformers.models.qwen2.modeling_qwen2 import (Qwen2DecoderLayer, Qwen2RMSNorm,
                                                          Qwen2RotaryEmbedding)

    if patch:
        apply()
    cfg = qwen2_config(**overrides)
    device = torch.device(device)
    std = cfg.initializer_range
    torch.manual_seed(seed)

    def init_(module):
        """transformers' initialization of one module's own parameters, rounded to fp16."""
        with torch.no_grad():
            if isinstance(module, (torch.nn.Linear, torch.nn.Embedding)):
                module.weight.normal_(0.0, std)
                if getattr(module, "bias", None) is not None:
                    module.bias.zero_()
            elif isinstance(module, Qwen2RMSNorm):
                module.weight.fill_(1.0)
            for p in module.parameters(recurse=False):
                p.copy_(p.to(torch.float16))

    with torch.device("meta"):
        model = Qwen2ForCausalLM(cfg)
    inner = model.model
    with torch.device(device):
        inner.embed_tokens = torch.nn.Embedding(cfg.vocab_size, cfg.hidden_size,
                                                cfg.pad_token_id)
        init_(inner.embed_tokens)
        if cfg.pad_token_id is not None:
            with torch.no_grad():
                inner.embed_tokens.weight[cfg.pad_token_id].zero_()
        inner.norm = Qwen2RMSNorm(cfg.hidden_size, eps=cfg.rms_norm_eps)
        init_(inner.norm)
        inner.rotary_emb = Qwen2RotaryEmbedding(config=cfg)
        if cfg.tie_word_embeddings:
            model.lm_head.weight = inner.embed_tokens.weight
        else:
            model.lm_head = torch.nn.Linear(cfg.hidden_size, cfg.vocab_size, bias=False)
            init_(model.lm_head)
        for i in range(cfg.num_hidden_layers):
            layer = Qwen2DecoderLayer(cfg, i)
            for module in layer.modules():
                init_(module)
            layer.requires_grad_(False)
            for block_name, names in NF4_TARGETS:
                block = getattr(layer, block_name)
                for name in names:
                    lin = getattr(block, name)
                    out_dtype = torch.float32 if name in RESIDUAL_OUTPUTS else None
                    setattr(block, name, NF4Linear.from_weight(lin.weight, bias=lin.bias,
                                                               out_dtype=out_dtype))
                    del lin
            for name in LORA_TARGETS:
                base = getattr(layer.self_attn, name)
                setattr(layer.self_attn, name, LoRALinear(base, r=r, alpha=alpha,
                                                          dropout=dropout))
            inner.layers[i] = layer
    left = [n for n, t in list(model.named_parameters()) + list(model.named_buffers())
            if t.is_meta]
    if left:
        raise RuntimeError(f"build_model left tensors unmaterialized: {left[:4]}")
    for n, p in model.named_parameters():
        p.requires_grad_("lora_" in n)
    model.train()
    if device.type == "cuda":
        torch.cuda.empty_cache()
    return model


def lora_parameters(model):
    return [p for n, p in model.named_parameters() if "lora_" in n]


def make_batch(device, seed=0, batch=4, lo=64, hi=512, vocab=QWEN25_1P5B["vocab_size"]):
    """Right-padded ids [batch, max_len], attention mask and labels (-100 at the pads); the
    row lengths are uniform in [lo, hi] (seeded)."""
    g = torch.Generator().manual_seed(seed)
    lengths = torch.randint(lo, hi + 1, (batch,), generator=g)
    width = int(lengths.max())
    ids = torch.randint(0, vocab, (batch, width), generator=g)
    mask = (torch.arange(width)[None, :] < lengths[:, None]).to(torch.int64)
    ids = ids * mask
    labels = torch.where(mask.bool(), ids, torch.full_like(ids, -100))
    return dict(input_ids=ids.to(device), attention_mask=mask.to(device),
                labels=labels.to(device)), lengths


def make_optimizer(model, lr=2e-4):
    """The optimizer transformers' Trainer builds with its defaults (task/task.yaml sets only the
    learning rate): `optim="adamw_torch_fused"` (the default for torch >= 2.8), i.e. torch's
    fused AdamW, betas (0.9, 0.999), eps 1e-8, weight decay 0."""
    return torch.optim.AdamW(lora_parameters(model), lr=lr, betas=(0.9, 0.999), eps=1e-8,
                             weight_decay=0.0, fused=True)


def train_step(model, opt, scaler, batch, fused=True, metrics=None):
    """Forward (fp16 autocast), scaled backward, optimizer step; returns the loss tensor.

    With a `metrics` dict, the step also fills in what TRL's compute_loss logs every step
    (`trl_metrics`: the attention-mask weighted entropy, num_tokens, mean_token_accuracy), from
    the fused head's per-token terms, or from the logits when the forward built them; like TRL
    it reads them on the host before the backward."""
    if fused:
        model.__dict__[_REQUEST_ATTR] = True
    try:
        with torch.autocast("cuda", dtype=torch.float16):
            out = model(**batch, use_cache=False)
    finally:
        model.__dict__.pop(_REQUEST_ATTR, None)
    terms = model.__dict__.pop(_STEP_ATTR, None)
    if metrics is not None:
        if terms is None:
            terms = head_metrics_from_logits(out.logits.detach(), batch["labels"])
        metrics.update(trl_metrics(terms, batch))
    scaler.scale(out.loss).backward()
    scaler.step(opt)
    scaler.update()
    opt.zero_grad(set_to_none=True)
    return out.loss.detach()


_CAPTURE_STREAMS = {}


def _capture_stream(device):
    """The one side stream of `device` on which every GraphedStep warms up and captures. torch
    keeps a hipBLAS and a hipBLASLt workspace per stream (76 MiB each on this stack) for as long
    as the process lives, so a fresh stream per capture would pin another pair every time."""
    s = _CAPTURE_STREAMS.get(device)
    if s is None:
        s = _CAPTURE_STREAMS[device] = torch.cuda.Stream(device)
    return s


class GraphedStep:
    """The same training step with the packed forward and the scaled backward replayed from one
    HIP graph. The step issues ~5000 kernels, and in eager mode the host's launch cost exceeds
    their device time; a replay issues them without the host.

    What stays outside the graph, because it synchronises with the host: packing the batch
    (`_pack_batch` reads the number of real tokens), and the GradScaler step (its inf check) with
    AdamW. The graph is captured for one packed shape; `load` copies another batch of that
    packed shape into its inputs: with `bucket`, every batch whose real tokens round up to the
    same multiple of the bucket (the packed batch's filler row makes up the rest, and the
    attention reads its rows from the device image `load` rewrites), else the same row lengths.
    The gradients live in the graph's buffers: they are overwritten by each replay, and `step`
    points the LoRA parameters at them before the optimizer step. Nothing in the captured region
    allocates outside torch's graph pool or synchronises (the kernel library never does; the
    RMSNorm tiny-column map is computed in the warm-up), and LoRA dropout draws from torch's
    graph-safe generator, so every replay has fresh masks. Graphs given one `pool` share its
    memory for their activations (replayed one at a time, never concurrently)."""

    def __init__(self, model, opt, scaler, batch, warmup=3, bucket=None, pool=None):
        self.model, self.opt, self.scaler = model, opt, scaler
        self.params = lora_parameters(model)
        self.bucket = bucket
        with torch.autocast("cuda", dtype=torch.float16):
            shrink_tied_embedding(model)  # as the fused head's forward does
        self.packed = self._pack(batch)
        device = next(model.parameters()).device
        self.packed.rows.image_on(device)  # the rows' device image, made before the capture
        side = _capture_stream(device)
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(warmup):
                self._zero()
                self._forward_backward()
        torch.cuda.current_stream().wait_stream(side)
        self._zero()
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph, pool=pool, stream=side):
            self.loss = self._forward_backward()
        self.terms = model.__dict__.pop(_STEP_ATTR, None)  # packed per-token terms, [1, N]
        self.grads = [p.grad for p in self.params]

    def _pack(self, batch):
        kwargs = dict(input_ids=batch["input_ids"], attention_mask=batch["attention_mask"],
                      use_cache=False)
        packed = _pack_batch(self.model, kwargs, batch["labels"], bucket=self.bucket)
        if packed is None:
            raise ValueError("GraphedStep needs a padded batch with pads to pack out")
        return packed

    def _zero(self):
        for p in self.params:
            p.grad = None

    def _forward_backward(self):
        with torch.autocast("cuda", dtype=torch.float16):
            out = _packed_forward(self.model, dict(use_cache=False), self.packed, unpack=False)
        self.scaler.scale(out.loss).backward()
        return out.loss.detach()

    def load(self, batch, packed=None):
        """Copy a batch with this graph's packed shape into the graph's inputs (`packed`: the
        batch already packed for this graph's bucket)."""
        packed = packed if packed is not None else self._pack(batch)
        if packed.ids.shape != self.packed.ids.shape or (
                self.bucket is None and packed.rows.bounds != self.packed.rows.bounds):
            # without a bucket, the rows' capacity is their own padded count: same rows only
            raise ValueError("the batch packs to another shape: capture a new GraphedStep")
        self.packed.rows.load(packed.rows.bounds)
        for name in ("ids", "pos", "mask", "target"):
            getattr(self.packed, name).copy_(getattr(packed, name))
        self.packed.B, self.packed.T, self.packed.index = packed.B, packed.T, packed.index

    def pool_bytes(self):
        """Bytes of the segments of the graph's private memory pool: the activations and
        temporaries of the captured pass, which replays reuse. torch counts them as allocated
        only while the capture runs, so a replay's allocated bytes leave them out."""
        pool = tuple(self.graph.pool())
        return sum(seg["total_size"] for seg in torch.cuda.memory_snapshot()
                   if tuple(seg.get("segment_pool_id", ())) == pool)

    def step(self, metrics=None, inputs=None):
        """Replay forward + backward, then the GradScaler step with AdamW; the loss tensor. With
        a `metrics` dict (and the batch as `inputs`), TRL's three metrics of the loaded batch
        are filled in from the replay's per-token terms."""
        self.graph.replay()
        if metrics is not None:
            p = self.packed
            terms = HeadTerms(p.unpack(self.terms.token_loss), p.unpack(self.terms.token_entropy),
                              self.terms.correct, self.terms.labelled)
            metrics.update(trl_metrics(terms, inputs))
        for p, g in zip(self.params, self.grads):
            p.grad = g
        self.scaler.step(self.opt)
        self.scaler.update()
        return self.loss.clone()


class BucketedGraphSteps:
    """Training steps over batches of any packed length, each replayed from a captured HIP
    graph: a batch's real tokens are packed to the next multiple of `bucket` (a filler row with
    ignored labels), and the first batch of each bucket captures that bucket's GraphedStep
    (then ~70-150 ms); later batches of the bucket only load their tokens and rows into it. The
    graphs share one memory pool, so the activations take the largest bucket's, not the sum.
    Only the first capture runs eager warm-up passes (the lazy state they set up: BLAS handles
    and workspaces, the RMSNorm tiny-column maps, the NF4 descriptors, is shared by every
    bucket), so later captures add no eager activations beside the pool."""

    def __init__(self, model, opt, scaler, bucket=256, warmup=1):
        self.model, self.opt, self.scaler = model, opt, scaler
        self.bucket, self.warmup = bucket, warmup
        self.graphs = {}
        self.pool = torch.cuda.graph_pool_handle()
        self.capture_ms = []

    def step(self, batch, metrics=None):
        kwargs = dict(input_ids=batch["input_ids"], attention_mask=batch["attention_mask"],
                      use_cache=False)
        packed = _pack_batch(self.model, kwargs, batch["labels"], bucket=self.bucket)
        if packed is None:
            raise ValueError("BucketedGraphSteps needs padded batches with pads to pack out")
        total = packed.ids.shape[1]
        g = self.graphs.get(total)
        if g is None:
            t0 = time.perf_counter()
            g = self.graphs[total] = GraphedStep(
                self.model, self.opt, self.scaler, batch,
                warmup=0 if self.capture_ms else self.warmup, bucket=self.bucket,
                pool=self.pool)
            torch.cuda.empty_cache()  # the warm-up's eager blocks outside the graph pool
            self.capture_ms.append((time.perf_counter() - t0) * 1e3)
        else:
            g.load(batch, packed)
        return g.step(metrics, batch)

    def pool_bytes(self):
        """Bytes of the shared graph pool's segments."""
        if not self.graphs:
            return 0
        return next(iter(self.graphs.values())).pool_bytes()


def time_steps(model, opt, scaler, batch, steps, warmup, graphed=False):
    """Median and all per-step wall times (ms), each step between two device syncs as the
    reference's harness probe times them; peak HBM over the timed steps. With graphed, the
    steps replay a GraphedStep captured first (the capture and its warm-up are not timed), and
    graph_pool_gb is the size of its private pool, which the replay's allocated bytes leave
    out."""
    if graphed:
        gstep = GraphedStep(model, opt, scaler, batch)
        run = gstep.step
    else:
        def run():
            return train_step(model, opt, scaler, batch)
    for _ in range(warmup):
        run()
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats()
    times, losses = [], []
    for _ in range(steps):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        losses.append(run())
        torch.cuda.synchronize()
        times.append((time.perf_counter() - t0) * 1e3)
    ordered = sorted(times)
    out = dict(median_ms=ordered[len(ordered) // 2], step_ms=times,
               peak_allocated_gb=torch.cuda.max_memory_allocated() / 2 ** 30,
               peak_reserved_gb=torch.cuda.max_memory_reserved() / 2 ** 30,
               losses=[float(x) for x in losses])
    if graphed:
        out["graph_pool_gb"] = gstep.pool_bytes() / 2 ** 30
    return out


def time_distinct_batches(model, opt, scaler, steps, warmup, seed0=1000, mode="eager",
                          bucket=256):
    """Per-step wall times (ms) over a fresh batch every step (new U[64, 512] lengths, so the
    packed shape changes every step, as in SFT), each step between two device syncs, with TRL's
    three metrics computed every step as its compute_loss does. mode: "eager"; "capture_each"
    (every step captures a new GraphedStep for its batch and replays it once); "bucketed"
    (BucketedGraphSteps: a step replays its bucket's graph, and the first batch of a bucket
    captures it, inside the timed step). Returns the median, the times, the real tokens per
    step, the peak HBM, and for "bucketed" the captures made while timing and the graph pool's
    size."""
    def batch_of(i):
        return make_batch(next(model.parameters()).device, seed=seed0 + i)

    runner = BucketedGraphSteps(model, opt, scaler, bucket) if mode == "bucketed" else None

    def run(batch):
        if mode == "capture_each":
            return GraphedStep(model, opt, scaler, batch, warmup=1).step(metrics={},
                                                                         inputs=batch)
        if mode == "bucketed":
            return runner.step(batch, metrics={})
        if mode != "eager":
            raise ValueError(f"unknown mode {mode!r}")
        return train_step(model, opt, scaler, batch, metrics={})

    for i in range(warmup):
        run(batch_of(i)[0])
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats()
    captured_before = len(runner.capture_ms) if runner else 0
    times, tokens = [], []
    for i in range(steps):
        batch, lengths = batch_of(warmup + i)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        run(batch)
        torch.cuda.synchronize()
        times.append((time.perf_counter() - t0) * 1e3)
        tokens.append(int(lengths.sum()))
    ordered = sorted(times)
    out = dict(median_ms=ordered[len(ordered) // 2], mean_ms=sum(times) / len(times),
               step_ms=times, tokens=tokens, tokens_per_s=sum(tokens) / (sum(times) * 1e-3),
               peak_allocated_gb=torch.cuda.max_memory_allocated() / 2 ** 30,
               peak_reserved_gb=torch.cuda.max_memory_reserved() / 2 ** 30)
    if runner is not None:
        out.update(captures_timed=len(runner.capture_ms) - captured_before,
                   capture_ms=runner.capture_ms[captured_before:],
                   buckets=sorted(runner.graphs), graph_pool_gb=runner.pool_bytes() / 2 ** 30)
    return out


class VramPoller:
    """Device memory in use (MiB), sampled every `interval` s from a thread while the block runs,
    as the reference's harness samples nvidia-smi's memory.used every 100 ms
    (harness/common.py:48-85). The figure is device-level, total minus free
    (torch.cuda.mem_get_info): every process on the device, the runtime's own allocations and
    torch's cache, not only torch's allocated bytes (amd-smi on these boxes reports no per-device
    use). `start` is the first sample, `peak` the largest."""

    def __init__(self, device=None, interval=0.1):
        self.device = torch.device("cuda", torch.cuda.current_device()) if device is None \
            else torch.device(device)
        self.interval, self.start, self.peak, self.samples = interval, None, 0.0, 0
        self._stop = threading.Event()

    def _used_mib(self):
        free, total = torch.cuda.mem_get_info(self.device)
        return (total - free) / 2 ** 20

    def _run(self):
        while not self._stop.is_set():
            used = self._used_mib()
            self.peak = max(self.peak, used)
            self.samples += 1
            self._stop.wait(self.interval)

    def __enter__(self):
        self.start = self._used_mib()
        self.peak = self.start
        self._thread = threading.Thread(target=self._run, daemon=True)
        self._thread.start()
        return self

    def __exit__(self, *exc):
        self._stop.set()
        self._thread.join(timeout=5)
        self.peak = max(self.peak, self._used_mib())
        return False


@contextlib.contextmanager
def unpatched():
    """The stock transformers Qwen2 code paths (RMSNorm, RoPE, MLP, attention block, decoder
    layer, causal-LM forward, sdpa attention) and the plain LoRA computation (nn.Dropout + two linears) for the duration of the block; the kernel
    set's paths are put back afterwards. NF4Linear keeps its dequant kernel (bit-exact to the
    NF4 oracle, so the weights are the same either way)."""
    from transformers.models.qwen2 import modeling_qwen2 as mq

    from . import lora

    from transformers.modeling_utils import AttentionInterface

    saved = [(lora, "_branch_applies", lora._branch_applies)]
    lora._branch_applies = lambda *args: False
    sdpa = AttentionInterface._global_mapping.get("sdpa")
    if getattr(sdpa, "_original", None) is not None:
        saved.append((AttentionInterface._global_mapping, "sdpa", sdpa))
        AttentionInterface._global_mapping["sdpa"] = sdpa._original
    for owner, attr in ((mq.Qwen2RMSNorm, "forward"), (mq.Qwen2MLP, "forward"),
                        (mq.Qwen2ForCausalLM, "forward"), (mq.Qwen2Attention, "forward"),
                        (mq.Qwen2DecoderLayer, "forward"), (mq, "apply_rotary_pos_emb")):
        current = getattr(owner, attr)
        original = getattr(current, "_original", None)
        if original is not None:
            saved.append((owner, attr, current))
            setattr(owner, attr, original)
    try:
        yield
    finally:
        for owner, attr, current in saved:
            if isinstance(owner, dict):
                owner[attr] = current
            else:
                setattr(owner, attr, current)
