"""The host glue around the kernels that only runs with third-party libraries absent here
(bitsandbytes 0.50.2, peft 0.20.0, TRL 0.29.1), exercised on the CPU against stand-ins that have
the attributes and call signatures the glue uses: which calls each patch takes over and which
it leaves to the library, idempotence, and TRL's compute_loss path end to end (the fused
forward's per-token terms turned into the logged metrics). Also the guards of the RoPE and
RMSNorm patches. No kernel runs: the calls that would launch are the ones handed to the
libraries' own code, or intercepted."""

import sys
import types
from collections import defaultdict
from types import SimpleNamespace

import pytest
import torch

from claudemaxing_amd import lm_head_loss as LH
from claudemaxing_amd import lora, nf4, rmsnorm, rope
from claudemaxing_amd._patching import install, tagged


class _FakeCuda(torch.Tensor):
    @property
    def is_cuda(self):
        return True


def _cuda(t):
    return t.as_subclass(_FakeCuda)


# -- bitsandbytes --------------------------------------------------------------------------------
@pytest.fixture
def fake_bnb(monkeypatch):
    calls = []
    functional = types.ModuleType("bitsandbytes.functional")

    class QuantState:
        def __init__(self, absmax, shape=None, code=None, blocksize=64, quant_type="nf4",
                     dtype=torch.float16, offset=None, state2=None):
            self.absmax, self.shape, self.code, self.blocksize = absmax, shape, code, blocksize
            self.quant_type, self.dtype, self.offset, self.state2 = quant_type, dtype, offset, state2

        @property
        def nested(self):
            return self.state2 is not None

    functional.QuantState = QuantState
    functional.dequantize_4bit = lambda *a, **k: calls.append(("dequantize_4bit", a, k)) or "bnb"
    ops = types.ModuleType("bitsandbytes.backends.cuda.ops")
    ops._dequant_linear_fallback = lambda *a, **k: calls.append(("fallback", a, k)) or "bnb"
    pkg = types.ModuleType("bitsandbytes")
    pkg.functional = functional
    for name, mod in (("bitsandbytes", pkg), ("bitsandbytes.functional", functional),
                      ("bitsandbytes.backends", types.ModuleType("bitsandbytes.backends")),
                      ("bitsandbytes.backends.cuda", types.ModuleType("bitsandbytes.backends.cuda")),
                      ("bitsandbytes.backends.cuda.ops", ops)):
        monkeypatch.setitem(sys.modules, name, mod)
    sys.modules["bitsandbytes.backends.cuda"].ops = ops
    monkeypatch.setattr(nf4, "ORIGINALS", {})
    return SimpleNamespace(functional=functional, ops=ops, calls=calls, QuantState=QuantState)


def test_bnb_patch_leaves_what_the_kernel_does_not_take(fake_bnb):
    nf4.patch_bnb_nf4_dequant()
    routed_fallback, routed_dequant = fake_bnb.ops._dequant_linear_fallback, \
        fake_bnb.functional.dequantize_4bit
    assert set(nf4.ORIGINALS) == {"fallback", "dequant"}
    nf4.patch_bnb_nf4_dequant()  # idempotent: not wrapped twice
    assert fake_bnb.ops._dequant_linear_fallback is routed_fallback
    a_cpu = torch.zeros(3, 64)
    b = torch.zeros(64 * 32 // 2, 1, dtype=torch.uint8)
    absmax = torch.ones(32)
    # a CPU input, an fp4 weight, a bf16 input, an incomplete double quantization: bitsandbytes
    for args, kw in [((a_cpu, b, (32, 64), absmax, 64, "nf4"), {}),
                     ((_cuda(a_cpu), b, (32, 64), absmax, 64, "fp4"), {}),
                     ((_cuda(a_cpu.bfloat16()), b, (32, 64), absmax, 64, "nf4"), {}),
                     ((_cuda(a_cpu), b, (32, 64), absmax, 64, "nf4"),
                      dict(absmax_8bit=absmax.to(torch.uint8), absmax_code=None))]:
        fake_bnb.calls.clear()
        assert routed_fallback(*args, **kw) == "bnb"
        assert [c[0] for c in fake_bnb.calls] == ["fallback"]
        assert fake_bnb.calls[0][1][:6] == args[:6]
    # an NF4 state that is not on the GPU, an `out` buffer, no state: bitsandbytes
    state = fake_bnb.QuantState(absmax, shape=torch.Size((32, 64)), code=torch.zeros(16))
    for kw in [dict(quant_state=state), dict(quant_state=state, out=torch.empty(32, 64)),
               dict(quant_state=None, absmax=absmax)]:
        fake_bnb.calls.clear()
        assert routed_dequant(b, **kw) == "bnb"
        assert [c[0] for c in fake_bnb.calls] == ["dequantize_4bit"]


def test_bnb_state_of_a_double_quantized_call(fake_bnb):
    a = torch.zeros(2, 64, dtype=torch.float16)
    q8, absmax2, code2, off = torch.zeros(32, dtype=torch.uint8), torch.ones(1), \
        torch.zeros(256), torch.tensor(0.5)
    st = nf4._bnb_linear_state(fake_bnb.QuantState, a, (32, 64), absmax2, 64, q8, code2, off)
    assert st.absmax is q8 and st.offset is off and st.blocksize == 64 and st.quant_type == "nf4"
    assert st.state2.absmax is absmax2 and st.state2.code is code2 and st.state2.blocksize == 256
    assert tuple(st.shape) == (32, 64) and st.dtype == torch.float16
    plain = nf4._bnb_linear_state(fake_bnb.QuantState, a, (32, 64), absmax2, 64, None, None, None)
    assert plain.state2 is None and plain.absmax is absmax2


# -- peft ----------------------------------------------------------------------------------------
def _peft_layer(**over):
    layer = SimpleNamespace(
        active_adapters=["default"], disable_adapters=False, merged=False,
        lora_A=torch.nn.ModuleDict({"default": torch.nn.Linear(16, 4, bias=False)}),
        lora_B=torch.nn.ModuleDict({"default": torch.nn.Linear(4, 8, bias=False)}),
        lora_dropout=torch.nn.ModuleDict({"default": torch.nn.Dropout(0.05)}),
        scaling={"default": 2.0}, training=True, use_dora={}, fan_in_fan_out=False)
    for k, v in over.items():
        setattr(layer, k, v)
    return layer


def test_peft_adapter_selection(monkeypatch):
    monkeypatch.setattr(lora, "_branch_applies", lambda *a: True)
    x = torch.zeros(2, 16)
    wa, wb, p, s = lora._peft_adapter(_peft_layer(), x, (), {})
    assert wa.shape == (4, 16) and wb.shape == (8, 4) and p == pytest.approx(0.05) and s == 2.0
    refused = [
        (_peft_layer(), (1,), {}),
        (_peft_layer(), (), {"adapter_names": ["default"]}),
        (_peft_layer(disable_adapters=True), (), {}),
        (_peft_layer(merged=True), (), {}),
        (_peft_layer(active_adapters=["default", "other"]), (), {}),
        (_peft_layer(active_adapters=["missing"]), (), {}),
        (_peft_layer(use_dora={"default": True}), (), {}),
        (_peft_layer(fan_in_fan_out=True), (), {}),
        (_peft_layer(lora_variant={"default": object()}), (), {}),
        (_peft_layer(lora_dropout=torch.nn.ModuleDict({"default": torch.nn.Identity()})), (), {}),
        (_peft_layer(lora_A=torch.nn.ModuleDict({"default": torch.nn.Linear(16, 4)})), (), {}),
    ]
    for layer, args, kwargs in refused:
        assert lora._peft_adapter(layer, x, args, kwargs) is None
    monkeypatch.setattr(lora, "_branch_applies", lambda *a: False)
    assert lora._peft_adapter(_peft_layer(), x, (), {}) is None


def test_peft_forward_falls_back_to_peft(monkeypatch):
    seen = []

    def original(self, x, *args, **kwargs):
        seen.append((args, kwargs))
        return "peft"

    class Layer:
        pass

    Layer.forward = original
    forward = install(Layer, "forward", "lora_branch", lora._peft_forward)
    assert tagged(forward, "lora_branch") and forward._original is original
    assert install(Layer, "forward", "lora_branch", lora._peft_forward) is None  # idempotent
    assert forward(_peft_layer(), torch.zeros(2, 16), 3, scale=1) == "peft"
    assert seen == [((3,), {"scale": 1})]


# -- TRL -----------------------------------------------------------------------------------------
class _FusedLM(torch.nn.Module):
    """A causal LM whose forward (marked as the fused head) returns the loss and leaves
    HeadTerms behind when the request attribute is set, as the patched Qwen2 forward does."""

    def __init__(self):
        super().__init__()
        self.head = torch.nn.Linear(4, 10, bias=False)
        self.head.requires_grad_(False)
        self.config = SimpleNamespace(final_logit_softcapping=None)

    def get_output_embeddings(self):
        return self.head

    def forward(self, input_ids=None, attention_mask=None, labels=None, **kw):
        asked = self.__dict__.pop(LH._REQUEST_ATTR, False)
        b, t = input_ids.shape
        ent = torch.arange(b * t, dtype=torch.float32).view(b, t) / 10
        self.__dict__[LH._STEP_ATTR] = LH.HeadTerms(torch.ones(b, t), ent, torch.tensor(3),
                                                    torch.tensor(4))
        return SimpleNamespace(loss=torch.tensor(2.5), logits=None, asked=asked)


_FusedLM.forward._cm_patch = LH._HEAD_TAG


def _trainer(model, **args):
    base = dict(n_gpu=1, use_liger_kernel=False)
    base.update(args)
    return SimpleNamespace(model=model, args=SimpleNamespace(**base),
                           _metrics=defaultdict(lambda: defaultdict(list)),
                           _total_train_tokens=0,
                           accelerator=SimpleNamespace(gather_for_metrics=lambda t: t))


def test_fusable_causal_lm_conditions(monkeypatch):
    model = _FusedLM()
    model.train()
    monkeypatch.setattr(type(model.head.weight), "is_cuda", property(lambda self: True))
    inputs = {"labels": torch.zeros(1, 3)}
    assert LH._fusable_causal_lm(_trainer(model), model, inputs) is model
    outer = torch.nn.Module()  # DDP / accelerate wrappers are unwrapped through .module
    outer.module = model
    assert LH._fusable_causal_lm(_trainer(model), outer, inputs) is model
    for trainer, inp in [(_trainer(model, n_gpu=2), inputs),
                         (_trainer(model, use_liger_kernel=True), inputs),
                         (_trainer(model), {"input_ids": torch.zeros(1, 3)}),
                         (_trainer(model), {"labels": 1, "shift_labels": 1})]:
        assert LH._fusable_causal_lm(trainer, model, inp) is None
    t = _trainer(model)
    t.label_smoother = object()
    assert LH._fusable_causal_lm(t, model, inputs) is None
    model.eval()
    assert LH._fusable_causal_lm(_trainer(model), model, inputs) is None


def test_trl_compute_loss_end_to_end(monkeypatch):
    """patch_sft_compute_loss on a stand-in SFTTrainer: a fusable step asks the model for the
    fused head, logs TRL's three metrics from its HeadTerms and leaves the per-token losses for
    Soup; a step that is not fusable runs TRL's own compute_loss."""
    class Trainer:
        def compute_loss(self, model, inputs, return_outputs=False, num_items_in_batch=None):
            out = model(**inputs)
            return (out.loss, out) if return_outputs else out.loss

    class SFTTrainer(Trainer):
        def compute_loss(self, model, inputs, return_outputs=False, num_items_in_batch=None):
            return "trl"

    sft = types.ModuleType("trl.trainer.sft_trainer")
    sft.SFTTrainer = SFTTrainer
    for name, mod in (("trl", types.ModuleType("trl")), ("trl.trainer",
                                                        types.ModuleType("trl.trainer")),
                      ("trl.trainer.sft_trainer", sft)):
        monkeypatch.setitem(sys.modules, name, mod)
    sys.modules["trl.trainer"].sft_trainer = sft
    LH.patch_sft_compute_loss()
    LH.patch_sft_compute_loss()  # idempotent
    assert tagged(SFTTrainer.compute_loss, LH._HEAD_TAG)
    model = _FusedLM()
    model.train()
    monkeypatch.setattr(type(model.head.weight), "is_cuda", property(lambda self: True))
    trainer = SFTTrainer()
    vars(trainer).update(vars(_trainer(model)))
    mask = torch.tensor([[1, 1, 1, 0], [1, 1, 0, 0]])
    inputs = {"input_ids": torch.zeros(2, 4, dtype=torch.long), "attention_mask": mask,
              "labels": torch.zeros(2, 4, dtype=torch.long)}
    loss, out = trainer.compute_loss(model, dict(inputs), return_outputs=True)
    assert float(loss) == 2.5 and out.asked is True and LH._REQUEST_ATTR not in model.__dict__
    log = trainer._metrics["train"]
    ent = torch.arange(8, dtype=torch.float32).view(2, 4) / 10
    assert log["entropy"] == [pytest.approx(float((ent * mask).sum() / 5))]
    assert log["num_tokens"] == [5] and log["mean_token_accuracy"] == [0.75]
    assert torch.equal(getattr(trainer, LH.SOUP_STEP_ATTR).token_loss, torch.ones(2, 4))
    model.eval()  # not a training step: TRL's own path, and no stale Soup losses
    assert trainer.compute_loss(model, dict(inputs)) == "trl"
    assert getattr(trainer, LH.SOUP_STEP_ATTR) is None


# -- RoPE / RMSNorm guards -----------------------------------------------------------------------
def _qkcs(batch=1, hq=4, hk=2, seq=9, dim=64, dtype=torch.float16):
    q = _cuda(torch.zeros(batch, hq, seq, dim, dtype=dtype))
    k = _cuda(torch.zeros(batch, hk, seq, dim, dtype=dtype))
    cos = _cuda(torch.zeros(1, seq, dim, dtype=dtype))
    sin = _cuda(torch.zeros(1, seq, dim, dtype=dtype))
    return q, k, cos, sin


def test_rope_guard():
    q, k, cos, sin = _qkcs()
    assert rope._kernel_covers(q, k, cos, sin, 1)
    assert not rope._kernel_covers(q, k, cos, sin, 2)
    assert not rope._kernel_covers(q, k, cos.as_subclass(torch.Tensor), sin, 1)  # on the host
    for kw in [dict(dim=48), dict(dim=258), dict(dim=7)]:  # half not a power of two; too wide
        assert not rope._kernel_covers(*_qkcs(**kw), 1)
    q2, k2, c2, s2 = _qkcs(batch=2)
    assert rope._kernel_covers(q2, k2, c2, s2, 1)  # one row of positions for the batch
    assert not rope._kernel_covers(q2, k2[:1], c2, s2, 1)
    assert not rope._kernel_covers(q, k, cos[:, :5], sin[:, :5], 1)
    assert not rope._kernel_covers(q, k, cos, sin.float(), 1)
    assert not rope._kernel_covers(q.double(), k, cos, sin, 1)


def test_rmsnorm_guard():
    x = _cuda(torch.zeros(3, 256))
    w = _cuda(torch.ones(256))
    assert rmsnorm._kernel_covers(x, w)
    assert not rmsnorm._kernel_covers(x, _cuda(torch.ones(128)))
    assert not rmsnorm._kernel_covers(x.as_subclass(torch.Tensor), w)
    assert not rmsnorm._kernel_covers(_cuda(torch.zeros(3, 256, dtype=torch.float64)), w)
    wide = _cuda(torch.zeros(1, rmsnorm.MAX_COLS + 8))
    assert not rmsnorm._kernel_covers(wide, _cuda(torch.ones(rmsnorm.MAX_COLS + 8)))


def test_install_is_idempotent_and_records_the_original():
    def stock(x):
        return x + 1

    table = {"f": stock}
    new = install(table, "f", "demo", lambda orig: (lambda x: orig(x) * 10))
    assert table["f"] is new and new._original is stock and tagged(new, "demo")
    assert new(1) == 20
    assert install(table, "f", "demo", lambda orig: None) is None and table["f"] is new
    # another patch stacks on top and keeps the first as its original
    other = install(table, "f", "other", lambda orig: (lambda x: orig(x) + 5))
    assert other._original is new and other(1) == 25
    assert install(None, "f", "demo", lambda orig: orig) is None  # class absent
    assert install({}, "f", "demo", lambda orig: orig) is None  # attribute absent


# -- Qwen2MLP ------------------------------------------------------------------------------------
def _mlp(act="silu"):
    from transformers.models.qwen2 import modeling_qwen2 as modeling

    torch.manual_seed(0)
    return modeling.Qwen2MLP(modeling.Qwen2Config(hidden_size=32, intermediate_size=64,
                                                  hidden_act=act))


def test_mlp_patch_falls_back_for_host_tensors_and_other_activations(monkeypatch):
    """The reference's test_patch_falls_back_for_cpu_and_other_activations: a host input, or an
    activation other than silu on a GPU input, runs the original forward, unchanged."""
    from transformers.models.qwen2 import modeling_qwen2 as modeling

    from claudemaxing_amd import swiglu_recompute as SR

    saved = modeling.Qwen2MLP.forward
    original = getattr(saved, "_original", saved)
    monkeypatch.setattr(modeling.Qwen2MLP, "forward", saved)
    SR.patch_qwen2_mlp_recompute()
    assert tagged(modeling.Qwen2MLP.forward, "mlp_recompute")
    launched = []
    monkeypatch.setattr(SR, "_swiglu_fwd", lambda *a: launched.append(a))
    monkeypatch.setattr(SR.MLPInputRecompute, "apply", lambda *a: launched.append(a))
    mlp = _mlp()
    x = torch.randn(2, 5, 32, requires_grad=True)
    assert torch.equal(mlp(x), original(mlp, x))
    r = torch.randn(2, 5, 32)  # the decoder layer's residual, added to the original's output
    assert torch.equal(mlp(x, residual=r), r + original(mlp, x))
    gelu = _mlp("gelu")
    xg = _cuda(torch.randn(2, 5, 32))  # looks like a GPU tensor to the guard
    assert torch.equal(gelu(xg), original(gelu, xg))
    assert not launched


def test_mlp_patch_is_idempotent(monkeypatch):
    from transformers.models.qwen2 import modeling_qwen2 as modeling

    from claudemaxing_amd import swiglu_recompute as SR

    saved = modeling.Qwen2MLP.forward
    monkeypatch.setattr(modeling.Qwen2MLP, "forward", saved)
    SR.patch_qwen2_mlp_recompute()
    first = modeling.Qwen2MLP.forward
    SR.patch_qwen2_mlp_recompute()
    assert modeling.Qwen2MLP.forward is first
    assert tagged(first, "mlp_recompute")
    assert getattr(first, "_original", None) in (saved, getattr(saved, "_original", None))


def test_mlp_patch_routes_frozen_and_trainable_projections(monkeypatch):
    """On a GPU input with silu: frozen gate/up projections under a gradient take
    MLPInputRecompute (told the down projection's 4-bit compute dtype, None for a dense one);
    trainable projections, or no gradient, take the recomputing activation between the layer's
    own projections. The kernels are intercepted, so nothing launches."""
    from transformers.models.qwen2 import modeling_qwen2 as modeling

    from claudemaxing_amd import swiglu_recompute as SR

    monkeypatch.setattr(modeling.Qwen2MLP, "forward", modeling.Qwen2MLP.forward)
    SR.patch_qwen2_mlp_recompute()
    seen = []
    monkeypatch.setattr(SR.MLPInputRecompute, "apply",
                        lambda x, g, u, dc: (seen.append(("recompute", dc)),
                                             torch.zeros(*x.shape[:-1], 64))[1])
    monkeypatch.setattr(SR, "swiglu_recompute",
                        lambda gate, up, inplace=False: (seen.append(("activation", inplace)),
                                                         gate * 0)[1])
    mlp = _mlp()
    x = _cuda(torch.randn(2, 5, 32)).requires_grad_(True)
    # a dense down projection: the residual is added after it
    r = torch.ones(2, 5, 32)
    got = mlp(x, residual=r)
    assert torch.equal(got.as_subclass(torch.Tensor),
                       r + mlp.down_proj(torch.zeros(2, 5, 64)).as_subclass(torch.Tensor))
    seen.clear()
    mlp(x)  # trainable projections
    mlp.requires_grad_(False)
    mlp(x)  # frozen: the input is all that is kept
    with torch.no_grad():
        mlp(x)  # no gradient
    assert seen == [("activation", True), ("recompute", None), ("activation", True)]


# -- Qwen2DecoderLayer ---------------------------------------------------------------------------
def _layer():
    from transformers.models.qwen2 import modeling_qwen2 as modeling

    torch.manual_seed(0)
    cfg = modeling.Qwen2Config(hidden_size=32, intermediate_size=64, num_attention_heads=2,
                               num_key_value_heads=1)
    cfg._attn_implementation = "eager"
    return modeling.Qwen2DecoderLayer(cfg, 0), cfg


def test_decoder_patch_is_idempotent_and_runs_the_original_on_the_host(monkeypatch):
    from transformers.models.qwen2 import modeling_qwen2 as modeling

    from claudemaxing_amd import decoder as D

    saved = modeling.Qwen2DecoderLayer.forward
    original = getattr(saved, "_original", saved)
    monkeypatch.setattr(modeling.Qwen2DecoderLayer, "forward", saved)
    D.patch_qwen2_decoder_residual()
    first = modeling.Qwen2DecoderLayer.forward
    D.patch_qwen2_decoder_residual()
    assert modeling.Qwen2DecoderLayer.forward is first and tagged(first, "decoder_residual")
    layer, cfg = _layer()
    x = torch.randn(1, 5, 32)
    pos = torch.arange(5).unsqueeze(0)
    pe = modeling.Qwen2RotaryEmbedding(cfg)(x, pos)
    got = layer(x, position_ids=pos, position_embeddings=pe)
    want = original(layer, x, position_ids=pos, position_embeddings=pe)
    assert torch.equal(got, want)


def test_decoder_patch_routes_only_fusable_layers(monkeypatch):
    """A GPU-looking fp32 stream through the package's norms takes norm_pass, the attention,
    add_norm and the MLP with the last add in torch; an fp16 stream, a hooked norm, or the stock
    norm forward takes the original layer. The kernels are intercepted, so nothing launches."""
    from transformers.models.qwen2 import modeling_qwen2 as modeling

    from claudemaxing_amd import decoder as D
    from claudemaxing_amd import rmsnorm as RN

    monkeypatch.setattr(modeling.Qwen2DecoderLayer, "forward",
                        modeling.Qwen2DecoderLayer.forward)
    monkeypatch.setattr(modeling.Qwen2RMSNorm, "forward", modeling.Qwen2RMSNorm.forward)
    D.patch_qwen2_decoder_residual()
    seen = []
    monkeypatch.setattr(D, "norm_pass", lambda x, w, eps: (seen.append("norm_pass"), (x, x))[1])
    monkeypatch.setattr(D, "add_norm",
                        lambda r, x, w, eps: (seen.append("add_norm"), (x, r + x))[1])

    class Attn(torch.nn.Module):
        def forward(self, hidden_states, **kwargs):
            seen.append("attn")
            return hidden_states * 2, None

    class Mlp(torch.nn.Module):
        def forward(self, x):
            seen.append("mlp")
            return x * 3

    layer, _ = _layer()
    layer.self_attn, layer.mlp = Attn(), Mlp()
    x = _cuda(torch.ones(1, 4, 32))
    stock_norm = modeling.Qwen2RMSNorm.forward
    if not tagged(stock_norm, "rmsnorm"):
        RN.patch_qwen2_rmsnorm()
    # fused: h = x + 2x, out = h + 3 * (2x)
    out = layer(x)
    assert seen == ["norm_pass", "attn", "add_norm", "mlp"]
    assert torch.equal(out.as_subclass(torch.Tensor), torch.full((1, 4, 32), 9.0))
    seen.clear()
    for case in ("fp16", "hook", "stock norm"):
        xs = x
        handle = None
        if case == "fp16":
            xs = _cuda(torch.ones(1, 4, 32, dtype=torch.float16))
        elif case == "hook":
            handle = layer.input_layernorm.register_forward_hook(lambda *a: None)
        else:
            monkeypatch.setattr(modeling.Qwen2RMSNorm, "forward",
                                modeling.Qwen2RMSNorm.forward._original)
        assert not D._norms_fusable(layer, xs), case
        if handle is not None:
            handle.remove()
    assert not seen
