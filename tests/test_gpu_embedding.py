"""The tied embedding / head weight held in fp16 (claudemaxing_amd/embedding.py,
shrink_tied_embedding), against the behaviour the reference specifies for it
(solution/embedding.py:1-79; its tests_local/test_embedding.py): converted only when no value
changes and the weight is frozen and tied, decided once under fp16 autocast, the embedding's
fp32 outputs unchanged (module hooks and deepcopy included), the GPU never holding both copies,
and the fused LM head then reading the fp16 weight itself."""

import copy

import pytest
import torch

from claudemaxing_amd.embedding import HalfStoredEmbedding, shrink_tied_embedding
from tests.conftest import banner

pytestmark = pytest.mark.gpu


class _TiedLM(torch.nn.Module):
    """The two modules shrink_tied_embedding looks at, as a causal LM exposes them."""

    def __init__(self, dev, vocab=3000, hidden=96, tied=True, seed=0):
        super().__init__()
        g = torch.Generator().manual_seed(seed)
        # fp16 numbers held in fp32: a checkpoint loaded in fp16 and upcast
        table = (torch.randn(vocab, hidden, generator=g) * 0.02).half().float()
        self.embed = torch.nn.Embedding(vocab, hidden, _weight=table.to(dev))
        self.head = torch.nn.Linear(hidden, vocab, bias=False, device=dev)
        if tied:
            self.head.weight = self.embed.weight
        for p in self.parameters():
            p.requires_grad_(False)

    def get_input_embeddings(self):
        return self.embed

    def get_output_embeddings(self):
        return self.head


def _fp16_decision(lm):
    with torch.autocast("cuda", dtype=torch.float16):
        return shrink_tied_embedding(lm)


def _spoil(lm):
    lm.embed.weight.data[1234, 17] = 1.0 / 3.0  # no fp16 number


def _untie(lm):
    lm.head.weight = torch.nn.Parameter(lm.embed.weight.detach().clone(), requires_grad=False)


def _train(lm):
    lm.embed.weight.requires_grad_(True)


def _pre_hook(lm):
    lm.embed.register_forward_pre_hook(lambda m, i: None)


@pytest.mark.parametrize("change", [_spoil, _untie, _train, _pre_hook],
                         ids=["inexact value", "untied", "trainable", "pre-hook"])
def test_weights_that_do_not_qualify_stay_fp32(change, dev):
    banner(f"tied embedding refuses: {change.__name__}")
    lm = _TiedLM(dev)
    change(lm)
    before = lm.embed.weight.detach().clone()
    assert _fp16_decision(lm) is False
    assert lm.embed.weight.dtype == torch.float32 and torch.equal(lm.embed.weight, before)
    assert type(lm.embed) is torch.nn.Embedding
    assert _fp16_decision(lm) is False  # decided: not looked at again


def test_decided_under_fp16_autocast_only(dev):
    banner("tied embedding: decided under fp16 autocast")
    lm = _TiedLM(dev)
    assert shrink_tied_embedding(lm) is False  # no autocast: undecided
    with torch.autocast("cuda", dtype=torch.bfloat16):
        assert shrink_tied_embedding(lm) is False  # bf16 autocast: still undecided
    assert lm.embed.weight.dtype == torch.float32
    assert _fp16_decision(lm) is True
    assert shrink_tied_embedding(lm) is True  # kept, with or without autocast


def test_rows_hooks_and_copies_are_unchanged(dev):
    banner("tied embedding: the same fp32 rows")
    lm = _TiedLM(dev, vocab=5000, hidden=128, seed=3)
    table = lm.embed.weight.detach().clone()
    ids = torch.randint(0, 5000, (3, 41), generator=torch.Generator().manual_seed(4)).to(dev)
    expected = lm.embed(ids)
    dtypes = []
    lm.embed.register_forward_hook(lambda m, i, o: dtypes.append(o.dtype))  # before conversion
    assert _fp16_decision(lm) is True
    w = lm.embed.weight
    assert w.dtype == torch.float16 and lm.head.weight is w and torch.equal(w.float(), table)
    assert isinstance(lm.embed, HalfStoredEmbedding)
    for got in (lm.embed(ids), copy.deepcopy(lm.embed)(ids)):
        assert got.dtype == torch.float32 and torch.equal(got, expected)
    with torch.autocast("cuda", dtype=torch.float16):
        assert torch.equal(lm.embed(ids), expected)
    assert dtypes and set(dtypes) == {torch.float32}


def test_conversion_never_holds_both_copies(dev):
    banner("tied embedding: peak memory of the conversion")
    lm = _TiedLM(dev, vocab=40000, hidden=256)
    n = lm.embed.weight.numel()
    torch.cuda.synchronize()
    base = torch.cuda.memory_allocated()
    torch.cuda.reset_peak_memory_stats()
    assert _fp16_decision(lm) is True
    torch.cuda.synchronize()
    block = 8192 * 256  # elements of one verified row block
    # never the fp32 weight plus the whole fp16 one: at most one block's temporaries on top
    assert torch.cuda.max_memory_allocated() - base <= 7 * block + 2 ** 20
    # half the bytes remain; the caching allocator may hand the fp16 copy a cached block up to
    # 1 MiB larger than asked (it splits a large block only when more than 1 MiB would remain),
    # and counts the whole block as allocated
    assert base - torch.cuda.memory_allocated() >= 2 * n - 2 ** 20


def test_fused_head_reads_the_fp16_weight(dev):
    banner("tied embedding: the fused head uses the fp16 weight itself")
    from transformers import Qwen2Config, Qwen2ForCausalLM

    from claudemaxing_amd import apply
    from claudemaxing_amd.lm_head_loss import _REQUEST_ATTR, fp16_head_weight

    apply()
    cfg = Qwen2Config(vocab_size=1000, hidden_size=64, intermediate_size=128,
                      num_hidden_layers=1, num_attention_heads=4, num_key_value_heads=2,
                      tie_word_embeddings=True)
    torch.manual_seed(0)
    model = Qwen2ForCausalLM(cfg).half().to(dev)
    emb = model.get_input_embeddings()
    emb.weight.data = emb.weight.data.float()
    model.tie_weights()
    model.requires_grad_(False)
    ids = torch.randint(0, 1000, (2, 40), device=dev)
    labels = ids.masked_fill(torch.arange(40, device=dev) >= 35, -100)
    model.__dict__[_REQUEST_ATTR] = True
    with torch.autocast("cuda", dtype=torch.float16):
        out = model(input_ids=ids, attention_mask=torch.ones_like(ids), labels=labels,
                    use_cache=False)
    assert torch.isfinite(out.loss)
    w = model.get_input_embeddings().weight
    assert w.dtype == torch.float16
    w16 = fp16_head_weight(w)
    assert w16.data_ptr() == w.data_ptr()
