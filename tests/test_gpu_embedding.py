"""fp16 storage of the tied embedding / head weight (claudemaxing_amd/embedding.py), the cases of
the reference's tests_local/test_embedding.py: lossless with the same outputs (hooks and deepcopy
included), a weight with a non-fp16 value left alone, untied or trainable weights left alone,
and a conversion that never holds both copies on the GPU; plus the fused head reading the fp16
weight itself (no second fp16 copy)."""

import copy

import pytest
import torch

from tests.conftest import banner


def _tiny(dev, tied=True):
    from transformers import Qwen2Config, Qwen2ForCausalLM

    cfg = Qwen2Config(vocab_size=1000, hidden_size=64, intermediate_size=128,
                      num_hidden_layers=1, num_attention_heads=4, num_key_value_heads=2,
                      tie_word_embeddings=tied)
    torch.manual_seed(0)
    model = Qwen2ForCausalLM(cfg).half().to(dev)  # loaded in fp16 ...
    emb = model.get_input_embeddings()
    emb.weight.data = emb.weight.data.float()
    if tied:
        model.tie_weights()
    for p in model.parameters():  # ... upcast and frozen, as for k-bit training
        p.requires_grad_(False)
    return model


@pytest.mark.gpu
def test_lossless_and_same_outputs(dev):
    banner("tied embedding: fp16 storage, same outputs")
    from claudemaxing_amd.embedding import shrink_tied_embedding

    model = _tiny(dev)
    emb, head = model.get_input_embeddings(), model.get_output_embeddings()
    assert head.weight is emb.weight and emb.weight.dtype == torch.float32
    ref = emb.weight.detach().clone()
    ids = torch.randint(0, 1000, (2, 17), device=dev)
    out_ref = emb(ids)
    seen = []
    emb.register_forward_hook(lambda m, i, o: seen.append(o.dtype))
    assert shrink_tied_embedding(model) is False  # not under fp16 autocast: undecided
    with torch.autocast("cuda", dtype=torch.float16):
        assert shrink_tied_embedding(model) is True
    assert emb.weight.dtype == torch.float16 and head.weight is emb.weight
    assert torch.equal(emb.weight.float(), ref)
    out = emb(ids)
    assert out.dtype == torch.float32 and torch.equal(out, out_ref)
    assert seen == [torch.float32]
    assert shrink_tied_embedding(model) is True  # decided once
    with torch.autocast("cuda", dtype=torch.float16):
        assert torch.equal(emb(ids), out_ref)
    assert torch.equal(copy.deepcopy(emb)(ids), out_ref)


@pytest.mark.gpu
def test_not_exact_left_alone(dev):
    banner("tied embedding: a non-fp16 value")
    from claudemaxing_amd.embedding import shrink_tied_embedding

    model = _tiny(dev)
    w = model.get_input_embeddings().weight
    w.data[5, 3] = 1.0 + 2 ** -20
    with torch.autocast("cuda", dtype=torch.float16):
        assert shrink_tied_embedding(model) is False
    assert w.dtype == torch.float32 and w.data[5, 3].item() == 1.0 + 2 ** -20


@pytest.mark.gpu
def test_untied_or_trainable_left_alone(dev):
    banner("tied embedding: untied / trainable")
    from claudemaxing_amd.embedding import shrink_tied_embedding

    with torch.autocast("cuda", dtype=torch.float16):
        assert shrink_tied_embedding(_tiny(dev, tied=False)) is False
        model = _tiny(dev)
        model.get_input_embeddings().weight.requires_grad_(True)
        assert shrink_tied_embedding(model) is False


@pytest.mark.gpu
def test_conversion_never_holds_both_copies(dev):
    banner("tied embedding: peak memory of the conversion")
    from claudemaxing_amd.embedding import shrink_tied_embedding

    model = _tiny(dev)
    w = model.get_input_embeddings().weight
    torch.cuda.synchronize()
    before = torch.cuda.memory_allocated()
    torch.cuda.reset_peak_memory_stats()
    with torch.autocast("cuda", dtype=torch.float16):
        assert shrink_tied_embedding(model) is True
    fp32_bytes = w.numel() * 4
    # the fp32 weight plus the temporaries of one checked chunk, never fp32 + the full fp16
    assert torch.cuda.max_memory_allocated() - before < fp32_bytes * 0.5 + 8192 * 64 * 8
    assert torch.cuda.memory_allocated() - before <= -fp32_bytes // 2 + 4096


@pytest.mark.gpu
def test_fused_head_reads_the_fp16_weight(dev):
    banner("tied embedding: the fused head uses the fp16 weight itself")
    from claudemaxing_amd import apply
    from claudemaxing_amd.lm_head_loss import _REQUEST_ATTR, fp16_head_weights

    apply()
    model = _tiny(dev)
    ids = torch.randint(0, 1000, (2, 40), device=dev)
    labels = ids.clone()
    labels[:, -5:] = -100
    model.__dict__[_REQUEST_ATTR] = True
    with torch.autocast("cuda", dtype=torch.float16):
        out = model(input_ids=ids, attention_mask=torch.ones_like(ids), labels=labels,
                    use_cache=False)
    assert torch.isfinite(out.loss)
    w = model.get_input_embeddings().weight
    assert w.dtype == torch.float16
    w16, _ = fp16_head_weights(w, False)
    assert w16.data_ptr() == w.data_ptr()
