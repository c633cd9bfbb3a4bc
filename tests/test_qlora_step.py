"""The QLoRA step driver's model surgery and batch (CPU): which layers are NF4, which carry LoRA,
what trains, and the padded batch's layout. The step itself runs on the GPU
(test_gpu_qlora_step.py)."""

import torch

from claudemaxing_amd import qlora_step
from claudemaxing_amd._patching import tagged
from claudemaxing_amd.lora import LoRALinear
from claudemaxing_amd.nf4_linear import NF4Linear

TINY = dict(num_hidden_layers=2, vocab_size=1024, hidden_size=256, intermediate_size=512,
            num_attention_heads=2, num_key_value_heads=1)


def test_model_surgery():
    model = qlora_step.build_model("cpu", seed=0, **TINY)
    assert model.config.hidden_size // model.config.num_attention_heads == 128
    for layer in model.model.layers:
        attn, mlp = layer.self_attn, layer.mlp
        for name in ("q_proj", "v_proj"):
            lin = getattr(attn, name)
            assert isinstance(lin, LoRALinear) and isinstance(lin.base_layer, NF4Linear)
            assert lin.base_layer.bias is not None  # Qwen2's q/k/v carry a bias
            assert lin.scaling == 2.0 and lin.p == 0.05 and lin.r == 16
            assert torch.count_nonzero(lin.lora_B.weight) == 0
        assert isinstance(attn.k_proj, NF4Linear) and attn.k_proj.bias is not None
        assert isinstance(attn.o_proj, NF4Linear) and attn.o_proj.bias is None
        assert attn.o_proj.out_dtype == torch.float32 and attn.k_proj.out_dtype is None
        assert mlp.down_proj.out_dtype == torch.float32
        for name in ("gate_proj", "up_proj", "down_proj"):
            lin = getattr(mlp, name)
            assert isinstance(lin, NF4Linear) and lin.bias is None
    # only the LoRA matrices train: r * (in + out) per q and v per layer
    h, r = TINY["hidden_size"], 16
    kv = TINY["num_key_value_heads"] * 128
    expected = TINY["num_hidden_layers"] * (r * (h + h) + r * (h + kv))
    trainable = [p for p in model.parameters() if p.requires_grad]
    assert sum(p.numel() for p in trainable) == expected
    assert all(p.dtype == torch.float32 for p in trainable)
    assert len(qlora_step.lora_parameters(model)) == 4 * TINY["num_hidden_layers"]
    # tied, frozen head
    assert model.lm_head.weight is model.model.embed_tokens.weight
    assert not model.lm_head.weight.requires_grad


def test_nf4_linear_keeps_the_weight():
    from oracle import nf4 as onf4

    torch.manual_seed(0)
    w = torch.randn(64, 128) * 0.02
    lin = NF4Linear.from_weight(w, bias=torch.randn(64))
    st = lin.quant_state
    ref = onf4.dequant(lin.packed.numpy(), st.absmax.numpy(), nested=True,
                       code2=st.state2.code.numpy(), absmax2=st.state2.absmax.numpy(),
                       offset=st.offset.numpy().astype("float32"), blocksize=64,
                       blocksize2=256).reshape(64, 128)
    # NF4 keeps each weight within half a code step of its block's scale
    assert float((torch.from_numpy(ref).float() - w).abs().max()) < 0.02 * 4 * 0.2


def test_batch_layout():
    batch, lengths = qlora_step.make_batch("cpu", seed=0)
    ids, mask, labels = batch["input_ids"], batch["attention_mask"], batch["labels"]
    assert ids.shape == mask.shape == labels.shape == (4, int(lengths.max()))
    assert ((lengths >= 64) & (lengths <= 512)).all()
    assert torch.equal(mask.sum(1), lengths)
    for b in range(4):
        n = int(lengths[b])
        assert mask[b, :n].all() and not mask[b, n:].any()  # right padding
        assert torch.equal(labels[b, :n], ids[b, :n]) and (labels[b, n:] == -100).all()
    again, _ = qlora_step.make_batch("cpu", seed=0)
    assert torch.equal(again["input_ids"], ids)  # seeded


def test_unpatched_restores_and_reapplies():
    from transformers.models.qwen2 import modeling_qwen2 as mq

    from claudemaxing_amd import apply, lora

    from transformers.modeling_utils import AttentionInterface

    from claudemaxing_amd import patch_qwen2_grouped_sdpa

    apply()
    patch_qwen2_grouped_sdpa()
    sdpa = AttentionInterface._global_mapping["sdpa"]
    assert tagged(sdpa, "packed_sdpa")
    patched = (mq.Qwen2RMSNorm.forward, mq.Qwen2MLP.forward, mq.Qwen2ForCausalLM.forward,
               mq.apply_rotary_pos_emb, mq.Qwen2DecoderLayer.forward, lora._branch_applies)
    with qlora_step.unpatched():
        assert AttentionInterface._global_mapping["sdpa"] is sdpa._original
        assert mq.Qwen2RMSNorm.forward is patched[0]._original
        assert mq.Qwen2MLP.forward is patched[1]._original
        assert mq.Qwen2ForCausalLM.forward is patched[2]._original
        assert mq.apply_rotary_pos_emb is patched[3]._original
        assert mq.Qwen2DecoderLayer.forward is patched[4]._original
        assert lora._branch_applies(None, 0.5, None, None, True) is False
    assert (mq.Qwen2RMSNorm.forward, mq.Qwen2MLP.forward, mq.Qwen2ForCausalLM.forward,
            mq.apply_rotary_pos_emb, mq.Qwen2DecoderLayer.forward, lora._branch_applies) == patched
    assert AttentionInterface._global_mapping["sdpa"] is sdpa


def test_shrink_needs_cuda_autocast():
    """Without CUDA fp16 autocast nothing is decided and the weight is left alone."""
    from transformers import Qwen2Config, Qwen2ForCausalLM

    from claudemaxing_amd.embedding import shrink_tied_embedding

    cfg = Qwen2Config(vocab_size=100, hidden_size=32, intermediate_size=64, num_hidden_layers=1,
                      num_attention_heads=2, num_key_value_heads=1, tie_word_embeddings=True)
    model = Qwen2ForCausalLM(cfg)
    assert shrink_tied_embedding(model) is False
    assert model.get_input_embeddings().weight.dtype == torch.float32
    assert not hasattr(model, "_fp16_tied_embedding")


def test_build_model_weights_are_fp16_values():
    model = qlora_step.build_model("cpu", seed=0, patch=False, num_hidden_layers=1,
                                   vocab_size=512, hidden_size=128, intermediate_size=256,
                                   num_attention_heads=2, num_key_value_heads=1)
    w = model.get_input_embeddings().weight
    assert w.dtype == torch.float32 and torch.equal(w.half().float(), w)
