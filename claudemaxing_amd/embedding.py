"""fp16 storage of the frozen, tied embedding / LM-head weight of the 4-bit model.

Reference: solution/embedding.py:1-79 (`shrink_tied_embedding`), called by the fused head's
Qwen2ForCausalLM.forward (solution/lm_head_loss.py:388) on every fused training step.

A QLoRA model is loaded in fp16 and then has its non-quantized parameters upcast to fp32 (peft's
prepare_model_for_kbit_training), so the tied [151936, 1536] embedding is held as fp32 (890 MiB)
although every value is an fp16 number. Stored as fp16 it takes half of that and no value
changes: the embedding's output is cast back to fp32 (the residual stream sees the same
numbers), and the fused LM head computes in fp16 anyway (it casts the fp32 weight to fp16 for its
GEMMs; with the fp16 weight it reads the weight itself, with no second copy).

The conversion happens only when it is lossless (every value checked), under fp16 autocast (the
head is then only used through fp16 products), for a frozen weight shared by a plain
nn.Embedding and a plain nn.Linear head. It stages the fp16 values in pinned host memory chunk by
chunk, so the GPU never holds the fp32 and the fp16 copy at once. The decision is recorded on
the model; later calls return it.
"""

import types

import torch
import torch.nn.functional as F

_FLAG = "_fp16_tied_embedding"  # on the causal LM: True (stored in fp16 here) or False


def _forward_as_fp32(self, input):
    """nn.Embedding.forward over the fp16 weight, returning the fp32 values of the fp32 weight."""
    out = F.embedding(input, self.weight, self.padding_idx, self.max_norm, self.norm_type,
                      self.scale_grad_by_freq, self.sparse)
    return out.to(torch.float32)


def _store_as_fp16(param, rows=8192):
    """Replace the fp32 storage of `param` by fp16 if every value is an fp16 number; False (and
    param unchanged) otherwise. Chunks of `rows` rows are checked and staged in pinned host memory;
    the fp32 storage is released before the fp16 tensor is uploaded."""
    data = param.data
    staged = torch.empty(data.shape, dtype=torch.float16, pin_memory=True)
    for r0 in range(0, data.shape[0], rows):
        part = data[r0:r0 + rows]
        half = part.to(torch.float16)
        if not torch.equal(half.to(torch.float32), part):
            return False
        staged[r0:r0 + rows].copy_(half)
    device = data.device
    del data, part, half  # views of the fp32 storage
    param.data = torch.empty(0, dtype=torch.float16, device=device)
    param.data = staged.to(device)
    return True


def _fp16_autocast():
    return torch.is_autocast_enabled("cuda") and torch.get_autocast_dtype("cuda") == torch.float16


def shrink_tied_embedding(lm):
    """Store the tied fp32 embedding / head weight of the causal LM `lm` in fp16 when that is
    lossless. True when the weight is (now) held in fp16 by this function; False when it is left
    as it is (decided once, under fp16 autocast; outside it nothing is decided yet)."""
    done = getattr(lm, _FLAG, None)
    if done is not None:
        return done
    if not _fp16_autocast():
        return False
    emb, head = lm.get_input_embeddings(), lm.get_output_embeddings()
    w = getattr(emb, "weight", None)
    eligible = (type(emb) is torch.nn.Embedding and type(head) is torch.nn.Linear
                and w is not None and head.weight is w and w.dtype == torch.float32
                and w.is_cuda and not w.requires_grad and emb.max_norm is None
                and not emb.sparse and not emb._forward_pre_hooks
                and "forward" not in emb.__dict__ and not hasattr(emb, "_hf_hook"))
    stored = False
    if eligible:
        with torch.no_grad():
            stored = _store_as_fp16(w)
        if stored:
            # an instance attribute: module hooks still run around it and deepcopy keeps it
            emb.forward = types.MethodType(_forward_as_fp32, emb)
    setattr(lm, _FLAG, stored)
    return stored
