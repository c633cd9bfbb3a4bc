"""The frozen tied embedding / LM-head weight of the 4-bit model held in fp16.

Public surface: `shrink_tied_embedding(lm)` (the reference's solution/embedding.py:1-79, called
by the fused head's Qwen2ForCausalLM.forward, solution/lm_head_loss.py:388).

Why it is lossless. A QLoRA model is loaded in fp16 and its non-quantized parameters are then
upcast to fp32 for k-bit training, so the tied [151936, 1536] weight occupies 890 MiB of fp32
that are all fp16 numbers. Held as fp16 it takes half, and nothing downstream sees a different
value: the embedding module returns the fp32 rows it returned before, and the fused LM head,
which computes in fp16 under autocast, reads the fp16 weight as it is (no per-step cast, no
second copy).

How. The decision is taken once per model, on the first call under fp16 autocast, and recorded
on the model. `_TiedFp16` checks that the weight qualifies (a frozen fp32 CUDA weight shared by
a plain nn.Embedding and a plain nn.Linear head, with no hooks or replaced forward on the
embedding), moves the weight through pinned host memory in row blocks -- each block verified on
the GPU to survive fp32 -> fp16 -> fp32 unchanged before it leaves -- so the GPU never holds the
fp32 and the fp16 copy at once, then gives the embedding module the class `HalfStoredEmbedding`,
whose forward widens the looked-up rows back to fp32 (module hooks still run around it, and
deepcopy keeps it).
"""

import torch
import torch.nn.functional as F

_DECIDED = "_fp16_tied_embedding"  # on the causal LM: True (held in fp16 here) or False


class HalfStoredEmbedding(torch.nn.Embedding):
    """nn.Embedding over an fp16 weight whose output is fp32: the rows of the fp32 weight it
    replaced, exactly."""

    def forward(self, input):
        rows = F.embedding(input, self.weight, self.padding_idx, self.max_norm, self.norm_type,
                           self.scale_grad_by_freq, self.sparse)
        return rows.to(torch.float32)


class _TiedFp16:
    """One causal LM's tied embedding / head pair and its conversion to fp16."""

    BLOCK_ROWS = 8192  # rows verified and staged at a time

    def __init__(self, lm):
        self.emb = lm.get_input_embeddings()
        self.head = lm.get_output_embeddings()
        self.weight = getattr(self.emb, "weight", None)

    def qualifies(self):
        emb, w = self.emb, self.weight
        if type(emb) is not torch.nn.Embedding or type(self.head) is not torch.nn.Linear:
            return False
        if w is None or self.head.weight is not w:  # not tied
            return False
        if w.dtype != torch.float32 or not w.is_cuda or w.requires_grad:
            return False
        # the module's forward is replaced below: nothing else may depend on it
        return (emb.max_norm is None and not emb.sparse and not emb._forward_pre_hooks
                and "forward" not in emb.__dict__ and not hasattr(emb, "_hf_hook"))

    @torch.no_grad()
    def convert(self):
        """Replace the fp32 storage by fp16 if every value survives the round trip; False
        (nothing changed) otherwise."""
        w = self.weight
        host = torch.empty(w.shape, dtype=torch.float16, pin_memory=True)
        n = w.shape[0]
        block = narrow = None
        for start in range(0, n, self.BLOCK_ROWS):
            block = w.data[start:start + self.BLOCK_ROWS]
            narrow = block.to(torch.float16)
            if not bool((narrow.to(torch.float32) == block).all()):
                return False
            host[start:start + self.BLOCK_ROWS].copy_(narrow)
        device = w.device
        del block, narrow  # views and temporaries of the fp32 storage
        w.data = torch.empty(0, dtype=torch.float16, device=device)  # the fp32 storage goes
        w.data = host.to(device)
        self.emb.__class__ = HalfStoredEmbedding
        return True


def _fp16_autocast():
    return torch.is_autocast_enabled("cuda") and torch.get_autocast_dtype("cuda") == torch.float16


def shrink_tied_embedding(lm):
    """Hold the tied fp32 embedding / head weight of the causal LM `lm` in fp16 when that
    changes no value. Returns True once the weight is held in fp16 by this function, False
    otherwise; the decision is taken under fp16 autocast (before that, False and undecided) and
    kept."""
    decided = getattr(lm, _DECIDED, None)
    if decided is not None:
        return decided
    if not _fp16_autocast():
        return False
    pair = _TiedFp16(lm)
    done = pair.qualifies() and pair.convert()
    setattr(lm, _DECIDED, done)
    return done
