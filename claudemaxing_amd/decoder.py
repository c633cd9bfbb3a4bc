"""Qwen2's decoder layer with its residual adds fused into its RMSNorms (gfx950).

transformers' Qwen2DecoderLayer.forward (modeling_qwen2.py) runs

    residual = h;  h = input_layernorm(h);  h = self_attn(h);  h = residual + h
    residual = h;  h = post_attention_layernorm(h);  h = mlp(h);  h = residual + h

and autograd adds the two gradients of each residual (the norm's and the bypass's) in torch, after
which the projection that produced the layer input casts the sum to fp16. The reference leaves
this layer alone (it patches the norm, solution/rmsnorm.py:224-246, the MLP and the attention);
each of those torch adds and casts is one more launch of a few microseconds on a 1.2k-token
batch. `patch_qwen2_decoder_residual` runs the same arithmetic as

    y, residual = norm_pass(h)                  one launch forward; backward: the norm's gradient
                                                plus the bypass's, and its fp16 copy, one launch
    h = self_attn(y)
    y, h = add_norm(residual, h)                residual + h and its norm, one launch each way
    h = mlp(y, residual=h)                      the package's MLP adds h in its down projection's
                                                last launch (the split-K GEMM's slice sum)

with every add the same fp32 add (so the layer's outputs and gradients are the bits of the unfused
layer with the same kernels). The projections take the fp16 copies through
rmsnorm.fp16_grad_copy_of.

It applies where the norms are the package's (patch_qwen2_rmsnorm installed, no hooks on the norm
modules) and take the kernels, on an fp32 residual stream; any other call runs the original.
"""

import torch

from . import expand
from ._patching import install, tagged
from .rmsnorm import _kernel_covers, add_norm, norm_pass


def _mlp_takes_residual(mlp):
    """The MLP's forward is the package's (which takes `residual`) and no hook would see the
    extra argument."""
    return (tagged(type(mlp).forward, "mlp_recompute")
            and not (mlp._forward_hooks or mlp._forward_pre_hooks))


def _norms_fusable(layer, hidden):
    """Both norms of `layer` are Qwen2RMSNorm modules without hooks, the package's norm forward is
    installed, and the kernels cover an fp32 CUDA residual stream of this width."""
    from transformers.models.qwen2 import modeling_qwen2

    cls = getattr(modeling_qwen2, "Qwen2RMSNorm", None)
    if cls is None or not tagged(cls.forward, "rmsnorm"):
        return False
    if not (torch.is_tensor(hidden) and hidden.is_cuda and hidden.dtype == torch.float32):
        return False
    for norm in (layer.input_layernorm, layer.post_attention_layernorm):
        if (type(norm) is not cls or norm._forward_hooks or norm._forward_pre_hooks
                or not _kernel_covers(hidden, norm.weight)):
            return False
    return True


def patch_qwen2_decoder_residual():
    """Qwen2DecoderLayer.forward (class-level, idempotent): the fused residual layer where
    `_norms_fusable` holds and the attention output has the stream's shape, the original
    forward otherwise."""
    from transformers.models.qwen2 import modeling_qwen2

    def build(stock):
        def forward(self, hidden_states, attention_mask=None, position_ids=None,
                    past_key_values=None, use_cache=False, position_embeddings=None, **kwargs):
            if not _norms_fusable(self, hidden_states):
                return stock(self, hidden_states, attention_mask=attention_mask,
                             position_ids=position_ids, past_key_values=past_key_values,
                             use_cache=use_cache, position_embeddings=position_embeddings,
                             **kwargs)
            n1, n2 = self.input_layernorm, self.post_attention_layernorm
            expand.expand_layer(self, hidden_states)  # the layer's NF4 expansions, one launch
            y, residual = norm_pass(hidden_states, n1.weight, n1.variance_epsilon)
            attn, _ = self.self_attn(hidden_states=y, attention_mask=attention_mask,
                                     position_ids=position_ids, past_key_values=past_key_values,
                                     use_cache=use_cache, position_embeddings=position_embeddings,
                                     **kwargs)
            if (torch.is_tensor(attn) and attn.shape == residual.shape and attn.is_cuda
                    and attn.dtype in (torch.float32, torch.float16, torch.bfloat16)):
                y, h = add_norm(residual, attn, n2.weight, n2.variance_epsilon)
            else:
                h = residual + attn
                y = n2(h)
            out = self.mlp(y, residual=h) if _mlp_takes_residual(self.mlp) else h + self.mlp(y)
            expand.drop(hidden_states.device)
            return out

        return forward

    install(getattr(modeling_qwen2, "Qwen2DecoderLayer", None), "forward", "decoder_residual",
            build)
