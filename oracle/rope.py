"""RoPE oracle (torch on the CPU) -- test infrastructure only.

Restates transformers' apply_rotary_pos_emb / rotate_half (modeling_qwen2.py:105-135), which
the reference's test compares against (tests_local/test_rope.py:21-25): q * cos + rotate_half(q)
* sin with cos/sin unsqueezed at dim 1. The backward of that (autograd) is the transposed
rotation the kernel computes (solution/rope.py:35-40). cos/sin follow Qwen2RotaryEmbedding
(modeling_qwen2.py:51-102): inv_freq = 1 / theta^(arange(0, d, 2) / d), freqs = pos * inv_freq,
emb = cat(freqs, freqs), cos/sin in fp32 then cast to the q dtype.

What pins it (tests/test_oracle_float.py): equality with the installed transformers
apply_rotary_pos_emb; the rotation's norm preservation per pair and the inverse property
(backward of forward with the same angles is the identity) in fp64.
"""

import torch


def rotate_half(x):
    x1 = x[..., : x.shape[-1] // 2]
    x2 = x[..., x.shape[-1] // 2:]
    return torch.cat((-x2, x1), dim=-1)


def forward(q, k, cos, sin):
    c, s = cos.unsqueeze(1), sin.unsqueeze(1)
    return q * c + rotate_half(q) * s, k * c + rotate_half(k) * s


def forward_backward(q, k, cos, sin, gq, gk):
    q1 = q.detach().clone().requires_grad_(True)
    k1 = k.detach().clone().requires_grad_(True)
    oq, ok = forward(q1, k1, cos, sin)
    torch.autograd.backward((oq, ok), (gq.to(oq.dtype), gk.to(ok.dtype)))
    return oq.detach(), ok.detach(), q1.grad, k1.grad


def cos_sin(positions, head_dim, theta, dtype):
    """cos/sin [1, T, head_dim] for a 1-D tensor of positions, as Qwen2RotaryEmbedding."""
    inv = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.int64).float() / head_dim))
    freqs = positions.float()[:, None] * inv[None, :]
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos().to(dtype)[None], emb.sin().to(dtype)[None]
