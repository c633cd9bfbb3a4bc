"""Seeded CPU generators of the benchmark configurations -- test infrastructure only.

The shapes and distributions are those of BASELINE.json's configs (Qwen2.5-1.5B sizes): NF4
weight [8960,1536] N(0,0.02) blocksize 64 double-quantized; 4 packed rows of U[128,512] tokens,
hidden 1536, 12/2 heads of 128, theta 1e6; SwiGLU [2048,8960]; LM head hidden [2048,1536] and
tied weight [151936,1536] with 10% ignored labels. Everything is drawn on the CPU with
torch.Generator so the GPU run and the oracle see the same values.
"""

import torch

H, F, V, HD, NQ, NKV = 1536, 8960, 151936, 128, 12, 2


def gen(seed):
    return torch.Generator().manual_seed(seed)


def rmsnorm_rope(seed=0, lengths=None, w_dtype=torch.float32):
    """Config 2: x [N,1536] fp16 N(0,1); norm weight U(0.5,1.5) with 5% of channels 1e-4;
    q [1,12,N,128] / k [1,2,N,128] strided views of projection outputs; positions restarting
    per row; cos/sin fp16; incoming grads N(0,1)."""
    g = gen(seed)
    if lengths is None:
        lengths = torch.randint(128, 513, (4,), generator=g).tolist()
    n = sum(lengths)
    x = torch.randn(n, H, generator=g).to(torch.float16)
    w = torch.rand(H, generator=g) + 0.5
    tiny = torch.randperm(H, generator=g)[: round(0.05 * H)]
    w[tiny] = 1e-4
    w = w.to(w_dtype)
    dy = torch.randn(n, H, generator=g)
    qp = torch.randn(1, n, NQ * HD, generator=g).to(torch.float16)
    kp = torch.randn(1, n, NKV * HD, generator=g).to(torch.float16)
    q = qp.view(1, n, NQ, HD).transpose(1, 2)
    k = kp.view(1, n, NKV, HD).transpose(1, 2)
    pos = torch.cat([torch.arange(length) for length in lengths])
    gq = torch.randn(1, NQ, n, HD, generator=g).to(torch.float16)
    gk = torch.randn(1, NKV, n, HD, generator=g).to(torch.float16)
    return dict(lengths=lengths, n=n, x=x, w=w, dy=dy, q=q, k=k, pos=pos, gq=gq, gk=gk,
                eps=1e-6, theta=1e6)


def swiglu(seed=0, rows=2048, cols=F):
    g = gen(seed)
    gate = torch.randn(rows, cols, generator=g).to(torch.float16)
    up = torch.randn(rows, cols, generator=g).to(torch.float16)
    dy = torch.randn(rows, cols, generator=g).to(torch.float16)
    return gate, up, dy


def nf4_weight(seed=0, rows=F, cols=H, std=0.02):
    g = gen(seed)
    return torch.randn(rows, cols, generator=g) * std


def lm_head(seed=0, n=2048, vocab=V, hidden=H, ignore=0.1):
    g = gen(seed)
    h = torch.randn(n, hidden, generator=g).to(torch.float16)
    w = (torch.randn(vocab, hidden, generator=g) * 0.02).to(torch.float16)
    t = torch.randint(0, vocab, (n,), generator=g)
    t[torch.rand(n, generator=g) < ignore] = -100
    return h, w, t
