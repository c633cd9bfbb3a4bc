"""Fused LM-head cross-entropy oracle (torch on the CPU) -- test infrastructure only.

Restates the base path the reference's fused head reproduces (tests_local/test_lm_head_loss.py:
66-86; solution/lm_head_loss.py:108-160, 192-254): logits z = fp16(h16 @ w16^T) with fp32
accumulation (fp16 autocast); per row lse = logsumexp(z), loss = label ? lse - z[t] : 0,
entropy = lse - sum softmax(z) z, correct = label and (first argmax of z) == t; the hidden-state
gradient of sum(loss) is (softmax(z) - onehot(t)) @ w for labelled rows and 0 otherwise, which
the caller scales by grad_loss / denominator. Labels of -100 are ignored.

What pins it (tests/test_oracle_float.py): loss against torch's F.cross_entropy(reduction=
'none'), entropy against -sum(softmax * log_softmax), the gradient against autograd of
F.cross_entropy on the fp32 logits, the argmax against a pure-Python scan on tiny rows; the
reference's own invariants (rows without labels give zero loss and zero grad but positive
entropy, test_lm_head_loss.py:192-203; chunking does not change the result, 182-189).
"""

import torch

IGNORE_INDEX = -100


def head(h16, w16, target, want_grad=True, rows_per_block=256):
    """(loss [N], entropy [N], correct [N] int32, grad [N,H] fp32 or None, argmax [N], z16 or
    None). Rows are processed in blocks so big vocabularies stay within memory."""
    n = h16.shape[0]
    loss = torch.zeros(n)
    entropy = torch.zeros(n)
    correct = torch.zeros(n, dtype=torch.int32)
    best = torch.zeros(n, dtype=torch.int64)
    grad = torch.zeros(n, h16.shape[1]) if want_grad else None
    w32 = w16.float()
    for r0 in range(0, n, rows_per_block):
        r1 = min(n, r0 + rows_per_block)
        z = (h16[r0:r1].float() @ w32.t()).to(torch.float16).float()
        t = target[r0:r1]
        lbl = t != IGNORE_INDEX
        lse = torch.logsumexp(z, dim=-1)
        p = torch.softmax(z, dim=-1)
        zt = z.gather(1, t.clamp(min=0)[:, None]).squeeze(1)
        loss[r0:r1] = torch.where(lbl, lse - zt, torch.zeros_like(lse))
        entropy[r0:r1] = lse - (p * z).sum(-1)
        b = z.argmax(-1)  # first index of the maximum
        best[r0:r1] = b
        correct[r0:r1] = (lbl & (b == t)).to(torch.int32)
        if want_grad:
            d = p.clone()
            d[torch.arange(r1 - r0), t.clamp(min=0)] -= lbl.float()
            d[~lbl] = 0
            grad[r0:r1] = d @ w32
        del z, p
    return loss, entropy, correct, grad, best


def grad_f64(h16, w16, target, rows_per_block=256):
    """The hidden-state gradient of sum(loss) evaluated in float64 from the fp16 logits:
    (softmax(z) - onehot(t)) @ w per labelled row, 0 otherwise. In float64 the label's p_t - 1
    keeps its relative precision even for p_t within 1e-7 of 1, where the fp32 evaluation of
    `head` (like any fp32 softmax) quantises it to steps of 2^-24."""
    n = h16.shape[0]
    out = torch.zeros(n, h16.shape[1], dtype=torch.float64)
    w32, w64 = w16.float(), w16.double()
    for r0 in range(0, n, rows_per_block):
        r1 = min(n, r0 + rows_per_block)
        z = (h16[r0:r1].float() @ w32.t()).to(torch.float16).double()
        t = target[r0:r1]
        lbl = t != IGNORE_INDEX
        d = torch.softmax(z, dim=-1)
        d[torch.arange(r1 - r0), t.clamp(min=0)] -= lbl.double()
        d[~lbl] = 0
        out[r0:r1] = d @ w64
        del z, d
    return out


def top2_gap(h16, w16, rows_per_block=256):
    """Per row, the gap between the largest and second-largest fp16 logit (0 on ties). Rows
    whose gap is at most one fp16 ulp of the maximum have an argmax that depends on the last
    bit of fp32 accumulation order."""
    n = h16.shape[0]
    gaps = torch.zeros(n)
    ulps = torch.zeros(n)
    w32 = w16.float()
    for r0 in range(0, n, rows_per_block):
        r1 = min(n, r0 + rows_per_block)
        z = (h16[r0:r1].float() @ w32.t()).to(torch.float16).float()
        top = z.topk(2, dim=-1).values
        gaps[r0:r1] = top[:, 0] - top[:, 1]
        m = top[:, 0].abs().clamp(min=2.0 ** -14)
        ulps[r0:r1] = 2.0 ** (torch.floor(torch.log2(m)) - 10)
    return gaps, ulps
