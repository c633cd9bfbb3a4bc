"""Pins the floating-point oracles (oracle/rmsnorm.py, rope.py, swiglu.py, lm_head.py) against
the installed transformers modules, torch's textbook routines, fp64 evaluations and closed
forms -- not against a retyped copy of their own formulas."""

import pytest
import torch
import torch.nn.functional as F

from oracle import lm_head as OL
from oracle import rmsnorm as ON
from oracle import rope as OR
from oracle import swiglu as OS

modeling = pytest.importorskip("transformers.models.qwen2.modeling_qwen2")


# ---- RMSNorm ----------------------------------------------------------------------------------
@pytest.mark.parametrize("x_dtype,w_dtype", [(torch.float16, torch.float32),
                                             (torch.float16, torch.float16),
                                             (torch.float32, torch.float32)])
def test_rmsnorm_equals_installed_qwen2_rmsnorm(x_dtype, w_dtype):
    g = torch.Generator().manual_seed(0)
    x = (torch.randn(3, 40, 1536, generator=g) * 3).to(x_dtype)
    w = (1 + 0.5 * torch.randn(1536, generator=g)).to(w_dtype)
    norm = modeling.Qwen2RMSNorm(1536, eps=1e-6)
    norm.weight.data = w.clone()
    ref = norm(x)
    ours = ON.forward(x, w, 1e-6)
    assert ours.dtype == ref.dtype == torch.promote_types(x_dtype, w_dtype)
    assert torch.equal(ours, ref)


def test_rmsnorm_backward_against_fp64():
    g = torch.Generator().manual_seed(1)
    x = torch.randn(8, 256, generator=g) * 3
    w = torch.rand(256, generator=g) + 0.5
    gr = torch.randn(8, 256, generator=g)
    _, dx, dw, rstd = ON.forward_backward(x, w, 1e-6, gr, need_dw=True)
    x64 = x.double().requires_grad_(True)
    w64 = w.double().requires_grad_(True)
    (w64 * x64 * torch.rsqrt(x64.pow(2).mean(-1, keepdim=True) + 1e-6)).backward(gr.double())
    torch.testing.assert_close(dx.double(), x64.grad, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(dw.double(), w64.grad, rtol=1e-5, atol=1e-4)
    torch.testing.assert_close(rstd.double(), 1 / x.double().pow(2).mean(-1).add(1e-6).sqrt(),
                               rtol=1e-6, atol=0)


# ---- RoPE -------------------------------------------------------------------------------------
def _qk(dtype, b=2, t=37, hq=4, hk=2, d=64, seed=0):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(b, t, hq * d, generator=g).to(dtype).view(b, t, hq, d).transpose(1, 2)
    k = torch.randn(b, t, hk * d, generator=g).to(dtype).view(b, t, hk, d).transpose(1, 2)
    return q, k


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_rope_equals_installed_apply_rotary_pos_emb(dtype):
    q, k = _qk(dtype)
    cos, sin = OR.cos_sin(torch.arange(37), 64, 1e6, dtype)
    rq, rk = modeling.apply_rotary_pos_emb(q, k, cos, sin)
    oq, ok = OR.forward(q, k, cos, sin)
    assert torch.equal(oq, rq) and torch.equal(ok, rk)


def test_rope_cos_sin_equal_qwen2_rotary_embedding():
    cfg = modeling.Qwen2Config(hidden_size=1536, num_attention_heads=12,
                               num_key_value_heads=2, rope_theta=1e6,
                               max_position_embeddings=1024)
    rot = modeling.Qwen2RotaryEmbedding(cfg)
    pos = torch.cat([torch.arange(5), torch.arange(9)])[None]
    x = torch.zeros(1, pos.shape[1], 128, dtype=torch.float16)
    cos, sin = rot(x, pos)
    oc, os_ = OR.cos_sin(pos[0], 128, 1e6, torch.float16)
    torch.testing.assert_close(oc.float(), cos.float(), rtol=0, atol=1e-3)
    torch.testing.assert_close(os_.float(), sin.float(), rtol=0, atol=1e-3)


def test_rope_rotation_properties_fp64():
    q, k = _qk(torch.float64, t=9, d=32)
    cos, sin = OR.cos_sin(torch.arange(9), 32, 1e6, torch.float64)
    oq, ok, dq, dk = OR.forward_backward(q, k, cos, sin, q, k)
    h = 16
    # each (i, i + d/2) pair is rotated: its norm is unchanged
    n_in = q[..., :h] ** 2 + q[..., h:] ** 2
    n_out = oq[..., :h] ** 2 + oq[..., h:] ** 2
    torch.testing.assert_close(n_out, n_in)
    # backward is the transposed rotation: applied to the forward output it gives the input
    _, _, back_q, back_k = OR.forward_backward(q, k, cos, sin, oq, ok)
    torch.testing.assert_close(back_q, q)
    torch.testing.assert_close(back_k, k)


# ---- SwiGLU -----------------------------------------------------------------------------------
def test_silu_against_fp64_sigmoid():
    x = torch.linspace(-30, 30, 10001)
    up = torch.ones_like(x)
    ref = (x.double() / (1 + torch.exp(-x.double()))).float()
    torch.testing.assert_close(OS.forward(x, up), ref, rtol=1e-6, atol=1e-7)


def test_swiglu_gradient_against_central_difference():
    g = torch.linspace(-8, 8, 401, dtype=torch.float64)
    u = torch.linspace(1.5, -2.5, 401, dtype=torch.float64)
    _, dg, du = OS.forward_backward(g, u, torch.ones_like(g))
    eps = 1e-6
    f = lambda a, b: a * torch.sigmoid(a) * b  # noqa: E731
    torch.testing.assert_close(dg, (f(g + eps, u) - f(g - eps, u)) / (2 * eps), rtol=1e-6,
                               atol=1e-8)
    torch.testing.assert_close(du, g * torch.sigmoid(g), rtol=1e-12, atol=1e-12)
    ddg, ddu = OS.backward_unrounded(g.float(), u.float(), torch.ones(401))
    torch.testing.assert_close(ddg.double(), dg, rtol=1e-5, atol=1e-6)


def test_swiglu_rounds_silu_to_the_gate_dtype():
    """F.silu on fp16 returns fp16: the product sees the rounded silu."""
    g = torch.tensor([0.3337], dtype=torch.float16)
    u = torch.tensor([3.0], dtype=torch.float16)
    s16 = F.silu(g)
    assert s16.dtype == torch.float16
    assert torch.equal(OS.forward(g, u), s16 * u)


# ---- LM head ----------------------------------------------------------------------------------
def _head_case(n=48, v=301, h=32, seed=0):
    g = torch.Generator().manual_seed(seed)
    h16 = torch.randn(n, h, generator=g).half()
    w16 = (torch.randn(v, h, generator=g) * h ** -0.5).half()
    t = torch.randint(0, v, (n,), generator=g)
    t[::4] = -100
    return h16, w16, t


def test_head_loss_entropy_grad_against_torch_routines():
    h16, w16, t = _head_case()
    loss, ent, corr, grad, best = OL.head(h16, w16, t)
    z = (h16.float() @ w16.float().t()).half().float().requires_grad_(True)
    ce = F.cross_entropy(z, t, ignore_index=-100, reduction="none")
    torch.testing.assert_close(loss, ce.detach(), rtol=1e-6, atol=1e-6)
    logp = F.log_softmax(z.detach(), -1)
    torch.testing.assert_close(ent, -(logp.exp() * logp).sum(-1), rtol=1e-5, atol=1e-6)
    ce.sum().backward()
    torch.testing.assert_close(grad, z.grad @ w16.float(), rtol=1e-5, atol=1e-6)
    assert torch.equal(corr, ((z.detach().argmax(-1) == t) & (t != -100)).int())


def test_head_argmax_is_the_first_maximum():
    h16 = torch.ones(1, 8).half()
    w16 = torch.zeros(6, 8).half()
    w16[2] = 1.0
    w16[4] = 1.0  # tie with row 2: the first index wins
    loss, ent, corr, grad, best = OL.head(h16, w16, torch.tensor([4]))
    assert best.item() == 2 and corr.item() == 0
    loss, ent, corr, grad, best = OL.head(h16, w16, torch.tensor([2]))
    assert corr.item() == 1


def test_head_unlabelled_rows_and_row_blocking():
    """Rows without labels give zero loss and zero grad but positive entropy
    (tests_local/test_lm_head_loss.py:192-203); blocking rows does not change the result."""
    h16, w16, t = _head_case(n=40)
    t[:10] = -100
    a = OL.head(h16, w16, t, rows_per_block=256)
    b = OL.head(h16, w16, t, rows_per_block=7)
    for x, y in zip(a, b):
        assert torch.equal(x, y)
    assert torch.all(a[0][:10] == 0) and torch.all(a[3][:10] == 0) and torch.all(a[1] > 0)


def test_head_single_row_by_hand():
    """A 1-row, 3-column case computed with math.log / math.exp."""
    import math

    h16 = torch.tensor([[1.0, 0.0]]).half()
    w16 = torch.tensor([[0.5, 0.0], [2.0, 0.0], [-1.0, 0.0]]).half()
    loss, ent, corr, grad, best = OL.head(h16, w16, torch.tensor([1]))
    z = [0.5, 2.0, -1.0]
    lse = math.log(sum(math.exp(v) for v in z))
    p = [math.exp(v - lse) for v in z]
    assert abs(loss.item() - (lse - 2.0)) < 1e-6
    assert abs(ent.item() - (lse - sum(pi * zi for pi, zi in zip(p, z)))) < 1e-6
    g0 = sum((p[i] - (i == 1)) * w16[i, 0].item() for i in range(3))
    assert abs(grad[0, 0].item() - g0) < 1e-6 and corr.item() == 1


def _brute_top2(row):
    """Largest and second-largest entries by a plain scan (a tie gives gap 0) and the fp16
    spacing of the largest |value|'s binade: 2^(e - 11) for |x| = m 2^e with m in [0.5, 1)
    (math.frexp), 2^-24 in the subnormal range below 2^-14."""
    import math

    vals = sorted(float(v) for v in row)
    top, second = vals[-1], vals[-2]
    if abs(top) < 2.0 ** -14:
        return top - second, 2.0 ** -24
    _, e = math.frexp(abs(top))
    return top - second, 2.0 ** (e - 11)


def test_top2_gap_against_brute_force():
    """OL.top2_gap decides which argmax mismatches the GPU tests excuse: pinned on tiny rows
    whose fp16 logits are set directly (identity hidden states, z = W^T): exact ties, a gap of
    one ulp, negative maxima, maxima at power-of-two boundaries and in the fp16 subnormal
    range."""
    rows = [
        [1.0, 1.0, 0.5, -2.0],                  # exact tie
        [1.0, 1.0 - 2 ** -11, 0.0, 0.0],        # one ulp below 1 (ulp above 1 is 2^-10)
        [-3.0, -3.5, -4.0, -5.0],               # all negative
        [2.0, 1.0, 0.25, 0.0],                  # power-of-two maximum
        [2.0 ** -15, 2.0 ** -16, 0.0, -1.0],    # subnormal maximum: ulp 2^-24
        [-0.0, -1e-3, -2.0, -65504.0],          # maximum -0
        [65504.0, 65504.0, 1.0, 0.0],           # fp16 max, tied
        [7.0, -7.5, 6.9, 6.875],                # gap smaller than the row's spread
    ]
    n = len(rows)
    w16 = torch.tensor(rows).t().contiguous().half()  # [V=4, H=n]
    h16 = torch.eye(n).half()
    gaps, ulps = OL.top2_gap(h16, w16)
    for r, row in enumerate(rows):
        z = [float(torch.tensor(v).half()) for v in row]
        gap, ulp = _brute_top2(z)
        assert gaps[r].item() == gap, (r, gaps[r].item(), gap)
        assert ulps[r].item() == ulp, (r, ulps[r].item(), ulp)
    assert gaps[0] == 0 and gaps[6] == 0 and ulps[4] == 2.0 ** -24 and ulps[6] == 32.0


def test_head_grad_f64_against_float64_autograd():
    """grad_f64 against autograd of F.cross_entropy in float64 on the same fp16 logits,
    including a row whose label holds all but ~1e-9 of the probability."""
    h16, w16, t = _head_case(n=24, v=97, h=16, seed=3)
    h16[5] = 0
    h16[5, 0] = 8.0
    w16[:, 0] = 0
    w16[40, 0] = 3.0  # row 5: z_40 = 24 against 0 elsewhere, p_40 = 1 - ~4e-9
    t[5] = 40
    ours = OL.grad_f64(h16, w16, t)
    z = (h16.float() @ w16.float().t()).half().double().requires_grad_(True)
    F.cross_entropy(z, t, ignore_index=-100, reduction="sum").backward()
    ref = z.grad @ w16.double()
    torch.testing.assert_close(ours, ref, rtol=1e-12, atol=1e-15)
    assert 0 < ref[5].abs().max() < 1e-6  # a tiny, nonzero row survives in float64
    assert torch.all(ours[t == -100] == 0)
