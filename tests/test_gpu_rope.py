"""RoPE forward/backward on the GPU against the oracle (transformers' apply_rotary_pos_emb with
CPU autograd), tolerances of tests_local/test_rope.py:41-43."""

import pytest
import torch

from claudemaxing_amd.rope import rope
from oracle import inputs, rope as O
from tests.conftest import banner
from tests.helpers import assert_close

pytestmark = pytest.mark.gpu

F16, F32, BF16 = torch.float16, torch.float32, torch.bfloat16


def make(b, t, h, kv, d, dtype, seed=0, cos_batch=None):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(b, t, h * d, generator=g).to(dtype).view(b, t, h, d).transpose(1, 2)
    k = torch.randn(b, t, kv * d, generator=g).to(dtype).view(b, t, kv, d).transpose(1, 2)
    pos = torch.arange(t, dtype=F32)[None].expand(cos_batch or b, t)
    inv = 1.0 / (1e6 ** (torch.arange(0, d, 2, dtype=F32) / d))
    emb = torch.cat((pos[..., None] * inv, pos[..., None] * inv), -1)
    return q, k, emb.cos().to(dtype), emb.sin().to(dtype)


@pytest.mark.parametrize("cos_batch", [None, 1])
@pytest.mark.parametrize("dtype", [F32, F16, BF16])
@pytest.mark.parametrize("shape", [(4, 512, 12, 2, 128), (2, 37, 4, 4, 64), (1, 1, 2, 1, 128),
                                   (2, 9, 3, 1, 6)])
def test_forward_backward_match(dtype, shape, cos_batch, dev):
    banner(f"rope {shape} {dtype} cos_batch={cos_batch}")
    q, k, cos, sin = make(*shape, dtype, cos_batch=cos_batch)
    g = torch.Generator().manual_seed(1)
    gq = torch.randn(q.shape, generator=g).to(dtype)
    gk = torch.randn(k.shape, generator=g).to(dtype)
    rq, rk, rdq, rdk = O.forward_backward(q, k, cos, sin, gq, gk)
    tol = {F16: 2e-3, F32: 1e-5, BF16: 1e-2}[dtype]
    qd, kd = q.to(dev).requires_grad_(), k.to(dev).requires_grad_()
    oq, ok = rope(qd, kd, cos.to(dev), sin.to(dev))
    torch.autograd.backward((oq, ok), (gq.to(dev), gk.to(dev)))
    assert oq.dtype == rq.dtype and ok.dtype == rk.dtype
    assert oq.shape == rq.shape and ok.shape == rk.shape
    assert_close(oq, rq, tol, "q")
    assert_close(ok, rk, tol, "k")
    assert_close(qd.grad, rdq, tol, "dq")
    assert_close(kd.grad, rdk, tol, "dk")


def test_config2_packed_positions(dev):
    banner("rope config 2")
    c = inputs.rmsnorm_rope(0)
    cos, sin = O.cos_sin(c["pos"], 128, c["theta"], F16)
    rq, rk, rdq, rdk = O.forward_backward(c["q"], c["k"], cos, sin, c["gq"], c["gk"])
    qp = c["q"].transpose(1, 2).contiguous().to(dev)  # the [1, N, 12, 128] projection layout
    kp = c["k"].transpose(1, 2).contiguous().to(dev)
    qd = qp.transpose(1, 2).requires_grad_()
    kd = kp.transpose(1, 2).requires_grad_()
    oq, ok = rope(qd, kd, cos.to(dev), sin.to(dev))
    torch.autograd.backward((oq, ok), (c["gq"].to(dev), c["gk"].to(dev)))
    assert_close(oq, rq, 2e-3, "q")
    assert_close(ok, rk, 2e-3, "k")
    assert_close(qd.grad, rdq, 2e-3, "dq")
    assert_close(kd.grad, rdk, 2e-3, "dk")


def test_non_contiguous_gradient(dev):
    banner("rope non-contiguous grad")
    q, k, cos, sin = make(2, 64, 4, 2, 128, F32)
    qd, kd = q.to(dev).requires_grad_(), k.to(dev).requires_grad_()
    oq, ok = rope(qd, kd, cos.to(dev), sin.to(dev))
    (oq.transpose(1, 2).sum() + ok.mean()).backward()
    q1, k1 = q.clone().requires_grad_(), k.clone().requires_grad_()
    rq, rk = O.forward(q1, k1, cos, sin)
    (rq.transpose(1, 2).sum() + rk.mean()).backward()
    assert_close(qd.grad, q1.grad, 1e-5, "dq")
    assert_close(kd.grad, k1.grad, 1e-5, "dk")


def test_mixed_dtypes_one_launch_equals_separate(dev):
    """The training step's pair -- fp32 q, fp16 k, fp32 cos/sin -- rotated in one launch each way
    (fp32 outputs forward; fp32 dq and fp16 dk backward): the bits of rotating each tensor alone,
    the fp16 dk being the fp32 gradient's cast, and within the fp32 tolerance of the oracle."""
    banner("rope mixed q fp32 / k fp16, one launch")
    from claudemaxing_amd.rope import _rotate_pair

    q, k, cos, sin = make(1, 1193, 12, 2, 128, F32, seed=4)
    k = k.to(F16)
    g = torch.Generator().manual_seed(5)
    gq = torch.randn(q.shape, generator=g)
    gk = torch.randn(k.shape, generator=g)
    qd, kd = q.to(dev).requires_grad_(), k.to(dev).requires_grad_()
    cd, sd = cos.to(dev), sin.to(dev)
    oq, ok = rope(qd, kd, cd, sd)
    torch.autograd.backward((oq, ok), (gq.to(dev), gk.to(dev)))
    assert (oq.dtype, ok.dtype, qd.grad.dtype, kd.grad.dtype) == (F32, F32, F32, F16)
    aq, _ = _rotate_pair(q.to(dev), None, cd, sd, F32, None, backward=False)
    _, ak = _rotate_pair(None, k.to(dev), cd, sd, None, F32, backward=False)
    bq, _ = _rotate_pair(gq.to(dev), None, cd, sd, F32, None, backward=True)
    _, bk = _rotate_pair(None, gk.to(dev), cd, sd, None, F32, backward=True)
    torch.cuda.synchronize()
    assert torch.equal(oq, aq) and torch.equal(ok, ak)
    assert torch.equal(qd.grad, bq) and torch.equal(kd.grad, bk.to(F16))
    rq, rk, rdq, rdk = O.forward_backward(q, k.float(), cos, sin, gq, gk)
    assert_close(oq, rq, 1e-5, "q")
    assert_close(ok, rk, 1e-5, "k")
    assert_close(qd.grad, rdq, 1e-5, "dq")
    assert_close(kd.grad.float(), rdk, 2e-3, "dk (fp16)")
