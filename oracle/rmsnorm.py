"""RMSNorm oracle (torch on the CPU, fp32 arithmetic) -- test infrastructure only.

Restates the reference's own torch reference, tests_local/test_rmsnorm.py:32-38 (the body of
transformers' Qwen2RMSNorm.forward, modeling_qwen2.py:238-253): the input is upcast to fp32,
variance = mean(x^2), normed = x * rsqrt(variance + eps) rounded back to the input dtype, then
multiplied by the weight, output dtype promote(x, w). Backward is torch autograd through the
same ops, which is what the kernel (solution/rmsnorm.py:51-91) reproduces: gn = round_x(dy * w),
dx = round_x((gn - n * mean(gn * n)) * rstd) with the unrounded normalised value n.

What pins it (tests/test_oracle_float.py): bit equality with the installed
transformers Qwen2RMSNorm on CPU; dx against an fp64 autograd evaluation of the same formula.
"""

import torch


def forward(x, weight, eps):
    input_dtype = x.dtype
    h = x.to(torch.float32)
    variance = h.pow(2).mean(-1, keepdim=True)
    h = h * torch.rsqrt(variance + eps)
    return weight * h.to(input_dtype)


def forward_backward(x, weight, eps, grad, need_dw=False):
    """(out, dx, dw or None, rstd [rows]) with torch autograd on the CPU."""
    xr = x.detach().clone().requires_grad_(True)
    wr = weight.detach().clone().requires_grad_(need_dw)
    out = forward(xr, wr, eps)
    out.backward(grad.to(out.dtype))
    with torch.no_grad():
        rstd = torch.rsqrt(x.float().pow(2).mean(-1) + eps).reshape(-1)
    return out.detach(), xr.grad, (wr.grad if need_dw else None), rstd
