"""SwiGLU oracle (torch on the CPU) -- test infrastructure only.

Restates the reference's torch reference, tests_local/test_swiglu_recompute.py:33-34:
F.silu(gate) * up, whose rounding the kernels reproduce (solution/swiglu_recompute.py:14-17):
silu in fp32 rounded to the gate dtype before it meets up, output dtype promote(gate, up);
backward is torch autograd (the product's gradient rounded to the gate dtype before it goes
back through silu). The MLP fast path without that rounding (ROUND_SILU off, fp16 buffers of
an fp32 reference) has its backward in `backward_unrounded`.

What pins it (tests/test_oracle_float.py): silu(x) = x * sigmoid(x) against fp64; the derivative
sig * (1 + g (1 - sig)) against a central difference in fp64.
"""

import torch
import torch.nn.functional as F


def forward(gate, up):
    return F.silu(gate) * up


def forward_backward(gate, up, grad):
    g = gate.detach().clone().requires_grad_(True)
    u = up.detach().clone().requires_grad_(True)
    out = forward(g, u)
    out.backward(grad.to(out.dtype))
    return out.detach(), g.grad, u.grad


def backward_unrounded(gate, up, grad):
    """(d_gate, d_up) in the buffers' dtypes without the gate-dtype rounding of silu."""
    g, u, d = gate.float(), up.float(), grad.float()
    sig = torch.sigmoid(g)
    d_up = d * g * sig
    d_gate = d * u * sig * (1 + g * (1 - sig))
    return d_gate.to(gate.dtype), d_up.to(up.dtype)
