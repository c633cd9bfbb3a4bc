"""A frozen NF4 linear layer whose weight is expanded by the HIP dequant kernel.

The reference's 4-bit layers are bitsandbytes' Linear4bit, whose matmul (`matmul_4bit`, the
MatMul4Bit autograd function) dequantizes the weight to the compute dtype, runs `F.linear`, and
in backward dequantizes again for the input gradient; solution/nf4.py:102-130 routes both
dequantizations through its kernel. bitsandbytes is not part of this stack, so this module
provides the same computation directly: `matmul_nf4` (forward dequant + linear, backward
dequant + matmul; the weight is frozen and gets no gradient) and `NF4Linear` (a bias-free
Linear4bit equivalent that casts its input to `compute_dtype` and its output back to the
input's dtype, as Linear4bit does).
"""

import torch

from .nf4 import dequantize_nf4, quantize_nf4


class MatMulNF4(torch.autograd.Function):
    """x @ W.T for a frozen NF4 weight W [out, in]; W is expanded in x's dtype each way."""

    @staticmethod
    def forward(ctx, x, packed, state):
        w = dequantize_nf4(packed, state, x.dtype)
        ctx.packed, ctx.state = packed, state
        return torch.nn.functional.linear(x, w)

    @staticmethod
    def backward(ctx, grad):
        if not ctx.needs_input_grad[0]:
            return None, None, None
        w = dequantize_nf4(ctx.packed, ctx.state, grad.dtype)
        return torch.matmul(grad, w), None, None


def matmul_nf4(x, packed, state):
    return MatMulNF4.apply(x, packed, state)


class NF4Linear(torch.nn.Module):
    """Frozen linear layer stored as NF4 (blocksize 64, double-quantized absmax), with an
    optional frozen bias added in the compute dtype (as Linear4bit adds its bias)."""

    def __init__(self, packed, state, compute_dtype=torch.float16, bias=None):
        super().__init__()
        self.register_buffer("packed", packed, persistent=False)
        self.register_buffer("bias", None if bias is None else bias.detach().clone(),
                             persistent=False)
        self.quant_state = state
        self.compute_dtype = compute_dtype
        self.out_features, self.in_features = state.shape

    @classmethod
    def from_weight(cls, weight, compute_dtype=torch.float16, blocksize=64, bias=None):
        packed, state = quantize_nf4(weight.detach(), blocksize=blocksize,
                                     compress_statistics=True)
        return cls(packed, state, compute_dtype, bias)

    def _apply(self, fn, recurse=True):
        super()._apply(fn, recurse)
        dev = self.packed.device
        if self.quant_state.absmax.device != dev:
            self.quant_state = self.quant_state.to(dev)
        return self

    def forward(self, x):
        out = matmul_nf4(x.to(self.compute_dtype), self.packed, self.quant_state)
        if self.bias is not None:
            out = out + self.bias.to(self.compute_dtype)
        return out.to(x.dtype)

    def extra_repr(self):
        return (f"in_features={self.in_features}, out_features={self.out_features}, "
                f"bias={self.bias is not None}, nf4")
