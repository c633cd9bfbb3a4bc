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

from .nf4 import QuantState, dequantize_nf4, quantize_nf4
from .rmsnorm import fp16_copy_of


class MatMulNF4(torch.autograd.Function):
    """x @ W.T (+ bias) for a frozen NF4 weight W [out, in], computed in `compute` dtype (x's
    own when None) with W expanded in that dtype each way; an optional frozen bias in that
    dtype. An fp32 x is taken through the fp16 copy the preceding norm wrote of it when there
    is one (rmsnorm.fp16_copy_of: the same values as x.to(fp16)), else cast. The output is in
    the compute dtype; the input gradient is returned in x's dtype."""

    @staticmethod
    def forward(ctx, x, packed, state, bias=None, compute=None):
        compute = compute or x.dtype
        xc = x
        if x.dtype != compute:
            low = fp16_copy_of(x) if compute == torch.float16 else None
            xc = low if low is not None else x.to(compute)
        w = dequantize_nf4(packed, state, compute)
        ctx.packed, ctx.state, ctx.x_dtype = packed, state, x.dtype
        return torch.nn.functional.linear(xc, w, bias)

    @staticmethod
    def backward(ctx, grad):
        if not ctx.needs_input_grad[0]:
            return None, None, None, None, None
        w = dequantize_nf4(ctx.packed, ctx.state, grad.dtype)
        return torch.matmul(grad, w).to(ctx.x_dtype), None, None, None, None


def matmul_nf4(x, packed, state, bias=None, compute=None):
    return MatMulNF4.apply(x, packed, state, bias, compute)


class NF4Linear(torch.nn.Module):
    """Frozen linear layer stored as NF4 (blocksize 64, double-quantized absmax), with an
    optional frozen bias added in the compute dtype (as Linear4bit adds its bias). The output is
    in the input's dtype (Linear4bit's rule) unless `out_dtype` names another: a layer whose
    output is added to an fp32 residual stream can hand over fp32 (the same values, widened
    once), which spares torch's mixed-dtype add."""

    def __init__(self, packed, state, compute_dtype=torch.float16, bias=None, out_dtype=None):
        super().__init__()
        self.out_dtype = out_dtype
        self.register_buffer("packed", packed, persistent=False)
        self.register_buffer("bias", None if bias is None else bias.detach().clone(),
                             persistent=False)
        self.quant_state = state
        self.compute_dtype = compute_dtype
        self.out_features, self.in_features = state.shape
        self._bias_c = None  # (version, dtype, bias in the compute dtype)

    @classmethod
    def from_weight(cls, weight, compute_dtype=torch.float16, blocksize=64, bias=None,
                    out_dtype=None):
        packed, state = quantize_nf4(weight.detach(), blocksize=blocksize,
                                     compress_statistics=True)
        return cls(packed, state, compute_dtype, bias, out_dtype)

    def _apply(self, fn, recurse=True):
        super()._apply(fn, recurse)
        dev = self.packed.device
        if self.quant_state.absmax.device != dev:
            self.quant_state = self.quant_state.to(dev)
        return self

    # State dict in bitsandbytes Linear4bit's form: "weight" = the packed bytes [numel/2, 1]
    # uint8, "weight.<field>" = the serialized QuantState (QuantState.as_dict(packed=True)),
    # "bias" when there is one.
    def _save_to_state_dict(self, destination, prefix, keep_vars):
        destination[prefix + "weight"] = self.packed.reshape(-1, 1)
        for k, v in self.quant_state.as_dict(packed=True).items():
            destination[prefix + "weight." + k] = v
        if self.bias is not None:
            destination[prefix + "bias"] = self.bias

    def _load_from_state_dict(self, state_dict, prefix, local_metadata, strict, missing_keys,
                              unexpected_keys, error_msgs):
        key = prefix + "weight"
        if key not in state_dict:
            missing_keys.append(key)
            return
        dev = self.packed.device
        fields = {k[len(key) + 1:]: v for k, v in state_dict.items() if k.startswith(key + ".")}
        state = QuantState.from_dict(fields, dev)
        if tuple(state.shape) != (self.out_features, self.in_features):
            error_msgs.append(f"{key}: shape {tuple(state.shape)} against "
                              f"{(self.out_features, self.in_features)}")
            return
        self.packed = state_dict[key].to(dev, torch.uint8).reshape(-1, 1).contiguous()
        self.quant_state = state
        if prefix + "bias" in state_dict:
            self.bias = state_dict[prefix + "bias"].detach().to(dev).clone()
            self._bias_c = None
        elif self.bias is not None:
            missing_keys.append(prefix + "bias")
        for k in state_dict:
            if k.startswith(prefix) and k != key and not k.startswith(key + ".") \
                    and k != prefix + "bias" and "." not in k[len(prefix):]:
                unexpected_keys.append(k)

    @classmethod
    def from_state_dict(cls, state_dict, prefix="", compute_dtype=torch.float16, out_dtype=None,
                        device=None):
        """An NF4Linear from a bitsandbytes Linear4bit state dict (keys "<prefix>weight",
        "<prefix>weight.<quant_state fields>", optionally "<prefix>bias")."""
        key = prefix + "weight"
        fields = {k[len(key) + 1:]: v for k, v in state_dict.items() if k.startswith(key + ".")}
        state = QuantState.from_dict(fields, device)
        packed = state_dict[key].to(torch.uint8).reshape(-1, 1).contiguous()
        if device is not None:
            packed = packed.to(device)
        bias = state_dict.get(prefix + "bias")
        if bias is not None and device is not None:
            bias = bias.to(device)
        return cls(packed, state, compute_dtype, bias, out_dtype)

    def _bias_in(self, dtype):
        """The frozen bias in `dtype`, converted once per bias version."""
        if self.bias is None:
            return None
        cached = self._bias_c
        key = (self.bias._version, self.bias.data_ptr(), dtype)
        if cached is None or cached[0] != key:
            cached = (key, self.bias.to(dtype))
            self._bias_c = cached
        return cached[1]

    def forward(self, x):
        out = matmul_nf4(x, self.packed, self.quant_state, self._bias_in(self.compute_dtype),
                         self.compute_dtype)
        return out.to(self.out_dtype or x.dtype)

    def extra_repr(self):
        return (f"in_features={self.in_features}, out_features={self.out_features}, "
                f"bias={self.bias is not None}, nf4")
