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

import ctypes
import weakref

import torch

from . import _lib, expand
from .gemm import gemm_f32, gemm_f32_supported, split_k_pays
from .nf4 import _BLOCKSIZES, QuantState, _nf4_code, _offset_tensor, dequantize_nf4, quantize_nf4
from .rmsnorm import fp16_copy_of, fp16_grad_copy_of

# ---------------------------------------------------------------------------------------------
# The fused path: NF4 weights expanded inside the GEMM (csrc/nf4_gemm.hip), fp16 compute.


def fused_supported(packed, state):
    """Whether cm_nf4_linear_* takes this weight: an fp16-compute NF4 QuantState on the GPU
    whose rows and columns are multiples of 64 (every Qwen2.5 projection)."""
    if state is None or getattr(state, "quant_type", None) != "nf4" or not packed.is_cuda:
        return False
    shape = getattr(state, "shape", None)
    if shape is None or len(shape) != 2 or shape[0] % 64 or shape[1] % 64:
        return False
    if packed.dtype != torch.uint8 or not packed.is_contiguous() or packed.data_ptr() % 16:
        return False
    if state.blocksize not in _BLOCKSIZES or not state.absmax.is_cuda:
        return False
    if state.code is not None and (state.code.numel() != 16 or state.code.dtype != torch.float32):
        return False
    if state.nested:
        s2 = state.state2
        return (state.absmax.dtype == torch.uint8 and s2.code.dtype == torch.float32
                and s2.absmax.dtype == torch.float32 and s2.blocksize > 0)
    return state.absmax.dtype == torch.float32


def _weight_key(packed, state):
    """What a weight's descriptor is built from: the addresses and versions of its tensors and
    its sizes. Equal keys of one QuantState give the same descriptor."""
    s2 = state.state2 if state.nested else None
    off = state.offset
    return (packed.data_ptr(), state.absmax.data_ptr(), state.absmax._version,
            None if state.code is None else state.code.data_ptr(),
            None if s2 is None else (s2.code.data_ptr(), s2.absmax.data_ptr(),
                                     s2.absmax._version, int(s2.blocksize)),
            (off.data_ptr(), off._version) if torch.is_tensor(off) else off,
            int(state.blocksize), tuple(state.shape))


def _descriptor(packed, state, scale_map=True):
    """(cm_nf4_weight, tensors it points into that must stay alive for the call). With the
    scale map, the descriptor is kept on the QuantState for the next call with the same key
    (the host cost of building one, ~8 us, is paid once per weight version)."""
    key = _weight_key(packed, state) if scale_map else None
    cached = getattr(state, "_cm_descriptor", None) if scale_map else None
    if cached is not None and cached[0] == key:
        return cached[1], cached[2]
    nested = bool(state.nested)
    s2 = state.state2 if nested else None
    code = _nf4_code(packed.device) if state.code is None else state.code
    offset = _offset_tensor(state.offset, packed.device) if nested else None
    smap = _scale_map(packed, state) if scale_map else None
    d = _lib.NF4Weight(packed.data_ptr(), state.absmax.data_ptr(), int(nested), code.data_ptr(),
                       _lib.ptr(s2.code if nested else None),
                       _lib.ptr(s2.absmax if nested else None), _lib.ptr(offset),
                       int(state.blocksize), int(s2.blocksize) if nested else 1,
                       int(state.shape[0]), int(state.shape[1]), _lib.ptr(smap))
    keep = (code, offset, smap)
    if scale_map:
        state._cm_descriptor = (key, d, keep)
    return d, keep


def _scale_map(packed, state):
    """The fp32 block scales of a frozen NF4 weight, [cols / blocksize, rows]
    (cm_nf4_scale_map), computed once per weight version and kept on its QuantState; None when
    the fused kernels take none (blocksize below 64 or not dividing the columns)."""
    rows, cols = int(state.shape[0]), int(state.shape[1])
    bs = int(state.blocksize)
    if bs < 64 or cols % bs or not packed.is_cuda:
        return None
    s2 = state.state2 if state.nested else None
    key = (packed.data_ptr(), state.absmax.data_ptr(), state.absmax._version,
           None if s2 is None else (s2.absmax.data_ptr(), s2.absmax._version))
    cached = getattr(state, "_cm_scale_map", None)
    if cached is not None and cached[0] == key:
        return cached[1]
    smap = torch.empty(rows * cols // bs, dtype=torch.float32, device=packed.device)
    d, keep = _descriptor(packed, state, scale_map=False)
    _lib.call("cm_nf4_scale_map", ctypes.byref(d), smap.data_ptr(), _lib.stream(packed.device))
    del keep
    state._cm_scale_map = (key, smap)
    return smap


def _weights(pairs):
    """(cm_nf4_weight array of the pairs, tensors it points into, {(m, backward): workspace
    bytes}, the pairs' QuantStates as weak references). Kept on the first pair's QuantState,
    keyed by every pair's weight key and checked against the pairs' QuantState objects
    themselves, so a cached array never outlives or mixes up the weights it describes."""
    keys = tuple(_weight_key(p, s) for p, s in pairs)
    cache = getattr(pairs[0][1], "_cm_arrays", None)
    if cache is None:
        cache = pairs[0][1]._cm_arrays = {}
    got = cache.get(keys)
    if got is not None and all(r() is s for r, (_, s) in zip(got[3], pairs)):
        return got
    descs, keep = [], []
    for packed, state in pairs:
        d, k = _descriptor(packed, state)
        descs.append(d)
        keep.append(k)
    got = ((_lib.NF4Weight * len(descs))(*descs), keep, {},
           tuple(weakref.ref(s) for _, s in pairs))
    if len(cache) > 16:  # a few groupings per weight at most; stale versions drop out
        cache.clear()
    cache[keys] = got
    return got


def _plain_weights(pairs):
    """(cm_nf4_weight array of the pairs without the fused GEMMs' scale maps, tensors it points
    into, the QuantStates as weak references): what the expansion kernels read, kept on the first
    pair's QuantState per weight version (as _weights keeps its arrays)."""
    keys = tuple(_weight_key(p, s) for p, s in pairs)
    cache = getattr(pairs[0][1], "_cm_plain_arrays", None)
    if cache is None:
        cache = pairs[0][1]._cm_plain_arrays = {}
    got = cache.get(keys)
    if got is not None and all(r() is s for r, (_, s) in zip(got[2], pairs)):
        return got
    built = [_descriptor(p, s, scale_map=False) for p, s in pairs]
    got = ((_lib.NF4Weight * len(built))(*[d for d, _ in built]), [k for _, k in built],
           tuple(weakref.ref(s) for _, s in pairs))
    if len(cache) > 16:
        cache.clear()
    cache[keys] = got
    return got


def dequantize_group(pairs, outs, checked=False):
    """Expand the NF4 weights `pairs` [(packed, QuantState)] into `outs` (contiguous tensors of
    one dtype on the weights' device, each of its weight's size) with one launch
    (cm_nf4_dequant_group): the values are dequantize_nf4's. `checked`: the caller made the
    outputs so (the checks below are skipped)."""
    if not pairs:
        return
    if len(pairs) != len(outs) or len(pairs) > 8:
        raise ValueError("dequantize_group: one output per weight, at most 8 weights")
    dtype = outs[0].dtype
    for (packed, state), out in zip(pairs, () if checked else outs):
        if (out.dtype != dtype or not out.is_contiguous() or out.device != packed.device
                or out.numel() != int(state.shape[0]) * int(state.shape[1])):
            raise ValueError("dequantize_group: each output must be a contiguous tensor of its "
                             "weight's size, all of one dtype, on the weights' device")
    w = _plain_weights(pairs)[0]
    out_arr = (ctypes.c_void_p * len(outs))(*[o.data_ptr() for o in outs])
    _lib.call("cm_nf4_dequant_group", w, len(pairs), out_arr, _lib.dtype_code(dtype),
              _lib.stream(outs[0].device))


# Products below this many FLOPs take the fused kernel; larger ones expand the weight with the
# dequant kernel and multiply with torch's GEMM. The fused kernel expands every weight element
# once per token tile (256 tokens), at ~4.6 VALU operations per element; the dequant kernel
# expands each element once, and the GEMM then runs at the library's rate. Measured on MI355X
# at 1276 tokens, fused vs dequant + GEMM: k/v projections 21 vs 30 us forward, 16 vs 30 us
# backward (back-to-back calls, launch gaps included); gate+up 122 vs 101 us; down 78 vs 71 us
# forward, 90 vs 48 us backward; the MLP input gradient 191 vs 186 us. The o projection (6
# GFLOP) in the graphed training step's kernel trace: 25.2 vs 23.0 us forward (fp32 output,
# the split-K partial sum included), 32.0 vs 24.5 us backward.
FUSED_MAX_FLOPS = 4.0e9


def fused_pays(m, n, k):
    """Whether the fused kernel is the faster way to multiply m tokens by an [n, k] weight."""
    return 2.0 * m * n * k < FUSED_MAX_FLOPS


def _rows16(t, k):
    """t as fp16 rows [M, k] with a row stride the kernel takes (unit column stride, a multiple
    of 8 elements, 16-byte aligned); copies only when it has to."""
    t2 = t.reshape(-1, k)
    if (t2.dtype != torch.float16 or t2.stride(1) != 1 or t2.stride(0) % 8
            or t2.data_ptr() % 16 or t2.stride(0) < k):
        t2 = t2.to(torch.float16).contiguous()
    return t2


def _workspace(m, weights, n, backward, device):
    """The fp32 partial-sum buffer a split contraction needs (None when the call does not split),
    from torch's caching allocator on the current stream; `weights` is what _weights returned,
    whose dict keeps the byte count per (m, backward)."""
    w, sizes = weights[0], weights[2]
    nbytes = sizes.get((m, backward))
    if nbytes is None:
        nbytes = _lib.load().cm_nf4_linear_workspace_bytes(m, w, n, backward)
        if nbytes < 0:
            raise RuntimeError("cm_nf4_linear_workspace_bytes: invalid weights")
        if len(sizes) > 64:
            sizes.clear()
        sizes[(m, backward)] = nbytes
    return torch.empty(nbytes, dtype=torch.uint8, device=device) if nbytes else None


def nf4_linear_fwd(x16, pairs, biases=None, out_dtype=torch.float16):
    """[x16 @ W_i.T (+ b_i) for (packed_i, state_i) in pairs] in one launch of the fused kernel;
    x16 fp16 [..., K], biases fp16 [N_i] or None, outputs [..., N_i] in out_dtype (fp16, or fp32
    = the fp16 result widened)."""
    k = pairs[0][1].shape[1]
    x2 = _rows16(x16, k)
    m = x2.shape[0]
    outs = [torch.empty(m, st.shape[0], dtype=out_dtype, device=x2.device) for _, st in pairs]
    weights = _weights(pairs)
    w = weights[0]
    n = len(pairs)
    bias_arr = None
    if biases is not None and any(b is not None for b in biases):
        biases = [None if b is None else b.to(torch.float16).contiguous() for b in biases]
        bias_arr = (ctypes.c_void_p * n)(*[_lib.ptr(b) for b in biases])
    out_arr = (ctypes.c_void_p * n)(*[o.data_ptr() for o in outs])
    ldo = (ctypes.c_int64 * n)(*[o.stride(0) for o in outs])
    ws = _workspace(m, weights, n, 0, x2.device)
    _lib.call("cm_nf4_linear_fwd", x2.data_ptr(), x2.stride(0), m, w, n, bias_arr, out_arr, ldo,
              _lib.dtype_code(out_dtype), _lib.ptr(ws), 0 if ws is None else ws.numel(),
              _lib.stream(x2.device))
    lead = x16.shape[:-1]
    return [o.view(*lead, o.shape[1]) for o in outs]


def nf4_linear_bwd(grads, pairs, dx_dtype=torch.float16):
    """sum_i grads_i @ W_i in one launch of the fused kernel, rounded once to fp16 (widened to
    fp32 when dx_dtype is fp32); grads_i [..., N_i] (cast to fp16 when they are not)."""
    k = pairs[0][1].shape[1]
    g2 = [_rows16(g, st.shape[0]) for g, (_, st) in zip(grads, pairs)]
    m = g2[0].shape[0]
    dx = torch.empty(m, k, dtype=dx_dtype, device=g2[0].device)
    weights = _weights(pairs)
    w = weights[0]
    n = len(pairs)
    g_arr = (ctypes.c_void_p * n)(*[g.data_ptr() for g in g2])
    ldg = (ctypes.c_int64 * n)(*[g.stride(0) for g in g2])
    ws = _workspace(m, weights, n, 1, dx.device)
    _lib.call("cm_nf4_linear_bwd", g_arr, ldg, m, w, n, dx.data_ptr(), dx.stride(0),
              _lib.dtype_code(dx_dtype), _lib.ptr(ws), 0 if ws is None else ws.numel(),
              _lib.stream(dx.device))
    return dx.view(*grads[0].shape[:-1], k)


class MatMulNF4(torch.autograd.Function):
    """x @ W.T (+ bias) for a frozen NF4 weight W [out, in], computed in `compute` dtype (x's
    own when None); an optional frozen bias in that dtype. An fp32 x is taken through the fp16
    copy the preceding norm wrote of it when there is one (rmsnorm.fp16_copy_of: the same values
    as x.to(fp16)), else cast. The output is the compute-dtype result, widened to `out_dtype`
    when that is given (an fp32 output of an fp16 product is written in fp32 by the GEMM, without
    the fp16 rounding); the input gradient is returned in x's dtype. With `residual` the result
    is residual + that output (a decoder layer's last add), added by the split-K GEMM's sum launch
    where the product takes it, by torch otherwise; the residual's gradient is the output's.

    In fp16 the weight is expanded inside the GEMM each way (cm_nf4_linear_fwd/bwd); otherwise
    it is expanded by the dequant kernel and multiplied by torch."""

    @staticmethod
    def forward(ctx, x, packed, state, bias=None, compute=None, out_dtype=None, residual=None):
        y = MatMulNF4._product(ctx, x, packed, state, bias, compute, out_dtype, residual)
        return y if residual is None or ctx.residual_added else residual + y

    @staticmethod
    def _product(ctx, x, packed, state, bias, compute, out_dtype, residual):
        ctx.residual_added = False
        compute = compute or x.dtype
        out_dtype = out_dtype or compute
        xc = x
        if x.dtype != compute:
            low = fp16_copy_of(x) if compute == torch.float16 else None
            xc = low if low is not None else x.to(compute)
        ctx.packed, ctx.state, ctx.x_dtype, ctx.compute = packed, state, x.dtype, compute
        ctx.fused = (compute == torch.float16 and out_dtype in (torch.float16, torch.float32)
                     and fused_supported(packed, state)
                     and fused_pays(xc.numel() // max(xc.shape[-1], 1), *state.shape))
        if ctx.fused:
            return nf4_linear_fwd(xc, [(packed, state)], [bias], out_dtype)[0]
        w = expand.take(packed, compute)  # expanded with the rest of its decoder layer
        if w is None:
            w = dequantize_nf4(packed, state, compute)
        if out_dtype == torch.float32 and compute != torch.float32 and xc.is_cuda:
            # the GEMM writes fp32 itself (fp32 sums, no fp16 rounding and no cast launch)
            x2 = xc.reshape(-1, xc.shape[-1])
            if bias is None and split_k_pays(x2.shape[0], w.shape[0], x2.shape[1]) and \
                    gemm_f32_supported(x2.shape[0], w.shape[0], (x2, w)):
                # narrow output, long contraction: split along k; a residual of the output's
                # shape is added by the sum launch
                r2 = None
                if (residual is not None and residual.dtype == torch.float32
                        and residual.is_contiguous()
                        and residual.shape == (*xc.shape[:-1], w.shape[0])):
                    r2 = residual.view(x2.shape[0], w.shape[0])
                y = gemm_f32((x2, w), residual=r2)
                ctx.residual_added = r2 is not None
            else:
                y = (torch.mm(x2, w.t(), out_dtype=torch.float32) if bias is None else
                     torch.addmm(bias.float(), x2, w.t(), out_dtype=torch.float32))
            return y.view(*xc.shape[:-1], w.shape[0])
        return torch.nn.functional.linear(xc, w, bias).to(out_dtype)

    @staticmethod
    def backward(ctx, grad):
        d_res = grad if ctx.needs_input_grad[6] else None
        if not ctx.needs_input_grad[0]:
            return None, None, None, None, None, None, d_res
        low = fp16_grad_copy_of(grad) if ctx.compute == torch.float16 else None
        g = low if low is not None else grad.to(ctx.compute)
        if ctx.fused and ctx.x_dtype in (torch.float16, torch.float32):
            dx = nf4_linear_bwd([g], [(ctx.packed, ctx.state)], ctx.x_dtype)
            return dx, None, None, None, None, None, d_res
        w = expand.take(ctx.packed, g.dtype)
        if w is None:  # the first expansion of a layer's backward expands the layer's group
            w = expand.backward_group(ctx.packed, g.dtype)
        if w is None:
            w = dequantize_nf4(ctx.packed, ctx.state, g.dtype)
        return torch.matmul(g, w).to(ctx.x_dtype), None, None, None, None, None, d_res


def matmul_nf4(x, packed, state, bias=None, compute=None, out_dtype=None, residual=None):
    return MatMulNF4.apply(x, packed, state, bias, compute, out_dtype, residual)


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

    def forward(self, x, residual=None):
        """x W^T (+ bias); with `residual`, residual + that (the add folded into the product's
        last launch where it can be)."""
        return matmul_nf4(x, self.packed, self.quant_state, self._bias_in(self.compute_dtype),
                          self.compute_dtype, self.out_dtype or x.dtype, residual)

    def extra_repr(self):
        return (f"in_features={self.in_features}, out_features={self.out_features}, "
                f"bias={self.bias is not None}, nf4")
