"""A decoder layer's NF4 weight expansions issued as one launch.

In the training step a decoder layer multiplies four frozen NF4 weights whose products are too
large for the NF4-fused GEMM to pay: the attention's o projection and the MLP's gate, up and
down projections. Each is expanded to fp16 by the dequant kernel right before its product, in
the forward and again in the backward. Those are short launches (6-9 us each at
Qwen2.5-1.5B's shapes, of which the ramp and the drain of a launch are a large part), so the
layer issues them together, through cm_nf4_dequant_group:

* forward: the patched decoder layer calls `expand_layer` first. It expands the weights whose
  products will take the dequant route at this token count (o and down into their own fp16
  weights, gate and up into one [2F, K] weight, the MLP's merged product) in one launch and
  leaves them for `take` / `take_pair`, which the o and down projections' MatMulNF4 and the MLP
  call instead of expanding; the layer calls `drop` at its end.
* backward: the down projection's input gradient is the first expansion of the layer's
  backward. `backward_group`, called there, finds the layer's group (recorded by `expand_layer`)
  and expands down, gate/up and o together the same way, for the MLP's input gradient and then
  the o projection's.

Every weight is expanded by the dequant kernel's own code (the values of dequantize_nf4, bit
for bit), and a consumer that finds nothing left for it expands its weight itself: the values
and the routes are the same with or without the grouping. Everything runs on the caller's
current stream, in order, so a captured step replays it as it runs eagerly.
"""

import weakref

import torch

_READY = {}   # device index -> {key: fp16 weight}; key = packed pointer, or ("pair", gate, up)
_GROUPS = {}  # down projection's packed pointer -> weak reference to its decoder layer


def _nf4_module(m):
    from .nf4_linear import NF4Linear

    return (isinstance(m, NF4Linear) and m.compute_dtype == torch.float16
            and not (m._forward_hooks or m._forward_pre_hooks))


def _single_route(m, tokens):
    """MatMulNF4 expands this layer's weight with the dequant kernel (not the fused GEMM) for
    `tokens` rows in fp16."""
    from .nf4_linear import fused_pays, fused_supported

    if not _nf4_module(m):
        return False
    state = m.quant_state
    return not (fused_supported(m.packed, state) and fused_pays(tokens, *state.shape))


def _pair_route(mlp, tokens, x_dtype):
    """The MLP's recompute takes its merged gate/up product for `tokens` rows of an x_dtype
    input (swiglu_recompute._merged_route), through MLPInputRecompute: a call with gradients
    enabled (the MLP input of a decoder layer with trainable adapters needs its gradient)."""
    from . import swiglu_recompute as SR

    gp, up = getattr(mlp, "gate_proj", None), getattr(mlp, "up_proj", None)
    if not (_nf4_module(gp) and _nf4_module(up)) or gp.bias is not None or up.bias is not None:
        return False
    if not (torch.is_grad_enabled() and SR._frozen(gp) and SR._frozen(up)):
        return False
    return SR._merged_route(tokens, gp.packed.is_cuda, x_dtype, gp, up)


def _issue(dev, singles, pair):
    """Expand `singles` (NF4Linear modules) and `pair` ((gate, up) or None) in one launch; the
    {key: weight} map of the results."""
    from .nf4_linear import dequantize_group

    pairs, outs, ready = [], [], {}
    for m in singles:
        w = torch.empty(m.quant_state.shape, dtype=torch.float16, device=dev)
        pairs.append((m.packed, m.quant_state))
        outs.append(w)
        ready[m.packed.data_ptr()] = w
    if pair is not None:
        gp, up = pair
        f, k = gp.quant_state.shape
        w2 = torch.empty(2 * f, k, dtype=torch.float16, device=dev)
        pairs += [(gp.packed, gp.quant_state), (up.packed, up.quant_state)]
        outs += [w2[:f], w2[f:]]
        ready[("pair", gp.packed.data_ptr(), up.packed.data_ptr())] = w2
    dequantize_group(pairs, outs, checked=True)
    return ready


def _plan(layer, hidden, tokens):
    """(singles, pair, o, down) of the layer for this call: the o / down modules whose products
    take the dequant route, the (gate, up) pair of the merged product or None, and the o and
    down modules. Kept on the layer per (token count, dtype, device, gradient mode, modules): the
    routes depend on nothing else. The backward's group reads the plan of the layer's last
    forward."""
    attn, mlp = getattr(layer, "self_attn", None), getattr(layer, "mlp", None)
    o = getattr(attn, "o_proj", None)
    down = getattr(mlp, "down_proj", None)
    gp, up = getattr(mlp, "gate_proj", None), getattr(mlp, "up_proj", None)
    key = (tokens, hidden.dtype, hidden.device, torch.is_grad_enabled(), id(o), id(down),
           id(gp), id(up))
    cached = layer.__dict__.get("_cm_expand_plan")
    if cached is not None and cached[0] == key:
        return cached[1]
    singles = [m for m in (o, down) if _single_route(m, tokens)]
    pair = (gp, up) if _pair_route(mlp, tokens, hidden.dtype) else None
    plan = (singles, pair, o, down)
    layer.__dict__["_cm_expand_plan"] = (key, plan)
    return plan


def expand_layer(layer, hidden):
    """At the start of a decoder layer's forward on `hidden` (its input, [..., H] on the GPU):
    expand, in one launch, the o / down projections' weights and the merged gate/up weight that
    this call's products will expand, when there are at least two."""
    drop(hidden.device)
    singles, pair, o, down = _plan(layer, hidden, hidden.numel() // max(hidden.shape[-1], 1))
    if len(singles) + (2 if pair else 0) < 2:
        return
    _READY[hidden.device.index] = _issue(hidden.device, singles, pair)
    if down in singles and torch.is_grad_enabled():
        # the backward finds the layer (and its plan: the same routes) from the down weight
        ref = _GROUPS.get(down.packed.data_ptr())
        if ref is None or ref() is not layer:
            if len(_GROUPS) > 1024:  # entries of models that are gone
                _GROUPS.clear()
            _GROUPS[down.packed.data_ptr()] = weakref.ref(layer)


def take(packed, dtype):
    """The fp16 expansion of `packed` left by the group launch, once; None when there is none
    (or `dtype` is not fp16)."""
    ready = _READY.get(packed.device.index)
    if not ready or dtype != torch.float16:
        return None
    return ready.pop(packed.data_ptr(), None)


def take_pair(gate_proj, up_proj):
    """The merged [2F, K] fp16 weight [Wg; Wu] left by the group launch, once; or None."""
    ready = _READY.get(gate_proj.packed.device.index)
    if not ready:
        return None
    return ready.pop(("pair", gate_proj.packed.data_ptr(), up_proj.packed.data_ptr()), None)


def backward_group(packed, dtype):
    """In the backward, for the down projection of a layer whose forward recorded a group: expand
    down, the merged gate/up weight and o in one launch, leave the other two for `take_pair` /
    `take`, and return the down weight; None for any other weight."""
    ref = _GROUPS.get(packed.data_ptr())
    layer = None if ref is None else ref()
    plan = None if layer is None else layer.__dict__.get("_cm_expand_plan")
    if plan is None or dtype != torch.float16:
        return None
    singles, pair, o, down = plan[1]
    if down not in singles or down.packed is not packed:
        return None
    singles = [down] + ([o] if o in singles else [])
    drop(packed.device)
    ready = _issue(packed.device, singles, pair)
    w = ready.pop(packed.data_ptr())
    _READY[packed.device.index] = ready
    return w


def drop(device):
    """Forget what was left on `device` (unused expansions are freed)."""
    _READY.pop(device.index, None)
