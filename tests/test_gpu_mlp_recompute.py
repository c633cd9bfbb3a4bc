"""MLPInputRecompute and the patched Qwen2MLP on their own (the reference's
tests_local/test_swiglu_recompute.py:194-268: the patched MLP against the original, output and
every gradient; frozen projections keep only the MLP input for the backward).

MLPInputRecompute's backward recomputes gate/up and the input gradient by one of five routes
(claudemaxing_amd/swiglu_recompute.py): the NF4-fused GEMM (small products), the merged [2F, K]
weight (large products with an fp32 input gradient: one product each way, the row-strided
SwiGLU kernels on its halves, a k-major split-K input gradient), the transposed NF4 expansion
(fp16 input gradient), the natural NF4 expansion (other dtypes or widths), and autograd
re-running the projections (any other layer). Each route is forced by its natural
condition, checked to be the one taken, and its output and input gradient are compared with

  * an fp32 evaluation of the same layers (the NF4 weights expanded by the CPU oracle, fp32
    products, silu and the gradient by fp32 autograd): the route's error must be within twice
    the error of the stock path (the same layers called through autograd, no recompute) plus
    a small floor;
  * the stock path itself at the reference's tolerance (2e-3 relative to the largest value for
    fp16, 1e-2 for bf16).
"""

import numpy as np
import pytest
import torch

from claudemaxing_amd import swiglu_recompute as SR
from claudemaxing_amd.nf4_linear import NF4Linear
from oracle import nf4 as onf4
from tests.conftest import banner

H, F = 1536, 8960


def nf4_layer(out_f, in_f, seed, compute, dev, out_dtype=None):
    g = torch.Generator().manual_seed(seed)
    w = torch.randn(out_f, in_f, generator=g) * 0.02
    return NF4Linear.from_weight(w, compute_dtype=compute, out_dtype=out_dtype).to(dev)


def oracle_weight(layer):
    """The layer's NF4 weight expanded to fp32 by the CPU oracle."""
    st = layer.quant_state
    s2 = st.state2
    flat = onf4.dequant(layer.packed.cpu().numpy(), st.absmax.cpu().numpy(), nested=True,
                        code2=s2.code.cpu().numpy(), absmax2=s2.absmax.cpu().numpy(),
                        offset=np.float32(st.offset.item() if torch.is_tensor(st.offset)
                                          else st.offset),
                        blocksize=int(st.blocksize), blocksize2=int(s2.blocksize),
                        out_dtype="f32")
    return torch.from_numpy(flat.reshape(tuple(st.shape)))


def fp32_reference(x, wg, wu, grad):
    """silu(x Wg^T) * (x Wu^T) and its input gradient, in fp32 on the CPU."""
    xf = x.detach().float().cpu().requires_grad_(True)
    gate, up = xf @ wg.t(), xf @ wu.t()
    out = torch.nn.functional.silu(gate) * up
    out.backward(grad.float().cpu())
    return out.detach(), xf.grad


def stock(x, gate_proj, up_proj, grad):
    """The layers called through autograd as the unpatched Qwen2MLP calls them (no recompute)."""
    xs = x.detach().clone().requires_grad_(True)
    out = torch.nn.functional.silu(gate_proj(xs)) * up_proj(xs)
    out.backward(grad.to(out.dtype))
    return out.detach(), xs.grad


def routed(x, gate_proj, up_proj, grad, monkeypatch, down_compute=None):
    """MLPInputRecompute's output and input gradient, and the name of the backward route it
    took."""
    taken = []
    for name in ("_dx_fused", "_dx_merged", "_dx_transposed", "_dx_expanded", "_dx_autograd"):
        fn = getattr(SR, name)
        monkeypatch.setattr(SR, name, lambda *a, _f=fn, _n=name: (taken.append(_n), _f(*a))[1])
    xr = x.detach().clone().requires_grad_(True)
    out = SR.MLPInputRecompute.apply(xr, gate_proj, up_proj, down_compute)
    out.backward(grad.to(out.dtype))
    return out.detach(), xr.grad, taken


def err(a, b):
    return float((a.float().cpu() - b.float().cpu()).abs().max())


def check(name, got, stock_v, ref, tol):
    """`got` within twice the stock path's error against fp32 plus tol of the largest value,
    and within tol of the stock path (the reference's comparison)."""
    scale = float(ref.abs().max())
    e_got, e_stock = err(got, ref), err(stock_v, ref)
    assert e_got <= 2 * e_stock + tol * scale, \
        f"{name}: error {e_got:.3g} against fp32, stock path {e_stock:.3g} (max {scale:.3g})"
    s = float(stock_v.float().abs().max())
    torch.testing.assert_close(got.float().cpu(), stock_v.float().cpu(), rtol=tol, atol=tol * s,
                               msg=lambda m: f"{name} vs the stock path: {m}")


# (route, tokens, in_features, compute dtype, x dtype)
ROUTES = [
    ("_dx_fused", 96, H, torch.float16, torch.float32),        # 2.6 GFLOP per product: fused
    ("_dx_fused", 96, H, torch.float16, torch.float16),
    ("_dx_merged", 384, H, torch.float16, torch.float32),      # 10.6 GFLOP, fp32 dx: split-K
    ("_dx_merged", 1276, H, torch.float16, torch.float32),     # the training step's batch
    ("_dx_transposed", 384, H, torch.float16, torch.float16),  # fp16 dx: expanded, transposed
    ("_dx_merged", 384, 1600, torch.float16, torch.float32),   # width not a multiple of 128
    ("_dx_expanded", 384, 1600, torch.float16, torch.float16),  # ... and an fp16 dx
    ("_dx_expanded", 160, H, torch.bfloat16, torch.float32),   # bf16 compute
    ("_dx_expanded", 160, H, torch.bfloat16, torch.bfloat16),
]


@pytest.mark.gpu
@pytest.mark.parametrize("route,tokens,in_f,compute,x_dtype", ROUTES,
                         ids=[f"{r[0][4:]}-{r[1]}x{r[2]}-{str(r[3])[6:]}-x{str(r[4])[6:]}"
                              for r in ROUTES])
def test_nf4_route_against_fp32(route, tokens, in_f, compute, x_dtype, dev, monkeypatch):
    banner(f"MLPInputRecompute {route} tokens={tokens} in={in_f} compute={compute} x={x_dtype}")
    gp = nf4_layer(F, in_f, 1, compute, dev)
    upp = nf4_layer(F, in_f, 2, compute, dev)
    g = torch.Generator().manual_seed(3)
    x = (torch.randn(tokens, in_f, generator=g) * 2).to(x_dtype).to(dev)
    grad = torch.randn(tokens, F, generator=g).to(dev)
    out, dx, taken = routed(x, gp, upp, grad, monkeypatch)
    assert taken == [route], taken
    assert out.dtype == x_dtype and dx.dtype == x_dtype
    s_out, s_dx = stock(x, gp, upp, grad)
    r_out, r_dx = fp32_reference(x, oracle_weight(gp), oracle_weight(upp),
                                 grad.to(out.dtype))
    tol = 1e-2 if torch.bfloat16 in (compute, x_dtype) else 2e-3
    check(f"{route} output", out, s_out, r_out, tol)
    check(f"{route} input gradient", dx, s_dx, r_dx, tol)


@pytest.mark.gpu
def test_fp16_output_for_a_4bit_down_projection(dev, monkeypatch):
    """With a 4-bit fp16 down projection after it, the output is written in fp16 directly, the
    dtype that projection computes in."""
    banner("MLPInputRecompute fp16 output for a 4-bit down projection")
    gp, upp = nf4_layer(F, H, 4, torch.float16, dev), nf4_layer(F, H, 5, torch.float16, dev)
    g = torch.Generator().manual_seed(6)
    x = torch.randn(384, H, generator=g).to(dev)
    grad = torch.randn(384, F, generator=g).to(dev)
    out, dx, taken = routed(x, gp, upp, grad, monkeypatch, down_compute=torch.float16)
    assert taken == ["_dx_merged"] and out.dtype == torch.float16
    assert dx.dtype == torch.float32
    s_out, s_dx = stock(x, gp, upp, grad)
    r_out, r_dx = fp32_reference(x, oracle_weight(gp), oracle_weight(upp), grad)
    check("output", out, s_out, r_out, 2e-3)
    check("input gradient", dx, s_dx, r_dx, 2e-3)


@pytest.mark.gpu
@pytest.mark.parametrize("autocast", [False, True])
def test_dense_projections_take_autograd(autocast, dev, monkeypatch):
    """Frozen dense projections (the reference's test_frozen_mlp_recomputes_gate_and_up): the
    autograd route, under the forward's autocast state, against the stock path and fp32."""
    banner(f"MLPInputRecompute dense projections autocast={autocast}")
    torch.manual_seed(7)
    dt = torch.float32 if autocast else torch.float16
    gp = torch.nn.Linear(256, 704, bias=False).to(dev, dt).requires_grad_(False)
    upp = torch.nn.Linear(256, 704, bias=False).to(dev, dt).requires_grad_(False)
    x = (torch.randn(4, 96, 256) * 2).to(dev, dt)
    grad = torch.randn(4, 96, 704).to(dev)
    with torch.autocast("cuda", dtype=torch.float16, enabled=autocast):
        out, dx, taken = routed(x, gp, upp, grad, monkeypatch)
        s_out, s_dx = stock(x, gp, upp, grad)
    assert taken == ["_dx_autograd"]
    assert out.dtype == s_out.dtype and dx.dtype == x.dtype
    r_out, r_dx = fp32_reference(x, gp.weight.float().cpu(), upp.weight.float().cpu(),
                                 grad.to(out.dtype))
    check("dense output", out, s_out, r_out, 2e-3)
    check("dense input gradient", dx, s_dx, r_dx, 2e-3)


@pytest.mark.gpu
def test_only_the_input_is_kept(dev):
    """The memory contract: the NF4 routes keep one tensor for the backward, the fp16 copy of
    the MLP input (no gate/up activations); the dense route keeps the input itself."""
    banner("MLPInputRecompute saved tensors")
    gp, upp = nf4_layer(F, H, 8, torch.float16, dev), nf4_layer(F, H, 9, torch.float16, dev)
    x = torch.randn(300, H, device=dev, requires_grad=True)
    kept = []
    with torch.autograd.graph.saved_tensors_hooks(lambda t: (kept.append(t), t)[1],
                                                  lambda t: t):
        SR.MLPInputRecompute.apply(x, gp, upp, None)
    assert len(kept) == 1, [tuple(t.shape) for t in kept]
    assert kept[0].dtype == torch.float16 and kept[0].shape == x.shape
    assert torch.equal(kept[0], x.detach().half())

    dense_g = torch.nn.Linear(256, 704, bias=False).to(dev).requires_grad_(False)
    dense_u = torch.nn.Linear(256, 704, bias=False).to(dev).requires_grad_(False)
    xd = torch.randn(4, 96, 256, device=dev, requires_grad=True)
    kept = []
    with torch.autograd.graph.saved_tensors_hooks(lambda t: (kept.append(t.data_ptr()), t)[1],
                                                  lambda t: t):
        SR.MLPInputRecompute.apply(xd, dense_g, dense_u, None)
    assert kept == [xd.data_ptr()]


def _small_mlp(dev):
    from transformers.models.qwen2 import modeling_qwen2 as modeling

    cfg = modeling.Qwen2Config(hidden_size=256, intermediate_size=704, hidden_act="silu")
    torch.manual_seed(10)
    return modeling.Qwen2MLP(cfg).to(dev).half()


@pytest.mark.gpu
def test_patched_mlp_matches_the_original(dev, monkeypatch):
    """Trainable projections (the reference's test_patched_qwen2_mlp_matches_the_original): the
    patched forward runs the recomputing activation between the layer's own projections; output,
    input gradient and every parameter gradient match the original forward."""
    banner("patched Qwen2MLP, trainable projections")
    from transformers.models.qwen2 import modeling_qwen2 as modeling

    saved = modeling.Qwen2MLP.forward
    original = getattr(saved, "_original", saved)
    monkeypatch.setattr(modeling.Qwen2MLP, "forward", saved)  # put back after the test
    SR.patch_qwen2_mlp_recompute()
    mlp = _small_mlp(dev)
    x = (torch.randn(4, 96, 256, device=dev) * 2).half()
    grad = torch.randn(4, 96, 256, device=dev).half()
    xr = x.clone().requires_grad_(True)
    ref = original(mlp, xr)
    ref.backward(grad)
    ref_grads = {n: p.grad.clone() for n, p in mlp.named_parameters()}
    mlp.zero_grad()
    xn = x.clone().requires_grad_(True)
    out = mlp(xn)
    out.backward(grad)
    tol = dict(rtol=2e-3, atol=2e-3 * float(ref.abs().max()))
    assert out.dtype == ref.dtype
    torch.testing.assert_close(out, ref.detach(), **tol)
    torch.testing.assert_close(xn.grad, xr.grad, rtol=2e-3, atol=2e-3 * float(xr.grad.abs().max()))
    for n, p in mlp.named_parameters():
        torch.testing.assert_close(p.grad, ref_grads[n], rtol=2e-3,
                                   atol=2e-3 * float(ref_grads[n].abs().max()), msg=n)


@pytest.mark.gpu
def test_patched_nf4_mlp_matches_the_original(dev, monkeypatch):
    """The 4-bit layout of the training step: NF4 gate/up/down (fp16 compute), fp32 input, fp16
    autocast. The patched forward takes MLPInputRecompute (checked), hands the 4-bit down
    projection its fp16 input, and matches the original forward's output and input gradient."""
    banner("patched Qwen2MLP, NF4 projections")
    from transformers.models.qwen2 import modeling_qwen2 as modeling

    saved = modeling.Qwen2MLP.forward
    original = getattr(saved, "_original", saved)
    monkeypatch.setattr(modeling.Qwen2MLP, "forward", saved)  # put back after the test
    SR.patch_qwen2_mlp_recompute()
    mlp = _small_mlp(dev).float()
    for name in ("gate_proj", "up_proj", "down_proj"):
        lin = getattr(mlp, name)
        setattr(mlp, name, NF4Linear.from_weight(lin.weight.detach().cpu()).to(dev))
    mlp.requires_grad_(False)
    calls = []
    real = SR.MLPInputRecompute.apply
    monkeypatch.setattr(SR.MLPInputRecompute, "apply",
                        lambda *a: (calls.append(len(a)), real(*a))[1])
    x = (torch.randn(3, 80, 256, device=dev) * 2)
    grad = torch.randn(3, 80, 256, device=dev)
    xr = x.clone().requires_grad_(True)
    with torch.autocast("cuda", dtype=torch.float16):
        ref = original(mlp, xr)
    ref.backward(grad.to(ref.dtype))
    xn = x.clone().requires_grad_(True)
    with torch.autocast("cuda", dtype=torch.float16):
        out = mlp(xn)
    out.backward(grad.to(out.dtype))
    assert calls == [4]
    torch.testing.assert_close(out.float(), ref.float(), rtol=2e-3,
                               atol=2e-3 * float(ref.abs().max()))
    torch.testing.assert_close(xn.grad, xr.grad, rtol=2e-3,
                               atol=2e-3 * float(xr.grad.abs().max()))
