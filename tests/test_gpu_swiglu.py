"""SwiGLU forward / recompute-backward on the GPU against the oracle (F.silu(gate) * up with
CPU autograd), tolerance rtol 2e-3 + atol 2e-3 * max|ref| for fp16 (tests_local/
test_swiglu_recompute.py:37-45)."""

import pytest
import torch

from claudemaxing_amd.swiglu_recompute import swiglu_recompute
from oracle import inputs, swiglu as O
from tests.conftest import banner
from tests.helpers import assert_close, tolerance

pytestmark = pytest.mark.gpu

F16, F32, BF16 = torch.float16, torch.float32, torch.bfloat16
DTYPES = [(F16, F16), (F16, F32), (F32, F16), (F32, F32), (BF16, BF16)]
SHAPES = [(4, 512, 8960), (3, 77, 1001), (1, 1, 8960), (5, 3)]


def make(shape, g_dtype, u_dtype, seed=0):
    gen = torch.Generator().manual_seed(seed)
    gate = (torch.randn(shape, generator=gen) * 3).to(g_dtype)
    up = (torch.randn(shape, generator=gen) * 2).to(u_dtype)
    return gate, up


@pytest.mark.parametrize("g_dtype,u_dtype", DTYPES)
@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("inplace", [False, True])
def test_forward_backward_match(g_dtype, u_dtype, shape, inplace, dev):
    banner(f"swiglu {shape} {g_dtype} {u_dtype} inplace={inplace}")
    gate, up = make(shape, g_dtype, u_dtype)
    out_dtype = torch.promote_types(g_dtype, u_dtype)
    grad = torch.randn(shape, generator=torch.Generator().manual_seed(1)).to(out_dtype)
    r_out, r_dg, r_du = O.forward_backward(gate, up, grad)
    g = gate.to(dev).requires_grad_(True)
    u = up.to(dev).requires_grad_(True)
    gi, ui = (g * 1.0, u * 1.0) if inplace else (g, u)
    out = swiglu_recompute(gi, ui, inplace)
    out.backward(grad.to(dev))
    tol = tolerance(g_dtype, u_dtype)
    assert out.dtype == r_out.dtype and out.shape == r_out.shape
    assert g.grad.dtype == g_dtype and u.grad.dtype == u_dtype
    assert_close(out, r_out, tol, "out")
    assert_close(g.grad, r_dg, tol, "dgate")
    assert_close(u.grad, r_du, tol, "dup")


def test_config3_forward_and_inplace_backward(dev):
    banner("swiglu config 3")
    gate, up, dy = inputs.swiglu(0)
    r_out, r_dg, r_du = O.forward_backward(gate, up, dy)
    g, u = gate.to(dev), up.to(dev)
    gl, ul = g.clone().requires_grad_(True), u.clone().requires_grad_(True)
    gt, ut = gl * 1.0, ul * 1.0
    ptrs = (gt.data_ptr(), ut.data_ptr())
    seen = {}
    gt.register_hook(lambda x: seen.__setitem__("g", x.data_ptr()))
    ut.register_hook(lambda x: seen.__setitem__("u", x.data_ptr()))
    out = swiglu_recompute(gt, ut, True)
    out.backward(dy.to(dev))
    assert (seen["g"], seen["u"]) == ptrs  # gradients written over the input buffers
    assert_close(out, r_out, 2e-3, "out")
    assert_close(gl.grad, r_dg, 2e-3, "dgate")
    assert_close(ul.grad, r_du, 2e-3, "dup")


def test_backward_keeps_only_the_inputs(dev):
    banner("swiglu saved tensors")
    gate, up = make((4, 256, 8960), F16, F16)
    gate, up = gate.to(dev).requires_grad_(), up.to(dev).requires_grad_()
    saved = []
    with torch.autograd.graph.saved_tensors_hooks(lambda t: (saved.append(t.data_ptr()), t)[1],
                                                  lambda t: t):
        swiglu_recompute(gate, up)
    assert sorted(saved) == sorted([gate.data_ptr(), up.data_ptr()])


@pytest.mark.parametrize("inplace", [False, True])
def test_only_one_input_needs_grad(inplace, dev):
    banner(f"swiglu one grad inplace={inplace}")
    gate, up = make((3, 64, 1001), F16, F16)
    grad = torch.randn(gate.shape, generator=torch.Generator().manual_seed(3)).half()
    _, r_dg, r_du = O.forward_backward(gate, up, grad)
    g = gate.to(dev).requires_grad_()
    swiglu_recompute(g, up.to(dev).clone(), inplace).backward(grad.to(dev))
    assert_close(g.grad, r_dg, 2e-3, "dgate")
    u = up.to(dev).requires_grad_()
    swiglu_recompute(gate.to(dev).clone(), u, inplace).backward(grad.to(dev))
    assert_close(u.grad, r_du, 2e-3, "dup")


def test_not_inplace_leaves_inputs_untouched(dev):
    banner("swiglu not inplace")
    gate, up = make((2, 128, 1001), F16, F16)
    g, u = gate.to(dev).requires_grad_(), up.to(dev).requires_grad_()
    swiglu_recompute(g, u, False).backward(torch.ones(gate.shape, device=dev, dtype=F16))
    assert torch.equal(g.detach().cpu(), gate) and torch.equal(u.detach().cpu(), up)


def test_non_contiguous_input(dev):
    banner("swiglu non-contiguous")
    base = (torch.randn(4, 64, 2 * 1001, generator=torch.Generator().manual_seed(4)) * 3).half()
    gate = base[..., :1001]
    up = (torch.randn(4, 64, 1001, generator=torch.Generator().manual_seed(5)) * 2).half()
    out = swiglu_recompute(base.to(dev)[..., :1001], up.to(dev))
    assert_close(out, O.forward(gate, up), 2e-3, "out")


def test_extreme_gate_values(dev):
    banner("swiglu extremes")
    gate = torch.tensor([-1e4, -100.0, -88.0, -20.0, 0.0, -0.0, 20.0, 88.0, 100.0, 1e4,
                         float("inf"), float("-inf")], dtype=F32)
    up = torch.ones_like(gate)
    out = swiglu_recompute(gate.to(dev), up.to(dev))
    ref = O.forward(gate, up)
    assert torch.equal(torch.isnan(out.cpu()), torch.isnan(ref))
    fin = torch.isfinite(ref)
    assert_close(out.cpu()[fin], ref[fin], 1e-4, "extremes")


@pytest.mark.parametrize("dtype", [F16, BF16, F32])
@pytest.mark.parametrize("rows,f", [(1276, 8960), (3, 1000), (1, 8)])
def test_row_kernels_read_the_halves_of_a_merged_product(dtype, rows, f, dev):
    """cm_swiglu_fwd_rows / cm_swiglu_bwd_rows on y = [gate | up] ([rows, 2f], the MLP's merged
    gate/up product): bit-identical to the flat kernels on contiguous copies of the halves, the
    backward in place over y, and within the oracle's tolerance."""
    from claudemaxing_amd import swiglu_recompute as SR

    banner(f"swiglu rows={rows} f={f} {dtype}")
    gen = torch.Generator().manual_seed(7)
    y = (torch.randn(rows, 2 * f, generator=gen) * 3).to(dtype).to(dev)
    grad = torch.randn(rows, f, generator=gen).to(dtype).to(dev)
    gate, up = y[:, :f].contiguous(), y[:, f:].contiguous()
    for round_silu in (True, False):
        out = torch.empty(rows, f, dtype=dtype, device=dev)
        SR._swiglu_fwd_rows(y, f, out, round_silu)
        flat = torch.empty_like(out)
        SR._swiglu_fwd(gate, up, flat, round_silu)
        assert torch.equal(out, flat)
        yb = y.clone()
        SR._swiglu_bwd_rows(grad, yb, f, round_silu)
        dg, du = torch.empty_like(gate), torch.empty_like(up)
        SR._swiglu_bwd(grad, gate, up, dg, du, round_silu)
        assert torch.equal(yb[:, :f], dg) and torch.equal(yb[:, f:], du)
    r_out, r_dg, r_du = O.forward_backward(gate.cpu(), up.cpu(), grad.cpu())
    tol = tolerance(dtype, dtype)
    assert_close(out, r_out, tol, "out")
    assert_close(yb[:, :f], r_dg, tol, "dgate")
    assert_close(yb[:, f:], r_du, tol, "dup")



@pytest.mark.parametrize("dtype", [F16, F32])
def test_row_kernels_honour_a_padded_row_stride(dtype, dev):
    """Rows of the merged product further apart than 2f (a padded buffer): the kernels read and
    write the halves at the row stride, and the padding columns are left alone."""
    from claudemaxing_amd import swiglu_recompute as SR

    banner(f"swiglu rows with a padded stride {dtype}")
    rows, f, pad = 300, 1000, 24
    gen = torch.Generator().manual_seed(8)
    full = (torch.randn(rows, 2 * f + pad, generator=gen) * 3).to(dtype).to(dev)
    y = full[:, :2 * f]
    grad = torch.randn(rows, f, generator=gen).to(dtype).to(dev)
    gate, up = y[:, :f].contiguous(), y[:, f:].contiguous()
    out = torch.empty(rows, f, dtype=dtype, device=dev)
    SR._swiglu_fwd_rows(y, f, out, True)
    flat = torch.empty_like(out)
    SR._swiglu_fwd(gate, up, flat, True)
    assert torch.equal(out, flat)
    before = full[:, 2 * f:].clone()
    SR._swiglu_bwd_rows(grad, y, f, True)
    dg, du = torch.empty_like(gate), torch.empty_like(up)
    SR._swiglu_bwd(grad, gate, up, dg, du, True)
    assert torch.equal(y[:, :f], dg) and torch.equal(y[:, f:], du)
    assert torch.equal(full[:, 2 * f:], before)
