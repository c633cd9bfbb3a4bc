"""The fused rank-16 LoRA adapter on an NF4 base (claudemaxing_amd.lora.NF4LoRA, kernels
csrc/lora_fused.hip) against the unfused path it replaces (LoRABranch with the pack/unpack
kernels, the base NF4Linear, the widening add), both held against an fp32 evaluation of the
same layer with the same dropout mask: output, input gradient and both adapter weight
gradients must be within 2x the unfused path's error (plus a small floor). The adapter's
rounding points are the reference's (solution/lora.py:78-107); only the order of the rank-16
sums differs, so most values agree bit for bit."""

import pytest
import torch

from tests.conftest import banner


def _layer(dev, out_f, seed, in_f=1536):
    from claudemaxing_amd.lora import LoRALinear
    from claudemaxing_amd.nf4_linear import NF4Linear

    g = torch.Generator().manual_seed(seed)
    w = torch.randn(out_f, in_f, generator=g) * 0.02
    b = torch.randn(out_f, generator=g) * 0.1
    base = NF4Linear.from_weight(w.half().float(), bias=b.half().float()).to(dev)
    lin = LoRALinear(base, r=16, alpha=32, dropout=0.05).to(dev)
    with torch.no_grad():
        lin.lora_B.weight.copy_(torch.randn(out_f, 16, generator=g) * 0.02)
    return lin


def _run(lin, x, gout, fused, seed, want_x=True):
    from claudemaxing_amd import lora

    original = lora._nf4_lora_applies
    if not fused:
        lora._nf4_lora_applies = lambda *a: False
    try:
        lin.zero_grad(set_to_none=True)
        xi = x.detach().clone().requires_grad_(want_x)
        torch.manual_seed(seed)  # the same dropout draws for every path
        with torch.autocast("cuda", dtype=torch.float16):
            y = lin(xi)
        y.backward(gout)
    finally:
        lora._nf4_lora_applies = original
    return (y.detach(), xi.grad, lin.lora_A.weight.grad.clone(), lin.lora_B.weight.grad.clone())


def _reference(lin, x, gout, seed):
    """fp32 evaluation with the mask torch draws for the same seed."""
    from claudemaxing_amd.nf4 import dequantize_nf4

    torch.manual_seed(seed)
    _, mask = torch.native_dropout(x, lin.p, True)
    base = lin.base_layer
    w = dequantize_nf4(base.packed, base.quant_state, torch.float32)
    xr = x.detach().clone().requires_grad_()
    a_w = lin.lora_A.weight.detach().clone().requires_grad_()
    b_w = lin.lora_B.weight.detach().clone().requires_grad_()
    xd = xr * mask / (1 - lin.p)
    y = xr @ w.t() + base.bias + ((xd @ a_w.t()) @ b_w.t()) * lin.scaling
    y.backward(gout)
    return y.detach(), xr.grad, a_w.grad, b_w.grad


def _check(name, ours, ref16, ref):
    e_o = float((ours.float() - ref).abs().max())
    e_r = float((ref16.float() - ref).abs().max())
    floor = 2e-3 * max(float(ref.abs().max()), 1e-6)
    print(f"  {name}: |fused - fp32| {e_o:.3e}  |unfused - fp32| {e_r:.3e}  max {float(ref.abs().max()):.3e}")
    assert e_o <= 2 * e_r + floor, (name, e_o, e_r)


@pytest.mark.gpu
@pytest.mark.parametrize("rows,out_f", [(1276, 1536), (1276, 256), (37, 1536)])
def test_fused_adapter_matches(dev, rows, out_f):
    banner(f"fused LoRA adapter rows={rows} out={out_f}")
    lin = _layer(dev, out_f, seed=rows + out_f)
    g = torch.Generator(device=dev).manual_seed(1)
    x = torch.randn(1, rows, 1536, generator=g, device=dev)
    gout = torch.randn(1, rows, out_f, generator=g, device=dev)
    fused = _run(lin, x, gout, True, seed=5)
    unfused = _run(lin, x, gout, False, seed=5)
    ref = _reference(lin, x, gout, seed=5)
    assert fused[0].dtype == torch.float32 and fused[1].dtype == torch.float32
    for name, a, b, c in zip(("out", "dx", "dA", "dB"), fused, unfused, ref):
        _check(name, a, b, c)
    # most outputs agree bit for bit with the unfused path where both run the base product on
    # the fused NF4 GEMM (an fp16 result); above fused_pays' bound the unfused NF4Linear writes
    # its fp32 output straight from the GEMM (no fp16 rounding), so there the two agree to fp16
    # precision of the output's scale
    from claudemaxing_amd.nf4_linear import fused_pays

    same = float((fused[0] == unfused[0]).float().mean())
    print(f"  identical outputs: {100 * same:.1f}%")
    if fused_pays(rows, out_f, 1536):
        assert same > 0.9
    else:
        diff = float((fused[0] - unfused[0]).abs().max())
        assert diff <= 2.0 ** -10 * float(unfused[0].abs().max()), diff


@pytest.mark.gpu
@pytest.mark.parametrize("in_f,out_f", [(896, 896), (896, 128), (2048, 2048), (2048, 256)])
def test_fused_adapter_other_qwen_widths(dev, in_f, out_f):
    """The q and v adapters of Qwen2.5-0.5B (896 -> 896, 128) and 3B (2048 -> 2048, 256)."""
    banner(f"fused LoRA adapter in={in_f} out={out_f}")
    lin = _layer(dev, out_f, seed=in_f + out_f, in_f=in_f)
    g = torch.Generator(device=dev).manual_seed(2)
    x = torch.randn(1, 300, in_f, generator=g, device=dev)
    gout = torch.randn(1, 300, out_f, generator=g, device=dev)
    fused = _run(lin, x, gout, True, seed=6)
    unfused = _run(lin, x, gout, False, seed=6)
    ref = _reference(lin, x, gout, seed=6)
    for name, a, b, c in zip(("out", "dx", "dA", "dB"), fused, unfused, ref):
        _check(name, a, b, c)


@pytest.mark.gpu
def test_fused_adapter_without_input_grad(dev):
    banner("fused LoRA adapter, input without grad (first layer)")
    lin = _layer(dev, 256, seed=3)
    g = torch.Generator(device=dev).manual_seed(2)
    x = torch.randn(1, 100, 1536, generator=g, device=dev)
    gout = torch.randn(1, 100, 256, generator=g, device=dev)
    fused = _run(lin, x, gout, True, seed=9, want_x=False)
    unfused = _run(lin, x, gout, False, seed=9, want_x=False)
    assert fused[1] is None and unfused[1] is None
    torch.testing.assert_close(fused[2], unfused[2], rtol=2e-3, atol=2e-3 * float(unfused[2].abs().max()))
    torch.testing.assert_close(fused[3], unfused[3], rtol=2e-3, atol=2e-3 * float(unfused[3].abs().max()))


@pytest.mark.gpu
@pytest.mark.parametrize("tokens", [1276, 37, 300, 5000])
def test_weight_grads_batch_matches_fp64(tokens, dev):
    """cm_lora_weight_grads (the q and v adapters' four weight gradients in one call) against an
    fp64 evaluation of the same fp16 operands; the same inputs give the same bits."""
    from claudemaxing_amd.lora import _weight_grads

    banner(f"lora weight grads tokens={tokens}")
    g = torch.Generator(device=dev).manual_seed(tokens)
    ga = torch.randn(tokens, 16, generator=g, device=dev).half()
    xd = torch.randn(tokens, 1536, generator=g, device=dev).half()
    gq = torch.randn(tokens, 1536, generator=g, device=dev).half()
    gv = torch.randn(tokens, 256, generator=g, device=dev).half()
    a16 = torch.randn(tokens, 16, generator=g, device=dev).half()
    pairs = [(ga, xd), (gq, a16), (ga, xd[:, :1024]), (gv, a16)]  # the last two: other widths
    out = _weight_grads(pairs)
    assert out is not None and [o.shape for o in out] == [(16, 1536), (1536, 16), (16, 1024),
                                                          (256, 16)]
    for (p, q), o in zip(pairs, out):
        ref = p.double().t() @ q.double()
        err = float((o.double() - ref).abs().max())
        assert err <= 2e-5 * float(ref.abs().max()) + 1e-5, err
    again = _weight_grads(pairs)
    assert all(torch.equal(a, b) for a, b in zip(out, again))


@pytest.mark.gpu
def test_weight_grads_batch_no_tokens(dev):
    from claudemaxing_amd.lora import _weight_grads

    ga = torch.empty(0, 16, device=dev, dtype=torch.float16)
    xd = torch.empty(0, 1536, device=dev, dtype=torch.float16)
    out = _weight_grads([(ga, xd)])
    assert out is not None and torch.count_nonzero(out[0]) == 0


@pytest.mark.gpu
@pytest.mark.parametrize("t", [1276, 37])
def test_multi_adapter_launches_equal_single_ones(dev, t):
    """cm_lora_fused_fwd_multi / cm_lora_fused_bwd1_multi over the q and v adapters of a block
    (widths 1536 and 256, their own masks): every output bit-identical to one call per
    adapter."""
    import ctypes

    from claudemaxing_amd import _lib

    banner(f"lora fused multi-adapter launches t={t}")
    k = 1536
    g = torch.Generator(device=dev).manual_seed(t)
    x = torch.randn(t, k, generator=g, device=dev)
    st = _lib.stream(dev)
    P = ctypes.c_void_p
    ads = []
    for n in (1536, 256):
        ads.append(dict(
            n=n, keep=torch.rand(t, k, generator=g, device=dev) > 0.05,
            a=torch.randn(16, k, generator=g, device=dev) * 0.05,
            b=torch.randn(n, 16, generator=g, device=dev) * 0.05,
            base=torch.randn(t, n, generator=g, device=dev).half(),
            grad=torch.randn(t, n, generator=g, device=dev)))

    def outs_fwd():
        return [dict(out=torch.empty(t, d["n"], device=dev),
                     bits=torch.empty(t * k // 8, dtype=torch.uint8, device=dev),
                     a16=torch.empty(t, 16, dtype=torch.float16, device=dev)) for d in ads]

    single, multi = outs_fwd(), outs_fwd()
    for d, o in zip(ads, single):
        _lib.call("cm_lora_fused_fwd", x.data_ptr(), d["keep"].data_ptr(), d["a"].data_ptr(),
                  d["b"].data_ptr(), d["base"].data_ptr(), o["out"].data_ptr(),
                  o["bits"].data_ptr(), o["a16"].data_ptr(), t, k, d["n"], 16, 1 / 0.95, 2.0, st)

    def arr(vals):
        return (P * len(vals))(*vals)

    _lib.call("cm_lora_fused_fwd_multi", x.data_ptr(), t, k, 16, 1 / 0.95, 2.0, 2,
              arr([d["keep"].data_ptr() for d in ads]), arr([d["a"].data_ptr() for d in ads]),
              arr([d["b"].data_ptr() for d in ads]), arr([d["base"].data_ptr() for d in ads]),
              arr([o["out"].data_ptr() for o in multi]), arr([o["bits"].data_ptr() for o in multi]),
              arr([o["a16"].data_ptr() for o in multi]), (ctypes.c_int * 2)(1536, 256), st)
    for o1, o2 in zip(single, multi):
        for key in o1:
            assert torch.equal(o1[key], o2[key]), key

    def outs_bwd():
        return [dict(gbase=torch.empty(t, d["n"], dtype=torch.float16, device=dev),
                     g16=torch.empty(t, d["n"], dtype=torch.float16, device=dev),
                     ga16=torch.empty(t, 16, dtype=torch.float16, device=dev)) for d in ads]

    single, multi = outs_bwd(), outs_bwd()
    for d, o in zip(ads, single):
        _lib.call("cm_lora_fused_bwd1", d["grad"].data_ptr(), d["b"].data_ptr(),
                  o["gbase"].data_ptr(), o["g16"].data_ptr(), o["ga16"].data_ptr(), t, d["n"],
                  16, 2.0, st)
    _lib.call("cm_lora_fused_bwd1_multi", t, 16, 2.0, 2, arr([d["grad"].data_ptr() for d in ads]),
              arr([d["b"].data_ptr() for d in ads]), arr([o["gbase"].data_ptr() for o in multi]),
              arr([o["g16"].data_ptr() for o in multi]), arr([o["ga16"].data_ptr() for o in multi]),
              (ctypes.c_int * 2)(1536, 256), st)
    for o1, o2 in zip(single, multi):
        for key in o1:
            assert torch.equal(o1[key], o2[key]), key
