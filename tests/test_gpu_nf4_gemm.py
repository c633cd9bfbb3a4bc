"""The NF4-fused GEMM (cm_nf4_linear_fwd / cm_nf4_linear_bwd) on the GPU.

Checks, in order of strength:
  - the weight expansion inside the GEMM is bit-exact with the CPU oracle's dequantization: with an
    identity matrix on the token side every output is one weight element times 1 (no sums), so
    the forward returns W^T and the backward W, bit for bit;
  - products against an fp64 evaluation of x16 @ W16^T with W16 = the oracle's fp16 weight, within
    half an fp16 ulp of the exact value plus an fp32-summation allowance (|x| @ |W|^T * 2^-20),
    which catches a dropped stage, a wrong block scale or a transposed operand;
  - several weights in one launch give the same bits as one launch per weight;
  - the autograd layer (NF4Linear) through the fused path against the fp32 evaluation.
"""

import pytest
import torch

from claudemaxing_amd.nf4 import quantize_nf4
from claudemaxing_amd.nf4_linear import (NF4Linear, fused_supported, nf4_linear_bwd,
                                          nf4_linear_fwd)
from tests.conftest import banner
from tests.helpers import assert_bits_equal, assert_close
from tests.test_gpu_nf4 import oracle_of

pytestmark = pytest.mark.gpu


def make_weight(n, k, seed, nested=True, scale=0.02):
    w = torch.randn(n, k, generator=torch.Generator().manual_seed(seed)) * scale
    packed, state = quantize_nf4(w, 64, nested)
    w16 = oracle_of(packed, state, torch.float16)  # the exact fp16 expansion (CPU oracle)
    return packed, state, w16


def to_dev(packed, state, dev):
    return packed.to(dev), state.to(dev)


def half_ulp(v):
    """Half an fp16 ulp of |v| (normal range; the subnormal spacing below it)."""
    a = v.abs().clamp(min=2.0 ** -14)
    return torch.exp2(torch.floor(torch.log2(a)) - 11)


def check_product(out, x16, ws, what, bias=None, trans=False, grads=None):
    """out (fp16 or widened fp32) against the fp64 product, within half an fp16 ulp plus the
    fp32 summation allowance."""
    if trans:
        exact = sum(g.double().cpu() @ w.double() for g, w in zip(grads, ws))
        mag = sum(g.double().abs().cpu() @ w.double().abs() for g, w in zip(grads, ws))
    else:
        exact = x16.double().cpu() @ ws.double().t()
        mag = x16.double().abs().cpu() @ ws.double().abs().t()
        if bias is not None:
            exact = exact + bias.double().cpu()
            mag = mag + bias.double().abs().cpu()
    got = out.double().cpu().reshape(exact.shape)
    bound = half_ulp(exact) + mag * 2.0 ** -20 + 1e-7
    excess = (got - exact).abs() - bound
    worst = excess.max().item()
    assert worst <= 0, f"{what}: error exceeds the bound by {worst:.3e} at {excess.argmax().item()}"
    # and the rounding itself: the output is an fp16 number
    assert torch.equal(got.to(torch.float16).double(), got), f"{what}: not fp16-valued"


# (256, 1536): 256-row tiles with a split contraction; (1536, 128): unsplit; (192, 640): the
# general kernel forward; (384, 576): 128-row tiles forward, the general kernel backward
IDENTITY_SHAPES = [(256, 1536), (1536, 128), (192, 640), (384, 576)]


@pytest.mark.parametrize("nested", [True, False])
@pytest.mark.parametrize("n,k", IDENTITY_SHAPES)
def test_forward_expansion_is_bitexact(n, k, nested, dev):
    banner(f"nf4_gemm fwd identity n={n} k={k} nested={nested}")
    packed, state, w16 = make_weight(n, k, 1, nested)
    eye = torch.eye(k, dtype=torch.float16, device=dev)
    (y,) = nf4_linear_fwd(eye, [to_dev(packed, state, dev)])
    torch.cuda.synchronize()
    assert_bits_equal(y, w16.t().contiguous(), f"fwd identity {n}x{k}")


@pytest.mark.parametrize("nested", [True, False])
@pytest.mark.parametrize("n,k", IDENTITY_SHAPES)
def test_backward_expansion_is_bitexact(n, k, nested, dev):
    banner(f"nf4_gemm bwd identity n={n} k={k} nested={nested}")
    packed, state, w16 = make_weight(n, k, 2, nested)
    eye = torch.eye(n, dtype=torch.float16, device=dev)
    dx = nf4_linear_bwd([eye], [to_dev(packed, state, dev)])
    torch.cuda.synchronize()
    assert_bits_equal(dx, w16, f"bwd identity {n}x{k}")


def test_two_weights_expand_bitexact_both_ways(dev):
    banner("nf4_gemm two weights identity")
    p1, s1, w1 = make_weight(128, 256, 3)
    p2, s2, w2 = make_weight(320, 256, 4)
    pairs = [to_dev(p1, s1, dev), to_dev(p2, s2, dev)]
    eye = torch.eye(256, dtype=torch.float16, device=dev)
    y1, y2 = nf4_linear_fwd(eye, pairs)
    assert_bits_equal(y1, w1.t().contiguous(), "fwd w1")
    assert_bits_equal(y2, w2.t().contiguous(), "fwd w2")
    # backward with g1 = [I 0], g2 = [0 I] picks rows of each weight in turn
    m = 128 + 320
    g1 = torch.zeros(m, 128, dtype=torch.float16, device=dev)
    g2 = torch.zeros(m, 320, dtype=torch.float16, device=dev)
    g1[:128] = torch.eye(128, dtype=torch.float16, device=dev)
    g2[128:] = torch.eye(320, dtype=torch.float16, device=dev)
    dx = nf4_linear_bwd([g1, g2], pairs)
    assert_bits_equal(dx, torch.cat([w1, w2]), "bwd concatenated")


SHAPES = [(1536, 1536), (256, 1536), (8960, 1536), (1536, 8960)]


@pytest.mark.parametrize("m", [1, 37, 1276, 2048])
@pytest.mark.parametrize("n,k", SHAPES)
def test_forward_matches_exact_product(m, n, k, dev):
    banner(f"nf4_gemm fwd m={m} n={n} k={k}")
    packed, state, w16 = make_weight(n, k, 5)
    x16 = torch.randn(m, k, generator=torch.Generator().manual_seed(6)).half()
    bias = (torch.randn(n, generator=torch.Generator().manual_seed(7)) * 0.1).half()
    pd = to_dev(packed, state, dev)
    (y,) = nf4_linear_fwd(x16.to(dev), [pd], [bias.to(dev)])
    (y32,) = nf4_linear_fwd(x16.to(dev), [pd], [bias.to(dev)], torch.float32)
    torch.cuda.synchronize()
    assert y.dtype == torch.float16 and y32.dtype == torch.float32
    check_product(y, x16, w16, f"fwd {m}x{n}x{k}", bias)
    assert_bits_equal(y32.half(), y, "fp32 output = the fp16 output widened")
    # and against the path it replaces (dequant + hipBLASLt) within fp16 tolerance
    ref = torch.nn.functional.linear(x16.to(dev), w16.to(dev), bias.to(dev))
    assert_close(y, ref, 2e-3, f"fwd vs F.linear {m}x{n}x{k}")


@pytest.mark.parametrize("m", [1, 37, 1276])
@pytest.mark.parametrize("n,k", SHAPES)
def test_backward_matches_exact_product(m, n, k, dev):
    banner(f"nf4_gemm bwd m={m} n={n} k={k}")
    packed, state, w16 = make_weight(n, k, 8)
    g = torch.randn(m, n, generator=torch.Generator().manual_seed(9)).half()
    pd = to_dev(packed, state, dev)
    dx = nf4_linear_bwd([g.to(dev)], [pd])
    dx32 = nf4_linear_bwd([g.to(dev)], [pd], torch.float32)
    torch.cuda.synchronize()
    check_product(dx, None, [w16], f"bwd {m}x{n}x{k}", trans=True, grads=[g])
    assert_bits_equal(dx32.half(), dx, "fp32 dx = the fp16 dx widened")


# the projections of Qwen2.5-0.5B (hidden 896, kv 128, intermediate 4864) and 7B (3584, 512,
# 18944): weight extents that are multiples of 128 but not of 256, and long contractions
OTHER_QWEN = [(896, 896), (128, 896), (4864, 896), (896, 4864),
              (3584, 3584), (512, 3584), (18944, 3584), (3584, 18944)]


@pytest.mark.parametrize("m", [37, 300])
@pytest.mark.parametrize("n,k", OTHER_QWEN)
def test_other_qwen_shapes(m, n, k, dev):
    banner(f"nf4_gemm fwd+bwd m={m} n={n} k={k}")
    packed, state, w16 = make_weight(n, k, 14)
    pd = to_dev(packed, state, dev)
    x16 = torch.randn(m, k, generator=torch.Generator().manual_seed(15)).half()
    (y,) = nf4_linear_fwd(x16.to(dev), [pd], [None])
    g = torch.randn(m, n, generator=torch.Generator().manual_seed(16)).half()
    dx = nf4_linear_bwd([g.to(dev)], [pd])
    torch.cuda.synchronize()
    check_product(y, x16, w16, f"fwd {m}x{n}x{k}")
    check_product(dx, None, [w16], f"bwd {m}x{n}x{k}", trans=True, grads=[g])


def test_mlp_shapes_two_weights(dev):
    banner("nf4_gemm gate+up fwd, dgate Wg + dup Wu bwd, m=1276")
    m, f, h = 1276, 8960, 1536
    pg, sg, wg = make_weight(f, h, 10)
    pu, su, wu = make_weight(f, h, 11)
    pairs = [to_dev(pg, sg, dev), to_dev(pu, su, dev)]
    x16 = torch.randn(m, h, generator=torch.Generator().manual_seed(12)).half()
    gate, up = nf4_linear_fwd(x16.to(dev), pairs)
    (gate1,) = nf4_linear_fwd(x16.to(dev), pairs[:1])
    (up1,) = nf4_linear_fwd(x16.to(dev), pairs[1:])
    assert_bits_equal(gate, gate1, "gate in a two-weight launch")
    assert_bits_equal(up, up1, "up in a two-weight launch")
    check_product(up, x16, wu, "up")
    dg = torch.randn(m, f, generator=torch.Generator().manual_seed(13)).half()
    du = torch.randn(m, f, generator=torch.Generator().manual_seed(14)).half()
    dx = nf4_linear_bwd([dg.to(dev), du.to(dev)], pairs, torch.float32)
    torch.cuda.synchronize()
    check_product(dx, None, [wg, wu], "dgate Wg + dup Wu", trans=True, grads=[dg, du])


def test_three_weights_with_biases_and_strided_input(dev, monkeypatch):
    banner("nf4_gemm q/k/v in one launch, strided x")
    import claudemaxing_amd.nf4_linear as NL

    m, h = 517, 1536
    ws = [make_weight(n, h, 20 + i) for i, n in enumerate((1536, 256, 256))]
    pairs = [to_dev(p, s, dev) for p, s, _ in ws]
    biases = [(torch.randn(n, generator=torch.Generator().manual_seed(30 + i)) * 0.1).half()
              for i, n in enumerate((1536, 256, 256))]
    big = torch.randn(m, h + 64, generator=torch.Generator().manual_seed(31)).half().to(dev)
    x = big[:, 32:32 + h]  # row stride 1600 elements, 64-byte aligned start
    outs = nf4_linear_fwd(x, pairs, [b.to(dev) for b in biases])
    # single launches without a split contraction sum every output in the same order (stages in
    # sequence, the same MFMA substeps), whatever the tile shape: the same bits
    monkeypatch.setattr(NL, "_workspace", lambda *a: None)
    for i, ((p, s, w16), b, o) in enumerate(zip(ws, biases, outs)):
        (single,) = nf4_linear_fwd(x.contiguous(), [pairs[i]], [b.to(dev)])
        assert_bits_equal(o, single, f"weight {i} of three")
        check_product(o, x.cpu(), w16, f"weight {i}", b)


def test_unsplit_without_workspace(dev, monkeypatch):
    banner("nf4_gemm split contraction vs no workspace")
    import claudemaxing_amd.nf4_linear as NL

    m, n, k = 1276, 1536, 8960  # down_proj: split in two slices when the workspace is there
    packed, state, w16 = make_weight(n, k, 60)
    pd = to_dev(packed, state, dev)
    x16 = torch.randn(m, k, generator=torch.Generator().manual_seed(61)).half()
    bias = (torch.randn(n, generator=torch.Generator().manual_seed(62)) * 0.1).half()
    (split,) = nf4_linear_fwd(x16.to(dev), [pd], [bias.to(dev)])
    monkeypatch.setattr(NL, "_workspace", lambda *a: None)
    (whole,) = nf4_linear_fwd(x16.to(dev), [pd], [bias.to(dev)])
    torch.cuda.synchronize()
    check_product(split, x16, w16, "split", bias)
    check_product(whole, x16, w16, "unsplit", bias)


def test_scale_map_is_the_decoded_absmax(dev):
    banner("nf4 scale map")
    from claudemaxing_amd.nf4_linear import _scale_map
    from oracle import nf4 as O

    for nested in (True, False):
        packed, state, _ = make_weight(384, 1536, 70, nested)
        pd, sd = to_dev(packed, state, dev)
        smap = _scale_map(pd, sd).cpu().view(1536 // 64, 384)
        kw = {}
        if nested:
            kw = dict(code2=state.state2.code.numpy(), absmax2=state.state2.absmax.numpy(),
                      offset=state.offset.numpy().reshape(()), blocksize2=state.state2.blocksize)
        ref = O.block_scales(state.absmax.numpy(), nested, **kw).reshape(384, 1536 // 64)
        assert_bits_equal(smap, torch.from_numpy(ref).t().contiguous(), f"nested={nested}")
        assert _scale_map(pd, sd) is _scale_map(pd, sd)  # computed once per weight


def test_supported_predicate(dev):
    packed, state, _ = make_weight(256, 1536, 40)
    assert fused_supported(*to_dev(packed, state, dev))
    assert not fused_supported(packed, state)  # on the CPU
    p2, s2, _ = make_weight(96, 128, 41)  # 96 rows: not a multiple of 64
    assert not fused_supported(*to_dev(p2, s2, dev))


@pytest.mark.parametrize("out_dtype", [None, torch.float32])
@pytest.mark.parametrize("x_dtype", [torch.float16, torch.float32])
def test_nf4linear_autograd_fused(x_dtype, out_dtype, dev):
    banner(f"NF4Linear fused autograd x={x_dtype} out={out_dtype}")
    torch.manual_seed(50)
    w = torch.randn(1536, 1536) * 0.02
    bias = torch.randn(1536) * 0.1
    layer = NF4Linear.from_weight(w, bias=bias, out_dtype=out_dtype).to(dev)
    x = torch.randn(3, 97, 1536, device=dev, dtype=x_dtype, requires_grad=True)
    y = layer(x)
    assert y.dtype == (out_dtype or x_dtype)
    gy = torch.randn_like(y)
    y.backward(gy)
    w16 = oracle_of(layer.packed.cpu(), layer.quant_state.to("cpu"), torch.float16).to(dev)
    x16 = x.detach().half().float()
    ref = x16 @ w16.float().t() + layer.bias.half().float()
    assert_close(y, ref, 2e-3, "NF4Linear forward")
    gref = gy.half().float() @ w16.float()
    assert x.grad.dtype == x_dtype
    assert_close(x.grad, gref, 2e-3, "NF4Linear input gradient")
