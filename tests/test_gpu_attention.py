"""The training forward's attention (claudemaxing_amd/attention.py) on the GPU.

The packed causal attention kernels (cm_attn_fwd / cm_attn_bwd) are held against an fp32
reference of the same attention, computed row by row from the same fp16-rounded q/k/v
(softmax(q k^T * scale) v with the causal mask, gradients by autograd in fp32), and against
transformers' stock sdpa attention with the packed block-diagonal causal mask (the reference's
path, solution/lm_head_loss.py:332-336 + solution/attention.py:332-373): the kernels' error
against fp32 must be within 2x stock fp16 SDPA's own error plus a small absolute floor. Also:
bit-identical repeated backward passes, a HIP-graph replay, fp32 inputs under fp16 autocast
(the training step's case), and the reference's grouped SDPA on a general boolean mask."""

import pytest
import torch

from tests.conftest import banner


class _Module(torch.nn.Module):
    num_key_value_groups = 6
    is_causal = True
    training = True


def _inputs(dev, n, seed, dtype=torch.float16, heads=12, groups=2):
    g = torch.Generator(device=dev).manual_seed(seed)
    q = torch.randn(1, heads, n, 128, generator=g, device=dev).to(dtype).requires_grad_()
    k = torch.randn(1, groups, n, 128, generator=g, device=dev).to(dtype).requires_grad_()
    v = torch.randn(1, groups, n, 128, generator=g, device=dev).to(dtype).requires_grad_()
    do = torch.randn(1, n, heads, 128, generator=g, device=dev).half()
    return q, k, v, do


def _bounds(lengths):
    b = [0]
    for n in lengths:
        b.append(b[-1] + n)
    return tuple(b)


def _packed_mask(lengths, dev):
    from claudemaxing_amd.attention import ROWS_ATTR, PackedRows

    row = torch.cat([torch.full((n,), i) for i, n in enumerate(lengths)]).to(dev)
    col = torch.cat([torch.arange(n) for n in lengths]).to(dev)
    mask = ((row[:, None] == row[None, :]) & (col[None, :] <= col[:, None]))[None, None]
    setattr(mask, ROWS_ATTR, PackedRows(_bounds(lengths)))
    return mask


def _reference(q, k, v, lengths, do, scale):
    """fp32 attention of the fp16-rounded inputs, per row; output [1, N, H, D] and the
    gradients of q, k, v (fp32)."""
    qf, kf, vf = (t.detach().half().float().requires_grad_() for t in (q, k, v))
    groups = q.shape[1] // k.shape[1]
    outs = []
    s0 = 0
    for n in lengths:
        if n == 0:
            continue
        qs = qf[0, :, s0:s0 + n]
        ks = kf[0, :, s0:s0 + n].repeat_interleave(groups, 0)
        vs = vf[0, :, s0:s0 + n].repeat_interleave(groups, 0)
        s = torch.matmul(qs, ks.transpose(1, 2).contiguous()) * scale
        causal = torch.ones(n, n, dtype=torch.bool, device=q.device).tril()
        p = torch.softmax(s.masked_fill(~causal, float("-inf")), -1)
        outs.append(torch.matmul(p, vs).transpose(0, 1))  # [n, H, D]
        s0 += n
    out = torch.cat(outs, 0)[None]
    out.backward(do.float())
    return out.detach(), [t.grad for t in (qf, kf, vf)]


def _err(a, b):
    return float((a.float() - b.float()).abs().max())


def _check(name, ours, stock, ref):
    e_ours, e_stock = _err(ours, ref), _err(stock, ref)
    floor = 2e-3 * max(float(ref.abs().max()), 1e-3)
    print(f"  {name}: |ours - fp32| {e_ours:.3e}  |stock - fp32| {e_stock:.3e}  max {float(ref.abs().max()):.3e}")
    assert e_ours <= 2 * e_stock + floor, (name, e_ours, e_stock)


def _run(fn, q, k, v, mask, do):
    for t in (q, k, v):
        t.grad = None
    out, _ = fn(_Module(), q, k, v, mask, dropout=0.0, scaling=128 ** -0.5)
    out.backward(do)
    return out.detach(), [t.grad.detach() for t in (q, k, v)]


LENGTHS = [
    [154, 284, 482, 356],  # the config-5 batch of seed 0
    [64, 1, 512, 7],
    [300],
    [1],
    [63, 64, 65, 128, 129],
    [2048],
    [int(x) for x in torch.randint(1, 40, (100,), generator=torch.Generator().manual_seed(3))],
    # the kernels locate a block's row with one lane per row below 64 rows, by walking the table
    # from 64 on: both sides of that edge
    [int(x) for x in torch.randint(1, 20, (63,), generator=torch.Generator().manual_seed(4))],
    [int(x) for x in torch.randint(1, 20, (64,), generator=torch.Generator().manual_seed(5))],
]


@pytest.mark.gpu
@pytest.mark.parametrize("lengths", LENGTHS, ids=lambda x: f"{len(x)}rows_{sum(x)}tok")
def test_packed_attention_matches_fp32(dev, lengths):
    banner(f"packed causal attention rows={lengths[:6]}{'...' if len(lengths) > 6 else ''}")
    from transformers.integrations.sdpa_attention import sdpa_attention_forward as stock
    from transformers.modeling_utils import AttentionInterface

    from claudemaxing_amd import attention

    attention.patch_qwen2_grouped_sdpa()
    ours = AttentionInterface._global_mapping["sdpa"]
    n = sum(lengths)
    q, k, v, do = _inputs(dev, n, 0)
    mask = _packed_mask(lengths, dev)
    o_ref, g_ref = _reference(q, k, v, lengths, do, 128 ** -0.5)
    o_st, g_st = _run(stock, q, k, v, mask, do)
    o, g = _run(ours, q, k, v, mask, do)
    assert o.dtype == torch.float16 and o.shape == (1, n, 12, 128)
    _check("out", o, o_st, o_ref)
    for a, b, c, name in zip(g, g_st, g_ref, "qkv"):
        assert a.dtype == torch.float16
        _check(f"d{name}", a, b, c)


@pytest.mark.gpu
@pytest.mark.parametrize("heads,kv", [(14, 2), (16, 2), (28, 4), (40, 8)],
                         ids=lambda x: str(x))
def test_qwen_head_layouts(dev, heads, kv):
    """The query/key-value head counts of the other Qwen2.5 models (0.5B 14/2, 3B 16/2, 7B 28/4,
    14B 40/8: groups of 7, 8, 7 and 5 query heads per key-value head), on config 5's rows."""
    banner(f"packed causal attention heads={heads} kv={kv}")
    from transformers.integrations.sdpa_attention import sdpa_attention_forward as stock
    from transformers.modeling_utils import AttentionInterface

    from claudemaxing_amd import attention

    attention.patch_qwen2_grouped_sdpa()
    ours = AttentionInterface._global_mapping["sdpa"]
    lengths = [154, 284, 482, 356]
    n = sum(lengths)
    q, k, v, do = _inputs(dev, n, 9, heads=heads, groups=kv)
    mask = _packed_mask(lengths, dev)
    o_ref, g_ref = _reference(q, k, v, lengths, do, 128 ** -0.5)

    class Mod(_Module):
        num_key_value_groups = heads // kv

    def run(fn):
        for t in (q, k, v):
            t.grad = None
        out, _ = fn(Mod(), q, k, v, mask, dropout=0.0, scaling=128 ** -0.5)
        out.backward(do)
        return out.detach(), [t.grad.detach() for t in (q, k, v)]

    o_st, g_st = run(stock)
    o, g = run(ours)
    assert o.shape == (1, n, heads, 128)
    _check("out", o, o_st, o_ref)
    for a, b, c, name in zip(g, g_st, g_ref, "qkv"):
        _check(f"d{name}", a, b, c)


@pytest.mark.gpu
def test_fp32_inputs_under_autocast(dev):
    """The training step's case: fp32 q/k/v (after RoPE) inside fp16 autocast; gradients fp32."""
    banner("packed causal attention, fp32 inputs under fp16 autocast")
    from transformers.integrations.sdpa_attention import sdpa_attention_forward as stock
    from transformers.modeling_utils import AttentionInterface

    from claudemaxing_amd import attention

    attention.patch_qwen2_grouped_sdpa()
    ours = AttentionInterface._global_mapping["sdpa"]
    lengths = [154, 284, 482, 356]
    q, k, v, do = _inputs(dev, sum(lengths), 4, dtype=torch.float32)
    mask = _packed_mask(lengths, dev)
    o_ref, g_ref = _reference(q, k, v, lengths, do, 128 ** -0.5)
    with torch.autocast("cuda", dtype=torch.float16):
        o_st, g_st = _run(stock, q, k, v, mask, do)
        o, g = _run(ours, q, k, v, mask, do)
    assert o.dtype == torch.float16
    _check("out", o, o_st, o_ref)
    for a, b, c, name in zip(g, g_st, g_ref, "qkv"):
        assert a.dtype == torch.float32
        _check(f"d{name}", a, b, c)


@pytest.mark.gpu
def test_backward_is_deterministic_and_graph_replays_match(dev):
    banner("packed causal attention: repeated backward, HIP-graph replay")
    from claudemaxing_amd.attention import packed_causal_attention

    lengths = [154, 284, 482, 356]
    bounds = _bounds(lengths)
    q, k, v, do = _inputs(dev, sum(lengths), 7)

    def step():
        for t in (q, k, v):
            t.grad = None
        out = packed_causal_attention(q, k, v, bounds)
        out.backward(do)
        return out.detach().clone(), [t.grad.detach().clone() for t in (q, k, v)]

    o1, g1 = step()
    o2, g2 = step()
    assert torch.equal(o1, o2)
    for a, b in zip(g1, g2):
        assert torch.equal(a, b)

    # graph: forward + backward into static grads
    static_q = q.detach().clone().requires_grad_()
    static_k = k.detach().clone().requires_grad_()
    static_v = v.detach().clone().requires_grad_()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            out = packed_causal_attention(static_q, static_k, static_v, bounds)
            out.backward(do)
    torch.cuda.current_stream().wait_stream(side)
    for t in (static_q, static_k, static_v):
        t.grad = None
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        g_out = packed_causal_attention(static_q, static_k, static_v, bounds)
        g_out.backward(do)
    statics = (static_q, static_k, static_v)
    for i in range(3):
        f = 1.0 + 0.1 * i
        with torch.no_grad():
            for s, t in zip(statics, (q, k, v)):
                s.copy_(t * f)
        graph.replay()
        torch.cuda.synchronize()
        # eager work between replays, then the same inputs eagerly
        qi, ki, vi = (t.detach().mul(f).requires_grad_() for t in (q, k, v))
        out = packed_causal_attention(qi, ki, vi, bounds)
        out.backward(do)
        assert torch.equal(g_out, out.detach()), i
        for s, t in zip(statics, (qi, ki, vi)):
            assert torch.equal(s.grad, t.grad), i


@pytest.mark.gpu
def test_grouped_general_mask_matches(dev):
    banner("attention grouped sdpa, random boolean mask")
    from transformers.integrations.sdpa_attention import sdpa_attention_forward as stock

    from claudemaxing_amd import attention

    n = 256
    q, k, v, do = _inputs(dev, n, 1)
    g = torch.Generator(device=dev).manual_seed(2)
    mask = torch.rand(1, 1, n, n, generator=g, device=dev) < 0.7
    mask |= torch.eye(n, dtype=torch.bool, device=dev)[None, None]  # every query sees a key

    def grouped(module, q, k, v, mask, dropout, scaling):
        return attention._grouped_sdpa(q, k, v, mask, scaling), None

    o_ref, g_ref = _run(stock, q, k, v, mask, do)
    o, gr = _run(grouped, q, k, v, mask, do)
    torch.testing.assert_close(o.float(), o_ref.float(), rtol=2e-3, atol=2e-3)
    for a, b, name in zip(gr, g_ref, "qkv"):
        scale = float(b.abs().max())
        torch.testing.assert_close(a.float(), b.float(), rtol=2e-3, atol=2e-3 * max(scale, 1.0),
                                   msg=f"d{name}")


@pytest.mark.gpu
def test_pack_batch_records_rows(dev):
    banner("pack batch row bounds")
    from types import SimpleNamespace

    from claudemaxing_amd import qlora_step
    from claudemaxing_amd.attention import packed_rows
    from claudemaxing_amd.lm_head_loss import _pack_batch

    batch, lengths = qlora_step.make_batch(dev, seed=5)
    head = torch.nn.Linear(1536, 151936, bias=False).requires_grad_(False)
    lm = SimpleNamespace(lm_head=head, config=SimpleNamespace(_attn_implementation="sdpa"))
    packed = _pack_batch(lm, dict(input_ids=batch["input_ids"],
                                  attention_mask=batch["attention_mask"]), batch["labels"])
    bounds = packed_rows(packed.mask).bounds
    assert bounds == tuple([0] + torch.cumsum(lengths, 0).tolist())
    # the recorded rows are exactly the blocks of the mask
    m = packed.mask[0, 0].cpu()
    for s, e in zip(bounds[:-1], bounds[1:]):
        assert torch.equal(m[s:e, s:e], torch.ones(e - s, e - s, dtype=torch.bool).tril())
        assert not m[s:e, :s].any() and not m[s:e, e:].any()


def _rope_tables(lengths, dev, dim=128, theta=1e6):
    """cos / sin [1, N, D] fp32 of packed rows whose positions restart at 0 (Qwen2's rotary
    embedding over packed position ids)."""
    pos = torch.cat([torch.arange(n, dtype=torch.float32) for n in lengths])
    inv = 1.0 / (theta ** (torch.arange(0, dim, 2, dtype=torch.float32) / dim))
    emb = torch.cat((pos[:, None] * inv, pos[:, None] * inv), -1)
    return emb.cos()[None].to(dev), emb.sin()[None].to(dev)


@pytest.mark.gpu
@pytest.mark.parametrize("lengths", [[154, 284, 482, 356], [1, 63, 64, 65, 128, 129], [700]],
                         ids=["config5", "edges", "one_row"])
@pytest.mark.parametrize("layout", ["step", "fp16"])
def test_fused_rope_equals_rope_then_attention(dev, lengths, layout):
    """cm_attn_fwd_rope / cm_attn_bwd_rope on q, k before the rotation against RoPE's kernel
    followed by the attention on the rotated q, k: output and every gradient the same bits. The
    step's layout: q fp32 and v fp32 views of the projection outputs [N, H * D], k fp16 (the
    fused q/k/v block's outputs) under fp16 autocast; and all fp16."""
    banner(f"fused rope attention {layout} {lengths}")
    from claudemaxing_amd.attention import packed_causal_attention
    from claudemaxing_amd.rope import rope

    n = sum(lengths)
    g = torch.Generator(device=dev).manual_seed(11)
    dtq, dtk = (torch.float32, torch.float16) if layout == "step" else (torch.float16,) * 2
    base_q = torch.randn(1, n, 12 * 128, generator=g, device=dev).to(dtq)
    base_k = torch.randn(1, n, 2 * 128, generator=g, device=dev).to(dtk)
    base_v = torch.randn(1, n, 2 * 128, generator=g, device=dev).to(dtq)
    do = torch.randn(1, n, 12, 128, generator=g, device=dev).half()
    cos, sin = _rope_tables(lengths, dev)
    bounds = _bounds(lengths)

    def leaves():
        q = base_q.clone().requires_grad_()
        k = base_k.clone().requires_grad_()
        v = base_v.clone().requires_grad_()
        view = lambda t, h: t.view(1, n, h, 128).transpose(1, 2)  # noqa: E731
        return (q, k, v), (view(q, 12), view(k, 2), view(v, 2))

    with torch.autocast("cuda", dtype=torch.float16, enabled=layout == "step"):
        (q1, k1, v1), (qv, kv, vv) = leaves()
        qr, kr = rope(qv, kv, cos, sin)
        o1 = packed_causal_attention(qr, kr, vv, bounds)
        torch.autograd.backward(o1, do)
        (q2, k2, v2), (qv, kv, vv) = leaves()
        o2 = packed_causal_attention(qv, kv, vv, bounds, cos=cos, sin=sin)
        torch.autograd.backward(o2, do)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2), "out"
    for a, b, name in ((q1, q2, "dq"), (k1, k2, "dk"), (v1, v2, "dv")):
        assert a.grad.dtype == b.grad.dtype, name
        assert torch.equal(a.grad, b.grad), (name, float((a.grad.float() - b.grad.float()).abs().max()))
