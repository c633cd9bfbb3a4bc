"""The training forward's attention (claudemaxing_amd/attention.py) against transformers' own
sdpa attention with the same mask: the packed block-diagonal causal mask (per-row causal SDPA)
and a general boolean mask (grouped SDPA), outputs and gradients of q/k/v, fp16, GQA 12/2
heads of 128. The reference's grouped path (solution/attention.py:332-373) claims the same
values as repeat_kv + one call; both comparisons hold it to fp16-level tolerance."""

import pytest
import torch

from tests.conftest import banner


class _Module(torch.nn.Module):
    num_key_value_groups = 6
    is_causal = True
    training = True


def _inputs(dev, n, seed):
    g = torch.Generator(device=dev).manual_seed(seed)
    q = torch.randn(1, 12, n, 128, generator=g, device=dev).half().requires_grad_()
    k = torch.randn(1, 2, n, 128, generator=g, device=dev).half().requires_grad_()
    v = torch.randn(1, 2, n, 128, generator=g, device=dev).half().requires_grad_()
    do = torch.randn(1, n, 12, 128, generator=g, device=dev).half()
    return q, k, v, do


def _run(fn, q, k, v, mask, do):
    for t in (q, k, v):
        t.grad = None
    out, _ = fn(_Module(), q, k, v, mask, dropout=0.0, scaling=128 ** -0.5)
    out.backward(do)
    return out.detach().float(), [t.grad.detach().float() for t in (q, k, v)]


def _close(a, b, what):
    scale = float(b.abs().max())
    torch.testing.assert_close(a, b, rtol=2e-3, atol=2e-3 * max(scale, 1.0), msg=what)


def _packed_mask(lengths, dev):
    from claudemaxing_amd.attention import ROWS_ATTR

    row = torch.cat([torch.full((n,), i) for i, n in enumerate(lengths)]).to(dev)
    col = torch.cat([torch.arange(n) for n in lengths]).to(dev)
    mask = ((row[:, None] == row[None, :]) & (col[None, :] <= col[:, None]))[None, None]
    bounds = [0]
    for n in lengths:
        bounds.append(bounds[-1] + n)
    setattr(mask, ROWS_ATTR, tuple(bounds))
    return mask


@pytest.mark.gpu
@pytest.mark.parametrize("lengths", [[154, 284, 482, 356], [64, 1, 512, 7], [300]])
def test_packed_rows_match_masked_sdpa(dev, lengths):
    banner(f"attention packed rows {lengths}")
    from transformers.integrations.sdpa_attention import sdpa_attention_forward as stock

    from claudemaxing_amd import attention
    from transformers.modeling_utils import AttentionInterface

    attention.patch_qwen2_grouped_sdpa()
    ours = AttentionInterface._global_mapping["sdpa"]
    n = sum(lengths)
    q, k, v, do = _inputs(dev, n, 0)
    mask = _packed_mask(lengths, dev)
    o_ref, g_ref = _run(stock, q, k, v, mask, do)
    o, g = _run(ours, q, k, v, mask, do)
    _close(o, o_ref, "out")
    for a, b, name in zip(g, g_ref, "qkv"):
        _close(a, b, f"d{name}")


@pytest.mark.gpu
def test_grouped_general_mask_matches(dev):
    banner("attention grouped sdpa, random boolean mask")
    from transformers.integrations.sdpa_attention import sdpa_attention_forward as stock

    from claudemaxing_amd import attention
    from transformers.modeling_utils import AttentionInterface

    attention.patch_qwen2_grouped_sdpa()
    ours = AttentionInterface._global_mapping["sdpa"]
    n = 256
    q, k, v, do = _inputs(dev, n, 1)
    g = torch.Generator(device=dev).manual_seed(2)
    mask = torch.rand(1, 1, n, n, generator=g, device=dev) < 0.7
    mask |= torch.eye(n, dtype=torch.bool, device=dev)[None, None]  # every query sees a key
    o_ref, g_ref = _run(stock, q, k, v, mask, do)
    o, gr = _run(ours, q, k, v, mask, do)
    _close(o, o_ref, "out")
    for a, b, name in zip(gr, g_ref, "qkv"):
        _close(a, b, f"d{name}")


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
    bounds = packed_rows(packed.mask)
    assert bounds == tuple([0] + torch.cumsum(lengths, 0).tolist())
    # the recorded rows are exactly the blocks of the mask
    m = packed.mask[0, 0].cpu()
    for s, e in zip(bounds[:-1], bounds[1:]):
        assert torch.equal(m[s:e, s:e], torch.ones(e - s, e - s, dtype=torch.bool).tril())
        assert not m[s:e, :s].any() and not m[s:e, e:].any()
