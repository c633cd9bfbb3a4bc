"""cm_lmhead_ce_noalloc -- the fused LM head on the library's own per-GPU scratch array, no
allocation -- against cm_lmhead_ce with a caller workspace, through the C ABI. With the same
vocabulary chunk the two run the same kernels on the same layout, so every output must be the
same bits; two calls in a row (the second smaller, on a scratch that still holds the first
call's contents) show that nothing depends on what the array held before. The chunk the entry
point picks itself is checked against the workspace entry point's default within the LM head's
tolerances, and sizes that do not fit are refused before any launch."""

import pytest
import torch

from claudemaxing_amd import _lib
from claudemaxing_amd import lm_head_loss as LH
from oracle import inputs, lm_head as O
from tests.conftest import banner
from tests.helpers import assert_close as _assert_close


def assert_close(actual, expected, tol, what=""):
    """The reference's LM-head tolerance (test_lm_head_loss.py:105-108): atol is tol times the
    largest expected value itself, however small (the hidden gradient's is ~0.1)."""
    _assert_close(actual, expected, tol, what, floor=1e-6)


pytestmark = pytest.mark.gpu

F16 = torch.float16


def _noalloc(h16, w16, tgt, chunk, want_grad=True):
    n, hidden = h16.shape
    dev = h16.device
    loss = torch.full((n,), -7.0, device=dev)
    ent = torch.full((n,), -7.0, device=dev)
    corr = torch.full((n,), -7, dtype=torch.int32, device=dev)
    grad = torch.full((n, hidden), -7.0, device=dev) if want_grad else None
    before = torch.cuda.memory_allocated(dev)
    rc = _lib.load().cm_lmhead_ce_noalloc(
        h16.data_ptr(), h16.stride(0), w16.data_ptr(), w16.stride(0),
        tgt.data_ptr(), n, w16.shape[0], hidden, chunk, loss.data_ptr(), ent.data_ptr(),
        corr.data_ptr(), _lib.ptr(grad), 1.0, _lib.stream(dev))
    assert torch.cuda.memory_allocated(dev) == before  # no allocation through torch either
    return rc, (loss, ent, corr, grad)


def _same_bits(a, b, what):
    for x, y, name in zip(a, b, ("loss", "entropy", "correct", "grad")):
        if x is None and y is None:
            continue
        assert torch.equal(x.cpu().view(-1), y.cpu().view(-1)), f"{what}: {name} differs"


def test_noalloc_equals_workspace_entry_two_calls(dev):
    banner("lmhead noalloc: two calls, explicit chunks")
    # call 1: 1100 rows, H 512, the full Qwen vocabulary in 4096-column chunks
    h, w, t = inputs.lm_head(5, n=1100, hidden=512)
    h16, w16, td = h.to(dev), w.to(dev), t.to(dev)
    rc, got = _noalloc(h16, w16, td, 4096)
    assert rc == 0, _lib.load().cm_error_string(rc)
    ref = LH._fused_rows(h16, w16, td, True, 4096)
    torch.cuda.synchronize()
    _same_bits(got, ref, "call 1")
    rows = torch.arange(0, 1100, 37)
    o = O.head(h[rows], w, t[rows])
    assert_close(got[0][rows.to(dev)], o[0], 1e-4, "call 1 loss vs oracle")
    assert_close(got[3][rows.to(dev)], o[3], 1e-2, "call 1 grad vs oracle")
    # call 2, smaller: 300 rows, H 256, a 50,000-column vocabulary in 2048-column chunks, on
    # the scratch call 1 filled
    h, w, t = inputs.lm_head(6, n=300, vocab=50000, hidden=256)
    h16, w16, td = h.to(dev), w.to(dev), t.to(dev)
    rc, got = _noalloc(h16, w16, td, 2048)
    assert rc == 0, _lib.load().cm_error_string(rc)
    ref = LH._fused_rows(h16, w16, td, True, 2048)
    torch.cuda.synchronize()
    _same_bits(got, ref, "call 2")
    o = O.head(h, w, t)
    assert_close(got[0], o[0], 1e-4, "call 2 loss vs oracle")
    assert_close(got[3], o[3], 1e-2, "call 2 grad vs oracle")
    # and without a gradient (forward terms only)
    rc, fwd = _noalloc(h16, w16, td, 2048, want_grad=False)
    assert rc == 0
    torch.cuda.synchronize()
    _same_bits(fwd[:3], ref[:3], "call 3, no gradient")


def test_noalloc_own_chunk_and_refusal(dev):
    banner("lmhead noalloc: own chunk at config 4, refusal")
    h, w, t = inputs.lm_head(0)
    hd, wd, td = h.to(dev), w.to(dev), t.to(dev)
    w16 = LH.fp16_head_weight(wd)
    rc, got = _noalloc(hd, w16, td, 0)
    assert rc == 0, _lib.load().cm_error_string(rc)
    ref = LH._fused_rows(hd, w16, td, True, None)
    torch.cuda.synchronize()
    assert_close(got[0], ref[0], 1e-5, "loss")
    assert_close(got[1], ref[1], 1e-5, "entropy")
    assert_close(got[3], ref[3], 1e-3, "grad")
    diff = (got[2].cpu() != ref[2].cpu()).nonzero().flatten()
    if diff.numel():  # only rows whose top two fp16 logits are within an ulp may differ
        gaps, ulps = O.top2_gap(h[diff], w)
        assert torch.all(gaps <= ulps)
    # a whole-vocabulary chunk at this size needs ~650 MB: refused, nothing written
    rc, out = _noalloc(hd, w16, td, 151936)
    assert rc == 20001  # CM_ERROR_SCRATCH_TOO_SMALL
    assert b"scratch" in _lib.load().cm_error_string(rc)
    torch.cuda.synchronize()
    assert torch.all(out[0] == -7.0) and torch.all(out[3] == -7.0)


def test_noalloc_fewer_slices_at_config4_chunk8192(dev):
    """Config 4 at its stated 8192-column chunk: the chunk's buffers (35 MiB) and the workspace
    entry's four gradient K-slices (three 12.6 MB accumulators beside the output) exceed the
    64 MiB scratch, so the entry point runs three slices. The logits pass is the same (same
    chunk), so loss, entropy and correct are the workspace entry's bits; the gradient sums its
    slices in another fp32 order and agrees within tolerance, and a seeded 64-row subset
    matches the oracle."""
    banner("lmhead noalloc: config 4, chunk 8192, fewer slices")
    assert LH.fused_head_plan(2048, 151936, 1536, 8192) == (8192, 4)
    assert LH.fused_head_plan(2048, 151936, 1536, 8192, noalloc=True) == (8192, 3)
    h, w, t = inputs.lm_head(0)
    hd, wd, td = h.to(dev), w.to(dev), t.to(dev)
    w16 = LH.fp16_head_weight(wd)
    rc, got = _noalloc(hd, w16, td, 8192)
    assert rc == 0, _lib.load().cm_error_string(rc)
    ref = LH._fused_rows(hd, w16, td, True, 8192)
    torch.cuda.synchronize()
    _same_bits(got[:3], ref[:3], "forward terms")
    assert_close(got[3], ref[3], 1e-3, "grad vs the workspace entry")
    rows = torch.randperm(2048, generator=torch.Generator().manual_seed(2))[:64]
    o = O.head(h[rows], w, t[rows])
    assert_close(got[0][rows.to(dev)], o[0], 1e-4, "loss vs oracle")
    assert_close(got[3][rows.to(dev)], o[3], 1e-2, "grad vs oracle")
