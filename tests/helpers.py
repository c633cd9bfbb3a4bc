"""Comparison helpers shared by the tests (tolerances follow tests_local/*.py of the
reference: atol = tol * max(max|expected|, floor), rtol = tol)."""

import torch


def assert_close(actual, expected, tol, what="", floor=1.0):
    """rtol = tol, atol = tol * max(max|expected|, floor). The reference's RMSNorm, RoPE and
    SwiGLU tests take floor 1 (test_rmsnorm.py:48); its LM-head tests take the largest value
    itself (floor 1e-6, test_lm_head_loss.py:106), which the LM-head tests here pass."""
    scale = expected.float().abs().max().clamp(min=floor).item() if expected.numel() else 1.0
    torch.testing.assert_close(actual.float().cpu(), expected.float().cpu(), rtol=tol,
                               atol=tol * scale, msg=lambda m: f"{what}: {m}")


def assert_bits_equal(actual, expected, what=""):
    a, e = actual.cpu().contiguous(), expected.cpu().contiguous()
    assert a.dtype == e.dtype and a.shape == e.shape, (what, a.dtype, e.dtype, a.shape, e.shape)
    if a.dtype in (torch.float16, torch.bfloat16):
        a, e = a.view(torch.int16), e.view(torch.int16)
    elif a.dtype == torch.float32:
        a, e = a.view(torch.int32), e.view(torch.int32)
    diff = (a != e).nonzero()
    assert diff.numel() == 0, f"{what}: {diff.shape[0]} elements differ, first at {diff[:5].tolist()}"


def tolerance(*dtypes):
    if torch.bfloat16 in dtypes:
        return 1e-2
    return 2e-3 if torch.float16 in dtypes else 1e-4
