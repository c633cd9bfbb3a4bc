"""Comparison helpers shared by the tests (tolerances follow tests_local/*.py of the
reference: atol = tol * max(|expected|, 1), rtol = tol)."""

import torch


def assert_close(actual, expected, tol, what=""):
    scale = expected.float().abs().max().clamp(min=1.0).item() if expected.numel() else 1.0
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
