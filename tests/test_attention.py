"""Host side of the packed causal attention (no GPU): padded token counts, workspace sizes,
argument checks of cm_attn_fwd / cm_attn_bwd before any HIP call, and the routing predicate."""

import ctypes

import pytest
import torch

from claudemaxing_amd import _lib, attention

INVALID = 1  # hipErrorInvalidValue


def _arr(bounds):
    return (ctypes.c_int64 * len(bounds))(*bounds)


def _fwd(lib, bounds, H=12, G=2, D=128, q_stride=(1024, 128), out=None, ws_bytes=1 << 30):
    arr = _arr(bounds)
    fake = 1 << 20  # never dereferenced: every case below fails or returns before a launch
    return lib.cm_attn_fwd(fake, 0, q_stride[0], q_stride[1], fake, 0, 1024, 128, fake, 0, 1024,
                           128, arr, len(bounds) - 1, H, G, D, 0.088, out or fake, fake, fake,
                           ws_bytes, None)


def test_padded_tokens(lib):
    b = [0, 154, 438, 920, 1276]  # rows 154, 284, 482, 356
    assert lib.cm_attn_padded_tokens(_arr(b), 4) == 192 + 320 + 512 + 384
    assert lib.cm_attn_padded_tokens(_arr([0, 64]), 1) == 64
    assert lib.cm_attn_padded_tokens(_arr([0, 65]), 1) == 128
    assert lib.cm_attn_padded_tokens(_arr([0, 0, 1]), 2) == 64  # empty rows take no blocks


@pytest.mark.parametrize("bounds", [[1, 5], [0, 5, 3], [0], [0] + list(range(1, 130))])
def test_invalid_bounds(lib, bounds):
    assert lib.cm_attn_padded_tokens(_arr(bounds), len(bounds) - 1) == -1
    if len(bounds) > 1:
        assert _fwd(lib, bounds) == INVALID


def test_workspace_bytes(lib):
    f = lib.cm_attn_workspace_bytes(1408, 12, 2, 128, 0)
    b = lib.cm_attn_workspace_bytes(1408, 12, 2, 128, 1)
    assert f >= 2 * 2 * 1408 * 128 * 2
    assert b >= (4 * 12 + 3 * 2) * 1408 * 128 * 2 + 2 * 12 * 1408 * 128 * 4
    assert lib.cm_attn_workspace_bytes(1408, 12, 2, 64, 0) == -1
    assert lib.cm_attn_workspace_bytes(-1, 12, 2, 128, 1) == -1


def test_argument_checks(lib):
    b = [0, 100, 300]
    assert _fwd(lib, b, D=64) == INVALID                  # head_dim must be 128
    assert _fwd(lib, b, H=12, G=5) == INVALID             # H not a multiple of G
    assert _fwd(lib, b, q_stride=(1024, 130)) == INVALID  # token stride breaks 16-B chunks
    assert _fwd(lib, b, ws_bytes=1024) == INVALID         # workspace too small
    assert _fwd(lib, [0, 0]) == 0                         # no tokens: nothing to do


def test_routing_predicate():
    q = torch.zeros(1, 12, 10, 128, dtype=torch.float16)
    k = torch.zeros(1, 2, 10, 128, dtype=torch.float16)
    assert attention._native_ok(q, k, k, (0, 4, 10))
    # fp32 inputs without fp16 autocast: the caller expects fp32 arithmetic
    assert not attention._native_ok(q.float(), k.float(), k.float(), (0, 4, 10))
    assert not attention._native_ok(q[..., :64], k[..., :64], k[..., :64], (0, 4, 10))
    assert not attention._native_ok(q, k, k, tuple(range(130)))
