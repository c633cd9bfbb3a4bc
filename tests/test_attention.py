"""Host side of the packed causal attention (no GPU): padded token counts, the rows image the
kernels read from device memory, workspace sizes, argument checks of cm_attn_fwd / cm_attn_bwd
before any HIP call, PackedRows and the bucket capacity, and the routing predicate."""

import ctypes

import pytest
import torch

from claudemaxing_amd import _lib, attention

INVALID = 1  # hipErrorInvalidValue


def _arr(bounds):
    return (ctypes.c_int64 * len(bounds))(*bounds)


def _fwd(lib, n_tokens=300, n_pad=384, H=12, G=2, D=128, q_stride=(1024, 128), out=None,
         ws_bytes=1 << 30, rows=1 << 20):
    fake = 1 << 20  # never dereferenced: every case below fails or returns before a launch
    return lib.cm_attn_fwd(fake, 0, q_stride[0], q_stride[1], fake, 0, 1024, 128, fake, 0, 1024,
                           128, rows, n_tokens, n_pad, H, G, D, 0.088, out or fake, fake, fake,
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
    image = (ctypes.c_uint8 * lib.cm_attn_rows_bytes())()
    assert lib.cm_attn_rows_image(_arr(bounds), len(bounds) - 1, image) == -1


def test_rows_image(lib):
    """The image the kernels read: int32 start[129], pstart[129], then the row count."""
    b = [0, 154, 438, 920, 1276]
    nbytes = lib.cm_attn_rows_bytes()
    assert nbytes == (2 * 129 + 1) * 4
    image = (ctypes.c_uint8 * nbytes)()
    assert lib.cm_attn_rows_image(_arr(b), 4, image) == 1408
    words = torch.frombuffer(bytearray(image), dtype=torch.int32)
    assert words[:5].tolist() == b
    assert words[129:134].tolist() == [0, 192, 512, 1024, 1408]
    assert int(words[258]) == 4


def test_workspace_bytes(lib):
    f = lib.cm_attn_workspace_bytes(1408, 12, 2, 128, 0)
    b = lib.cm_attn_workspace_bytes(1408, 12, 2, 128, 1)
    assert f >= 2 * 2 * 1408 * 128 * 2
    assert b >= (4 * 12 + 3 * 2) * 1408 * 128 * 2 + 2 * 12 * 1408 * 128 * 4
    assert lib.cm_attn_workspace_bytes(1408, 12, 2, 64, 0) == -1
    assert lib.cm_attn_workspace_bytes(-1, 12, 2, 128, 1) == -1


def test_argument_checks(lib):
    assert _fwd(lib, D=64) == INVALID                  # head_dim must be 128
    assert _fwd(lib, H=12, G=5) == INVALID             # H not a multiple of G
    assert _fwd(lib, q_stride=(1024, 130)) == INVALID  # token stride breaks 16-B chunks
    assert _fwd(lib, ws_bytes=1024) == INVALID         # workspace too small
    assert _fwd(lib, n_pad=400) == INVALID             # capacity not whole 64-position blocks
    assert _fwd(lib, n_pad=0) == INVALID
    assert _fwd(lib, n_pad=64 * 65536) == INVALID      # more padded blocks than a grid dimension
    assert _fwd(lib, rows=0) == INVALID                # no rows image
    assert _fwd(lib, rows=(1 << 20) + 8) == INVALID    # image not 16-byte aligned
    assert _fwd(lib, n_tokens=0) == 0                  # no tokens: nothing to do


def test_packed_rows_capacity_and_load():
    rows = attention.PackedRows((0, 154, 438, 920, 1276))
    assert rows.n_pad == rows.capacity == 1408
    with pytest.raises(ValueError):
        attention.PackedRows((0, 154, 438, 920, 1276), capacity=1344)  # below 1408
    with pytest.raises(ValueError):
        attention.PackedRows((0, 5, 3))
    big = attention.PackedRows((0, 1000, 1276), capacity=1600)
    big.load((0, 154, 438, 920, 1276))  # 1408 padded positions fit 1600
    assert big.bounds == (0, 154, 438, 920, 1276) and big.n_pad == 1408
    with pytest.raises(ValueError):
        big.load((0, 154, 438, 920, 1277))  # another token count
    with pytest.raises(ValueError):
        attention.PackedRows((0, 1, 2), capacity=64).load((0, 1, 2))  # 128 > 64


def test_bucket_capacity_holds_every_packing():
    """Any split of N tokens into at most R rows pads to at most bucket_capacity(N, R)."""
    from claudemaxing_amd.lm_head_loss import bucket_capacity

    g = torch.Generator().manual_seed(0)
    for n in (1, 63, 64, 65, 256, 1280, 2048):
        for r in (1, 2, 5):
            cap = bucket_capacity(n, r)
            assert cap % 64 == 0
            for _ in range(50):
                cuts = sorted(torch.randint(0, n + 1, (r - 1,), generator=g).tolist())
                b = [0, *cuts, n]
                assert attention._padded_tokens(tuple(b)) <= cap, (n, r, b)
            worst = [0] + [min(n, 65 * i) for i in range(1, r)] + [n]  # 65-token rows
            assert attention._padded_tokens(tuple(worst)) <= cap


def test_routing_predicate():
    q = torch.zeros(1, 12, 10, 128, dtype=torch.float16)
    k = torch.zeros(1, 2, 10, 128, dtype=torch.float16)
    assert attention._native_ok(q, k, k, (0, 4, 10))
    # fp32 inputs without fp16 autocast: the caller expects fp32 arithmetic
    assert not attention._native_ok(q.float(), k.float(), k.float(), (0, 4, 10))
    assert not attention._native_ok(q[..., :64], k[..., :64], k[..., :64], (0, 4, 10))
    assert not attention._native_ok(q, k, k, tuple(range(130)))
