"""Pins the NF4 oracle (oracle/nf4.py) independently of the code under test."""

import numpy as np
import pytest
import torch

from oracle import nf4 as O

F32 = np.float32


def test_table_matches_its_normal_quantile_construction():
    built = O.nf4_table_from_quantiles()
    np.testing.assert_allclose(O.NF4_TABLE.astype(np.float64), built, rtol=0, atol=5e-7)  # fp32 rounding of the quantiles
    assert O.NF4_TABLE[7] == 0.0 and O.NF4_TABLE[0] == -1.0 and O.NF4_TABLE[15] == 1.0
    assert np.all(np.diff(O.NF4_TABLE) > 0)


def test_package_table_is_the_oracle_table():
    from claudemaxing_amd.nf4 import NF4_CODE_VALUES

    assert np.array_equal(np.array(NF4_CODE_VALUES, dtype=F32), O.NF4_TABLE)


def test_dynamic_map_shape():
    m = O.dynamic_map()
    assert m.shape == (256,) and np.all(np.diff(m) >= 0)
    assert m.max() == 1.0 and m.min() < -0.99 and 0.0 in m
    # 127 magnitudes per sign over 7 decades
    assert np.sum(m > 0) == 128 and np.sum(m < 0) == 127


@pytest.mark.parametrize("nested", [True, False])
def test_vectorised_equals_elementwise(nested):
    rng = np.random.default_rng(1)
    w = (rng.standard_normal((6, 64)) * 0.05).astype(F32)
    q = O.quantize(w, 64, nested, blocksize2=4)
    kw = dict(nested=nested, blocksize=64)
    if nested:
        kw.update(code2=q["code2"], absmax2=q["absmax2"], offset=q["offset"], blocksize2=4)
    a = O.dequant(q["packed"], q["absmax"], **kw)
    b = O.dequant_bruteforce(q["packed"], q["absmax"], **kw)
    assert np.array_equal(a.view(np.int16), b.view(np.int16))


def test_every_byte_with_every_q8_code():
    """All 256 packed byte values against all 256 absmax codes: 65,536 bytes, one absmax block
    per code (blocksize 512 elements = 256 bytes), offset and absmax2 arbitrary."""
    code2 = O.dynamic_map()
    packed = np.tile(np.arange(256, dtype=np.uint8), 256)
    q8 = np.arange(256, dtype=np.uint8)
    absmax2 = np.array([0.37, 1.5], dtype=F32)
    offset = F32(0.0123)
    out = O.dequant(packed, q8, nested=True, code2=code2, absmax2=absmax2, offset=offset,
                    blocksize=512, blocksize2=128)
    b = np.arange(256)
    s = ((code2[q8] * absmax2[b // 128]).astype(F32) + offset).astype(F32)
    for blk in (0, 1, 127, 128, 255):
        got = out[blk * 512:(blk + 1) * 512].reshape(256, 2)
        hi = (O.NF4_TABLE[np.arange(256) >> 4] * s[blk]).astype(np.float16)
        lo = (O.NF4_TABLE[np.arange(256) & 15] * s[blk]).astype(np.float16)
        assert np.array_equal(got[:, 0].view(np.int16), hi.view(np.int16))
        assert np.array_equal(got[:, 1].view(np.int16), lo.view(np.int16))


def test_nibble_order_and_block_index_on_planted_elements():
    # element 2 of block 1 (blocksize 64): byte 33, high nibble; element 3: byte 33, low nibble
    w = np.zeros((2, 64), dtype=F32)
    w[1, 2] = 1.0
    w[1, 3] = -0.5
    q = O.quantize(w, 64, compress_statistics=False)
    # +1.0 -> code 15; -0.5 lies below the midpoint of codes 2 and 3 (-0.46): code 2
    assert q["packed"][33] >> 4 == 15 and (q["packed"][33] & 15) == 2
    assert q["absmax"][0] == 0 and q["absmax"][1] == 1.0
    out = O.dequant(q["packed"], q["absmax"], blocksize=64).astype(F32)
    assert out[64 + 2] == 1.0 and out[64 + 3] == np.float16(O.NF4_TABLE[2])
    assert np.count_nonzero(out) == 2


def test_known_answer_special_values():
    """tests_local/test_nf4.py:21: zeros, a tiny value and outliers in one block."""
    rng = np.random.default_rng(0)
    w = (rng.standard_normal((4, 64)) * 0.05).astype(F32)
    w[0, :5] = [0.0, -0.0, 1e-7, 3.0, -2.5]
    q = O.quantize(w, 64, compress_statistics=False)
    out = O.dequant(q["packed"], q["absmax"], blocksize=64).astype(F32)
    assert q["absmax"][0] == F32(3.0)
    assert out[0] == 0.0 and out[1] == 0.0 and out[2] == 0.0  # code 7 is exactly 0
    assert out[3] == 3.0  # the block maximum comes back exactly (code 15 = 1.0)
    # -2.5 / 3 = -0.8333 lies above the midpoint of codes 0 and 1 (-0.8481): code 1
    assert out[4] == np.float16(F32(O.NF4_TABLE[1]) * F32(3.0))


def test_block_max_roundtrips_exactly_without_double_quant():
    rng = np.random.default_rng(3)
    w = (rng.standard_normal((32, 64)) * 0.05).astype(F32)
    q = O.quantize(w, 64, compress_statistics=False)
    out = O.dequant(q["packed"], q["absmax"], blocksize=64, out_dtype="f32").reshape(32, 64)
    idx = np.abs(w).argmax(axis=1)
    assert np.array_equal(out[np.arange(32), idx], w[np.arange(32), idx])


def test_scale_is_multiply_then_add_not_fma():
    # values where fl(fl(a*b)+c) != fl(a*b+c): a single rounding would differ
    a, b, c = F32(1.0000001), F32(1.0000001), F32(-1.0000002)
    s = O.block_scales(np.array([0], np.uint8), True, np.array([a], F32), np.array([b], F32), c,
                       blocksize2=1)
    assert s[0] == F32(F32(a * b) + c)
    exact = np.float64(a) * np.float64(b) + np.float64(c)
    assert s[0] != F32(exact)


def test_package_quantizer_matches_the_oracle_quantizer():
    from claudemaxing_amd.nf4 import quantize_nf4

    w = torch.randn(64, 256, generator=torch.Generator().manual_seed(5)) * 0.02
    packed, state = quantize_nf4(w, 64, True)
    q = O.quantize(w.numpy(), 64, True)
    assert np.array_equal(packed.reshape(-1).numpy(), q["packed"])
    assert state.offset.item() == q["offset"]
    # the dynamic maps are built with torch vs numpy linspace: equal to fp32 rounding
    np.testing.assert_allclose(state.state2.code.numpy(), q["code2"], rtol=1e-6, atol=1e-12)
    mismatch = np.count_nonzero(state.absmax.numpy() != q["absmax"])
    assert mismatch <= 2


def test_to_bf16_bits_matches_torch_rounding():
    """The oracle's fp32 -> bf16 rounding (the checker of the kernels' bf16 outputs) against
    torch's own `.to(torch.bfloat16)`: every fp16 value, fp32 specials, subnormals, exact
    halfway cases (ties to even, both parities), the overflow edge and random bit patterns."""
    fp16_all = np.arange(65536, dtype=np.uint16).view(np.float16).astype(F32)
    specials = np.array([0.0, -0.0, np.inf, -np.inf, np.finfo(F32).max, -np.finfo(F32).max,
                         np.finfo(F32).tiny, np.finfo(F32).tiny / 3, 1e-45, -1e-45], dtype=F32)
    rng = np.random.default_rng(7)
    hi = rng.integers(0, 1 << 16, 4096, dtype=np.uint32) << 16
    halves = np.concatenate([hi | 0x8000, hi | 0x7FFF, hi | 0x8001]).view(F32)  # ties + edges
    edge = np.array([0x7F7F8000, 0x7F7F7FFF, 0xFF7F8000], dtype=np.uint32).view(F32)
    randbits = rng.integers(0, 1 << 32, 1 << 20, dtype=np.uint64).astype(np.uint32).view(F32)
    x = np.concatenate([fp16_all, specials, halves, edge, randbits])
    nan = np.isnan(x)
    ours = O.to_bf16_bits(x)
    ref = torch.from_numpy(x.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours[~nan], ref[~nan])
    # NaN stays NaN (sign kept, quiet bit set), as the kernel's conversion does
    nan_in = np.array([0x7FC00000, 0xFF800001, 0x7F800001], dtype=np.uint32).view(F32)
    out = O.to_bf16_bits(nan_in)
    assert np.all((out & 0x7F80) == 0x7F80) and np.all(out & 0x0040)
    assert list(out >> 15) == [0, 1, 0]
    # a plausible slip, truncation instead of rounding, fails the same comparison
    trunc = (x.view(np.uint32) >> 16).astype(np.uint16)
    assert not np.array_equal(trunc[~nan], ref[~nan])
