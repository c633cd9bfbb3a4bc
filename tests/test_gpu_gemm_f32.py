"""cm_gemm_f32 (fp16 products with an fp32 result, split along the contraction) against an fp64
evaluation of the same fp16 operands, and against torch's fp32-output product."""

import pytest
import torch

from claudemaxing_amd.gemm import gemm_f32, gemm_f32_supported
from tests.conftest import banner

pytestmark = pytest.mark.gpu


def _pair(m, n, k, dev, seed, scale=0.05):
    g = torch.Generator(device=dev).manual_seed(seed)
    a = torch.randn(m, k, device=dev, generator=g).half()
    b = (torch.randn(n, k, device=dev, generator=g) * scale).half()
    return a, b


def _check(out, ref, name):
    # fp32 sums of exact fp16 products: the error grows with sqrt(K) ulps of the partial sums
    err = float((out.double() - ref).abs().max())
    bound = 2e-5 * float(ref.abs().max()) + 1e-6
    assert err <= bound, (name, err, bound)


@pytest.mark.parametrize("m,n,k", [(1276, 1536, 8960), (37, 1536, 8960), (300, 200, 1032),
                                   (8, 8, 8), (2048, 1536, 4096),
                                   # down projections of Qwen2.5-0.5B and 7B
                                   (300, 896, 4864), (300, 3584, 18944)])
def test_one_pair_matches_fp64(m, n, k, dev):
    banner(f"gemm_f32 m={m} n={n} k={k}")
    a, b = _pair(m, n, k, dev, 1)
    assert gemm_f32_supported(m, n, (a, b))
    out = gemm_f32((a, b))
    torch.cuda.synchronize()
    _check(out, a.double() @ b.double().t(), "one pair")
    # the same inputs give the same bits (slices are added in order)
    assert torch.equal(out, gemm_f32((a, b)))
    # and agree with torch's fp32-output product to fp32 rounding of the sums
    torch.testing.assert_close(out, torch.mm(a, b.t(), out_dtype=torch.float32), rtol=1e-4,
                               atol=1e-4 * float(out.abs().max()))


@pytest.mark.parametrize("m,k0,k1", [(1276, 8960, 8960), (300, 1032, 264)])
def test_two_pairs_match_fp64(m, k0, k1, dev):
    banner(f"gemm_f32 two pairs m={m} k0={k0} k1={k1}")
    n = 1536
    a0, b0 = _pair(m, n, k0, dev, 2)
    a1, b1 = _pair(m, n, k1, dev, 3)
    out = gemm_f32((a0, b0), (a1, b1))
    torch.cuda.synchronize()
    _check(out, a0.double() @ b0.double().t() + a1.double() @ b1.double().t(), "two pairs")


def test_strided_rows(dev):
    """Row strides beyond K (a column block of a wider matrix)."""
    a, b = _pair(96, 64, 2048, dev, 4)
    wide = torch.zeros(96, 2048 + 64, device=dev, dtype=torch.float16)
    wide[:, :2048] = a
    av = wide[:, :2048]
    assert gemm_f32_supported(96, 64, (av, b))
    _check(gemm_f32((av, b)), a.double() @ b.double().t(), "strided")


def test_unsupported_operands_are_refused(dev):
    a, b = _pair(16, 16, 64, dev, 5)
    assert not gemm_f32_supported(16, 16, (a.float(), b))
    assert not gemm_f32_supported(16, 16, (a[:, :60], b[:, :60]))  # K not a multiple of 8
    assert not gemm_f32_supported(15, 16, (a, b))  # A's rows are not the output's M
    a3, b3 = _pair(3, 3, 64, dev, 6)
    assert not gemm_f32_supported(3, 3, (a3, b3))  # M * N not a multiple of 4


@pytest.mark.parametrize("m,k0,k1", [(1276, 8960, 0), (300, 1032, 264)])
def test_residual_added_in_the_sum_launch(m, k0, k1, dev):
    """cm_gemm_f32_add: residual + the product, the bits of torch's fp32 add of the two."""
    banner(f"gemm_f32 + residual m={m} k0={k0} k1={k1}")
    n = 1536
    pairs = [_pair(m, n, k0, dev, 5)] + ([_pair(m, n, k1, dev, 6)] if k1 else [])
    res = torch.randn(m, n, device=dev, generator=torch.Generator(device=dev).manual_seed(7))
    got = gemm_f32(*pairs, residual=res)
    want = res + gemm_f32(*pairs)
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    with pytest.raises(ValueError):
        gemm_f32(*pairs, residual=res.t().contiguous().t())  # not contiguous


@pytest.mark.parametrize("m,n,k0,k1", [(1276, 1536, 8960, 8960), (300, 200, 1032, 264),
                                       (37, 896, 4864, 0), (8, 8, 8, 0), (513, 1544, 72, 136)])
def test_kmajor_b_equals_rowmajor_on_the_transpose(m, n, k0, k1, dev):
    """cm_gemm_f32_kb (B given [K, N], a weight as stored) gives the bits of cm_gemm_f32 on the
    transposed operands (the same elements reach the same lanes in the same k order), and
    matches fp64; edge tiles in n and k, one or two pairs."""
    banner(f"gemm_f32 k-major B m={m} n={n} k0={k0} k1={k1}")
    a0, bt0 = _pair(m, n, k0, dev, 7)
    b0 = bt0.t().contiguous()  # [K0, N]
    pairs_kb, pairs_rm = [(a0, b0)], [(a0, bt0)]
    ref = a0.double() @ b0.double()
    if k1:
        a1, bt1 = _pair(m, n, k1, dev, 8)
        b1 = bt1.t().contiguous()
        pairs_kb.append((a1, b1))
        pairs_rm.append((a1, bt1))
        ref = ref + a1.double() @ b1.double()
    assert gemm_f32_supported(m, n, *pairs_kb, b_kmajor=True)
    out = gemm_f32(*pairs_kb, b_kmajor=True)
    torch.cuda.synchronize()
    assert torch.equal(out, gemm_f32(*pairs_rm))
    _check(out, ref, "k-major B")


def test_kmajor_b_row_stride(dev):
    """A k-major B whose rows are a column block of a wider matrix (ldb > N)."""
    a, bt = _pair(96, 64, 2048, dev, 9)
    wide = torch.zeros(2048, 64 + 32, device=dev, dtype=torch.float16)
    wide[:, :64] = bt.t()
    b = wide[:, :64]
    assert b.stride(0) == 96 and gemm_f32_supported(96, 64, (a, b), b_kmajor=True)
    out = gemm_f32((a, b), b_kmajor=True)
    assert torch.equal(out, gemm_f32((a, bt)))
    assert not gemm_f32_supported(96, 60, (a, b[:, :60]), b_kmajor=True)  # N % 8
