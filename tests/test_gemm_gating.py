"""Host-side gating of the split-K fp32 GEMM and the batched adapter weight gradients (no GPU):
which products take them, and that anything they cannot take falls back."""

import torch

from claudemaxing_amd.gemm import gemm_f32_supported, split_k_pays
from claudemaxing_amd.lora import _weight_grads


def test_split_k_pays_for_narrow_long_contractions():
    # the step's MLP products at 1276 tokens: 40 output tiles, K = 8960 or 2 x 8960
    assert split_k_pays(1276, 1536, 8960) and split_k_pays(1276, 1536, 17920)
    # short contraction (the attention projections) or a wide output (gate/up): the library GEMM
    assert not split_k_pays(1276, 1536, 1536)
    assert not split_k_pays(1276, 8960, 1536)
    assert not split_k_pays(32768, 1536, 8960)  # 128 x 8 tiles fill the chip by themselves


def test_cpu_operands_are_not_taken():
    a = torch.zeros(16, 64, dtype=torch.float16)
    b = torch.zeros(16, 64, dtype=torch.float16)
    assert not gemm_f32_supported(16, 16, (a, b))  # not on the GPU
    assert _weight_grads([(torch.zeros(8, 16, dtype=torch.float16),
                           torch.zeros(8, 64, dtype=torch.float16))]) is None


def test_weight_grads_refuse_products_without_a_rank_16_side():
    # neither operand is 16 wide: not an adapter weight gradient (checked before any launch,
    # so CPU tensors with is_cuda patched in are enough to reach the shape test)
    class FakeCuda(torch.Tensor):
        @property
        def is_cuda(self):
            return True

    g = torch.zeros(8, 32, dtype=torch.float16).as_subclass(FakeCuda)
    y = torch.zeros(8, 64, dtype=torch.float16).as_subclass(FakeCuda)
    assert _weight_grads([(g, y)]) is None
    assert _weight_grads([]) is None


class _FakeCuda(torch.Tensor):
    """A CPU tensor that reports is_cuda, to reach the host gates' layout checks."""

    @property
    def is_cuda(self):
        return True


def _fake(t):
    return t.as_subclass(_FakeCuda)


def test_gemm_f32_needs_both_operands_on_the_gpu():
    a = _fake(torch.zeros(16, 64, dtype=torch.float16))
    b = torch.zeros(16, 64, dtype=torch.float16)
    assert not gemm_f32_supported(16, 16, (a, b))  # B on the host
    assert gemm_f32_supported(16, 16, (a, _fake(b)))


def test_weight_grads_refuse_wide_rows_the_kernel_rejects(monkeypatch):
    """The wide operand's row stride must be even and at least its width (the entry point
    refuses anything else); such operands get None (the per-product fallback), never an error
    from the library."""
    from claudemaxing_amd import lora

    launched = []
    monkeypatch.setattr(lora._lib, "call", lambda *a: launched.append(a[0]))
    monkeypatch.setattr(lora._lib, "stream", lambda dev: None)
    rank = _fake(torch.zeros(8, 16, dtype=torch.float16))
    odd = _fake(torch.zeros(8, 129, dtype=torch.float16)[:, :64])
    assert odd.stride(0) == 129 and _weight_grads([(rank, odd)]) is None
    short = _fake(torch.zeros(8 * 64, dtype=torch.float16).as_strided((8, 64), (32, 1)))
    assert short.stride(0) < short.shape[1] and _weight_grads([(rank, short)]) is None
    assert not launched
    ok = _fake(torch.zeros(8, 130, dtype=torch.float16)[:, :64])
    out = _weight_grads([(rank, ok)])
    assert launched == ["cm_lora_weight_grads"] and out is not None and out[0].shape == (16, 64)
