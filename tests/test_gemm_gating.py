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
