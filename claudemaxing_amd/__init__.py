"""MI355X (gfx950) QLoRA training-step kernel set: a drop-in for the kernels that the
reference's `solution.apply()` (arturbaimuratov1-sys/claudemaxing, solution/__init__.py:25-34)
plugs into Qwen2.5 -- NF4 dequant, RMSNorm, RoPE, SwiGLU with recompute, LoRA dropout-mask
pack/unpack and the fused LM-head cross-entropy -- as hand-written HIP kernels behind a C ABI
(include/claudemaxing_amd.h), called from Python through ctypes.
"""

from .lm_head_loss import patch_fused_head_loss
from .lora import patch_peft_lora_4bit
from .nf4 import patch_bnb_nf4_dequant
from .rmsnorm import patch_qwen2_rmsnorm
from .rope import patch_qwen2_rope
from .swiglu_recompute import patch_qwen2_mlp_recompute


def apply():
    """Apply the patches in the reference's order (solution/__init__.py:25-34). The grouped
    SDPA patch of the reference (attention.py) is not part of this kernel set."""
    patch_qwen2_mlp_recompute()  # SwiGLU with recomputation
    patch_qwen2_rmsnorm()  # fused RMSNorm
    patch_fused_head_loss()  # head + loss + metrics without full logits
    patch_qwen2_rope()  # rotary embedding, q and k in one launch
    patch_bnb_nf4_dequant()  # NF4 dequantization (when bitsandbytes is installed)
    patch_peft_lora_4bit()  # LoRA branch with a packed dropout mask (when peft is installed)
