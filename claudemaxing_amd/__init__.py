"""MI355X (gfx950) QLoRA training-step kernel set: a drop-in for the kernels that the
reference's `solution.apply()` (arturbaimuratov1-sys/claudemaxing, solution/__init__.py:25-34)
plugs into Qwen2.5 -- NF4 dequant, RMSNorm, RoPE, SwiGLU with recompute, LoRA dropout-mask
pack/unpack and the fused LM-head cross-entropy -- as hand-written HIP kernels behind a C ABI
(include/claudemaxing_amd.h), called from Python through ctypes.
"""

from .attention import patch_qwen2_grouped_sdpa  # noqa: F401 - opt-in, see apply()
from .lm_head_loss import patch_fused_head_loss
from .lora import patch_peft_lora_4bit
from .nf4 import patch_bnb_nf4_dequant
from .rmsnorm import patch_qwen2_rmsnorm
from .rope import patch_qwen2_rope
from .swiglu_recompute import patch_qwen2_mlp_recompute


def apply():
    """Apply the patches in the reference's order (solution/__init__.py:25-34). The reference's
    last patch, grouped-query SDPA (attention.py here, `patch_qwen2_grouped_sdpa`), is not
    installed by default: on MI355X transformers' own path (repeat_kv + one SDPA call) is the
    faster one (425 us against 815 us per layer, forward + backward, at config 5), and the
    packed-row causal form saves attention time but adds more kernel launches than it saves in
    a training step that is bound by launch overhead. Call it explicitly to get it."""
    patch_qwen2_mlp_recompute()  # SwiGLU with recomputation
    patch_qwen2_rmsnorm()  # fused RMSNorm
    patch_fused_head_loss()  # head + loss + metrics without full logits
    patch_qwen2_rope()  # rotary embedding, q and k in one launch
    patch_bnb_nf4_dequant()  # NF4 dequantization (when bitsandbytes is installed)
    patch_peft_lora_4bit()  # LoRA branch with a packed dropout mask (when peft is installed)
