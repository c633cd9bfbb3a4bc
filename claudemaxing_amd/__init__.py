"""MI355X (gfx950) QLoRA training-step kernel set: a drop-in for the kernels that the
reference's `solution.apply()` (arturbaimuratov1-sys/claudemaxing, solution/__init__.py:25-34)
plugs into Qwen2.5 -- NF4 dequant, RMSNorm, RoPE, SwiGLU with recompute, LoRA dropout-mask
pack/unpack, the fused LM-head cross-entropy and causal attention over the packed batch -- as
hand-written HIP kernels behind a C ABI (include/claudemaxing_amd.h), called from Python
through ctypes.
"""

from .attention import patch_qwen2_grouped_sdpa
from .decoder import patch_qwen2_decoder_residual
from .lm_head_loss import patch_fused_head_loss
from .lora import patch_peft_lora_4bit
from .nf4 import patch_bnb_nf4_dequant
from .qkv import patch_qwen2_fused_qkv
from .rmsnorm import patch_qwen2_rmsnorm
from .rope import patch_qwen2_rope
from .swiglu_recompute import patch_qwen2_mlp_recompute


def apply():
    """Apply the patches in the reference's order (solution/__init__.py:25-34), with two of this
    package's own before the last (q/k/v as one fused NF4 GEMM, and the decoder layer's residual
    adds inside its norms: the same arithmetic in fewer launches). The last one,
    the attention patch (attention.py, `patch_qwen2_grouped_sdpa`), routes the packed batch of
    the fused training forward to the native packed causal attention kernels. Other boolean
    masks keep transformers' own path: the reference's per-kv-head grouped SDPA is slower than
    it on MI355X (815 against 425 us per layer, forward + backward, at config 5) and stays
    available as `patch_qwen2_grouped_sdpa(grouped=True)`."""
    patch_qwen2_mlp_recompute()  # SwiGLU with recomputation
    patch_qwen2_rmsnorm()  # fused RMSNorm
    patch_fused_head_loss()  # head + loss + metrics without full logits
    patch_qwen2_rope()  # rotary embedding, q and k in one launch
    patch_bnb_nf4_dequant()  # NF4 dequantization (when bitsandbytes is installed)
    patch_peft_lora_4bit()  # LoRA branch with a packed dropout mask (when peft is installed)
    patch_qwen2_fused_qkv()  # q/k/v of NF4 + LoRA blocks as one fused NF4 GEMM each way
    patch_qwen2_decoder_residual()  # the decoder layer's residual adds inside its norms
    patch_qwen2_grouped_sdpa()  # causal attention of the packed batch
