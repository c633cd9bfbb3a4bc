"""CPU oracle of the QLoRA step kernel set: TEST INFRASTRUCTURE ONLY.

A restatement, on the CPU, of what the reference (arturbaimuratov1-sys/claudemaxing,
solution/*.py and the torch references of tests_local/*.py) computes on the hot path. Only
tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import it, and only as the
checker (or the timed CPU baseline) -- never as the thing measured or shipped. The product
package claudemaxing_amd never imports it.

Modules (each function cites the reference lines it restates and names what pins it):
  nf4      -- NF4 dequant (numpy, bit-exact), NF4 table from normal quantiles, quantizer
  lora     -- dropout mask pack/unpack (numpy, bit-exact)
  rmsnorm  -- Qwen2RMSNorm forward/backward (torch CPU fp32)
  rope     -- apply_rotary_pos_emb forward/backward (torch CPU fp32)
  swiglu   -- F.silu(gate) * up forward/backward (torch CPU fp32)
  lm_head  -- fp16 logits -> cross-entropy, entropy, accuracy, hidden gradient (torch CPU)
  inputs   -- seeded CPU generators of the benchmark configurations
"""
