"""MI355X-native (gfx950) GPTQ-int4 W4A16 fused-MoE path.

Python/PyTorch-ROCm host code over hand-written HIP kernels (libmoe_w4a16.so, C ABI in
include/moe_w4a16.h). Public surface:
  mtp_amd.repack   the reference's repack API (load_topk_expert_mlp, TopKExpertMlp, ...)
  mtp_amd.moe      MoeBlock (router_topk / moe_tokens / fused forward)
  mtp_amd.ops      tensor-level wrappers of every C entry point
  mtp_amd.synth    seeded synthetic Qwen3.6-35B-A3B-shaped layers
"""

__version__ = "0.1.0"
