"""fusionllm_amd — MI355X-native DeepSeekMoE feed-forward block for FusionLLM.

Drop-in replacement for ``models.moe`` of FusionLLM: ``DeepSeekMoE`` and
``SwiGLUExpert`` with the reference's constructor, parameters and methods,
computed by hand-written gfx950 HIP kernels (libfusionmoe.so, C ABI in
include/fusionmoe.h); ``moe_residual`` runs FusionLLMBlock's FFN half
x + ffn(norm2(x)) with the RMSNorm and the residual fused into the kernels.
Under torch.compile the block is traced as the fusionllm::moe_fwd /
fusionllm::moe_bwd operators (fusionllm_amd.ops).
"""
from . import ops  # registers the fusionllm::moe_fwd / moe_bwd operators (torch.compile)
from .graph import DecodeGraph
from .moe import DeepSeekMoE, DenseFFN, SwiGLUExpert, dense_swiglu, moe_residual

__all__ = ["DecodeGraph", "DeepSeekMoE", "DenseFFN", "SwiGLUExpert", "dense_swiglu", "moe_residual"]
