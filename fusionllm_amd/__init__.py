"""fusionllm_amd — MI355X-native DeepSeekMoE feed-forward block for FusionLLM.

Drop-in replacement for ``models.moe`` of FusionLLM: ``DeepSeekMoE`` and
``SwiGLUExpert`` with the reference's constructor, parameters and methods,
computed by hand-written gfx950 HIP kernels (libfusionmoe.so, C ABI in
include/fusionmoe.h).
"""
from .moe import DeepSeekMoE, SwiGLUExpert

__all__ = ["DeepSeekMoE", "SwiGLUExpert"]
