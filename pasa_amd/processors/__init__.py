"""Attention processors for the diffusers Wan2.1 and HunyuanVideo transformers.

Same class names, constructors, class-attribute configuration and installers as
the reference's svg/models/wan and svg/models/hyvideo modules; the sparse branch
calls ``pasa_amd.ops.pisa_pg_attention`` (gfx950 kernels)."""
from .hunyuan import (Hunyuan_PASA_Processor, Hunyuan_SVGAttn_Processor2_0,
                      HunyuanVideoAttnProcessor2_0_FlashAttention, replace_hyvideo_attention,
                      replace_hyvideo_flashattention)
from .timestep_hook import current_timestep
from .wan import Wan_PASA_Processor, WanAttn_SVGAttn_Processor2_0, replace_wan_attention

__all__ = [
    "Hunyuan_PASA_Processor", "Hunyuan_SVGAttn_Processor2_0", "HunyuanVideoAttnProcessor2_0_FlashAttention",
    "replace_hyvideo_attention", "replace_hyvideo_flashattention", "Wan_PASA_Processor",
    "WanAttn_SVGAttn_Processor2_0", "replace_wan_attention", "current_timestep",
]
