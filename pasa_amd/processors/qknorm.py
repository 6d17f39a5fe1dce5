"""Q/K RMSNorm forms of the reference's processors, and the choice between the fused
prologue kernel (``pasa_amd.prologue``) and the step-by-step PyTorch route.

* Wan (svg/models/wan/attention.py:122-136) normalises with its Triton rmsnorm for any
  RMSNorm module (torch.nn.RMSNorm or diffusers' RMSNorm), one rounding, and raises
  ValueError for other norm types.
* HunyuanVideo (svg/models/hyvideo/attention.py:196-209) calls the norm module itself,
  so the rounding follows the module: torch.nn.RMSNorm rounds once; diffusers'
  RMSNorm (diffusers==0.34.0, not vendored) normalises in fp32, casts to the bf16
  weight's dtype, then multiplies by the weight in bf16 (two roundings).

The fused kernel runs when the tensors are bf16 on a ROCm device with head_dim 64 or
128 and bf16 affine RMSNorm weights; other inputs (fp32 models, CPU tensors in unit
tests) take the reference's own PyTorch composition.
"""
from __future__ import annotations

from typing import Optional

import torch

from ..prologue import MAX_ROW_CHANNELS


def is_torch_rmsnorm(m) -> bool:
    return isinstance(m, torch.nn.RMSNorm)


def is_diffusers_rmsnorm(m) -> bool:
    return type(m).__name__ == "RMSNorm" and type(m).__module__.startswith("diffusers")


def is_rmsnorm(m) -> bool:
    return is_torch_rmsnorm(m) or is_diffusers_rmsnorm(m)


def norm_eps(m, dtype) -> float:
    """The module's eps; with eps=None torch's rms_norm uses the epsilon of the type it
    computes in (fp32 for bf16 / fp16 inputs)."""
    eps = getattr(m, "eps", None)
    if eps is not None:
        return float(eps)
    return torch.finfo(torch.float64 if dtype == torch.float64 else torch.float32).eps


def rms_norm_once(x: torch.Tensor, weight: Optional[torch.Tensor], eps: float) -> torch.Tensor:
    """The Triton rmsnorm of the Wan processor (svg/kernels/triton/rmsnorm.py:29-44) in
    PyTorch: fp32 math, one cast back to x's dtype."""
    xf = x.float()
    y = xf * (1.0 / torch.sqrt((xf * xf).sum(-1, keepdim=True) / xf.shape[-1] + eps))
    if weight is not None:
        y = y * weight.float()
    return y.to(x.dtype)


def module_rounding(m) -> Optional[str]:
    """'once' / 'twice' for a norm module the fused kernel reproduces, else None."""
    if is_torch_rmsnorm(m):
        return "once"
    if is_diffusers_rmsnorm(m):
        return "twice"
    return None


def fusable(x: torch.Tensor, heads: int, norms, weight_len: int) -> bool:
    """True when the fused prologue kernel computes exactly what the step-by-step route would."""
    if not (x.is_cuda and x.dtype == torch.bfloat16 and x.dim() == 3):
        return False
    C = x.shape[-1]
    if C % heads or C // heads not in (64, 128) or C > MAX_ROW_CHANNELS:
        return False
    for m in norms:
        if m is None:
            continue
        w = getattr(m, "weight", None)
        if w is None or w.dtype != torch.bfloat16 or w.numel() != weight_len or not w.is_cuda:
            return False
    return True
