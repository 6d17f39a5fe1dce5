"""Rotary position embedding in the two forms the PASA processors receive.

* Wan (complex form): the reference's fallback (svg/models/wan/attention.py:49-57)
  rotates channel pairs (x[2i], x[2i+1]) as complex numbers, in float64, by a
  complex ``freqs`` tensor broadcast over [B, H, S, D/2].
* HunyuanVideo (real cos/sin form): the processors call diffusers'
  ``apply_rotary_emb(x, (cos, sin))`` (svg/models/hyvideo/attention.py:8, used at
  :211-230).  diffusers==0.34.0 (pyproject.toml:24; not vendored in the reference)
  defines it, for use_real=True and use_real_unbind_dim=-1, as
  out = x * cos + rot(x) * sin with rot(x)[2i] = -x[2i+1], rot(x)[2i+1] = x[2i],
  computed in float32 and cast back to x's dtype; cos / sin are [S, D].
"""
from __future__ import annotations

import torch


def apply_rotary_emb_complex(x: torch.Tensor, freqs: torch.Tensor) -> torch.Tensor:
    """x [B, H, S, D] rotated by complex freqs (broadcastable to [B, H, S, D/2])."""
    if isinstance(freqs, (tuple, list)):
        freqs = torch.complex(freqs[0].to(torch.float64), freqs[1].to(torch.float64))
    xc = torch.view_as_complex(x.to(torch.float64).unflatten(3, (-1, 2)))
    return torch.view_as_real(xc * freqs).flatten(3, 4).type_as(x)


def apply_rotary_emb_cos_sin(x: torch.Tensor, freqs_cis) -> torch.Tensor:
    """x [B, H, S, D]; freqs_cis = (cos, sin), each [S, D]."""
    cos, sin = freqs_cis
    cos = cos[None, None].to(x.device)
    sin = sin[None, None].to(x.device)
    x_real, x_imag = x.reshape(*x.shape[:-1], -1, 2).unbind(-1)
    x_rot = torch.stack([-x_imag, x_real], dim=-1).flatten(3)
    return (x.float() * cos + x_rot.float() * sin).to(x.dtype)
