"""CPU oracle for the processor prologue (K5): RMSNorm and rotary embedding.

TEST INFRASTRUCTURE ONLY.  Only tests/, ``__graft_entry__.smoke()`` and bench.py's
CPU-baseline leg may import this module, as the checker; no product code path
calls it.

Each function restates one step of the reference's processors, with the reference's
bf16 roundings between steps, in plain torch on the CPU:

* ``rms_norm_once``: svg/kernels/triton/rmsnorm.py:8-48 (``_rms_norm_fwd_fused``):
  fp32 x, var = sum(x*x)/N, rstd = 1/sqrt(var + eps), y = (x*rstd)*w, one cast.
  Pinned: equals torch.nn.functional.rms_norm on bf16 CPU tensors (a library routine
  with the same single rounding), closed forms, scale invariance.
* ``rms_norm_twice``: diffusers==0.34.0 ``RMSNorm.forward`` (pyproject.toml:24; the
  package is not vendored in the reference and not importable here), called by the
  HunyuanVideo fallback svg/models/hyvideo/attention.py:196-200:
  h = x * rsqrt(mean(x^2) + eps) in fp32, cast to the bf16 weight's dtype, then h*w
  in bf16.  The math is pinned as above; the placement of the intermediate rounding
  is restated from diffusers' published source and is otherwise parity unpinned.
* ``rope_cossin``: diffusers ``apply_rotary_emb(use_real=True, use_real_unbind_dim=-1)``
  as used at hyvideo/attention.py:211-230: out = x*cos + rot(x)*sin in fp32 steps,
  rot(x)[2i] = -x[2i+1], rot(x)[2i+1] = x[2i].  Pinned: rotation closed forms
  (angle 0, pi/2), norm preservation, agreement with the complex form.
* ``rope_complex``: svg/models/wan/attention.py:49-57: pairs as complex numbers in
  fp64 times the coefficient, cast back (fp64 -> fp32 -> bf16, torch's cast).
  Pinned: composition of rotations and the closed forms above.
"""
from __future__ import annotations

from typing import Optional

import numpy as np
import torch


def sqrt_rn(t: torch.Tensor) -> torch.Tensor:
    """Correctly rounded fp32 square root (numpy's; torch's CPU float32 sqrt is not
    correctly rounded on every host)."""
    return torch.from_numpy(np.sqrt(t.detach().cpu().numpy().astype(np.float32)))


def _bf16(x: torch.Tensor) -> torch.Tensor:
    return x.to(torch.bfloat16)


def rms_norm_once(x: torch.Tensor, w: Optional[torch.Tensor], eps: float) -> torch.Tensor:
    """RMSNorm over the last dim, one rounding (Triton rmsnorm.py:29-44)."""
    xf = x.float()
    var = (xf * xf).sum(-1, keepdim=True) / xf.shape[-1]
    rstd = 1.0 / sqrt_rn(var + eps)
    y = xf * rstd
    if w is not None:
        y = y * w.float()
    return _bf16(y)


def rms_norm_twice(x: torch.Tensor, w: Optional[torch.Tensor], eps: float) -> torch.Tensor:
    """diffusers 0.34.0 RMSNorm with a bf16 weight: normalise in fp32, cast, then * w in bf16."""
    xf = x.float()
    var = (xf * xf).mean(-1, keepdim=True)
    h = _bf16(xf * torch.rsqrt(var + eps))
    if w is None:
        return h
    return _bf16(h.float() * w.float())


def rope_cossin(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """x [..., S, D] bf16; cos / sin fp32 [S, D].  fp32 steps, then bf16."""
    xf = x.float()
    rot = torch.stack([-xf[..., 1::2], xf[..., 0::2]], dim=-1).flatten(-2)
    return _bf16(xf * cos.float() + rot * sin.float())


def rope_complex(x: torch.Tensor, re: torch.Tensor, im: torch.Tensor) -> torch.Tensor:
    """x [..., S, D] bf16; re / im fp64 [S, D/2].  fp64 complex product, fp64 -> fp32 -> bf16."""
    xc = torch.view_as_complex(x.double().unflatten(-1, (-1, 2)).contiguous())
    f = torch.complex(re.double(), im.double())
    out = torch.view_as_real(xc * f).flatten(-2)
    return _bf16(out.float())


def qkv_prologue(xq, xk, xv, heads: int, *, wq=None, wk=None, norm=None, rounding="once", eps=1e-6,
                 rope=None, rope_rows=None):
    """The composition the fused kernel computes, for [B, S, H*D] inputs: norm (row or
    head) of Q and K, head split to [B, H, S, D], rotation of rows < rope_rows.
    Returns (q, k, v) bf16 [B, H, S, D] (None where the input is None)."""
    fn = rms_norm_once if rounding == "once" else rms_norm_twice
    outs = []
    for t, (x, w) in enumerate(((xq, wq), (xk, wk), (xv, None))):
        if x is None:
            outs.append(None)
            continue
        B, S, C = x.shape
        D = C // heads
        y = x
        if t < 2 and norm is not None and w is not None:
            if norm == "row":
                y = fn(y, w, eps)
            else:
                y = fn(y.reshape(B, S, heads, D), w, eps).reshape(B, S, C)
        y = y.reshape(B, S, heads, D).permute(0, 2, 1, 3).contiguous()
        if t < 2 and rope is not None:
            kind, a, b = rope
            n = S if rope_rows is None else rope_rows
            head = y[:, :, :n]
            head = rope_cossin(head, a, b) if kind == "cossin" else rope_complex(head, a, b)
            y = torch.cat([head, y[:, :, n:]], dim=2)
        outs.append(y)
    return tuple(outs)
