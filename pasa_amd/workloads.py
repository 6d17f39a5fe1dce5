"""Synthetic PISA workloads and their seeded input generator.

Inputs follow the measurement contract: Q, K, V = N(0, 1) noise plus a smooth
3-D positional component of amplitude 1.0 — per (head, channel) a plane wave
sin(2*pi*(f/lf + y/ly + x/lx) + phi) with wavelengths lf, ly, lx ~ U[2, 8]
and phase phi ~ U[0, 2*pi).  Q and K share the wave (attention mass is then
local); V draws its own.  Text tokens (HunyuanVideo) are pure N(0, 1) and sit
after the video tokens.  Tokens are frame-major: t = f*(Hh*W) + y*W + x.

Everything is drawn on the CPU in fp32 from a per-head torch.Generator, so any
subset of heads can be regenerated bit-identically (the CPU baseline regenerates
only the heads it times), then scaled (``prescale``) and cast once.
"""
from __future__ import annotations

import math
import os
from concurrent.futures import ThreadPoolExecutor
from dataclasses import dataclass, field
from typing import Optional, Tuple

import torch


@dataclass(frozen=True)
class Workload:
    name: str
    heads: int
    head_dim: int
    grid: Tuple[int, int, int]     # (frames, height, width) of the latent video
    block_size: int
    density: float
    dtype: torch.dtype = torch.bfloat16
    text_tokens: int = 0
    prescale: float = 1.0          # Q <- Q * prescale (folds the softmax temperature)
    scale: Optional[float] = None  # softmax scale passed to the op (None = D^-1/2)
    batch: int = 1
    notes: str = ""

    @property
    def video_tokens(self) -> int:
        f, h, w = self.grid
        return f * h * w

    @property
    def seq_len(self) -> int:
        return self.video_tokens + self.text_tokens

    @property
    def op_scale(self) -> float:
        return self.head_dim ** -0.5 if self.scale is None else self.scale

    def num_blocks(self) -> int:
        """Key blocks of the blocked segment: the video rows (text rows, when present,
        are a separate dense segment)."""
        return math.ceil(self.video_tokens / self.block_size)

    def k4_flops(self, group_size: int = 32, ns: Optional[int] = None) -> float:
        """Algorithmic K4 FLOPs: BH*[4*D*BT^2*NT*NS + NT*NG*(4*BT*G*D + 2*BT*D^2)] + F_text,
        F_text = 4*D*(Tv*X + X*(Tv + X))*BH for X text tokens (video rows x text keys
        and dense text rows)."""
        nt = self.num_blocks()
        ng = math.ceil(nt / group_size)
        if ns is None:
            ns = min(max(1, int(self.density * nt)), nt)
        bt, d = self.block_size, self.head_dim
        bh = self.batch * self.heads
        tv, x = self.video_tokens, self.text_tokens
        f_text = 4.0 * d * (tv * x + x * (tv + x)) * bh
        return bh * (4.0 * d * bt * bt * nt * ns + nt * ng * (4.0 * bt * group_size * d + 2.0 * bt * d * d)) + f_text


A1_PRESCALE = 128 ** -0.5  # "pre-scaled by 1/sqrt(128)": folded into Q, op scale 1.0

WORKLOADS = {
    "c0": Workload("c0", heads=2, head_dim=64, grid=(4, 16, 16), block_size=64, density=0.25,
                   dtype=torch.float32, notes="CPU reference-path plumbing (fp32)"),
    "c1": Workload("c1", heads=12, head_dim=128, grid=(21, 30, 52), block_size=128, density=0.15,
                   prescale=A1_PRESCALE, scale=1.0, notes="Wan2.1-1.3B 480p/81f"),
    "c2": Workload("c2", heads=40, head_dim=128, grid=(21, 45, 80), block_size=128, density=0.10,
                   prescale=A1_PRESCALE, scale=1.0, notes="Wan2.1-14B 720p/81f (headline)"),
    "c3": Workload("c3", heads=24, head_dim=128, grid=(33, 45, 80), block_size=128, density=0.10,
                   text_tokens=256, prescale=A1_PRESCALE, scale=1.0,
                   notes="HunyuanVideo 720p/129f + 256 text tokens"),
}


def _plane_wave(gen: torch.Generator, grid, dim: int) -> torch.Tensor:
    """[T, dim] plane waves, one per channel, over the (f, y, x) grid."""
    F, Hh, W = grid
    lam = torch.rand(3, dim, generator=gen) * 6.0 + 2.0
    phi = torch.rand(dim, generator=gen) * (2.0 * math.pi)
    f = torch.arange(F, dtype=torch.float32)[:, None, None, None] / lam[0]
    y = torch.arange(Hh, dtype=torch.float32)[None, :, None, None] / lam[1]
    x = torch.arange(W, dtype=torch.float32)[None, None, :, None] / lam[2]
    return torch.sin(2.0 * math.pi * (f + y + x) + phi).reshape(F * Hh * W, dim)


def head_inputs(wl: Workload, head: int, seed: int = 0):
    """fp32 (q, k, v) [T, D] of one (batch 0) head, before prescale / cast."""
    gen = torch.Generator().manual_seed(seed * 1_000_003 + head)
    D = wl.head_dim
    wave_qk = _plane_wave(gen, wl.grid, D)
    wave_v = _plane_wave(gen, wl.grid, D)
    T, Tv = wl.seq_len, wl.video_tokens
    q = torch.randn(T, D, generator=gen)
    k = torch.randn(T, D, generator=gen)
    v = torch.randn(T, D, generator=gen)
    q[:Tv] += wave_qk
    k[:Tv] += wave_qk
    v[:Tv] += wave_v
    return q, k, v


def make_inputs(wl: Workload, seed: int = 0, heads: Optional[range] = None, device=None,
                dtype: Optional[torch.dtype] = None, threads: Optional[int] = None):
    """(q, k, v) [1, len(heads), T, D] in the workload dtype (or ``dtype``), on ``device``.

    Q is multiplied by ``wl.prescale`` in fp32 before the single cast."""
    heads = range(wl.heads) if heads is None else heads
    dtype = wl.dtype if dtype is None else dtype
    T, D = wl.seq_len, wl.head_dim
    out = [torch.empty(1, len(heads), T, D, dtype=dtype) for _ in range(3)]

    def one(i_h):
        i, h = i_h
        q, k, v = head_inputs(wl, h, seed)
        if wl.prescale != 1.0:
            q = q * wl.prescale
        for t, src in zip(out, (q, k, v)):
            t[0, i].copy_(src.to(dtype))

    threads = threads or min(8, os.cpu_count() or 1)
    with ThreadPoolExecutor(max_workers=threads) as ex:
        list(ex.map(one, enumerate(heads)))
    if device is not None:
        out = [t.to(device) for t in out]
    return tuple(out)


def small_workload(base: Workload, heads: int, grid: Tuple[int, int, int], **kw) -> Workload:
    """A reduced copy of ``base`` (parity tests at sizes the oracle finishes quickly)."""
    d = dict(base.__dict__)
    d.update(heads=heads, grid=grid, name=base.name + "-small", **kw)
    return Workload(**d)
