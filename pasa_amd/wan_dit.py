"""Random-init Wan2.1 DiT in plain PyTorch: the harness through which the PASA
processors are measured end to end (one denoising step of the 1.3B model at 480p /
81 frames, with a density sweep).

The architecture is diffusers==0.34.0's WanTransformer3DModel (pinned at the
reference's pyproject.toml:24; neither vendored in the reference nor installed here),
driven the way the reference drives it: its replacement block and model forwards
(svg/models/wan/custom_models.py:23-190, the branch without the Triton kernels) pass the
denoising ``timestep`` to each block's self-attention, and its installer
(svg/models/wan/inference.py:12-74, restated as
``pasa_amd.processors.replace_wan_attention``) puts a processor on every ``attn1``.

Attention modules keep diffusers' processor protocol: the module holds ``to_q``,
``to_k``, ``to_v``, ``to_out``, ``norm_q``, ``norm_k`` and ``heads`` and calls
``processor(attn, hidden_states, encoder_hidden_states=..., rotary_emb=..., **kwargs)``,
dropping keyword arguments the processor does not accept (as diffusers'
``Attention.forward`` does).  Without an installed processor they run
``WanAttnProcessor``, diffusers' dense processor: projections, RMSNorm across heads,
complex float64 RoPE, PyTorch SDPA.

Parity of the model itself against diffusers is not claimed (diffusers is absent); it is
a workload of the right shape and arithmetic for the processors, whose outputs the tests
compare with this module's own dense processor.
"""
from __future__ import annotations

import inspect
import math
from dataclasses import dataclass
from types import SimpleNamespace
from typing import Optional, Tuple

import torch
import torch.nn as nn
import torch.nn.functional as F

from .processors.rope import apply_rotary_emb_complex


@dataclass
class WanDiTConfig:
    """WanTransformer3DModel's configuration; the defaults are Wan2.1-T2V-1.3B."""
    patch_size: Tuple[int, int, int] = (1, 2, 2)
    in_channels: int = 16
    out_channels: int = 16
    text_dim: int = 4096
    freq_dim: int = 256
    ffn_dim: int = 8960
    num_layers: int = 30
    num_attention_heads: int = 12
    attention_head_dim: int = 128
    eps: float = 1e-6
    rope_max_seq_len: int = 1024

    @property
    def inner_dim(self) -> int:
        return self.num_attention_heads * self.attention_head_dim


class FP32LayerNorm(nn.LayerNorm):
    """LayerNorm computed in float32 and cast back to the input's dtype."""

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        w = self.weight.float() if self.weight is not None else None
        b = self.bias.float() if self.bias is not None else None
        return F.layer_norm(x.float(), self.normalized_shape, w, b, self.eps).to(x.dtype)


class WanAttnProcessor:
    """Dense attention of diffusers' Wan processor: q/k/v projections, RMSNorm over the
    full width, head split, complex RoPE on q and k, SDPA, output projection."""

    def __call__(self, attn, hidden_states, encoder_hidden_states=None, attention_mask=None,
                 rotary_emb=None):
        if encoder_hidden_states is None:
            encoder_hidden_states = hidden_states
        query = attn.to_q(hidden_states)
        key = attn.to_k(encoder_hidden_states)
        value = attn.to_v(encoder_hidden_states)
        if attn.norm_q is not None:
            query = attn.norm_q(query)
        if attn.norm_k is not None:
            key = attn.norm_k(key)
        query = query.unflatten(2, (attn.heads, -1)).transpose(1, 2)
        key = key.unflatten(2, (attn.heads, -1)).transpose(1, 2)
        value = value.unflatten(2, (attn.heads, -1)).transpose(1, 2)
        if rotary_emb is not None:
            query = apply_rotary_emb_complex(query, rotary_emb)
            key = apply_rotary_emb_complex(key, rotary_emb)
        out = F.scaled_dot_product_attention(query, key, value, attn_mask=attention_mask, dropout_p=0.0,
                                             is_causal=False)
        out = out.transpose(1, 2).flatten(2, 3).type_as(query)
        out = attn.to_out[0](out)
        return attn.to_out[1](out)


class WanAttention(nn.Module):
    """An attention module with diffusers' processor protocol (``qk_norm`` =
    "rms_norm_across_heads": one RMSNorm over heads * head_dim)."""

    def __init__(self, dim: int, heads: int, head_dim: int, eps: float):
        super().__init__()
        inner = heads * head_dim
        self.heads = heads
        self.to_q = nn.Linear(dim, inner, bias=True)
        self.to_k = nn.Linear(dim, inner, bias=True)
        self.to_v = nn.Linear(dim, inner, bias=True)
        self.to_out = nn.ModuleList([nn.Linear(inner, dim, bias=True), nn.Dropout(0.0)])
        self.norm_q = nn.RMSNorm(inner, eps=eps)
        self.norm_k = nn.RMSNorm(inner, eps=eps)
        self.processor = WanAttnProcessor()

    def set_processor(self, processor) -> None:
        self.processor = processor

    def forward(self, hidden_states, encoder_hidden_states=None, rotary_emb=None, **kwargs):
        accepted = inspect.signature(self.processor.__call__).parameters
        kwargs = {k: v for k, v in kwargs.items() if k in accepted}
        return self.processor(self, hidden_states, encoder_hidden_states=encoder_hidden_states,
                              rotary_emb=rotary_emb, **kwargs)


class WanBlock(nn.Module):
    """One DiT block: modulated self-attention, cross-attention to the text, modulated
    feed-forward (the reference's block forward, custom_models.py:23-115).

    ``fast_kernels`` (class attribute) selects the reference's ENABLE_FAST_KERNEL
    branch for bf16 device tensors: the LayerNorm / modulation / gated-residual steps
    run as four fused row-ops calls (``pasa_amd.modulate``) instead of PyTorch
    elementwise passes; off, the block is diffusers' PyTorch forward."""
    fast_kernels = True

    def __init__(self, cfg: WanDiTConfig):
        super().__init__()
        dim = cfg.inner_dim
        self.norm1 = FP32LayerNorm(dim, cfg.eps, elementwise_affine=False)
        self.attn1 = WanAttention(dim, cfg.num_attention_heads, cfg.attention_head_dim, cfg.eps)
        self.attn2 = WanAttention(dim, cfg.num_attention_heads, cfg.attention_head_dim, cfg.eps)
        self.norm2 = FP32LayerNorm(dim, cfg.eps, elementwise_affine=True)
        self.ffn = nn.Sequential(nn.Linear(dim, cfg.ffn_dim), nn.GELU(approximate="tanh"),
                                 nn.Linear(cfg.ffn_dim, dim))
        self.norm3 = FP32LayerNorm(dim, cfg.eps, elementwise_affine=False)
        self.scale_shift_table = nn.Parameter(torch.randn(1, 6, dim) / dim ** 0.5)

    def forward(self, hidden_states, encoder_hidden_states, temb, rotary_emb, timestep=0):
        shift_msa, scale_msa, gate_msa, c_shift_msa, c_scale_msa, c_gate_msa = (
            self.scale_shift_table + temb.float()).chunk(6, dim=1)
        if self.fast_kernels and _row_ops_ok(hidden_states):
            return self._forward_fused(hidden_states, encoder_hidden_states, rotary_emb, timestep,
                                       (shift_msa, scale_msa, gate_msa, c_shift_msa, c_scale_msa, c_gate_msa))
        norm = self.norm1(hidden_states.float())
        norm = (norm * (1 + scale_msa) + shift_msa).type_as(hidden_states)
        attn_out = self.attn1(norm, rotary_emb=rotary_emb, timestep=timestep)
        hidden_states = (hidden_states.float() + attn_out * gate_msa).type_as(hidden_states)

        norm = self.norm2(hidden_states.float()).type_as(hidden_states)
        hidden_states = hidden_states + self.attn2(norm, encoder_hidden_states=encoder_hidden_states)

        norm = self.norm3(hidden_states.float())
        norm = (norm * (1 + c_scale_msa) + c_shift_msa).type_as(hidden_states)
        ff = self.ffn(norm)
        return (hidden_states.float() + ff.float() * c_gate_msa).type_as(hidden_states)

    def _forward_fused(self, hidden_states, encoder_hidden_states, rotary_emb, timestep, mods):
        from . import modulate as M
        shift_msa, scale_msa, gate_msa, c_shift_msa, c_scale_msa, c_gate_msa = mods
        norm = M.ln_modulate(hidden_states, scale_msa, shift_msa, self.norm1.eps)
        attn_out = self.attn1(norm, rotary_emb=rotary_emb, timestep=timestep)
        # h = bf16(x + attn * gate) into a new tensor, and norm2(h), in one pass
        h = torch.empty_like(hidden_states)
        norm = torch.empty_like(hidden_states)
        M.row_ops(attn_out.contiguous(), residual=hidden_states.contiguous(), gate=gate_msa, h_out=h,
                  layernorm=True, weight=self.norm2.weight, bias=self.norm2.bias, y=norm, eps=self.norm2.eps)
        attn_out = self.attn2(norm, encoder_hidden_states=encoder_hidden_states)
        norm = M.residual_ln_modulate(h, attn_out, c_scale_msa, c_shift_msa, self.norm3.eps)
        M.gate_residual(h, self.ffn(norm), c_gate_msa)
        return h


def _row_ops_ok(x: torch.Tensor) -> bool:
    return (x.is_cuda and x.dtype == torch.bfloat16 and x.dim() == 3 and x.shape[-1] % 8 == 0
            and x.shape[-1] <= 8192)


def rope_1d(dim: int, positions: int, theta: float = 10000.0) -> torch.Tensor:
    """complex128 [positions, dim/2]: exp(i * p * theta^(-2j/dim))."""
    inv = 1.0 / (theta ** (torch.arange(0, dim, 2, dtype=torch.float64)[: dim // 2] / dim))
    ang = torch.outer(torch.arange(positions, dtype=torch.float64), inv)
    return torch.polar(torch.ones_like(ang), ang)


class WanRotaryPosEmbed(nn.Module):
    """3D RoPE: the head's channel pairs split over (frame, height, width) as
    (D/2 - 2*(D//6), D//6, D//6) pairs, each a 1D table of its axis position."""

    def __init__(self, head_dim: int, patch_size, max_seq_len: int):
        super().__init__()
        self.head_dim = head_dim
        self.patch_size = patch_size
        hw = 2 * (head_dim // 6)
        t = head_dim - 2 * hw
        # A plain attribute, not a buffer: Module.to(dtype) would cast a complex buffer to a
        # real dtype and drop its imaginary part.
        self.freqs = torch.cat([rope_1d(t, max_seq_len), rope_1d(hw, max_seq_len), rope_1d(hw, max_seq_len)],
                               dim=1)

    def forward(self, hidden_states: torch.Tensor) -> torch.Tensor:
        _, _, f, h, w = hidden_states.shape
        pt, ph, pw = self.patch_size
        nf, nh, nw = f // pt, h // ph, w // pw
        d6 = self.head_dim // 6
        if self.freqs.device != hidden_states.device:
            self.freqs = self.freqs.to(hidden_states.device)
        ft, fh, fw = self.freqs.split([self.head_dim // 2 - 2 * d6, d6, d6], dim=1)
        grid = torch.cat([ft[:nf].view(nf, 1, 1, -1).expand(nf, nh, nw, -1),
                          fh[:nh].view(1, nh, 1, -1).expand(nf, nh, nw, -1),
                          fw[:nw].view(1, 1, nw, -1).expand(nf, nh, nw, -1)], dim=-1)
        return grid.reshape(1, 1, nf * nh * nw, -1)


def timestep_embedding(t: torch.Tensor, dim: int, max_period: float = 10000.0) -> torch.Tensor:
    """Sinusoidal embedding [cos | sin] of the timesteps (float32)."""
    half = dim // 2
    freqs = torch.exp(-math.log(max_period) * torch.arange(half, dtype=torch.float32, device=t.device) / half)
    ang = t[:, None].float() * freqs[None]
    return torch.cat([torch.cos(ang), torch.sin(ang)], dim=-1)


class WanDiT(nn.Module):
    """WanTransformer3DModel: patch embedding, time / text conditioning, 3D RoPE,
    ``num_layers`` blocks, modulated output norm, projection and unpatchify."""

    def __init__(self, cfg: Optional[WanDiTConfig] = None):
        super().__init__()
        cfg = cfg or WanDiTConfig()
        self.cfg = cfg
        self.config = SimpleNamespace(patch_size=tuple(cfg.patch_size), num_layers=cfg.num_layers)
        dim = cfg.inner_dim
        self.rope = WanRotaryPosEmbed(cfg.attention_head_dim, cfg.patch_size, cfg.rope_max_seq_len)
        self.patch_embedding = nn.Conv3d(cfg.in_channels, dim, kernel_size=cfg.patch_size, stride=cfg.patch_size)
        self.time_embedder = nn.Sequential(nn.Linear(cfg.freq_dim, dim), nn.SiLU(), nn.Linear(dim, dim))
        self.time_proj = nn.Sequential(nn.SiLU(), nn.Linear(dim, 6 * dim))
        self.text_embedder = nn.Sequential(nn.Linear(cfg.text_dim, dim), nn.GELU(approximate="tanh"),
                                           nn.Linear(dim, dim))
        self.blocks = nn.ModuleList([WanBlock(cfg) for _ in range(cfg.num_layers)])
        self.norm_out = FP32LayerNorm(dim, cfg.eps, elementwise_affine=False)
        self.proj_out = nn.Linear(dim, cfg.out_channels * math.prod(cfg.patch_size))
        self.scale_shift_table = nn.Parameter(torch.randn(1, 2, dim) / dim ** 0.5)

    def forward(self, hidden_states: torch.Tensor, timestep: torch.Tensor,
                encoder_hidden_states: torch.Tensor) -> torch.Tensor:
        b, _, f, h, w = hidden_states.shape
        pt, ph, pw = self.cfg.patch_size
        nf, nh, nw = f // pt, h // ph, w // pw
        rotary_emb = self.rope(hidden_states)
        x = self.patch_embedding(hidden_states).flatten(2).transpose(1, 2).contiguous()

        wdtype = self.time_embedder[0].weight.dtype
        temb = self.time_embedder(timestep_embedding(timestep, self.cfg.freq_dim).to(wdtype))
        temb = temb.type_as(encoder_hidden_states)
        tproj = self.time_proj(temb).unflatten(1, (6, -1))
        text = self.text_embedder(encoder_hidden_states)

        for block in self.blocks:
            x = block(x, text, tproj, rotary_emb, timestep=timestep)

        shift, scale = (self.scale_shift_table + temb.unsqueeze(1)).chunk(2, dim=1)
        x = (self.norm_out(x.float()) * (1 + scale) + shift).type_as(x)
        return unpatchify(self.proj_out(x), (nf, nh, nw), self.cfg.patch_size)


def unpatchify(x: torch.Tensor, grid, patch) -> torch.Tensor:
    """[B, nf*nh*nw, pt*ph*pw*C] tokens -> [B, C, nf*pt, nh*ph, nw*pw]: channel c of
    pixel (f*pt + a, y*ph + i, x*pw + j) is element ((a*ph + i)*pw + j)*C + c of token
    (f*nh + y)*nw + x."""
    (nf, nh, nw), (pt, ph, pw) = grid, patch
    x = x.reshape(x.shape[0], nf, nh, nw, pt, ph, pw, -1).permute(0, 7, 1, 4, 2, 5, 3, 6)
    return x.flatten(6, 7).flatten(4, 5).flatten(2, 3)


class WanPipelineShape:
    """What ``replace_wan_attention`` reads from a diffusers WanPipeline: the
    transformer and the VAE's temporal / spatial compression factors."""

    def __init__(self, transformer: WanDiT, vae_scale_factor_temporal: int = 4, vae_scale_factor_spatial: int = 8):
        self.transformer = transformer
        self.vae_scale_factor_temporal = vae_scale_factor_temporal
        self.vae_scale_factor_spatial = vae_scale_factor_spatial


def latent_shape(num_frames: int, height: int, width: int, channels: int = 16, temporal: int = 4,
                 spatial: int = 8) -> Tuple[int, int, int, int]:
    """[C, F, H, W] of the VAE latent of a ``num_frames`` x ``height`` x ``width`` video."""
    return channels, 1 + (num_frames - 1) // temporal, height // spatial, width // spatial
