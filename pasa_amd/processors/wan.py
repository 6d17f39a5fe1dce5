"""Wan2.1 attention processor with PISA-PG sparse attention, and its installer.

Drop-in for the reference's Wan path (svg/models/wan/attention.py and
svg/models/wan/inference.py): same class names, constructor, class-attribute
configuration and call protocol of the diffusers attention processor

    processor(attn, hidden_states, encoder_hidden_states=None, attention_mask=None,
              rotary_emb=None, timestep=None) -> Tensor[B, S, C]

(svg/models/wan/attention.py:166-174).  Self-attention calls carry ``timestep``
(passed in, or taken from the forward hook of ``timestep_hook``); cross-attention
calls (timestep None) run dense SDPA, as in the reference (:218-221).  The sparse branch calls ``pasa_amd.ops.pisa_pg_attention``: the
reference calls the undefined name ``piecewise_sparse_attention`` at :384 while
importing ``pisa_pg_attention`` at :15, the only complete PISA op in its tree.
Left out (not on the hot path): the per-layer hidden-state L1 JSONL logging
(:182-258), flex/FlashInfer SVG masks (:290-348) and sample_mse (:264-288).
"""
from __future__ import annotations

import os
from typing import Optional

import torch
import torch.nn.functional as F

from .. import density as _density
from ..ops import pisa_pg_attention
from ..prologue import qkv_prologue, rope_tables_complex
from . import dense as _dense
from .qknorm import fusable, is_rmsnorm, norm_eps, rms_norm_once
from .rope import apply_rotary_emb_complex
from .timestep_hook import current_timestep, install_wan


class WanAttn_SVGAttn_Processor2_0:
    """Base processor (reference :93-301): projections, QK-norm, RoPE, dispatch, output."""
    version = None
    context_length = 0
    num_frame = 0
    frame_size = 0

    first_layers_fp = 0
    first_times_fp = 0

    num_sampled_rows = 32
    attention_masks = None
    sparsity = 0
    # bf16 device inputs: QK-norm, head split and RoPE in one HIP pass (pasa_amd.prologue).
    fused_prologue = True

    def __init__(self, layer_idx):
        self.layer_idx = layer_idx
        if not hasattr(F, "scaled_dot_product_attention"):
            raise ImportError("the Wan processors need torch.nn.functional.scaled_dot_product_attention (PyTorch >= 2.0)")

    def get_qkv(self, attn, hidden_states, encoder_hidden_states):
        return attn.to_q(hidden_states), attn.to_k(encoder_hidden_states), attn.to_v(encoder_hidden_states)

    def get_qk_norm(self, attn, query, key):
        # RMSNorm over the full hidden width, before the head split, with the Triton
        # rmsnorm's single rounding (reference :122-136).
        if attn.norm_q is not None:
            if not is_rmsnorm(attn.norm_q):
                raise ValueError(f"norm_q is {type(attn.norm_q).__name__}; only RMSNorm is handled")
            query = rms_norm_once(query, attn.norm_q.weight, norm_eps(attn.norm_q, query.dtype))
        if attn.norm_k is not None:
            if not is_rmsnorm(attn.norm_k):
                raise ValueError(f"norm_k is {type(attn.norm_k).__name__}; only RMSNorm is handled")
            key = rms_norm_once(key, attn.norm_k.weight, norm_eps(attn.norm_k, key.dtype))
        return query, key

    def fused_qkv(self, attn, hidden_states, encoder_hidden_states, rotary_emb):
        """get_qkv + get_qk_norm + get_transpose_qkv + get_rotary_emb in one kernel
        pass; None when the inputs are outside what the kernel reproduces."""
        H = attn.heads
        C = hidden_states.shape[-1]
        norms = (attn.norm_q, attn.norm_k)
        if not all(m is None or is_rmsnorm(m) for m in norms):
            return None
        if not fusable(hidden_states, H, norms, C) or encoder_hidden_states.dtype != hidden_states.dtype:
            return None
        query = attn.to_q(hidden_states)
        key, value = attn.to_k(encoder_hidden_states), attn.to_v(encoder_hidden_states)
        if query.shape[-1] != C or key.shape[-1] != C or not (query.is_contiguous() and key.is_contiguous()
                                                               and value.is_contiguous()):
            return None
        D = C // H
        rope = None
        if rotary_emb is not None:
            re, im = rope_tables_complex(rotary_emb, query.device, query.shape[1], D // 2)
            rope = ("complex", re, im)
        wq = None if attn.norm_q is None else attn.norm_q.weight
        wk = None if attn.norm_k is None else attn.norm_k.weight
        eq = norm_eps(attn.norm_q, query.dtype) if attn.norm_q is not None else 0.0
        ek = norm_eps(attn.norm_k, key.dtype) if attn.norm_k is not None else eq
        row = lambda *ws: "row" if any(w is not None for w in ws) else None
        if query.shape == key.shape and (wq is None or wk is None or eq == ek):
            return qkv_prologue(query, key, value, H, wq=wq, wk=wk, norm=row(wq, wk), rounding="once",
                                eps=eq if wq is not None else ek, rope=rope)
        # cross-attention (different lengths) or different eps: Q alone, then K and V
        (q, _, _) = qkv_prologue(query, None, None, H, wq=wq, norm=row(wq), rounding="once", eps=eq,
                                 rope=rope)
        (_, k, v) = qkv_prologue(None, key, value, H, wk=wk, norm=row(wk), rounding="once", eps=ek,
                                 rope=rope if key.shape[1] == query.shape[1] else None)
        return q, k, v

    def get_transpose_qkv(self, attn, query, key, value):
        query = query.unflatten(2, (attn.heads, -1)).transpose(1, 2).contiguous()
        key = key.unflatten(2, (attn.heads, -1)).transpose(1, 2).contiguous()
        value = value.unflatten(2, (attn.heads, -1)).transpose(1, 2).contiguous()
        return query, key, value

    def get_rotary_emb(self, query, key, rotary_emb):
        if rotary_emb is not None:
            query = apply_rotary_emb_complex(query, rotary_emb)
            key = apply_rotary_emb_complex(key, rotary_emb)
        return query, key

    def get_o(self, attn, query, hidden_states, hidden_states_img):
        hidden_states = hidden_states.transpose(1, 2).flatten(2, 3)
        hidden_states = hidden_states.type_as(query)
        if hidden_states_img is not None:
            hidden_states = hidden_states + hidden_states_img
        hidden_states = attn.to_out[0](hidden_states)
        hidden_states = attn.to_out[1](hidden_states)
        return hidden_states

    def __call__(self, attn, hidden_states: torch.Tensor,
                 encoder_hidden_states: Optional[torch.Tensor] = None,
                 attention_mask: Optional[torch.Tensor] = None,
                 rotary_emb: Optional[torch.Tensor] = None,
                 timestep=None) -> torch.Tensor:
        encoder_hidden_states_img = None
        self_attention = encoder_hidden_states is None
        if getattr(attn, "add_k_proj", None) is not None:
            encoder_hidden_states_img = encoder_hidden_states[:, :257]
            encoder_hidden_states = encoder_hidden_states[:, 257:]
        if encoder_hidden_states is None:
            encoder_hidden_states = hidden_states

        qkv = (self.fused_qkv(attn, hidden_states, encoder_hidden_states, rotary_emb)
               if self.fused_prologue else None)
        if qkv is not None:
            query, key, value = qkv
        else:
            query, key, value = self.get_qkv(attn, hidden_states, encoder_hidden_states)
            query, key = self.get_qk_norm(attn, query, key)
            query, key, value = self.get_transpose_qkv(attn, query, key, value)
            query, key = self.get_rotary_emb(query, key, rotary_emb)

        hidden_states_img = None
        if encoder_hidden_states_img is not None:  # I2V image branch (reference :195-208)
            key_img = attn.norm_added_k(attn.add_k_proj(encoder_hidden_states_img))
            value_img = attn.add_v_proj(encoder_hidden_states_img)
            key_img = key_img.unflatten(2, (attn.heads, -1)).transpose(1, 2)
            value_img = value_img.unflatten(2, (attn.heads, -1)).transpose(1, 2)
            hidden_states_img = F.scaled_dot_product_attention(query, key_img, value_img, dropout_p=0.0,
                                                               is_causal=False)
            hidden_states_img = hidden_states_img.transpose(1, 2).flatten(2, 3).type_as(query)

        if timestep is None and self_attention:
            timestep = current_timestep()      # set by the installed forward hook
        if timestep is None:  # cross-attention
            hidden_states = F.scaled_dot_product_attention(query, key, value, attn_mask=attention_mask,
                                                           dropout_p=0.0, is_causal=False)
        else:
            hidden_states = self.attention_core_logic(query, key, value, timestep)
        return self.get_o(attn, query, hidden_states, hidden_states_img)

    def flash_attention(self, query, key, value):
        """Dense attention (reference :299-301): the HIP exact-tile path for bf16 device
        tensors with head_dim 128, else PyTorch SDPA (``processors.dense``)."""
        return _dense.attention(query, key, value)

    def attention_core_logic(self, query, key, value, timestep):  # pragma: no cover - abstract
        raise NotImplementedError


class Wan_PASA_Processor(WanAttn_SVGAttn_Processor2_0):
    """PASA processor (reference :350-390)."""
    rescaled_density: dict = {}
    base_density = 0.15
    block_size = 64        # the reference's call site passes block_size=64 (:387)
    use_random = False
    logging_file = None
    num_layers = 0

    def __init__(self, layer_idx):
        super().__init__(layer_idx)
        self.layer_idx = layer_idx

    def attention_core_logic(self, query, key, value, timestep):
        cfg, num_heads, seq_len, dim = query.size()
        assert cfg == 1, f"the sparse path attends one sample per call, got a batch of {cfg}"
        context_length, num_frame, frame_size = self.context_length, self.num_frame, self.frame_size
        assert seq_len == context_length + num_frame * frame_size, (
            f"{seq_len} tokens, expected {context_length} text + {num_frame} frames x {frame_size}")

        full_attention_flag = False
        if self.layer_idx < self.first_layers_fp:
            full_attention_flag = True
        if timestep[0] > self.first_times_fp:
            full_attention_flag = True

        if full_attention_flag:
            out = self.flash_attention(query, key, value)
            return out.reshape(cfg, num_heads, seq_len, dim)

        ts_key = int(timestep[0].item()) if torch.is_tensor(timestep[0]) else int(timestep[0])
        density = self.rescaled_density.get(ts_key)
        assert density is not None, f"no density is scheduled for timestep {ts_key}"
        out = pisa_pg_attention(query.contiguous(), key.contiguous(), value.contiguous(),
                                density=density, block_size=self.block_size,
                                use_random=self.use_random)
        return out.reshape(cfg, num_heads, seq_len, dim)


def replace_sparse_forward():
    """Make the denoising timestep reach each block's self-attention processor.

    The reference replaces diffusers' WanTransformerBlock / WanTransformer3DModel
    forwards for this (svg/models/wan/custom_models.py:23-207); here the model's
    forward is wrapped instead (``timestep_hook``).  Returns False when diffusers is
    not importable; callers that pass ``timestep=`` to the processor need neither."""
    return install_wan()


def replace_wan_attention(pipe, height, width, num_frames, first_layers_fp, first_times_fp,
                          pattern="PASA", logging_file=None, base_density=0.15):
    """Install Wan_PASA_Processor on every block's self-attention (reference
    svg/models/wan/inference.py:12-74)."""
    context_length = 0
    num_frame_patches = 1 + num_frames // (pipe.vae_scale_factor_temporal * pipe.transformer.config.patch_size[0])
    mod_value = pipe.vae_scale_factor_spatial * pipe.transformer.config.patch_size[1]
    frame_patches_one_frame = int(height // mod_value) * int(width // mod_value)

    replace_sparse_forward()
    num_layers = len(pipe.transformer.blocks)

    if pattern != "PASA":
        raise ValueError(f"unknown attention pattern {pattern!r} (expected 'PASA')")
    if logging_file is not None:
        os.makedirs(os.path.dirname(logging_file) or ".", exist_ok=True)
        with open(logging_file, "w") as f:
            f.write("")

    AttnModule = Wan_PASA_Processor
    AttnModule.first_layers_fp = first_layers_fp
    AttnModule.first_times_fp = first_times_fp
    AttnModule.logging_file = logging_file
    AttnModule.context_length = context_length
    AttnModule.num_frame = num_frame_patches
    AttnModule.frame_size = frame_patches_one_frame
    AttnModule.num_layers = num_layers
    AttnModule.base_density = base_density
    AttnModule.rescaled_density = _density.wan_rescaled_density(base_density)

    for layer_idx, m in enumerate(pipe.transformer.blocks):
        if hasattr(m.attn1, "processor"):
            m.attn1.set_processor(AttnModule(layer_idx=layer_idx))
    print(f"[pasa_amd] {pattern} processors installed on {num_layers} attention layers")
