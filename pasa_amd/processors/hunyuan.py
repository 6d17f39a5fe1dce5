"""HunyuanVideo attention processors with PISA-PG sparse attention, and their installers.

Drop-in for the reference's HunyuanVideo path (svg/models/hyvideo/attention.py and
svg/models/hyvideo/inference.py): same class names, constructor, class-attribute
configuration and call protocol

    processor(attn, hidden_states, encoder_hidden_states=None, attention_mask=None,
              image_rotary_emb=None, timestep=None) -> (hidden_states, encoder_hidden_states)

(svg/models/hyvideo/attention.py:341-380).  The joint sequence is
[video tokens (frame-major), text tokens]; ``attention_mask`` ([B, 1, 1, N] bool,
built by the model, svg/models/hyvideo/custom_models.py:174-186) marks the valid
prefix.  Dense attention is block-diagonal over [0, valid) and [valid, N), the
reference's varlen call with cu_seqlens = [0, mask.sum(), N] (:315-323, :450-476);
here it is two PyTorch-ROCm SDPA calls on the two segments.

Notes on the reference:
* ``Hunyuan_PASA_Processor`` derives from ``Hunyuan_SAPAttn_Processor2_0`` (:644),
  a name the module never defines; the evident base is ``Hunyuan_SVGAttn_Processor2_0``
  (:234), which this module uses.
* With ``use_group=False`` the reference calls ``piecewise_sparse_attention``
  (svg/kernels/triton/pisa_attention.py), a different operator that is outside this
  build; that setting raises ``NotImplementedError``.
* The sparse call passes the whole joint sequence, text tokens included, to
  ``pisa_pg_attention`` with block_size=64 (:680): text tokens are ordinary tokens.
  ``text_segment = True`` (class attribute) instead treats the trailing
  ``context_length`` tokens as a text segment (``pisa_pg_attention(text_tokens=...)``)
  and honours the attention mask there as the dense path does: the text tokens past
  the mask's valid prefix are padding (``text_valid=...``), a segment of their own.
Left out (not on the hot path): sample_mse / flex-attention SVG masks (:382-411).
"""
from __future__ import annotations

import os
from typing import Optional, Tuple

import torch
import torch.nn.functional as F

from .. import density as _density
from ..ops import pisa_pg_attention
from ..placement import hunyuan_hidden_states_placement, hunyuan_sparse_head_placement
from ..prologue import qkv_prologue, rope_tables_cossin
from . import dense as _dense
from .qknorm import fusable, module_rounding, norm_eps
from .rope import apply_rotary_emb_cos_sin
from .timestep_hook import current_timestep, install_hunyuan


def _split_heads(attn, x):
    return x.unflatten(2, (attn.heads, -1)).transpose(1, 2)


def block_diagonal_attention(query, key, value, valid: int):
    """softmax attention restricted to [0, valid) x [0, valid) and [valid, N) x [valid, N)
    (the HIP dense path for bf16 device tensors, see ``processors.dense``)."""
    return _dense.attention(query, key, value, valid)


def _valid_length(attention_mask, n: int) -> int:
    if attention_mask is None:
        return n
    return int(attention_mask.sum().item())


def fused_hunyuan_qkv(attn, hidden_states, encoder_hidden_states, image_rotary_emb):
    """Projections, per-head QK-norm, RoPE (video rows) and the text concat of the
    HunyuanVideo processors (reference :52-100, :248-300) with the fused prologue
    kernel: one pass per stream, written straight into the joint [B, H, N, D]
    tensors.  Returns None when the inputs are outside what the kernel reproduces."""
    H = attn.heads
    C = hidden_states.shape[-1]
    if C % H:
        return None
    D = C // H
    joint = attn.add_q_proj is not None and encoder_hidden_states is not None
    dt = hidden_states.dtype

    def norm_args(mq, mk):
        """(norm, rounding, eps) of one kernel call, or None if the pair is not reproducible."""
        present = [m for m in (mq, mk) if m is not None]
        if not present:
            return None, "once", 0.0
        rnd = {module_rounding(m) for m in present}
        eps = {norm_eps(m, dt) for m in present}
        if None in rnd or len(rnd) > 1 or len(eps) > 1:
            return None
        return "head", rnd.pop(), eps.pop()

    video = norm_args(attn.norm_q, attn.norm_k)
    text = norm_args(attn.norm_added_q, attn.norm_added_k) if joint else (None, "once", 0.0)
    norms = [attn.norm_q, attn.norm_k] + ([attn.norm_added_q, attn.norm_added_k] if joint else [])
    if video is None or text is None or not fusable(hidden_states, H, norms, D):
        return None
    w = lambda m: None if m is None else m.weight

    single_text = attn.add_q_proj is None and encoder_hidden_states is not None
    x = torch.cat([hidden_states, encoder_hidden_states], dim=1) if single_text else hidden_states
    q_in, k_in, v_in = attn.to_q(x), attn.to_k(x), attn.to_v(x)
    if not (q_in.is_contiguous() and k_in.is_contiguous() and v_in.is_contiguous()):
        return None
    B, S = x.shape[0], x.shape[1]
    txt = encoder_hidden_states.shape[1] if encoder_hidden_states is not None else 0
    N = S + txt if joint else S
    rope, rope_rows = None, None
    if image_rotary_emb is not None:
        cos, sin = rope_tables_cossin(image_rotary_emb[0], image_rotary_emb[1], x.device)
        rope_rows = S - txt if single_text else S
        if cos.shape != (rope_rows, D) or sin.shape != (rope_rows, D):
            return None
        rope = ("cossin", cos, sin)
    outs = [torch.empty(B, H, N, D, device=x.device, dtype=x.dtype) for _ in range(3)]
    qkv_prologue(q_in, k_in, v_in, H, wq=w(attn.norm_q), wk=w(attn.norm_k), norm=video[0], rounding=video[1],
                 eps=video[2], rope=rope, rope_rows=rope_rows, out=outs, out_seq_len=N)
    if joint:
        e = encoder_hidden_states
        eq, ek, ev = attn.add_q_proj(e), attn.add_k_proj(e), attn.add_v_proj(e)
        qkv_prologue(eq.contiguous(), ek.contiguous(), ev.contiguous(), H, wq=w(attn.norm_added_q),
                     wk=w(attn.norm_added_k), norm=text[0], rounding=text[1], eps=text[2], out=outs,
                     out_seq_len=N, out_row0=S)
    return tuple(outs)


def _rope_single(query, key, image_rotary_emb, txt_len):
    """RoPE on the video part of a single-stream sequence (text last) (:211-223)."""
    img_q, txt_q = query[:, :, :-txt_len], query[:, :, -txt_len:]
    img_k, txt_k = key[:, :, :-txt_len], key[:, :, -txt_len:]
    img_q = apply_rotary_emb_cos_sin(img_q, image_rotary_emb)
    img_k = apply_rotary_emb_cos_sin(img_k, image_rotary_emb)
    return torch.cat([img_q, txt_q], dim=2), torch.cat([img_k, txt_k], dim=2)


class HunyuanVideoAttnProcessor2_0_FlashAttention:
    """Dense processor (reference :41-157): the model's masked attention as block-diagonal
    varlen attention."""

    def __init__(self, layer_idx):
        self.layer_idx = layer_idx
        if not hasattr(F, "scaled_dot_product_attention"):
            raise ImportError("the HunyuanVideo processors need torch.nn.functional.scaled_dot_product_attention (PyTorch >= 2.0)")

    fused_prologue = True

    def __call__(self, attn, hidden_states, encoder_hidden_states=None, attention_mask=None,
                 image_rotary_emb=None):
        qkv = (fused_hunyuan_qkv(attn, hidden_states, encoder_hidden_states, image_rotary_emb)
               if self.fused_prologue else None)
        if qkv is not None:
            query, key, value = qkv
            return self._attend_and_project(attn, query, key, value, encoder_hidden_states, attention_mask)
        if attn.add_q_proj is None and encoder_hidden_states is not None:
            hidden_states = torch.cat([hidden_states, encoder_hidden_states], dim=1)
        query = _split_heads(attn, attn.to_q(hidden_states))
        key = _split_heads(attn, attn.to_k(hidden_states))
        value = _split_heads(attn, attn.to_v(hidden_states))
        if attn.norm_q is not None:
            query = attn.norm_q(query)
        if attn.norm_k is not None:
            key = attn.norm_k(key)
        if image_rotary_emb is not None:
            if attn.add_q_proj is None and encoder_hidden_states is not None:
                query, key = _rope_single(query, key, image_rotary_emb, encoder_hidden_states.shape[1])
            else:
                query = apply_rotary_emb_cos_sin(query, image_rotary_emb)
                key = apply_rotary_emb_cos_sin(key, image_rotary_emb)
        if attn.add_q_proj is not None and encoder_hidden_states is not None:
            eq = _split_heads(attn, attn.add_q_proj(encoder_hidden_states))
            ek = _split_heads(attn, attn.add_k_proj(encoder_hidden_states))
            ev = _split_heads(attn, attn.add_v_proj(encoder_hidden_states))
            if attn.norm_added_q is not None:
                eq = attn.norm_added_q(eq)
            if attn.norm_added_k is not None:
                ek = attn.norm_added_k(ek)
            query = torch.cat([query, eq], dim=2)
            key = torch.cat([key, ek], dim=2)
            value = torch.cat([value, ev], dim=2)
        return self._attend_and_project(attn, query, key, value, encoder_hidden_states, attention_mask)

    def _attend_and_project(self, attn, query, key, value, encoder_hidden_states, attention_mask):
        out = block_diagonal_attention(query, key, value, _valid_length(attention_mask, query.shape[2]))
        out = out.transpose(1, 2).flatten(2, 3).to(query.dtype)
        if encoder_hidden_states is not None:
            out, encoder_hidden_states = out[:, : -encoder_hidden_states.shape[1]], \
                out[:, -encoder_hidden_states.shape[1]:]
            if getattr(attn, "to_out", None) is not None:
                out = attn.to_out[0](out)
                out = attn.to_out[1](out)
            if getattr(attn, "to_add_out", None) is not None:
                encoder_hidden_states = attn.to_add_out(encoder_hidden_states)
        return out, encoder_hidden_states


class Hunyuan_SVGAttn_Processor2_0:
    """Base processor (reference :234-531): projections, QK-norm, RoPE, text concat,
    dispatch, output projection."""
    num_sampled_rows = 32
    attention_masks = None

    prompt_length = 0
    context_length = 256
    num_frame = 33
    frame_size = 3600

    first_layers_fp = 0
    first_times_fp = 0
    # bf16 device inputs: projections' QK-norm, RoPE and text concat in fused HIP passes.
    fused_prologue = True

    def __init__(self, layer_idx):
        self.layer_idx = layer_idx
        if not hasattr(F, "scaled_dot_product_attention"):
            raise ImportError("the HunyuanVideo processors need torch.nn.functional.scaled_dot_product_attention (PyTorch >= 2.0)")

    def get_qkv(self, attn, hidden_states):
        return attn.to_q(hidden_states), attn.to_k(hidden_states), attn.to_v(hidden_states)

    def get_transpose_qkv(self, attn, query, key, value):
        return (_split_heads(attn, query).contiguous(), _split_heads(attn, key).contiguous(),
                _split_heads(attn, value).contiguous())

    def get_qk_norm(self, attn, query, key):
        # Per-head RMSNorm over D, after the head split (reference :275-278, :204-209).
        if attn.norm_q is not None:
            query = attn.norm_q(query)
        if attn.norm_k is not None:
            key = attn.norm_k(key)
        return query, key

    def get_rotary_emb(self, attn, query, key, image_rotary_emb, encoder_hidden_states):
        if image_rotary_emb is not None:
            if attn.add_q_proj is None and encoder_hidden_states is not None:
                query, key = _rope_single(query, key, image_rotary_emb, encoder_hidden_states.shape[1])
            else:
                query = apply_rotary_emb_cos_sin(query, image_rotary_emb)
                key = apply_rotary_emb_cos_sin(key, image_rotary_emb)
        return query, key

    def get_encoder_condition_and_concat(self, attn, query, key, value, encoder_hidden_states):
        if attn.add_q_proj is not None and encoder_hidden_states is not None:
            eq = _split_heads(attn, attn.add_q_proj(encoder_hidden_states))
            ek = _split_heads(attn, attn.add_k_proj(encoder_hidden_states))
            ev = _split_heads(attn, attn.add_v_proj(encoder_hidden_states))
            if attn.norm_added_q is not None:
                eq = attn.norm_added_q(eq)
            if attn.norm_added_k is not None:
                ek = attn.norm_added_k(ek)
            query = torch.cat([query, eq], dim=2)
            key = torch.cat([key, ek], dim=2)
            value = torch.cat([value, ev], dim=2)
        return query, key, value

    def get_cu_max_seqlen(self, attention_mask, device):
        """(cu_seqlens_q, cu_seqlens_kv, max_seqlen_q, max_seqlen_kv) of the two segments (:315-323)."""
        n = attention_mask.numel()
        cu = torch.tensor([0, int(attention_mask.sum().item()), n], dtype=torch.int32, device=device)
        return cu, cu.clone(), n, n

    def get_o(self, attn, hidden_states, encoder_hidden_states):
        if encoder_hidden_states is not None:
            hidden_states, encoder_hidden_states = (hidden_states[:, : -encoder_hidden_states.shape[1]],
                                                    hidden_states[:, -encoder_hidden_states.shape[1]:])
            if getattr(attn, "to_out", None) is not None:
                hidden_states = attn.to_out[0](hidden_states)
                hidden_states = attn.to_out[1](hidden_states)
            if getattr(attn, "to_add_out", None) is not None:
                encoder_hidden_states = attn.to_add_out(encoder_hidden_states)
        return hidden_states, encoder_hidden_states

    def __call__(self, attn, hidden_states: torch.Tensor,
                 encoder_hidden_states: Optional[torch.Tensor] = None,
                 attention_mask: Optional[torch.Tensor] = None,
                 image_rotary_emb=None, timestep=None):
        qkv = (fused_hunyuan_qkv(attn, hidden_states, encoder_hidden_states, image_rotary_emb)
               if self.fused_prologue else None)
        if qkv is not None:
            query, key, value = qkv
        else:
            if attn.add_q_proj is None and encoder_hidden_states is not None:
                hidden_states = torch.cat([hidden_states, encoder_hidden_states], dim=1)
            query, key, value = self.get_qkv(attn, hidden_states)
            query, key, value = self.get_transpose_qkv(attn, query, key, value)
            query, key = self.get_qk_norm(attn, query, key)
            query, key = self.get_rotary_emb(attn, query, key, image_rotary_emb, encoder_hidden_states)
            query, key, value = self.get_encoder_condition_and_concat(attn, query, key, value,
                                                                      encoder_hidden_states)
        if attention_mask is None:
            attention_mask = torch.ones(query.shape[2], dtype=torch.bool, device=query.device)
        if timestep is None:
            timestep = current_timestep()      # set by the installed forward hook
        cu_max_seqlens = self.get_cu_max_seqlen(attention_mask, query.device)
        hidden_states = self.attention_core_logic(query, key, value, timestep, self.layer_idx, cu_max_seqlens)
        hidden_states = hidden_states.transpose(1, 2).flatten(2, 3).to(query.dtype)
        return self.get_o(attn, hidden_states, encoder_hidden_states)

    def flash_attention(self, query, key, value, cu_max_seqlens):
        """Dense block-diagonal attention over the two cu_seqlens segments (:459-476)."""
        cu = cu_max_seqlens[0]
        return block_diagonal_attention(query, key, value, int(cu[1].item()))

    def flashinfer_attention(self, query, key, value, cu_max_seqlens):
        """Same semantics as ``flash_attention`` (the reference's FlashInfer variant, :450-457)."""
        return self.flash_attention(query, key, value, cu_max_seqlens)

    def sparse_head_placement(self, query, key, value, query_out, key_out, value_out, best_mask_idx,
                              context_length, num_frame, frame_size):
        hunyuan_sparse_head_placement(query, key, value, query_out, key_out, value_out, best_mask_idx,
                                      context_length, num_frame, frame_size)
        return query_out, key_out, value_out

    fast_sparse_head_placement = sparse_head_placement

    def hidden_states_placement(self, hidden_states, output_hidden_states, best_mask_idx, context_length,
                                num_frame, frame_size):
        hunyuan_hidden_states_placement(hidden_states, output_hidden_states, best_mask_idx, context_length,
                                        num_frame, frame_size)

    fast_hidden_states_placement = hidden_states_placement

    def attention_core_logic(self, query, key, value, timestep, layer_idx, cu_max_seqlens):
        """Dense by default; subclasses override the sparse branch."""
        cfg, num_heads, seq_len, dim = query.size()
        return self.flash_attention(query, key, value, cu_max_seqlens).reshape(cfg, num_heads, seq_len, dim)


class Hunyuan_PASA_Processor(Hunyuan_SVGAttn_Processor2_0):
    """PASA processor (reference :644-683)."""
    rescaled_density: dict = {}
    base_density = 0.15
    use_group = True
    use_random = True
    block_size = 64        # the reference's call site passes block_size=64 (:680)
    logging_file = None
    # False (the reference): the text tokens are ordinary tokens of the sparse call.
    # True: the last context_length tokens are a text segment (exact prompt keys for
    # every video query block, dense text rows, the mask's padding a segment of its
    # own as in the dense path); needs head_dim 128.
    text_segment = False

    def __init__(self, layer_idx):
        super().__init__(layer_idx)

    def attention_core_logic(self, query, key, value, timestep, layer_idx, cu_max_seqlens):
        cfg, num_heads, seq_len, dim = query.size()
        assert cfg == 1, f"the sparse path attends one sample per call, got a batch of {cfg}"
        context_length, num_frame, frame_size = self.context_length, self.num_frame, self.frame_size
        assert seq_len == context_length + num_frame * frame_size, (
            f"{seq_len} tokens, expected {context_length} text + {num_frame} frames x {frame_size}")

        full_attention_flag = False
        if self.layer_idx < self.first_layers_fp:
            full_attention_flag = True
        if timestep is None or timestep[0] > self.first_times_fp:
            full_attention_flag = True

        if full_attention_flag:
            out = self.flashinfer_attention(query, key, value, cu_max_seqlens)
            return out.reshape(cfg, num_heads, seq_len, dim)

        ts = int(timestep[0].item()) if torch.is_tensor(timestep[0]) else int(timestep[0])
        density = _density.lookup_rescaled_density(self.rescaled_density, ts)
        assert density is not None, f"no density is scheduled for timestep {ts}"
        if not self.use_group:
            raise NotImplementedError("use_group=False selects piecewise_sparse_attention "
                                      "(svg/kernels/triton/pisa_attention.py), which this build does not provide")
        extra = {}
        if self.text_segment:
            video = seq_len - context_length
            valid = int(cu_max_seqlens[0][1])   # cu_seqlens [0, valid, N]
            extra = {"text_tokens": context_length, "text_valid": min(max(valid - video, 0), context_length)}
        out = pisa_pg_attention(query.contiguous(), key.contiguous(), value.contiguous(), density=density,
                                block_size=self.block_size, use_random=self.use_random, **extra)
        return out.reshape(cfg, num_heads, seq_len, dim)


def replace_sparse_forward() -> bool:
    """Make the denoising timestep reach every block's attention processor.

    The reference replaces diffusers' HunyuanVideo block and model forwards for this
    (svg/models/hyvideo/custom_models.py:16-263); here the model's forward is wrapped
    (``timestep_hook``).  False when diffusers is not importable."""
    return install_hunyuan()


def replace_hyvideo_flashattention(pipe):
    """Install the dense processor on every double- and single-stream block (reference
    svg/models/hyvideo/inference.py:14-28)."""
    n_double = len(pipe.transformer.transformer_blocks)
    for layer_idx, m in enumerate(pipe.transformer.transformer_blocks):
        m.attn.processor = HunyuanVideoAttnProcessor2_0_FlashAttention(layer_idx=layer_idx)
    for layer_idx, m in enumerate(pipe.transformer.single_transformer_blocks):
        m.attn.processor = HunyuanVideoAttnProcessor2_0_FlashAttention(layer_idx=layer_idx + n_double)


def replace_hyvideo_attention(pipe, height, width, num_frames, prompt_length, first_layers_fp, first_times_fp,
                              pattern="PASA", logging_file=None, base_density=0.15, use_dynamic=True,
                              use_group=True, use_random=True) -> float:
    """Configure and install Hunyuan_PASA_Processor (reference svg/models/hyvideo/inference.py:31-92).

    The latent grid follows the reference: 256 context (text) tokens, 1 + num_frames // 4
    latent frames of height * width / 256 tokens.  Returns width / frame_size as the
    reference does."""
    context_length, num_frame = 256, 1 + num_frames // 4
    frame_size = height * width // 256
    if pattern == "PASA":
        if logging_file is not None:
            os.makedirs(os.path.dirname(logging_file) or ".", exist_ok=True)
            with open(logging_file, "w") as f:
                f.write("")
        M = Hunyuan_PASA_Processor
        M.prompt_length = prompt_length
        M.context_length = context_length
        M.num_frame = num_frame
        M.frame_size = frame_size
        M.first_layers_fp = first_layers_fp
        M.first_times_fp = first_times_fp
        M.logging_file = logging_file
        M.base_density = base_density
        M.use_group = use_group
        M.use_random = use_random
        M.rescaled_density = _density.hunyuan_rescaled_density(base_density, use_dynamic)
        replace_sparse_forward()
        n_double = len(pipe.transformer.transformer_blocks)
        for layer_idx, m in enumerate(pipe.transformer.transformer_blocks):
            m.attn.processor = M(layer_idx=layer_idx)
        for layer_idx, m in enumerate(pipe.transformer.single_transformer_blocks):
            m.attn.processor = M(layer_idx=layer_idx + n_double)
    elif pattern != "dense":
        raise ValueError(f"unknown attention pattern {pattern!r} (expected 'PASA' or 'dense')")
    return width / frame_size
