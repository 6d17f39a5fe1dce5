"""PISA-PG sparse attention on MI355X: the Python operator layer.

``pisa_pg_attention`` keeps the signature of the reference operator
(svg/kernels/triton/group_pisa_attention.py:307-318) so that the attention
processors call it unchanged.  Each stage is also exposed on its own:

* ``block_stats``        K2  (reference :66-129, :268-301)
* ``select_blocks``      K3  (reference :365-375)
* ``select_from_scores`` K3's top-k on given scores (bit-exact parity entry)
* ``sparse_attn``        K4  (reference :135-262)
* ``dense_attention``    K4's exact-tile path without selection (dense warm-up layers)

All device work goes through libpasa_amd.so (ctypes, ``pasa_amd._lib``).  This
module allocates outputs and workspace with torch's caching allocator and passes
torch's current HIP stream; nothing here synchronises.  There is no CPU path:
tensors must live on a ROCm device and the library must be built.
"""
from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass
from typing import Optional

import torch

from . import _lib

_DTYPES = {torch.bfloat16: _lib.DTYPE_BF16, torch.float16: _lib.DTYPE_F16, torch.float32: _lib.DTYPE_F32}

GROUP_SIZE = 32


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _check_device(*ts: torch.Tensor) -> None:
    for t in ts:
        if not t.is_cuda:
            raise ValueError("PISA kernels need ROCm device tensors (there is no CPU path)")
        if not t.is_contiguous():
            raise ValueError("PISA kernels need contiguous tensors")


def _check_qkv(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> None:
    """q, k, v: one [B, H, T, D] shape and one dtype (the kernels index k and v with q's
    sizes and read all three as q's element type)."""
    if q.dim() != 4:
        raise ValueError(f"q, k, v must be [B, H, T, D], got {tuple(q.shape)}")
    if k.shape != q.shape or v.shape != q.shape:
        raise ValueError(f"q, k, v must have one shape, got {tuple(q.shape)}, {tuple(k.shape)}, {tuple(v.shape)}")
    if k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError(f"q, k, v must have one dtype, got {q.dtype}, {k.dtype}, {v.dtype}")


def _check_stats(stats: "BlockStats", q: torch.Tensor, block_size: int, text_tokens: int,
                 group_size: int = GROUP_SIZE) -> None:
    """The statistics must be block_stats' for q's shape, this block size and group size: the
    kernels read kc, vc and hgroup with the sizes derived from q."""
    B, H, T, D = q.shape
    NT = math.ceil((T - int(text_tokens)) / block_size)
    NG = math.ceil(NT / group_size)
    want = {"kc": (B, H, NT, D), "vc": (B, H, NT, D), "hgroup": (B, H, NG, D, D)}
    for name, shape in want.items():
        t = getattr(stats, name)
        if tuple(t.shape) != shape or t.dtype != torch.float32:
            raise ValueError(f"stats.{name} must be float32 {list(shape)} for block_size {block_size}, "
                             f"got {t.dtype} {tuple(t.shape)}")


def tuned_shape(dtype: torch.dtype, head_dim: int, block_size: int, group_size: int = GROUP_SIZE,
                text_tokens: int = 0) -> bool:
    """Whether an attention call of this shape runs on the tuned gfx950 kernels: bf16 (or fp16
    at head_dim 128), head_dim 64 or 128, block size 64 or 128, group size 32, and a text
    segment only at head_dim 128.  Every other shape the library takes (fp32 inputs, head dims
    1 .. 128, block sizes 16 .. 256 that are powers of two, any group size) runs on the
    any-shape kernels: the same mathematics with plain VALU arithmetic, for completeness
    rather than speed."""
    return (head_dim in (64, 128) and block_size in (64, 128) and group_size == GROUP_SIZE
            and (dtype == torch.bfloat16 or (dtype == torch.float16 and head_dim == 128))
            and (text_tokens == 0 or head_dim == 128))


def num_selected(density: float, num_blocks: int) -> int:
    """NS = min(max(1, int(density * NT)), NT) (reference :373), via the C ABI."""
    ns = _lib.load().pasa_num_selected(float(density), int(num_blocks))
    if ns < 0:
        _lib.check("pasa_num_selected", int(ns))
    return int(ns)


@dataclass
class BlockStats:
    """Outputs of K2.  Statistics fp32: qc/kc/vc [B,H,NT,D], hnorm [B,H,NT], hgroup
    [B,H,NG,D,D].  With a placement, also the token-major view of k and v (in q's dtype),
    which the placed attention call reads; q_tm stays None (that call gathers q's rows
    frame-major)."""
    qc: torch.Tensor
    kc: torch.Tensor
    vc: torch.Tensor
    hnorm: torch.Tensor
    hgroup: torch.Tensor
    q_tm: Optional[torch.Tensor] = None
    k_tm: Optional[torch.Tensor] = None
    v_tm: Optional[torch.Tensor] = None


@dataclass
class Placement:
    """The token-major view of frame-major q, k, v (the HunyuanVideo placement,
    reference svg/models/hyvideo/placement.py:73-100, :124-153): for heads whose flag
    is set, logical row p*num_frame + f of the first num_frame*frame_size rows is
    stored at row f*frame_size + p; the text tail and unflagged heads are in place.
    ``head_is_temporal``: [H] or [B, H] flags, like the reference's best_mask_idx
    (None: every head)."""
    num_frame: int
    frame_size: int
    head_is_temporal: Optional[torch.Tensor] = None

    def struct(self, device, batch: int, heads: int):
        flags = None
        n = heads
        if self.head_is_temporal is not None:
            flags = self.head_is_temporal.to(device=device, dtype=torch.int32).reshape(-1).contiguous()
            n = flags.numel()
            if n not in (heads, batch * heads):
                raise ValueError(f"head_is_temporal has {n} entries for {batch} x {heads} slices")
        st = _lib.Placement(int(self.num_frame), int(self.frame_size),
                            None if flags is None else flags.data_ptr(), int(n))
        return st, flags  # keep flags alive for the call


def block_stats(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, block_size: int = 64,
                group_size: int = GROUP_SIZE, text_tokens: int = 0,
                placement: Optional[Placement] = None, split: bool = True) -> BlockStats:
    """Block means of Q/K, block sums of V, ||H_j||_F and the group mean of H_j.

    Replaces fused_chunk_reduce (reference :268-288; hc is never materialised)
    followed by compute_h_group (:291-301).  With ``text_tokens`` the blocks cover
    the first T - text_tokens rows only.  With ``placement`` the statistics are those
    of the token-major view of frame-major q, k, v, and the view of k and v is written to
    the returned ``k_tm``, ``v_tm`` in the same pass (the attention call reads q frame-major
    through the placement map, so ``q_tm`` is None).  ``split`` lets small grids (few
    heads x groups) spread each group over several workgroups (``pasa_block_stats_ws``;
    deterministic, the group sum in a different fixed order)."""
    _check_qkv(q, k, v)
    _check_device(q, k, v)
    B, H, T, D = q.shape
    NT = math.ceil((T - text_tokens) / block_size)
    NG = math.ceil(NT / group_size)
    f32 = dict(device=q.device, dtype=torch.float32)
    qc = torch.empty(B, H, NT, D, **f32)
    kc = torch.empty(B, H, NT, D, **f32)
    vc = torch.empty(B, H, NT, D, **f32)
    hnorm = torch.empty(B, H, NT, **f32)
    hgroup = torch.empty(B, H, NG, D, D, **f32)
    args = (q.data_ptr(), k.data_ptr(), v.data_ptr(), qc.data_ptr(), kc.data_ptr(), vc.data_ptr(),
            hnorm.data_ptr(), hgroup.data_ptr(), B * H, T, int(text_tokens), D, block_size, group_size)
    ws_bytes = _lib.load().pasa_block_stats_workspace_bytes(B * H, T, int(text_tokens), D, block_size,
                                                            group_size) if split else 0
    ws = torch.empty(ws_bytes, device=q.device, dtype=torch.uint8) if ws_bytes > 0 else None
    ws_ptr = None if ws is None else ws.data_ptr()
    if placement is None and ws is not None:
        _lib.call("pasa_block_stats_ws", *args, _DTYPES.get(q.dtype, -1), ws_ptr, ws_bytes, _stream(q))
    elif placement is None:
        _lib.call("pasa_block_stats", *args, _DTYPES.get(q.dtype, -1), _stream(q))
    else:
        st, _keep = placement.struct(q.device, B, H)
        k_tm, v_tm = torch.empty_like(k), torch.empty_like(v)
        _lib.call("pasa_block_stats_placed", q.data_ptr(), k.data_ptr(), v.data_ptr(), None,
                  k_tm.data_ptr(), v_tm.data_ptr(), *args[3:], ctypes.byref(st), _DTYPES.get(q.dtype, -1),
                  ws_ptr, ws_bytes, _stream(q))
        return BlockStats(qc, kc, vc, hnorm, hgroup, None, k_tm, v_tm)
    return BlockStats(qc, kc, vc, hnorm, hgroup)


@dataclass
class Selection:
    """Outputs of K3.  idx int32 [B,H,NT,NS] (score desc, index asc), or None when not
    requested (K4 reads only selmask); selmask int32 view of uint32 words
    [B,H,NT,ceil(NT/32)]; scores fp32 [B,H,NT,NT] when requested."""
    idx: Optional[torch.Tensor]
    selmask: torch.Tensor
    scores: Optional[torch.Tensor]
    ns: int


def select_blocks(stats: BlockStats, density: float, scale: float, use_cov_bias: bool = True,
                  noise: Optional[torch.Tensor] = None, return_scores: bool = False,
                  indices: bool = True) -> Selection:
    """Covariance-aware top-k of key blocks per query block (reference :365-375).

    ``noise``: optional fp32 [B,H,NT], one draw per key block (the reference's
    ``use_random``), added to the log bias only when ``use_cov_bias``.
    ``indices=False`` skips the index list (Selection.idx is None): the bitmask alone
    drives the attention kernel, and the per-row sort is not run."""
    qc, kc, hnorm = stats.qc, stats.kc, stats.hnorm
    _check_device(qc, kc, hnorm)
    B, H, NT, D = qc.shape
    ns = num_selected(density, NT)
    idx = torch.empty(B, H, NT, ns, device=qc.device, dtype=torch.int32) if indices else None
    nw = (NT + 31) // 32
    selmask = torch.empty(B, H, NT, nw, device=qc.device, dtype=torch.int32)
    if noise is not None:
        _check_device(noise)
        if noise.dtype != torch.float32 or noise.numel() != B * H * NT:
            raise ValueError("noise must be fp32 with B*H*NT elements")
    scores = torch.empty(B, H, NT, NT, device=qc.device, dtype=torch.float32)
    _lib.call("pasa_select", qc.data_ptr(), kc.data_ptr(), hnorm.data_ptr(), _ptr(noise),
              float(scale), float(density), int(bool(use_cov_bias)), _ptr(idx),
              selmask.data_ptr(), scores.data_ptr(), None, 0, B * H, NT, D, _stream(qc))
    return Selection(idx, selmask, scores if return_scores else None, ns)


def select_from_scores(scores: torch.Tensor, ns: int) -> Selection:
    """Top-``ns`` of fp32 scores [B,H,NT,NT] with ties to the lowest index."""
    _check_device(scores)
    if scores.dtype != torch.float32:
        raise ValueError("scores must be fp32")
    B, H, NT, NT2 = scores.shape
    if NT != NT2:
        raise ValueError("scores must be [B,H,NT,NT]")
    idx = torch.empty(B, H, NT, int(ns), device=scores.device, dtype=torch.int32)
    selmask = torch.empty(B, H, NT, (NT + 31) // 32, device=scores.device, dtype=torch.int32)
    _lib.call("pasa_select_from_scores", scores.data_ptr(), int(ns), idx.data_ptr(),
              selmask.data_ptr(), B * H, NT, _stream(scores))
    return Selection(idx, selmask, scores, int(ns))


def pack_phase2(q: torch.Tensor, stats: BlockStats, block_size: int = 64, text_tokens: int = 0) -> torch.Tensor:
    """Phase-2 operands (kbar, V^T, Hbar^T) per (slice, group), in q's dtype (bf16 or
    fp16), as the tuned K4 stages them in LDS (tuned shapes only: ``tuned_shape``)."""
    if q.dim() != 4:
        raise ValueError(f"q must be [B, H, T, D], got {tuple(q.shape)}")
    _check_stats(stats, q, block_size, text_tokens)
    B, H, T, D = q.shape
    lib = _lib.load()
    nbytes = int(lib.pasa_sparse_attn_workspace_bytes(B * H, T, int(text_tokens), D, block_size, GROUP_SIZE))
    if nbytes == 0:
        raise ValueError(f"unsupported shape for the gfx950 kernels: D={D}, block_size={block_size}")
    pack = torch.empty(nbytes, device=q.device, dtype=torch.uint8)
    _check_device(stats.kc, stats.vc, stats.hgroup)
    _lib.call("pasa_pack_phase2", stats.kc.data_ptr(), stats.vc.data_ptr(), stats.hgroup.data_ptr(),
              pack.data_ptr(), pack.numel(), B * H, T, int(text_tokens), D, block_size, GROUP_SIZE,
              _DTYPES.get(q.dtype, -1), _stream(q))
    return pack


def _check_out(v: torch.Tensor, out: Optional[torch.Tensor]) -> torch.Tensor:
    """The output buffer: a new tensor like ``v``, or ``out`` if it matches ``v`` exactly
    (the kernels store every row of it without bounds checks)."""
    if out is None:
        return torch.empty_like(v)
    _check_device(out)
    if out.shape != v.shape or out.dtype != v.dtype or out.device != v.device:
        raise ValueError(f"out must be a contiguous {v.dtype} tensor of shape {tuple(v.shape)} on {v.device}, "
                         f"got {out.dtype} {tuple(out.shape)} on {out.device}")
    return out


def _check_selection(sel: Selection, q: torch.Tensor, block_size: int, text_tokens: int) -> None:
    """The selection must be the one pasa_select writes for this shape and block size:
    K4 reads selmask rows ceil(NT/32) words apart without bounds checks."""
    B, H, T, _ = q.shape
    NT = math.ceil((T - int(text_tokens)) / block_size)
    nw = (NT + 31) // 32
    _check_device(sel.selmask)
    if sel.selmask.dtype not in (torch.int32, torch.uint32) or tuple(sel.selmask.shape) != (B, H, NT, nw):
        raise ValueError(f"selmask must be int32 [{B}, {H}, {NT}, {nw}] for block_size {block_size}, "
                         f"got {sel.selmask.dtype} {tuple(sel.selmask.shape)}")
    if sel.idx is None:
        return
    _check_device(sel.idx)
    if sel.idx.dtype != torch.int32 or tuple(sel.idx.shape[:3]) != (B, H, NT) or sel.idx.dim() != 4:
        raise ValueError(f"idx must be int32 [{B}, {H}, {NT}, ns] for block_size {block_size}, "
                         f"got {sel.idx.dtype} {tuple(sel.idx.shape)}")


def sparse_attn_packed(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, pack: torch.Tensor,
                       sel: Selection, scale: float, block_size: int = 64, gamma: str = "literal",
                       out: Optional[torch.Tensor] = None, text_tokens: int = 0,
                       text_valid: Optional[int] = None, placement: Optional[Placement] = None) -> torch.Tensor:
    """K4 on operands from ``pack_phase2``.  ``text_valid`` (default: all
    ``text_tokens``) is the number of prompt rows at the start of the text segment;
    the rest are padding (see ``pisa_pg_attention``).  ``placement``: q is frame-major
    (the tensor given to ``block_stats(..., placement)``), k and v are the token-major
    view that call returned (``k_tm``, ``v_tm``), and the output is stored frame-major."""
    _check_qkv(q, k, v)
    _check_device(q, k, v, pack)
    if gamma not in ("literal", "consistent"):
        raise ValueError("gamma must be 'literal' or 'consistent'")
    B, H, T, D = q.shape
    _check_selection(sel, q, block_size, text_tokens)
    o = _check_out(v, out)
    args = (q.data_ptr(), k.data_ptr(), v.data_ptr(), pack.data_ptr(), pack.numel(), _ptr(sel.idx),
            sel.selmask.data_ptr(), o.data_ptr(), float(scale), B * H, T, int(text_tokens),
            int(text_tokens if text_valid is None else text_valid), D, block_size, GROUP_SIZE, sel.ns,
            int(gamma == "literal"))
    if placement is None:
        _lib.call("pasa_sparse_attn_packed", *args, _DTYPES.get(q.dtype, -1), _stream(q))
    else:
        st, _keep = placement.struct(q.device, B, H)
        _lib.call("pasa_sparse_attn_packed_placed", *args, ctypes.byref(st), _DTYPES.get(q.dtype, -1), _stream(q))
    return o


def sparse_attn(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, stats: BlockStats,
                sel: Selection, scale: float, block_size: int = 64, gamma: str = "literal",
                out: Optional[torch.Tensor] = None, text_tokens: int = 0,
                text_valid: Optional[int] = None, placement: Optional[Placement] = None,
                group_size: int = GROUP_SIZE) -> torch.Tensor:
    """Exact attention over the selected blocks plus the per-group first-order
    correction of the rest (reference pisa_pg_fwd_kernel :135-262); with
    ``text_tokens``, the prompt keys are exact for every video query block and the
    text rows are dense within their segment.  With ``placement`` (q, k, v frame-major)
    the call reads q's rows through the placement map and k, v from the token-major view
    ``stats`` holds, and stores o frame-major.  ``group_size`` must be the one ``stats``
    was computed with.  Shapes outside ``tuned_shape`` run on the any-shape kernels
    (``pasa_sparse_attn`` reads the statistics directly; no pack, no placement)."""
    _check_qkv(q, k, v)
    B, H, T, D = q.shape
    if placement is None and not tuned_shape(q.dtype, D, block_size, group_size, text_tokens):
        _check_stats(stats, q, block_size, text_tokens, group_size)
        _check_device(q, k, v, stats.kc, stats.vc, stats.hgroup)
        if gamma not in ("literal", "consistent"):
            raise ValueError("gamma must be 'literal' or 'consistent'")
        _check_selection(sel, q, block_size, text_tokens)
        o = _check_out(v, out)
        _lib.call("pasa_sparse_attn", q.data_ptr(), k.data_ptr(), v.data_ptr(), stats.kc.data_ptr(),
                  stats.vc.data_ptr(), stats.hgroup.data_ptr(), _ptr(sel.idx), sel.selmask.data_ptr(),
                  o.data_ptr(), float(scale), B * H, T, int(text_tokens),
                  int(text_tokens if text_valid is None else text_valid), D, block_size, int(group_size), sel.ns,
                  int(gamma == "literal"), _DTYPES.get(q.dtype, -1), None, 0, _stream(q))
        return o
    if group_size != GROUP_SIZE:
        raise ValueError(f"the placed call runs on the tuned kernels, which use group_size={GROUP_SIZE}")
    pack = pack_phase2(q, stats, block_size, text_tokens)
    if placement is not None:  # the token-major k, v K2 wrote; the output goes back frame-major
        if stats.k_tm is None or stats.v_tm is None:
            raise ValueError("placement needs the statistics of block_stats(..., placement=...)")
        k, v = stats.k_tm, stats.v_tm
    return sparse_attn_packed(q, k, v, pack, sel, scale, block_size, gamma, out, text_tokens, text_valid,
                              placement)


def sparse_attn_noalloc(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, stats: BlockStats,
                        sel: Selection, scale: float, block_size: int = 64, gamma: str = "literal",
                        out: Optional[torch.Tensor] = None, text_tokens: int = 0,
                        text_valid: Optional[int] = None, group_size: int = GROUP_SIZE) -> torch.Tensor:
    """``sparse_attn`` through ``pasa_sparse_attn_noalloc``: the phase-2 pack lives in the
    library's static device array, so with ``out`` given the call allocates nothing
    (for code under HIP graph capture).  Shapes whose pack exceeds
    ``_lib.NOALLOC_SCRATCH_BYTES`` raise PasaError (PASA_ERR_WORKSPACE)."""
    _check_qkv(q, k, v)
    _check_stats(stats, q, block_size, text_tokens, group_size)
    _check_device(q, k, v, stats.kc, stats.vc, stats.hgroup)
    if gamma not in ("literal", "consistent"):
        raise ValueError("gamma must be 'literal' or 'consistent'")
    B, H, T, D = q.shape
    _check_selection(sel, q, block_size, text_tokens)
    o = _check_out(v, out)
    _lib.call("pasa_sparse_attn_noalloc", q.data_ptr(), k.data_ptr(), v.data_ptr(), stats.kc.data_ptr(),
              stats.vc.data_ptr(), stats.hgroup.data_ptr(), _ptr(sel.idx), sel.selmask.data_ptr(),
              o.data_ptr(), float(scale), B * H, T, int(text_tokens),
              int(text_tokens if text_valid is None else text_valid), D, block_size, int(group_size), sel.ns,
              int(gamma == "literal"), _DTYPES.get(q.dtype, -1), _stream(q))
    return o


def dense_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: Optional[float] = None,
                    text_tokens: int = 0, text_valid: Optional[int] = None,
                    out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Dense softmax attention on K4's exact-tile path (bf16 or fp16 at head_dim 128; fp32 and
    other head dims up to 128 on the any-shape kernel), for the processors' warm-up layers (reference flash_attention, svg/models/wan/attention.py:299-301,
    svg/models/hyvideo/attention.py:459-476).  With ``text_tokens`` / ``text_valid``
    the attention is block-diagonal over [0, T - text_tokens + text_valid) and the
    rest (the dense HunyuanVideo path's cu_seqlens).  q, k, v: [B, H, T, D]."""
    _check_qkv(q, k, v)
    _check_device(q, k, v)
    B, H, T, D = q.shape
    scale = D ** -0.5 if scale is None else scale
    o = _check_out(v, out)
    tv = text_tokens if text_valid is None else text_valid
    _lib.call("pasa_dense_attn", q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), float(scale), B * H, T,
              int(text_tokens), int(tv), D, _DTYPES.get(q.dtype, -1), _stream(q))
    return o


def kernel_head_dim(head_dim: int, dtype: torch.dtype, text_tokens: int = 0, placed: bool = False) -> int:
    """The head dim the gfx950 kernels run a call of ``head_dim`` at: 64 (bf16, no text
    segment, no placement) or 128.  ``pisa_pg_attention`` zero-pads smaller head dims to it,
    as the reference pads to BK = min(128, next_pow2(D)) (:346-347)."""
    if head_dim < 1 or head_dim > 128:
        raise ValueError(f"head_dim must be in [1, 128] (the reference's BK = min(128, next_pow2(D))), got {head_dim}")
    if head_dim <= 64 and dtype == torch.bfloat16 and not text_tokens and not placed:
        return 64
    return 128


def pisa_pg_attention(
    q, k, v,
    density=0.15,
    timestep=0,
    block_size=64,
    group_size=32,
    scale=None,
    use_cov_bias=True,
    use_random=False,
    verbose=False,
    prompt_token_length: Optional[int] = None,
    *,
    noise: Optional[torch.Tensor] = None,
    gamma: str = "literal",
    text_tokens: int = 0,
    text_valid: Optional[int] = None,
    placement: Optional[Placement] = None,
):
    """PISA with per-group first-order correction (drop-in for reference :307-398).

    q, k, v: [B, H, T, D] contiguous bf16, fp16 or fp32, D <= 128, on a ROCm device; returns o
    like v.  ``group_size`` may be any positive integer and ``block_size`` any power of two in
    [16, 256], as in the reference (:311-312); shapes outside ``tuned_shape`` run on the
    any-shape kernels.
    ``timestep``, ``verbose`` and ``prompt_token_length`` do not change the math
    (as in the reference, where ``prompt_token_length`` is documented but unused).
    ``use_random`` adds one N(0,1) draw per key block to the selection score; pass
    ``noise`` (fp32 [B,H,NT]) to make it reproducible, else it is drawn on the
    device from torch's default generator like the reference's ``randn_like``.
    ``gamma='consistent'`` rescales the zero-order denominator with the running max
    (the reference's literal form does not).
    ``text_tokens``: the last rows are a text segment (HunyuanVideo's layout):
    blocks, selection and correction cover the video rows, every video query block
    attends to the text keys exactly and text rows attend densely to all keys.  The
    default 0 is the reference's behaviour (text as ordinary tokens).
    ``text_valid``: only the first ``text_valid`` text rows are the prompt, the rest
    padding (HunyuanVideo pads its prompt; its dense path attends block-diagonally
    over cu_seqlens [0, T - text_tokens + text_valid, T], reference
    svg/models/hyvideo/attention.py:314-322).  Video and prompt rows then see the
    video rows and the prompt keys; padding rows see the padding keys.  Default:
    ``text_tokens`` (no padding).
    ``placement``: q, k, v are frame-major (HunyuanVideo's layout) and the operator
    runs on their token-major view, returning o frame-major; equal to the
    reference's hunyuan_sparse_head_placement -> attention -> hunyuan_hidden_states_placement
    (svg/models/hyvideo/attention.py:412-446) in one pass (block_size 128).
    Head dims other than 64 and 128 (and 64 where the call needs the 128 kernels: fp16, a
    text segment, a placement) run zero-padded to ``kernel_head_dim``: zero features add
    nothing to a score, a block mean or the first-order moment, so the result is the
    unpadded math; the padded output features are dropped."""
    _check_qkv(q, k, v)
    B, H, T, D = q.shape
    scale = D ** -0.5 if scale is None else scale
    Dk = kernel_head_dim(D, q.dtype, text_tokens, placement is not None)
    # Zero-pad to the tuned kernels' head dim when that makes the call tuned; other calls
    # (fp32, other group or block sizes) run at their own head dim on the any-shape kernels.
    if Dk != D and (placement is not None or tuned_shape(q.dtype, Dk, block_size, group_size, text_tokens)):
        pad = lambda t: torch.nn.functional.pad(t, (0, Dk - D)).contiguous()
        o = pisa_pg_attention(pad(q), pad(k), pad(v), density, timestep, block_size, group_size, scale,
                              use_cov_bias, use_random, verbose, prompt_token_length, noise=noise, gamma=gamma,
                              text_tokens=text_tokens, text_valid=text_valid, placement=placement)
        return o[..., :D].contiguous()
    NT = math.ceil((T - text_tokens) / block_size)
    stats = block_stats(q, k, v, block_size, group_size, text_tokens, placement)
    if use_random and use_cov_bias and noise is None:
        noise = torch.randn(B, H, NT, device=q.device, dtype=torch.float32)
    # The operator returns o only, and K4 reads the selection bitmask, so the index
    # list (the reference's topk order) is not built.
    sel = select_blocks(stats, density, scale, use_cov_bias, noise if use_cov_bias else None, indices=False)
    if verbose:
        print(f"NT={NT}, N_GROUPS={stats.hgroup.shape[2]}, GROUP_SIZE={group_size}")
        print(f"top_k={sel.ns}, density={density}")
    return sparse_attn(q, k, v, stats, sel, scale, block_size, gamma, text_tokens=text_tokens,
                       text_valid=text_valid, placement=placement, group_size=group_size)
