"""Host logic of the attention processors and installers (CPU).

The processors' projections, QK-norm, RoPE, text concat and output split are
checked against plain-torch restatements of the reference's processor steps
(svg/models/hyvideo/attention.py:41-157, 234-380; svg/models/wan/attention.py:166-301)
on small random modules.  The sparse branch is exercised with a recording stand-in
for ``pisa_pg_attention`` (dispatch, density lookup, arguments); the kernels
themselves are covered by the GPU tests."""
import math
import types

import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

from pasa_amd import density as D
from pasa_amd.processors import hunyuan as HY
from pasa_amd.processors import timestep_hook, wan as WAN
from pasa_amd.processors.rope import apply_rotary_emb_complex, apply_rotary_emb_cos_sin


class MockAttn(nn.Module):
    """The attributes of diffusers' Attention that the processors read."""

    def __init__(self, C, heads, *, joint_text=False, norm_dim=None, i2v=False):
        super().__init__()
        self.heads = heads
        self.to_q, self.to_k, self.to_v = nn.Linear(C, C), nn.Linear(C, C), nn.Linear(C, C)
        nd = norm_dim or C // heads
        self.norm_q, self.norm_k = nn.RMSNorm(nd, eps=1e-6), nn.RMSNorm(nd, eps=1e-6)
        with torch.no_grad():
            self.norm_q.weight.uniform_(0.5, 1.5)
            self.norm_k.weight.uniform_(0.5, 1.5)
        self.add_q_proj = self.add_k_proj = self.add_v_proj = None
        self.norm_added_q = self.norm_added_k = None
        self.to_add_out = None
        if joint_text:
            self.add_q_proj, self.add_k_proj, self.add_v_proj = nn.Linear(C, C), nn.Linear(C, C), nn.Linear(C, C)
            self.norm_added_q, self.norm_added_k = nn.RMSNorm(C // heads), nn.RMSNorm(C // heads)
            self.to_add_out = nn.Linear(C, C)
        if i2v:
            self.add_k_proj, self.add_v_proj = nn.Linear(C, C), nn.Linear(C, C)
            self.norm_added_k = nn.RMSNorm(C)
        self.to_out = nn.ModuleList([nn.Linear(C, C), nn.Dropout(0.0)])


def heads(x, h):
    B, S, C = x.shape
    return x.reshape(B, S, h, C // h).permute(0, 2, 1, 3)


def merge(x):
    B, H, S, Dh = x.shape
    return x.permute(0, 2, 1, 3).reshape(B, S, H * Dh)


def attend(q, k, v):
    w = torch.softmax(q @ k.transpose(-1, -2) / math.sqrt(q.shape[-1]), dim=-1)
    return w @ v


def rope_tables(S, Dh, seed=0):
    g = torch.Generator().manual_seed(seed)
    ang = torch.rand(S, Dh // 2, generator=g) * 6.0
    cos = torch.cos(ang).repeat_interleave(2, dim=-1)
    sin = torch.sin(ang).repeat_interleave(2, dim=-1)
    return cos, sin


def rope_ref(x, cos, sin):
    """out[2i] = x[2i] cos - x[2i+1] sin, out[2i+1] = x[2i+1] cos + x[2i] sin."""
    out = torch.empty_like(x)
    out[..., 0::2] = x[..., 0::2] * cos[..., 0::2] - x[..., 1::2] * sin[..., 0::2]
    out[..., 1::2] = x[..., 1::2] * cos[..., 1::2] + x[..., 0::2] * sin[..., 1::2]
    return out


# ---------------------------------------------------------------- density --

def test_density_tables_shape_and_checksums():
    assert len(D.WAN_TIMESTEP_FACTORS) == 40 and len(D.HUNYUAN_TIMESTEP_FACTORS) == 44
    for table in (D.WAN_TIMESTEP_FACTORS, D.HUNYUAN_TIMESTEP_FACTORS):
        keys = [t for t, _ in table]
        assert keys == sorted(keys, reverse=True) and len(set(keys)) == len(keys)
    # Sums of the reference tables (svg/models/wan/utils.py:182-222, svg/models/hyvideo/utils.py:155-200).
    assert sum(t for t, _ in D.WAN_TIMESTEP_FACTORS) == 28014
    assert sum(t for t, _ in D.HUNYUAN_TIMESTEP_FACTORS) == 33929
    assert sum(f for _, f in D.WAN_TIMESTEP_FACTORS) == pytest.approx(40.18051124970705, abs=1e-12)
    assert sum(f for _, f in D.HUNYUAN_TIMESTEP_FACTORS) == pytest.approx(44.0, abs=1e-12)
    assert D.WAN_TIMESTEP_FACTORS[0] == (952, 0.9751290602409638)
    assert D.HUNYUAN_TIMESTEP_FACTORS[-1] == (125, 2.2366760448475045)


def test_rescaled_density_and_lookup():
    w = D.wan_rescaled_density(0.2)
    assert w[952] == 0.2 * 0.9751290602409638 and len(w) == 40
    h = D.hunyuan_rescaled_density(0.1, use_dynamic=True)
    assert h[125] == 0.1 * 2.2366760448475045
    assert set(D.hunyuan_rescaled_density(0.1, use_dynamic=False).values()) == {0.1}
    tab = {100: 1.0, 110: 2.0, 130: 3.0}
    assert D.lookup_rescaled_density(tab, 110) == 2.0          # exact
    assert D.lookup_rescaled_density(tab, 105) == 1.0          # tie -> lower key
    assert D.lookup_rescaled_density(tab, 121) == 3.0          # nearest
    assert D.lookup_rescaled_density(tab, 50) == 1.0           # clamped low
    assert D.lookup_rescaled_density(tab, 999) == 3.0          # clamped high
    assert D.lookup_rescaled_density({}, 5) is None


# ---------------------------------------------------------------- rope -----

def test_rope_cos_sin_matches_pairwise_rotation():
    x = torch.randn(1, 2, 7, 8)
    cos, sin = rope_tables(7, 8)
    torch.testing.assert_close(apply_rotary_emb_cos_sin(x, (cos, sin)), rope_ref(x, cos, sin))


def test_rope_complex_matches_pairwise_rotation():
    x = torch.randn(1, 2, 5, 8)
    ang = torch.rand(5, 4, dtype=torch.float64)
    freqs = torch.polar(torch.ones_like(ang), ang)[None, None]
    cos = torch.cos(ang).repeat_interleave(2, -1).float()
    sin = torch.sin(ang).repeat_interleave(2, -1).float()
    torch.testing.assert_close(apply_rotary_emb_complex(x, freqs), rope_ref(x, cos, sin), rtol=1e-5, atol=1e-5)


# ---------------------------------------------------------------- hunyuan --

def hunyuan_double_reference(attn, x, enc, mask_valid, cos, sin):
    """Double-stream block: video QKV + text QKV, per-head norms, RoPE on video, joint
    block-diagonal attention, split, output projections (reference :52-157)."""
    h = attn.heads
    q, k, v = heads(attn.to_q(x), h), heads(attn.to_k(x), h), heads(attn.to_v(x), h)
    q, k = attn.norm_q(q), attn.norm_k(k)
    q, k = rope_ref(q, cos, sin), rope_ref(k, cos, sin)
    eq, ek, ev = heads(attn.add_q_proj(enc), h), heads(attn.add_k_proj(enc), h), heads(attn.add_v_proj(enc), h)
    eq, ek = attn.norm_added_q(eq), attn.norm_added_k(ek)
    q, k, v = torch.cat([q, eq], 2), torch.cat([k, ek], 2), torch.cat([v, ev], 2)
    N = q.shape[2]
    o = torch.empty_like(q)
    o[:, :, :mask_valid] = attend(q[:, :, :mask_valid], k[:, :, :mask_valid], v[:, :, :mask_valid])
    if mask_valid < N:
        o[:, :, mask_valid:] = attend(q[:, :, mask_valid:], k[:, :, mask_valid:], v[:, :, mask_valid:])
    o = merge(o)
    L = enc.shape[1]
    vid, txt = o[:, :-L], o[:, -L:]
    return attn.to_out[0](vid), attn.to_add_out(txt)


@pytest.mark.parametrize("valid_text", [4, 6])
def test_hunyuan_dense_double_stream(valid_text):
    torch.manual_seed(0)
    C, H, Sv, L = 32, 4, 10, 6
    attn = MockAttn(C, H, joint_text=True)
    x, enc = torch.randn(1, Sv, C), torch.randn(1, L, C)
    mask = torch.zeros(1, 1, 1, Sv + L, dtype=torch.bool)
    mask[..., : Sv + valid_text] = True
    cos, sin = rope_tables(Sv, C // H)
    with torch.no_grad():
        want = hunyuan_double_reference(attn, x, enc, Sv + valid_text, cos, sin)
        got = HY.HunyuanVideoAttnProcessor2_0_FlashAttention(0)(attn, x, enc, mask, (cos, sin))
        got2 = HY.Hunyuan_SVGAttn_Processor2_0(0)(attn, x, enc, mask, (cos, sin), timestep=None)
    for a, b in ((got, want), (got2, want)):
        torch.testing.assert_close(a[0], b[0], rtol=1e-5, atol=1e-5)
        torch.testing.assert_close(a[1], b[1], rtol=1e-5, atol=1e-5)


def test_hunyuan_single_stream_rope_skips_text():
    torch.manual_seed(1)
    C, H, Sv, L = 32, 4, 9, 5
    attn = MockAttn(C, H)
    x, enc = torch.randn(1, Sv, C), torch.randn(1, L, C)
    cos, sin = rope_tables(Sv, C // H)
    with torch.no_grad():
        hs = torch.cat([x, enc], 1)
        q, k, v = heads(attn.to_q(hs), H), heads(attn.to_k(hs), H), heads(attn.to_v(hs), H)
        q, k = attn.norm_q(q), attn.norm_k(k)
        q = torch.cat([rope_ref(q[:, :, :Sv], cos, sin), q[:, :, Sv:]], 2)
        k = torch.cat([rope_ref(k[:, :, :Sv], cos, sin), k[:, :, Sv:]], 2)
        o = merge(attend(q, k, v))
        want = attn.to_out[0](o[:, :Sv])
        got, got_txt = HY.HunyuanVideoAttnProcessor2_0_FlashAttention(0)(attn, x, enc, None, (cos, sin))
    torch.testing.assert_close(got, want, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(got_txt, o[:, Sv:], rtol=1e-5, atol=1e-5)


class Recorder:
    def __init__(self):
        self.calls = []

    def __call__(self, q, k, v, **kw):
        self.calls.append(kw)
        return torch.zeros_like(q)


@pytest.fixture
def hy_config():
    M = HY.Hunyuan_PASA_Processor
    saved = {a: getattr(M, a) for a in ("context_length", "num_frame", "frame_size", "first_layers_fp",
                                        "first_times_fp", "rescaled_density", "use_group", "use_random")}
    M.context_length, M.num_frame, M.frame_size = 3, 2, 4
    M.first_layers_fp, M.first_times_fp = 2, 900
    M.rescaled_density = D.hunyuan_rescaled_density(0.2, use_dynamic=True)
    M.use_group, M.use_random = True, True
    yield M
    for a, val in saved.items():
        setattr(M, a, val)


def test_hunyuan_pasa_dispatch(monkeypatch, hy_config):
    rec = Recorder()
    monkeypatch.setattr(HY, "pisa_pg_attention", rec)
    q = torch.randn(1, 2, 11, 8)
    cu = (torch.tensor([0, 11, 11]), torch.tensor([0, 11, 11]), 11, 11)
    dense = HY.block_diagonal_attention(q, q, q, 11)
    # layer below first_layers_fp -> dense
    out = hy_config(1).attention_core_logic(q, q, q, torch.tensor([500]), 1, cu)
    torch.testing.assert_close(out, dense)
    # timestep above first_times_fp -> dense
    out = hy_config(5).attention_core_logic(q, q, q, torch.tensor([950]), 5, cu)
    torch.testing.assert_close(out, dense)
    assert rec.calls == []
    # sparse: nearest calibrated key of 500 is 488 (factor 0.9239564591192239)
    hy_config(5).attention_core_logic(q, q, q, torch.tensor([500]), 5, cu)
    assert rec.calls == [dict(density=0.2 * 0.9239564591192239, block_size=64, use_random=True)]
    hy_config.text_segment = True
    try:
        hy_config(5).attention_core_logic(q, q, q, torch.tensor([500]), 5, cu)
        assert rec.calls[-1] == dict(density=0.2 * 0.9239564591192239, block_size=64, use_random=True,
                                     text_tokens=3, text_valid=3)
        # mask valid prefix 9 of 11: 8 video tokens + 1 prompt token, 2 padding
        cu9 = (torch.tensor([0, 9, 11]), torch.tensor([0, 9, 11]), 9, 9)
        hy_config(5).attention_core_logic(q, q, q, torch.tensor([500]), 5, cu9)
        assert rec.calls[-1]["text_tokens"] == 3 and rec.calls[-1]["text_valid"] == 1
    finally:
        hy_config.text_segment = False


def test_hunyuan_pasa_use_group_false_raises(monkeypatch, hy_config):
    monkeypatch.setattr(HY, "pisa_pg_attention", Recorder())
    hy_config.use_group = False
    q = torch.randn(1, 2, 11, 8)
    cu = (torch.tensor([0, 11, 11]), torch.tensor([0, 11, 11]), 11, 11)
    with pytest.raises(NotImplementedError):
        hy_config(5).attention_core_logic(q, q, q, torch.tensor([500]), 5, cu)


def test_hunyuan_pasa_shape_assert(hy_config):
    q = torch.randn(1, 2, 12, 8)
    with pytest.raises(AssertionError):
        hy_config(5).attention_core_logic(q, q, q, torch.tensor([500]), 5, None)


def test_replace_hyvideo_attention_installs(hy_config):
    blocks = [types.SimpleNamespace(attn=types.SimpleNamespace(processor=None)) for _ in range(3)]
    singles = [types.SimpleNamespace(attn=types.SimpleNamespace(processor=None)) for _ in range(2)]
    pipe = types.SimpleNamespace(transformer=types.SimpleNamespace(transformer_blocks=blocks,
                                                                   single_transformer_blocks=singles))
    r = HY.replace_hyvideo_attention(pipe, 720, 1280, 129, 0, first_layers_fp=1, first_times_fp=950,
                                     base_density=0.1, use_dynamic=False, use_random=False)
    M = HY.Hunyuan_PASA_Processor
    assert (M.context_length, M.num_frame, M.frame_size) == (256, 33, 3600)
    assert r == 1280 / 3600
    assert set(M.rescaled_density.values()) == {0.1} and not M.use_random
    idx = [b.attn.processor.layer_idx for b in blocks + singles]
    assert idx == [0, 1, 2, 3, 4] and all(isinstance(b.attn.processor, M) for b in blocks + singles)
    HY.replace_hyvideo_flashattention(pipe)
    assert all(isinstance(b.attn.processor, HY.HunyuanVideoAttnProcessor2_0_FlashAttention) for b in blocks)


# ---------------------------------------------------------------- wan ------

@pytest.fixture
def wan_config():
    M = WAN.Wan_PASA_Processor
    saved = {a: getattr(M, a) for a in ("context_length", "num_frame", "frame_size", "first_layers_fp",
                                        "first_times_fp", "rescaled_density")}
    M.context_length, M.num_frame, M.frame_size = 0, 3, 4
    M.first_layers_fp, M.first_times_fp = 1, 900
    M.rescaled_density = D.wan_rescaled_density(0.15)
    yield M
    for a, val in saved.items():
        setattr(M, a, val)


def test_wan_self_attention_dense_and_sparse(monkeypatch, wan_config):
    torch.manual_seed(2)
    C, H, S = 32, 4, 12
    attn = MockAttn(C, H, norm_dim=C)
    x = torch.randn(1, S, C)
    ang = torch.rand(S, C // H // 2, dtype=torch.float64)
    freqs = torch.polar(torch.ones_like(ang), ang)[None, None]
    with torch.no_grad():
        q, k = attn.norm_q(attn.to_q(x)), attn.norm_k(attn.to_k(x))        # norm before the head split
        q, k, v = heads(q, H), heads(k, H), heads(attn.to_v(x), H)
        q, k = apply_rotary_emb_complex(q, freqs), apply_rotary_emb_complex(k, freqs)
        want = attn.to_out[0](merge(attend(q, k, v)))
        got = wan_config(0)(attn, x, None, None, freqs, timestep=torch.tensor([800]))   # layer 0 < 1: dense
    torch.testing.assert_close(got, want, rtol=1e-5, atol=1e-5)
    rec = Recorder()
    monkeypatch.setattr(WAN, "pisa_pg_attention", rec)
    with torch.no_grad():
        wan_config(3)(attn, x, None, None, freqs, timestep=torch.tensor([796]))
        with pytest.raises(AssertionError):                                     # not a calibrated key
            wan_config(3)(attn, x, None, None, freqs, timestep=torch.tensor([795]))
    assert rec.calls == [dict(density=0.15 * 0.8654704578313253, block_size=64, use_random=False)]


def test_wan_cross_attention_stays_dense(monkeypatch, wan_config):
    rec = Recorder()
    monkeypatch.setattr(WAN, "pisa_pg_attention", rec)
    torch.manual_seed(3)
    C, H = 32, 4
    attn = MockAttn(C, H, norm_dim=C)
    x, enc = torch.randn(1, 12, C), torch.randn(1, 7, C)
    with torch.no_grad():
        q, k = attn.norm_q(attn.to_q(x)), attn.norm_k(attn.to_k(enc))
        q, k, v = heads(q, H), heads(k, H), heads(attn.to_v(enc), H)
        want = attn.to_out[0](merge(attend(q, k, v)))
        tok = timestep_hook._TIMESTEP.set(torch.tensor([500]))   # a hooked forward is running
        try:
            got = wan_config(3)(attn, x, enc)
        finally:
            timestep_hook._TIMESTEP.reset(tok)
    torch.testing.assert_close(got, want, rtol=1e-5, atol=1e-5)
    assert rec.calls == []


def test_replace_wan_attention_installs(wan_config):
    class Block:
        def __init__(self):
            self.attn1 = types.SimpleNamespace(processor=None)
            self.attn1.set_processor = lambda p, a=self.attn1: setattr(a, "processor", p)

    blocks = [Block() for _ in range(4)]
    cfg = types.SimpleNamespace(patch_size=(1, 2, 2))
    pipe = types.SimpleNamespace(vae_scale_factor_temporal=4, vae_scale_factor_spatial=8,
                                 transformer=types.SimpleNamespace(config=cfg, blocks=blocks))
    WAN.replace_wan_attention(pipe, 720, 1280, 81, first_layers_fp=2, first_times_fp=900, base_density=0.1)
    M = WAN.Wan_PASA_Processor
    assert (M.num_frame, M.frame_size, M.context_length) == (21, 45 * 80, 0)
    assert M.rescaled_density[952] == 0.1 * 0.9751290602409638
    assert [b.attn1.processor.layer_idx for b in blocks] == [0, 1, 2, 3]


# ---------------------------------------------------------------- hook -----

def test_timestep_hook_exposes_forward_timestep():
    seen = []

    class Model:
        def forward(self, hidden_states, timestep, encoder_hidden_states=None):
            seen.append(timestep_hook.current_timestep())
            return hidden_states

    timestep_hook.wrap_forward(Model)
    timestep_hook.wrap_forward(Model)                 # idempotent
    m = Model()
    m.forward(1, torch.tensor([7]))
    m.forward(1, timestep=torch.tensor([9]))
    assert [int(t) for t in seen] == [7, 9]
    assert timestep_hook.current_timestep() is None   # reset after the call
