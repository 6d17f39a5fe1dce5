"""The Wan2.1 DiT harness (pasa_amd.wan_dit) on the CPU: closed forms of its RoPE grid,
timestep embedding and unpatchify, the installer on its pipeline shape, and the PASA
processor's dense branch against the harness's own dense processor."""
import cmath
import math

import torch

from pasa_amd import wan_dit as W
from pasa_amd.processors import Wan_PASA_Processor, replace_wan_attention


def tiny_cfg(layers=2):
    return W.WanDiTConfig(text_dim=64, freq_dim=32, ffn_dim=512, num_layers=layers, num_attention_heads=2,
                          attention_head_dim=128, rope_max_seq_len=64)


def test_rope_grid_closed_form():
    rope = W.WanRotaryPosEmbed(128, (1, 2, 2), 64)
    lat = torch.zeros(1, 16, 3, 4, 6)
    f = rope(lat)
    assert f.shape == (1, 1, 3 * 2 * 3, 64) and f.dtype == torch.complex128
    for n in range(18):
        fr, y, x = n // 6, (n // 3) % 2, n % 3
        for j in range(64):
            if j < 22:
                ang = fr * 10000.0 ** (-2 * j / 44)
            elif j < 43:
                ang = y * 10000.0 ** (-2 * (j - 22) / 42)
            else:
                ang = x * 10000.0 ** (-2 * (j - 43) / 42)
            assert abs(complex(f[0, 0, n, j]) - cmath.exp(1j * ang)) < 1e-12


def test_timestep_embedding_closed_form():
    t = torch.tensor([0.0, 500.0])
    e = W.timestep_embedding(t, 8)
    assert torch.equal(e[0], torch.tensor([1.0, 1, 1, 1, 0, 0, 0, 0]))
    for i in range(4):
        w = math.exp(-math.log(10000.0) * i / 4)
        assert abs(float(e[1, i]) - math.cos(500 * w)) < 1e-4
        assert abs(float(e[1, 4 + i]) - math.sin(500 * w)) < 1e-4


def test_unpatchify_brute_force():
    nf, nh, nw, pt, ph, pw, C = 2, 3, 2, 1, 2, 2, 3
    x = torch.randn(1, nf * nh * nw, pt * ph * pw * C)
    out = W.unpatchify(x, (nf, nh, nw), (pt, ph, pw))
    assert out.shape == (1, C, nf * pt, nh * ph, nw * pw)
    for f in range(nf):
        for y in range(nh):
            for xx in range(nw):
                tok = (f * nh + y) * nw + xx
                for a in range(pt):
                    for i in range(ph):
                        for j in range(pw):
                            for c in range(C):
                                assert out[0, c, f * pt + a, y * ph + i, xx * pw + j] == \
                                    x[0, tok, ((a * ph + i) * pw + j) * C + c]


def test_forward_shape_and_latent_shape():
    torch.manual_seed(0)
    m = W.WanDiT(tiny_cfg())
    assert W.latent_shape(81, 480, 832) == (16, 21, 60, 104)
    lat = torch.randn(1, 16, 3, 4, 6)
    out = m(lat, torch.tensor([500]), torch.randn(1, 7, 64))
    assert out.shape == lat.shape and torch.isfinite(out).all()


def test_installer_on_pipeline_shape():
    torch.manual_seed(0)
    pipe = W.WanPipelineShape(W.WanDiT(tiny_cfg(3)))
    replace_wan_attention(pipe, height=32, width=48, num_frames=9, first_layers_fp=1, first_times_fp=900)
    for i, blk in enumerate(pipe.transformer.blocks):
        assert isinstance(blk.attn1.processor, Wan_PASA_Processor) and blk.attn1.processor.layer_idx == i
        assert isinstance(blk.attn2.processor, W.WanAttnProcessor)
    # latent [16, 3, 4, 6] -> 3 frames of 2 x 3 patches
    assert (Wan_PASA_Processor.num_frame, Wan_PASA_Processor.frame_size) == (3, 6)
    assert Wan_PASA_Processor.context_length == 0 and Wan_PASA_Processor.num_layers == 3


def test_pasa_dense_branch_matches_stock_processor():
    """With every timestep above first_times_fp the PASA processor attends densely; its
    projections, RMSNorm, head split and RoPE must then reproduce the stock processor."""
    torch.manual_seed(0)
    m = W.WanDiT(tiny_cfg())
    lat, ts, text = torch.randn(1, 16, 3, 4, 6), torch.tensor([500]), torch.randn(1, 7, 64)
    with torch.no_grad():
        ref = m(lat, ts, text)
        replace_wan_attention(W.WanPipelineShape(m), height=32, width=48, num_frames=9, first_layers_fp=0,
                              first_times_fp=0)
        out = m(lat, ts, text)
    torch.testing.assert_close(out, ref, rtol=1e-4, atol=1e-5)


def test_rope_survives_dtype_cast():
    """Casting the model to bf16 must leave the complex RoPE table complex128."""
    m = W.WanDiT(tiny_cfg(1)).to(torch.bfloat16)
    f = m.rope(torch.zeros(1, 16, 3, 4, 6))
    assert f.dtype == torch.complex128 and f.imag.abs().max() > 0.5
