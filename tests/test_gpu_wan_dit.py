"""The Wan2.1 DiT harness on the GPU with the PASA processors installed by
``replace_wan_attention``: every block's sparse self-attention call is checked against
the CPU oracle on the tensors it received (selection shared), and the full-density and
dense-branch forwards against the harness's stock dense forward."""
import pytest
import torch
import torch.nn.functional as F

from oracle import pisa_oracle as O
from pasa_amd import ops
from pasa_amd import wan_dit as W
from pasa_amd.processors import replace_wan_attention
from pasa_amd.processors import wan as WAN

from test_gpu_processors import Spy, check_call

pytestmark = pytest.mark.gpu

ATTRS = ("context_length", "num_frame", "frame_size", "first_layers_fp", "first_times_fp", "rescaled_density",
         "block_size", "num_layers", "base_density", "logging_file")


@pytest.fixture
def restore_wan():
    saved = {a: getattr(WAN.Wan_PASA_Processor, a) for a in ATTRS}
    yield WAN.Wan_PASA_Processor
    for a, v in saved.items():
        setattr(WAN.Wan_PASA_Processor, a, v)


def small_model(device, layers=2):
    torch.manual_seed(0)
    cfg = W.WanDiTConfig(text_dim=64, freq_dim=32, ffn_dim=512, num_layers=layers, num_attention_heads=2,
                         attention_head_dim=128, rope_max_seq_len=64)
    with torch.device(device):
        m = W.WanDiT(cfg)
    return m.to(torch.bfloat16).eval()


def inputs(device):
    # 17 frames at 256 x 256 -> latent 16 x 5 x 32 x 32 -> 5 frames of 16 x 16 patches = 1280 tokens
    g = torch.Generator().manual_seed(1)
    lat = torch.randn(1, *W.latent_shape(17, 256, 256), generator=g).to(device, torch.bfloat16)
    text = torch.randn(1, 24, 64, generator=g).to(device, torch.bfloat16)
    return lat, torch.tensor([796], device=device), text


def install(m, first_layers_fp, first_times_fp):
    replace_wan_attention(W.WanPipelineShape(m), height=256, width=256, num_frames=17,
                          first_layers_fp=first_layers_fp, first_times_fp=first_times_fp)


def cos(a, b):
    return float(F.cosine_similarity(a.float().flatten(), b.float().flatten(), dim=0))


def test_dit_sparse_layers_match_oracle(device, monkeypatch, restore_wan):
    m = small_model(device, layers=3)
    install(m, first_layers_fp=1, first_times_fp=900)       # block 0 dense, blocks 1-2 sparse
    restore_wan.rescaled_density, restore_wan.block_size = {796: 0.3}, 128
    spy = Spy(WAN.pisa_pg_attention)
    monkeypatch.setattr(WAN, "pisa_pg_attention", spy)
    with torch.no_grad():
        out = m(*inputs(device))
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    assert len(spy.calls) == 2
    for call in spy.calls:
        assert call[0].shape == (1, 2, 1280, 128)
        assert call[4] == dict(density=0.3, block_size=128, use_random=False)
        check_call(call)


def test_dit_full_density_matches_stock_dense(device, restore_wan):
    m = small_model(device)
    x = inputs(device)
    with torch.no_grad():
        ref = m(*x)
    install(m, first_layers_fp=0, first_times_fp=900)
    restore_wan.rescaled_density, restore_wan.block_size = {796: 1.0}, 128   # every key block exact
    with torch.no_grad():
        out = m(*x)
    c = cos(out, ref)
    print(f"[dit] full density vs stock dense: cos={c:.7f}", flush=True)
    assert c >= 0.999


def test_dit_dense_branch_matches_stock_dense(device, restore_wan):
    m = small_model(device)
    x = inputs(device)
    with torch.no_grad():
        ref = m(*x)
    install(m, first_layers_fp=0, first_times_fp=0)          # timestep 796 > 0: warm-up (dense) branch
    with torch.no_grad():
        out = m(*x)
    c = cos(out, ref)
    print(f"[dit] dense branch vs stock dense: cos={c:.7f}", flush=True)
    assert c >= 0.9995


def test_dit_fused_block_ops_match_torch_block(device, restore_wan):
    """The block's fused row-ops path against its PyTorch elementwise path, stock
    processors both times: the only differences are LayerNorm summation orders."""
    m = small_model(device)
    x = inputs(device)
    saved = W.WanBlock.fast_kernels
    try:
        W.WanBlock.fast_kernels = False
        with torch.no_grad():
            ref = m(*x)
        W.WanBlock.fast_kernels = True
        with torch.no_grad():
            out = m(*x)
    finally:
        W.WanBlock.fast_kernels = saved
    c = cos(out, ref)
    print(f"[dit] fused block ops vs PyTorch block: cos={c:.7f}", flush=True)
    assert c >= 0.9999


class LayerSpy:
    """Records the sparse attention call of one block (a full forward makes one per block)."""

    def __init__(self, fn, which):
        self.fn, self.which, self.n, self.calls = fn, which, 0, []

    def __call__(self, q, k, v, **kw):
        o = self.fn(q, k, v, **kw)
        if self.n == self.which:
            self.calls.append((q.detach().clone(), k.detach().clone(), v.detach().clone(), o.detach().clone(), kw))
        self.n += 1
        return o


@pytest.mark.parametrize("density", [0.05, 0.3])
def test_dit_full_size_sparse_layer_matches_oracle(device, monkeypatch, restore_wan, density):
    """Config c4 at its stated size: the 30-block Wan2.1-1.3B DiT at 480p / 81 frames
    (32,760 tokens, 512 text tokens, random init), every block sparse at ``density``
    (block 128).  Block 15's call is checked against the oracle on heads 0 and 11 with
    the call's own selection: the north_star bound, and within 1.5x (+ one ulp) of the
    error of the reference's own bf16 roundings.  The two densities select 12 and 76
    key blocks per query block, so the check tells them apart (the whole-step cosine
    against the dense model cannot: random weights make attention diffuse)."""
    cfg = W.WanDiTConfig()
    torch.manual_seed(0)
    with torch.device(device):
        model = W.WanDiT(cfg)
    model = model.to(torch.bfloat16).eval()
    g = torch.Generator().manual_seed(0)
    latent = W.latent_shape(81, 480, 832)
    lat = torch.randn(1, *latent, generator=g).to(device, torch.bfloat16)
    text = torch.randn(1, 512, cfg.text_dim, generator=g).to(device, torch.bfloat16)
    ts = torch.tensor([952], device=device)
    replace_wan_attention(W.WanPipelineShape(model), 480, 832, 81, first_layers_fp=0, first_times_fp=0)
    restore_wan.block_size, restore_wan.first_times_fp = 128, 1000
    restore_wan.rescaled_density = {952: density}
    spy = LayerSpy(WAN.pisa_pg_attention, which=15)
    monkeypatch.setattr(WAN, "pisa_pg_attention", spy)
    print(f"[dit] c4 full size, density {density}: {cfg.num_layers} blocks, forward", flush=True)
    with torch.no_grad():
        out = model(lat, ts, text)
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    assert spy.n == cfg.num_layers and len(spy.calls) == 1
    q, k, v, o, kw = spy.calls[0]
    assert q.shape == (1, 12, 32760, 128)
    assert kw == dict(density=density, block_size=128, use_random=False)
    scale = 128 ** -0.5
    st = ops.block_stats(q, k, v, 128, 32)
    sel = ops.select_blocks(st, density, scale)            # deterministic: the call's own selection
    assert sel.ns == O.num_selected(density, 256)
    for h in (0, 11):
        qh, kh, vh = (t[:, h:h + 1].cpu().float() for t in (q, k, v))
        idx = sel.idx[:, h:h + 1].cpu()
        ref = O.pisa_pg_attention(qh, kh, vh, density, 128, 32, scale, indices=idx)
        rp = O.pisa_pg_attention(qh, kh, vh, density, 128, 32, scale, indices=idx, ref_precision=True)
        m = O.parity_metrics(o[:, h:h + 1].cpu().float(), ref)
        fl = O.parity_metrics(rp, ref)
        ulp = float(O.bf16_ulp(torch.tensor(ref.abs().max().item())))
        print(f"[dit] block 15 head {h} density {density} (NS {sel.ns}): cos={m['cos']:.7f} "
              f"excess/rms={m['excess_over_rms']:.3e} max_abs/rms={m['max_abs_over_rms']:.3e} "
              f"floor max_abs/rms={fl['max_abs_over_rms']:.3e}", flush=True)
        assert m["bound_ok"], m
        assert m["max_abs"] <= 1.5 * fl["max_abs"] + ulp, (m, fl)
