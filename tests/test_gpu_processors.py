"""The PASA processors on the GPU: one sparse self-attention call each, through the
real kernels, checked against the CPU oracle on the tensors the processor handed
to ``pisa_pg_attention`` (selection shared, so a near tie cannot mask the check)."""
import pytest
import torch

from oracle import pisa_oracle as O
from pasa_amd import ops
from pasa_amd.processors import hunyuan as HY
from pasa_amd.processors import wan as WAN

from test_processors import MockAttn, rope_tables

pytestmark = pytest.mark.gpu


class Spy:
    def __init__(self, fn):
        self.fn, self.calls = fn, []

    def __call__(self, q, k, v, **kw):
        o = self.fn(q, k, v, **kw)
        self.calls.append((q.detach().clone(), k.detach().clone(), v.detach().clone(), o.detach().clone(), kw))
        return o


def check_call(call, gamma="literal"):
    q, k, v, o, kw = call
    bt, density = kw["block_size"], kw["density"]
    scale = q.shape[-1] ** -0.5
    st = ops.block_stats(q, k, v, bt, 32)
    sel = ops.select_blocks(st, density, scale)            # deterministic: the call's own selection
    ref = O.pisa_pg_attention(q.cpu().float(), k.cpu().float(), v.cpu().float(), density, bt, 32, scale,
                              indices=sel.idx.cpu(), gamma=gamma)
    m = O.parity_metrics(o.cpu().float(), ref)
    print(f"[proc] T={q.shape[2]} density={density:.4f} cos={m['cos']:.7f} excess/rms={m['excess_over_rms']:.3e}",
          flush=True)
    assert m["bound_ok"], m


def test_hunyuan_pasa_processor_sparse_call(device, monkeypatch):
    torch.manual_seed(0)
    M = HY.Hunyuan_PASA_Processor
    saved = {a: getattr(M, a) for a in ("context_length", "num_frame", "frame_size", "first_layers_fp",
                                        "first_times_fp", "rescaled_density", "use_group", "use_random")}
    try:
        M.context_length, M.num_frame, M.frame_size = 16, 4, 60       # T = 256
        M.first_layers_fp, M.first_times_fp = 0, 900
        M.rescaled_density, M.use_group, M.use_random = {500: 0.5}, True, False
        spy = Spy(HY.pisa_pg_attention)
        monkeypatch.setattr(HY, "pisa_pg_attention", spy)
        C, H = 256, 2
        attn = MockAttn(C, H, joint_text=True).to(device, torch.bfloat16)
        x = torch.randn(1, 240, C, device=device, dtype=torch.bfloat16)
        enc = torch.randn(1, 16, C, device=device, dtype=torch.bfloat16)
        cos, sin = rope_tables(240, C // H)
        with torch.no_grad():
            out, txt = M(3)(attn, x, enc, None, (cos.to(device), sin.to(device)), timestep=torch.tensor([500]))
        torch.cuda.synchronize()
        assert len(spy.calls) == 1 and out.shape == (1, 240, C) and txt.shape == (1, 16, C)
        assert spy.calls[0][4] == dict(density=0.5, block_size=64, use_random=False)
        check_call(spy.calls[0])
    finally:
        for a, val in saved.items():
            setattr(M, a, val)


def test_wan_pasa_processor_sparse_call(device, monkeypatch):
    torch.manual_seed(1)
    M = WAN.Wan_PASA_Processor
    saved = {a: getattr(M, a) for a in ("context_length", "num_frame", "frame_size", "first_layers_fp",
                                        "first_times_fp", "rescaled_density")}
    try:
        M.context_length, M.num_frame, M.frame_size = 0, 5, 64         # T = 320
        M.first_layers_fp, M.first_times_fp = 0, 900
        M.rescaled_density = {796: 0.4}
        spy = Spy(WAN.pisa_pg_attention)
        monkeypatch.setattr(WAN, "pisa_pg_attention", spy)
        C, H = 256, 2
        attn = MockAttn(C, H, norm_dim=C).to(device, torch.bfloat16)
        x = torch.randn(1, 320, C, device=device, dtype=torch.bfloat16)
        ang = torch.rand(320, C // H // 2, dtype=torch.float64)
        freqs = torch.polar(torch.ones_like(ang), ang)[None, None].to(device)
        with torch.no_grad():
            out = M(2)(attn, x, None, None, freqs, timestep=torch.tensor([796]))
        torch.cuda.synchronize()
        assert len(spy.calls) == 1 and out.shape == (1, 320, C)
        check_call(spy.calls[0])
    finally:
        for a, val in saved.items():
            setattr(M, a, val)


def test_hunyuan_pasa_processor_text_segment_with_padding(device, monkeypatch):
    # text_segment: the mask's padding is a segment of its own, as in the dense path
    torch.manual_seed(2)
    M = HY.Hunyuan_PASA_Processor
    saved = {a: getattr(M, a) for a in ("context_length", "num_frame", "frame_size", "first_layers_fp",
                                        "first_times_fp", "rescaled_density", "use_random", "text_segment")}
    try:
        M.context_length, M.num_frame, M.frame_size = 40, 4, 60       # 240 video + 40 text tokens
        M.first_layers_fp, M.first_times_fp = 0, 900
        M.rescaled_density, M.use_random, M.text_segment = {500: 0.5}, False, True
        spy = Spy(HY.pisa_pg_attention)
        monkeypatch.setattr(HY, "pisa_pg_attention", spy)
        C, H = 256, 2
        attn = MockAttn(C, H, joint_text=True).to(device, torch.bfloat16)
        x = torch.randn(1, 240, C, device=device, dtype=torch.bfloat16)
        enc = torch.randn(1, 40, C, device=device, dtype=torch.bfloat16)
        mask = torch.zeros(1, 1, 1, 280, dtype=torch.bool, device=device)
        mask[..., :240 + 23] = True                                    # 23 prompt tokens, 17 padding
        cos, sin = rope_tables(240, C // H)
        with torch.no_grad():
            M(3)(attn, x, enc, mask, (cos.to(device), sin.to(device)), timestep=torch.tensor([500]))
        torch.cuda.synchronize()
        assert len(spy.calls) == 1
        q, k, v, o, kw = spy.calls[0]
        assert kw["text_tokens"] == 40 and kw["text_valid"] == 23
        scale = q.shape[-1] ** -0.5
        st = ops.block_stats(q, k, v, 64, 32, text_tokens=40)
        sel = ops.select_blocks(st, 0.5, scale)
        ref = O.pisa_pg_attention(q.cpu().float(), k.cpu().float(), v.cpu().float(), 0.5, 64, 32, scale,
                                  indices=sel.idx.cpu(), text_tokens=40, text_valid=23)
        m = O.parity_metrics(o.cpu().float(), ref)
        print(f"[proc] hunyuan text segment 23/40 cos={m['cos']:.7f} excess/rms={m['excess_over_rms']:.3e}",
              flush=True)
        assert m["bound_ok"], m
    finally:
        for a, val in saved.items():
            setattr(M, a, val)
