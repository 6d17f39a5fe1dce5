"""K5 (processor prologue) on the GPU through the C ABI, against the CPU oracle.

Bar: at most 1e-3 of the outputs not bit-identical to the oracle, and each of those
within one bf16 ulp of itself or, for rotated channels, within 2^-6 of its channel
pair's magnitude.  The only freedom is the order of the fp32 sum of squares inside the
norm (the oracle sums with torch on the CPU), which moves rstd by an fp32 ulp and,
rarely, a normalised value by one bf16 ulp (<= 2^-7 of the pair); a rotation that
nearly cancels carries that into its small result, and the final rounding adds at most
another 2^-7 of the pair.  Layout moves (V) and rotations without a norm are bit-exact."""
import pytest
import torch
import torch.nn.functional as F

from oracle import prologue_oracle as P
from pasa_amd import prologue as K5
from pasa_amd.processors import hunyuan as HY
from pasa_amd.processors import wan as WAN

from test_processors import MockAttn

pytestmark = pytest.mark.gpu

MISMATCH_MAX = 1e-3


def say(msg):
    print(msg, flush=True)


def ulp_diff(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    def ordered(t):
        bits = t.contiguous().view(torch.int16).int()
        mag = bits & 0x7FFF
        return torch.where(bits < 0, -mag, mag)
    return (ordered(a.cpu()) - ordered(b.cpu())).abs()


def check(got, want, what):
    got, want = got.cpu(), want.cpu()
    d = ulp_diff(got, want)
    frac = float((d > 0).float().mean())
    w = want.float()
    ulp = torch.exp2(torch.floor(torch.log2(w.abs().clamp_min(2.0 ** -126))) - 7)
    pair = torch.sqrt(w[..., 0::2] ** 2 + w[..., 1::2] ** 2).repeat_interleave(2, -1)
    bound = torch.maximum(ulp, pair * 2.0 ** -6)
    ratio = float(((got.float() - w).abs() / bound).max())
    say(f"[K5] {what}: max ulp {int(d.max())}, mismatch fraction {frac:.2e}, max |err|/bound {ratio:.3f}")
    assert ratio <= 1.0, what
    assert frac <= MISMATCH_MAX, what


def rand_bf16(*shape, seed=0, scale=2.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(torch.bfloat16)


def weights(n, seed):
    g = torch.Generator().manual_seed(seed)
    return (torch.rand(n, generator=g) + 0.5).to(torch.bfloat16)


def angles(S, half, seed):
    return torch.rand(S, half, generator=torch.Generator().manual_seed(seed), dtype=torch.float64) * 6.0


@pytest.mark.parametrize("S,H,D", [(333, 40, 128), (70, 12, 128), (45, 8, 64)])
def test_row_norm_complex_rope(device, S, H, D):
    """Wan: RMSNorm over H*D (one rounding), head split, complex fp64 RoPE."""
    say(f"[K5] row norm + complex rope S={S} H={H} D={D}")
    xq, xk, xv = (rand_bf16(1, S, H * D, seed=s, scale=3.0) for s in (1, 2, 3))
    wq, wk = weights(H * D, 4), weights(H * D, 5)
    ang = angles(S, D // 2, 6)
    re, im = torch.cos(ang), torch.sin(ang)
    got = K5.qkv_prologue(*(t.to(device) for t in (xq, xk, xv)), H, wq=wq.to(device), wk=wk.to(device),
                          norm="row", rounding="once", eps=1e-6, rope=("complex", re.to(device), im.to(device)))
    want = P.qkv_prologue(xq, xk, xv, H, wq=wq, wk=wk, norm="row", rounding="once", eps=1e-6,
                          rope=("complex", re, im))
    check(got[0], want[0], "q")
    check(got[1], want[1], "k")
    assert torch.equal(got[2].cpu(), want[2])


@pytest.mark.parametrize("S,txt,H,D,rounding", [(300, 40, 24, 128, "twice"), (129, 0, 4, 128, "once"),
                                                 (77, 13, 6, 64, "twice"), (5, 2, 2, 64, "once")])
def test_head_norm_cossin_rope_text_last(device, S, txt, H, D, rounding):
    """HunyuanVideo: per-head RMSNorm, fp32 cos/sin RoPE on the video rows only."""
    say(f"[K5] head norm ({rounding}) + cos/sin rope S={S} txt={txt} H={H} D={D}")
    xq, xk, xv = (rand_bf16(2, S, H * D, seed=s) for s in (7, 8, 9))
    wq, wk = weights(D, 10), weights(D, 11)
    ang = angles(S - txt, D // 2, 12)
    cos = torch.cos(ang).repeat_interleave(2, -1).float()
    sin = torch.sin(ang).repeat_interleave(2, -1).float()
    got = K5.qkv_prologue(*(t.to(device) for t in (xq, xk, xv)), H, wq=wq.to(device), wk=wk.to(device),
                          norm="head", rounding=rounding, eps=1e-6, rope=("cossin", cos.to(device), sin.to(device)),
                          rope_rows=S - txt)
    want = P.qkv_prologue(xq, xk, xv, H, wq=wq, wk=wk, norm="head", rounding=rounding, eps=1e-6,
                          rope=("cossin", cos, sin), rope_rows=S - txt)
    check(got[0], want[0], "q")
    check(got[1], want[1], "k")
    assert torch.equal(got[2].cpu(), want[2])


def test_two_calls_fill_one_joint_sequence(device):
    """Video rows (rotated) and text rows (own weights, not rotated) written into one
    [B, H, S + txt, D] buffer by out_row0; every row written exactly once."""
    B, S, txt, H, D = 1, 96, 17, 4, 128
    say(f"[K5] joint sequence S={S} txt={txt}")
    x = [rand_bf16(B, S, H * D, seed=20 + i) for i in range(3)]
    e = [rand_bf16(B, txt, H * D, seed=30 + i) for i in range(3)]
    w = [weights(D, 40 + i) for i in range(4)]
    ang = angles(S, D // 2, 44)
    cos = torch.cos(ang).repeat_interleave(2, -1).float()
    sin = torch.sin(ang).repeat_interleave(2, -1).float()
    outs = [torch.full((B, H, S + txt, D), float("nan"), device=device, dtype=torch.bfloat16) for _ in range(3)]
    K5.qkv_prologue(*(t.to(device) for t in x), H, wq=w[0].to(device), wk=w[1].to(device), norm="head",
                    rounding="twice", rope=("cossin", cos.to(device), sin.to(device)), out=outs, out_seq_len=S + txt)
    K5.qkv_prologue(*(t.to(device) for t in e), H, wq=w[2].to(device), wk=w[3].to(device), norm="head",
                    rounding="twice", out=outs, out_seq_len=S + txt, out_row0=S)
    a = P.qkv_prologue(*x, H, wq=w[0], wk=w[1], norm="head", rounding="twice", rope=("cossin", cos, sin))
    b = P.qkv_prologue(*e, H, wq=w[2], wk=w[3], norm="head", rounding="twice")
    for i, name in enumerate("qkv"):
        assert not torch.isnan(outs[i].float()).any(), name
        check(outs[i], torch.cat([a[i], b[i]], dim=2), f"joint {name}")


def test_drop_in_names_in_place(device):
    B, H, L, D, txt = 1, 3, 50, 128, 6
    say("[K5] drop-in names: rms_norm_forward, rope txtlast / complex, triton_rmsnorm_forward")
    x = rand_bf16(B, H, L, D, seed=50)
    w = weights(D, 51)
    xd = x.to(device)
    r = K5.rms_norm_forward(xd, w.to(device), 1e-6)
    assert r.data_ptr() == xd.data_ptr()
    check(xd, P.rms_norm_twice(x, w, 1e-6), "rms_norm_forward")

    q, k = rand_bf16(B, H, L, D, seed=52), rand_bf16(B, H, L, D, seed=53)
    ang = angles(L - txt, D // 2, 54)
    cos = torch.cos(ang).repeat_interleave(2, -1).float()
    sin = torch.sin(ang).repeat_interleave(2, -1).float()
    qd, kd = q.to(device), k.to(device)
    K5.apply_qk_rope_inplace_cossin_txtlast(qd, kd, cos.to(device), sin.to(device), txt)
    for got, src in ((qd, q), (kd, k)):
        want = torch.cat([P.rope_cossin(src[:, :, :L - txt], cos, sin), src[:, :, L - txt:]], dim=2)
        assert torch.equal(got.cpu(), want)          # no norm: the fp32 steps are reproduced exactly

    ang2 = angles(L, D // 2, 55)
    qd, kd = q.to(device), k.to(device)
    K5.apply_qk_rope_inplace_cossin_complex(qd, kd, torch.cos(ang2).to(device), torch.sin(ang2).to(device), 0)
    check(qd, P.rope_complex(q, torch.cos(ang2), torch.sin(ang2)), "rope complex q")
    check(kd, P.rope_complex(k, torch.cos(ang2), torch.sin(ang2)), "rope complex k")

    xr = rand_bf16(2, 33, 5120, seed=56)
    wr = weights(5120, 57)
    y = K5.triton_rmsnorm_forward(xr.to(device), wr.to(device), 1e-6)
    assert y.shape == xr.shape
    check(y, P.rms_norm_once(xr, wr, 1e-6), "triton_rmsnorm_forward")
    check(y, F.rms_norm(xr.to(device), (5120,), wr.to(device), 1e-6), "vs torch rms_norm on the GPU")


def test_wan_processor_fused_prologue_matches_steps(device):
    torch.manual_seed(60)
    C, H, S = 512, 4, 96
    attn = MockAttn(C, H, norm_dim=C).to(device, torch.bfloat16)
    x = torch.randn(1, S, C, device=device, dtype=torch.bfloat16)
    ang = torch.rand(S, C // H // 2, dtype=torch.float64)
    freqs = torch.polar(torch.ones_like(ang), ang)[None, None].to(device)
    proc = WAN.Wan_PASA_Processor(0)
    with torch.no_grad():
        fused = proc.fused_qkv(attn, x, x, freqs)
        assert fused is not None
        q, k, v = proc.get_qkv(attn, x, x)
        q, k = proc.get_qk_norm(attn, q, k)
        q, k, v = proc.get_transpose_qkv(attn, q, k, v)
        q, k = proc.get_rotary_emb(q, k, freqs)
    say("[K5] Wan processor fused vs step-by-step")
    for a, b, n in zip(fused, (q, k, v), "qkv"):
        check(a, b, f"wan {n}")


@pytest.mark.parametrize("joint", [True, False])
def test_hunyuan_processor_fused_prologue_matches_steps(device, joint):
    torch.manual_seed(61)
    C, H, Sv, L = 256, 2, 60, 12
    attn = MockAttn(C, H, joint_text=joint).to(device, torch.bfloat16)
    x = torch.randn(1, Sv, C, device=device, dtype=torch.bfloat16)
    enc = torch.randn(1, L, C, device=device, dtype=torch.bfloat16)
    g = torch.Generator().manual_seed(62)
    ang = torch.rand(Sv, C // H // 2, generator=g) * 6
    rot = (torch.cos(ang).repeat_interleave(2, -1).to(device), torch.sin(ang).repeat_interleave(2, -1).to(device))
    proc = HY.Hunyuan_SVGAttn_Processor2_0(0)
    with torch.no_grad():
        fused = HY.fused_hunyuan_qkv(attn, x, enc, rot)
        assert fused is not None
        hs = x if joint else torch.cat([x, enc], dim=1)
        q, k, v = proc.get_qkv(attn, hs)
        q, k, v = proc.get_transpose_qkv(attn, q, k, v)
        q, k = proc.get_qk_norm(attn, q, k)
        q, k = proc.get_rotary_emb(attn, q, k, rot, enc)
        q, k, v = proc.get_encoder_condition_and_concat(attn, q, k, v, enc)
    say(f"[K5] Hunyuan processor fused vs step-by-step (joint={joint})")
    for a, b, n in zip(fused, (q, k, v), "qkv"):
        check(a, b, f"hunyuan {n}")
