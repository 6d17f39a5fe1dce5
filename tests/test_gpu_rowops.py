"""K6 row operations on the GPU, bit-exact against the oracle (oracle/rowops_oracle.py),
which restates the kernel's arithmetic and its summation order: every fused call of the
Wan block, the three drop-in names of the reference's Triton kernels, per-batch
modulation rows, widths from one chunk to the 8192-column limit, and the c4 row count."""
import pytest
import torch

from oracle import rowops_oracle as R
from pasa_amd import modulate as MOD

pytestmark = pytest.mark.gpu


def rnd(shape, g, dtype=torch.bfloat16, scale=1.0, shift=0.0):
    return (torch.randn(shape, generator=g) * scale + shift).to(dtype)


def same(got, ref, what):
    got = got.cpu()
    assert got.dtype == ref.dtype and got.shape == ref.shape, what
    diff = got.float() != ref.float()
    n = int(diff.sum())
    print(f"[rowops] {what}: {n} of {diff.numel()} differ", flush=True)
    for idx in diff.nonzero()[:8].tolist():
        print(f"[rowops]   at {idx}: got {got[tuple(idx)].item()!r} expected {ref[tuple(idx)].item()!r}", flush=True)
    assert n == 0, f"{what}: max |d| {(got.float() - ref.float()).abs().max().item()}"


@pytest.mark.parametrize("N", [8, 520, 1536, 3072, 5120, 8192])
def test_ln_modulate(device, N):
    g = torch.Generator().manual_seed(N)
    x = rnd((1, 130, N), g, scale=2.0, shift=0.3)
    sc, sh = rnd((1, 1, N), g, torch.float32, 0.2), rnd((1, 1, N), g, torch.float32, 0.2)
    y = MOD.ln_modulate(x.to(device), sc.to(device), sh.to(device), 1e-6)
    same(y, R.row_ops(x, layernorm=True, scale=sc, shift=sh)[1], f"ln_modulate N={N}")


def test_gate_residual_ln_in_place(device):
    g = torch.Generator().manual_seed(1)
    N = 1536
    h, x = rnd((1, 257, N), g), rnd((1, 257, N), g, scale=0.5)
    gate = rnd((1, 1, N), g, torch.float32)
    w, b = rnd((N,), g, scale=0.3, shift=1.0), rnd((N,), g, scale=0.1)
    hd = h.to(device)
    y = MOD.gate_residual_ln(hd, x.to(device), gate.to(device), 1e-6, weight=w.to(device), bias=b.to(device))
    h_ref, y_ref = R.row_ops(x, residual=h, gate=gate, layernorm=True, weight=w, bias=b)
    same(hd, h_ref, "gated residual (in place)")
    same(y, y_ref, "norm2 after the gated residual")


def test_residual_ln_modulate_and_gate_residual(device):
    g = torch.Generator().manual_seed(2)
    N = 1536
    h, x, f = rnd((1, 200, N), g), rnd((1, 200, N), g), rnd((1, 200, N), g)
    sc, sh, gate = (rnd((1, 1, N), g, torch.float32, 0.3) for _ in range(3))
    hd = h.to(device)
    y = MOD.residual_ln_modulate(hd, x.to(device), sc.to(device), sh.to(device), 1e-6)
    h1, y_ref = R.row_ops(x, residual=h, layernorm=True, scale=sc, shift=sh)
    same(hd, h1, "cross-attention residual (in place)")
    same(y, y_ref, "norm3 + modulation")
    MOD.gate_residual(hd, f.to(device), gate.to(device))
    same(hd, R.row_ops(f, residual=h1, gate=gate, y_dtype=None)[0], "feed-forward gated residual")


def test_per_batch_rows(device):
    g = torch.Generator().manual_seed(3)
    B, S, N = 3, 64, 1024
    h, x = rnd((B, S, N), g), rnd((B, S, N), g)
    gate = rnd((B, 1, N), g, torch.float32)
    w, b = rnd((N,), g, torch.float32), rnd((N,), g, torch.float32)
    hd = h.to(device)
    y = MOD.gate_residual_ln(hd, x.to(device), gate.to(device), 1e-5, weight=w.to(device), bias=b.to(device))
    h_ref, y_ref = R.row_ops(x, residual=h, gate=gate, layernorm=True, weight=w, bias=b, eps=1e-5)
    same(hd, h_ref, "per-batch gate")
    same(y, y_ref, "fp32 affine")
    sc, sh = rnd((B, 1, N), g, torch.float32), rnd((1, N), g, torch.float32)     # per batch + broadcast
    y = MOD.ln_modulate(x.to(device), sc.to(device), sh.to(device), 1e-6)
    same(y, R.row_ops(x, layernorm=True, scale=sc, shift=sh.expand(B, N).reshape(B, 1, N))[1], "mixed rows")


def test_reference_kernel_names(device):
    g = torch.Generator().manual_seed(4)
    N = 1536
    x = rnd((1, 96, N), g, scale=3.0)
    w, b = rnd((N,), g), rnd((N,), g)
    sc, sh = rnd((1, 1, N), g, torch.float32, 0.2), rnd((1, 1, N), g, torch.float32, 0.2)
    xd = x.to(device)
    ln = MOD.triton_layernorm_forward(xd, None, None, 1e-6, elementwise_affine=False)
    same(ln, R.row_ops(x, layernorm=True, y_dtype=torch.float32)[1], "layernorm, no affine -> fp32")
    lna = MOD.triton_layernorm_forward(xd, w.to(device), b.to(device), 1e-6)
    same(lna, R.row_ops(x, layernorm=True, weight=w, bias=b, y_dtype=torch.float32)[1], "layernorm affine")
    xf = x.float()
    same(MOD.triton_layernorm_forward(xf.to(device), None, None, 1e-6, False),
         R.row_ops(xf, layernorm=True, y_dtype=torch.float32)[1], "layernorm of fp32 input")
    mod = MOD.triton_modulate_shift_forward(ln, sc.to(device), sh.to(device), output_dtype=torch.bfloat16)
    same(mod, R.row_ops(ln.cpu(), scale=sc, shift=sh)[1], "modulate shift")
    # the fused call equals the two-kernel composition it replaces
    same(MOD.ln_modulate(xd, sc.to(device), sh.to(device), 1e-6), mod.cpu(), "fused = layernorm then modulate")
    r = rnd((1, 96, N), g)
    gate = rnd((1, 1, N), g, torch.float32)
    for out_dt in (torch.float32, torch.bfloat16):
        got = MOD.triton_modulate_gate_residual_forward(r.to(device), xd, gate.to(device), output_dtype=out_dt)
        same(got, R.row_ops(x, residual=r, gate=gate, h_dtype=out_dt, y_dtype=None)[0], f"gate residual {out_dt}")
    rf = r.float() * 1.001
    got = MOD.triton_modulate_gate_residual_forward(rf.to(device), xd, gate.to(device))
    same(got, R.row_ops(x, residual=rf, gate=gate, h_dtype=torch.float32, y_dtype=None)[0], "fp32 residual")


def test_c4_rows(device):
    """The Wan-1.3B 480p/81f row count: 32,760 rows of 1536."""
    g = torch.Generator().manual_seed(5)
    N = 1536
    x = rnd((1, 32760, N), g, scale=4.0)
    sc, sh = rnd((1, 1, N), g, torch.float32, 0.2), rnd((1, 1, N), g, torch.float32, 0.2)
    y = MOD.ln_modulate(x.to(device), sc.to(device), sh.to(device), 1e-6)
    torch.cuda.synchronize()
    same(y, R.row_ops(x, layernorm=True, scale=sc, shift=sh)[1], "c4 rows")


def test_streamed_rows_equal_cached_rows(device):
    """Row tensors of 256 MB or more take the streamed (nontemporal) kernel; rows are
    independent, so one call over 16,400 x 8192 bf16 rows (269 MB) must equal the same
    rows in two calls of 8,200 (134 MB each, the cached kernel) bit for bit: the gated
    residual in place plus LayerNorm affine, the heaviest call of the block."""
    M, N = 16400, 8192
    g = torch.Generator(device=device).manual_seed(7)
    x = torch.randn(1, M, N, device=device, dtype=torch.bfloat16, generator=g)
    h0 = torch.randn(1, M, N, device=device, dtype=torch.bfloat16, generator=g)
    gate = torch.randn(1, 1, N, device=device, generator=g)
    w = torch.randn(N, device=device, dtype=torch.bfloat16, generator=g)
    b = torch.randn(N, device=device, dtype=torch.bfloat16, generator=g)
    h_one, y_one = h0.clone(), torch.empty_like(h0)
    MOD.row_ops(x, residual=h_one, gate=gate, h_out=h_one, layernorm=True, weight=w, bias=b, y=y_one, eps=1e-6)
    h_two, y_two = h0.clone(), torch.empty_like(h0)
    for r0 in (0, M // 2):
        sl = slice(r0, r0 + M // 2)
        hs, ys = h_two[:, sl].contiguous(), torch.empty(1, M // 2, N, device=device, dtype=torch.bfloat16)
        MOD.row_ops(x[:, sl].contiguous(), residual=hs, gate=gate, h_out=hs, layernorm=True, weight=w, bias=b,
                    y=ys, eps=1e-6)
        h_two[:, sl] = hs
        y_two[:, sl] = ys
    torch.cuda.synchronize()
    same(h_one, h_two.cpu(), "streamed vs cached gated residual")
    same(y_one, y_two.cpu(), "streamed vs cached LayerNorm")
