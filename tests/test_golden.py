"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py).

CPU: the oracle still produces every stored value (guards the oracle against drift).
GPU: the kernels, called through the C ABI, reproduce the stored values — K1 and K3's
top-k bit-exactly, K2 to fp32 tolerance, K3's indices exactly (the fixtures' score
margins are far above fp32 rounding), K4 within the parity bound."""
import os

import numpy as np
import pytest
import torch

from oracle import pisa_oracle as O

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
ATTN = ["attn_d64_bt64.npz", "attn_d128_bt128_noise.npz"]


def load(name):
    return dict(np.load(os.path.join(GOLDEN, name)))


def bits_to_f32(b):
    return torch.from_numpy(b.astype(np.uint16).view(np.int16)).view(torch.bfloat16).float()


def bits_to_bf16(b):
    return torch.from_numpy(b.astype(np.uint16).view(np.int16)).view(torch.bfloat16)


# ------------------------------------------------------------------ CPU ------

@pytest.mark.parametrize("name", ATTN)
def test_oracle_reproduces_attention_fixture(name):
    d = load(name)
    q, k, v = (bits_to_f32(d[x]) for x in ("q", "k", "v"))
    bt = int(d["block_size"])
    noise = torch.from_numpy(d["noise"]) if "noise" in d else None
    out, aux = O.pisa_pg_attention(q, k, v, float(d["density"]), bt, 32, float(d["scale"]), noise=noise,
                                   return_aux=True)
    st = aux["stats"]
    for key, got in (("qc", st.qc), ("kc", st.kc), ("vc", st.vc), ("hnorm", st.hnorm),
                     ("hgroup", aux["hgroup"]), ("scores", aux["scores"])):
        np.testing.assert_allclose(got.numpy(), d[key], rtol=1e-5, atol=1e-5, err_msg=key)
    np.testing.assert_array_equal(aux["idx"].numpy(), d["idx"])
    np.testing.assert_array_equal(O.selection_mask(aux["idx"], st.qc.shape[1]), d["selmask"])
    np.testing.assert_allclose(out.numpy(), d["o_literal"], rtol=1e-5, atol=1e-5)
    out_c = O.pisa_pg_attention(q, k, v, float(d["density"]), bt, 32, float(d["scale"]), noise=noise,
                                gamma="consistent")
    np.testing.assert_allclose(out_c.numpy(), d["o_consistent"], rtol=1e-5, atol=1e-5)


def test_oracle_reproduces_permute_fixture():
    d = load("permute_small.npz")
    F, P, ctx = int(d["num_frame"]), int(d["frame_size"]), int(d["context_length"])
    np.testing.assert_array_equal(O.permute(d["x"], F, P, ctx), d["forward"])
    np.testing.assert_array_equal(O.permute(d["x"], F, P, ctx, inverse=True), d["inverse"])
    np.testing.assert_array_equal(O.permute(d["x"], F, P, ctx, head_is_temporal=d["head_is_temporal"]),
                                  d["forward_masked"])


def test_oracle_reproduces_topk_fixture():
    d = load("topk_ties.npz")
    idx = O.topk_indices(torch.from_numpy(d["scores"]), int(d["ns"]))
    np.testing.assert_array_equal(idx.numpy(), d["idx"])
    assert d["idx"][1, 0].tolist() == list(range(int(d["ns"])))   # all-tied row: lowest indices


# ------------------------------------------------------------------ GPU ------

@pytest.mark.gpu
def test_gpu_permute_fixture(device):
    from pasa_amd import placement
    d = load("permute_small.npz")
    F, P, ctx = int(d["num_frame"]), int(d["frame_size"]), int(d["context_length"])
    x = torch.from_numpy(d["x"]).to(device).view(torch.float32)   # 4-byte elements, copied as bits
    out = torch.empty_like(x)
    placement.permute([x], [out], F, P, ctx)
    np.testing.assert_array_equal(out.cpu().view(torch.int32).numpy(), d["forward"])
    placement.permute([x], [out], F, P, ctx, inverse=True)
    np.testing.assert_array_equal(out.cpu().view(torch.int32).numpy(), d["inverse"])
    mask = torch.from_numpy(d["head_is_temporal"]).to(device)
    placement.permute([x], [out], F, P, ctx, head_is_temporal=mask)
    np.testing.assert_array_equal(out.cpu().view(torch.int32).numpy(), d["forward_masked"])


@pytest.mark.gpu
def test_gpu_topk_fixture(device):
    from pasa_amd import ops
    d = load("topk_ties.npz")
    sel = ops.select_from_scores(torch.from_numpy(d["scores"])[None].to(device), int(d["ns"]))
    np.testing.assert_array_equal(sel.idx[0].cpu().numpy(), d["idx"])
    np.testing.assert_array_equal(sel.selmask[0].cpu().numpy().view(np.uint32), d["selmask"])


@pytest.mark.gpu
@pytest.mark.parametrize("name", ATTN)
@pytest.mark.parametrize("gamma", ["literal", "consistent"])
def test_gpu_attention_fixture(device, name, gamma):
    from pasa_amd import ops
    d = load(name)
    print(f"[golden] {name} gamma={gamma}", flush=True)
    q, k, v = (bits_to_bf16(d[x]).to(device) for x in ("q", "k", "v"))
    bt = int(d["block_size"])
    scale = float(d["scale"])
    noise = torch.from_numpy(d["noise"]).to(device) if "noise" in d else None
    st = ops.block_stats(q, k, v, bt, 32)
    for key in ("qc", "kc", "vc", "hnorm", "hgroup"):
        got = getattr(st, key).cpu().numpy().reshape(d[key].shape)
        np.testing.assert_allclose(got, d[key], rtol=2e-5, atol=2e-5 * float(np.abs(d[key]).max()),
                                   err_msg=key)
    sel = ops.select_blocks(st, float(d["density"]), scale, True, noise)
    np.testing.assert_array_equal(sel.idx.cpu().numpy().reshape(d["idx"].shape), d["idx"])
    np.testing.assert_array_equal(sel.selmask.cpu().numpy().view(np.uint32).reshape(d["selmask"].shape),
                                  d["selmask"])
    o = ops.sparse_attn(q, k, v, st, sel, scale, bt, gamma)
    ref = torch.from_numpy(d["o_" + gamma])
    m = O.parity_metrics(o.cpu(), ref)
    print(f"[golden]   cos={m['cos']:.7f} excess/rms={m['excess_over_rms']:.3e}", flush=True)
    assert m["bound_ok"], m
