"""Host-side argument checks of the Python operator API (CPU tensors, no GPU).

Every op rejects q, k, v of different shapes or dtypes and statistics that do not belong
to q's shape and block size before anything reaches the library, and every op refuses
CPU tensors: there is no CPU path."""
import pytest
import torch

from pasa_amd import ops


def qkv(T=256, D=128, dtype=torch.bfloat16, H=2):
    return [torch.zeros(1, H, T, D, dtype=dtype) for _ in range(3)]


def fake_stats(B, H, NT, NG, D):
    f = dict(dtype=torch.float32)
    return ops.BlockStats(torch.zeros(B, H, NT, D, **f), torch.zeros(B, H, NT, D, **f), torch.zeros(B, H, NT, D, **f),
                          torch.zeros(B, H, NT, **f), torch.zeros(B, H, NG, D, D, **f))


@pytest.mark.parametrize("fn", [lambda q, k, v: ops.block_stats(q, k, v, 64),
                                lambda q, k, v: ops.dense_attention(q, k, v)])
def test_qkv_shape_and_dtype_mismatch_rejected(fn):
    q, k, v = qkv()
    with pytest.raises(ValueError, match="one shape"):
        fn(q, k[:, :, :128], v)
    with pytest.raises(ValueError, match="one shape"):
        fn(q, k, v[:, :1])
    with pytest.raises(ValueError, match="one dtype"):
        fn(q, k.half(), v)
    with pytest.raises(ValueError, match=r"\[B, H, T, D\]"):
        fn(q[0], k[0], v[0])


def test_cpu_tensors_have_no_path():
    q, k, v = qkv()
    with pytest.raises(ValueError, match="ROCm device tensors"):
        ops.block_stats(q, k, v, 64)
    with pytest.raises(ValueError, match="ROCm device tensors"):
        ops.dense_attention(q, k, v)


def test_pack_rejects_statistics_of_another_block_size():
    q, k, v = qkv(T=256)
    good64 = fake_stats(1, 2, 4, 1, 128)      # T 256 at block 64: NT 4, NG 1
    with pytest.raises(ValueError, match="stats.kc"):
        ops.pack_phase2(q, good64, 128)        # block 128 wants NT 2
    with pytest.raises(ValueError, match="stats.hgroup"):
        ops.pack_phase2(q, fake_stats(1, 2, 4, 2, 128), 64)
    bad = fake_stats(1, 2, 4, 1, 128)
    bad.kc = bad.kc.double()
    with pytest.raises(ValueError, match="float32"):
        ops.pack_phase2(q, bad, 64)


def test_kernel_head_dim():
    """The head dim a call runs at: 64 for bf16 without a text segment or placement, else
    128 (the reference's BK = min(128, next_pow2(D)) padding, at the two widths the kernels
    take); above 128 is an error."""
    bf, f16 = torch.bfloat16, torch.float16
    assert [ops.kernel_head_dim(d, bf) for d in (1, 32, 63, 64)] == [64] * 4
    assert [ops.kernel_head_dim(d, bf) for d in (65, 80, 96, 128)] == [128] * 4
    assert ops.kernel_head_dim(64, f16) == 128
    assert ops.kernel_head_dim(32, bf, text_tokens=256) == 128
    assert ops.kernel_head_dim(64, bf, placed=True) == 128
    for d in (0, 129, 256):
        with pytest.raises(ValueError, match="head_dim"):
            ops.kernel_head_dim(d, bf)


def test_tuned_shape_routing_table():
    """Which calls run on the tuned kernels (the rule capi.hip's tuned_attn_shape applies): bf16 at
    head_dim 64 or 128, fp16 at 128, block size 64 or 128, group size 32, a text segment only at
    head_dim 128.  Everything else goes to the any-shape kernels."""
    bf, f16, f32 = torch.bfloat16, torch.float16, torch.float32
    tuned = [(bf, 64, 64, 32, 0), (bf, 128, 128, 32, 0), (bf, 128, 64, 32, 256), (f16, 128, 128, 32, 0),
             (f16, 128, 64, 32, 100)]
    other = [(f32, 128, 128, 32, 0), (f32, 64, 64, 32, 0), (f16, 64, 64, 32, 0), (bf, 96, 128, 32, 0),
             (bf, 128, 32, 32, 0), (bf, 128, 256, 32, 0), (bf, 128, 128, 16, 0), (bf, 64, 64, 32, 10),
             (bf, 48, 64, 32, 0)]
    for dt, d, bt, g, text in tuned:
        assert ops.tuned_shape(dt, d, bt, g, text), (dt, d, bt, g, text)
    for dt, d, bt, g, text in other:
        assert not ops.tuned_shape(dt, d, bt, g, text), (dt, d, bt, g, text)
