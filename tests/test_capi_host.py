"""Host-side tests of the C ABI: the library loads, exports every entry point the
header declares, and every validation error path returns its status code and
message before any HIP call (so these run without a GPU)."""
import ctypes
import re
import subprocess
from pathlib import Path

import pytest

from pasa_amd import _lib

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "pasa.h"


def header_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(pasa_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not _lib.LIB_PATH.exists():
        pytest.fail(f"{_lib.LIB_PATH} not built: run `python -m pasa_amd.build`")
    return _lib.load()


def test_exports_match_header(lib):
    declared = header_functions()
    assert declared, "no declarations parsed"
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\bT (pasa_[a-z0-9_]+)$", out, flags=re.M))
    assert set(declared) <= exported, set(declared) - exported
    assert set(declared) == set(_lib.SIGNATURES), "ctypes table out of sync with the header"


def test_version_and_status_strings(lib):
    assert lib.pasa_abi_version() == _lib.ABI_VERSION
    for code in _lib.STATUS:
        assert lib.pasa_status_string(code)
    assert lib.pasa_status_string(12345) == b"unknown status"


@pytest.mark.parametrize("density,nt,expect", [
    (0.1, 591, 59), (0.15, 256, 38), (0.25, 16, 4), (0.10, 929, 92), (1.0, 10, 10),
    (0.0, 10, 1), (2.0, 10, 10), (0.29, 100, 28), (-0.5, 8, 1), (0.999999, 3, 2)])
def test_num_selected_matches_python(lib, density, nt, expect):
    assert lib.pasa_num_selected(density, nt) == expect == min(max(1, int(density * nt)), nt)


def test_num_selected_errors(lib):
    assert lib.pasa_num_selected(float("nan"), 10) == -9
    assert b"finite" in lib.pasa_last_error()
    assert lib.pasa_num_selected(float("inf"), 10) == -9
    assert lib.pasa_num_selected(0.5, 0) == -2


FAKE = 0x1000  # never dereferenced: every call below fails validation first


def permute(lib, **kw):
    a = dict(src0=FAKE, src1=FAKE * 2, src2=FAKE * 3, dst0=FAKE * 4, dst1=FAKE * 5, dst2=FAKE * 6,
             n=3, bh=2, F=4, P=8, ctx=0, D=128, dtype=0, mask=None, inverse=0)
    a.update(kw)
    return lib.pasa_permute(a["src0"], a["src1"], a["src2"], a["dst0"], a["dst1"], a["dst2"], a["n"],
                            a["bh"], a["F"], a["P"], a["ctx"], a["D"], a["dtype"], a["mask"],
                            a["inverse"], None)


@pytest.mark.parametrize("kw,code,msg", [
    (dict(n=0), -9, b"n_tensors"),
    (dict(n=4), -9, b"n_tensors"),
    (dict(src1=None), -1, b"NULL"),
    (dict(dst2=None), -1, b"NULL"),
    (dict(dtype=7), -7, b"dtype"),
    (dict(D=100), -3, b"multiple of 16"),
    (dict(D=4, dtype=0), -3, b"multiple of 16"),
    (dict(F=0), -2, b"num_frame"),
    (dict(ctx=-1), -2, b"context_length"),
    (dict(bh=0), -2, b"must be > 0"),
    (dict(bh=70000), -6, b"exceeds"),
    (dict(F=1 << 20, P=1 << 20), -6, b"overflows"),
    (dict(inverse=2), -9, b"inverse"),
    (dict(dst0=FAKE), -9, b"overlaps"),
])
def test_permute_validation(lib, kw, code, msg):
    assert permute(lib, **kw) == code
    assert msg in lib.pasa_last_error()


def stats(lib, **kw):
    a = dict(q=FAKE, k=FAKE, v=FAKE, qc=FAKE, kc=FAKE, vc=FAKE, hn=FAKE, hg=FAKE, bh=4, T=1000,
             text=0, D=128, BT=128, G=32, dtype=0)
    a.update(kw)
    return lib.pasa_block_stats(a["q"], a["k"], a["v"], a["qc"], a["kc"], a["vc"], a["hn"], a["hg"],
                                a["bh"], a["T"], a["text"], a["D"], a["BT"], a["G"], a["dtype"], None)


@pytest.mark.parametrize("kw,code", [
    (dict(q=None), -1), (dict(hg=None), -1), (dict(dtype=3), -7), (dict(dtype=-1), -7), (dict(dtype=5), -7),
    (dict(D=129), -3), (dict(D=0), -3), (dict(BT=48), -4), (dict(BT=512), -4), (dict(BT=8), -4),
    (dict(T=0), -2), (dict(bh=-1), -2), (dict(G=0), -12),
    (dict(T=1 << 31), -6), (dict(T=(1 << 24) - 100), -6),
    (dict(text=-1), -10), (dict(text=1000), -10),
    # the any-shape route (fp32, head dims other than 64 / 128, block sizes 16 .. 256)
    (dict(dtype=2, G=0), -12), (dict(D=96, BT=24), -4), (dict(dtype=2, text=1000), -10),
    (dict(D=96, bh=70000), -6), (dict(dtype=2, T=0), -2), (dict(dtype=2, q=None), -1),
])
def test_block_stats_validation(lib, kw, code):
    assert stats(lib, **kw) == code
    assert lib.pasa_last_error()


def select(lib, **kw):
    a = dict(qc=FAKE, kc=FAKE, hn=FAKE, noise=None, scale=0.1, density=0.1, cov=1, idx=FAKE,
             mask=FAKE, scores=FAKE, ws=None, wsb=0, bh=2, nt=100, D=128)
    a.update(kw)
    return lib.pasa_select(a["qc"], a["kc"], a["hn"], a["noise"], a["scale"], a["density"], a["cov"],
                           a["idx"], a["mask"], a["scores"], a["ws"], a["wsb"], a["bh"], a["nt"],
                           a["D"], None)


@pytest.mark.parametrize("kw,code", [
    (dict(qc=None), -1), (dict(mask=None), -1), (dict(idx=None, mask=None), -1), (dict(hn=None), -1),
    (dict(idx=None, nt=0), -2), (dict(nt=0), -2),
    (dict(nt=70000), -13), (dict(nt=10000, density=0.9), -13), (dict(D=129), -3), (dict(D=0), -3), (dict(scale=float("inf")), -9),
    (dict(density=float("nan")), -9), (dict(scores=None), -8),
    (dict(scores=None, ws=FAKE, wsb=100), -8), (dict(bh=1 << 20), -6),
])
def test_select_validation(lib, kw, code):
    assert select(lib, **kw) == code
    assert lib.pasa_last_error()


def test_select_from_scores_validation(lib):
    f = lib.pasa_select_from_scores
    assert f(None, 1, FAKE, FAKE, 1, 10, None) == -1
    assert f(FAKE, 1, FAKE, None, 1, 10, None) == -1  # selmask is required
    assert f(FAKE, 0, None, FAKE, 1, 10, None) == -5  # idx is optional: the shape checks still run
    assert f(FAKE, 0, FAKE, FAKE, 1, 10, None) == -5
    assert f(FAKE, 11, FAKE, FAKE, 1, 10, None) == -5
    assert f(FAKE, 3, FAKE, FAKE, 1, 65537, None) == -13
    assert f(FAKE, 8193, FAKE, FAKE, 1, 10000, None) == -13   # an index list past the LDS sort
    assert lib.pasa_select_workspace_bytes(2, 10) == 800
    assert lib.pasa_select_workspace_bytes(0, 10) == 0


def attn(lib, **kw):
    a = dict(q=FAKE, k=FAKE, v=FAKE, kc=FAKE, vc=FAKE, hg=FAKE, idx=FAKE, mask=FAKE, o=FAKE, scale=0.1,
             bh=2, T=1000, text=0, tv=None, D=128, BT=128, G=32, ns=2, lit=1, dtype=0, ws=FAKE, wsb=1 << 30)
    a.update(kw)
    tv = a["text"] if a["tv"] is None else a["tv"]
    return lib.pasa_sparse_attn(a["q"], a["k"], a["v"], a["kc"], a["vc"], a["hg"], a["idx"], a["mask"],
                                a["o"], a["scale"], a["bh"], a["T"], a["text"], tv, a["D"], a["BT"], a["G"],
                                a["ns"], a["lit"], a["dtype"], a["ws"], a["wsb"], None)


@pytest.mark.parametrize("kw,code", [
    (dict(o=None), -1), (dict(mask=None), -1), (dict(idx=None, mask=None), -1), (dict(idx=None, D=256), -3),
    (dict(dtype=3), -7), (dict(dtype=-1), -7), (dict(D=256), -3), (dict(D=0), -3),
    (dict(BT=512), -4), (dict(BT=100), -4), (dict(G=0), -12), (dict(ns=0), -5), (dict(ns=9), -5),
    (dict(scale=0.0), -9), (dict(scale=-1.0), -9), (dict(scale=float("nan")), -9),
    (dict(lit=2), -9), (dict(ws=None), -8), (dict(wsb=10), -8), (dict(T=0), -2),
    (dict(T=(1 << 24) - 100), -6), (dict(text=1000), -10), (dict(text=-3), -10),
    (dict(text=200, ns=8), -5), (dict(text=100, tv=101), -10),
    (dict(text=100, tv=-1), -10), (dict(text=0, tv=1), -10),
    # the any-shape route: its own shape checks, and the same argument checks
    (dict(dtype=2, G=0), -12), (dict(G=16, BT=24), -4), (dict(dtype=2, D=200), -3), (dict(G=16, ns=9), -5),
    (dict(dtype=2, scale=0.0), -9), (dict(G=16, lit=2), -9), (dict(dtype=2, text=1000), -10),
    (dict(D=64, text=100, tv=101), -10), (dict(G=16, mask=None), -1), (dict(dtype=2, T=0), -2),
])
def test_sparse_attn_validation(lib, kw, code):
    assert attn(lib, **kw) == code
    assert lib.pasa_last_error()


def attn_noalloc(lib, **kw):
    a = dict(q=FAKE, k=FAKE, v=FAKE, kc=FAKE, vc=FAKE, hg=FAKE, idx=FAKE, mask=FAKE, o=FAKE, scale=0.1,
             bh=2, T=1000, text=0, tv=None, D=128, BT=128, G=32, ns=2, lit=1, dtype=0)
    a.update(kw)
    tv = a["text"] if a["tv"] is None else a["tv"]
    return lib.pasa_sparse_attn_noalloc(a["q"], a["k"], a["v"], a["kc"], a["vc"], a["hg"], a["idx"], a["mask"],
                                        a["o"], a["scale"], a["bh"], a["T"], a["text"], tv, a["D"], a["BT"],
                                        a["G"], a["ns"], a["lit"], a["dtype"], None)


@pytest.mark.parametrize("kw,code", [
    (dict(o=None), -1), (dict(kc=None), -1), (dict(dtype=3), -7), (dict(D=256), -3), (dict(BT=512), -4),
    (dict(G=0), -12), (dict(ns=9), -5), (dict(scale=0.0), -9), (dict(lit=2), -9), (dict(dtype=2, G=0), -12),
    (dict(text=100, tv=101), -10),
    # the pack of 1261 slice-groups (53,248 bytes each) exceeds the 64 MiB static scratch
    (dict(bh=1261, T=4096, ns=1), -8),
    # Wan2.1-14B 720p at block size 64: 40 slices x 37 groups
    (dict(bh=40, T=75600, BT=64, ns=118), -8),
])
def test_sparse_attn_noalloc_validation(lib, kw, code):
    assert attn_noalloc(lib, **kw) == code
    msg = lib.pasa_last_error()
    assert msg
    if code == -8:
        assert b"static scratch" in msg


def test_noalloc_scratch_limit_matches_header(lib):
    text = HEADER.read_text()
    assert "#define PASA_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)" in text
    assert _lib.NOALLOC_SCRATCH_BYTES == 64 << 20
    per_group = lib.pasa_sparse_attn_workspace_bytes(1, 4096, 0, 128, 128, 32)
    assert per_group == 53248 and _lib.NOALLOC_SCRATCH_BYTES // per_group == 1260
    # the shapes the header names as fitting
    for bh, T, text, BT in [(40, 75600, 0, 128), (24, 118800 + 256, 256, 128), (12, 32760, 0, 64)]:
        assert lib.pasa_sparse_attn_workspace_bytes(bh, T, text, 128, BT, 32) <= _lib.NOALLOC_SCRATCH_BYTES


def test_packed_entry_validation(lib):
    pk = lib.pasa_pack_phase2
    need = lib.pasa_sparse_attn_workspace_bytes(2, 1000, 0, 128, 128, 32)
    assert pk(FAKE, FAKE, FAKE, FAKE, need - 1, 2, 1000, 0, 128, 128, 32, 0, None) == -8
    assert pk(None, FAKE, FAKE, FAKE, need, 2, 1000, 0, 128, 128, 32, 0, None) == -1
    assert pk(FAKE, FAKE, FAKE, FAKE, need, 2, 1000, 0, 128, 128, 16, 0, None) == -12
    assert pk(FAKE, FAKE, FAKE, FAKE, need, 2, 1000, 1000, 128, 128, 32, 0, None) == -10
    assert pk(FAKE, FAKE, FAKE, FAKE, need, 2, 1000, 0, 128, 128, 32, 2, None) == -7    # fp32 pack
    need64 = lib.pasa_sparse_attn_workspace_bytes(2, 1000, 0, 64, 64, 32)
    assert pk(FAKE, FAKE, FAKE, FAKE, need64, 2, 1000, 0, 64, 64, 32, 1, None) == -7    # fp16 needs D 128
    f = lib.pasa_sparse_attn_packed
    args = [FAKE, FAKE, FAKE, FAKE, need, FAKE, FAKE, FAKE, 0.1, 2, 1000, 0, 0, 128, 128, 32, 2, 1, 0, None]
    bad = list(args); bad[4] = 0
    assert f(*bad) == -8
    bad = list(args); bad[16] = 100
    assert f(*bad) == -5
    bad = list(args); bad[18] = 2
    assert f(*bad) == -7
    bad = list(args); bad[11] = -1
    assert f(*bad) == -10
    bad = list(args); bad[12] = 1     # text_valid > text_len
    assert f(*bad) == -10


def test_workspace_bytes(lib):
    f = lib.pasa_sparse_attn_workspace_bytes
    # c2: 40 slices, NT = 591, NG = 19 groups of a 53248-byte phase-2 LDS image
    assert f(40, 75600, 0, 128, 128, 32) == 40 * 19 * 53248
    assert f(40, 75600, 0, 128, 128, 16) == 0
    assert f(1, 1024, 0, 64, 64, 32) > 0
    # c3: 118800 video rows (NT 929, NG 30) + 256 text rows
    assert f(24, 118800 + 256, 256, 128, 128, 32) == 24 * 30 * 53248
    assert f(24, 1000, 1000, 128, 128, 32) == 0


def test_last_error_cleared_on_success(lib):
    assert lib.pasa_num_selected(float("nan"), 10) < 0
    assert lib.pasa_last_error() != b""
    assert lib.pasa_num_selected(0.5, 10) == 5
    assert lib.pasa_last_error() == b""


def prologue(lib, **kw):
    a = dict(xq=FAKE, xk=FAKE, xv=FAKE, q=FAKE + 1, k=FAKE + 2, v=FAKE + 3, wq=FAKE, wk=FAKE, B=1, S=100,
             H=40, D=128, il=1, ol=0, OS=None, row0=0, norm=2, rnd=0, eps=1e-6, cos=FAKE, sin=FAKE, rope=2,
             rr=None, dtype=0)
    a.update(kw)
    OS = a["S"] if a["OS"] is None else a["OS"]
    rr = a["S"] if a["rr"] is None else a["rr"]
    return lib.pasa_qkv_prologue(a["xq"], a["xk"], a["xv"], a["q"], a["k"], a["v"], a["wq"], a["wk"], a["B"],
                                 a["S"], a["H"], a["D"], a["il"], a["ol"], OS, a["row0"], a["norm"], a["rnd"],
                                 a["eps"], a["cos"], a["sin"], a["rope"], rr, a["dtype"], None)


@pytest.mark.parametrize("kw,code", [
    (dict(xq=None, xk=None, xv=None, q=None, k=None, v=None), -1),   # nothing to do
    (dict(q=None), -1), (dict(xv=None), -1),                        # input without output and back
    (dict(dtype=2), -7), (dict(D=96), -3), (dict(S=0), -2), (dict(H=0), -2), (dict(B=70000), -2),
    (dict(H=65), -2),                                                # H*D > 8192
    (dict(OS=99), -2), (dict(OS=150, row0=51), -2), (dict(row0=-1, OS=200), -2),
    (dict(il=2), -9), (dict(ol=-1), -9), (dict(norm=3), -9), (dict(rnd=2), -9),
    (dict(eps=float("nan")), -9), (dict(eps=-1.0), -9),
    (dict(wq=None, wk=None), -1),                                    # a norm needs a weight
    (dict(rope=3), -9), (dict(cos=None), -1), (dict(rr=101), -2), (dict(rr=-1), -2),
    (dict(q=FAKE), -9),                                              # in place across layouts
    (dict(q=FAKE, il=0, ol=0, OS=200), -9),                          # in place into a longer output
])
def test_prologue_validation(lib, kw, code):
    assert prologue(lib, **kw) == code
    assert lib.pasa_last_error()


@pytest.mark.parametrize("kw,code", [
    (dict(o=None), -1), (dict(q=None), -1), (dict(dtype=3), -7), (dict(D=129), -3), (dict(D=0), -3),
    (dict(T=0), -2), (dict(bh=0), -2), (dict(text=1000), -10), (dict(text=-1), -10), (dict(text=10, tv=11), -10),
    (dict(text=10, tv=-1), -10), (dict(scale=0.0), -9), (dict(scale=float("inf")), -9),
    (dict(T=(1 << 24) - 100), -6),
    # the any-shape route (fp32, head dims other than 128)
    (dict(dtype=2, text=10, tv=11), -10), (dict(D=64, scale=0.0), -9), (dict(D=64, T=0), -2),
    (dict(dtype=2, o=None), -1), (dict(D=64, text=1000), -10),
])
def test_dense_attn_validation(lib, kw, code):
    a = dict(q=FAKE, k=FAKE, v=FAKE, o=FAKE, scale=0.1, bh=2, T=1000, text=0, tv=None, D=128, dtype=0)
    a.update(kw)
    tv = a["text"] if a["tv"] is None else a["tv"]
    assert lib.pasa_dense_attn(a["q"], a["k"], a["v"], a["o"], a["scale"], a["bh"], a["T"], a["text"], tv, a["D"],
                               a["dtype"], None) == code
    assert lib.pasa_last_error()


def test_placed_entries_validation(lib):
    import ctypes
    from pasa_amd._lib import Placement
    bs, sp = lib.pasa_block_stats_placed, lib.pasa_sparse_attn_packed_placed
    need = lib.pasa_sparse_attn_workspace_bytes(2, 1000, 40, 128, 128, 32)

    def stats(pl, D=128, BT=128, T=1000, text=40, bh=2, copy=FAKE):
        return bs(FAKE, FAKE, FAKE, FAKE, FAKE, copy, FAKE, FAKE, FAKE, FAKE, FAKE, bh, T, text, D, BT, 32, pl, 0,
                  None, 0, None)

    def attn(pl, D=128, BT=128, T=1000, text=40, bh=2):
        return sp(FAKE, FAKE, FAKE, FAKE, need, FAKE, FAKE, FAKE, 0.1, bh, T, text, text, D, BT, 32, 2, 1, pl, 0,
                  None)

    good = Placement(8, 120, None, 2)                # 8 * 120 = 1000 - 40 video rows
    for fn in (stats, attn):
        assert fn(None) == -1
        assert fn(ctypes.byref(good), D=64) == -3
        assert fn(ctypes.byref(good), BT=64) == -4
        assert fn(ctypes.byref(Placement(8, 121, None, 2))) == -2    # F*P != video rows
        assert fn(ctypes.byref(Placement(0, 120, None, 2))) == -2
        assert fn(ctypes.byref(Placement(8, 120, None, 3))) == -2    # heads must divide bh
        big = Placement(2, (1 << 23) + 1, None, 1)                   # F*P > 2^24 rows
        assert fn(ctypes.byref(big), T=2 * ((1 << 23) + 1), text=0, bh=1) == -6
        assert lib.pasa_last_error()
    assert stats(ctypes.byref(good), copy=None) == -1  # the token-major copies are outputs


F16 = 1 << 40            # 16-byte aligned fake device addresses, far apart
G16 = 2 << 40
H16 = 3 << 40
Y16 = 4 << 40


@pytest.mark.parametrize("q_tm,k_tm,v_tm", [
    (None, G16, Y16),              # k_tm is k (an in-place permutation)
    (None, Y16, H16 + 4096),       # v_tm starts inside v
    (F16, Y16, Y16 + (1 << 36)),   # q_tm is q
    (None, Y16, Y16 + 4096),       # the two copies overlap
])
def test_placed_copies_must_not_overlap(lib, q_tm, k_tm, v_tm):
    """pasa_block_stats_placed writes the token-major copies while it reads q, k, v: a copy
    that overlaps an input or another copy is rejected before any launch."""
    import ctypes
    from pasa_amd._lib import Placement
    pl = Placement(8, 120, None, 2)
    rc = lib.pasa_block_stats_placed(F16, G16, H16, q_tm, k_tm, v_tm, FAKE, FAKE, FAKE, FAKE, FAKE, 2, 1000, 40,
                                     128, 128, 32, ctypes.byref(pl), 0, None, 0, None)
    assert rc == -9 and b"overlaps" in lib.pasa_last_error()


def row_ops(lib, **kw):
    a = dict(x=F16, xdt=0, r=G16, rdt=0, gate=F16 + (1 << 36), h=G16, hdt=0, ln=1, w=None, b=None, wbdt=0,
             scale=F16 + (2 << 36), shift=F16 + (3 << 36), y=Y16, ydt=0, M=64, N=1536, S=64, ps=0, eps=1e-6)
    a.update(kw)
    return lib.pasa_row_ops(a["x"], a["xdt"], a["r"], a["rdt"], a["gate"], a["h"], a["hdt"], a["ln"], a["w"],
                            a["b"], a["wbdt"], a["scale"], a["shift"], a["y"], a["ydt"], a["M"], a["N"], a["S"],
                            a["ps"], a["eps"], None)


@pytest.mark.parametrize("kw,code", [
    (dict(x=None), -1),
    (dict(r=None), -1),                                  # gate / h_out without a residual
    (dict(r=None, gate=None, h=None, y=None), -1),       # nothing to compute
    (dict(h=None, y=None), -1),                          # residual without an output
    (dict(y=None), -1),                                  # stage B arguments without y
    (dict(shift=None), -1),                              # scale without shift
    (dict(xdt=1), -7), (dict(ydt=3), -7), (dict(rdt=1), -7), (dict(wbdt=1), -7),
    (dict(M=0), -2), (dict(N=0), -2), (dict(N=1540), -2), (dict(N=8200), -2), (dict(S=0), -2),
    (dict(M=65, S=64), -2),                              # rows not a whole number of batches
    (dict(ps=8), -2), (dict(ps=1538), -2), (dict(ps=-4), -2),
    (dict(eps=float("nan")), -9), (dict(eps=-1.0), -9),
    (dict(x=F16 + 8), -9),                               # misaligned
    (dict(y=G16 + 1024), -9),                            # partial overlap
    (dict(h=G16, hdt=2), -9),                            # h aliases the residual with another dtype
])
def test_row_ops_validation(lib, kw, code):
    assert row_ops(lib, **kw) == code
    assert lib.pasa_last_error()


def test_block_stats_workspace(lib):
    # the c2 grid (40 slices x 19 groups) needs no split; c1's (12 x 8) splits 8 ways
    assert lib.pasa_block_stats_workspace_bytes(40, 75600, 0, 128, 128, 32) == 0
    assert lib.pasa_block_stats_workspace_bytes(12, 32760, 0, 128, 128, 32) == 12 * 8 * 8 * 128 * 128 * 4
    assert lib.pasa_block_stats_workspace_bytes(12, 32760, 0, 64, 128, 32) == 0       # D = 64 kernels do not split
    assert lib.pasa_block_stats_workspace_bytes(0, 32760, 0, 128, 128, 32) == 0
    need = lib.pasa_block_stats_workspace_bytes(12, 32760, 0, 128, 128, 32)
    args = [FAKE] * 8 + [12, 32760, 0, 128, 128, 32, 0]
    assert lib.pasa_block_stats_ws(*args, F16, need - 1, None) == -8                  # too small
    assert b"workspace" in lib.pasa_last_error()
    assert lib.pasa_block_stats_ws(*args, F16 + 4, need, None) == -9                  # misaligned
    a2 = [FAKE] * 7 + [None] + [12, 32760, 0, 128, 128, 32, 0]
    assert lib.pasa_block_stats_ws(*a2, F16, need, None) == -1                        # hgroup NULL


def header_arity():
    """Number of parameters of every prototype in the header (0 for `(void)`)."""
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    arity = {}
    for name, params in re.findall(r"\b(pasa_[a-z0-9_]+)\s*\(([^;{]*?)\)\s*;", text, flags=re.S):
        params = params.strip()
        arity[name] = 0 if params in ("", "void") else params.count(",") + 1
    return arity


def test_integration_stub_matches_header():
    """The ctypes stub INTEGRATION.md shows a maintainer declares every argument list with as
    many entries as the header's prototype has parameters."""
    doc = (ROOT / "INTEGRATION.md").read_text()
    stub = doc[doc.index("## 3. Binding the C ABI directly"):]
    stub = stub[stub.index("```python"):]
    stub = stub[:stub.index("```", 9)]
    aliases = {"_vp": ctypes.c_void_p, "_i64": ctypes.c_int64, "_int": ctypes.c_int,
               "_dbl": ctypes.c_double, "_sz": ctypes.c_size_t}
    arity = header_arity()
    checked = 0
    for name, both, expr in re.findall(r"_lib\.(pasa_[a-z0-9_]+)\.argtypes(, _lib\.\1\.restype)? = (.+)", stub):
        if both:  # "argtypes, restype = [...], type": keep the list
            expr = expr[:expr.rindex("]") + 1]
        lst = eval(expr, {}, dict(aliases))
        assert name in arity, name
        assert len(lst) == arity[name], (name, len(lst), arity[name])
        checked += 1
    assert checked >= 5, checked
