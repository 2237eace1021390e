"""The C ABI library without a GPU: it loads, exports every declared symbol,
and rejects bad arguments on the host before anything is enqueued."""

import os
import re

import pytest

from gsa_gdn_benchmarkstudy_amd import _abi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "gsa_hip.h")

# Fake device addresses: never dereferenced, every call below is rejected
# before a launch.
P = 0x10000          # 16-byte aligned
MIS = 0x10002        # 2-byte aligned only


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(gsa_\w+)\s*\(", text)))


def _macros():
    text = open(HEADER).read()
    return {k: int(v) for k, v in re.findall(r"#define\s+(GSA_\w+)\s+(-?\d+)\b", text)}


@pytest.fixture(scope="module")
def lib():
    return _abi.load()


def test_exports_every_declared_symbol(lib):
    decl = _declared()
    assert decl == sorted(_abi.EXPORTS)
    for name in decl:
        assert hasattr(lib, name), name


def test_constants_match_header(lib):
    m = _macros()
    assert lib.gsa_abi_version() == m["GSA_ABI_VERSION"] == _abi.ABI_VERSION
    assert (m["GSA_DTYPE_F32"], m["GSA_DTYPE_BF16"]) == (_abi.DTYPE_F32, _abi.DTYPE_BF16)
    assert (m["GSA_ORDER_INDEX_ASC"], m["GSA_ORDER_SCORE_DESC"]) == (_abi.ORDER_INDEX_ASC, _abi.ORDER_SCORE_DESC)
    assert (m["GSA_ATTN_ROPE_Q"], m["GSA_ATTN_OUT_GATE"], m["GSA_ATTN_MASKS_READY"], m["GSA_ATTN_ROPE_HALVES"]) == (
        _abi.ATTN_ROPE_Q, _abi.ATTN_OUT_GATE, _abi.ATTN_MASKS_READY, _abi.ATTN_ROPE_HALVES)
    assert m["GSA_TOPK_DESC_MAX_K"] == _abi.TOPK_DESC_MAX_K


def test_status_strings(lib):
    for code in range(0, 8):
        assert _abi.status_string(code) not in ("", "unknown status")
    assert "HIP" in _abi.status_string(-1)
    assert _abi.status_string(99) == "unknown status"


def _scores(lib, **kw):
    a = dict(q=P, qsb=0, qst=256, k=P, ksb=0, kst=64, w=P, wsb=0, wst=4, bias=P, scale=0.125,
             B=1, T=32, Hi=4, di=64, causal=1, dtype=1, out=P, osb=0, ost=32)
    a.update(kw)
    return lib.gsa_indexer_scores(a["q"], a["qsb"], a["qst"], a["k"], a["ksb"], a["kst"], a["w"], a["wsb"],
                                  a["wst"], a["bias"], a["scale"], a["B"], a["T"], a["Hi"], a["di"],
                                  a["causal"], a["dtype"], a["out"], a["osb"], a["ost"], None)


def test_indexer_scores_validation(lib):
    assert _scores(lib, q=None) == 1
    assert _scores(lib, out=None) == 1
    assert _scores(lib, dtype=7) == 3
    assert _scores(lib, Hi=8) == 2
    assert _scores(lib, di=32) == 2
    assert _scores(lib, T=0) == 2
    assert _scores(lib, q=MIS) == 4
    assert _scores(lib, qst=260) == 4        # row stride not a multiple of 8 bf16
    # key tiles are addressed by 32-bit offsets: 16 rows of k must span < 2 GiB
    assert _scores(lib, kst=1 << 26) == 2
    assert _scores(lib, kst=-64) == 2


NWS_T32 = 2 * 512    # indexer-select workspace at B=1, T=32: two 16-row groups' store slots


def _select(lib, **kw):
    a = dict(q=P, qsb=0, qst=256, k=P, ksb=0, kst=64, w=P, wsb=0, wst=4, bias=P, scale=0.125,
             B=1, T=32, Hi=4, di=64, k_eff=8, dtype=1, bits=P, bsb=0, bst=2, idx=P, cnt=P, ws=P, nws=NWS_T32)
    a.update(kw)
    return lib.gsa_indexer_select(a["q"], a["qsb"], a["qst"], a["k"], a["ksb"], a["kst"], a["w"], a["wsb"],
                                  a["wst"], a["bias"], a["scale"], a["B"], a["T"], a["Hi"], a["di"],
                                  a["k_eff"], a["dtype"], a["bits"], a["bsb"], a["bst"], a["idx"], a["cnt"],
                                  a["ws"], a["nws"], None)


def test_indexer_select_validation(lib):
    assert _select(lib, bias=None) == 1
    assert _select(lib, bits=None) == 1
    assert _select(lib, cnt=None) == 1            # idx without count
    assert _select(lib, k_eff=0) == 5
    assert _select(lib, k_eff=33) == 5
    assert _select(lib, dtype=-1) == 3
    assert _select(lib, k=MIS) == 4
    assert _select(lib, bst=1) == 2               # fewer words than 2*ceil(T/64)
    assert _select(lib, bits=P + 4) == 4          # rows must be 8-byte aligned
    assert _select(lib, ws=None) == 1
    assert _select(lib, nws=NWS_T32 - 1) == 2     # workspace too small
    assert _select(lib, ws=P + 8) == 4
    assert _select(lib, T=65537, k_eff=8, bst=2 * 1025, nws=1 << 30) == 2   # past the fused selector's largest T
    assert _select(lib, kst=1 << 26) == 2         # 16 key rows past 2 GiB (32-bit tile offsets)
    # the candidate lists live in LDS: per 16-row group the workspace holds
    # only 64 8-byte store slots -- linear in T, 2 MiB at T = 65536
    assert lib.gsa_indexer_select_workspace_bytes(1, 32) == NWS_T32 == 2 * 512
    assert lib.gsa_indexer_select_workspace_bytes(2, 100) == 2 * 7 * 512
    assert lib.gsa_indexer_select_workspace_bytes(1, 65536) == 4096 * 512
    assert lib.gsa_indexer_select_workspace_bytes(0, 5) == 0


def _noalloc(lib, **kw):
    a = dict(q=P, qsb=0, qst=256, k=P, ksb=0, kst=64, w=P, wsb=0, wst=4, bias=P, scale=0.125,
             B=1, T=32, Hi=4, di=64, k_eff=8, dtype=1, bits=P, bsb=0, bst=2, idx=P, cnt=P)
    a.update(kw)
    return lib.gsa_indexer_select_noalloc(a["q"], a["qsb"], a["qst"], a["k"], a["ksb"], a["kst"], a["w"],
                                          a["wsb"], a["wst"], a["bias"], a["scale"], a["B"], a["T"], a["Hi"],
                                          a["di"], a["k_eff"], a["dtype"], a["bits"], a["bsb"], a["bst"],
                                          a["idx"], a["cnt"], None)


def test_indexer_select_noalloc_validation(lib):
    # the static scratch: 4 MiB = 8192 groups of 16 rows x 512 bytes of store slots
    assert lib.gsa_indexer_select_noalloc_max_bytes() == 4 << 20
    assert _abi.status_string(7).startswith("sizes exceed the static scratch")
    assert _noalloc(lib, bias=None) == 1
    assert _noalloc(lib, bits=None) == 1
    assert _noalloc(lib, cnt=None) == 1
    assert _noalloc(lib, k_eff=0) == 5
    assert _noalloc(lib, dtype=-1) == 3
    assert _noalloc(lib, k=MIS) == 4
    assert _noalloc(lib, bst=1) == 2
    # 8192 groups fit (B=2, T=65536); one more group does not
    W = 2 * 1024
    assert _noalloc(lib, B=4, T=32768 + 1, bst=W, bsb=(32768 + 1) * W) == 7
    assert _noalloc(lib, B=8193, T=16, bst=2, bsb=32) == 7
    assert _noalloc(lib, T=65537, bst=2 * 1025) == 2      # past the fused selector's largest T


def _adaptive(lib, **kw):
    a = dict(q=P, qsb=0, qst=256, k=P, ksb=0, kst=64, w=P, wsb=0, wst=4, bias=P, scale=0.125,
             B=1, T=32, Hi=4, di=64, kb=8, kmin=2, kmax=16, dtype=1, bits=P, bsb=0, bst=2, idx=P, cnt=P,
             kout=P, vout=P, ws=P, nws=NWS_A32)
    a.update(kw)
    return lib.gsa_indexer_select_adaptive(
        a["q"], a["qsb"], a["qst"], a["k"], a["ksb"], a["kst"], a["w"], a["wsb"], a["wst"], a["bias"],
        a["scale"], a["B"], a["T"], a["Hi"], a["di"], a["kb"], a["kmin"], a["kmax"], a["dtype"], a["bits"],
        a["bsb"], a["bst"], a["idx"], a["cnt"], a["kout"], a["vout"], a["ws"], a["nws"], None)


# adaptive workspace at B=1, T=32, each part rounded up to 256 bytes: the fixed
# selector's, the sample histograms (2 groups x 16 rows x 513 words of two
# 16-bit counts), then var and k (128 B each)
NWS_A32 = NWS_T32 + (2 * 16 * 513 * 4 + 255) // 256 * 256 + 2 * 256


def test_indexer_select_adaptive_validation(lib):
    assert lib.gsa_indexer_select_adaptive_workspace_bytes(1, 32) == NWS_A32
    hist = 4096 * 16 * 513 * 4
    fixed = lib.gsa_indexer_select_workspace_bytes(1, 65536)
    assert lib.gsa_indexer_select_adaptive_workspace_bytes(1, 65536) == fixed + hist + 2 * 65536 * 4
    assert lib.gsa_indexer_select_adaptive_workspace_bytes(0, 8) == 0
    assert _adaptive(lib, bias=None) == 1
    assert _adaptive(lib, ws=None) == 1
    assert _adaptive(lib, idx=None) == 1          # count without idx
    assert _adaptive(lib, kb=0) == 5
    assert _adaptive(lib, kmin=0) == 5
    assert _adaptive(lib, kmin=17) == 5           # k_min > k_max
    assert _adaptive(lib, kout=P + 2) == 4
    assert _adaptive(lib, nws=NWS_A32 - 1) == 2
    assert _adaptive(lib, dtype=7) == 3


def test_topk_adaptive_validation(lib):
    f = lib.gsa_topk_select_adaptive

    def call(scores=P, B=1, T=32, Tkv=32, kb=8, kmin=2, kmax=16, order=0, kout=P, vout=P):
        return f(scores, 0, 32, B, T, Tkv, kb, kmin, kmax, order, P, P, None, kout, vout, None)

    assert call(scores=None) == 1
    assert call(kout=None) == 1
    assert call(vout=None) == 1
    assert call(kmin=0) == 5
    assert call(kmin=20) == 5
    assert call(kb=0) == 5
    assert call(order=3) == 6
    assert call(T=0) == 2
    assert call(kout=P + 1) == 4
    assert call(Tkv=8192, kmax=5000, order=1) == 5   # desc order width cap


def test_dense_path_validation(lib):
    f = lib.gsa_selection_mask
    assert f(None, 0, 8, 8, None, None, 1, 4, 4, P, 0, 2, None) == 1
    assert f(P, 0, 8, 8, None, None, 1, 4, 4, P + 4, 0, 2, None) == 4
    assert f(P, 0, 8, 8, None, None, 1, 4, 1 << 20, P, 0, 2, None) == 2     # mask row too long for LDS
    g = lib.gsa_dense_attn
    ok = dict(q=P, qsb=0, qst=2048, k=P, ksb=0, kst=2048, vt=P, vtsb=0, vtsh=8192, ldv=64, bits=P, bsb=0, bst=2,
              og=P, osb=0, ost=2048, cos=P, sin=P, cst=128, out=P, outsb=0, outst=2048,
              B=1, T=4, Tkv=4, H=16, d=128, scale=0.088, dtype=1, flags=3, causal=1, ws=P, wsb=8 * 1024)

    def call(**kw):
        a = dict(ok)
        a.update(kw)
        return g(a["q"], a["qsb"], a["qst"], a["k"], a["ksb"], a["kst"], a["vt"], a["vtsb"], a["vtsh"], a["ldv"],
                 a["bits"], a["bsb"], a["bst"], a["og"], a["osb"], a["ost"], a["cos"], a["sin"], a["cst"],
                 a["out"], a["outsb"], a["outst"], a["B"], a["T"], a["Tkv"], a["H"], a["d"], a["scale"],
                 a["dtype"], a["flags"], a["causal"], a["ws"], a["wsb"], None)

    # 1 KiB of mask operands per (batch, 32-row group, 64-key tile); groups cover whole 256-row blocks
    assert lib.gsa_dense_attn_workspace_bytes(1, 4, 4) == 8 * 1024
    assert lib.gsa_dense_attn_workspace_bytes(2, 100, 130) == 2 * 8 * 3 * 1024
    assert lib.gsa_dense_attn_workspace_bytes(1, 257, 64) == 16 * 1024
    # 256-row blocks at every key count
    assert _abi.dense_block_rows(32767) == 256 and _abi.dense_block_rows(65536) == 256
    assert lib.gsa_dense_attn_workspace_bytes(1, 4, 32768) == 8 * 512 * 1024
    assert lib.gsa_dense_attn_workspace_bytes(2, 385, 40000) == 2 * 16 * 625 * 1024
    assert call(bits=None) == 1
    assert call(ws=None) == 1
    assert call(wsb=8 * 1024 - 1) == 2            # workspace too small
    assert call(dtype=0) == 3                     # bf16 only
    assert call(ldv=32) == 2                      # rows shorter than ceil(Tkv/64)*64
    assert call(flags=16) == 6                    # unknown flag
    assert call(flags=8) == 6 and call(flags=10) == 6   # packed RoPE table without RoPE(q)
    assert call(flags=1, sin=None) == 1           # RoPE(q) reads sin ...
    assert call(flags=9, sin=None, wsb=1) == 2    # ... except from the packed table (then the size check fails)
    assert call(flags=9, cos=None) == 1
    assert call(bst=3) == 4
    # row strides past 2^24 elements: the staging tiles' 32-row offsets are 32-bit
    big = (1 << 24) + 8
    assert call(qst=big) == 2 and call(outst=big) == 2
    assert call(ost=big) == 2 and call(ost=big, flags=1, og=None) != 2     # o_st matters only with the gate
    assert call(cst=big) == 2 and call(cst=big, flags=2) != 2               # cs_st only with RoPE(q)
    lmk = lib.gsa_dense_lane_masks
    assert lmk(None, 0, 2, 1, 4, 4, 1, P, 8 * 1024, None) == 1
    assert lmk(P, 0, 2, 1, 4, 4, 1, None, 8 * 1024, None) == 1
    assert lmk(P, 0, 2, 1, 4, 4, 1, P, 8 * 1024 - 1, None) == 2   # workspace too small
    assert lmk(P, 0, 1, 1, 4, 4, 1, P, 8 * 1024, None) == 2       # row of W words shorter than 2*ceil(Tkv/64)
    assert lmk(P, 0, 3, 1, 4, 4, 1, P, 8 * 1024, None) == 4       # 8-byte aligned rows
    assert lmk(P, 0, 2, 1, 4, 4, 1, P + 8, 8 * 1024, None) == 4   # 16-byte aligned workspace
    p = lib.gsa_prologue_vt
    assert p(P, 0, 2048, P, 0, 2048, P, 0, 2048, P, P, 128, 1, 4, 16, 128, 1, P, P, 100, None) == 2   # ldv % 64
    assert p(P, 0, 2048, None, 0, 2048, P, 0, 2048, P, P, 128, 1, 4, 16, 128, 1, P, P, 64, None) == 1


def test_topk_validation(lib):
    f = lib.gsa_topk_select
    assert f(None, 0, 32, 1, 32, 32, 4, 0, P, P, None, None) == 1
    assert f(P, 0, 32, 1, 32, 32, 0, 0, P, P, None, None) == 5
    assert f(P, 0, 32, 1, 32, 32, 33, 0, P, P, None, None) == 5
    assert f(P, 0, 8192, 1, 8, 8192, 5000, 1, P, P, None, None) == 5   # desc order k cap
    assert f(P, 0, 32, 1, 32, 32, 4, 9, P, P, None, None) == 6
    assert f(P, 0, 32, 0, 32, 32, 4, 0, P, P, None, None) == 2
    assert f(P + 2, 0, 32, 1, 32, 32, 4, 0, P, P, None, None) == 4


def test_prologue_validation(lib):
    f = lib.gsa_prologue
    ok = dict(k=P, ksb=0, kst=2048, v=P, vsb=0, vst=2048, g=P, gsb=0, gst=2048, cos=P, sin=P, cst=128,
              B=1, T=4, H=16, d=128, dtype=1, ko=P, vo=P)

    def call(**kw):
        a = dict(ok)
        a.update(kw)
        return f(a["k"], a["ksb"], a["kst"], a["v"], a["vsb"], a["vst"], a["g"], a["gsb"], a["gst"],
                 a["cos"], a["sin"], a["cst"], a["B"], a["T"], a["H"], a["d"], a["dtype"], a["ko"], a["vo"], None)

    assert call(k=None, v=None) == 1
    assert call(cos=None) == 1
    assert call(g=None) == 1
    assert call(d=64) == 2
    assert call(H=65) == 2
    assert call(dtype=5) == 3
    assert call(vo=MIS) == 4
    assert call(kst=2052) == 4


def test_sparse_attn_validation(lib):
    f = lib.gsa_sparse_attn
    ok = dict(q=P, qsb=0, qst=2048, k=P, ksb=0, kst=2048, v=P, vsb=0, vst=2048, idx=P, isb=0, ist=8, ksel=8,
              cnt=P, mask=None, og=P, osb=0, ost=2048, cos=P, sin=P, cst=128, out=P, outsb=0, outst=2048,
              B=1, T=4, Tkv=4, H=16, d=128, scale=0.088, dtype=1, flags=3)

    def call(**kw):
        a = dict(ok)
        a.update(kw)
        return f(a["q"], a["qsb"], a["qst"], a["k"], a["ksb"], a["kst"], a["v"], a["vsb"], a["vst"],
                 a["idx"], a["isb"], a["ist"], a["ksel"], a["cnt"], a["mask"], a["og"], a["osb"], a["ost"],
                 a["cos"], a["sin"], a["cst"], a["out"], a["outsb"], a["outst"], a["B"], a["T"], a["Tkv"],
                 a["H"], a["d"], a["scale"], a["dtype"], a["flags"], None)

    assert call(idx=None) == 1
    assert call(og=None) == 1                 # OUT_GATE without og
    assert call(cos=None) == 1                # ROPE_Q without tables
    assert call(flags=8) == 6
    assert call(d=96) == 2
    assert call(ksel=-1) == 5
    assert call(q=MIS) == 4
    assert call(idx=P + 2) == 4


def test_proj_validation(lib):
    assert lib.gsa_proj_packed_bytes(2048, 16) == 5 * 2048 * 2048 * 2
    assert lib.gsa_proj_packed_bytes(256, 2) == 5 * 256 * 256 * 2
    assert lib.gsa_proj_packed_bytes(384, 3) == 0          # odd head count: no 256-column tiles
    assert lib.gsa_proj_packed_bytes(2048, 8) == 0         # d_head != 128
    pk = lib.gsa_proj_pack
    assert pk(None, 2048, None, 2048, 16, 1, P, P, None) == 1
    assert pk(P, 2048, None, 2048, 16, 0, P, P, None) == 3
    assert pk(P, 2048, None, 384, 3, 1, P, P, None) == 2
    assert pk(P, 1000, None, 2048, 16, 1, P, P, None) == 2   # row stride < D
    assert pk(MIS, 2048, None, 2048, 16, 1, P, P, None) == 4
    f = lib.gsa_proj_fused
    ok = dict(x=P, xst=2048, B=1, T=512, D=2048, H=16, dtype=1, wp=P, bp=P, cos=P, sin=P, cst=128,
              q=P, qst=4096, og=P, ogst=4096, ko=P, vt=P, ldv=512)

    def call(**kw):
        a = dict(ok)
        a.update(kw)
        return f(a["x"], a["xst"], a["B"], a["T"], a["D"], a["H"], a["dtype"], a["wp"], a["bp"], a["cos"],
                 a["sin"], a["cst"], a["q"], a["qst"], a["og"], a["ogst"], a["ko"], a["vt"], a["ldv"], None)

    assert call(x=None) == 1
    assert call(vt=None) == 1
    assert call(dtype=0) == 3
    assert call(T=100) == 2                       # T % 64
    assert call(D=384, H=3) == 2
    assert call(ldv=448) == 2                     # ldv < T
    assert call(ldv=576 + 8) == 2                 # ldv % 64
    assert call(xst=1000) == 2                    # row stride < D
    assert call(x=MIS) == 4
    assert call(xst=2052) == 4                    # rows not 16-byte aligned
    assert call(qst=4098) == 4
    assert call(cst=130) == 4
