"""Kernel-level parity on the GPU: each C-ABI entry point against the oracle.

Tolerances (written per test): the selector and the fused indexer+select are
bit-exact against the oracle's tie-aware selector on identical fp32 scores;
indexer scores within rtol 2e-5 of the fp32 oracle; the bf16 elementwise
producer matches the oracle's op-by-op bf16 rounding; attention within one
bf16 rounding (bf16) or 1e-5 (fp32) of a float64 evaluation.
"""

import os

import numpy as np
import pytest
import torch

from gsa_gdn_benchmarkstudy_amd import _abi
from gsa_gdn_benchmarkstudy_amd import gsa as G
from oracle import gsa_oracle as orc

pytestmark = pytest.mark.gpu

DTYPES = [torch.bfloat16, torch.float32]


def _log(msg):
    print(msg, flush=True)


def _indexer_inputs(B, T, dtype, seed=0, pad=0):
    """q/k/w as strided views into one wider buffer, like the fused projection output."""
    g = torch.Generator().manual_seed(seed)
    width = 256 + 64 + 4 + pad
    buf = (torch.randn(B, T, width, generator=g)).to(dtype)
    q = buf[..., :256].view(B, T, 4, 64)
    k = buf[..., 256:320]
    w = buf[..., 320:324]
    bias = torch.randn(4, generator=g) * 0.5
    return buf, q, k, w, bias


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("B,T", [(1, 48), (2, 33), (1, 300)])
def test_indexer_scores_vs_oracle(dev, dtype, B, T):
    _log(f"indexer_scores dtype={dtype} B={B} T={T}")
    buf, q, k, w, bias = _indexer_inputs(B, T, dtype, seed=T, pad=60)
    bd = buf.to(dev)
    qd = bd[..., :256].view(B, T, 4, 64)
    kd, wd = bd[..., 256:320], bd[..., 320:324]
    s = _abi.indexer_scores(qd, kd, wd, bias.to(dev), 0.125).cpu()
    ref = orc.indexer_scores(q, k, w, bias, 0.125)
    assert torch.equal(torch.isinf(s), torch.isinf(ref))
    fin = torch.isfinite(ref)
    assert torch.allclose(s[fin], ref[fin], rtol=2e-5, atol=1e-6)


def test_indexer_scores_noncausal(dev):
    _, q, k, w, bias = _indexer_inputs(1, 40, torch.bfloat16, seed=9)
    s = _abi.indexer_scores(q.to(dev), k.to(dev), w.to(dev), bias.to(dev), 0.125, causal=False).cpu()
    ref = orc.indexer_scores(q, k, w, bias, 0.125, causal=False)
    assert torch.isfinite(s).all()
    assert torch.allclose(s, ref, rtol=2e-5, atol=1e-6)


def _tie_scores(B, T, levels, seed):
    g = torch.Generator().manual_seed(seed)
    s = torch.randint(0, levels, (B, T, T), generator=g).float() / levels
    return s.masked_fill(torch.triu(torch.ones(T, T, dtype=torch.bool), 1), float("-inf"))


@pytest.mark.parametrize("k", [1, 7, 33, 70])
def test_topk_select_golden_ties(dev, k):
    z = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "select_ties_T70.npz"))
    s = torch.from_numpy(z["scores"])
    _log(f"topk golden ties k={k}")
    idx, cnt, mask = _abi.topk_select(s.to(dev), k, _abi.ORDER_SCORE_DESC, want_mask=True)
    assert np.array_equal(idx.cpu().numpy(), z[f"idx_desc_k{k}"])
    assert np.array_equal(mask.cpu().numpy().astype(bool), z[f"mask_k{k}"])
    ia, ca, _ = _abi.topk_select(s.to(dev), k, _abi.ORDER_INDEX_ASC)
    assert np.array_equal(ia.cpu().numpy(), z[f"idx_asc_k{k}"])
    assert np.array_equal(ca.cpu().numpy(), z[f"count_k{k}"])


@pytest.mark.parametrize("T,k,levels", [(257, 64, 3), (1100, 300, 1000), (600, 600, 4), (2049, 2048, 50)])
def test_topk_select_bitexact(dev, T, k, levels):
    _log(f"topk bitexact T={T} k={k}")
    s = _tie_scores(1, T, levels, seed=T)
    idx, mask = orc.select_topk(s, k)
    ia, ca = orc.select_ascending(s, k)
    if k <= _abi.TOPK_DESC_MAX_K:
        gi, _, gm = _abi.topk_select(s.to(dev), k, _abi.ORDER_SCORE_DESC, want_mask=True)
        assert torch.equal(gi.cpu().long(), idx)
        assert torch.equal(gm.cpu().bool(), mask)
    gi, gc, _ = _abi.topk_select(s.to(dev), k, _abi.ORDER_INDEX_ASC)
    assert torch.equal(gi.cpu(), ia)
    assert torch.equal(gc.cpu(), ca)


def test_topk_select_special_values(dev):
    s = torch.tensor([[[0.5, float("nan"), 2.0, float("inf"), -1e9, float("-inf"), -3.0, 0.5]]])
    gi, gc, gm = _abi.topk_select(s.to(dev), 5, _abi.ORDER_INDEX_ASC, want_mask=True)
    # NaN ranks above +inf, -inf counts as -1e9 (ties with the real -1e9, lowest index first)
    assert gi.cpu().tolist() == [[[0, 1, 2, 3, 7]]]
    assert gc.item() == 5
    gi, gc, gm = _abi.topk_select(s.to(dev), 8, _abi.ORDER_INDEX_ASC, want_mask=True)
    assert gi.cpu().tolist() == [[[0, 1, 2, 3, 4, 6, 7, 5]]]
    assert gc.item() == 7 and gm.cpu().tolist() == [[[1, 1, 1, 1, 1, 1, 1, 0]]]


def _bits_to_sets(bits):
    """Per-row sets of set-bit positions of an int32 [B,T,W] bitmask."""
    w = bits.cpu().numpy().view(np.uint32)
    B, T, W = w.shape
    unpacked = np.unpackbits(w.view(np.uint8).reshape(B, T, W * 4), axis=-1, bitorder="little")
    return [[set(np.nonzero(unpacked[b, t])[0].tolist()) for t in range(T)] for b in range(B)]


class _NoForce:
    def __enter__(self):
        return self

    def __exit__(self, *exc):
        return False


def _select_mode(forced):
    """The fused selector's normal path (sampled band, candidates, resolve) or,
    forced, its exact fallback (radix select over recomputed scores)."""
    return _abi.forced_select_fallback() if forced else _NoForce()


@pytest.mark.parametrize("forced", [False, True])
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("B,T,k", [(1, 48, 16), (2, 33, 8), (1, 512, 256), (1, 1000, 100), (3, 130, 129),
                                   (1, 2100, 700), (1, 4100, 2048)])
def test_indexer_select_equals_scores_then_topk(dev, dtype, B, T, k, forced):
    """The fused kernel selects exactly what the score kernel + selector select,
    on its normal path and on its fallback path."""
    _log(f"indexer_select fused==unfused dtype={dtype} B={B} T={T} k={k} forced_fallback={forced}")
    buf, q, k_, w, bias = _indexer_inputs(B, T, dtype, seed=B * 1000 + T, pad=4)
    bd = buf.to(dev)
    qd = bd[..., :256].view(B, T, 4, 64)
    kd, wd, bias_d = bd[..., 256:320], bd[..., 320:324], bias.to(dev)
    with _select_mode(forced):
        fb, fi, fc = _abi.indexer_select(qd, kd, wd, bias_d, 0.125, k)
    s = _abi.indexer_scores(qd, kd, wd, bias_d, 0.125)
    ui, uc, _ = _abi.topk_select(s, k, _abi.ORDER_INDEX_ASC)
    assert torch.equal(fc.cpu(), uc.cpu())
    assert torch.equal(fi.cpu(), ui.cpu())
    ub = _abi.selection_mask(ui, T, count=uc)
    assert torch.equal(fb.cpu(), ub.cpu())
    # and the unfused path is bit-exact with the oracle selector on the same scores
    oi, oc = orc.select_ascending(s.cpu(), k)
    assert torch.equal(ui.cpu(), oi) and torch.equal(uc.cpu(), oc)


def test_indexer_select_long_rows_equal_scores_then_topk(dev):
    """Rows of more than 832 causal mask words (keys past 26624): the resolve ORs
    their band winners into the stored words in two bitmap chunks.  Fused select
    against the score kernel + selector on the same inputs, bit for bit (the
    unfused path is pinned to the oracle's selector at smaller T)."""
    B, T, k = 1, 27000, 2048
    _log(f"indexer_select long rows B={B} T={T} k={k}")
    buf, q, k_, w, bias = _indexer_inputs(B, T, torch.bfloat16, seed=27, pad=4)
    bd = buf.to(dev)
    qd = bd[..., :256].view(B, T, 4, 64)
    kd, wd, bias_d = bd[..., 256:320], bd[..., 320:324], bias.to(dev)
    fb, fi, fc = _abi.indexer_select(qd, kd, wd, bias_d, 0.125, k)
    s = _abi.indexer_scores(qd, kd, wd, bias_d, 0.125)
    ui, uc, _ = _abi.topk_select(s, k, _abi.ORDER_INDEX_ASC)
    del s
    assert torch.equal(fc, uc) and torch.equal(fi, ui)
    assert torch.equal(fb, _abi.selection_mask(ui, T, count=uc))


@pytest.mark.parametrize("forced", [False, True])
@pytest.mark.parametrize("T,k", [(700, 100), (300, 299), (1500, 40), (3000, 1000)])
def test_indexer_select_all_ties_overflow_path(dev, T, k, forced):
    """q = 0: every score of a row is equal, so the band holds the whole row: short
    rows resolve the ties among their candidates by index, rows with more keys
    than the candidate lists hold (T=3000) take the exact fallback; the lowest
    indices win."""
    _log(f"indexer_select all-ties T={T} k={k} forced_fallback={forced}")
    buf, q, k_, w, bias = _indexer_inputs(1, T, torch.bfloat16, seed=5, pad=4)
    buf[..., :256] = 0
    bd = buf.to(dev)
    qd = bd[..., :256].view(1, T, 4, 64)
    with _select_mode(forced):
        fb, fi, fc = _abi.indexer_select(qd, bd[..., 256:320], bd[..., 320:324], bias.to(dev), 0.125, k)
    fi, fc = fi.cpu(), fc.cpu()
    exp = torch.arange(k, dtype=torch.int32).expand(T, k)
    assert torch.equal(fi[0], exp)
    assert torch.equal(fc[0], torch.clamp(torch.arange(T) + 1, max=k).int())
    sets = _bits_to_sets(fb)[0]
    for t in range(T):
        assert sets[t] == set(range(min(t + 1, k)))


@pytest.mark.parametrize("forced", [False, True])
@pytest.mark.parametrize("dtype", DTYPES)
def test_indexer_select_nonfinite_and_extreme_inputs(dev, dtype, forced):
    """Planted non-finite and extreme inputs: a key with a NaN component (NaN
    scores in every later row, which rank above every number), a key with an
    infinite component (logits of +-inf), keys scaled so far that the sigmoid
    sum's common denominator overflows (the per-head form runs), and a query row
    whose gate weight is NaN (a whole row of NaN scores: ties, lowest indices
    win).  The fused selection equals score kernel + selector and the oracle's
    selector on those scores, on both selection paths."""
    B, T, k = 1, 1000, 100
    _log(f"indexer_select non-finite dtype={dtype} forced_fallback={forced}")
    buf, q, k_, w, bias = _indexer_inputs(B, T, dtype, seed=31, pad=4)
    buf[0, 200, 256 + 3] = float("nan")           # key 200: NaN dots
    buf[0, 350, 256 + 7] = float("inf")           # key 350: +-inf dots
    buf[0, 500:520, 256:320] *= 1e4               # keys 500..519: |logit| in the thousands
    buf[0, 700, 320 + 1] = float("nan")           # row 700: sigmoid(w) NaN
    bd = buf.to(dev)
    qd = bd[..., :256].view(B, T, 4, 64)
    kd, wd, bias_d = bd[..., 256:320], bd[..., 320:324], bias.to(dev)
    with _select_mode(forced):
        fb, fi, fc = _abi.indexer_select(qd, kd, wd, bias_d, 0.125, k)
    s = _abi.indexer_scores(qd, kd, wd, bias_d, 0.125)
    sc = s.cpu()
    assert torch.isnan(sc[0, 300, 200]) and torch.isnan(sc[0, 700, :701]).all()
    ui, uc, _ = _abi.topk_select(s, k, _abi.ORDER_INDEX_ASC)
    assert torch.equal(fc.cpu(), uc.cpu())
    assert torch.equal(fi.cpu(), ui.cpu())
    assert torch.equal(fb.cpu(), _abi.selection_mask(ui, T, count=uc).cpu())
    oi, oc = orc.select_ascending(sc, k)
    assert torch.equal(ui.cpu(), oi) and torch.equal(uc.cpu(), oc)
    # NaN ranks first: every row past key 200 selects it (but row 700, whose scores
    # are all NaN: there the lowest indices win)
    assert all(200 in set(fi[0, t, :fc[0, t]].tolist()) for t in range(201, T) if t != 700)
    assert fi[0, 700].tolist() == list(range(k))


def test_indexer_select_equals_scores_then_topk_T16384(dev):
    """T=16384, k=2048 on synthetic projections: the fused selection (sampled band,
    candidates, resolve) is bit-identical to the full score matrix followed by the
    standalone selector, every row (compared on the GPU)."""
    T, k = 16384, 2048
    _log("indexer_select fused==unfused T=16384")
    g = torch.Generator().manual_seed(7)
    x = torch.randn(1, T, 2048, generator=g).to(torch.bfloat16)
    W = (torch.randn(328, 2048, generator=g) * 0.02).to(torch.bfloat16)
    proj = torch.nn.functional.linear(x.to(dev), W.to(dev))
    q, kk, w = proj[..., :256].view(1, T, 4, 64), proj[..., 256:320], proj[..., 320:324]
    bias = torch.zeros(4, device=dev)
    fb, fi, fc = _abi.indexer_select(q, kk, w, bias, 0.125, k)
    s = _abi.indexer_scores(q, kk, w, bias, 0.125)
    ui, uc, _ = _abi.topk_select(s, k, _abi.ORDER_INDEX_ASC)
    del s
    assert torch.equal(fc, uc)
    assert torch.equal(fi, ui)
    assert torch.equal(fb, _abi.selection_mask(ui, T, count=uc))


def test_indexer_select_overlap_c2(dev):
    """T=4096, k=2048 on synthetic projections: the fused kernel's index sets vs the
    oracle's fp32 scores on identical bf16 inputs; overlap >= 99.9%."""
    T, k = 4096, 2048
    _log("indexer_select overlap c2 T=4096")
    g = torch.Generator().manual_seed(0)
    x = torch.randn(1, T, 2048, generator=g).to(torch.bfloat16)
    W = (torch.randn(328, 2048, generator=g) * 0.02).to(torch.bfloat16)   # rows padded to 16 bytes
    proj = torch.nn.functional.linear(x.to(dev), W.to(dev))          # [1,T,328] bf16 on the GPU
    q, kk, w = proj[..., :256].view(1, T, 4, 64), proj[..., 256:320], proj[..., 320:324]
    bias = torch.zeros(4)
    _, fi, fc = _abi.indexer_select(q, kk, w, bias.to(dev), 0.125, k)
    pc = proj.cpu()
    s = orc.indexer_scores(pc[..., :256].view(1, T, 4, 64), pc[..., 256:320], pc[..., 320:324], bias, 0.125)
    oi, oc = orc.select_ascending(s, k)
    assert torch.equal(fc.cpu(), oc)
    # set overlap on rows with more than k causal keys
    fi, oi = fi.cpu()[0, k:], oi[0, k:]
    same = 0
    for t in range(fi.shape[0]):
        same += np.intersect1d(fi[t].numpy(), oi[t].numpy(), assume_unique=True).size
    overlap = same / fi.numel()
    _log(f"  overlap={overlap:.6f}")
    assert overlap >= 0.999


def test_indexer_select_long_rows_T65536(dev):
    """T=65536: rows longer than 65535 keys take the kernel's 32-bit histogram
    variant.  Sampled rows (around the trivial-row boundary and the longest) of
    the fused selection vs the oracle's fp32 scores on identical bf16 inputs:
    counts exact, index overlap >= 99.9%."""
    T, k = 65536, 2048
    _log("indexer_select long rows T=65536")
    g = torch.Generator().manual_seed(3)
    x = torch.randn(1, T, 256, generator=g).to(torch.bfloat16)
    W = (torch.randn(328, 256, generator=g) * 0.06).to(torch.bfloat16)
    proj = torch.nn.functional.linear(x.to(dev), W.to(dev))
    q, kk, w = proj[..., :256].view(1, T, 4, 64), proj[..., 256:320], proj[..., 320:324]
    bias = torch.zeros(4)
    _, fi, fc = _abi.indexer_select(q, kk, w, bias.to(dev), 0.125, k)
    fi, fc = fi.cpu(), fc.cpu()
    pc = proj.cpu()
    same = total = 0
    for t in (2046, 2047, 2048, 30000, 65534, 65535):
        s = orc.indexer_scores(pc[:, t:t + 1, :256].view(1, 1, 4, 64), pc[..., 256:320], pc[:, t:t + 1, 320:324],
                               bias, 0.125, q_offset=t)
        oi, oc = orc.select_ascending(s, k)
        assert int(fc[0, t]) == int(oc[0, 0]) == min(t + 1, k)
        same += np.intersect1d(fi[0, t].numpy(), oi[0, 0].numpy(), assume_unique=True).size
        total += k
    _log(f"  overlap={same / total:.6f}")
    assert same / total >= 0.999


@pytest.mark.parametrize("dtype,k_scale,H", [(torch.bfloat16, 1.0, 4), (torch.float32, 1.0, 4),
                                             (torch.bfloat16, 1e-37, 4), (torch.bfloat16, 1e37, 4),
                                             (torch.bfloat16, 1.0, 64), (torch.float32, 1.0, 64)])
def test_prologue_vs_oracle(dev, dtype, k_scale, H):
    """RoPE(k) bit-exact with the oracle's bf16 ops (every product and sum rounded to
    bf16, round-to-nearest-even; random bf16 operands hit exact ties about once per
    256 products); k_scale 1e-37 puts the products and sums among fp32 subnormals,
    1e37 near the top of the range; 64 heads: one 1024-thread block per row."""
    B, T = 2, 40
    _log(f"prologue dtype={dtype} k_scale={k_scale} H={H}")
    g = torch.Generator().manual_seed(1)
    k = (torch.randn(B, T, H, 128, generator=g) * k_scale).to(dtype)
    v = torch.randn(B, T, H, 128, generator=g).to(dtype)
    vg = (torch.randn(B, T, H, 128, generator=g) * 3).to(dtype)
    cos, sin = orc.RopeCache(128, dtype).tables(T, dtype)
    ko, vo = _abi.prologue(k=k.to(dev), v=v.to(dev), vg=vg.to(dev), cos=cos.to(dev), sin=sin.to(dev))
    rk = orc.apply_rope(k, cos[None, :, None], sin[None, :, None])
    rv = v * torch.sigmoid(vg)
    assert torch.equal(ko.cpu(), rk)          # same ops, same rounding points
    if dtype == torch.bfloat16:
        # the sigmoid is the hardware exp2/rcp: allow a one-ulp bf16 difference on a few elements
        diff = (vo.cpu().float() - rv.float()).abs()
        ulp = rv.float().abs() * 2 ** -7 + 1e-30
        assert (diff <= ulp).all()
        assert (diff > 0).float().mean() < 2e-3
    else:
        assert torch.allclose(vo.cpu(), rv, rtol=2e-6, atol=1e-7)


def _attn_case(dtype, B, T, H, k, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, T, H, 128, generator=g).to(dtype)
    kk = torch.randn(B, T, H, 128, generator=g).to(dtype)
    v = torch.randn(B, T, H, 128, generator=g).to(dtype)
    s = torch.rand(B, T, T, generator=g).masked_fill(
        torch.triu(torch.ones(T, T, dtype=torch.bool), 1), float("-inf"))
    idx, mask = orc.select_topk(s, k)
    return q, kk, v, idx, mask


def _attn_ref64(q, k, v, idx, mask, scale):
    return orc.sparse_attention(q.double(), k.double(), v.double(), idx, mask, scale)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("B,T,H,k", [(1, 64, 16, 16), (2, 37, 4, 37), (1, 300, 2, 100), (1, 100, 64, 30)])
def test_sparse_attention_vs_oracle(dev, dtype, B, T, H, k):
    _log(f"sparse_attn dtype={dtype} B={B} T={T} H={H} k={k}")
    q, kk, v, idx, mask = _attn_case(dtype, B, T, H, k, seed=T)
    scale = 128 ** -0.5
    out = G.fused_sparse_attention(q.to(dev), kk.to(dev), v.to(dev), idx.to(dev), mask.to(dev), scale).cpu()
    ref = _attn_ref64(q, kk, v, idx, mask, scale)
    if dtype == torch.bfloat16:
        assert torch.all((out.double() - ref).abs() <= ref.abs() * 2 ** -8 + 1e-6)
    else:
        assert torch.allclose(out.double(), ref, atol=1e-5, rtol=1e-5)
    # rows with every entry masked give exactly zero
    assert torch.all(out[mask.sum(-1) == 0] == 0)


@pytest.mark.parametrize("dtype", DTYPES)
def test_sparse_attention_fused_rope_gate_count(dev, dtype):
    """ROPE_Q + OUT_GATE + ascending indices with counts == oracle composition."""
    B, T, H, k = 1, 96, 16, 24
    _log(f"sparse_attn fused flags dtype={dtype}")
    q, kk, v, _, _ = _attn_case(dtype, B, T, H, k, seed=3)
    g = torch.Generator().manual_seed(4)
    og = torch.randn(B, T, H, 128, generator=g).to(dtype)
    s = torch.rand(B, T, T, generator=g).masked_fill(
        torch.triu(torch.ones(T, T, dtype=torch.bool), 1), float("-inf"))
    ia, cnt = orc.select_ascending(s, k)
    cos, sin = orc.RopeCache(128, dtype).tables(T, dtype)
    out = _abi.sparse_attn(q.to(dev), kk.to(dev), v.to(dev), ia.to(dev), 128 ** -0.5, count=cnt.to(dev),
                           og=og.to(dev), cos=cos.to(dev), sin=sin.to(dev),
                           flags=_abi.ATTN_ROPE_Q | _abi.ATTN_OUT_GATE).cpu()
    qr = orc.apply_rope(q, cos[None, :, None], sin[None, :, None])
    mask = torch.arange(k)[None, None, :] < cnt[..., None]
    att = orc.sparse_attention(qr.double(), kk.double(), v.double(), ia, mask, 128 ** -0.5)
    if dtype == torch.bfloat16:
        # two bf16 roundings in a row (attention cast, gated product), each within
        # one ulp (<= 2^-7 relative) of the reference's: <= 2 ulps everywhere,
        # <= 1 ulp on all but 1% of the elements
        ref = (att.to(dtype) * torch.sigmoid(og)).double()
        diff = (out.double() - ref).abs()
        _log(f"  max rel {(diff / (ref.abs() + 1e-6)).max().item():.3e}")
        assert torch.all(diff <= ref.abs() * 2 ** -6 + 1e-6)
        assert (diff > ref.abs() * 2 ** -7 + 1e-6).double().mean() < 0.01
    else:
        ref = att * torch.sigmoid(og.double())
        assert torch.allclose(out.double(), ref, atol=1e-5, rtol=1e-5)


# ---------------------------------------------------------------------------
# block-dense attention path
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("B,T,H", [(2, 100, 4), (1, 130, 64)])
def test_prologue_vt_matches_prologue(dev, B, T, H):
    _log(f"prologue_vt B={B} T={T} H={H}")
    g = torch.Generator().manual_seed(11)
    k = torch.randn(B, T, H, 128, generator=g).to(torch.bfloat16).to(dev)
    v = torch.randn(B, T, H, 128, generator=g).to(torch.bfloat16).to(dev)
    vg = (torch.randn(B, T, H, 128, generator=g) * 3).to(torch.bfloat16).to(dev)
    cos, sin = orc.RopeCache(128, torch.bfloat16).tables(T, torch.bfloat16)
    cos, sin = cos.to(dev), sin.to(dev)
    ko, vo = _abi.prologue(k=k, v=v, vg=vg, cos=cos, sin=sin)
    ko2, vt = _abi.prologue_vt(v, vg, k=k, cos=cos, sin=sin)
    assert vt.shape == (B, H, 128, _abi.vt_len(T))
    assert torch.equal(ko.cpu(), ko2.cpu())
    assert torch.equal(vt[..., :T].cpu(), vo.permute(0, 2, 3, 1).cpu())
    assert torch.all(vt[..., T:].cpu() == 0)


def test_selection_mask_bits(dev):
    B, T, k = 2, 130, 20
    _log("selection_mask")
    s = _tie_scores(B, T, 1000, seed=3)
    ia, cnt = orc.select_ascending(s, k)
    bits = _abi.selection_mask(ia.to(dev), T, count=cnt.to(dev)).cpu()
    assert bits.shape == (B, T, 2 * ((T + 63) // 64))
    words = bits.numpy().view(np.uint32)
    for b in range(B):
        for t in range(T):
            got = {w * 32 + i for w in range(words.shape[2]) for i in range(32) if (words[b, t, w] >> i) & 1}
            assert got == set(ia[b, t, :cnt[b, t]].tolist())


def _dense_case(B, T, H, k, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, T, H, 128, generator=g).to(torch.bfloat16)
    kk = torch.randn(B, T, H, 128, generator=g).to(torch.bfloat16)
    v = torch.randn(B, T, H, 128, generator=g).to(torch.bfloat16)
    og = torch.randn(B, T, H, 128, generator=g).to(torch.bfloat16)
    s = torch.rand(B, T, T, generator=g).masked_fill(
        torch.triu(torch.ones(T, T, dtype=torch.bool), 1), float("-inf"))
    ia, cnt = orc.select_ascending(s, k)
    return q, kk, v, og, ia, cnt


@pytest.mark.parametrize("B,T,H,k", [(1, 64, 16, 16), (2, 100, 4, 37), (1, 300, 2, 100), (1, 1030, 16, 256),
                                     # 256-row query blocks and 64-key tiles: one short of, at and
                                     # one past the boundaries; one head; odd batch counts
                                     (1, 255, 1, 64), (3, 256, 2, 32), (1, 257, 1, 256), (2, 513, 2, 100),
                                     (1, 767, 3, 767),
                                     # more heads than the layer's 16, up to the ABI's 64 (the grid
                                     # puts heads fastest; 40 is no power of two)
                                     (2, 200, 40, 60), (1, 300, 64, 100)])
def test_dense_attention_vs_oracle_and_gather(dev, B, T, H, k):
    _log(f"dense_attn B={B} T={T} H={H} k={k}")
    q, kk, v, og, ia, cnt = _dense_case(B, T, H, k, seed=T + H)
    cos, sin = orc.RopeCache(128, torch.bfloat16).tables(T, torch.bfloat16)
    qd, kd, vd, ogd, iad, cntd = (t.to(dev) for t in (q, kk, v, og, ia, cnt))
    cosd, sind = cos.to(dev), sin.to(dev)
    ldv = _abi.vt_len(T)
    vt = torch.zeros(B, H, 128, ldv, dtype=torch.bfloat16, device=dev)
    vt[..., :T] = vd.permute(0, 2, 3, 1)
    bits = _abi.selection_mask(iad, T, count=cntd)
    flags = _abi.ATTN_ROPE_Q | _abi.ATTN_OUT_GATE
    dense = _abi.dense_attn(qd, kd, vt, bits, 128 ** -0.5, og=ogd, cos=cosd, sin=sind, flags=flags).cpu()
    gather = _abi.sparse_attn(qd, kd, vd, iad, 128 ** -0.5, count=cntd, og=ogd, cos=cosd, sin=sind,
                              flags=flags).cpu()
    qr = orc.apply_rope(q, cos[None, :, None], sin[None, :, None])
    mask = torch.arange(k)[None, None, :] < cnt[..., None]
    att = orc.sparse_attention(qr.double(), kk.double(), v.double(), ia, mask, 128 ** -0.5)
    ref = (att.to(torch.bfloat16) * torch.sigmoid(og)).double()
    for name, out in (("dense", dense), ("gather", gather)):
        diff = (out.double() - ref).abs()
        rel = (torch.linalg.vector_norm(out.double() - ref) / torch.linalg.vector_norm(ref)).item()
        _log(f"  {name}: rel-L2 {rel:.2e} max|diff| {diff.max().item():.2e}")
        # The dense kernel rounds P to bf16 before P.V: each normalised weight
        # moves by at most 2^-9 of itself, so the output moves by at most
        # 2^-8 * max|v|; plus two bf16 output roundings (2^-6 relative)
        assert torch.all(diff <= ref.abs() * 2 ** -6 + 2 ** -8 * v.abs().max().item() + 1e-6)
        assert rel < 5e-3


@pytest.mark.parametrize("flags", [0, 1, 2, 3])
def test_dense_attention_flags_and_strided_rows(dev, flags):
    """Every combination of RoPE(q) and the output gate, with q, og and out as
    row-strided views (row stride H*128 + 64 elements, like the layer's views of
    its fused projection) and T = 300 (the last 32-row wave of the second query
    block is partly past T): the staged prologue and epilogue read and write
    exactly the rows and columns of the views, and the result matches the
    float64 oracle within the bound of the test above; the padding columns
    beside out's rows stay untouched."""
    B, T, H, k = 2, 300, 3, 100
    fl = (_abi.ATTN_ROPE_Q if flags & 1 else 0) | (_abi.ATTN_OUT_GATE if flags & 2 else 0)
    _log(f"dense_attn flags={fl} strided rows B={B} T={T} H={H} k={k}")
    q, kk, v, og, ia, cnt = _dense_case(B, T, H, k, seed=31 + flags)
    cos, sin = orc.RopeCache(128, torch.bfloat16).tables(T, torch.bfloat16)
    HD = H * 128

    def strided(x):
        buf = torch.full((B, T, HD + 64), 7.0, dtype=torch.bfloat16, device=dev)
        buf[..., :HD] = x.reshape(B, T, HD).to(dev)
        return buf, buf[..., :HD].view(B, T, H, 128)

    _, qv = strided(q)
    _, ogv = strided(og)
    obuf, outv = strided(torch.zeros(B, T, H, 128, dtype=torch.bfloat16))
    assert qv.stride(1) == HD + 64 and not qv.is_contiguous()
    vt = torch.zeros(B, H, 128, _abi.vt_len(T), dtype=torch.bfloat16, device=dev)
    vt[..., :T] = v.to(dev).permute(0, 2, 3, 1)
    bits = _abi.selection_mask(ia.to(dev), T, count=cnt.to(dev))
    _abi.dense_attn(qv, kk.to(dev), vt, bits, 128 ** -0.5, og=ogv if fl & _abi.ATTN_OUT_GATE else None,
                    cos=cos.to(dev), sin=sin.to(dev), flags=fl, out=outv)
    out = outv.cpu()
    qr = orc.apply_rope(q, cos[None, :, None], sin[None, :, None]) if fl & _abi.ATTN_ROPE_Q else q
    mask = torch.arange(k)[None, None, :] < cnt[..., None]
    att = orc.sparse_attention(qr.double(), kk.double(), v.double(), ia, mask, 128 ** -0.5).to(torch.bfloat16)
    ref = (att * torch.sigmoid(og) if fl & _abi.ATTN_OUT_GATE else att).double()
    diff = (out.double() - ref).abs()
    _log(f"  max|diff| {diff.max().item():.2e}")
    assert torch.all(diff <= ref.abs() * 2 ** -6 + 2 ** -8 * v.abs().max().item() + 1e-6)
    assert torch.all(obuf[..., HD:].cpu() == 7.0)


def test_dense_attention_packed_rope_table(dev):
    """ATTN_ROPE_HALVES: the cos|sin halves packed into one table (here a
    row-strided view, row stride 192 elements) give the same bits as the full
    cos and sin tables, which repeat their first 64 entries as RotaryEmbedding
    builds them; T = 300 leaves the second query block's last wave partly past
    T, where the staging tile's rows are clamped."""
    B, T, H, k = 2, 300, 3, 100
    _log(f"dense_attn packed RoPE table B={B} T={T} H={H} k={k}")
    q, kk, v, og, ia, cnt = _dense_case(B, T, H, k, seed=41)
    cos, sin = orc.RopeCache(128, torch.bfloat16).tables(T, torch.bfloat16)
    assert torch.equal(cos[:, :64], cos[:, 64:]) and torch.equal(sin[:, :64], sin[:, 64:])
    buf = torch.full((T, 192), 9.0, dtype=torch.bfloat16)
    buf[:, :64], buf[:, 64:128] = cos[:, :64], sin[:, :64]
    packed = buf.to(dev)[:, :128]
    assert packed.stride(0) == 192
    vt = torch.zeros(B, H, 128, _abi.vt_len(T), dtype=torch.bfloat16, device=dev)
    vt[..., :T] = v.to(dev).permute(0, 2, 3, 1)
    bits = _abi.selection_mask(ia.to(dev), T, count=cnt.to(dev))
    fl = _abi.ATTN_ROPE_Q | _abi.ATTN_OUT_GATE
    qd, kd, ogd = q.to(dev), kk.to(dev), og.to(dev)
    full = _abi.dense_attn(qd, kd, vt, bits, 128 ** -0.5, og=ogd, cos=cos.to(dev), sin=sin.to(dev), flags=fl)
    half = _abi.dense_attn(qd, kd, vt, bits, 128 ** -0.5, og=ogd, cos=packed, flags=fl | _abi.ATTN_ROPE_HALVES)
    assert torch.equal(full, half)
    # and RoPE is really applied: without it the output differs
    plain = _abi.dense_attn(qd, kd, vt, bits, 128 ** -0.5, og=ogd, flags=_abi.ATTN_OUT_GATE)
    assert not torch.equal(plain, half)


@pytest.mark.parametrize("slope", [12.0, -12.0])
def test_dense_attention_moving_softmax_reference(dev, slope):
    """Logits that climb (or fall) by about `slope` log2 units per 64-key tile.
    Climbing, every tile moves every row's lazy softmax reference, so O and l
    are rescaled by about 2^-12 over and over while they hold earlier keys'
    weight; falling, the first tile's reference holds and later weights fade
    towards 0.  Against a float64 oracle: a rescale that is skipped, applied
    twice or applied after a half's PV product shows as an O(1) error."""
    _log(f"dense_attn moving reference slope={slope}")
    B, T, H, k = 1, 640, 2, 160
    g = torch.Generator().manual_seed(17)
    scale = 128 ** -0.5
    a = 4.0                                           # query component along dim 0
    gamma = slope / (64 * scale * 1.4426950408889634) / a   # key j carries gamma * j along dim 0
    q = 0.1 * torch.randn(B, T, H, 128, generator=g)
    q[..., 0] = a
    kk = 0.1 * torch.randn(B, T, H, 128, generator=g)
    kk[..., 0] = gamma * torch.arange(T, dtype=torch.float32).view(1, T, 1)
    q, kk = q.to(torch.bfloat16), kk.to(torch.bfloat16)
    v = torch.randn(B, T, H, 128, generator=g).to(torch.bfloat16)
    s = torch.rand(B, T, T, generator=g).masked_fill(
        torch.triu(torch.ones(T, T, dtype=torch.bool), 1), float("-inf"))
    ia, cnt = orc.select_ascending(s, k)
    vt = torch.zeros(B, H, 128, _abi.vt_len(T), dtype=torch.bfloat16, device=dev)
    vt[..., :T] = v.to(dev).permute(0, 2, 3, 1)
    bits = _abi.selection_mask(ia.to(dev), T, count=cnt.to(dev))
    out = _abi.dense_attn(q.to(dev), kk.to(dev), vt, bits, scale).cpu()
    mask = torch.arange(k)[None, None, :] < cnt[..., None]
    ref = orc.sparse_attention(q.double(), kk.double(), v.double(), ia, mask, scale)
    diff = (out.double() - ref).abs()
    _log(f"  max|diff| {diff.max().item():.2e}")
    # the bound of test_dense_attention_vs_oracle_and_gather: P rounded to bf16
    # (2^-8 * max|v|) and one bf16 output rounding
    assert torch.all(diff <= ref.abs() * 2 ** -7 + 2 ** -8 * v.abs().max().item() + 1e-6)


def test_dense_attention_noncausal_selection(dev):
    """A selection with keys after the query (non-causal) is honoured with causal=False."""
    B, T, H, k = 1, 128, 2, 8
    g = torch.Generator().manual_seed(5)
    q = torch.randn(B, T, H, 128, generator=g).to(torch.bfloat16)
    kk = torch.randn(B, T, H, 128, generator=g).to(torch.bfloat16)
    v = torch.randn(B, T, H, 128, generator=g).to(torch.bfloat16)
    s = torch.rand(B, T, T, generator=g)
    ia, cnt = orc.select_ascending(s, k)
    vt = torch.zeros(B, H, 128, 128, dtype=torch.bfloat16)
    vt[..., :T] = v.permute(0, 2, 3, 1)
    bits = _abi.selection_mask(ia.to(dev), T, count=cnt.to(dev))
    out = _abi.dense_attn(q.to(dev), kk.to(dev), vt.to(dev), bits, 0.1, causal=False).cpu()
    mask = torch.arange(k)[None, None, :] < cnt[..., None]
    ref = orc.sparse_attention(q.double(), kk.double(), v.double(), ia, mask, 0.1)
    assert (torch.linalg.vector_norm(out.double() - ref) / torch.linalg.vector_norm(ref)).item() < 5e-3


def _long_keys_case(T, Tkv, H, k, seed, causal, key_limit=None, B=1):
    """q [B,T,H,d], k/v [B,Tkv,H,d] and k selected keys per row: random
    among the row's causal prefix (causal) or among all keys below key_limit."""
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, T, H, 128, generator=g).to(torch.bfloat16)
    kk = torch.randn(B, Tkv, H, 128, generator=g).to(torch.bfloat16)
    v = torch.randn(B, Tkv, H, 128, generator=g).to(torch.bfloat16)
    og = torch.randn(B, T, H, 128, generator=g).to(torch.bfloat16)
    s = torch.rand(B, T, Tkv, generator=g)
    if causal:
        s = s.masked_fill(torch.arange(Tkv)[None, None, :] > torch.arange(T)[None, :, None], float("-inf"))
    if key_limit is not None:
        s[..., key_limit:] = float("-inf")
    ia, cnt = orc.select_ascending(s, k)
    return q, kk, v, og, ia, cnt


def _vt_of(v, dev):
    B, Tkv, H, _ = v.shape
    vt = torch.zeros(B, H, 128, _abi.vt_len(Tkv), dtype=torch.bfloat16, device=dev)
    vt[..., :Tkv] = v.to(dev).permute(0, 2, 3, 1)
    return vt


@pytest.mark.parametrize("B,T,Tkv,H,k,causal", [(1, 800, 33000, 2, 300, False), (1, 800, 33000, 2, 300, True),
                                                (1, 385, 32768, 1, 64, False), (2, 400, 32768, 3, 96, True)])
def test_dense_attention_long_keys_vs_oracle(dev, B, T, Tkv, H, k, causal):
    """Long key ranges (more than 512 tiles per row): ragged query blocks (T =
    3*256 + 32, 256 + 129), a ragged last key tile (33000 = 515*64 + 40), causal
    and non-causal selections, RoPE(q) and the output gate, against the float64
    oracle with the bound of the short-key test; a batch of two sequences
    checks the per-sequence offsets."""
    _log(f"dense_attn long keys B={B} T={T} Tkv={Tkv} H={H} k={k} causal={causal}")
    q, kk, v, og, ia, cnt = _long_keys_case(T, Tkv, H, k, seed=T + Tkv, causal=causal, B=B)
    cos, sin = orc.RopeCache(128, torch.bfloat16).tables(T, torch.bfloat16)
    bits = _abi.selection_mask(ia.to(dev), Tkv, count=cnt.to(dev))
    flags = _abi.ATTN_ROPE_Q | _abi.ATTN_OUT_GATE
    out = _abi.dense_attn(q.to(dev), kk.to(dev), _vt_of(v, dev), bits, 128 ** -0.5, og=og.to(dev),
                          cos=cos.to(dev), sin=sin.to(dev), flags=flags, causal=causal).cpu()
    qr = orc.apply_rope(q, cos[None, :, None], sin[None, :, None])
    mask = torch.arange(k)[None, None, :] < cnt[..., None]
    att = orc.sparse_attention(qr.double(), kk.double(), v.double(), ia, mask, 128 ** -0.5)
    ref = (att.to(torch.bfloat16) * torch.sigmoid(og)).double()
    diff = (out.double() - ref).abs()
    rel = (torch.linalg.vector_norm(out.double() - ref) / torch.linalg.vector_norm(ref)).item()
    _log(f"  rel-L2 {rel:.2e} max|diff| {diff.max().item():.2e}")
    assert torch.all(diff <= ref.abs() * 2 ** -6 + 2 ** -8 * v.abs().max().item() + 1e-6)
    assert rel < 5e-3


def test_dense_attention_masked_tiles_add_nothing(dev):
    """32768 keys against the first 32000 of the same keys, on a selection that
    only uses keys below 32000: the 12 extra tiles of every row are fully
    masked (their mask products start the scores near -8e36, so their p are
    exact zeros), so the outputs agree bit for bit."""
    T, H, k = 1000, 2, 256
    _log(f"dense_attn masked tiles T={T} H={H} k={k}")
    q, kk, v, og, ia, cnt = _long_keys_case(T, 32768, H, k, seed=7, causal=False, key_limit=32000)
    cos, sin = orc.RopeCache(128, torch.bfloat16).tables(T, torch.bfloat16)
    qd, ogd, cosd, sind, iad, cntd = (t.to(dev) for t in (q, og, cos, sin, ia, cnt))
    flags = _abi.ATTN_ROPE_Q | _abi.ATTN_OUT_GATE
    outs = []
    for Tkv in (32768, 32000):
        bits = _abi.selection_mask(iad, Tkv, count=cntd)
        outs.append(_abi.dense_attn(qd, kk[:, :Tkv].contiguous().to(dev), _vt_of(v[:, :Tkv], dev), bits,
                                    128 ** -0.5, og=ogd, cos=cosd, sin=sind, flags=flags, causal=False).cpu())
    assert torch.equal(outs[0], outs[1])


@pytest.mark.parametrize("causal_masks", [True, False])
def test_dense_lane_masks_then_attention_equals_one_call(dev, causal_masks):
    """gsa_dense_lane_masks on another stream, then gsa_dense_attn with
    GSA_ATTN_MASKS_READY: the same output as the one-call path, bit for bit,
    with the causal call's own masks or with masks of every tile."""
    B, T, H, k = 2, 300, 4, 64
    q, kk, v, og, ia, cnt = _dense_case(B, T, H, k, seed=91)
    cos, sin = orc.RopeCache(128, torch.bfloat16).tables(T, torch.bfloat16)
    qd, kd, ogd = q.to(dev), kk.to(dev), og.to(dev)
    cosd, sind = cos.to(dev), sin.to(dev)
    vt = torch.zeros(B, H, 128, _abi.vt_len(T), dtype=torch.bfloat16, device=dev)
    vt[..., :T] = v.to(dev).permute(0, 2, 3, 1)
    bits = _abi.selection_mask(ia.to(dev), T, count=cnt.to(dev))
    flags = _abi.ATTN_ROPE_Q | _abi.ATTN_OUT_GATE
    one = _abi.dense_attn(qd, kd, vt, bits, 128 ** -0.5, og=ogd, cos=cosd, sin=sind, flags=flags)
    side = torch.cuda.Stream(device=dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        ws = _abi.dense_lane_masks(bits, T, causal=causal_masks)
    torch.cuda.current_stream(dev).wait_stream(side)
    two = _abi.dense_attn(qd, kd, vt, bits, 128 ** -0.5, og=ogd, cos=cosd, sin=sind, flags=flags,
                          ws=ws, masks_ready=True)
    torch.cuda.synchronize()
    assert torch.equal(one.cpu(), two.cpu())


def test_causal_masks_refused_by_a_non_causal_call(dev):
    """Mask operands built for a causal attention leave the tiles past each
    query block unwritten: dense_attn refuses them for a non-causal call
    (before any launch) and takes them for a causal one."""
    B, T, H, k = 1, 300, 2, 64
    q, kk, v, og, ia, cnt = _dense_case(B, T, H, k, seed=17)
    qd, kd = q.to(dev), kk.to(dev)
    vt = torch.zeros(B, H, 128, _abi.vt_len(T), dtype=torch.bfloat16, device=dev)
    vt[..., :T] = v.to(dev).permute(0, 2, 3, 1)
    bits = _abi.selection_mask(ia.to(dev), T, count=cnt.to(dev))
    ws = _abi.dense_lane_masks(bits, T, causal=True)
    with pytest.raises(ValueError):
        _abi.dense_attn(qd, kd, vt, bits, 128 ** -0.5, causal=False, ws=ws, masks_ready=True)
    a = _abi.dense_attn(qd, kd, vt, bits, 128 ** -0.5, causal=True, ws=ws, masks_ready=True)
    b = _abi.dense_attn(qd, kd, vt, bits, 128 ** -0.5, causal=True)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


def _lane_masks_expected(bits, T, Tkv):
    """The dense attention's mask operands, stated from the bitmask alone:
    record [b, g, kt, l] (16 bytes, lane l = 32h + n) holds 32 e2m1 nibbles,
    nibble i (bits 4i..4i+3, little-endian u32 words) 0x0 if row 32g + n (< T)
    selects key 64kt + 32h + i and 0xF (-6.0) if not (rows past T select nothing)."""
    B = bits.shape[0]
    NT = (Tkv + 63) // 64
    rows_per_block = _abi.dense_block_rows(Tkv)                          # groups cover whole blocks
    G = (T + rows_per_block - 1) // rows_per_block * (rows_per_block // 32)
    w = bits.cpu().numpy().view(np.uint32)[..., :2 * NT].astype(np.uint64)   # [B, T, 2NT]
    rows = np.zeros((B, G * 32, 2 * NT), np.uint64)
    rows[:, :T] = w
    rows = rows.reshape(B, G, 32, NT, 2).transpose(0, 1, 3, 4, 2)           # [B, G, NT, h, n]
    sel = (rows[..., None] >> np.arange(32, dtype=np.uint64)) & np.uint64(1)   # [B, G, NT, h, n, 32]
    nib = ((np.uint64(1) - sel) * np.uint64(15)).reshape(B, G, NT, 2, 32, 4, 8)
    words = (nib << (np.uint64(4) * np.arange(8, dtype=np.uint64))).sum(-1)   # [B, G, NT, h, n, 4]
    return words.reshape(B, G, NT, 64, 4).astype(np.uint32)


@pytest.mark.parametrize("B,T,Tkv,density", [(2, 300, 300, 0.5), (1, 777, 1000, 0.1), (1, 64, 64, 0.9),
                                             (3, 520, 130, 0.03),
                                             # more than 512 key tiles
                                             (1, 400, 32800, 0.01), (2, 390, 32800, 0.01)])
@pytest.mark.parametrize("causal", [False, True])
def test_dense_lane_masks_layout(dev, B, T, Tkv, density, causal):
    """gsa_dense_lane_masks against the layout stated from the bitmask, on a random
    (not causal: every word populated) selection, ragged T and T != Tkv.  With
    causal, the tiles up to the last row of each group's query block (the ones a
    causal attention reads) hold the same words and the rest of the workspace is
    left as it was."""
    _log(f"lane masks layout B={B} T={T} Tkv={Tkv} density={density} causal={causal}")
    g = torch.Generator().manual_seed(T + Tkv)
    sel = torch.rand(B, T, (Tkv + 63) // 64 * 64, generator=g) < density
    sel[..., Tkv:] = False
    words = (sel.view(B, T, -1, 32).to(torch.int64) << torch.arange(32)).sum(-1)
    bits = words.to(torch.int32).contiguous().to(dev)
    want = _lane_masks_expected(bits, T, Tkv)
    ws = torch.full((want.size * 4,), 0xA5, dtype=torch.uint8, device=dev)
    _abi.dense_lane_masks(bits, Tkv, ws=ws, causal=causal)
    torch.cuda.synchronize()
    got = ws.cpu().numpy().view(np.uint32).reshape(want.shape)
    if not causal:
        assert np.array_equal(got, want)
        return
    rows = _abi.dense_block_rows(Tkv)
    nt = np.minimum(want.shape[2], ((32 * np.arange(want.shape[1])) // rows + 1) * rows // 64)   # per group
    read = np.arange(want.shape[2])[None, :] < nt[:, None]                                     # [G, NT]
    assert np.array_equal(got[:, read], want[:, read])
    assert np.all(got[:, ~read] == np.uint32(0xA5A5A5A5))


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("B,T,H", [(1, 100, 2), (2, 256, 4), (1, 700, 3)])
def test_prologue_vt_lane_masks_equals_two_launches(dev, B, T, H, causal):
    """gsa_prologue_vt_lane_masks (producer and lane masks in one launch, blocks
    interleaved) writes exactly what gsa_prologue_vt and gsa_dense_lane_masks write."""
    _log(f"prologue_vt+lane masks B={B} T={T} H={H} causal={causal}")
    g = torch.Generator().manual_seed(T + H)
    k = torch.randn(B, T, H, 128, generator=g).to(torch.bfloat16).to(dev)
    v = torch.randn(B, T, H, 128, generator=g).to(torch.bfloat16).to(dev)
    vg = (torch.randn(B, T, H, 128, generator=g) * 3).to(torch.bfloat16).to(dev)
    cos, sin = orc.RopeCache(128, torch.bfloat16).tables(T, torch.bfloat16)
    cos, sin = cos.to(dev), sin.to(dev)
    s = torch.rand(B, T, T, generator=g).masked_fill(torch.triu(torch.ones(T, T, dtype=torch.bool), 1), float("-inf"))
    idx, mask = orc.select_topk(s, min(40, T))
    bits = _abi.selection_mask(idx.to(torch.int32).to(dev), T, mask=mask.to(dev))
    ko, vt = _abi.prologue_vt(v, vg, k=k, cos=cos, sin=sin)
    nbytes = _abi.load().gsa_dense_attn_workspace_bytes(B, T, T)
    lm = _abi.dense_lane_masks(bits, T, ws=torch.full((nbytes,), 0x5A, dtype=torch.uint8, device=dev),
                               causal=causal)
    ko2, vt2, lm2 = _abi.prologue_vt(v, vg, k=k, cos=cos, sin=sin, bits=bits, Tkv=T, causal=causal,
                                     ws=torch.full((nbytes,), 0x5A, dtype=torch.uint8, device=dev))
    torch.cuda.synchronize()
    assert torch.equal(ko.cpu(), ko2.cpu()) and torch.equal(vt.cpu(), vt2.cpu())
    # both calls write the same words (and, causal, leave the same tiles unwritten)
    assert torch.equal(lm.cpu(), lm2.cpu())
