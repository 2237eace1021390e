"""Variance-based adaptive k on the GPU (gsa_explained.ipynb:577-592) against
the oracle, for the standalone selector (gsa_topk_select_adaptive), the fused
indexer + select (gsa_indexer_select_adaptive) and the layer in variance mode.

Bars (written per test):
- var_t: within rtol 2e-5 of a float64 two-pass variance of the same fp32
  scores (standalone, two-pass in fp32), 1e-4 for the fused kernel's shifted
  one-pass sums.
- k_t: inside the band floor(r(1 -+ 2e-4)) of the float64 ratio
  r = k_base*avg/var_t, and equal to the oracle's adaptive_k on the same scores
  except on at most 2% of the rows (a floor boundary between two fp32
  variances), there by one.
- selection: given the kernel's own k_t, bit-exact with the oracle's tie-aware
  selector on the same fp32 scores.
"""

import numpy as np
import pytest
import torch

from gsa_gdn_benchmarkstudy_amd import GatedSparseAttention, _abi
from oracle import gsa_oracle as orc

pytestmark = pytest.mark.gpu


def _log(msg):
    print(msg, flush=True)


def _var64(S):
    """float64 two-pass population variance of each row's finite entries."""
    s = S.double().numpy()
    fin = np.isfinite(s)
    n = np.maximum(fin.sum(-1), 1)
    z = np.where(fin, s, 0.0)
    mean = z.sum(-1) / n
    d = np.where(fin, s - mean[..., None], 0.0)
    return (d * d).sum(-1) / n


def _check_k(k_dev, S, k_base, k_min, k_max, cap, eps=2e-4):
    """k_dev int [B,T] against the oracle's adaptive_k on fp32 scores S [B,T,Tkv].

    Every k_t must lie in [floor(r(1-eps)), floor(r(1+eps))] (clamped), r the
    float64 ratio k_base*avg/var_t, eps above the variance tolerance; at most 2%
    of the rows may differ from the oracle's fp32 value (a floor boundary
    between the two fp32 variances), by one."""
    k_orc = orc.adaptive_k(S, k_base, k_min, k_max).clamp(max=cap).numpy()
    v = _var64(S)
    r = k_base * max(v.mean(), 1e-6) / np.maximum(v, 1e-6)
    lo = np.clip(np.floor(r * (1 - eps)), k_min, k_max).clip(max=cap)
    hi = np.clip(np.floor(r * (1 + eps)), k_min, k_max).clip(max=cap)
    k = k_dev.numpy()
    assert np.all((k >= lo) & (k <= hi)), f"{int(((k < lo) | (k > hi)).sum())} rows outside the float64 band"
    diff = k != k_orc
    assert np.all(np.abs(k - k_orc) <= 1)
    assert diff.mean() <= 0.02, f"{diff.mean():.4f} of rows differ from the oracle"
    _log(f"  k range [{k.min()}, {k.max()}], {int(diff.sum())} of {k.size} rows differ from the oracle by one")
    return k


def _sigma_scores(B, T, seed):
    """Causal fp32 scores with row statistics that vary across rows and batches."""
    g = torch.Generator().manual_seed(seed)
    sig = 0.2 + 1.8 * torch.rand(B, T, 1, generator=g)
    S = torch.sigmoid(torch.randn(B, T, T, generator=g) * sig) * 4.0
    S = S.masked_fill(torch.ones(T, T, dtype=torch.bool).triu(1), float("-inf"))
    return S.contiguous()


@pytest.mark.parametrize("order", [0, 1])
@pytest.mark.parametrize("B,T,k_base,k_min,k_max", [(2, 300, 40, 8, 96), (1, 1100, 200, 32, 400),
                                                    (3, 70, 16, 4, 80)])
def test_topk_select_adaptive_vs_oracle(dev, order, B, T, k_base, k_min, k_max):
    _log(f"topk_select_adaptive B={B} T={T} k=({k_base},{k_min},{k_max}) order={order}")
    S = _sigma_scores(B, T, seed=T + order)
    idx, cnt, mask, k_rows, var = _abi.topk_select_adaptive(S.to(dev), k_base, k_min, k_max, order,
                                                            want_mask=True)
    idx, cnt, mask, k_rows, var = (t.cpu() for t in (idx, cnt, mask, k_rows, var))
    W = min(k_max, T)
    assert idx.shape == (B, T, W)
    v64 = _var64(S)
    assert np.allclose(var.double().numpy(), v64, rtol=2e-5, atol=1e-9)
    k = _check_k(k_rows, S, k_base, k_min, k_max, W)
    for kv in np.unique(k):
        rows = np.argwhere(k == kv)
        Sr = S[rows[:, 0], rows[:, 1]].unsqueeze(0)          # [1, n, Tkv]
        if order == 0:
            oi, oc = orc.select_ascending(Sr, int(kv))
            assert torch.equal(idx[rows[:, 0], rows[:, 1], :kv], oi[0]), f"k={kv}"
            assert torch.equal(cnt[rows[:, 0], rows[:, 1]], oc[0])
        else:
            oi, om = orc.select_topk(Sr, int(kv))
            assert torch.equal(idx[rows[:, 0], rows[:, 1], :kv].long(), oi[0]), f"k={kv}"
            assert torch.equal(mask[rows[:, 0], rows[:, 1], :kv].bool(), om[0])
        assert torch.all(idx[rows[:, 0], rows[:, 1], kv:] == 0)
        assert torch.all(mask[rows[:, 0], rows[:, 1], kv:] == 0)


def _indexer_inputs(B, T, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    sig = 0.5 + 1.5 * torch.rand(B, 1, 1, generator=g)          # per-sequence scale, as in the c4 workload
    buf = (torch.randn(B, T, 328, generator=g) * sig).to(dtype)
    bias = torch.randn(4, generator=g) * 0.5
    return buf, bias


def _bits_sets(bits):
    w = bits.cpu().numpy().view(np.uint32)
    B, T, W = w.shape
    un = np.unpackbits(w.view(np.uint8).reshape(B, T, W * 4), axis=-1, bitorder="little")
    return un


@pytest.mark.parametrize("forced", [False, True])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("B,T,k_base,k_min,k_max", [(2, 600, 64, 16, 160), (1, 2100, 256, 64, 700),
                                                    (4, 129, 32, 8, 64), (1, 4100, 1024, 256, 2048)])
def test_indexer_select_adaptive_vs_oracle(dev, dtype, B, T, k_base, k_min, k_max, forced):
    """forced: every row with more keys than its k_t takes the fused selector's exact
    fallback path instead of the sampled band."""
    _log(f"indexer_select_adaptive dtype={dtype} B={B} T={T} k=({k_base},{k_min},{k_max}) forced={forced}")
    buf, bias = _indexer_inputs(B, T, dtype, seed=B * 7 + T)
    bd = buf.to(dev)
    qd = bd[..., :256].view(B, T, 4, 64)
    kd, wd, bias_d = bd[..., 256:320], bd[..., 320:324], bias.to(dev)
    prev = _abi.load().gsa_debug_force_select_fallback(int(forced))
    try:
        bits, idx, cnt, k_rows, var = _abi.indexer_select_adaptive(qd, kd, wd, bias_d, 0.125, k_base, k_min,
                                                                   k_max)
    finally:
        _abi.load().gsa_debug_force_select_fallback(prev)
    # the fused kernel's scores are bit-identical to the score kernel's
    S = _abi.indexer_scores(qd, kd, wd, bias_d, 0.125).cpu()
    k_rows, var, idx, cnt = k_rows.cpu(), var.cpu(), idx.cpu(), cnt.cpu()
    v64 = _var64(S)
    rel = np.abs(var.double().numpy() - v64) / np.maximum(v64, 1e-12)
    _log(f"  var max rel err {rel.max():.2e}")
    assert np.all((rel <= 1e-4) | (np.abs(var.double().numpy() - v64) <= 1e-9))
    W = min(k_max, T)
    k = _check_k(k_rows, S, k_base, k_min, k_max, W)
    un = _bits_sets(bits)
    t_all = np.arange(T)
    assert torch.equal(cnt, torch.from_numpy(np.minimum(k, t_all[None] + 1)).int())
    for kv in np.unique(k):
        rows = np.argwhere(k == kv)
        Sr = S[rows[:, 0], rows[:, 1]].unsqueeze(0)
        oi, oc = orc.select_ascending(Sr, int(kv))
        assert torch.equal(idx[rows[:, 0], rows[:, 1], :kv], oi[0]), f"k={kv}"
        exp = np.zeros((len(rows), un.shape[-1]), dtype=np.uint8)
        for r, (n, sel) in enumerate(zip(oc[0].tolist(), oi[0].tolist())):
            exp[r, sel[:n]] = 1
        assert np.array_equal(un[rows[:, 0], rows[:, 1]], exp), f"bitmask k={kv}"


def test_indexer_select_adaptive_long_rows(dev):
    """Variance-based k at T=27000: rows past key 26624 (more than 832 causal mask
    words) take two LDS bitmap chunks in the resolve.  On sampled rows, each row's
    variance against float64 and its selection against the oracle's selector at the
    kernel's own k_t, indices and bitmask bit for bit (k_t itself is checked against
    the oracle's formula at smaller T)."""
    B, T, k_base, k_min, k_max = 1, 27000, 2048, 256, 4096
    _log(f"indexer_select_adaptive long rows B={B} T={T}")
    buf, bias = _indexer_inputs(B, T, torch.bfloat16, seed=270)
    bd = buf.to(dev)
    qd = bd[..., :256].view(B, T, 4, 64)
    kd, wd, bias_d = bd[..., 256:320], bd[..., 320:324], bias.to(dev)
    bits, idx, cnt, k_rows, var = _abi.indexer_select_adaptive(qd, kd, wd, bias_d, 0.125, k_base, k_min, k_max)
    rows = [0, 1, 2047, 4096, 13000] + list(range(26600, 26640)) + list(range(T - 48, T))
    rsel = torch.tensor(rows, device=dev)
    S = _abi.indexer_scores(qd, kd, wd, bias_d, 0.125)[0].index_select(0, rsel).cpu()
    k_rows, var, idx, cnt = k_rows[0].cpu(), var[0].cpu(), idx[0].cpu(), cnt[0].cpu()
    v64 = _var64(S)
    vr = var[rows].double().numpy()
    rel = np.abs(vr - v64) / np.maximum(v64, 1e-12)
    assert np.all((rel <= 1e-4) | (np.abs(vr - v64) <= 1e-9)), f"var max rel err {rel.max():.2e}"
    un = _bits_sets(bits[:, rows])[0]
    for r, t in enumerate(rows):
        kt = int(k_rows[t])
        oi, oc = orc.select_ascending(S[r].view(1, 1, T), kt)
        n = int(oc[0, 0])
        assert int(cnt[t]) == n and torch.equal(idx[t, :n], oi[0, 0, :n]), f"row {t} k={kt}"
        exp = np.zeros(un.shape[-1], dtype=np.uint8)
        exp[oi[0, 0, :n].numpy()] = 1
        assert np.array_equal(un[r], exp), f"bitmask row {t}"
    _log(f"  k_t on the sampled rows {int(k_rows[rows].min())}..{int(k_rows[rows].max())}")


def test_indexer_select_adaptive_degenerate_scores(dev):
    """Every score equal (q = 0): every variance is 0, so k_t = k_base (clamped)
    everywhere and ties resolve to the lowest indices (the overflow path)."""
    B, T = 1, 900
    q = torch.zeros(B, T, 4, 64, dtype=torch.bfloat16, device=dev)
    k = torch.randn(B, T, 64, device=dev).to(torch.bfloat16)
    w = torch.zeros(B, T, 4, dtype=torch.bfloat16, device=dev)
    bits, idx, cnt, k_rows, var = _abi.indexer_select_adaptive(q, k, w, torch.zeros(4, device=dev), 0.125,
                                                               300, 50, 600)
    assert torch.all(var.cpu().abs() <= 1e-9)
    assert torch.all(k_rows.cpu() == 300)
    t = torch.arange(T)
    assert torch.equal(cnt.cpu()[0], torch.minimum(t + 1, torch.tensor(300)).int())
    for r in (0, 299, 300, 301, 899):
        n = min(r + 1, 300)
        assert idx.cpu()[0, r, :n].tolist() == list(range(n))


@pytest.mark.parametrize("impl", ["dense", "gather"])
def test_layer_variance_mode_vs_oracle(dev, impl):
    """The layer in variance mode against the oracle fed the layer's own k_t; the
    k_t themselves against the oracle's adaptive_k on the layer's scores."""
    _log(f"layer variance mode impl={impl}")
    cfg = orc.GSAConfig(hidden_size=512, num_heads=4, k_max=160, k_base=64, k_min=16)
    dt = torch.bfloat16
    sd = orc.cast_state(orc.synthetic_state(cfg, seed=11), dt)
    B, T = 2, 384
    sigma = torch.tensor([0.6, 1.8])
    x = orc.synthetic_input(B, T, cfg.hidden_size, seed=12, sigma=sigma).to(dt)
    m = GatedSparseAttention(cfg.hidden_size, cfg.num_heads, k_max=cfg.k_max, d_indexer=cfg.d_indexer,
                             n_idx_heads=cfg.n_idx_heads, k_base=cfg.k_base, k_min=cfg.k_min)
    m.attn_impl = impl
    m.topk_selector.mode = "variance"
    m = m.to(dev).to(dt).eval()
    m.load_state_dict({k: v.to(dev) for k, v in sd.items()}, strict=True)
    m.fuse_projections()
    xd = x.to(dev)
    with torch.no_grad():
        y = m(xd).cpu()
        k_rows = m.topk_selector.last_k.cpu()
        views = m.project(xd)
        S = _abi.indexer_scores(views["iq"], views["ik"], views["iw"], m._idx_bias32, m.indexer.scale).cpu()
    k = _check_k(k_rows, S, cfg.k_base, cfg.k_min, cfg.k_max, min(cfg.k_max, T))
    assert len(np.unique(k)) > 4          # the per-sequence scale spreads k
    # oracle rows with the layer's k_t: top-k_cap by (score desc, index asc), first k_t kept
    p = orc.project(sd, cfg, x)
    scores = orc.indexer_scores(p.q_idx, p.k_idx, p.w_idx, sd["indexer.idx_bias"], 0.125)
    W = min(cfg.k_max, T)
    oi, om = orc.select_topk(scores, W)
    om = om & (torch.arange(W)[None, None, :] < k_rows[..., None].long())
    ref = orc.attend_rows(sd, cfg, p, 0, T, idx=oi, mask=om).float()
    err = (y.float() - ref).abs()
    rel = (torch.linalg.vector_norm(y.float() - ref) / torch.linalg.vector_norm(ref)).item()
    _log(f"  bf16 rel-L2 {rel:.3e} max|err| {err.max().item():.3e}")
    assert torch.all(err <= 2e-2 + 1e-2 * ref.abs())
    assert rel < 2e-2


def test_indexer_select_adaptive_indices_stay_in_range(dev):
    """Past its count, row t holds t+1, t+2, ... up to entry k_t - 1 (rows with
    t+1 < k_t), then index 0 up to the output width: every entry lies in [0, T)."""
    B, T = 1, 700
    g = torch.Generator().manual_seed(21)
    buf = torch.randn(B, T, 324, generator=g).to(torch.bfloat16)
    sig = torch.linspace(0.2, 3.0, T).view(1, T, 1)
    q = (buf[..., :256].float() * sig).to(torch.bfloat16).view(B, T, 4, 64)
    k, w = buf[..., 256:320], buf[..., 320:324]
    _, idx, cnt, k_rows, _ = _abi.indexer_select_adaptive(q.to(dev), k.to(dev), w.to(dev),
                                                          torch.zeros(4, device=dev), 0.125, 64, 16, 400)
    idx, cnt, k_rows = idx.cpu(), cnt.cpu(), k_rows.cpu()
    assert idx.shape[-1] == 400
    assert int(idx.min()) >= 0 and int(idx.max()) < T
    t = torch.arange(T)
    assert torch.equal(cnt[0].long(), torch.minimum(t + 1, k_rows[0].long()))
    short = (cnt[0] < 400).nonzero().flatten()
    assert short.numel() > 0 and bool((k_rows[0, short] < torch.minimum(t[short] + 1, torch.tensor(400))).any())
    for r in short.tolist():
        n, kr = int(cnt[0, r]), int(k_rows[0, r])
        assert idx[0, r, n:kr].tolist() == list(range(r + 1, r + 1 + max(0, kr - n)))
        assert torch.all(idx[0, r, max(n, kr):] == 0)
