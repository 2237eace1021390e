"""Pin the CPU oracle against independent formulations (CPU only).

Every oracle function is checked against something that does not restate its
own formula: float64 brute-force loops, a closed form, a library routine
(scaled_dot_product_attention, Python's sorted), or an invariant.  Planted
mistakes (a sign flip, a transposed operand, a dropped term) are shown to
fail the same checks.
"""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import gsa_oracle as orc


def _sig(x):
    return 1.0 / (1.0 + math.exp(-x))


# ---------------------------------------------------------------------------
# RoPE
# ---------------------------------------------------------------------------

def _rope_closed_form(x, cos, sin):
    """float64 rotation of pairs (i, i+d/2) by the table angles."""
    x = x.double()
    c, s = cos.double(), sin.double()
    h = x.shape[-1] // 2
    out = torch.empty_like(x)
    out[..., :h] = x[..., :h] * c[..., :h] - x[..., h:] * s[..., :h]
    out[..., h:] = x[..., h:] * c[..., h:] + x[..., :h] * s[..., h:]
    return out


def test_rope_tables_are_the_angles():
    rc = orc.RopeCache(128, torch.float32)
    cos, sin = rc.tables(300, torch.float32)
    inv = 1.0 / (10000.0 ** (np.arange(0, 128, 2) / 128.0))
    t = np.arange(300)[:, None]
    ang = t * inv[None, :]
    ang = np.concatenate([ang, ang], axis=1)
    assert np.abs(cos.numpy() - np.cos(ang)).max() < 2e-4
    assert np.abs(sin.numpy() - np.sin(ang)).max() < 2e-4
    # position 0 is the identity
    assert torch.all(cos[0] == 1) and torch.all(sin[0] == 0)


def test_rope_is_a_pairwise_rotation():
    g = torch.Generator().manual_seed(3)
    x = torch.randn(2, 50, 3, 128, generator=g)
    rc = orc.RopeCache(128, torch.float32)
    cos, sin = rc.tables(50, torch.float32)
    c4, s4 = cos[None, :, None, :], sin[None, :, None, :]
    y = orc.apply_rope(x, c4, s4)
    assert torch.allclose(y.double(), _rope_closed_form(x, c4, s4), atol=1e-5)
    assert torch.equal(y[:, 0], x[:, 0])
    # norm of each (i, i+64) pair is preserved
    n0 = x[..., :64] ** 2 + x[..., 64:] ** 2
    n1 = y[..., :64] ** 2 + y[..., 64:] ** 2
    assert torch.allclose(n0, n1, rtol=1e-4, atol=1e-5)


def test_rope_planted_sign_flip_is_caught(monkeypatch):
    g = torch.Generator().manual_seed(4)
    x = torch.randn(1, 20, 2, 128, generator=g)
    rc = orc.RopeCache(128, torch.float32)
    cos, sin = rc.tables(20, torch.float32)
    c4, s4 = cos[None, :, None, :], sin[None, :, None, :]
    monkeypatch.setattr(orc, "rotate_half",
                        lambda t: torch.cat((t[..., 64:], -t[..., :64]), dim=-1))
    y = orc.apply_rope(x, c4, s4)
    assert not torch.allclose(y.double(), _rope_closed_form(x, c4, s4), atol=1e-3)


def test_rope_bf16_rebuild_quirk():
    """T > 8192 rebuilds from the bf16-cast inv_freq; shorter requests then reuse it."""
    rc = orc.RopeCache(128, torch.bfloat16)
    short_before = rc.tables(100, torch.bfloat16)[0].clone()
    inv_true = 1.0 / (10000.0 ** (np.arange(0, 128, 2) / 128.0))
    t = np.arange(100)[:, None]
    ref_true = np.cos(np.concatenate([t * inv_true, t * inv_true], axis=1))
    # construction cache: bf16 of the true angles (within one bf16 ulp)
    assert np.abs(short_before.float().numpy() - ref_true).max() <= 2 ** -8 + 1e-6

    cos, _ = rc.tables(8193, torch.bfloat16)
    inv_b = torch.tensor(inv_true, dtype=torch.float32).to(torch.bfloat16).double().numpy()
    tt = np.arange(8193)[:, None]
    ref_q = np.cos(np.concatenate([tt * inv_b, tt * inv_b], axis=1))
    # fp32 angles t*inv are exact to ~t*2^-24; compare within that plus one bf16 ulp
    bound = 2 ** -8 + 8193 * 2.0 ** -23
    assert np.abs(cos.float().numpy() - ref_q).max() <= bound
    # the quirk is visible: far from the true angles at large t
    ref_tt = np.cos(np.concatenate([tt * inv_true, tt * inv_true], axis=1))
    assert np.abs(cos.float().numpy()[8000:] - ref_tt[8000:]).max() > 0.5
    # the rebuilt cache persists for a later, shorter request
    short_after = rc.tables(100, torch.bfloat16)[0]
    assert not torch.equal(short_before, short_after)


# ---------------------------------------------------------------------------
# Indexer
# ---------------------------------------------------------------------------

def _indexer_brute(q, k, w, bias, scale):
    B, T, Hi, di = q.shape
    out = np.full((B, T, T), -np.inf)
    qd, kd, wd, bd = q.double().numpy(), k.double().numpy(), w.double().numpy(), bias.double().numpy()
    for b in range(B):
        for i in range(T):
            for j in range(i + 1):
                s = 0.0
                for h in range(Hi):
                    dot = float(np.dot(qd[b, i, h], kd[b, j]))
                    s += _sig(wd[b, i, h]) * _sig(dot * scale + bd[h])
                out[b, i, j] = s
    return out


def _indexer_inputs(seed=5, B=2, T=7):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, T, 4, 64, generator=g)
    k = torch.randn(B, T, 64, generator=g)
    w = torch.randn(B, T, 4, generator=g)
    bias = torch.randn(4, generator=g)
    return q, k, w, bias


def test_indexer_matches_float64_brute_force():
    q, k, w, bias = _indexer_inputs()
    s = orc.indexer_scores(q, k, w, bias, 0.125)
    ref = _indexer_brute(q, k, w, bias, 0.125)
    fin = np.isfinite(ref)
    assert np.array_equal(np.isfinite(s.numpy()), fin)
    assert np.allclose(s.numpy()[fin], ref[fin], rtol=2e-6, atol=1e-7)
    # -inf exactly above the diagonal
    T = q.shape[1]
    assert np.array_equal(fin[0], np.tril(np.ones((T, T), dtype=bool)))


def test_indexer_planted_transpose_is_caught(monkeypatch):
    q, k, w, bias = _indexer_inputs(seed=6)
    ref = _indexer_brute(q, k, w, bias, 0.125)
    real = torch.einsum

    def swapped(eq, *ops):
        if eq == "bqhd,bkd->bhqk":
            return real("bqhd,bkd->bhkq", *ops)
        return real(eq, *ops)

    monkeypatch.setattr(torch, "einsum", swapped)
    s = orc.indexer_scores(q, k, w, bias, 0.125)
    fin = np.isfinite(ref)
    assert not np.allclose(s.numpy()[fin], ref[fin], rtol=1e-3)


def test_indexer_special_case_zero_queries():
    _, k, w, _ = _indexer_inputs(seed=7, B=1, T=9)
    q = torch.zeros(1, 9, 4, 64)
    s = orc.indexer_scores(q, k, w, torch.zeros(4), 0.125)
    expect = 0.5 * torch.sigmoid(w).sum(-1)          # [1, T]
    for i in range(9):
        assert torch.allclose(s[0, i, : i + 1], expect[0, i].expand(i + 1), rtol=1e-6)


def test_indexer_q_offset_matches_unchunked():
    q, k, w, bias = _indexer_inputs(seed=8, B=1, T=40)
    full = orc.indexer_scores(q, k, w, bias, 0.125)
    part = orc.indexer_scores(q[:, 16:29], k, w[:, 16:29], bias, 0.125, q_offset=16)
    assert torch.equal(torch.isfinite(part), torch.isfinite(full[:, 16:29]))
    fin = torch.isfinite(part)
    assert torch.allclose(part[fin], full[:, 16:29][fin], rtol=1e-6)


# ---------------------------------------------------------------------------
# Selector
# ---------------------------------------------------------------------------

def _tie_scores(seed, B, T, levels=5):
    g = torch.Generator().manual_seed(seed)
    s = torch.randint(0, levels, (B, T, T), generator=g).float() / levels
    causal = torch.triu(torch.ones(T, T, dtype=torch.bool), diagonal=1)
    return s.masked_fill(causal, float("-inf"))


def _select_brute(row, k):
    vals = [(-1e9 if v == float("-inf") else v) for v in row]
    order = sorted(range(len(vals)), key=lambda j: (-vals[j], j))
    return order[:k]


@pytest.mark.parametrize("k", [1, 3, 8, 20])
def test_select_matches_brute_force_with_ties(k):
    s = _tie_scores(11, 2, 20)
    idx, mask = orc.select_topk(s, k)
    for b in range(2):
        for t in range(20):
            row = s[b, t].tolist()
            assert idx[b, t].tolist() == _select_brute(row, k)
            assert mask[b, t].tolist() == [row[j] != float("-inf") for j in idx[b, t].tolist()]


def test_select_value_multiset_equals_torch_topk():
    s = _tie_scores(12, 1, 64, levels=7)
    filled = s.masked_fill(s == float("-inf"), -1e9)
    idx, _ = orc.select_topk(s, 16)
    ours = torch.gather(filled, -1, idx).sort(dim=-1).values
    theirs = torch.topk(filled, 16, dim=-1).values.sort(dim=-1).values
    assert torch.equal(ours, theirs)


def test_select_invariants():
    g = torch.Generator().manual_seed(13)
    T, k = 50, 12
    s = torch.rand(1, T, T, generator=g)
    s = s.masked_fill(torch.triu(torch.ones(T, T, dtype=torch.bool), 1), float("-inf"))
    idx, cnt = orc.select_ascending(s, k)
    for t in range(T):
        n = int(cnt[0, t])
        assert n == min(t + 1, k)
        sel = idx[0, t, :n].tolist()
        assert sel == sorted(sel) and all(j <= t for j in sel)
        if t < k:
            assert sel == list(range(t + 1))
            assert idx[0, t, n:].tolist() == list(range(t + 1, k))
        rest = [j for j in range(t + 1) if j not in sel]
        if rest:
            assert max(s[0, t, rest]) <= min(s[0, t, sel])


def test_adaptive_k_formula():
    s = torch.tensor([[[0.5, float("-inf"), float("-inf")],
                       [0.1, 0.9, float("-inf")],
                       [0.2, 0.4, 0.9]]])
    k = orc.adaptive_k(s, k_base=4, k_min=2, k_max=6)
    var = np.array([0.0, np.var([0.1, 0.9]), np.var([0.2, 0.4, 0.9])])
    avg = max(var.mean(), 1e-6)
    exp = np.clip(np.floor(4 * avg / np.maximum(var, 1e-6)), 2, 6)
    assert k[0].tolist() == exp.astype(int).tolist()


def _adaptive_k_numpy(s, k_base, k_min, k_max, per_sequence_mean=False):
    """The notebook rule (gsa_explained.ipynb:577-592) evaluated row by row in
    float64: population variance of each row's finite scores, the mean of those
    variances over every (batch, row) -- or, for the planted mutant, over each
    sequence's rows only -- and k = clip(floor(k_base * avg / var), k_min, k_max)
    with both variances floored at 1e-6."""
    a = s.numpy().astype(np.float64)
    B, T, _ = a.shape
    var = np.zeros((B, T))
    for b in range(B):
        for t in range(T):
            row = a[b, t][np.isfinite(a[b, t])]
            var[b, t] = np.var(row) if row.size else 0.0
    avg = var.mean(axis=1, keepdims=True) if per_sequence_mean else np.full((B, 1), var.mean())
    avg = np.maximum(avg, 1e-6)
    return np.clip(np.floor(k_base * avg / np.maximum(var, 1e-6)), k_min, k_max).astype(np.int64)


def test_adaptive_k_mean_over_all_sequences():
    """B=2 sequences whose scores spread differently (uniform on [0,1) and on
    [0,3)): the oracle's k equals the float64 row-by-row evaluation with the
    variance mean taken over all B*T rows, and a per-sequence mean -- a
    plausible misreading of the notebook's variance.mean() -- gives other k
    on most rows, so the check tells the two apart."""
    T, k_base, k_min, k_max = 40, 16, 4, 64
    g = torch.Generator().manual_seed(77)
    s = torch.rand(2, T, T, generator=g, dtype=torch.float64)
    s[1] *= 3.0
    s = s.masked_fill(torch.triu(torch.ones(T, T, dtype=torch.bool), 1), float("-inf"))
    got = orc.adaptive_k(s, k_base, k_min, k_max).numpy()
    want = _adaptive_k_numpy(s, k_base, k_min, k_max)
    assert np.array_equal(got, want)
    mutant = _adaptive_k_numpy(s, k_base, k_min, k_max, per_sequence_mean=True)
    assert (mutant != want).mean() > 0.5
    # the variance itself against numpy, every row
    var = orc.row_variance(s).numpy()
    for b in range(2):
        for t in range(T):
            assert abs(var[b, t] - np.var(s[b, t, :t + 1].numpy())) <= 1e-12
    # the spread of sequence 1 is 9x that of sequence 0: its rows get smaller k
    assert want[1, 4:].mean() < want[0, 4:].mean()


# ---------------------------------------------------------------------------
# Sparse attention
# ---------------------------------------------------------------------------

def _attn_inputs(seed, B=2, T=24, H=3, d=128):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, T, H, d, generator=g)
    k = torch.randn(B, T, H, d, generator=g)
    v = torch.randn(B, T, H, d, generator=g)
    return q, k, v


def test_sparse_attention_equals_masked_sdpa():
    q, k, v = _attn_inputs(21)
    B, T, H, d = q.shape
    g = torch.Generator().manual_seed(22)
    s = torch.rand(B, T, T, generator=g).masked_fill(
        torch.triu(torch.ones(T, T, dtype=torch.bool), 1), float("-inf"))
    idx, mask = orc.select_topk(s, 6)
    out = orc.sparse_attention(q, k, v, idx, mask, d ** -0.5)
    dense = torch.zeros(B, T, T, dtype=torch.bool)
    for b in range(B):
        for t in range(T):
            for j, m in zip(idx[b, t].tolist(), mask[b, t].tolist()):
                if m:
                    dense[b, t, j] = True
    ref = F.scaled_dot_product_attention(q.transpose(1, 2).double(), k.transpose(1, 2).double(),
                                         v.transpose(1, 2).double(), attn_mask=dense[:, None])
    assert torch.allclose(out.double(), ref.transpose(1, 2), atol=1e-5)


def test_sparse_attention_full_selection_is_causal_sdpa():
    q, k, v = _attn_inputs(23, B=1, T=16, H=2)
    T, d = 16, 128
    s = torch.rand(1, T, T).masked_fill(torch.triu(torch.ones(T, T, dtype=torch.bool), 1), float("-inf"))
    idx, mask = orc.select_topk(s, T)
    out = orc.sparse_attention(q, k, v, idx, mask, d ** -0.5)
    ref = F.scaled_dot_product_attention(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2),
                                         is_causal=True)
    assert torch.allclose(out, ref.transpose(1, 2), atol=1e-5)


def test_sparse_attention_float64_brute_force_and_all_masked():
    q, k, v = _attn_inputs(24, B=1, T=5, H=2)
    idx = torch.tensor([[[0, 0, 0], [1, 0, 4], [2, 1, 0], [3, 3, 2], [4, 0, 1]]])
    mask = torch.tensor([[[False, False, False], [True, True, False], [True, True, True],
                          [True, False, True], [True, True, True]]])
    out = orc.sparse_attention(q, k, v, idx, mask, 0.1)
    assert torch.all(out[0, 0] == 0)
    qd, kd, vd = q.double(), k.double(), v.double()
    for t in range(1, 5):
        for h in range(2):
            js = [j for j, m in zip(idx[0, t].tolist(), mask[0, t].tolist()) if m]
            sc = torch.stack([0.1 * torch.dot(qd[0, t, h], kd[0, j, h]) for j in js])
            p = torch.softmax(sc, 0)
            ref = sum(p[i] * vd[0, j, h] for i, j in enumerate(js))
            assert torch.allclose(out[0, t, h].double(), ref, atol=1e-5)


# ---------------------------------------------------------------------------
# Gates and the whole layer
# ---------------------------------------------------------------------------

SMALL = orc.GSAConfig(hidden_size=256, num_heads=2, k_max=64, k_base=16, k_min=4)


def test_gates_closed_form():
    cfg = SMALL
    sd = orc.synthetic_state(cfg, seed=0)
    sd["value_gate.gate_proj.weight"].zero_()
    sd["output_gate.gate_proj.weight"].zero_()
    x = orc.synthetic_input(1, 8, cfg.hidden_size, seed=2)
    p = orc.project(sd, cfg, x)
    v_raw = F.linear(x, sd["v_proj.weight"]).view(1, 8, 2, 128)
    assert torch.allclose(p.v, v_raw * 0.6224593312018546, rtol=1e-6, atol=1e-7)
    assert torch.allclose(p.og, torch.full_like(p.og, 0.6224593312018546))


def test_layer_with_full_selection_is_gated_causal_sdpa():
    cfg = orc.GSAConfig(hidden_size=256, num_heads=2, k_max=4096, k_base=2048)
    sd = orc.synthetic_state(cfg, seed=1)
    x = orc.synthetic_input(1, 24, cfg.hidden_size, seed=3)
    y = orc.gsa_forward(sd, cfg, x)
    p = orc.project(sd, cfg, x)
    att = F.scaled_dot_product_attention(p.q.transpose(1, 2), p.k.transpose(1, 2), p.v.transpose(1, 2),
                                         is_causal=True).transpose(1, 2)
    ref = F.linear((att * p.og.view(1, 24, 2, 128)).reshape(1, 24, 256), sd["o_proj.weight"])
    assert torch.allclose(y, ref, atol=1e-6, rtol=1e-5)


def test_chunked_forward_matches_unchunked():
    cfg = SMALL
    sd = orc.synthetic_state(cfg, seed=2)
    x = orc.synthetic_input(2, 40, cfg.hidden_size, seed=4)
    a = orc.gsa_forward(sd, cfg, x)
    b = orc.gsa_forward_chunked(sd, cfg, x, chunk=13)
    assert torch.allclose(a, b, atol=1e-7, rtol=1e-6)


def test_state_keys_complete():
    sd = orc.synthetic_state(SMALL)
    assert tuple(sorted(sd)) == tuple(sorted(orc.STATE_KEYS))
