"""Pin the oracle's layer wiring with an independent float64 brute force (CPU only).

``gsa_forward`` and ``attend_rows`` join the oracle's pieces into the layer of
gsa_ref.py:276-325: which projection feeds which operand, RoPE on q *and* k,
the indexer scale 1/sqrt(d_indexer) (gsa_ref.py:86) with both indexer biases,
the selection at k < T, both gates and o_proj.  The brute force below writes
every one of those steps out again from the mathematics, per row and per key,
in float64 numpy:

  * projections as float64 matrix products (biases on the two gates and on
    idx_w only);
  * RoPE as an explicit rotation of the pairs (i, i+64) of each head by the
    angle t * 10000^(-2i/128);
  * the indexer per (t, j <= t, h): sigmoid(w_h) * sigmoid(<q_h, k_j>/8 + b_h);
  * the selection as Python's ``sorted`` by (-score, index), first k;
  * a softmax per (t, head) over the selected keys, the output gate, o_proj.

Every bias is drawn non-zero so that a dropped term shows.  Planted mistakes
(RoPE left off q, the indexer scaled by 1/sqrt(d_head), the idx_w bias
dropped, the value gate dropped) are shown to fail the same comparison.
"""

import math

import numpy as np
import pytest
import torch

from oracle import gsa_oracle as orc

CFG = orc.GSAConfig(hidden_size=256, num_heads=2, k_max=64, k_base=5, k_min=2)   # k_eff = 5 < T
B, T = 2, 24


def _state():
    sd = orc.synthetic_state(CFG, seed=11)
    g = torch.Generator().manual_seed(12)
    # non-zero biases everywhere the layer has one
    sd["indexer.idx_bias"] = torch.tensor([0.3, -0.2, 0.5, -0.4])
    sd["indexer.idx_w_proj.bias"] = torch.randn(CFG.n_idx_heads, generator=g)
    sd["value_gate.gate_proj.bias"] = torch.randn(CFG.hidden_size, generator=g)
    sd["output_gate.gate_proj.bias"] = torch.randn(CFG.hidden_size, generator=g)
    # larger indexer weights: scores spread over the sigmoid's curved range
    sd["indexer.idx_q_proj.weight"] = sd["indexer.idx_q_proj.weight"] * 8
    sd["indexer.idx_k_proj.weight"] = sd["indexer.idx_k_proj.weight"] * 8
    sd["indexer.idx_w_proj.weight"] = sd["indexer.idx_w_proj.weight"] * 20
    return sd


def _sig(z):
    return 1.0 / (1.0 + np.exp(-z))


def _rotate(vec, t, d):
    """Rotate the pairs (i, i + d/2) of ``vec`` by t * 10000^(-2i/d)."""
    out = np.empty(d)
    h = d // 2
    for i in range(h):
        th = t * 10000.0 ** (-2.0 * i / d)
        c, s = math.cos(th), math.sin(th)
        out[i] = vec[i] * c - vec[i + h] * s
        out[i + h] = vec[i + h] * c + vec[i] * s
    return out


def brute_layer(sd, cfg, x, k):
    """float64 layer forward, row by row: (y [B,T,D], scores [B,T,T], selections)."""
    W = {n: v.double().numpy() for n, v in sd.items()}
    X = x.double().numpy()
    Bn, Tn, D = X.shape
    H, d, Hi, di = cfg.num_heads, cfg.d_head, cfg.n_idx_heads, cfg.d_indexer
    y = np.zeros((Bn, Tn, D))
    scores = np.full((Bn, Tn, Tn), -np.inf)
    sels = []
    for b in range(Bn):
        xb = X[b]
        q = xb @ W["q_proj.weight"].T
        kk = xb @ W["k_proj.weight"].T
        v = (xb @ W["v_proj.weight"].T) * _sig(xb @ W["value_gate.gate_proj.weight"].T
                                                 + W["value_gate.gate_proj.bias"])
        og = _sig(xb @ W["output_gate.gate_proj.weight"].T + W["output_gate.gate_proj.bias"])
        iq = xb @ W["indexer.idx_q_proj.weight"].T
        ik = xb @ W["indexer.idx_k_proj.weight"].T
        iw = xb @ W["indexer.idx_w_proj.weight"].T + W["indexer.idx_w_proj.bias"]
        ib = W["indexer.idx_bias"]
        qr = np.stack([np.concatenate([_rotate(q[t, h * d:(h + 1) * d], t, d) for h in range(H)])
                       for t in range(Tn)])
        kr = np.stack([np.concatenate([_rotate(kk[t, h * d:(h + 1) * d], t, d) for h in range(H)])
                       for t in range(Tn)])
        attn = np.zeros((Tn, D))
        bsel = []
        for t in range(Tn):
            for j in range(t + 1):
                scores[b, t, j] = sum(_sig(iw[t, h]) * _sig(iq[t, h * di:(h + 1) * di] @ ik[j] / 8.0 + ib[h])
                                      for h in range(Hi))
            sel = sorted(range(t + 1), key=lambda j: (-scores[b, t, j], j))[:k]
            bsel.append(sorted(sel))
            for h in range(H):
                sl = slice(h * d, (h + 1) * d)
                logit = np.array([qr[t, sl] @ kr[j, sl] / math.sqrt(d) for j in sel])
                p = np.exp(logit - logit.max())
                p /= p.sum()
                o = sum(p[i] * v[j, sl] for i, j in enumerate(sel))
                attn[t, sl] = o * og[t, sl]
        y[b] = attn @ W["o_proj.weight"].T
        sels.append(bsel)
    return y, scores, sels


@pytest.fixture(scope="module")
def case():
    sd = _state()
    x = orc.synthetic_input(B, T, CFG.hidden_size, seed=13)
    y, s, sel = brute_layer(sd, CFG, x, orc.k_effective(CFG.k_base, CFG.k_max, T))
    return sd, x, y, s, sel


def _mismatch(sd, x, y_ref, s_ref, sel_ref):
    """Largest deviations of the oracle's forward and its chunked rows from the brute force."""
    y, aux = orc.gsa_forward(sd, CFG, x, return_aux=True)
    s = aux["scores"].double().numpy()
    fin = np.isfinite(s_ref)
    err = {
        "scores": float(np.abs(s[fin] - s_ref[fin]).max()),
        "mask": bool(np.array_equal(np.isfinite(s), fin)),
        "y": float(np.abs(y.double().numpy() - y_ref).max() / np.abs(y_ref).max()),
    }
    idx = aux["idx"]
    mask = aux["mask"]
    err["sel"] = all(sorted(idx[b, t][mask[b, t]].tolist()) == sel_ref[b][t] for b in range(B) for t in range(T))
    # query-chunked rows (the form the GPU parity tests use at scale)
    p = orc.project(sd, CFG, x)
    yc = orc.attend_rows(sd, CFG, p, 7, 19)
    err["rows"] = float(np.abs(yc.double().numpy() - y_ref[:, 7:19]).max() / np.abs(y_ref).max())
    return err


def _ok(err):
    # scores lie in (0, 4): 1e-5 is a few fp32 ulps of the dot products' rounding
    return err["scores"] < 1e-5 and err["mask"] and err["sel"] and err["y"] < 1e-5 and err["rows"] < 1e-5


def test_case_is_discriminating(case):
    """The selection really is partial (k < T) and its boundary is not a near-tie."""
    _, _, _, s, sel = case
    assert orc.k_effective(CFG.k_base, CFG.k_max, T) == 5 < T
    gaps = []
    for b in range(B):
        for t in range(5, T):
            row = np.sort(s[b, t, :t + 1])[::-1]
            gaps.append(row[4] - row[5])
    assert min(gaps) > 5e-6        # >> the ~2e-7 fp32 error of a score
    # the scores use the sigmoid's curved range (a linear stand-in would not do)
    fin = s[np.isfinite(s)]
    assert fin.max() - fin.min() > 0.5


def test_layer_matches_float64_brute_force(case):
    sd, x, y, s, sel = case
    err = _mismatch(sd, x, y, s, sel)
    assert _ok(err), err


def _planted_q_without_rope(monkeypatch):
    """project() applies RoPE to q first, then k: leave the q call's input unchanged."""
    real = orc.apply_rope
    calls = [0]

    def apply_rope(x, cos, sin):
        calls[0] += 1
        return x if calls[0] % 2 == 1 else real(x, cos, sin)

    monkeypatch.setattr(orc, "apply_rope", apply_rope)


def _planted_indexer_scale(monkeypatch):
    """Indexer scaled by 1/sqrt(d_head) instead of 1/sqrt(d_indexer)."""
    real = orc.indexer_scores

    def indexer_scores(q, k, w, bias, scale, *a, **kw):
        return real(q, k, w, bias, 1.0 / math.sqrt(CFG.d_head), *a, **kw)

    monkeypatch.setattr(orc, "indexer_scores", indexer_scores)


def _planted_idx_w_bias_dropped(monkeypatch):
    real = orc.project

    def project(sd, cfg, x, rope=None):
        sd2 = dict(sd)
        sd2["indexer.idx_w_proj.bias"] = torch.zeros_like(sd["indexer.idx_w_proj.bias"])
        return real(sd2, cfg, x, rope)

    monkeypatch.setattr(orc, "project", project)


def _planted_value_gate_dropped(monkeypatch):
    real = torch.sigmoid
    calls = [0]

    def sigmoid(t, *a, **kw):   # the value gate is project()'s first sigmoid
        calls[0] += 1
        out = real(t, *a, **kw)
        return torch.ones_like(out) if calls[0] == 1 else out

    monkeypatch.setattr(orc.torch, "sigmoid", sigmoid)


@pytest.mark.parametrize("plant", [_planted_q_without_rope, _planted_indexer_scale,
                                   _planted_idx_w_bias_dropped, _planted_value_gate_dropped])
def test_planted_wiring_mistakes_fail(case, monkeypatch, plant):
    sd, x, y, s, sel = case
    plant(monkeypatch)
    err = _mismatch(sd, x, y, s, sel)
    assert not _ok(err), f"{plant.__name__} went unnoticed: {err}"


def test_partial_projection_equals_full_rows():
    """project(x[:, r0:r1], pos0=r0, seq_len=T) is the full projection's rows, also
    past the 8192-entry RoPE cache (the call over T rows rebuilds the tables from
    the bf16 inv_freq, and the slice must read those), and attend_rows with the
    query rows given separately equals attend_rows on the full projection."""
    cfg = orc.GSAConfig(hidden_size=256, num_heads=2, k_max=64, k_base=16, k_min=4)
    sd = orc.cast_state(orc.synthetic_state(cfg, seed=21), torch.bfloat16)
    Tn = 8200
    x = orc.synthetic_input(1, Tn, cfg.hidden_size, seed=22).to(torch.bfloat16)
    full = orc.project(sd, cfg, x)
    keys = orc.project(sd, cfg, x, parts=("k", "v", "k_idx"))
    assert keys.q is None and keys.og is None
    for r0, r1 in ((0, 40), (8150, 8200)):
        part = orc.project(sd, cfg, x[:, r0:r1], pos0=r0, seq_len=Tn, parts=("q", "og", "q_idx", "w_idx"))
        for name in ("q", "og", "q_idx", "w_idx"):
            assert torch.equal(getattr(part, name), getattr(full, name)[:, r0:r1]), name
        a = orc.attend_rows(sd, cfg, full, r0, r1)
        b = orc.attend_rows(sd, cfg, keys, r0, r1, rows=part)
        assert torch.equal(a, b)
    # the slice really reads the rebuilt tables: a call over r1 rows only (no rebuild) differs
    short = orc.project(sd, cfg, x[:, 8150:8190], pos0=8150, seq_len=8190, parts=("q",))
    assert not torch.equal(short.q, full.q[:, 8150:8190])
    with pytest.raises(ValueError):
        orc.project(sd, cfg, x[:, :10], pos0=Tn - 5, seq_len=Tn)
