"""CPU restatement of the Gated Sparse Attention forward (the oracle).

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this module, and only to check
results against (or as the timed CPU baseline).  The product path
(``gsa_gdn_benchmarkstudy_amd``) never imports it and fails loudly when its HIP
library is missing.

The arithmetic of the reference path is PyTorch, so this restatement uses torch
CPU ops in the reference's own order and dtype: in bf16 every tensor op rounds
its output to bf16, exactly as ``gsa_ref.py`` does on the CPU, and the indexer
runs in fp32 (``gsa_ref.py:104-118``).  Each function cites the reference lines
it restates (paths relative to the reference repository root).

Pinning (see ``tests/test_oracle.py``): every function here is checked against
an independent formulation (float64 brute force, a closed form, a library
routine such as ``scaled_dot_product_attention``, or an invariant), so a dropped
term, a sign error or a transposed operand fails a test.  The reference ships no
golden vectors for this path.

Tie rule of the selector: ``torch.topk`` leaves the order of equal scores
implementation-defined.  The oracle's selector is the deterministic restatement
"sort by (score descending, index ascending), take the first k", which selects
the same value multiset as ``torch.topk`` and breaks ties at the k-th value by
lowest index.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Dict, Optional, Tuple

import torch
import torch.nn.functional as F

# The reference precomputes this many RoPE positions at construction
# (gsa_triton/gsa_ref.py:44, gsa_triton/gsa_opt.py:405).
ROPE_CACHE_LEN = 8192
ROPE_BASE = 10000.0

STATE_KEYS = (
    "q_proj.weight", "k_proj.weight", "v_proj.weight", "o_proj.weight",
    "indexer.idx_q_proj.weight", "indexer.idx_k_proj.weight",
    "indexer.idx_w_proj.weight", "indexer.idx_w_proj.bias", "indexer.idx_bias",
    "value_gate.gate_proj.weight", "value_gate.gate_proj.bias",
    "output_gate.gate_proj.weight", "output_gate.gate_proj.bias",
    "rotary_emb.inv_freq",
)


# ---------------------------------------------------------------------------
# RoPE  (gsa_triton/gsa_ref.py:27-70)
# ---------------------------------------------------------------------------

def rope_inv_freq(dim: int, base: float = ROPE_BASE) -> torch.Tensor:
    """inv_freq[i] = base^(-2i/dim) in fp32 (gsa_ref.py:47)."""
    return 1.0 / (base ** (torch.arange(0, dim, 2).float() / dim))


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    """cat(-x[..., d/2:], x[..., :d/2]) (gsa_ref.py:29-32)."""
    half = x.shape[-1] // 2
    return torch.cat((-x[..., half:], x[..., :half]), dim=-1)


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """x*cos + rotate_half(x)*sin, each op rounding in x's dtype (gsa_ref.py:35-40)."""
    return (x * cos) + (rotate_half(x) * sin)


class RopeCache:
    """Stateful cos/sin cache with the reference's rebuild semantics.

    gsa_ref.py:43-70: the cache is built at construction for 8192 positions
    from the fp32 ``inv_freq``; ``Module.to(dtype)`` then casts both the cache
    and ``inv_freq``.  A request longer than the cache rebuilds it from
    ``arange(seq_len)`` (fp32) times the *current* ``inv_freq`` -- bf16 when
    the module was cast -- keeps the rebuilt cache in fp32 and casts at use.
    The rebuilt cache is kept for later, shorter requests.  (On a GPU the
    reference's rebuild mixes a CPU ``arange`` with a device buffer and
    raises; this restatement keeps the arithmetic and drops the error.)
    """

    def __init__(self, dim: int, dtype: torch.dtype, inv_freq: Optional[torch.Tensor] = None,
                 max_seq_len: int = ROPE_CACHE_LEN):
        # The construction-time cache always comes from the freshly computed
        # fp32 inv_freq (gsa_ref.py:47-49); a loaded or cast ``inv_freq``
        # buffer only matters for a rebuild.
        inv32 = rope_inv_freq(dim)
        t = torch.arange(max_seq_len, dtype=torch.float32)
        emb = torch.outer(t, inv32)
        emb = torch.cat((emb, emb), dim=-1)
        # construction in fp32, then the module cast (nn.Module.to(dtype))
        self.cos_cached = emb.cos().to(dtype)
        self.sin_cached = emb.sin().to(dtype)
        buf = inv32 if inv_freq is None else inv_freq.detach().cpu()
        self.inv_freq = buf.to(dtype)

    def tables(self, seq_len: int, dtype: torch.dtype) -> Tuple[torch.Tensor, torch.Tensor]:
        if seq_len > self.cos_cached.shape[0]:
            t = torch.arange(seq_len, dtype=torch.float32)
            emb = torch.outer(t, self.inv_freq)        # fp32 x (bf16|fp32) -> fp32
            emb = torch.cat((emb, emb), dim=-1)
            self.cos_cached = emb.cos()
            self.sin_cached = emb.sin()
        return self.cos_cached[:seq_len].to(dtype), self.sin_cached[:seq_len].to(dtype)


# ---------------------------------------------------------------------------
# Indexer  (gsa_triton/gsa_ref.py:97-126; q_offset: benchmark_models.ipynb:66-121)
# ---------------------------------------------------------------------------

def indexer_scores(q_idx: torch.Tensor, k_idx: torch.Tensor, w: torch.Tensor,
                   bias: torch.Tensor, scale: float, q_offset: int = 0,
                   causal: bool = True) -> torch.Tensor:
    """S[b,i,j] = sum_h sigmoid(w[b,i,h]) * sigmoid(scale*<q[b,i,h], k[b,j]> + bias[h]).

    q_idx [B,Tq,Hi,di], k_idx [B,Tk,di], w [B,Tq,Hi]; computed in fp32 after
    upcasting the model-dtype inputs (gsa_ref.py:104-118).  Query row i sits at
    absolute position ``q_offset + i``; keys after it are -inf (gsa_ref.py:120-124).
    Returns fp32 [B,Tq,Tk].
    """
    q = q_idx.float()
    k = k_idx.float()
    raw = torch.einsum("bqhd,bkd->bhqk", q, k) * scale
    gated = torch.sigmoid(raw + bias.float().view(1, -1, 1, 1))
    wsig = torch.sigmoid(w.float()).permute(0, 2, 1).unsqueeze(-1)
    scores = (gated * wsig).sum(dim=1)
    if causal:
        Tq, Tk = scores.shape[1], scores.shape[2]
        qpos = q_offset + torch.arange(Tq).unsqueeze(1)
        kpos = torch.arange(Tk).unsqueeze(0)
        scores = scores.masked_fill((kpos > qpos).unsqueeze(0), float("-inf"))
    return scores


# ---------------------------------------------------------------------------
# Selector  (gsa_triton/gsa_ref.py:131-150; ascending re-sort gsa_opt.py:674-677)
# ---------------------------------------------------------------------------

def k_effective(k_base: int, k_max: int, t_kv: int) -> int:
    """Fixed k: min(k_base, k_max, T_kv); k_min is unused (gsa_ref.py:142)."""
    return min(k_base, k_max, t_kv)


def select_topk(scores: torch.Tensor, k_eff: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """Tie-aware restatement of AdaptiveTopKSelector.forward (gsa_ref.py:138-150).

    -inf -> -1e9, then the k largest by (value desc, index asc).  Returns the
    indices in that order (int64) and mask = gathered score != -inf.
    """
    filled = scores.masked_fill(scores == float("-inf"), -1e9)
    order = torch.sort(filled, dim=-1, descending=True, stable=True).indices
    idx = order[..., :k_eff].contiguous()
    mask = torch.gather(scores, -1, idx) != float("-inf")
    return idx, mask


def select_ascending(scores: torch.Tensor, k_eff: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """Selected valid indices in ascending order, plus the per-row valid count.

    The optimized reference sorts the selector's indices ascending and permutes
    the mask with them (gsa_opt.py:674-677); the valid entries then form a
    prefix when the invalid ones are moved behind them.  Returns
    idx int32 [B,T,k_eff] (valid ascending, then invalid ascending) and
    count int32 [B,T].
    """
    idx, mask = select_topk(scores, k_eff)
    # valid first, each group ascending: sort key = (invalid, index)
    key = idx + (~mask).long() * (1 << 40)
    srt = torch.sort(key, dim=-1).values
    out = (srt & ((1 << 40) - 1)).to(torch.int32)
    return out, mask.sum(dim=-1).to(torch.int32)


def row_variance(scores: torch.Tensor) -> torch.Tensor:
    """Population variance of each row's valid (finite) scores (gsa_explained.ipynb:577-592)."""
    valid = scores != float("-inf")
    cnt = valid.sum(dim=-1, keepdim=True).clamp(min=1).float()
    sv = scores.masked_fill(~valid, 0.0)
    mean = sv.sum(dim=-1, keepdim=True) / cnt
    diff = (sv - mean * valid.float()).masked_fill(~valid, 0.0)
    return diff.pow(2).sum(dim=-1) / cnt.squeeze(-1)


def adaptive_k_from_variance(var: torch.Tensor, k_base: int, k_min: int, k_max: int) -> torch.Tensor:
    """k_t = clamp(floor(k_base * avg_var / var_t), k_min, k_max); avg_var = mean of var over every
    row (and batch); both variances clamped to >= 1e-6 (gsa_explained.ipynb:577-592)."""
    avg = var.mean().clamp(min=1e-6)
    return (k_base * avg / var.clamp(min=1e-6)).floor().clamp(min=k_min, max=k_max).long()


def adaptive_k(scores: torch.Tensor, k_base: int, k_min: int, k_max: int) -> torch.Tensor:
    """Variance-based per-row k (gsa_explained.ipynb:577-592).

    var_t = population variance of row t's valid (finite) scores; the mean of
    var over all rows (and batches) is avg_var; k_t = clamp(floor(k_base *
    avg_var / var_t), k_min, k_max), with both variances clamped to >= 1e-6.
    """
    return adaptive_k_from_variance(row_variance(scores), k_base, k_min, k_max)


# ---------------------------------------------------------------------------
# Sparse attention  (gsa_triton/gsa_ref.py:185-238)
# ---------------------------------------------------------------------------

def gather_rows(x: torch.Tensor, indices: torch.Tensor) -> torch.Tensor:
    """x [B,Tkv,H,d], indices [B,Tq,k] -> [B,Tq,k,H,d] after clamping to [0,Tkv-1].

    Same values as the reference's expand+gather (gsa_ref.py:185-199); a
    gather is exact, so direct indexing is used to keep memory bounded.
    """
    B, Tkv = x.shape[0], x.shape[1]
    idx = indices.clamp(0, Tkv - 1).long()
    bidx = torch.arange(B).view(B, 1, 1)
    return x[bidx, idx]


def sparse_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                     indices: torch.Tensor, mask: torch.Tensor, scale: float) -> torch.Tensor:
    """Per (b,t,h): softmax over the selected keys, masked entries excluded.

    gsa_ref.py:202-238: scores = <q, K[idx]>*scale; masked -> -inf; softmax;
    masked -> 0; NaN (all masked) -> 0; out = sum p * V[idx].  Ops run in q's
    dtype like the reference.
    """
    kg = gather_rows(k, indices).permute(0, 1, 3, 2, 4)
    vg = gather_rows(v, indices).permute(0, 1, 3, 2, 4)
    s = torch.einsum("bqhd,bqhkd->bqhk", q, kg) * scale
    m = mask.unsqueeze(2)
    s = s.masked_fill(~m, float("-inf"))
    p = torch.softmax(s, dim=-1)
    p = p.masked_fill(~m, 0.0).nan_to_num(0.0)
    return torch.einsum("bqhk,bqhkd->bqhd", p, vg)


# ---------------------------------------------------------------------------
# Parameters and the layer forward  (gsa_triton/gsa_ref.py:243-325)
# ---------------------------------------------------------------------------

@dataclass
class GSAConfig:
    hidden_size: int = 2048
    num_heads: int = 16
    k_max: int = 4096
    d_indexer: int = 64
    n_idx_heads: int = 4
    k_base: int = 2048
    k_min: int = 256

    @property
    def d_head(self) -> int:
        return self.hidden_size // self.num_heads

    @property
    def scale(self) -> float:
        return self.d_head ** -0.5


def synthetic_state(cfg: GSAConfig, seed: int = 0, std: float = 0.02,
                    gate_bias: float = 0.5) -> Dict[str, torch.Tensor]:
    """Synthetic fp32 weights in the reference's state_dict layout.

    Weights ~ N(0, std) drawn from one CPU generator in a fixed order
    (q, k, v, o, value-gate, output-gate, idx_q, idx_k, idx_w); gate biases =
    ``gate_bias``; indexer biases (idx_bias and idx_w_proj.bias) = 0;
    inv_freq as the reference computes it (gsa_ref.py:47).
    """
    g = torch.Generator().manual_seed(seed)
    D, Hi, di = cfg.hidden_size, cfg.n_idx_heads, cfg.d_indexer

    def n(*shape):
        return torch.randn(*shape, generator=g) * std

    sd = {}
    sd["q_proj.weight"] = n(D, D)
    sd["k_proj.weight"] = n(D, D)
    sd["v_proj.weight"] = n(D, D)
    sd["o_proj.weight"] = n(D, D)
    sd["value_gate.gate_proj.weight"] = n(D, D)
    sd["output_gate.gate_proj.weight"] = n(D, D)
    sd["indexer.idx_q_proj.weight"] = n(Hi * di, D)
    sd["indexer.idx_k_proj.weight"] = n(di, D)
    sd["indexer.idx_w_proj.weight"] = n(Hi, D)
    sd["indexer.idx_w_proj.bias"] = torch.zeros(Hi)
    sd["indexer.idx_bias"] = torch.zeros(Hi)
    sd["value_gate.gate_proj.bias"] = torch.full((D,), gate_bias)
    sd["output_gate.gate_proj.bias"] = torch.full((D,), gate_bias)
    sd["rotary_emb.inv_freq"] = rope_inv_freq(cfg.d_head)
    return sd


def cast_state(sd: Dict[str, torch.Tensor], dtype: torch.dtype) -> Dict[str, torch.Tensor]:
    """nn.Module.to(dtype): every floating tensor, buffers included."""
    return {k: v.to(dtype) for k, v in sd.items()}


def synthetic_input(B: int, T: int, D: int, seed: int = 1,
                    sigma: Optional[torch.Tensor] = None) -> torch.Tensor:
    """x ~ N(0,1) fp32 [B,T,D]; with ``sigma`` [B], row block b is scaled by sigma[b]."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(B, T, D, generator=g)
    if sigma is not None:
        x = x * sigma.view(B, 1, 1)
    return x


@dataclass
class Projections:
    q: Optional[torch.Tensor]       # [B,T,H,d] after RoPE
    k: Optional[torch.Tensor]       # [B,T,H,d] after RoPE
    v: Optional[torch.Tensor]       # [B,T,H,d] after the value gate
    og: Optional[torch.Tensor]      # [B,T,D] output-gate sigmoid
    q_idx: Optional[torch.Tensor]   # [B,T,Hi,di]
    k_idx: Optional[torch.Tensor]   # [B,T,di]
    w_idx: Optional[torch.Tensor]   # [B,T,Hi]


PARTS = ("q", "k", "v", "og", "q_idx", "k_idx", "w_idx")


def project(sd: Dict[str, torch.Tensor], cfg: GSAConfig, x: torch.Tensor,
            rope: Optional[RopeCache] = None, pos0: int = 0, seq_len: Optional[int] = None,
            parts=PARTS) -> Projections:
    """Steps 1-3 of gsa_ref.GatedSparseAttention.forward plus the indexer projections.

    q,k,v = Linear(x) (gsa_ref.py:283-285); v *= sigmoid(gate_v(x))
    (gsa_ref.py:163-166); RoPE on q,k (gsa_ref.py:295-298); idx_q/idx_k/idx_w
    projections (gsa_ref.py:100-102); sigmoid(gate_o(x)) (gsa_ref.py:178).

    ``x`` may be a row slice of the layer input: its first row sits at
    absolute position ``pos0`` of a layer call over ``seq_len`` rows (default
    pos0 + rows), and the RoPE tables are the ones that call requests
    (gsa_ref.py:293: ``rotary_emb(seq_len)``, which decides the >8192 rebuild)
    read at those positions.  ``parts`` names the projections to compute; the
    others are None.
    """
    B, T, D = x.shape
    H, d = cfg.num_heads, cfg.d_head
    dt = x.dtype
    seq_len = pos0 + T if seq_len is None else seq_len
    if pos0 < 0 or pos0 + T > seq_len:
        raise ValueError(f"rows [{pos0}, {pos0 + T}) outside a layer call over {seq_len} rows")
    unknown = set(parts) - set(PARTS)
    if unknown:
        raise ValueError(f"unknown projections {sorted(unknown)}")
    if rope is None:
        rope = RopeCache(d, dt, sd["rotary_emb.inv_freq"])
    out = dict.fromkeys(PARTS)
    if "q" in parts or "k" in parts:
        cos, sin = rope.tables(seq_len, dt)
        cos = cos[pos0:pos0 + T].unsqueeze(0).unsqueeze(2)
        sin = sin[pos0:pos0 + T].unsqueeze(0).unsqueeze(2)
    if "q" in parts:
        out["q"] = apply_rope(F.linear(x, sd["q_proj.weight"]).view(B, T, H, d), cos, sin)
    if "k" in parts:
        out["k"] = apply_rope(F.linear(x, sd["k_proj.weight"]).view(B, T, H, d), cos, sin)
    if "v" in parts:
        v = F.linear(x, sd["v_proj.weight"]).view(B, T, H, d)
        gv = torch.sigmoid(F.linear(x, sd["value_gate.gate_proj.weight"], sd["value_gate.gate_proj.bias"]))
        out["v"] = v * gv.view(B, T, H, d)
    if "og" in parts:
        out["og"] = torch.sigmoid(F.linear(x, sd["output_gate.gate_proj.weight"],
                                           sd["output_gate.gate_proj.bias"]))
    if "q_idx" in parts:
        out["q_idx"] = F.linear(x, sd["indexer.idx_q_proj.weight"]).view(B, T, cfg.n_idx_heads, cfg.d_indexer)
    if "k_idx" in parts:
        out["k_idx"] = F.linear(x, sd["indexer.idx_k_proj.weight"])
    if "w_idx" in parts:
        out["w_idx"] = F.linear(x, sd["indexer.idx_w_proj.weight"], sd["indexer.idx_w_proj.bias"])
    return Projections(**out)


def gsa_forward(sd: Dict[str, torch.Tensor], cfg: GSAConfig, x: torch.Tensor,
                rope: Optional[RopeCache] = None, return_aux: bool = False):
    """gsa_ref.GatedSparseAttention.forward (gsa_ref.py:276-325), unchunked.

    Memory is O(B*T*k*H*d) for the gathered rows, so this is for small T.
    """
    B, T, D = x.shape
    p = project(sd, cfg, x, rope)
    scores = indexer_scores(p.q_idx, p.k_idx, p.w_idx, sd["indexer.idx_bias"],
                            1.0 / math.sqrt(cfg.d_indexer))
    k_eff = k_effective(cfg.k_base, cfg.k_max, T)
    idx, mask = select_topk(scores, k_eff)
    attn = sparse_attention(p.q, p.k, p.v, idx, mask, cfg.scale)
    attn = attn * p.og.view(B, T, cfg.num_heads, cfg.d_head)
    out = F.linear(attn.reshape(B, T, D), sd["o_proj.weight"])
    if return_aux:
        return out, dict(proj=p, scores=scores, idx=idx, mask=mask, attn=attn, k_eff=k_eff)
    return out


def attend_rows(sd: Dict[str, torch.Tensor], cfg: GSAConfig, p: Projections,
                r0: int, r1: int, idx: Optional[torch.Tensor] = None,
                mask: Optional[torch.Tensor] = None, return_sel: bool = False,
                rows: Optional[Projections] = None):
    """Query rows [r0, r1) of the layer, given the keys' projections.

    Query-chunked form of gsa_ref.py:303-323: the indexer for the chunk uses
    the absolute-position causal mask of benchmark_models.ipynb:107-115.  The
    query-side projections (q, og, q_idx, w_idx) are ``p``'s rows [r0, r1),
    or ``rows``' when given (``rows`` then holds exactly those rows); k, v
    and k_idx come from ``p`` for every key.  With ``idx``/``mask`` given,
    the selection is taken from them (used to check the attention on the
    kernel's own indices).  Returns the layer output rows [B, r1-r0, D] (and
    the selection when asked).
    """
    B, T = p.k.shape[0], p.k.shape[1]
    D = cfg.hidden_size
    if rows is None:
        q, og, q_idx, w_idx = p.q[:, r0:r1], p.og[:, r0:r1], p.q_idx[:, r0:r1], p.w_idx[:, r0:r1]
    else:
        q, og, q_idx, w_idx = rows.q, rows.og, rows.q_idx, rows.w_idx
        if q.shape[1] != r1 - r0:
            raise ValueError(f"rows holds {q.shape[1]} query rows, expected {r1 - r0}")
    k_eff = k_effective(cfg.k_base, cfg.k_max, T)
    if idx is None:
        s = indexer_scores(q_idx, p.k_idx, w_idx, sd["indexer.idx_bias"], 1.0 / math.sqrt(cfg.d_indexer),
                           q_offset=r0)
        idx, mask = select_topk(s, k_eff)
    attn = sparse_attention(q, p.k, p.v, idx, mask, cfg.scale)
    attn = attn * og.view(B, r1 - r0, cfg.num_heads, cfg.d_head)
    out = F.linear(attn.reshape(B, r1 - r0, D), sd["o_proj.weight"])
    if return_sel:
        return out, idx, mask
    return out


def gsa_forward_chunked(sd: Dict[str, torch.Tensor], cfg: GSAConfig, x: torch.Tensor,
                        chunk: int = 64, rope: Optional[RopeCache] = None) -> torch.Tensor:
    """Query-chunked layer forward: same semantics as ``gsa_forward`` with bounded memory."""
    B, T, D = x.shape
    p = project(sd, cfg, x, rope)
    outs = [attend_rows(sd, cfg, p, r0, min(T, r0 + chunk)) for r0 in range(0, T, chunk)]
    return torch.cat(outs, dim=1)
