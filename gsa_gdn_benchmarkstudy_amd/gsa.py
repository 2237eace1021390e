"""Gated Sparse Attention forward on MI355X: the drop-in module.

Same constructor, forward, ``fuse_projections`` and state_dict keys as the
reference's ``gsa_triton/gsa_opt.py`` (and ``gsa_ref.py``), so a caller can
``load_state_dict(ref_state, strict=True)`` and swap the module.  The GEMMs
stay on PyTorch-ROCm (hipBLASLt); everything else runs in the hand-written
gfx950 kernels of ``libgsa_hip.so`` through ``_abi``:

  fused projection GEMM -> [indexer stream] gsa_indexer_select (MFMA indexer +
  exact streaming top-k) || [current stream] gsa_prologue (RoPE k, G2 gate)
  -> join -> gsa_sparse_attn (RoPE q, gather attention, G1 gate) -> o_proj GEMM

Forward only (inference); there is no autograd support, like the reference's
Triton kernels.  There is no CPU or eager fallback: the kernels need a GPU and
the built library, and raise otherwise.
"""

from __future__ import annotations

import math
from typing import Optional, Tuple

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import _abi
from .roctx import range_pop as _range_pop, range_push as _range_push


# Width of the fused projection output is padded to a multiple of this many
# elements so every row (and every slice offset) stays 16-byte aligned.
FUSED_ALIGN = 64


_CU_COUNT = {}
# Last-level (Infinity) cache of one MI355X.
_LLC_BYTES = 256 << 20


def _cu_count(dev: torch.device) -> int:
    """Compute units of the device (cached)."""
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    if idx not in _CU_COUNT:
        _CU_COUNT[idx] = torch.cuda.get_device_properties(idx).multi_processor_count
    return _CU_COUNT[idx]


# ---------------------------------------------------------------------------
# Launchers (gsa_opt.py:143-176, :349-383)
# ---------------------------------------------------------------------------

def fused_gated_indexer(q_idx: torch.Tensor, k_idx: torch.Tensor, w: torch.Tensor,
                        bias: torch.Tensor, scale: float, causal: bool = True) -> torch.Tensor:
    """Indexer scores fp32 [B,T,T] (-inf above the diagonal when causal).

    Same signature as gsa_opt.fused_gated_indexer (gsa_opt.py:143-150); strided
    views are read in place (no ``.contiguous()`` copies).
    """
    _range_push("gsa_hip/indexer_scores")
    try:
        return _abi.indexer_scores(q_idx, k_idx, w, bias.detach().float().contiguous(), scale, causal)
    finally:
        _range_pop()


def fused_sparse_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                           indices: torch.Tensor, mask: torch.Tensor, scale: float) -> torch.Tensor:
    """Sparse attention over selected keys (gsa_opt.py:349-356 signature).

    q,k,v [B,T,H,d]; indices [B,T,K] (any integer dtype, any order; clamped
    to [0, T_kv-1]); mask [B,T,K] bool (True = valid).  Returns q's dtype.
    """
    _range_push("gsa_hip/sparse_attn")
    try:
        idx = indices.to(torch.int32).contiguous()
        m = mask.to(torch.uint8).contiguous()
        q, k, v = (t if t.stride(-1) == 1 else t.contiguous() for t in (q, k, v))
        return _abi.sparse_attn(q, k, v, idx, scale, mask=m)
    finally:
        _range_pop()


# ---------------------------------------------------------------------------
# RoPE (gsa_opt.py:390-429)
# ---------------------------------------------------------------------------

def _rope_table(t: torch.Tensor, d: int) -> torch.Tensor:
    """[T, d] view of a cos/sin table given as [T,d] or broadcastable [1,T,1,d]."""
    t2 = t.reshape(-1, t.shape[-1])
    if t2.shape[-1] != d:
        raise ValueError(f"cos/sin last dim {t2.shape[-1]} != head dim {d}")
    return t2 if t2.stride(-1) == 1 else t2.contiguous()


def apply_rotary_pos_emb(q: torch.Tensor, k: torch.Tensor, cos: torch.Tensor,
                         sin: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """(q*cos + rotate_half(q)*sin, same for k), rounded per op in the input dtype."""
    d = q.shape[-1]
    c, s = _rope_table(cos, d), _rope_table(sin, d)
    q = q if q.stride(-1) == 1 else q.contiguous()
    k = k if k.stride(-1) == 1 else k.contiguous()
    q_out, _ = _abi.prologue(k=q, cos=c.to(q.dtype), sin=s.to(q.dtype))
    k_out, _ = _abi.prologue(k=k, cos=c.to(k.dtype), sin=s.to(k.dtype))
    return q_out, k_out


class RotaryEmbedding(nn.Module):
    """cos/sin tables with the reference's cache semantics (gsa_opt.py:404-429).

    The cache covers ``max_seq_len`` positions from the fp32 inv_freq at
    construction and is cast with the module.  A longer request rebuilds it
    from ``arange(seq_len)`` times the module's current inv_freq (bf16 when
    the module was cast); the rebuild runs on the host, where the reference's
    arithmetic runs, and the result moves to the requested device.
    """

    def __init__(self, dim: int, max_seq_len: int = 8192, base: float = 10000.0):
        super().__init__()
        self.dim = dim
        inv_freq = 1.0 / (base ** (torch.arange(0, dim, 2).float() / dim))
        self.register_buffer("inv_freq", inv_freq)
        self._build_cache(max_seq_len, inv_freq)

    def _build_cache(self, seq_len: int, inv_freq: torch.Tensor) -> None:
        pos = torch.arange(seq_len, dtype=torch.float32)
        ang = torch.outer(pos, inv_freq.detach().cpu())
        ang = torch.cat((ang, ang), dim=-1)
        dev = self.inv_freq.device
        self.register_buffer("cos_cached", ang.cos().to(dev), persistent=False)
        self.register_buffer("sin_cached", ang.sin().to(dev), persistent=False)

    def forward(self, seq_len: int, device: torch.device,
                dtype: Optional[torch.dtype] = None) -> Tuple[torch.Tensor, torch.Tensor]:
        if seq_len > self.cos_cached.shape[0]:
            self._build_cache(seq_len, self.inv_freq)
        # The cast tables are kept while the cache they came from is unchanged
        # (same storage and version): casting again would give the same values.
        key = (self.cos_cached.data_ptr(), self.cos_cached._version, self.sin_cached.data_ptr(),
               self.sin_cached._version, seq_len, torch.device(device), dtype)
        hit = getattr(self, "_cast", None)
        if hit is not None and hit[0] == key:
            return hit[1], hit[2]
        cos = self.cos_cached[:seq_len].to(device)
        sin = self.sin_cached[:seq_len].to(device)
        if dtype is not None:
            cos, sin = cos.to(dtype), sin.to(dtype)
        cos, sin = cos.contiguous(), sin.contiguous()
        self._cast = (key, cos, sin)
        return cos, sin

    def halves(self, seq_len: int, device: torch.device,
               dtype: Optional[torch.dtype] = None) -> Optional[torch.Tensor]:
        """The cast tables of ``forward`` packed for the dense attention's RoPE
        (``ATTN_ROPE_HALVES``): row t holds cos[t][:dim/2] then sin[t][:dim/2].
        The tables repeat their first half (the angles are cat(freqs, freqs)),
        so nothing is lost; None when they do not (a cache edited by hand).
        Kept, like the cast tables, while the cache is unchanged."""
        cos, sin = self.forward(seq_len, device, dtype)
        key = self._cast[0]
        hit = getattr(self, "_halves", None)
        if hit is not None and hit[0] == key:
            return hit[1]
        h = self.dim // 2
        t = None
        if torch.equal(cos[:, :h], cos[:, h:]) and torch.equal(sin[:, :h], sin[:, h:]):
            t = torch.cat((cos[:, :h], sin[:, :h]), dim=-1).contiguous()
        self._halves = (key, t)
        return t


# ---------------------------------------------------------------------------
# Sub-modules with the reference's state_dict keys (gsa_opt.py:432-507)
# ---------------------------------------------------------------------------

class GatedLightningIndexer(nn.Module):
    """score[q,k] = sum_h sigmoid(w[q,h]) * sigmoid(q_I[q,h].k_I[k]*scale + b[h])."""

    def __init__(self, hidden_size: int, d_indexer: int = 64, n_idx_heads: int = 4):
        super().__init__()
        self.d_indexer = d_indexer
        self.n_idx_heads = n_idx_heads
        self.scale = 1.0 / math.sqrt(d_indexer)
        self.idx_q_proj = nn.Linear(hidden_size, n_idx_heads * d_indexer, bias=False)
        self.idx_k_proj = nn.Linear(hidden_size, d_indexer, bias=False)
        self.idx_w_proj = nn.Linear(hidden_size, n_idx_heads, bias=True)
        self.idx_bias = nn.Parameter(torch.zeros(n_idx_heads))
        nn.init.xavier_uniform_(self.idx_q_proj.weight, gain=1.0)
        nn.init.xavier_uniform_(self.idx_k_proj.weight, gain=1.0)
        nn.init.xavier_uniform_(self.idx_w_proj.weight, gain=0.1)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        B, T, _ = x.shape
        q_idx = self.idx_q_proj(x).view(B, T, self.n_idx_heads, self.d_indexer)
        k_idx = self.idx_k_proj(x)
        w = self.idx_w_proj(x)
        return fused_gated_indexer(q_idx, k_idx, w, self.idx_bias, self.scale, causal=True)


class AdaptiveTopKSelector(nn.Module):
    """Per-row top-k selector (gsa_opt.py:466-483).

    ``mode = "fixed"`` (default, the reference's behaviour): every row takes
    k_eff = min(k_base, k_max, T_kv); k_min is kept but unused.

    ``mode = "variance"``: the variance-based rule of gsa_explained.ipynb:577-592.
    Row t takes k_t = min(clamp(floor(k_base * avg / var_t), k_min, k_max), T_kv),
    var_t the population variance of its finite scores and avg the mean of var_t
    over all rows of the batch (both clamped to >= 1e-6).  Outputs are then
    min(k_max, T_kv) wide, entries past k_t masked out; ``last_k`` holds the
    per-row k of the latest call (int32 [B,T], on the device).
    """

    MODES = ("fixed", "variance")

    def __init__(self, k_base: int = 2048, k_min: int = 256, k_max: int = 4096):
        super().__init__()
        self.k_base = k_base
        self.k_min = k_min
        self.k_max = k_max
        self.mode = "fixed"
        self.last_k: Optional[torch.Tensor] = None

    def adaptive(self) -> bool:
        if self.mode not in self.MODES:
            raise ValueError(f"selector mode {self.mode!r}: expected one of {self.MODES}")
        return self.mode == "variance"

    def k_effective(self, t_kv: int) -> int:
        """Output width: k_eff (fixed mode) or min(k_max, T_kv) (variance mode)."""
        if self.adaptive():
            return min(self.k_max, t_kv)
        return min(self.k_base, self.k_max, t_kv)

    def _select(self, s: torch.Tensor, k_eff: int, order: int, want_mask: bool = True):
        if self.adaptive():
            idx, cnt, mask, k_rows, _ = _abi.topk_select_adaptive(s, self.k_base, self.k_min, self.k_max,
                                                                  order, want_mask=want_mask)
            self.last_k = k_rows
            return idx, cnt, mask
        return _abi.topk_select(s, k_eff, order, want_mask=want_mask)

    def forward(self, scores: torch.Tensor):
        """(indices int64 [B,T,k] by (score desc, index asc), mask bool, k_eff)."""
        B, T, T_kv = scores.shape
        k_eff = self.k_effective(T_kv)
        s = scores if scores.dtype == torch.float32 and scores.stride(-1) == 1 else \
            scores.float().contiguous()
        _range_push("gsa_hip/topk_select")
        try:
            if k_eff <= _abi.TOPK_DESC_MAX_K:
                idx, _, mask = self._select(s, k_eff, _abi.ORDER_SCORE_DESC)
                return idx.long(), mask.bool(), k_eff
            # larger k: exact selection in index order, then a stable device sort by score
            idx, _, mask = self._select(s, k_eff, _abi.ORDER_INDEX_ASC)
            idx = idx.long()
            vals = torch.gather(s, -1, idx).masked_fill(~mask.bool(), -1e9)
            order = torch.sort(vals, dim=-1, descending=True, stable=True).indices
            idx = torch.gather(idx, -1, order)
            return idx, torch.gather(mask.bool(), -1, order), k_eff
        finally:
            _range_pop()

    def select_ascending(self, scores: torch.Tensor):
        """(idx int32 [B,T,k] valid-ascending, count int32 [B,T], k_eff)."""
        k_eff = self.k_effective(scores.shape[-1])
        idx, cnt, _ = self._select(scores, k_eff, _abi.ORDER_INDEX_ASC, want_mask=False)
        return idx, cnt, k_eff


def _gate(v: torch.Tensor, logits: torch.Tensor) -> torch.Tensor:
    """v * sigmoid(logits), both [B,T,H,d], rounded per op in v's dtype."""
    v = v if v.stride(-1) == 1 else v.contiguous()
    _, out = _abi.prologue(v=v, vg=logits)
    return out


class ValueGate(nn.Module):
    """G2: v = v * sigmoid(W x + b), bias initialised to 0.5."""

    def __init__(self, hidden_size: int):
        super().__init__()
        self.gate_proj = nn.Linear(hidden_size, hidden_size, bias=True)
        nn.init.constant_(self.gate_proj.bias, 0.5)

    def forward(self, v: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
        B, T, H, d = v.shape
        return _gate(v, self.gate_proj(x).view(B, T, H, d))


class OutputGate(nn.Module):
    """G1: o = o * sigmoid(W x + b), bias initialised to 0.5."""

    def __init__(self, hidden_size: int):
        super().__init__()
        self.gate_proj = nn.Linear(hidden_size, hidden_size, bias=True)
        nn.init.constant_(self.gate_proj.bias, 0.5)

    def forward(self, output: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
        B, T, H, d = output.shape
        return _gate(output, self.gate_proj(x).view(B, T, H, d))


# ---------------------------------------------------------------------------
# The layer (gsa_opt.py:512-730)
# ---------------------------------------------------------------------------

class GatedSparseAttention(nn.Module):
    """Drop-in replacement for gsa_ref/gsa_opt.GatedSparseAttention.

    Forward, per layer call (two streams; ``indexer_overlap`` places step 2):
      1. the indexer projections (one small GEMM over the fused weight's last,
         zero-padded 64-aligned row block) and the q/k/v/gate GEMM; the slices
         are strided views, never copied (``proj_impl="fused"``: one MFMA GEMM
         with step 3's producer in its epilogue instead);
      2. gsa_indexer_select -- MFMA indexer fused with the exact top-k,
         writing the selection as a bitmask, and for the gather attention
         ascending int32 indices with per-row counts (no score is stored:
         they are recomputed pass by pass and the candidates near each row's
         threshold stay in LDS) -- beside the q/k/v/gate GEMM while its grid leaves
         CUs free, before it while RoPE(k) and V^T fit the last-level cache,
         else beside the producer; the dense attention's lane masks
         (gsa_dense_lane_masks) follow on the second stream (with the
         indexer on the current stream: built in the producer's launch);
      3. current stream: RoPE(k) and v * sigmoid(vg) (gsa_prologue_vt, V
         transposed, or gsa_prologue);
      4. join, then the attention with RoPE(q) and the output gate fused --
         gsa_dense_attn (bf16: MFMA over every causal key tile, masked to the
         selection) or gsa_sparse_attn (per-row gather of the selected keys)
         -- and the o_proj GEMM.
    """

    def __init__(self, hidden_size: int, num_heads: int, k_max: int = 4096, d_indexer: int = 64,
                 n_idx_heads: int = 4, k_base: int = 2048, k_min: int = 256):
        super().__init__()
        self.hidden_size = hidden_size
        self.num_heads = num_heads
        self.d_head = hidden_size // num_heads
        self.scale = self.d_head ** -0.5

        self.q_proj = nn.Linear(hidden_size, hidden_size, bias=False)
        self.k_proj = nn.Linear(hidden_size, hidden_size, bias=False)
        self.v_proj = nn.Linear(hidden_size, hidden_size, bias=False)
        self.o_proj = nn.Linear(hidden_size, hidden_size, bias=False)

        self.indexer = GatedLightningIndexer(hidden_size, d_indexer, n_idx_heads)
        self.topk_selector = AdaptiveTopKSelector(k_base, k_min, k_max)
        self.value_gate = ValueGate(hidden_size)
        self.output_gate = OutputGate(hidden_size)
        self.rotary_emb = RotaryEmbedding(self.d_head)

        self._fused_weight: Optional[torch.Tensor] = None
        self._fused_bias: Optional[torch.Tensor] = None
        self._packed: Optional[tuple] = None
        self._idx_bias32: Optional[torch.Tensor] = None
        self._proj_sizes = [
            hidden_size, hidden_size, hidden_size, hidden_size, hidden_size,
            n_idx_heads * d_indexer, d_indexer, n_idx_heads,
        ]
        total = sum(self._proj_sizes)
        self._fused_width = (total + FUSED_ALIGN - 1) // FUSED_ALIGN * FUSED_ALIGN
        self._indexer_stream: Optional[torch.cuda.Stream] = None
        # Attention kernel: "dense" (block-dense MFMA over the causal key tiles
        # with the selection as a bitmask, bf16), "gather" (per-row gather of
        # the selected keys, bf16 and fp32), or "auto" (dense for bf16).
        self.attn_impl = "auto"
        # Where the fused indexer + top-k runs relative to the main projection
        # GEMM: "gemm" (on a side stream beside the GEMM), "producer" (after
        # the GEMM, on a side stream beside the RoPE/gate producer), "serial"
        # (everything on the current stream) or "auto": "gemm" while the
        # indexer's grid (one block per 16 query rows) leaves CUs free for the
        # GEMM -- fewer than 4 blocks per CU; else "serial" while RoPE(k) and
        # V^T together fit the 256 MB last-level cache (the producer then
        # runs right before the attention, which finds them cached); else
        # "producer".
        self.indexer_overlap = "auto"
        # Main projection on the bf16 block-dense path: "gemm" (hipBLASLt GEMM,
        # then the RoPE / value-gate producer kernel) or "fused" (own MFMA GEMM
        # with that producer in its epilogue; needs an even head count and
        # T % 64 == 0, else "gemm" runs).
        self.proj_impl = "gemm"
        # When the indexer runs on the current stream ("serial" placement), the
        # dense attention's lane masks are built by the producer's launch
        # (gsa_prologue_vt_lane_masks) instead of on a second stream beside
        # the GEMM: no join before the attention, and the GEMM has the GPU.
        self.lane_masks_with_producer = True
        # Optional per-kernel timing hook: a list to which forward appends
        # (start, end) event pairs around the sparse-attention launch.
        self.attn_events: Optional[list] = None
        self.register_load_state_dict_post_hook(lambda mod, _keys: mod._drop_fused())

    # -- fused projection weight -------------------------------------------
    def _drop_fused(self) -> None:
        self._fused_weight = None
        self._fused_bias = None
        self._packed = None
        self._idx_bias32 = None

    def fuse_projections(self) -> None:
        """Build the fused, padded projection weight/bias.  Call after load_state_dict()."""
        w = torch.cat([
            self.q_proj.weight, self.k_proj.weight, self.v_proj.weight,
            self.value_gate.gate_proj.weight, self.output_gate.gate_proj.weight,
            self.indexer.idx_q_proj.weight, self.indexer.idx_k_proj.weight,
            self.indexer.idx_w_proj.weight,
        ], dim=0).detach()
        pad = self._fused_width - w.shape[0]
        if pad:
            w = torch.cat([w, w.new_zeros(pad, w.shape[1])], dim=0)
        bias = w.new_zeros(self._fused_width)
        off = self._offsets()
        D = self.hidden_size
        bias[off["vg"]:off["vg"] + D] = self.value_gate.gate_proj.bias.detach()
        bias[off["og"]:off["og"] + D] = self.output_gate.gate_proj.bias.detach()
        bias[off["iw"]:off["iw"] + self.indexer.n_idx_heads] = self.indexer.idx_w_proj.bias.detach()
        self._fused_weight = w.contiguous()
        self._fused_bias = bias
        self._packed = None
        # fp32 copy of the indexer bias for the kernels (built here, not per call)
        self._idx_bias32 = self.indexer.idx_bias.detach().float().contiguous()

    def _get_fused_weight(self, like: Optional[torch.Tensor] = None):
        fw = self._fused_weight
        if fw is None or (like is not None and (fw.device != like.device or fw.dtype != like.dtype)):
            self.fuse_projections()
        return self._fused_weight, self._fused_bias

    def _offsets(self):
        names = ("q", "k", "v", "vg", "og", "iq", "ik", "iw")
        off, acc = {}, 0
        for n, sz in zip(names, self._proj_sizes):
            off[n] = acc
            acc += sz
        return off

    # -- forward pieces (also used by tests) -------------------------------
    def project_indexer(self, x: torch.Tensor):
        """GEMM of the indexer projections (idx_q, idx_k, idx_w: the fused weight's
        last, zero-padded 64-aligned row block) -> dict of strided views."""
        B, T, D = x.shape
        Hi, di = self.indexer.n_idx_heads, self.indexer.d_indexer
        w, b = self._get_fused_weight(x)
        off = self._offsets()
        base = off["iq"]
        comb = F.linear(x, w[base:], b[base:])
        return {"iq": comb[..., :Hi * di].view(B, T, Hi, di),
                "ik": comb[..., off["ik"] - base:off["ik"] - base + di],
                "iw": comb[..., off["iw"] - base:off["iw"] - base + Hi],
                "_ibuf": comb}

    def project_main(self, x: torch.Tensor):
        """GEMM of q, k, v and the two gate projections -> dict of strided views."""
        B, T, D = x.shape
        H, d = self.num_heads, self.d_head
        w, b = self._get_fused_weight(x)
        off = self._offsets()
        comb = F.linear(x, w[:off["iq"]], b[:off["iq"]])
        v = {n: comb[..., off[n]:off[n] + D].view(B, T, H, d) for n in ("q", "k", "v", "vg", "og")}
        v["_buf"] = comb
        return v

    def uses_fused_projection(self, x: torch.Tensor) -> bool:
        if self.proj_impl not in ("gemm", "fused"):
            raise ValueError(f"proj_impl {self.proj_impl!r}: expected 'gemm' or 'fused'")
        B, T, D = x.shape
        return (self.proj_impl == "fused" and self.uses_dense(x.dtype)
                and _abi.proj_supported(D, self.num_heads, T) and self.d_head == 128)

    def project_fused(self, x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor):
        """Main projection with the producer fused (gsa_proj_fused) -> dict with the raw q
        and og views, RoPE(k) and V^T = (v*sigmoid(vg))^T."""
        w, b = self._get_fused_weight(x)
        D = self.hidden_size
        if self._packed is None or self._packed[0].device != x.device:
            self._packed = _abi.proj_pack(w[:5 * D], b[:5 * D])
        wp, bp = self._packed
        q, og, k_rope, vt = _abi.proj_fused(x, wp, bp, cos, sin, self.num_heads)
        return {"q": q, "og": og, "_k_rope": k_rope, "_vt": vt}

    def project(self, x: torch.Tensor):
        """All eight projections -> dict of strided [B,T,...] views."""
        v = self.project_indexer(x)
        v.update(self.project_main(x))
        return v

    # Longest sequence the fused indexer + top-k takes (key positions and
    # sample counts are 16-bit there); longer ones go through the full score
    # matrix (gsa_indexer_scores, 4*B*T*T bytes) and the standalone selector.
    FUSED_SELECT_MAX_T = 65536

    def select(self, views, T: int, indices: bool = True):
        """Fused indexer + top-k on the current stream -> (bits, idx, count).

        bits: the selection bitmask int32 [B,T,2*ceil(T/64)]; idx/count
        (ascending int32, per-row count) only when ``indices``.
        """
        sel = self.topk_selector
        bias = self._idx_bias32
        if bias is None or bias.device != views["iq"].device:
            bias = self._idx_bias32 = self.indexer.idx_bias.detach().float().contiguous()
        if T > self.FUSED_SELECT_MAX_T:
            # the reference's own route (gsa_opt.py:660-677): the fp32 score
            # matrix, then the exact selection in index order
            scores = _abi.indexer_scores(views["iq"], views["ik"], views["iw"], bias, self.indexer.scale)
            idx, cnt, _ = sel.select_ascending(scores)
            del scores
            bits = _abi.selection_mask(idx, T, count=cnt)
            return (bits, idx, cnt) if indices else (bits, None, None)
        if sel.adaptive():
            bits, idx, cnt, k_rows, _ = _abi.indexer_select_adaptive(
                views["iq"], views["ik"], views["iw"], bias, self.indexer.scale, sel.k_base, sel.k_min,
                sel.k_max, indices=indices)
            sel.last_k = k_rows
            return bits, idx, cnt
        return _abi.indexer_select(views["iq"], views["ik"], views["iw"], bias, self.indexer.scale,
                                   sel.k_effective(T), indices=indices)

    def _side_stream(self, dev: torch.device) -> torch.cuda.Stream:
        """The layer's second stream (default priority), created on first use."""
        if self._indexer_stream is None or self._indexer_stream.device != dev:
            self._indexer_stream = torch.cuda.Stream(device=dev)
        return self._indexer_stream

    def uses_dense(self, dtype: torch.dtype) -> bool:
        if self.attn_impl not in ("auto", "dense", "gather"):
            raise ValueError(f"attn_impl {self.attn_impl!r}: expected 'auto', 'dense' or 'gather'")
        if self.attn_impl == "gather":
            return False
        if dtype != torch.bfloat16:
            if self.attn_impl == "dense":
                raise ValueError("the block-dense attention kernel is bf16 only")
            return False
        return True

    def forward(self, x: torch.Tensor, attention_mask: Optional[torch.Tensor] = None) -> torch.Tensor:
        if not x.is_cuda:
            raise RuntimeError("GatedSparseAttention (HIP) needs a device tensor")
        B, T, D = x.shape
        if D != self.hidden_size:
            raise ValueError(f"hidden size {D} != {self.hidden_size}")
        _range_push("gsa_hip/forward")
        dev = x.device
        cur = torch.cuda.current_stream(dev)

        dense = self.uses_dense(x.dtype)
        fused_proj = self.uses_fused_projection(x)
        cos, sin = self.rotary_emb(T, dev, x.dtype)
        cos, sin = cos.contiguous(), sin.contiguous()

        def main_projection():
            if fused_proj:
                return self.project_fused(x, cos, sin)
            return self.project_main(x)

        # Track A: the indexer projections, then the fused indexer + top-k
        # (and its bitmask), on a side stream that starts after the main
        # projection GEMM ("producer"), right after the small indexer GEMM
        # ("gemm"), or on the current stream ("serial").  The indexer and the
        # GEMM both fill the GPU and slow each other down when they share it.
        # Serially, the producer runs last before the attention and its
        # outputs (RoPE(k), V^T: 2*B*T*D elements) are still in the MI355X's
        # 256 MB last-level cache when the attention streams them; beyond
        # that size the producer is better hidden beside the indexer.
        mode = self.indexer_overlap
        if mode == "auto":
            if B * ((T + 15) // 16) < 4 * _cu_count(dev):
                mode = "gemm"
            elif 2 * B * T * D * x.element_size() <= _LLC_BYTES:
                mode = "serial"
            else:
                mode = "producer"
        elif mode not in ("producer", "gemm", "serial"):
            raise ValueError(f"indexer_overlap {mode!r}: expected 'auto', 'producer', 'gemm' or 'serial'")
        _range_push("gsa_hip/indexer_gemm")
        views = self.project_indexer(x)
        _range_pop()
        side = cur if mode == "serial" else self._side_stream(dev)
        if mode == "producer":
            _range_push("gsa_hip/main_gemm")
            views.update(main_projection())
            _range_pop()
        if side is not cur:
            side.wait_stream(cur)
        with torch.cuda.stream(side):
            _range_push("gsa_hip/indexer_select")
            bits, idx, cnt = self.select(views, T, indices=not dense)
            _range_pop()
        # The dense attention's lane masks, built from the bitmask off the
        # current stream (beside the projection GEMM / producer) on the
        # indexer's side stream; in "serial" mode by the producer's own launch
        # (lane_masks_with_producer), else on a second stream that starts after
        # the indexer.
        lm_ws, lm_stream = None, None
        lm_in_producer = (dense and not fused_proj and mode == "serial" and self.lane_masks_with_producer)
        if dense and not lm_in_producer:
            lm_stream = side if side is not cur else self._side_stream(dev)
            if lm_stream is not side:
                lm_stream.wait_stream(cur)
            with torch.cuda.stream(lm_stream):
                _range_push("gsa_hip/lane_masks")
                lm_ws = _abi.dense_lane_masks(bits, T, causal=True)   # the layer's attention is causal
                _range_pop()
        if mode != "producer":
            _range_push("gsa_hip/main_gemm")
            views.update(main_projection())
            _range_pop()

        # Track B: RoPE(k) and the value gate on the current stream
        _range_push("gsa_hip/prologue")
        if fused_proj:
            k_rope, v_gated = views["_k_rope"], views["_vt"]
        elif lm_in_producer:
            k_rope, v_gated, lm_ws = _abi.prologue_vt(views["v"], views["vg"], k=views["k"], cos=cos, sin=sin,
                                                      bits=bits, Tkv=T, causal=True)
        elif dense:
            k_rope, v_gated = _abi.prologue_vt(views["v"], views["vg"], k=views["k"], cos=cos, sin=sin)
        else:
            k_rope, v_gated = _abi.prologue(k=views["k"], v=views["v"], vg=views["vg"], cos=cos, sin=sin)
        _range_pop()

        if side is not cur:
            cur.wait_stream(side)
            for t in (idx, cnt, bits):
                if t is not None:
                    t.record_stream(cur)
            views["_ibuf"].record_stream(side)
        if lm_stream is not None:
            if lm_stream is not side:
                cur.wait_stream(lm_stream)
            lm_ws.record_stream(cur)

        _range_push("gsa_hip/sparse_attn")
        ev = None
        if self.attn_events is not None:
            ev = (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
            ev[0].record(cur)
        flags = _abi.ATTN_ROPE_Q | _abi.ATTN_OUT_GATE
        if dense:
            # one table load per block instead of two: cos and sin halves packed
            cs = self.rotary_emb.halves(T, dev, x.dtype)
            if cs is not None:
                attn = _abi.dense_attn(views["q"], k_rope, v_gated, bits, self.scale, og=views["og"],
                                       cos=cs, flags=flags | _abi.ATTN_ROPE_HALVES, causal=True, ws=lm_ws,
                                       masks_ready=True)
            else:
                attn = _abi.dense_attn(views["q"], k_rope, v_gated, bits, self.scale, og=views["og"],
                                       cos=cos, sin=sin, flags=flags, causal=True, ws=lm_ws, masks_ready=True)
        else:
            attn = _abi.sparse_attn(views["q"], k_rope, v_gated, idx, self.scale, count=cnt,
                                    og=views["og"], cos=cos, sin=sin, flags=flags)
        if ev is not None:
            ev[1].record(cur)
            self.attn_events.append(ev)
        _range_pop()

        _range_push("gsa_hip/o_proj")
        out = F.linear(attn.view(B, T, D), self.o_proj.weight)
        _range_pop()
        _range_pop()
        return out
