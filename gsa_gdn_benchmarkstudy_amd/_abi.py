"""ctypes binding of libgsa_hip.so (C ABI declared in include/gsa_hip.h).

The library is loaded after ``torch`` so that both share torch's HIP runtime
(one device context, one set of streams).  Every wrapper takes torch tensors,
checks their layout, passes raw pointers, strides and the current HIP stream,
and turns a non-zero status into ``RuntimeError``.  There is no fallback: a
missing library raises.
"""

from __future__ import annotations

import ctypes
import os
from typing import Optional

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libgsa_hip.so")

ABI_VERSION = 3

DTYPE_F32 = 0
DTYPE_BF16 = 1

ORDER_INDEX_ASC = 0
ORDER_SCORE_DESC = 1
TOPK_DESC_MAX_K = 4096

ATTN_ROPE_Q = 1
ATTN_OUT_GATE = 2
ATTN_MASKS_READY = 4
ATTN_ROPE_HALVES = 8

# Every symbol include/gsa_hip.h declares.
EXPORTS = (
    "gsa_abi_version", "gsa_status_string", "gsa_indexer_scores", "gsa_topk_select",
    "gsa_indexer_select", "gsa_prologue", "gsa_sparse_attn", "gsa_prologue_vt",
    "gsa_selection_mask", "gsa_dense_attn", "gsa_dense_attn_workspace_bytes",
    "gsa_indexer_select_workspace_bytes", "gsa_indexer_select_adaptive",
    "gsa_indexer_select_adaptive_workspace_bytes", "gsa_topk_select_adaptive",
    "gsa_proj_packed_bytes", "gsa_proj_pack", "gsa_proj_fused", "gsa_dense_lane_masks",
    "gsa_prologue_vt_lane_masks", "gsa_debug_force_select_fallback",
    "gsa_indexer_select_noalloc", "gsa_indexer_select_noalloc_max_bytes",
)

_vp, _i64, _i32, _f32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_float

_PROTOS = {
    "gsa_abi_version": ([], _i32),
    "gsa_status_string": ([_i32], ctypes.c_char_p),
    "gsa_indexer_scores": ([_vp, _i64, _i64, _vp, _i64, _i64, _vp, _i64, _i64, _vp, _f32,
                            _i32, _i32, _i32, _i32, _i32, _i32, _vp, _i64, _i64, _vp], _i32),
    "gsa_topk_select": ([_vp, _i64, _i64, _i32, _i32, _i32, _i32, _i32, _vp, _vp, _vp, _vp], _i32),
    "gsa_topk_select_adaptive": ([_vp, _i64, _i64, _i32, _i32, _i32, _i32, _i32, _i32, _i32,
                                  _vp, _vp, _vp, _vp, _vp, _vp], _i32),
    "gsa_indexer_select": ([_vp, _i64, _i64, _vp, _i64, _i64, _vp, _i64, _i64, _vp, _f32,
                            _i32, _i32, _i32, _i32, _i32, _i32, _vp, _i64, _i64, _vp, _vp,
                            _vp, ctypes.c_size_t, _vp], _i32),
    "gsa_indexer_select_workspace_bytes": ([_i32, _i32], ctypes.c_size_t),
    "gsa_indexer_select_noalloc": ([_vp, _i64, _i64, _vp, _i64, _i64, _vp, _i64, _i64, _vp, _f32,
                                    _i32, _i32, _i32, _i32, _i32, _i32, _vp, _i64, _i64, _vp, _vp,
                                    _vp], _i32),
    "gsa_indexer_select_noalloc_max_bytes": ([], ctypes.c_size_t),
    "gsa_indexer_select_adaptive": ([_vp, _i64, _i64, _vp, _i64, _i64, _vp, _i64, _i64, _vp, _f32,
                                     _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32,
                                     _vp, _i64, _i64, _vp, _vp, _vp, _vp,
                                     _vp, ctypes.c_size_t, _vp], _i32),
    "gsa_indexer_select_adaptive_workspace_bytes": ([_i32, _i32], ctypes.c_size_t),
    "gsa_debug_force_select_fallback": ([_i32], _i32),
    "gsa_prologue": ([_vp, _i64, _i64, _vp, _i64, _i64, _vp, _i64, _i64, _vp, _vp, _i64,
                      _i32, _i32, _i32, _i32, _i32, _vp, _vp, _vp], _i32),
    "gsa_sparse_attn": ([_vp, _i64, _i64, _vp, _i64, _i64, _vp, _i64, _i64,
                         _vp, _i64, _i64, _i32, _vp, _vp, _vp, _i64, _i64, _vp, _vp, _i64,
                         _vp, _i64, _i64, _i32, _i32, _i32, _i32, _i32, _f32, _i32, _i32, _vp], _i32),
    "gsa_prologue_vt": ([_vp, _i64, _i64, _vp, _i64, _i64, _vp, _i64, _i64, _vp, _vp, _i64,
                         _i32, _i32, _i32, _i32, _i32, _vp, _vp, _i32, _vp], _i32),
    "gsa_selection_mask": ([_vp, _i64, _i64, _i32, _vp, _vp, _i32, _i32, _i32, _vp, _i64, _i64, _vp], _i32),
    "gsa_dense_attn": ([_vp, _i64, _i64, _vp, _i64, _i64, _vp, _i64, _i64, _i32, _vp, _i64, _i64,
                        _vp, _i64, _i64, _vp, _vp, _i64, _vp, _i64, _i64,
                        _i32, _i32, _i32, _i32, _i32, _f32, _i32, _i32, _i32, _vp, ctypes.c_size_t, _vp], _i32),
    "gsa_dense_attn_workspace_bytes": ([_i32, _i32, _i32], ctypes.c_size_t),
    "gsa_proj_packed_bytes": ([_i32, _i32], ctypes.c_size_t),
    "gsa_dense_lane_masks": ([_vp, _i64, _i64, _i32, _i32, _i32, _i32, _vp, ctypes.c_size_t, _vp], _i32),
    "gsa_prologue_vt_lane_masks": ([_vp, _i64, _i64, _vp, _i64, _i64, _vp, _i64, _i64, _vp, _vp, _i64,
                                    _i32, _i32, _i32, _i32, _i32, _vp, _vp, _i32,
                                    _vp, _i64, _i64, _i32, _i32, _vp, ctypes.c_size_t, _vp], _i32),
    "gsa_proj_pack": ([_vp, _i64, _vp, _i32, _i32, _i32, _vp, _vp, _vp], _i32),
    "gsa_proj_fused": ([_vp, _i64, _i32, _i32, _i32, _i32, _i32, _vp, _vp, _vp, _vp, _i64,
                        _vp, _i64, _vp, _i64, _vp, _vp, _i32, _vp], _i32),
}

_lib: Optional[ctypes.CDLL] = None


def load() -> ctypes.CDLL:
    """Load libgsa_hip.so once; raise if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"{LIB_PATH} is missing: build it with `python -m gsa_gdn_benchmarkstudy_amd.build`")
    lib = ctypes.CDLL(LIB_PATH)
    for name, (args, res) in _PROTOS.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    if lib.gsa_abi_version() != ABI_VERSION:
        raise RuntimeError(f"libgsa_hip.so ABI {lib.gsa_abi_version()} != {ABI_VERSION}")
    _lib = lib
    return lib


def status_string(status: int) -> str:
    return load().gsa_status_string(status).decode()


def _check(status: int, what: str) -> None:
    if status != 0:
        raise RuntimeError(f"{what} failed: status {status} ({status_string(status)})")


def dtype_code(dt: torch.dtype) -> int:
    if dt == torch.bfloat16:
        return DTYPE_BF16
    if dt == torch.float32:
        return DTYPE_F32
    raise TypeError(f"unsupported dtype {dt}: the HIP kernels take bfloat16 or float32")


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _need_cuda(*ts: Optional[torch.Tensor]) -> None:
    for t in ts:
        if t is not None and not t.is_cuda:
            raise RuntimeError("the HIP kernels need device tensors (got a CPU tensor)")


def _expect(cond: bool, msg: str) -> None:
    if not cond:
        raise ValueError(msg)


def _rows(t: torch.Tensor, inner: int):
    """(batch stride, row stride) of a [B, T, ...] tensor whose trailing ``inner``
    elements per row are contiguous."""
    flat = 1
    for d in range(t.dim() - 1, 1, -1):
        if t.stride(d) != flat:
            raise ValueError(f"tensor {tuple(t.shape)} strides {t.stride()}: inner dims must be contiguous")
        flat *= t.shape[d]
    if flat != inner:
        raise ValueError(f"tensor {tuple(t.shape)}: expected {inner} elements per row")
    return t.stride(0), t.stride(1)


# ---------------------------------------------------------------------------
# Wrappers
# ---------------------------------------------------------------------------

def indexer_scores(q_idx, k_idx, w, bias32, scale: float, causal: bool = True,
                   out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """fp32 [B,T,T] scores; q_idx [B,T,Hi,di], k_idx [B,T,di], w [B,T,Hi], bias32 fp32 [Hi]."""
    lib = load()
    _need_cuda(q_idx, k_idx, w, bias32)
    B, T, Hi, di = q_idx.shape
    _expect(tuple(k_idx.shape) == (B, T, di), f"k_idx {tuple(k_idx.shape)} != {(B, T, di)}")
    _expect(tuple(w.shape) == (B, T, Hi), f"w {tuple(w.shape)} != {(B, T, Hi)}")
    _expect(bias32.dtype == torch.float32 and bias32.numel() == Hi and bias32.is_contiguous(), "bias: fp32 [Hi]")
    _expect(k_idx.dtype == q_idx.dtype == w.dtype, "q_idx, k_idx, w must share a dtype")
    if out is None:
        out = torch.empty(B, T, T, device=q_idx.device, dtype=torch.float32)
    _expect(tuple(out.shape) == (B, T, T) and out.dtype == torch.float32, "out: fp32 [B,T,T]")
    qs, ks, ws, os_ = _rows(q_idx, Hi * di), _rows(k_idx, di), _rows(w, Hi), _rows(out, T)
    st = lib.gsa_indexer_scores(_ptr(q_idx), *qs, _ptr(k_idx), *ks, _ptr(w), *ws,
                                _ptr(bias32), float(scale), B, T, Hi, di, int(bool(causal)),
                                dtype_code(q_idx.dtype), _ptr(out), *os_, _stream(q_idx))
    _check(st, "gsa_indexer_scores")
    return out


def topk_select(scores: torch.Tensor, k_eff: int, order: int = ORDER_INDEX_ASC,
                want_mask: bool = False):
    """Exact per-row top-k of fp32 scores [B,T,Tkv] -> (idx int32, count int32, mask uint8|None)."""
    lib = load()
    _need_cuda(scores)
    if scores.dtype != torch.float32:
        raise TypeError("scores must be float32")
    _expect(scores.dim() == 3, "scores: [B,T,Tkv]")
    B, T, Tkv = scores.shape
    if scores.stride(2) != 1:
        raise ValueError("scores must have unit column stride")
    idx = torch.empty(B, T, k_eff, device=scores.device, dtype=torch.int32)
    cnt = torch.empty(B, T, device=scores.device, dtype=torch.int32)
    mask = torch.empty(B, T, k_eff, device=scores.device, dtype=torch.uint8) if want_mask else None
    st = lib.gsa_topk_select(_ptr(scores), scores.stride(0), scores.stride(1), B, T, Tkv, int(k_eff),
                             int(order), _ptr(idx), _ptr(cnt), _ptr(mask), _stream(scores))
    _check(st, "gsa_topk_select")
    return idx, cnt, mask


def topk_select_adaptive(scores: torch.Tensor, k_base: int, k_min: int, k_max: int,
                         order: int = ORDER_INDEX_ASC, want_mask: bool = False):
    """Per-row top-k with the variance-based k of fp32 scores [B,T,Tkv] ->
    (idx int32 [B,T,W], count int32 [B,T], mask uint8|None, k int32 [B,T],
    var fp32 [B,T]), W = min(k_max, Tkv)."""
    lib = load()
    _need_cuda(scores)
    if scores.dtype != torch.float32:
        raise TypeError("scores must be float32")
    _expect(scores.dim() == 3, "scores: [B,T,Tkv]")
    B, T, Tkv = scores.shape
    if scores.stride(2) != 1:
        raise ValueError("scores must have unit column stride")
    W = min(int(k_max), Tkv)
    dev = scores.device
    idx = torch.empty(B, T, W, device=dev, dtype=torch.int32)
    cnt = torch.empty(B, T, device=dev, dtype=torch.int32)
    mask = torch.empty(B, T, W, device=dev, dtype=torch.uint8) if want_mask else None
    k_rows = torch.empty(B, T, device=dev, dtype=torch.int32)
    var = torch.empty(B, T, device=dev, dtype=torch.float32)
    st = lib.gsa_topk_select_adaptive(_ptr(scores), scores.stride(0), scores.stride(1), B, T, Tkv,
                                      int(k_base), int(k_min), int(k_max), int(order), _ptr(idx),
                                      _ptr(cnt), _ptr(mask), _ptr(k_rows), _ptr(var), _stream(scores))
    _check(st, "gsa_topk_select_adaptive")
    return idx, cnt, mask, k_rows, var


def indexer_select_workspace_bytes(B: int, T: int) -> int:
    return int(load().gsa_indexer_select_workspace_bytes(B, T))


def indexer_select(q_idx, k_idx, w, bias32, scale: float, k_eff: int, indices: bool = True,
                   bits: Optional[torch.Tensor] = None, ws: Optional[torch.Tensor] = None):
    """Fused indexer + exact top-k.

    Returns (bits, idx, count): the selection bitmask int32 [B,T,W] (W =
    2*ceil(T/64)) and, when ``indices``, ascending int32 indices [B,T,k_eff]
    and counts int32 [B,T] (else None, None).  ``ws``: optional workspace
    (uint8 device tensor of at least indexer_select_workspace_bytes(B, T)).
    """
    lib = load()
    _need_cuda(q_idx, k_idx, w, bias32)
    B, T, Hi, di = q_idx.shape
    _expect(tuple(k_idx.shape) == (B, T, di), f"k_idx {tuple(k_idx.shape)} != {(B, T, di)}")
    _expect(tuple(w.shape) == (B, T, Hi), f"w {tuple(w.shape)} != {(B, T, Hi)}")
    _expect(bias32.dtype == torch.float32 and bias32.numel() == Hi and bias32.is_contiguous(), "bias: fp32 [Hi]")
    _expect(k_idx.dtype == q_idx.dtype == w.dtype, "q_idx, k_idx, w must share a dtype")
    W = mask_words(T)
    if bits is None:
        bits = torch.empty(B, T, W, device=q_idx.device, dtype=torch.int32)
    _expect(tuple(bits.shape) == (B, T, W) and bits.is_contiguous(), "bits: contiguous [B,T,W]")
    idx = cnt = None
    if indices:
        idx = torch.empty(B, T, k_eff, device=q_idx.device, dtype=torch.int32)
        cnt = torch.empty(B, T, device=q_idx.device, dtype=torch.int32)
    nbytes = lib.gsa_indexer_select_workspace_bytes(B, T)
    if ws is None:
        ws = torch.empty(nbytes, device=q_idx.device, dtype=torch.uint8)
    _expect(ws.numel() * ws.element_size() >= nbytes and ws.is_contiguous(), "workspace too small")
    qs, ks, wst = _rows(q_idx, Hi * di), _rows(k_idx, di), _rows(w, Hi)
    st = lib.gsa_indexer_select(_ptr(q_idx), *qs, _ptr(k_idx), *ks, _ptr(w), *wst, _ptr(bias32),
                                float(scale), B, T, Hi, di, int(k_eff), dtype_code(q_idx.dtype),
                                _ptr(bits), bits.stride(0), bits.stride(1), _ptr(idx), _ptr(cnt),
                                _ptr(ws), nbytes, _stream(q_idx))
    _check(st, "gsa_indexer_select")
    return bits, idx, cnt


def indexer_select_noalloc(q_idx, k_idx, w, bias32, scale: float, k_eff: int, bits: torch.Tensor,
                           idx: Optional[torch.Tensor] = None, cnt: Optional[torch.Tensor] = None) -> None:
    """gsa_indexer_select_noalloc: indexer_select into caller-given outputs
    (bits int32 [B,T,W]; optional idx int32 [B,T,k_eff] and cnt int32 [B,T])
    with no workspace -- the library's static device array stands in for it,
    so B * ceil(T/16) is limited (GSA_ERR_SCRATCH beyond).  Allocates nothing."""
    lib = load()
    _need_cuda(q_idx, k_idx, w, bias32, bits, idx, cnt)
    B, T, Hi, di = q_idx.shape
    _expect(tuple(k_idx.shape) == (B, T, di), f"k_idx {tuple(k_idx.shape)} != {(B, T, di)}")
    _expect(tuple(w.shape) == (B, T, Hi), f"w {tuple(w.shape)} != {(B, T, Hi)}")
    _expect(bias32.dtype == torch.float32 and bias32.numel() == Hi and bias32.is_contiguous(), "bias: fp32 [Hi]")
    _expect(k_idx.dtype == q_idx.dtype == w.dtype, "q_idx, k_idx, w must share a dtype")
    _expect(tuple(bits.shape) == (B, T, mask_words(T)) and bits.is_contiguous() and bits.dtype == torch.int32,
            "bits: contiguous int32 [B,T,W]")
    _expect((idx is None) == (cnt is None), "idx and cnt go together")
    if idx is not None:
        _expect(tuple(idx.shape) == (B, T, int(k_eff)) and idx.dtype == torch.int32 and idx.is_contiguous(),
                "idx: contiguous int32 [B,T,k_eff]")
        _expect(tuple(cnt.shape) == (B, T) and cnt.dtype == torch.int32 and cnt.is_contiguous(),
                "cnt: contiguous int32 [B,T]")
    qs, ks, wst = _rows(q_idx, Hi * di), _rows(k_idx, di), _rows(w, Hi)
    st = lib.gsa_indexer_select_noalloc(_ptr(q_idx), *qs, _ptr(k_idx), *ks, _ptr(w), *wst, _ptr(bias32),
                                        float(scale), B, T, Hi, di, int(k_eff), dtype_code(q_idx.dtype),
                                        _ptr(bits), bits.stride(0), bits.stride(1), _ptr(idx), _ptr(cnt),
                                        _stream(q_idx))
    _check(st, "gsa_indexer_select_noalloc")


class forced_select_fallback:
    """Context manager: the fused selector's rows take its exact fallback path
    (gsa_debug_force_select_fallback; a test hook)."""

    def __enter__(self):
        self._prev = load().gsa_debug_force_select_fallback(1)
        return self

    def __exit__(self, *exc):
        load().gsa_debug_force_select_fallback(self._prev)
        return False


def indexer_select_adaptive_workspace_bytes(B: int, T: int) -> int:
    return int(load().gsa_indexer_select_adaptive_workspace_bytes(B, T))


def indexer_select_adaptive(q_idx, k_idx, w, bias32, scale: float, k_base: int, k_min: int,
                            k_max: int, indices: bool = True, bits: Optional[torch.Tensor] = None,
                            ws: Optional[torch.Tensor] = None):
    """Fused indexer + exact top-k with the variance-based per-row k.

    Returns (bits, idx, count, k_rows, var): the selection bitmask int32
    [B,T,W]; when ``indices``, ascending int32 indices [B,T,min(k_max,T)] and
    counts int32 [B,T] (else None, None); the per-row k int32 [B,T] and the
    per-row score variance fp32 [B,T].
    """
    lib = load()
    _need_cuda(q_idx, k_idx, w, bias32)
    B, T, Hi, di = q_idx.shape
    _expect(tuple(k_idx.shape) == (B, T, di), f"k_idx {tuple(k_idx.shape)} != {(B, T, di)}")
    _expect(tuple(w.shape) == (B, T, Hi), f"w {tuple(w.shape)} != {(B, T, Hi)}")
    _expect(bias32.dtype == torch.float32 and bias32.numel() == Hi and bias32.is_contiguous(), "bias: fp32 [Hi]")
    _expect(k_idx.dtype == q_idx.dtype == w.dtype, "q_idx, k_idx, w must share a dtype")
    dev = q_idx.device
    W = mask_words(T)
    if bits is None:
        bits = torch.empty(B, T, W, device=dev, dtype=torch.int32)
    _expect(tuple(bits.shape) == (B, T, W) and bits.is_contiguous(), "bits: contiguous [B,T,W]")
    idx = cnt = None
    if indices:
        idx = torch.empty(B, T, min(int(k_max), T), device=dev, dtype=torch.int32)
        cnt = torch.empty(B, T, device=dev, dtype=torch.int32)
    k_rows = torch.empty(B, T, device=dev, dtype=torch.int32)
    var = torch.empty(B, T, device=dev, dtype=torch.float32)
    nbytes = lib.gsa_indexer_select_adaptive_workspace_bytes(B, T)
    if ws is None:
        ws = torch.empty(nbytes, device=dev, dtype=torch.uint8)
    _expect(ws.numel() * ws.element_size() >= nbytes and ws.is_contiguous(), "workspace too small")
    qs, ks, wst = _rows(q_idx, Hi * di), _rows(k_idx, di), _rows(w, Hi)
    st = lib.gsa_indexer_select_adaptive(
        _ptr(q_idx), *qs, _ptr(k_idx), *ks, _ptr(w), *wst, _ptr(bias32), float(scale), B, T, Hi, di,
        int(k_base), int(k_min), int(k_max), dtype_code(q_idx.dtype),
        _ptr(bits), bits.stride(0), bits.stride(1), _ptr(idx), _ptr(cnt), _ptr(k_rows), _ptr(var),
        _ptr(ws), nbytes, _stream(q_idx))
    _check(st, "gsa_indexer_select_adaptive")
    return bits, idx, cnt, k_rows, var


def prologue(k=None, v=None, vg=None, cos=None, sin=None, k_out=None, v_out=None):
    """RoPE(k) -> k_out and/or v*sigmoid(vg) -> v_out; tensors [B,T,H,d], cos/sin [T,d]."""
    lib = load()
    ref = k if k is not None else v
    _need_cuda(k, v, vg, cos, sin)
    B, T, H, d = ref.shape
    HD = H * d
    for t, nm in ((k, "k"), (v, "v"), (vg, "vg"), (k_out, "k_out"), (v_out, "v_out")):
        if t is not None:
            _expect(tuple(t.shape) == (B, T, H, d) and t.dtype == ref.dtype, f"{nm}: {ref.dtype} [B,T,H,d]")
    if k is not None:
        _expect(cos is not None and sin is not None, "RoPE needs cos and sin")
        _expect(cos.dim() == 2 and cos.shape[0] >= T and cos.shape[1] == d and tuple(sin.shape) == tuple(cos.shape)
                and cos.dtype == sin.dtype == ref.dtype, "cos/sin: [>=T, d] in the tensor dtype")
    if v is not None:
        _expect(vg is not None, "the gate needs its logits")
    if k is not None and k_out is None:
        k_out = torch.empty(B, T, H, d, device=ref.device, dtype=ref.dtype)
    if v is not None and v_out is None:
        v_out = torch.empty(B, T, H, d, device=ref.device, dtype=ref.dtype)
    ks = _rows(k, HD) if k is not None else (0, 0)
    vs = _rows(v, HD) if v is not None else (0, 0)
    gs = _rows(vg, HD) if vg is not None else (0, 0)
    cs = cos.stride(0) if cos is not None else 0
    if cos is not None and (cos.stride(-1) != 1 or sin.stride(0) != cs or sin.stride(-1) != 1):
        raise ValueError("cos/sin must be [T, d] with unit element stride and equal row strides")
    for t in (k_out, v_out):
        if t is not None and not t.is_contiguous():
            raise ValueError("outputs must be contiguous")
    st = lib.gsa_prologue(_ptr(k), *ks, _ptr(v), *vs, _ptr(vg), *gs, _ptr(cos), _ptr(sin), cs,
                          B, T, H, d, dtype_code(ref.dtype), _ptr(k_out), _ptr(v_out), _stream(ref))
    _check(st, "gsa_prologue")
    return k_out, v_out


def sparse_attn(q, k, v, idx, scale: float, count=None, mask=None, og=None, cos=None, sin=None,
                flags: int = 0, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Gather attention -> out [B,T,H,d]; idx int32 [B,T,k_sel] (mask uint8 with the same strides)."""
    lib = load()
    _need_cuda(q, k, v, idx, count, mask, og, cos, sin)
    B, T, H, d = q.shape
    Tkv = k.shape[1]
    HD = H * d
    _expect(k.shape[0] == B and tuple(k.shape[2:]) == (H, d) and tuple(v.shape) == tuple(k.shape),
            "k, v: [B,Tkv,H,d] matching q")
    _expect(k.dtype == v.dtype == q.dtype, "q, k, v must share a dtype")
    _expect(idx.dim() == 3 and tuple(idx.shape[:2]) == (B, T), "idx: [B,T,k_sel]")
    if mask is not None:
        _expect(tuple(mask.shape) == tuple(idx.shape), "mask: idx's shape")
    if count is not None:
        _expect(tuple(count.shape) == (B, T), "count: [B,T]")
    if og is not None:
        _expect(tuple(og.shape) == (B, T, H, d) and og.dtype == q.dtype, "og: [B,T,H,d] in q's dtype")
    if flags & ATTN_ROPE_Q:
        _expect(cos is not None and sin is not None and cos.dim() == 2 and cos.shape[0] >= T
                and cos.shape[1] == d and tuple(sin.shape) == tuple(cos.shape)
                and cos.dtype == sin.dtype == q.dtype and cos.stride(1) == 1 and sin.stride() == cos.stride(),
                "cos/sin: [>=T, d] in q's dtype")
    if out is not None:
        _expect(tuple(out.shape) == (B, T, H, d) and out.dtype == q.dtype, "out: [B,T,H,d] in q's dtype")
    if idx.dtype != torch.int32 or (count is not None and count.dtype != torch.int32):
        raise TypeError("idx and count must be int32")
    if idx.stride(2) != 1:
        raise ValueError("idx must have unit stride along k")
    if mask is not None and (mask.dtype not in (torch.uint8, torch.bool) or mask.stride() != idx.stride()):
        raise ValueError("mask must be uint8/bool with idx's strides")
    if count is not None and not count.is_contiguous():
        raise ValueError("count must be contiguous [B,T]")
    if out is None:
        out = torch.empty(B, T, H, d, device=q.device, dtype=q.dtype)
    os_ = _rows(og, HD) if og is not None else (0, 0)
    cs = cos.stride(0) if cos is not None else 0
    st = lib.gsa_sparse_attn(_ptr(q), *_rows(q, HD), _ptr(k), *_rows(k, HD), _ptr(v), *_rows(v, HD),
                             _ptr(idx), idx.stride(0), idx.stride(1), idx.shape[2],
                             _ptr(count), _ptr(mask), _ptr(og), *os_, _ptr(cos), _ptr(sin), cs,
                             _ptr(out), *_rows(out, HD), B, T, Tkv, H, d, float(scale),
                             dtype_code(q.dtype), int(flags), _stream(q))
    _check(st, "gsa_sparse_attn")
    return out


# ---------------------------------------------------------------------------
# Block-dense attention path
# ---------------------------------------------------------------------------

def vt_len(T: int) -> int:
    """Row length of the transposed V buffer: T rounded up to a multiple of 64."""
    return (T + 63) // 64 * 64


def mask_words(Tkv: int) -> int:
    """uint32 words per row of a selection bitmask."""
    return 2 * ((Tkv + 63) // 64)


def dense_block_rows(Tkv: int) -> int:
    """Query rows per block of gsa_dense_attn (8 waves of 32 rows), whatever the
    key count.  The mask-operand workspace counts whole blocks of this size
    (gsa_dense_attn_workspace_bytes)."""
    return 256


def prologue_vt(v, vg, k=None, cos=None, sin=None, k_out=None, vt=None, bits=None, Tkv=None, ws=None,
                causal: bool = False):
    """RoPE(k) -> k_out [B,T,H,d] and (v*sigmoid(vg))^T -> vt [B,H,d,ldv] (bf16).

    With ``bits`` (the selection bitmask [B,T,W] of keys 0..Tkv-1): the dense
    attention's lane masks are built in the same launch (gsa_prologue_vt_lane_masks)
    into ``ws`` (allocated when None), returned third: (k_out, vt, ws).  ``causal``:
    only the tiles a causal dense_attn reads (the masks then serve causal calls only)."""
    lib = load()
    _need_cuda(k, v, vg, cos, sin, bits, ws)
    B, T, H, d = v.shape
    HD = H * d
    ldv = vt_len(T)
    for t, nm in ((k, "k"), (vg, "vg"), (k_out, "k_out")):
        if t is not None:
            _expect(tuple(t.shape) == (B, T, H, d) and t.dtype == v.dtype, f"{nm}: {v.dtype} [B,T,H,d]")
    if k is not None:
        _expect(cos is not None and sin is not None and cos.dim() == 2 and cos.shape[0] >= T
                and cos.shape[1] == d and tuple(sin.shape) == tuple(cos.shape) and cos.dtype == sin.dtype == v.dtype
                and cos.stride(1) == 1 and sin.stride() == cos.stride(), "cos/sin: [>=T, d] in v's dtype")
        if k_out is None:
            k_out = torch.empty(B, T, H, d, device=v.device, dtype=v.dtype)
        _expect(k_out.is_contiguous(), "k_out must be contiguous")
    if vt is None:
        vt = torch.empty(B, H, d, ldv, device=v.device, dtype=v.dtype)
    _expect(tuple(vt.shape) == (B, H, d, ldv) and vt.is_contiguous() and vt.dtype == v.dtype,
            "vt: contiguous [B,H,d,ldv]")
    ks = _rows(k, HD) if k is not None else (0, 0)
    cs = cos.stride(0) if cos is not None else 0
    if bits is None:
        st = lib.gsa_prologue_vt(_ptr(k), *ks, _ptr(v), *_rows(v, HD), _ptr(vg), *_rows(vg, HD), _ptr(cos),
                                 _ptr(sin), cs, B, T, H, d, dtype_code(v.dtype), _ptr(k_out), _ptr(vt), ldv,
                                 _stream(v))
        _check(st, "gsa_prologue_vt")
        return k_out, vt
    Tkv = T if Tkv is None else Tkv
    _expect(tuple(bits.shape) == (B, T, mask_words(Tkv)) and bits.stride(2) == 1 and bits.dtype == torch.int32,
            "bits: int32 [B,T,W]")
    nbytes = lib.gsa_dense_attn_workspace_bytes(B, T, Tkv)
    if ws is None:
        ws = torch.empty(nbytes, device=v.device, dtype=torch.uint8)
    _expect(ws.numel() * ws.element_size() >= nbytes and ws.is_contiguous(), "workspace too small")
    st = lib.gsa_prologue_vt_lane_masks(_ptr(k), *ks, _ptr(v), *_rows(v, HD), _ptr(vg), *_rows(vg, HD), _ptr(cos),
                                        _ptr(sin), cs, B, T, H, d, dtype_code(v.dtype), _ptr(k_out), _ptr(vt),
                                        ldv, _ptr(bits), bits.stride(0), bits.stride(1), Tkv, int(bool(causal)),
                                        _ptr(ws), nbytes, _stream(v))
    _check(st, "gsa_prologue_vt_lane_masks")
    _tag_masks(ws, causal)
    return k_out, vt, ws


def proj_supported(D: int, H: int, T: int) -> bool:
    """Shapes the fused projection kernel takes: d_head 128, an even head count, T % 64 == 0."""
    return H >= 2 and H <= 64 and D == 128 * H and D % 256 == 0 and T % 64 == 0


def proj_pack(w, bias=None):
    """Packed weight (bf16, flat) and fp32 bias of the fused projection from the q, k, v,
    value-gate and output-gate rows ``w`` [5D, D] (row stride may exceed D) and their bias [5D]."""
    lib = load()
    _need_cuda(w, bias)
    n, D = w.shape
    _expect(n == 5 * D and w.dtype == torch.bfloat16 and w.stride(1) == 1, "w: bf16 [5D, D] with unit column stride")
    H = D // 128
    nbytes = lib.gsa_proj_packed_bytes(D, H)
    _expect(nbytes > 0, f"fused projection: D={D} unsupported (needs D = 128*H, D % 256 == 0)")
    if bias is not None:
        _expect(bias.dim() == 1 and bias.shape[0] >= n and bias.dtype == w.dtype and bias.stride(0) == 1,
                "bias: bf16 [>=5D]")
    wp = torch.empty(nbytes // 2, device=w.device, dtype=torch.bfloat16)
    bp = torch.empty(n, device=w.device, dtype=torch.float32)
    st = lib.gsa_proj_pack(_ptr(w), w.stride(0), _ptr(bias), D, H, DTYPE_BF16, _ptr(wp), _ptr(bp), _stream(w))
    _check(st, "gsa_proj_pack")
    return wp, bp


def proj_fused(x, wp, bp, cos, sin, H: int, q=None, og=None, k_out=None, vt=None):
    """x [B,T,D] -> q, og (bf16 [B,T,H,128] views of one [B,T,2,D] buffer unless given),
    RoPE(k) [B,T,H,128] and (v*sigmoid(vg))^T [B,H,128,ldv], from the packed projection."""
    lib = load()
    _need_cuda(x, wp, bp, cos, sin)
    B, T, D = x.shape
    _expect(x.dtype == torch.bfloat16 and x.stride(2) == 1 and x.stride(0) == T * x.stride(1),
            "x: bf16 [B,T,D] with uniformly strided rows")
    _expect(proj_supported(D, H, T), f"fused projection: D={D} H={H} T={T} unsupported")
    _expect(wp.numel() * 2 == lib.gsa_proj_packed_bytes(D, H) and bp.numel() == 5 * D and bp.dtype == torch.float32,
            "wp/bp: from proj_pack for this D")
    _expect(cos.dim() == 2 and cos.shape[0] >= T and cos.shape[1] == 128 and tuple(sin.shape) == tuple(cos.shape)
            and cos.dtype == sin.dtype == x.dtype and cos.stride(1) == 1 and sin.stride() == cos.stride(),
            "cos/sin: [>=T, 128] bf16")
    dev, dt = x.device, x.dtype
    if q is None or og is None:
        qo = torch.empty(B, T, 2, H, 128, device=dev, dtype=dt)
        q, og = qo[:, :, 0], qo[:, :, 1]
    for t, nm in ((q, "q"), (og, "og")):
        _expect(tuple(t.shape) == (B, T, H, 128) and t.dtype == dt and t.stride(3) == 1 and t.stride(2) == 128
                and t.stride(0) == T * t.stride(1), f"{nm}: [B,T,H,128] with uniformly strided rows")
    if k_out is None:
        k_out = torch.empty(B, T, H, 128, device=dev, dtype=dt)
    _expect(tuple(k_out.shape) == (B, T, H, 128) and k_out.is_contiguous() and k_out.dtype == dt,
            "k_out: contiguous [B,T,H,128]")
    ldv = vt_len(T)
    if vt is None:
        vt = torch.empty(B, H, 128, ldv, device=dev, dtype=dt)
    _expect(tuple(vt.shape) == (B, H, 128, ldv) and vt.is_contiguous() and vt.dtype == dt,
            "vt: contiguous [B,H,128,ldv]")
    st = lib.gsa_proj_fused(_ptr(x), x.stride(1), B, T, D, H, DTYPE_BF16, _ptr(wp), _ptr(bp), _ptr(cos),
                            _ptr(sin), cos.stride(0), _ptr(q), q.stride(1), _ptr(og), og.stride(1),
                            _ptr(k_out), _ptr(vt), ldv, _stream(x))
    _check(st, "gsa_proj_fused")
    return q, og, k_out, vt


def selection_mask(idx, Tkv: int, count=None, mask=None, out=None):
    """uint32 bitmask [B,T,W] of the valid selected keys of every row."""
    lib = load()
    _need_cuda(idx, count, mask)
    B, T, K = idx.shape
    _expect(idx.dtype == torch.int32 and idx.stride(2) == 1, "idx: int32 with unit stride along k")
    if count is not None:
        _expect(tuple(count.shape) == (B, T) and count.dtype == torch.int32 and count.is_contiguous(),
                "count: contiguous int32 [B,T]")
    if mask is not None:
        _expect(tuple(mask.shape) == tuple(idx.shape) and mask.stride() == idx.stride(), "mask: idx's layout")
    W = mask_words(Tkv)
    if out is None:
        out = torch.empty(B, T, W, device=idx.device, dtype=torch.int32)
    _expect(tuple(out.shape) == (B, T, W) and out.is_contiguous(), "bits: contiguous [B,T,W]")
    st = lib.gsa_selection_mask(_ptr(idx), idx.stride(0), idx.stride(1), K, _ptr(count), _ptr(mask),
                                B, T, Tkv, _ptr(out), out.stride(0), out.stride(1), _stream(idx))
    _check(st, "gsa_selection_mask")
    return out


def _tag_masks(ws: torch.Tensor, causal: bool) -> None:
    # Masks built for a causal attention leave the tiles past each query
    # block's last row unwritten: record it on the tensor, so that dense_attn
    # refuses them for a call that reads every tile.
    ws._gsa_causal_masks = bool(causal)


def dense_lane_masks(bits, Tkv: int, ws: Optional[torch.Tensor] = None, causal: bool = False) -> torch.Tensor:
    """Mask operands of the dense attention from the selection bitmask [B,T,W] -> the
    workspace tensor holding them (pass it to dense_attn with masks_ready=True).
    ``causal``: only the tiles a causal dense_attn reads, up to the last row of each
    query block (such masks serve causal calls only); otherwise every tile."""
    lib = load()
    _need_cuda(bits, ws)
    B, T, W = bits.shape
    _expect(W == mask_words(Tkv) and bits.stride(2) == 1 and bits.dtype == torch.int32, "bits: int32 [B,T,W]")
    nbytes = lib.gsa_dense_attn_workspace_bytes(B, T, Tkv)
    if ws is None:
        ws = torch.empty(nbytes, device=bits.device, dtype=torch.uint8)
    _expect(ws.numel() * ws.element_size() >= nbytes and ws.is_contiguous(), "workspace too small")
    st = lib.gsa_dense_lane_masks(_ptr(bits), bits.stride(0), bits.stride(1), B, T, Tkv, int(bool(causal)),
                                  _ptr(ws), nbytes, _stream(bits))
    _check(st, "gsa_dense_lane_masks")
    _tag_masks(ws, causal)
    return ws


def dense_attn(q, k, vt, bits, scale: float, og=None, cos=None, sin=None, flags: int = 0,
               causal: bool = True, out: Optional[torch.Tensor] = None,
               ws: Optional[torch.Tensor] = None, masks_ready: bool = False) -> torch.Tensor:
    """Block-dense masked attention -> out [B,T,H,d] (bf16).  ``ws``: optional
    workspace (uint8 device tensor of at least dense_attn_workspace_bytes);
    ``masks_ready``: ws already holds dense_lane_masks(bits) (bits is then not read)."""
    lib = load()
    _need_cuda(q, k, vt, bits, og, cos, sin)
    B, T, H, d = q.shape
    Tkv = k.shape[1]
    HD = H * d
    _expect(k.shape[0] == B and tuple(k.shape[2:]) == (H, d) and k.dtype == q.dtype, "k: [B,Tkv,H,d]")
    _expect(vt.dim() == 4 and tuple(vt.shape[:3]) == (B, H, d) and vt.shape[3] >= vt_len(Tkv)
            and vt.stride(3) == 1 and vt.stride(2) == vt.shape[3] and vt.dtype == q.dtype,
            "vt: [B,H,d,ldv] rows of ldv >= Tkv rounded up to 64")
    _expect(tuple(bits.shape) == (B, T, mask_words(Tkv)) and bits.stride(2) == 1, "bits: [B,T,W]")
    _expect(not masks_ready or ws is not None, "masks_ready needs the workspace that holds the masks")
    _expect(not (masks_ready and not causal and getattr(ws, "_gsa_causal_masks", False)),
            "masks_ready: these masks were built for a causal attention (tiles past each query block are "
            "unwritten) and cannot serve a non-causal call")
    if og is not None:
        _expect(tuple(og.shape) == (B, T, H, d) and og.dtype == q.dtype, "og: [B,T,H,d] in q's dtype")
    _expect(not (flags & ATTN_ROPE_HALVES) or flags & ATTN_ROPE_Q, "ATTN_ROPE_HALVES goes with ATTN_ROPE_Q")
    if flags & ATTN_ROPE_HALVES:
        # cos: packed [>=T, d] rows of cos[:d/2] then sin[:d/2]; sin is not read
        _expect(cos is not None and cos.dim() == 2 and cos.shape[0] >= T and cos.shape[1] == d
                and cos.dtype == q.dtype and cos.stride(1) == 1, "cos: packed [>=T, d] cos|sin table in q's dtype")
        sin = None
    elif flags & ATTN_ROPE_Q:
        _expect(cos is not None and sin is not None and cos.dim() == 2 and cos.shape[0] >= T
                and cos.shape[1] == d and tuple(sin.shape) == tuple(cos.shape)
                and cos.dtype == sin.dtype == q.dtype and cos.stride(1) == 1 and sin.stride() == cos.stride(),
                "cos/sin: [>=T, d] in q's dtype")
    if out is None:
        out = torch.empty(B, T, H, d, device=q.device, dtype=q.dtype)
    _expect(tuple(out.shape) == (B, T, H, d) and out.dtype == q.dtype, "out: [B,T,H,d] in q's dtype")
    nbytes = lib.gsa_dense_attn_workspace_bytes(B, T, Tkv)
    if ws is None:
        ws = torch.empty(nbytes, device=q.device, dtype=torch.uint8)
    _expect(ws.numel() * ws.element_size() >= nbytes and ws.is_contiguous(), "workspace too small")
    os_ = _rows(og, HD) if og is not None else (0, 0)
    cs = cos.stride(0) if cos is not None else 0
    st = lib.gsa_dense_attn(_ptr(q), *_rows(q, HD), _ptr(k), *_rows(k, HD), _ptr(vt), vt.stride(0),
                            vt.stride(1), vt.shape[3], _ptr(bits), bits.stride(0), bits.stride(1),
                            _ptr(og), *os_, _ptr(cos), _ptr(sin), cs, _ptr(out), *_rows(out, HD),
                            B, T, Tkv, H, d, float(scale), dtype_code(q.dtype),
                            int(flags) | (ATTN_MASKS_READY if masks_ready else 0), int(bool(causal)),
                            _ptr(ws), nbytes, _stream(q))
    _check(st, "gsa_dense_attn")
    return out
