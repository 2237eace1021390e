"""Benchmark harness for the GSA layer forward on MI355X: verify, sweep, trace, counters.

    python -m gsa_gdn_benchmarkstudy_amd.harness [--ref gsa_ref.py] [options]

The user-facing workflow of the reference's gsa_triton/benchmark.py, on
rocprofv3 and ROCTx instead of Nsight:

- verify (gsa_triton/benchmark.py:101-145): a reference layer and the HIP
  layer with the same weights and the same input, compared elementwise (max and
  mean |diff|, ``allclose`` at --atol/--rtol).  A mismatch ends the run with exit
  status 1 before any timing.
- sweep (:150-222): ms per forward, tokens/s and peak device memory for each
  (B, T, D) point.  A point that runs out of device memory is an ``OOM`` row, any
  other failure an ``ERR`` row; the sweep goes on with the next point.
- summary (:227-272): speedup and memory ratio per point, when a reference layer
  was swept too.
- ``--profile`` (:277-349, the Nsight Systems mode): warm-up outside the capture
  window, then PROFILE_ITERS forward passes per layer, each in its own ROCTx
  range, inside roctxProfilerResume/Pause, for
  ``rocprofv3 --kernel-trace --marker-trace --selected-regions --stats -- python -m ...``.
- ``--ncu``/``--counters`` (:354-436, the Nsight Compute mode): ONE forward pass
  per layer inside the window, for ``rocprofv3 --pmc ... --selected-regions``
  counter passes.

The reference layer is the caller's: ``--ref`` names a Python file or module
defining ``GatedSparseAttention`` with the reference constructor and state-dict
keys (the reference repository's ``gsa_triton/gsa_ref.py`` is one).  Without
``--ref`` only the HIP layer is swept and the verification is skipped, which
the output says.

Weights follow the reference harness: the reference layer is built under a fixed
``torch.manual_seed`` with its default initialisation and its state dict is
loaded into the HIP layer (strict); ``fuse_projections()`` is called on any
layer that has it.  Input x ~ N(0, 1).
"""

from __future__ import annotations

import argparse
import gc
import importlib
import importlib.util
import json
import math
import os
import sys
import time
from dataclasses import asdict, dataclass
from typing import Callable, Dict, List, Optional, Sequence, Tuple

import torch

from . import roctx

# Layer hyper-parameters of the reference sweep (gsa_triton/benchmark.py:82-90).
GSA_KWARGS = dict(hidden_size=2048, num_heads=16, k_max=4096, d_indexer=64,
                  n_idx_heads=4, k_base=2048, k_min=256)
WARMUP_ITERS = 5     # gsa_triton/benchmark.py:93
BENCH_ITERS = 10     # gsa_triton/benchmark.py:94
PROFILE_ITERS = 3    # gsa_triton/benchmark.py:95

# The reference sweeps B=1, D=2048 over T = 512 ... 262144 (gsa_triton/benchmark.py:70-80).
# This harness stops at 65536 by default, the longest sequence its GPU tests
# cover; --T reaches further.
DEFAULT_T = (512, 1024, 2048, 4096, 8192, 16384, 32768, 65536)

OK, OOM, ERR = "ok", "OOM", "ERR"


@dataclass
class Row:
    """One sweep point.  ``ms``/``tok_per_s``/``mem_mb`` are None unless status is ok."""

    B: int
    T: int
    D: int
    status: str = OK
    ms: Optional[float] = None
    tok_per_s: Optional[float] = None
    mem_mb: Optional[float] = None
    error: str = ""

    @property
    def key(self) -> Tuple[int, int, int]:
        return (self.B, self.T, self.D)


# ---------------------------------------------------------------------------
# Layers
# ---------------------------------------------------------------------------

def layer_kwargs(T: int, D: int = GSA_KWARGS["hidden_size"]) -> Dict[str, int]:
    """Constructor arguments at sequence length T: k_max clipped to T
    (gsa_triton/benchmark.py:116,168)."""
    kw = dict(GSA_KWARGS)
    kw["hidden_size"] = D
    kw["k_max"] = min(GSA_KWARGS["k_max"], T)
    return kw


def load_layer_class(spec: str):
    """``GatedSparseAttention`` from a Python file path or an importable module name.

    A file's own directory goes on ``sys.path`` first, so a module that imports its
    siblings (as the reference's do) loads as it would from its own folder.
    """
    if spec.endswith(".py") or os.sep in spec:
        path = os.path.abspath(spec)
        if not os.path.isfile(path):
            raise FileNotFoundError(f"--ref {spec!r}: no such file")
        folder = os.path.dirname(path)
        if folder not in sys.path:
            sys.path.insert(0, folder)
        name = "_gsa_ref_" + os.path.splitext(os.path.basename(path))[0]
        mspec = importlib.util.spec_from_file_location(name, path)
        mod = importlib.util.module_from_spec(mspec)
        sys.modules[name] = mod
        mspec.loader.exec_module(mod)
    else:
        mod = importlib.import_module(spec)
    cls = getattr(mod, "GatedSparseAttention", None)
    if cls is None:
        raise AttributeError(f"--ref {spec!r} defines no GatedSparseAttention")
    return cls


def build_layer(cls, kwargs: Dict[str, int], device, dtype, attn_impl: Optional[str] = None,
                state: Optional[Dict[str, torch.Tensor]] = None):
    """Instantiate, move, optionally load ``state`` (strict) and fuse projections."""
    m = cls(**kwargs).to(device).to(dtype).eval()
    if state is not None:
        m.load_state_dict(state, strict=True)
    if attn_impl is not None and hasattr(m, "attn_impl"):
        m.attn_impl = attn_impl
    if hasattr(m, "fuse_projections"):
        m.fuse_projections()
    return m


def this_build_layer():
    from .gsa import GatedSparseAttention

    return GatedSparseAttention


# ---------------------------------------------------------------------------
# Failure classification and timing
# ---------------------------------------------------------------------------

def classify_failure(exc: BaseException) -> str:
    """OOM for a device-memory exhaustion (torch's OutOfMemoryError or an
    "out of memory" message, as gsa_triton/benchmark.py:207 matches), else ERR."""
    oom_type = getattr(torch, "OutOfMemoryError", None)
    if oom_type is not None and isinstance(exc, oom_type):
        return OOM
    return OOM if "out of memory" in str(exc).lower() else ERR


def _release(device) -> None:
    gc.collect()
    if torch.device(device).type == "cuda":
        torch.cuda.empty_cache()


def event_timer(fn: Callable[[], object], iters: int, device) -> float:
    """Mean ms per call of ``fn`` over ``iters`` calls, from HIP events on the
    current stream, bracketed by device synchronisation."""
    torch.cuda.synchronize(device)
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(iters):
        fn()
    end.record()
    torch.cuda.synchronize(device)
    return start.elapsed_time(end) / iters


def wall_timer(fn: Callable[[], object], iters: int, device) -> float:
    """Mean ms per call from the host clock (host-only layers)."""
    t0 = time.perf_counter()
    for _ in range(iters):
        fn()
    return (time.perf_counter() - t0) * 1e3 / iters


def _peak_reset(device) -> None:
    if torch.device(device).type == "cuda":
        torch.cuda.reset_peak_memory_stats(device)


def _peak_mb(device) -> Optional[float]:
    if torch.device(device).type == "cuda":
        return torch.cuda.max_memory_allocated(device) / float(1 << 20)
    return None


# ---------------------------------------------------------------------------
# Verify
# ---------------------------------------------------------------------------

@dataclass
class VerifyResult:
    T: int
    dtype: str
    max_diff: float
    mean_diff: float
    rel_l2: float
    atol: float
    rtol: float
    passed: bool


def verify(ref_cls, opt_cls, device, dtype: torch.dtype, T: int, atol: float, rtol: float,
           B: int = 1, seed: int = 42, attn_impl: Optional[str] = None,
           out: Callable[[str], None] = print) -> VerifyResult:
    """Reference and candidate layer on the same weights and input
    (gsa_triton/benchmark.py:101-145).  k_max is clipped to T, so at the default
    T=512 every row attends to all of its causal keys (k_eff = T)."""
    out(f"\n{'=' * 60}\n  Numerical verification (T={T}, dtype={dtype})\n{'=' * 60}")
    torch.manual_seed(seed)
    kw = layer_kwargs(T)
    ref = build_layer(ref_cls, kw, device, dtype)
    opt = build_layer(opt_cls, kw, device, dtype, attn_impl=attn_impl, state=ref.state_dict())
    x = torch.randn(B, T, kw["hidden_size"], device=device, dtype=dtype)
    with torch.no_grad():
        r = ref(x).float()
        o = opt(x).float()
    diff = (r - o).abs()
    res = VerifyResult(T=T, dtype=str(dtype).replace("torch.", ""),
                       max_diff=diff.max().item(), mean_diff=diff.mean().item(),
                       rel_l2=(diff.norm() / r.norm().clamp_min(1e-30)).item(), atol=atol, rtol=rtol,
                       passed=bool(torch.allclose(r, o, atol=atol, rtol=rtol))
                       and bool(torch.isfinite(o).all()))
    out(f"  max  |ref - opt|: {res.max_diff:.6f}")
    out(f"  mean |ref - opt|: {res.mean_diff:.6f}")
    out(f"  ||ref - opt|| / ||ref||: {res.rel_l2:.3e}")
    out(f"  atol={atol}, rtol={rtol}")
    out(f"  result: {'PASS' if res.passed else 'FAIL'}")
    del ref, opt, x, r, o, diff
    _release(device)
    return res


# ---------------------------------------------------------------------------
# Sweep and summary
# ---------------------------------------------------------------------------

def format_row(r: Row) -> str:
    head = f"{r.B:<5} {r.T:<7} {r.D:<6}"
    if r.status == OK:
        return f"{head} | {r.ms:>9.3f} | {r.tok_per_s:>14,.0f} | {r.mem_mb if r.mem_mb is not None else 0:>9.0f}"
    tail = r.error[:72] if r.status == ERR else "-"
    return f"{head} | {r.status:>9} | {'-':>14} | {tail}"


def sweep(cls, label: str, points: Sequence[Tuple[int, int, int]], device, dtype: torch.dtype,
          warmup: int = WARMUP_ITERS, iters: int = BENCH_ITERS, attn_impl: Optional[str] = None,
          seed: int = 0, timer: Callable = event_timer, graph: bool = False,
          out: Callable[[str], None] = print) -> List[Row]:
    """Time ``cls`` at every (B, T, D) point (gsa_triton/benchmark.py:150-222).

    graph: time replays of a HIP graph of the forward (GraphedForward) instead of
    eager forwards (the HIP layer only)."""
    out(f"\n{'=' * 60}\n  {label}\n{'=' * 60}")
    out(f"{'B':<5} {'T':<7} {'D':<6} | {'ms':>9} | {'tok/s':>14} | {'MB':>9}")
    out("-" * 60)
    rows = []
    for B, T, D in points:
        _release(device)
        _peak_reset(device)
        row = Row(B, T, D)
        model = x = None
        try:
            torch.manual_seed(seed)
            model = build_layer(cls, layer_kwargs(T, D), device, dtype, attn_impl=attn_impl)
            x = torch.randn(B, T, D, device=device, dtype=dtype)
            with torch.no_grad():
                for _ in range(warmup):
                    model(x)
                fn = (lambda: model(x))
                if graph:
                    from .graph import GraphedForward
                    fn = GraphedForward(model, x, warmup=1)
                    fx = fn
                    fn = (lambda: fx(x))
                ms = timer(fn, iters, device)
            row.ms, row.tok_per_s, row.mem_mb = ms, B * T / (ms / 1e3), _peak_mb(device)
        except Exception as exc:  # every failure becomes a row; the sweep goes on
            row.status = classify_failure(exc)
            row.error = f"{type(exc).__name__}: {exc}".replace("\n", " ")
        out(format_row(row))
        rows.append(row)
        del model, x
    _release(device)
    return rows


def _ratio(num: Optional[float], den: Optional[float]) -> Optional[float]:
    if num is None or den is None or den <= 0 or not math.isfinite(num) or not math.isfinite(den):
        return None
    return num / den


def summary_lines(ref_rows: Sequence[Row], opt_rows: Sequence[Row]) -> List[str]:
    """Per point: ref/opt ms, speedup = ref_ms/opt_ms, ref/opt MB, memory
    saving = ref_MB/opt_MB (gsa_triton/benchmark.py:227-272).  Points are paired
    by (B, T, D); a failed side prints its status and the ratios print N/A."""
    ref_by = {r.key: r for r in ref_rows}
    lines = [
        "=" * 78,
        "  Summary: speedup and memory reduction",
        "=" * 78,
        f"{'B':<3} {'T':<7} | {'ref ms':>9} | {'opt ms':>9} | {'speedup':>8} | "
        f"{'ref MB':>8} | {'opt MB':>8} | {'mem save':>8}",
        "-" * 78,
    ]

    def ms(r: Optional[Row]) -> str:
        if r is None:
            return "-"
        return f"{r.ms:.2f}" if r.status == OK else r.status

    def mb(r: Optional[Row]) -> str:
        return f"{r.mem_mb:.0f}" if r is not None and r.status == OK and r.mem_mb is not None else "-"

    for o in opt_rows:
        r = ref_by.get(o.key)
        sp = _ratio(r.ms, o.ms) if r is not None and r.status == OK and o.status == OK else None
        ms_save = (_ratio(r.mem_mb, o.mem_mb)
                   if r is not None and r.status == OK and o.status == OK else None)
        lines.append(
            f"{o.B:<3} {o.T:<7} | {ms(r):>9} | {ms(o):>9} | "
            f"{(f'{sp:.2f}x' if sp is not None else 'N/A'):>8} | {mb(r):>8} | {mb(o):>8} | "
            f"{(f'{ms_save:.2f}x' if ms_save is not None else 'N/A'):>8}")
    return lines


# ---------------------------------------------------------------------------
# Profiler capture windows
# ---------------------------------------------------------------------------

def capture(ref_cls, opt_cls, device, dtype: torch.dtype, B: int, T: int, iters: int,
            tag: str, warmup: int = WARMUP_ITERS, attn_impl: Optional[str] = None,
            out: Callable[[str], None] = print) -> List[str]:
    """Warm up, then run ``iters`` forward passes of each given layer inside the
    rocprofv3 capture window, each pass in a ROCTx range named
    ``<tag>/<layer>/iter<i>``.  Either class may be None (the ``-only`` flags).
    Returns the range names, in order."""
    kw = layer_kwargs(T)
    D = kw["hidden_size"]
    torch.manual_seed(0)
    ref = build_layer(ref_cls, kw, device, dtype) if ref_cls is not None else None
    opt = None
    if opt_cls is not None:
        opt = build_layer(opt_cls, kw, device, dtype, attn_impl=attn_impl,
                          state=ref.state_dict() if ref is not None else None)
    x = torch.randn(B, T, D, device=device, dtype=dtype)
    layers = [(n, m) for n, m in (("gsa_ref", ref), ("gsa_hip", opt)) if m is not None]
    out(f"  [{'+'.join(n for n, _ in layers)}] B={B} T={T} D={D} dtype={dtype}: "
        f"warm-up {warmup} iters each")
    with torch.no_grad():
        for _ in range(warmup):
            for _, m in layers:
                m(x)
    torch.cuda.synchronize(device)
    names = []
    out(f"  roctxProfilerResume: capturing {iters} forward pass(es) per layer")
    roctx.profiler_resume()
    try:
        with torch.no_grad():
            for n, m in layers:
                for i in range(iters):
                    name = f"{tag}/{n}/iter{i}"
                    with roctx.region(name):
                        m(x)
                    names.append(name)
                torch.cuda.synchronize(device)
    finally:
        roctx.profiler_pause()
    out("  roctxProfilerPause: capture window closed")
    del ref, opt, x
    _release(device)
    return names


# ---------------------------------------------------------------------------
# CLI
# ---------------------------------------------------------------------------

def _int_list(text: str) -> List[int]:
    return [int(v) for v in text.replace(",", " ").split()]


def parse_args(argv: Optional[Sequence[str]] = None) -> argparse.Namespace:
    p = argparse.ArgumentParser(
        prog="python -m gsa_gdn_benchmarkstudy_amd.harness",
        description="GSA layer forward on MI355X: verify against a reference layer, sweep "
                    "sequence lengths, or open a rocprofv3 capture window.")
    p.add_argument("--ref", default=None,
                   help="Python file or module defining the reference GatedSparseAttention "
                        "(e.g. gsa_triton/gsa_ref.py); without it only the HIP layer is swept")
    p.add_argument("--skip-verify", action="store_true", help="skip numerical verification")
    p.add_argument("--verify-T", type=int, default=512, help="sequence length of the verification")
    p.add_argument("--dtype", choices=["bf16", "fp32"], default="bf16")
    p.add_argument("--atol", type=float, default=None,
                   help="absolute tolerance (default 2e-2 for bf16, 1e-4 for fp32)")
    p.add_argument("--rtol", type=float, default=None,
                   help="relative tolerance (default 1e-2 for bf16, 1e-4 for fp32)")
    p.add_argument("--B", type=int, default=1, help="batch of every sweep point")
    p.add_argument("--T", type=_int_list, default=list(DEFAULT_T),
                   help="sequence lengths of the sweep, comma separated")
    p.add_argument("--warmup", type=int, default=WARMUP_ITERS)
    p.add_argument("--iters", type=int, default=BENCH_ITERS)
    p.add_argument("--attn", choices=["auto", "dense", "gather"], default="auto",
                   help="attention kernel of the HIP layer")
    p.add_argument("--graph", action="store_true",
                   help="time HIP-graph replays of the HIP layer's forward (one launch per forward)")
    p.add_argument("--json", default=None, help="also write the results to this JSON file")
    # capture windows: the reference's --profile / --ncu flags, same names
    p.add_argument("--profile", action="store_true",
                   help="capture window of PROFILE_ITERS passes per layer for "
                        "rocprofv3 --selected-regions (kernel/marker traces)")
    p.add_argument("--profile-B", type=int, default=1)
    p.add_argument("--profile-T", type=int, default=2048)
    p.add_argument("--profile-ref-only", action="store_true")
    p.add_argument("--profile-opt-only", action="store_true")
    p.add_argument("--counters", "--ncu", dest="counters", action="store_true",
                   help="capture window of ONE pass per layer for rocprofv3 --pmc passes")
    p.add_argument("--counters-B", "--ncu-B", dest="counters_B", type=int, default=1)
    p.add_argument("--counters-T", "--ncu-T", dest="counters_T", type=int, default=2048)
    p.add_argument("--counters-ref-only", "--ncu-ref-only", dest="counters_ref_only",
                   action="store_true")
    p.add_argument("--counters-opt-only", "--ncu-opt-only", dest="counters_opt_only",
                   action="store_true")
    a = p.parse_args(argv)
    fp32 = a.dtype == "fp32"
    if a.atol is None:
        a.atol = 1e-4 if fp32 else 2e-2
    if a.rtol is None:
        a.rtol = 1e-4 if fp32 else 1e-2
    if a.profile_ref_only and a.profile_opt_only:
        p.error("--profile-ref-only and --profile-opt-only exclude each other")
    if a.counters_ref_only and a.counters_opt_only:
        p.error("--counters-ref-only and --counters-opt-only exclude each other")
    if any(t < 1 for t in a.T) or a.B < 1:
        p.error("--B and every --T must be positive")
    return a


def _pick(ref_cls, opt_cls, ref_only: bool, opt_only: bool):
    if ref_only:
        if ref_cls is None:
            raise SystemExit("a -ref-only capture needs --ref")
        return ref_cls, None
    return (None if opt_only else ref_cls), opt_cls


def main(argv: Optional[Sequence[str]] = None, out: Callable[[str], None] = print) -> int:
    a = parse_args(argv)
    if not torch.cuda.is_available():
        out("ERROR: a GPU is required (this layer runs HIP kernels on gfx950).")
        return 1
    device = torch.device("cuda:0")
    dtype = torch.float32 if a.dtype == "fp32" else torch.bfloat16
    out(f"Device: {torch.cuda.get_device_name(device)}")
    out(f"Dtype:  {dtype}")
    ref_cls = load_layer_class(a.ref) if a.ref else None
    opt_cls = this_build_layer()
    attn = None if a.attn == "auto" else a.attn

    if a.profile or a.counters:
        if a.profile:
            r, o = _pick(ref_cls, opt_cls, a.profile_ref_only, a.profile_opt_only)
            B, T, iters, tag = a.profile_B, a.profile_T, PROFILE_ITERS, "profile"
            out("  run under: rocprofv3 --kernel-trace --marker-trace --selected-regions "
                "--stats -d <dir> -- python -m gsa_gdn_benchmarkstudy_amd.harness --profile ...")
        else:
            r, o = _pick(ref_cls, opt_cls, a.counters_ref_only, a.counters_opt_only)
            B, T, iters, tag = a.counters_B, a.counters_T, 1, "counters"
            out("  run under: rocprofv3 --pmc <counters> --selected-regions -d <dir> "
                "-- python -m gsa_gdn_benchmarkstudy_amd.harness --counters ...")
        capture(r, o, device, dtype, B, T, iters, tag, warmup=a.warmup, attn_impl=attn, out=out)
        return 0

    report: Dict[str, object] = {"device": torch.cuda.get_device_name(device), "dtype": a.dtype,
                                 "graph": a.graph}
    if a.skip_verify:
        report["verify"] = "skipped"
    elif ref_cls is None:
        out("\n  verification skipped: no reference layer given (--ref)")
        report["verify"] = "no reference"
    else:
        res = verify(ref_cls, opt_cls, device, dtype, a.verify_T, a.atol, a.rtol,
                     attn_impl=attn, out=out)
        report["verify"] = asdict(res)
        if not res.passed:
            out("\nFATAL: numerical mismatch; benchmark aborted.")
            if a.json:
                _write_json(a.json, report)
            return 1

    out("\n" + "#" * 60 + "\n#  Throughput and memory\n" + "#" * 60)
    points = [(a.B, T, GSA_KWARGS["hidden_size"]) for T in a.T]
    ref_rows: List[Row] = []
    if ref_cls is not None:
        ref_rows = sweep(ref_cls, "reference layer (--ref)", points, device, dtype,
                         warmup=a.warmup, iters=a.iters, out=out)
    opt_rows = sweep(opt_cls, "gsa_hip (MI355X HIP kernels)" + (", HIP graph" if a.graph else ""), points,
                     device, dtype, warmup=a.warmup, iters=a.iters, attn_impl=attn, graph=a.graph, out=out)
    if ref_rows:
        for line in summary_lines(ref_rows, opt_rows):
            out(line)
    report["ref"] = [asdict(r) for r in ref_rows]
    report["opt"] = [asdict(r) for r in opt_rows]
    if a.json:
        _write_json(a.json, report)
    return 0


def _write_json(path: str, report: Dict[str, object]) -> None:
    folder = os.path.dirname(os.path.abspath(path))
    os.makedirs(folder, exist_ok=True)
    with open(path, "w") as f:
        json.dump(report, f, indent=1)


if __name__ == "__main__":
    sys.exit(main())
