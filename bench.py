"""Benchmark: GSA layer forward tokens/s on one MI355X, with the sparse-attention
roofline and the CPU oracle timed beside it.

python bench.py [--gpus 1] [--steps K] [--warmup W] [--config c3] [--cpu-seconds S]

One step = one GatedSparseAttention forward over one batch of synthetic input
already resident in HBM (fused projection GEMM, fused indexer + exact top-k,
RoPE/gate producer, sparse attention with the output gate, o_proj), with the
module's default attention kernel (block-dense MFMA for bf16).  The gather
attention kernel is timed on the same layer and input for its HBM roofline.
Prints ONE JSON line.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "GSA fwd tokens/sec @T=16384 bf16, 1 MI355X; indexer MFMA% + attn HBM GB/s%"
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0

# (B, T) per config; every config: D=2048, H=16, d=128, H_idx=4, d_idx=64, k_base=2048, k_max=4096
CONFIGS = {"c2": (1, 4096), "c3": (1, 16384), "c4": (4, 8192), "c5": (1, 65536)}
D, H, DH, HI, DI = 2048, 16, 128, 4, 64
K_BASE, K_MIN, K_MAX = 2048, 256, 4096


def synthetic_model(dev, dtype, seed=0):
    """Random-init GSA layer: weights N(0, 0.02), gate biases 0.5, indexer biases 0."""
    from gsa_gdn_benchmarkstudy_amd import GatedSparseAttention

    m = GatedSparseAttention(D, H, k_max=K_MAX, d_indexer=DI, n_idx_heads=HI, k_base=K_BASE, k_min=K_MIN)
    g = torch.Generator(device="cpu").manual_seed(seed)
    with torch.no_grad():
        for name, p in m.named_parameters():
            if name.endswith("gate_proj.bias"):
                p.fill_(0.5)
            elif name.endswith("bias"):
                p.zero_()
            else:
                p.copy_(torch.randn(p.shape, generator=g) * 0.02)
    m = m.to(dev).to(dtype).eval()
    m.fuse_projections()
    return m


def attn_bytes(B, T, k_eff, s=2, P=None):
    """Algorithmic bytes of one sparse-attention launch: gathered K+V rows of the
    valid selected entries, their int32 indices, the q read and out write, and
    the output-gate logits.  P = number of valid (row, key) pairs, by default
    B * sum_t min(t+1, k_eff)."""
    if P is None:
        P = B * sum(min(t + 1, k_eff) for t in range(T))
    return P * H * DH * 2 * s + 4 * P + 2 * B * T * H * DH * s + B * T * D * s, P


def indexer_flops(B, T):
    """Causal indexer MACs x2: every (i, j <= i) pair, 4 heads of 64."""
    return 2 * B * HI * DI * T * (T + 1) // 2


KERNEL_SOURCES = {"gsa_dense_attn": "dense_attn.hip", "gsa_indexer_select": "indexer.hip",
                  "gsa_sparse_attn": "sparse_attn.hip"}


def source_digest(kernel):
    """First 12 hex digits of the SHA-256 of the HIP source file that holds `kernel`."""
    import hashlib
    path = os.path.join(ROOT, "gsa_gdn_benchmarkstudy_amd", "csrc", KERNEL_SOURCES[kernel])
    with open(path, "rb") as f:
        return hashlib.sha256(f.read()).hexdigest()[:12]


def profiled_traffic(kernel, config):
    """HBM-side bytes per launch of `kernel` at `config` from the committed rocprofv3
    PMC summaries (FETCH_SIZE and WRITE_SIZE scaled by a plain-copy calibration):
    {"bytes", "source", "kernel_source", "measured_on_source", "source_matches"}, or
    None.  A summary line reads `traffic_bytes <kernel> <config> <bytes> [src=<file>@<sha12>]`;
    `source_matches` says whether the kernel's source file still has the digest that
    the counters were taken on (False: the figure predates a kernel change)."""
    pdir = os.path.join(ROOT, "profiles")
    try:
        names = sorted(f for f in os.listdir(pdir) if f.endswith("_pmc.md"))
    except OSError:
        return None
    for name in names:
        for line in open(os.path.join(pdir, name)):
            f = line.split()
            if len(f) in (4, 5) and f[0] == "traffic_bytes" and f[1] == kernel and f[2] == config:
                src = f[4][4:] if len(f) == 5 and f[4].startswith("src=") else None
                cur = f"{KERNEL_SOURCES[kernel]}@{source_digest(kernel)}"
                return {"bytes": int(f[3]), "source": f"profiles/{name}", "kernel_source": cur,
                        "measured_on_source": src, "source_matches": src == cur}
    return None


def cpu_c1_unchunked(reps=3):
    """The CPU oracle's unchunked fp32 forward at the reference's own CPU case
    (B=1, T=512, k_base=256, k_min=64, k_max=512): gsa_ref.py's op sequence,
    1 warm-up + `reps` timed forwards, as gsa_triton/benchmark.py:179-197 times
    its GPU runs."""
    from oracle import gsa_oracle as orc

    cfg = orc.GSAConfig(hidden_size=D, num_heads=H, k_max=512, d_indexer=DI, n_idx_heads=HI,
                        k_base=256, k_min=64)
    sd = orc.synthetic_state(cfg, seed=0)
    x = orc.synthetic_input(1, 512, D, seed=1)
    with torch.inference_mode():
        orc.gsa_forward(sd, cfg, x)
        t0 = time.perf_counter()
        for _ in range(reps):
            orc.gsa_forward(sd, cfg, x)
        sec = (time.perf_counter() - t0) / reps
    return {"workload": f"GSA layer forward B=1 T=512 D={D} H={H} fp32 k_base=256 k_max=512, unchunked",
            "ms_per_forward": sec * 1e3, "tokens_per_s": 512 / sec, "warmup": 1, "timed": reps}


def cpu_baseline(B, T, budget_s, dtype=torch.bfloat16):
    """The CPU oracle (restatement of gsa_ref.py's forward) on sampled query rows
    of the same workload: per-token cost = the token's own projections plus its
    indexer row, selection, gathered attention and o_proj, over row chunks spread
    evenly across the sequence, until the time budget is spent.  Every core of
    the process's affinity set runs torch's intra-op threads."""
    from oracle import gsa_oracle as orc

    ncores = len(os.sched_getaffinity(0))
    torch.set_num_threads(ncores)
    cfg = orc.GSAConfig(hidden_size=D, num_heads=H, k_max=K_MAX, d_indexer=DI, n_idx_heads=HI,
                        k_base=K_BASE, k_min=K_MIN)
    sd = orc.cast_state(orc.synthetic_state(cfg, seed=0), dtype)
    x = orc.synthetic_input(B, T, D, seed=1).to(dtype)
    chunk = 32
    with torch.inference_mode():
        p_all = orc.project(sd, cfg, x)                 # untimed: keys/values of every row
        starts = [int(i * (T - chunk) / 63) for i in range(64)]
        # order the chunks so any prefix is spread over the sequence
        order = sorted(range(64), key=lambda i: int(format(i, "06b")[::-1], 2))
        done_rows, spent = 0, 0.0
        orc.attend_rows(sd, cfg, p_all, starts[0], starts[0] + chunk)   # warm-up
        for i in order:
            r0 = starts[i]
            t0 = time.perf_counter()
            orc.project(sd, cfg, x[:, r0:r0 + chunk])
            orc.attend_rows(sd, cfg, p_all, r0, r0 + chunk)
            spent += time.perf_counter() - t0
            done_rows += chunk
            if spent >= budget_s:
                break
    cpu_model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu_model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {
        "value": B * done_rows / spent, "unit": "tokens/s", "cores": ncores, "kind": "port",
        "threads": torch.get_num_threads(),
        "c1_fp32_unchunked": cpu_c1_unchunked(),
        "sample": (f"CPU oracle (torch restatement of gsa_ref.py forward, {str(dtype).split('.')[-1]}) "
                   f"on {done_rows} of {T} query rows in {done_rows // chunk} chunks of {chunk} spread "
                   f"over the sequence; per row: its 8 projections + indexer row vs all keys + top-k "
                   f"+ gathered attention + gate + o_proj; keys/values of all rows precomputed untimed; "
                   f"{spent:.1f} s timed; {cpu_model}"),
    }


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    # the first ~20 forwards run measurably slower while the GPU settles into its
    # sustained state (c3: 2.36 ms/step after 3 warm-up forwards, 2.23-2.28 after
    # 20, 2.26 after 50, same box); 20 untimed forwards take ~50 ms at c3
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", choices=sorted(CONFIGS), default="c3")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--k-mode", choices=["fixed", "variance"], default="fixed",
                    help="selector: fixed k_eff (the reference) or the variance-based per-row k")
    ap.add_argument("--proj", choices=["gemm", "fused"], default="gemm",
                    help="main projection: hipBLASLt GEMM + producer kernel, or the fused MFMA GEMM "
                         "with the producer in its epilogue")
    ap.add_argument("--overlap", choices=["auto", "producer", "gemm", "serial"], default="auto",
                    help="where the indexer runs relative to the projection GEMM and the producer")
    ap.add_argument("--graph", action="store_true",
                    help="time HIP-graph replays of the forward (one launch per step)")
    ap.add_argument("--calib-copy-mib", type=int, default=0,
                    help="after timing, run one plain device copy of this many MiB (counter calibration)")
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py measures one GPU: --gpus {args.gpus} is not supported (this package runs the "
              f"GSA forward on a single MI355X; multi-GPU sharding is design-only)", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)

    from gsa_gdn_benchmarkstudy_amd import _abi

    dev = torch.device("cuda:0")
    B, T = CONFIGS[args.config]
    dtype = torch.bfloat16
    model = synthetic_model(dev, dtype)
    model.topk_selector.mode = args.k_mode
    model.proj_impl = args.proj
    model.indexer_overlap = args.overlap
    g = torch.Generator(device="cpu").manual_seed(1)
    x = torch.randn(B, T, D, generator=g)
    if args.config == "c4":   # per-sequence sigma ~ U(0.5, 2)
        x = x * (0.5 + 1.5 * torch.rand(B, generator=g)).view(B, 1, 1)
    x = x.to(dtype).to(dev)
    k_eff = model.topk_selector.k_effective(T)

    with torch.no_grad():
        for _ in range(args.warmup):
            model(x)
        torch.cuda.synchronize()
        torch.cuda.reset_peak_memory_stats(dev)
        step = (lambda: model(x))
        if args.graph:
            from gsa_gdn_benchmarkstudy_amd.graph import GraphedForward
            graphed = GraphedForward(model, x, warmup=1)
            step = (lambda: graphed(x))
            for _ in range(args.warmup):
                step()
            torch.cuda.synchronize()
        else:
            model.attn_events = []
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(args.steps):
            step()
        end.record()
        torch.cuda.synchronize()
        if args.graph:      # the attention kernel's own time from eager forwards
            model.attn_events = []
            for _ in range(min(args.steps, 5)):
                model(x)
            torch.cuda.synchronize()
        evs = model.attn_events
        model.attn_events = None
    total_ms = start.elapsed_time(end)
    peak_mem = torch.cuda.max_memory_allocated(dev)     # during the timed forwards
    ms = total_ms / args.steps
    attn_impl = "dense" if model.uses_dense(dtype) else "gather"
    attn_ms = sum(a.elapsed_time(b) for a, b in evs) / len(evs)
    P_sel = k_stats = None
    if args.k_mode == "variance":
        kr = model.topk_selector.last_k.cpu().long()
        P_sel = int(torch.minimum(kr, torch.arange(1, T + 1).view(1, T)).sum())
        k_stats = {"min": int(kr.min()), "mean": float(kr.float().mean()), "max": int(kr.max()),
                   "per_batch_mean": [float(v) for v in kr.float().mean(dim=1)]}

    # the gather kernel on the same layer and input, timed the same way
    gather_ms = None
    if attn_impl == "dense":
        with torch.no_grad():
            model.attn_impl = "gather"
            model(x)
            torch.cuda.synchronize()
            model.attn_events = []
            for _ in range(min(args.steps, 5)):
                model(x)
            torch.cuda.synchronize()
            gather_ms = sum(a.elapsed_time(b) for a, b in model.attn_events) / len(model.attn_events)
            model.attn_events = None
            model.attn_impl = "auto"
    else:
        gather_ms = attn_ms

    # indexer kernel alone (same stream discipline, timed separately)
    with torch.no_grad():
        views = model.project(x)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        # one untimed call first: the GPU runs it while the host records e0 and
        # enqueues the timed calls, so no host time falls between the events
        model.select(views, T, indices=not model.uses_dense(dtype))
        e0.record()
        n_idx = 5
        for _ in range(n_idx):
            model.select(views, T, indices=not model.uses_dense(dtype))
        e1.record()
        torch.cuda.synchronize()
        idx_ms = e0.elapsed_time(e1) / n_idx
        del views

    # the main projection and its producer both ways (hipBLASLt GEMM + producer
    # kernel; fused MFMA GEMM with the producer in its epilogue), timed alone
    proj = {"impl": args.proj}
    with torch.no_grad():
        cos, sin = model.rotary_emb(T, dev, dtype)
        cos, sin = cos.contiguous(), sin.contiguous()

        def unfused():
            v = model.project_main(x)
            return _abi.prologue_vt(v["v"], v["vg"], k=v["k"], cos=cos, sin=sin)

        ways = {"gemm_producer_ms": unfused}
        if _abi.proj_supported(D, H, T):
            ways["fused_ms"] = lambda: model.project_fused(x, cos, sin)
        for name, fn in ways.items():
            fn()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(5):
                fn()
            e1.record()
            torch.cuda.synchronize()
            proj[name] = e0.elapsed_time(e1) / 5

    if args.calib_copy_mib:
        n = args.calib_copy_mib * (1 << 20) // 4
        src = torch.ones(n, device=dev, dtype=torch.float32)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    abytes, P = attn_bytes(B, T, k_eff, P=P_sel)
    gather_gbs = abytes / (gather_ms * 1e-3) / 1e9
    aflops = 4 * P * H * DH                     # useful (selected-pair) QK and PV flops
    fidx = indexer_flops(B, T)
    i_prof = profiled_traffic("gsa_indexer_select", args.config)
    idx_tflops = fidx / (idx_ms * 1e-3) / 1e12
    g_prof = profiled_traffic("gsa_sparse_attn", args.config)
    g_traffic = None if g_prof is None else g_prof["bytes"]
    g_rate = None if g_traffic is None else g_traffic / (gather_ms * 1e-3) / 1e9
    gather_roof = {"kernel": "gsa_sparse_attn", "bound": "hbm", "achieved": g_rate, "peak": HBM_PEAK_GBS,
                   "unit": "GB/s", "frac": None if g_rate is None else g_rate / HBM_PEAK_GBS,
                   "traffic": g_traffic, "traffic_provenance": g_prof, "ms": gather_ms,
                   "note": "achieved = traffic (rocprofv3 FETCH_SIZE + WRITE_SIZE per launch beyond L2, "
                           "calibrated on a plain copy; it includes last-level-cache hits, so it bounds "
                           "the DRAM rate from above) / the kernel time measured here",
                   "algorithmic_rate": {"value": gather_gbs, "unit": "GB/s", "bytes": abytes, "valid_pairs": P,
                                        "note": "every selected K/V row counted as one read: rows that "
                                                "many queries select come from the caches, so this rate "
                                                "is not an HBM rate and may exceed the HBM peak"}}
    if attn_impl == "dense":
        d_prof = profiled_traffic("gsa_dense_attn", args.config)
        qrows = _abi.dense_block_rows(T)         # query rows per block of gsa_dense_attn
        nqb = (T + qrows - 1) // qrows
        # every 64-key tile up to the last row of each 32-row group (a wave of the
        # kernel), the groups padded to whole blocks
        dense_flops = 4 * B * H * DH * 32 * 64 * sum(min(32 * g + 31, T - 1) // 64 + 1
                                                      for g in range(nqb * qrows // 32))
        ach = aflops / (attn_ms * 1e-3) / 1e12
        ex = dense_flops / (attn_ms * 1e-3) / 1e12
        d_traffic = (d_prof or {}).get("bytes")
        d_rate = None if d_traffic is None else d_traffic / (attn_ms * 1e-3) / 1e9
        roofline = {"kernel": "gsa_dense_attn", "bound": "mfma", "achieved": ach, "peak": BF16_PEAK_TFLOPS,
                    "unit": "TFLOP/s", "frac": ach / BF16_PEAK_TFLOPS,
                    "traffic": d_traffic, "traffic_provenance": d_prof,
                    "hbm_rate": {"value": d_rate, "unit": "GB/s", "peak": HBM_PEAK_GBS,
                                 "frac": None if d_rate is None else d_rate / HBM_PEAK_GBS,
                                 "note": "the timed step's attention as an HBM figure: its profiled traffic "
                                         "beyond L2 (FETCH_SIZE + WRITE_SIZE, calibrated) over the time "
                                         "measured here; the kernel is MFMA-bound, so this is what it asks "
                                         "of HBM, not a limit it reaches"},
                    "algorithmic_flops": aflops, "executed_flops": dense_flops,
                    "executed_tflops": ex, "executed_frac": ex / BF16_PEAK_TFLOPS, "ms": attn_ms,
                    "note": "achieved/frac: the selected (useful) pairs' QK and PV flops; executed: the bf16 "
                            "MFMAs of every 64-key tile up to each 32-row group's last row, which the count "
                            "SQ_INSTS_VALU_MFMA_MOPS_BF16 x 512 gives within 0.5 %"}
    else:
        roofline = gather_roof

    out = {
        "metric": METRIC,
        "value": B * T / (ms * 1e-3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: x~N(0,1) (c4: per-sequence sigma~U(0.5,2)), weights~N(0,0.02), gate biases 0.5, "
                "indexer biases 0, random init",
        "config": {"workload": f"GSA layer forward B={B} T={T} D={D} H={H} d={DH} H_idx={HI} d_idx={DI} "
                               + (f"k_eff={k_eff}" if args.k_mode == "fixed" else
                                  f"variance-adaptive k (k_base={K_BASE}, k_min={K_MIN}, k_max={K_MAX})")
                               + " causal", "name": args.config, "batch": B, "seq_len": T,
                   "proj": args.proj, "overlap": args.overlap, "graph": args.graph, "k_mode": args.k_mode, "k_eff": k_eff if args.k_mode == "fixed" else k_stats},
        "roofline": roofline,
        "gather_attention": gather_roof,
        "indexer": {"kernel": "gsa_indexer_select", "bound": "mfma", "achieved": idx_tflops,
                    "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s", "frac": idx_tflops / BF16_PEAK_TFLOPS,
                    "traffic": (i_prof or {}).get("bytes"), "traffic_provenance": i_prof,
                    "flops": fidx, "ms": idx_ms},
        "projection": proj,
        "peak_mem_gib": peak_mem / 2**30,
    }
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(B, T, args.cpu_seconds)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
