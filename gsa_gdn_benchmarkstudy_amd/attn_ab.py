"""A/B timing of gsa_dense_attn across builds of libgsa_hip.so.

    python -m gsa_gdn_benchmarkstudy_amd.attn_ab --T 16384 LIB_A.so LIB_B.so [LIB_A.so ...]

Times the dense attention kernel alone (B=1 by default, H=16, d=128, causal,
RoPE on q and the output gate on, as the layer calls it) on one synthetic
input for every library in the list, in list order, in one process, and
compares each output with the first library's bit for bit.  The selection is
random with the layer's density: row t keeps each causal key with probability
min(1, k/(t+1)), k = 2048 by default.  The lane masks are built once per
library and are not part of the timed region.

Naming a library twice (A B A B) shows the box-to-box and run-to-run spread
beside the difference.  ``--rope halves`` passes RoPE as the packed cos|sin
table (ATTN_ROPE_HALVES), ``--rope both`` times each library with the full
tables and then with the packed one.  Each line reports the best of three timed runs of
`--iters` launches between two HIP events.  This is a tool for kernel work:
a copy of dense_attn.hip with a change is built into its own library
(`python -m gsa_gdn_benchmarkstudy_amd.build --dense-src COPY --out LIB`) and
timed against the default build.
"""

from __future__ import annotations

import argparse
import sys

import torch

from . import _abi


def synthetic_inputs(B: int, T: int, H: int, k: int, seed: int, dev: torch.device):
    """q, k, og [B,T,H,128], V^T [B,H,128,vt_len(T)], cos/sin [T,128] (bf16) and a
    causal selection bitmask [B,T,2*ceil(T/64)] with density min(1, k/(t+1))."""
    g = torch.Generator(device=dev).manual_seed(seed)
    bf = torch.bfloat16
    q = torch.randn(B, T, H, 128, device=dev, generator=g).to(bf)
    kk = torch.randn(B, T, H, 128, device=dev, generator=g).to(bf)
    og = torch.randn(B, T, H, 128, device=dev, generator=g).to(bf)
    vt = torch.zeros(B, H, 128, _abi.vt_len(T), device=dev, dtype=bf)
    vt[..., :T] = torch.randn(B, H, 128, T, device=dev, generator=g).to(bf)
    NT = (T + 63) // 64
    bits = torch.empty(B, T, 2 * NT, device=dev, dtype=torch.int32)
    pw = 2 ** torch.arange(32, device=dev, dtype=torch.int64)
    for b in range(B):
        for r0 in range(0, T, 2048):
            r1 = min(T, r0 + 2048)
            t = torch.arange(r0, r1, device=dev)
            p = torch.clamp(k / (t + 1).float(), max=1.0)
            sel = torch.rand(r1 - r0, NT * 64, device=dev, generator=g) < p[:, None]
            sel &= torch.arange(NT * 64, device=dev)[None, :] <= t[:, None]
            bits[b, r0:r1] = (sel.view(r1 - r0, 2 * NT, 32).to(torch.int64) * pw).sum(-1).to(torch.int32)
    cos = torch.randn(T, 128, device=dev, generator=g).to(bf)
    sin = torch.randn(T, 128, device=dev, generator=g).to(bf)
    return q, kk, og, vt, bits, cos, sin


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("libs", nargs="+", help="libgsa_hip.so builds, timed in this order")
    ap.add_argument("--T", type=int, default=16384)
    ap.add_argument("--B", type=int, default=1)
    ap.add_argument("--H", type=int, default=16)
    ap.add_argument("--k", type=int, default=2048)
    ap.add_argument("--iters", type=int, default=0, help="launches per timed run (default: 10, 3 past 16K keys)")
    ap.add_argument("--seed", type=int, default=5)
    ap.add_argument("--rope", choices=("full", "halves", "both"), default="full",
                    help="RoPE tables: full cos and sin, the packed cos|sin halves, or each in turn")
    args = ap.parse_args(argv)
    if not torch.cuda.is_available():
        print("attn_ab needs a GPU", file=sys.stderr)
        return 1
    dev = torch.device("cuda:0")
    T = args.T
    q, kk, og, vt, bits, cos, sin = synthetic_inputs(args.B, T, args.H, args.k, args.seed, dev)
    # RoPE tables whose entries d and d+64 repeat (as RotaryEmbedding builds them), and their packed form
    cos = torch.cat((cos[:, :64], cos[:, :64]), dim=-1).contiguous()
    sin = torch.cat((sin[:, :64], sin[:, :64]), dim=-1).contiguous()
    packed = torch.cat((cos[:, :64], sin[:, :64]), dim=-1).contiguous()
    flags = _abi.ATTN_ROPE_Q | _abi.ATTN_OUT_GATE
    scale = 128 ** -0.5
    iters = args.iters or (10 if T <= 16384 else 3)
    modes = {"full": [False], "halves": [True], "both": [False, True]}[args.rope]
    ref = None
    for path, halves in [(p, h) for p in args.libs for h in modes]:
        _abi._lib = None
        _abi.LIB_PATH = path
        _abi.load()
        ws = _abi.dense_lane_masks(bits, T, causal=True)

        def run(out=None):
            if halves:
                return _abi.dense_attn(q, kk, vt, bits, scale, og=og, cos=packed, flags=flags | _abi.ATTN_ROPE_HALVES,
                                       ws=ws, masks_ready=True, out=out)
            return _abi.dense_attn(q, kk, vt, bits, scale, og=og, cos=cos, sin=sin, flags=flags, ws=ws,
                                   masks_ready=True, out=out)

        out = run()
        torch.cuda.synchronize()
        if ref is None:
            same = "reference output"
            ref = out.clone()
        elif torch.equal(out, ref):
            same = "bit-identical"
        else:
            same = f"DIFFERS (max |diff| {(out.float() - ref.float()).abs().max().item():.3e})"
        for _ in range(5):
            run(out)
        runs = []
        for _ in range(3):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(iters):
                run(out)
            e1.record()
            torch.cuda.synchronize()
            runs.append(e0.elapsed_time(e1) / iters)
        tag = " (packed cos|sin)" if halves else ""
        print(f"B={args.B} T={T} {path}{tag}: {min(runs):.4f} ms (runs {', '.join(f'{x:.4f}' for x in runs)}), {same}",
              flush=True)
        del ws, out
    return 0


if __name__ == "__main__":
    sys.exit(main())
