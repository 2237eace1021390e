"""The fused projection (gsa_proj_pack + gsa_proj_fused): the main projection
GEMM with RoPE(k) and the value gate in its epilogue.

Checks, on the GPU:
  * against the oracle (oracle.gsa_oracle.project: the reference's Linear,
    value gate and RoPE in bf16 on the CPU): RoPE(q) of the raw q,
    RoPE(k), v*sigmoid(vg) and sigmoid(og) within the bf16 bar
    (atol 2e-2, rtol 1e-2) and with at most 1e-3 of the elements off by
    more than one bf16 ulp;
  * against the unfused path (the hipBLASLt GEMM, then gsa_prologue_vt),
    which rounds at the same points: equal except for rare one-ulp
    differences of the fp32 sum order (at most 1e-3 of the elements);
  * token tails (B*T not a multiple of the 256-token tile), odd batch counts,
    two heads, the smallest and the layer's width, and zeroed V^T padding;
  * the layer with proj_impl="fused" against proj_impl="gemm" and against the
    oracle layer.
"""

import ctypes

import pytest
import torch
import torch.nn.functional as F

from gsa_gdn_benchmarkstudy_amd import GatedSparseAttention, _abi
from oracle import gsa_oracle as orc

pytestmark = pytest.mark.gpu


def _log(msg):
    print(msg, flush=True)


def _ulp_bf16(x: torch.Tensor) -> torch.Tensor:
    """Spacing of bf16 numbers at |x| (2^(e-7) for x in [2^e, 2^(e+1)))."""
    a = x.float().abs().clamp_min(2.0 ** -126)
    return torch.exp2(torch.floor(torch.log2(a)) - 7)


def _close_bf16(got, ref, what, frac=1e-3):
    got, ref = got.float().cpu(), ref.float().cpu()
    err = (got - ref).abs()
    bad = err > 2e-2 + 1e-2 * ref.abs()
    assert not bad.any(), f"{what}: max err {err.max().item():.3e}"
    off = (err > _ulp_bf16(ref)).float().mean().item()
    _log(f"  {what}: max|err| {err.max().item():.3e}, > 1 ulp {off:.2e}")
    assert off <= frac, f"{what}: {off:.2e} of the elements differ by more than one ulp"


def _same_or_ulp(got, ref, what, frac=1e-3):
    got, ref = got.float().cpu(), ref.float().cpu()
    diff = got != ref
    assert torch.all((got - ref).abs()[diff] <= _ulp_bf16(ref)[diff] * 1.0001), f"{what}: a difference beyond one ulp"
    f = diff.float().mean().item()
    _log(f"  {what}: differing {f:.2e}")
    assert f <= frac


def _state(D, H, seed):
    cfg = orc.GSAConfig(hidden_size=D, num_heads=H, k_max=96, k_base=64, k_min=16)
    sd = orc.cast_state(orc.synthetic_state(cfg, seed=seed), torch.bfloat16)
    # non-zero gate biases so the bias path is exercised
    g = torch.Generator().manual_seed(seed + 100)
    sd["value_gate.gate_proj.bias"] = (torch.randn(D, generator=g) * 0.5).to(torch.bfloat16)
    sd["output_gate.gate_proj.bias"] = (torch.randn(D, generator=g) * 0.5).to(torch.bfloat16)
    return cfg, sd


def _weights(sd, dev):
    w = torch.cat([sd["q_proj.weight"], sd["k_proj.weight"], sd["v_proj.weight"],
                   sd["value_gate.gate_proj.weight"], sd["output_gate.gate_proj.weight"]], 0).to(dev)
    D = w.shape[1]
    b = torch.zeros(5 * D, dtype=torch.bfloat16)
    b[3 * D:4 * D] = sd["value_gate.gate_proj.bias"]
    b[4 * D:] = sd["output_gate.gate_proj.bias"]
    return w.contiguous(), b.to(dev)


@pytest.mark.parametrize("B,T,D", [(1, 256, 256), (2, 320, 512), (3, 64, 256), (1, 1024, 2048)])
def test_proj_fused_vs_oracle_and_unfused(dev, B, T, D):
    H = D // 128
    _log(f"proj_fused B={B} T={T} D={D}")
    cfg, sd = _state(D, H, seed=T + D)
    x = orc.synthetic_input(B, T, D, seed=3).to(torch.bfloat16)
    w, b = _weights(sd, dev)
    rope = orc.RopeCache(128, torch.bfloat16)
    cos, sin = rope.tables(T, torch.bfloat16)
    cos_d, sin_d = cos.to(dev).contiguous(), sin.to(dev).contiguous()

    wp, bp = _abi.proj_pack(w, b)
    q, og, k_rope, vt = _abi.proj_fused(x.to(dev), wp, bp, cos_d, sin_d, H)
    torch.cuda.synchronize()
    assert vt.shape == (B, H, 128, _abi.vt_len(T))

    # oracle: the reference's projections, value gate and RoPE in bf16 on the CPU
    p = orc.project(sd, cfg, x)
    c4, s4 = cos[None, :, None, :], sin[None, :, None, :]
    _close_bf16(orc.apply_rope(q.cpu(), c4, s4), p.q, "RoPE(q) vs oracle")
    _close_bf16(k_rope, p.k, "RoPE(k) vs oracle")
    _close_bf16(vt[..., :T].permute(0, 3, 1, 2), p.v, "v*sigmoid(vg) vs oracle")
    _close_bf16(torch.sigmoid(og.cpu().reshape(B, T, D)), p.og, "sigmoid(og) vs oracle")

    # unfused GPU path: same rounding points
    comb = F.linear(x.to(dev), w, b)
    views = {n: comb[..., i * D:(i + 1) * D].view(B, T, H, 128)
             for i, n in enumerate(("q", "k", "v", "vg", "og"))}
    k2, vt2 = _abi.prologue_vt(views["v"], views["vg"], k=views["k"], cos=cos_d, sin=sin_d)
    _same_or_ulp(q, views["q"], "q vs unfused")
    _same_or_ulp(og, views["og"], "og vs unfused")
    _same_or_ulp(k_rope, k2, "RoPE(k) vs unfused")
    _same_or_ulp(vt, vt2, "V^T vs unfused")


def test_proj_fused_pads_vt(dev):
    """ldv > T: keys [T, ldv) of every V^T row are zero (through the C ABI)."""
    B, T, D, H = 2, 128, 256, 2
    _log("proj_fused V^T padding")
    cfg, sd = _state(D, H, seed=9)
    x = orc.synthetic_input(B, T, D, seed=4).to(torch.bfloat16).to(dev)
    w, b = _weights(sd, dev)
    cos, sin = orc.RopeCache(128, torch.bfloat16).tables(T, torch.bfloat16)
    cos, sin = cos.to(dev).contiguous(), sin.to(dev).contiguous()
    wp, bp = _abi.proj_pack(w, b)
    q, og, k_rope, vt = _abi.proj_fused(x, wp, bp, cos, sin, H)
    ldv = T + 64
    vt_pad = torch.full((B, H, 128, ldv), 7.0, dtype=torch.bfloat16, device=dev)
    qo = torch.empty(B, T, 2, H, 128, dtype=torch.bfloat16, device=dev)
    ko = torch.empty(B, T, H, 128, dtype=torch.bfloat16, device=dev)
    lib = _abi.load()
    st = lib.gsa_proj_fused(x.data_ptr(), x.stride(1), B, T, D, H, _abi.DTYPE_BF16, wp.data_ptr(), bp.data_ptr(),
                            cos.data_ptr(), sin.data_ptr(), cos.stride(0), qo.data_ptr(), qo.stride(1),
                            qo[:, :, 1].data_ptr(), qo.stride(1), ko.data_ptr(), vt_pad.data_ptr(), ldv,
                            ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert st == 0, _abi.status_string(st)
    torch.cuda.synchronize()
    assert torch.equal(vt_pad[..., :T].cpu(), vt.cpu())
    assert torch.all(vt_pad[..., T:].cpu() == 0)
    assert torch.equal(ko.cpu(), k_rope.cpu())
    assert torch.equal(qo[:, :, 0].cpu(), q.cpu()) and torch.equal(qo[:, :, 1].cpu(), og.cpu())


def _layer(cfg, sd, dev, proj):
    m = GatedSparseAttention(cfg.hidden_size, cfg.num_heads, k_max=cfg.k_max, d_indexer=cfg.d_indexer,
                             n_idx_heads=cfg.n_idx_heads, k_base=cfg.k_base, k_min=cfg.k_min)
    m = m.to(dev).to(torch.bfloat16).eval()
    m.load_state_dict({k: v.to(dev) for k, v in sd.items()}, strict=True)
    m.fuse_projections()
    m.proj_impl = proj
    return m


@pytest.mark.parametrize("B,T", [(1, 256), (2, 192)])
def test_layer_fused_projection(dev, B, T):
    """The layer with the fused projection: against the default path and the oracle layer."""
    _log(f"layer proj_impl=fused B={B} T={T}")
    cfg, sd = _state(512, 4, seed=21)
    x = orc.synthetic_input(B, T, cfg.hidden_size, seed=22).to(torch.bfloat16)
    mf, mg = _layer(cfg, sd, dev, "fused"), _layer(cfg, sd, dev, "gemm")
    assert mf.uses_fused_projection(x.to(dev)) and not mg.uses_fused_projection(x.to(dev))
    with torch.no_grad():
        yf = mf(x.to(dev)).cpu()
        yg = mg(x.to(dev)).cpu()
    d = (yf.float() - yg.float()).abs()
    _log(f"  fused vs gemm: max|d| {d.max().item():.3e}")
    assert d.max().item() <= 2e-3
    ref = orc.gsa_forward(sd, cfg, x).float()
    err = (yf.float() - ref).abs()
    assert torch.all(err <= 2e-2 + 1e-2 * ref.abs()), f"max err {err.max().item():.3e}"
    rel = (torch.linalg.vector_norm(yf.float() - ref) / torch.linalg.vector_norm(ref)).item()
    _log(f"  vs oracle: rel-L2 {rel:.3e}")
    assert rel < 2e-2


def test_layer_fused_projection_falls_back(dev):
    """Shapes the fused kernel does not take (T % 64 != 0, odd head count) run the GEMM path."""
    cfg, sd = _state(384, 3, seed=23)
    m = _layer(cfg, sd, dev, "fused")
    x = orc.synthetic_input(1, 128, 384, seed=24).to(torch.bfloat16).to(dev)
    assert not m.uses_fused_projection(x)
    cfg2, sd2 = _state(256, 2, seed=25)
    m2 = _layer(cfg2, sd2, dev, "fused")
    x2 = orc.synthetic_input(1, 100, 256, seed=26).to(torch.bfloat16).to(dev)
    assert not m2.uses_fused_projection(x2)
    with torch.no_grad():
        y = m2(x2).cpu()
    assert torch.isfinite(y.float()).all()
