"""HIP-graph replay of the layer forward (GraphedForward) against eager forwards.

Each recorded graph is replayed several times with different inputs, with
eager forwards and synchronisations of the program's own between the
replays, and every replay must equal the eager forward of the same input bit
for bit (the same kernels run in both)."""

import pytest
import torch

from gsa_gdn_benchmarkstudy_amd import GatedSparseAttention
from gsa_gdn_benchmarkstudy_amd.graph import GraphedForward
from oracle import gsa_oracle as orc

pytestmark = pytest.mark.gpu


def _log(msg):
    print(msg, flush=True)


def _model(dev, dtype=torch.bfloat16, impl="auto", k_mode="fixed", proj="gemm", D=512, H=4):
    cfg = orc.GSAConfig(hidden_size=D, num_heads=H, k_max=96, k_base=64, k_min=16)
    sd = orc.cast_state(orc.synthetic_state(cfg, seed=31), dtype)
    m = GatedSparseAttention(cfg.hidden_size, cfg.num_heads, k_max=cfg.k_max, d_indexer=cfg.d_indexer,
                             n_idx_heads=cfg.n_idx_heads, k_base=cfg.k_base, k_min=cfg.k_min)
    m = m.to(dev).to(dtype).eval()
    m.load_state_dict({k: v.to(dev) for k, v in sd.items()}, strict=True)
    m.fuse_projections()
    m.attn_impl = impl
    m.topk_selector.mode = k_mode
    m.proj_impl = proj
    return m


@pytest.mark.parametrize("dtype,impl,k_mode,proj,B,T", [
    (torch.bfloat16, "auto", "fixed", "gemm", 1, 256),
    (torch.bfloat16, "auto", "fixed", "gemm", 2, 200),
    (torch.bfloat16, "gather", "fixed", "gemm", 1, 256),
    (torch.bfloat16, "auto", "variance", "gemm", 2, 192),
    (torch.bfloat16, "auto", "fixed", "fused", 2, 256),
    (torch.float32, "auto", "fixed", "gemm", 1, 128),
])
def test_graph_replays_equal_eager(dev, dtype, impl, k_mode, proj, B, T):
    _log(f"graph dtype={dtype} impl={impl} k={k_mode} proj={proj} B={B} T={T}")
    m = _model(dev, dtype, impl, k_mode, proj)
    xs = [orc.synthetic_input(B, T, 512, seed=40 + i).to(dtype).to(dev) for i in range(3)]
    with torch.no_grad():
        eager = [m(x).clone() for x in xs]
    torch.cuda.synchronize()
    g = GraphedForward(m, xs[0])
    for n, i in enumerate([0, 1, 2, 1, 0, 2]):
        y = g(xs[i]).clone()
        torch.cuda.synchronize()
        assert torch.equal(y, eager[i]), f"replay {n} (input {i}) differs from the eager forward"
        with torch.no_grad():          # the program's own eager work between replays
            z = m(xs[(i + 1) % 3])
        torch.cuda.synchronize()
        assert torch.equal(z, eager[(i + 1) % 3])


def test_graph_refuses_other_shapes_and_rebuilt_weights(dev):
    m = _model(dev)
    x = orc.synthetic_input(1, 128, 512, seed=50).to(torch.bfloat16).to(dev)
    g = GraphedForward(m, x)
    with pytest.raises(ValueError):
        g(x[:, :64])
    with pytest.raises(ValueError):
        g(x.float())
    m.fuse_projections()
    with pytest.raises(RuntimeError):
        g(x)


def test_graph_holds_its_rope_tables_and_refuses_after_a_cache_rebuild(dev):
    """The recorded forward reads its cast RoPE tables by address.  Eager forwards over
    other row counts cast other tables: replays must still equal the recorded input's
    eager result, also after those forwards' buffers were freed and the memory was
    filled with other data.  A forward over more rows than the cache holds rebuilds
    it (later, shorter calls read the rebuilt tables): the graph then refuses."""
    m = _model(dev)
    x = orc.synthetic_input(1, 128, 512, seed=51).to(torch.bfloat16).to(dev)
    with torch.no_grad():
        ref = m(x).clone()
    g = GraphedForward(m, x)
    with torch.no_grad():
        m(orc.synthetic_input(1, 64, 512, seed=52).to(torch.bfloat16).to(dev))   # casts 64-row tables
        m(orc.synthetic_input(1, 96, 512, seed=53).to(torch.bfloat16).to(dev))   # and 96-row ones
    junk = [torch.full((1 << 16,), 7.0, device=dev) for _ in range(64)]          # reuse freed memory
    torch.cuda.synchronize()
    for _ in range(3):
        y = g(x).clone()
        torch.cuda.synchronize()
        assert torch.equal(y, ref)
    with torch.no_grad():
        m(orc.synthetic_input(1, 8300, 512, seed=54).to(torch.bfloat16).to(dev))   # rebuilds the cache
    del junk
    with pytest.raises(RuntimeError, match="RoPE cache"):
        g(x)
