"""Host-side logic of the drop-in module, without a GPU: state_dict
compatibility, the fused/padded projection layout, the RoPE cache semantics
against the oracle, and that there is no CPU fallback."""

import pytest
import torch

from gsa_gdn_benchmarkstudy_amd import GatedSparseAttention, RotaryEmbedding
from oracle import gsa_oracle as orc

CFG = orc.GSAConfig(hidden_size=256, num_heads=2, k_max=64, k_base=16, k_min=4)


def _model(cfg=CFG):
    return GatedSparseAttention(cfg.hidden_size, cfg.num_heads, k_max=cfg.k_max, d_indexer=cfg.d_indexer,
                                n_idx_heads=cfg.n_idx_heads, k_base=cfg.k_base, k_min=cfg.k_min)


def test_state_dict_keys_match_reference():
    assert tuple(sorted(_model().state_dict())) == tuple(sorted(orc.STATE_KEYS))


def test_load_reference_state_strict_and_fused_layout():
    m = _model()
    sd = orc.synthetic_state(CFG, seed=3)
    sd["indexer.idx_w_proj.bias"] = torch.arange(4, dtype=torch.float32) + 1.0
    m.load_state_dict(sd, strict=True)
    m.fuse_projections()
    w, b = m._fused_weight, m._fused_bias
    D = CFG.hidden_size
    assert w.shape[0] % 64 == 0 and w.shape[0] >= 5 * D + 256 + 64 + 4
    order = ["q_proj.weight", "k_proj.weight", "v_proj.weight", "value_gate.gate_proj.weight",
             "output_gate.gate_proj.weight", "indexer.idx_q_proj.weight", "indexer.idx_k_proj.weight",
             "indexer.idx_w_proj.weight"]
    off = 0
    for key in order:
        n = sd[key].shape[0]
        assert torch.equal(w[off:off + n], sd[key]), key
        off += n
    assert torch.all(w[off:] == 0)
    offs = m._offsets()
    assert torch.equal(b[offs["vg"]:offs["vg"] + D], sd["value_gate.gate_proj.bias"])
    assert torch.equal(b[offs["og"]:offs["og"] + D], sd["output_gate.gate_proj.bias"])
    assert torch.equal(b[offs["iw"]:offs["iw"] + 4], sd["indexer.idx_w_proj.bias"])
    others = torch.ones_like(b, dtype=torch.bool)
    others[offs["vg"]:offs["vg"] + D] = False
    others[offs["og"]:offs["og"] + D] = False
    others[offs["iw"]:offs["iw"] + 4] = False
    assert torch.all(b[others] == 0)
    # every slice that is read with 16-byte vector loads starts 16-byte aligned
    for name in ("q", "k", "v", "vg", "og", "iq", "ik"):
        assert offs[name] % 8 == 0


def test_load_state_dict_invalidates_fused_weight():
    m = _model()
    m.fuse_projections()
    assert m._fused_weight is not None
    m.load_state_dict(orc.synthetic_state(CFG, seed=4), strict=True)
    assert m._fused_weight is None


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_rotary_matches_oracle_cache_semantics(dtype):
    rot = RotaryEmbedding(128).to(dtype)
    rc = orc.RopeCache(128, dtype)
    for T in (100, 8192, 8200, 300):      # rebuild at 8200 persists for 300
        c, s = rot(T, torch.device("cpu"), dtype)
        rc_c, rc_s = rc.tables(T, dtype)
        assert torch.equal(c, rc_c) and torch.equal(s, rc_s), T


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_rotary_halves_packs_the_oracle_tables(dtype):
    """The packed table of the dense attention's RoPE: row t = cos[t][:64] then
    sin[t][:64] of the oracle's tables, which repeat their first half (also
    after the rebuild past 8192 rows); a hand-edited cache that breaks the
    repetition gives None (the module then passes the full tables)."""
    rot = RotaryEmbedding(128).to(dtype)
    rc = orc.RopeCache(128, dtype)
    for T in (100, 8200):
        cs = rot.halves(T, torch.device("cpu"), dtype)
        rc_c, rc_s = rc.tables(T, dtype)
        assert torch.equal(rc_c[:, :64], rc_c[:, 64:]) and torch.equal(rc_s[:, :64], rc_s[:, 64:])
        assert cs.shape == (T, 128) and cs.is_contiguous()
        assert torch.equal(cs[:, :64], rc_c[:, :64]) and torch.equal(cs[:, 64:], rc_s[:, :64]), T
    assert rot.halves(8200, torch.device("cpu"), dtype) is rot.halves(8200, torch.device("cpu"), dtype)
    rot.cos_cached[5, 100] += 1.0        # the cache is edited: a new version, no longer symmetric
    assert rot.halves(8200, torch.device("cpu"), dtype) is None


def test_no_cpu_fallback():
    m = _model()
    with pytest.raises(RuntimeError):
        m(torch.randn(1, 8, CFG.hidden_size))


def test_selector_modes():
    from gsa_gdn_benchmarkstudy_amd import AdaptiveTopKSelector

    s = AdaptiveTopKSelector(k_base=2048, k_min=256, k_max=4096)
    assert s.mode == "fixed" and s.k_effective(16384) == 2048 and s.k_effective(1000) == 1000
    s.mode = "variance"          # outputs are min(k_max, T) wide; k_t varies per row
    assert s.k_effective(16384) == 4096 and s.k_effective(1000) == 1000
    s.mode = "median"
    with pytest.raises(ValueError):
        s.k_effective(10)
