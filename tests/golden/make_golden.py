"""Write the golden fixtures of the GSA forward path (run on the CPU).

The fixtures are the oracle's outputs (oracle/gsa_oracle.py, itself pinned by
tests/test_oracle.py) on small seeded inputs.  Weights are regenerated from
their seed by ``oracle.synthetic_state``; a checksum of the regenerated
weights is stored so that a change in the generator shows up as a fixture
error rather than as a kernel error.

Usage: python tests/golden/make_golden.py
"""

import hashlib
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import gsa_oracle as orc  # noqa: E402

# name: (dtype, B, T, config kwargs, weight seed, input seed)
CASES = {
    "layer_f32_T48": ("float32", 1, 48, dict(hidden_size=256, num_heads=2, k_max=64, k_base=16, k_min=4), 0, 1),
    "layer_bf16_T48": ("bfloat16", 1, 48, dict(hidden_size=256, num_heads=2, k_max=64, k_base=16, k_min=4), 0, 1),
    "layer_f32_fullk_T40": ("float32", 1, 40, dict(hidden_size=256, num_heads=2, k_max=4096, k_base=2048), 1, 2),
    "layer_bf16_B2_T33": ("bfloat16", 2, 33, dict(hidden_size=256, num_heads=2, k_max=8, k_base=64, k_min=4), 2, 3),
}


def weights_digest(sd):
    h = hashlib.sha256()
    for k in sorted(sd):
        h.update(k.encode())
        h.update(sd[k].float().contiguous().numpy().tobytes())
    return h.hexdigest()


def make_case(dtype_name, B, T, cfg_kw, wseed, xseed):
    dt = getattr(torch, dtype_name)
    cfg = orc.GSAConfig(**cfg_kw)
    sd = orc.cast_state(orc.synthetic_state(cfg, seed=wseed), dt)
    x = orc.synthetic_input(B, T, cfg.hidden_size, seed=xseed).to(dt)
    y, aux = orc.gsa_forward(sd, cfg, x, return_aux=True)
    idx_asc, cnt = orc.select_ascending(aux["scores"], aux["k_eff"])
    return dict(
        x=x.float().numpy(), y=y.float().numpy(), scores=aux["scores"].numpy(),
        idx=aux["idx"].numpy().astype(np.int32), mask=aux["mask"].numpy(),
        idx_asc=idx_asc.numpy(), count=cnt.numpy(), attn=aux["attn"].float().numpy(),
        k_eff=np.int32(aux["k_eff"]), wdigest=np.array(weights_digest(sd)),
    )


def ties_case():
    """Selector fixture: scores with many exact ties and causal -inf."""
    g = torch.Generator().manual_seed(77)
    T = 70
    s = torch.randint(0, 6, (2, T, T), generator=g).float() / 6
    s = s.masked_fill(torch.triu(torch.ones(T, T, dtype=torch.bool), 1), float("-inf"))
    out = dict(scores=s.numpy())
    for k in (1, 7, 33, 70):
        idx, mask = orc.select_topk(s, k)
        ia, c = orc.select_ascending(s, k)
        out[f"idx_desc_k{k}"] = idx.numpy().astype(np.int32)
        out[f"mask_k{k}"] = mask.numpy()
        out[f"idx_asc_k{k}"] = ia.numpy()
        out[f"count_k{k}"] = c.numpy()
    return out


def main():
    for name, (dt, B, T, kw, ws, xs) in CASES.items():
        np.savez_compressed(os.path.join(HERE, f"{name}.npz"), **make_case(dt, B, T, kw, ws, xs))
        print("wrote", name)
    np.savez_compressed(os.path.join(HERE, "select_ties_T70.npz"), **ties_case())
    print("wrote select_ties_T70")


if __name__ == "__main__":
    main()
