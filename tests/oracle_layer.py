"""The oracle as a reference layer for the benchmark harness's ``--ref``.

``GatedSparseAttention`` here has the reference constructor and state-dict keys
(it inherits the parameter layout of the drop-in module) and computes its
forward with the CPU oracle (``oracle/gsa_oracle.py``, the restatement of
gsa_triton/gsa_ref.py): inputs and weights are copied to the host, the
query-chunked oracle forward runs there in the layer's dtype, and the output is
copied back to the input's device.  Test infrastructure only.
"""

import os
import sys

import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

from gsa_gdn_benchmarkstudy_amd.gsa import GatedSparseAttention as _Layout  # noqa: E402
from oracle import gsa_oracle as orc  # noqa: E402


class GatedSparseAttention(_Layout):
    def __init__(self, hidden_size, num_heads, k_max=4096, d_indexer=64, n_idx_heads=4,
                 k_base=2048, k_min=256):
        super().__init__(hidden_size, num_heads, k_max=k_max, d_indexer=d_indexer,
                         n_idx_heads=n_idx_heads, k_base=k_base, k_min=k_min)
        self.cfg = orc.GSAConfig(hidden_size=hidden_size, num_heads=num_heads, k_max=k_max,
                                 d_indexer=d_indexer, n_idx_heads=n_idx_heads, k_base=k_base,
                                 k_min=k_min)

    def fuse_projections(self):  # the oracle reads the separate projection weights
        pass

    def forward(self, x, attention_mask=None):
        sd = {k: v.detach().cpu() for k, v in self.state_dict().items()}
        out = orc.gsa_forward_chunked(sd, self.cfg, x.detach().cpu())
        return out.to(x.device)
