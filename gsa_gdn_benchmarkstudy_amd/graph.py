"""HIP-graph replay of the GSA layer forward.

A forward launches about ten kernels from Python (two GEMMs, the fused
indexer + select on a side stream, the producer, lane masks, attention,
o_proj) plus the host work around them; below T ~ 4096 the GPU finishes
them faster than the host issues them.  ``GraphedForward`` records one
forward of a fixed input shape into a HIP graph (``torch.cuda.CUDAGraph`` is
a hipGraph on ROCm) and replays it: one launch per forward, the side-stream
fork/join kept as graph edges.

The forward records no memset nodes: every buffer it allocates is written
whole by the kernel that produces it.

Usage::

    g = GraphedForward(model, x)   # warms up eagerly, then records
    y = g(x_new)                   # copies x_new into the recorded input, replays

The returned tensor is the graph's own output buffer, overwritten by the next
replay (clone it to keep it).  The graph reads device memory by address, so
it holds references to everything the recorded forward read that the model
may replace: the fused projection weight and bias (and the fused GEMM's
packed copy), the fp32 indexer bias and the cast RoPE tables.  In-place
updates of ``o_proj.weight`` are seen by replays; the other projections are
read through the fused copy that ``fuse_projections`` makes, so updating
them means calling ``fuse_projections`` (or ``load_state_dict``) and
recording a new graph.  After the fused weight is rebuilt, or the RoPE
cache is (a forward over more rows than it holds rebuilds it, and the
reference's later, shorter calls read the rebuilt tables), the graph refuses
to replay.  Eager forwards over other row counts in between are fine: they
cast other tables, and the graph still holds its own.
"""

from __future__ import annotations

import torch


class GraphedForward:
    def __init__(self, model, x: torch.Tensor, warmup: int = 2):
        if not x.is_cuda:
            raise RuntimeError("GraphedForward needs a device tensor")
        self.model = model
        self.shape, self.dtype, self.device = tuple(x.shape), x.dtype, x.device
        self.static_x = x.detach().clone()
        cur = torch.cuda.current_stream(self.device)
        side = torch.cuda.Stream(device=self.device)
        side.wait_stream(cur)
        with torch.no_grad(), torch.cuda.stream(side):
            for _ in range(max(1, warmup)):   # builds the fused weight, caches, LDS limits
                model(self.static_x)
        cur.wait_stream(side)
        self.graph = torch.cuda.CUDAGraph()
        with torch.no_grad(), torch.cuda.graph(self.graph):
            self.static_y = model(self.static_x)
        # what the recorded kernels read by address, kept alive by these references
        cast = model.rotary_emb._cast
        halves = getattr(model.rotary_emb, "_halves", None)
        self._tables = (cast[1], cast[2], halves[1] if halves is not None else None)
        self._weights = self._weight_buffers()
        self._cache = self._rope_cache()

    def _weight_buffers(self):
        m = self.model
        return (m._fused_weight, m._fused_bias, m._packed, m._idx_bias32)

    def _rope_cache(self):
        r = self.model.rotary_emb
        return (r.cos_cached, r.sin_cached, r.cos_cached._version, r.sin_cached._version)

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        if tuple(x.shape) != self.shape or x.dtype != self.dtype or x.device != self.device:
            raise ValueError(f"GraphedForward recorded {self.shape} {self.dtype} on {self.device}; "
                             f"got {tuple(x.shape)} {x.dtype} on {x.device}")
        if any(a is not b for a, b in zip(self._weight_buffers(), self._weights)):
            raise RuntimeError("the fused projection weight was rebuilt after recording: record a new graph")
        c = self._rope_cache()
        if c[0] is not self._cache[0] or c[1] is not self._cache[1] or c[2:] != self._cache[2:]:
            raise RuntimeError("the RoPE cache was rebuilt after recording (a forward over more rows than "
                               "it held): record a new graph")
        if x.data_ptr() != self.static_x.data_ptr():
            self.static_x.copy_(x)
        self.graph.replay()
        return self.static_y
