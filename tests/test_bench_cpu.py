"""bench.py's contract pieces that run without a GPU: more than one GPU is refused
with a message, and the HBM traffic of the roofline objects comes from the committed
rocprofv3 summaries (one `traffic_bytes <kernel> <config> <bytes> [src=<file>@<sha12>]`
line each), with the kernel source digest the counters were taken on."""

import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.parametrize("n", [2, 8])
def test_bench_refuses_more_than_one_gpu(n):
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", str(n)],
                       capture_output=True, text=True, timeout=300, cwd=ROOT)
    assert r.returncode == 2
    assert "measures one GPU" in r.stderr and f"--gpus {n}" in r.stderr
    assert r.stdout == ""             # no JSON line


def test_profiled_traffic_lines():
    sys.path.insert(0, ROOT)
    try:
        import bench
    finally:
        sys.path.remove(ROOT)
    dense = bench.profiled_traffic("gsa_dense_attn", "c3")
    idx = bench.profiled_traffic("gsa_indexer_select", "c3")
    gather = bench.profiled_traffic("gsa_sparse_attn", "c3")
    # each kernel's HBM bytes per launch at c3, from FETCH_SIZE/WRITE_SIZE: the dense
    # kernel streams K and V^T tiles (128 MiB) through L2 many times; the indexer
    # reads q_I, k_I, w (10 MiB) and writes the 32 MiB bitmask, storing no score
    # (a stored causal score matrix alone would be 537 MB); the gather kernel misses
    # L2 on most of its 258 GB of gathered rows
    assert dense is not None and 0.5e9 < dense["bytes"] < 5e9
    assert idx is not None and 0.044e9 < idx["bytes"] < 0.537e9
    assert gather is not None and 1e11 < gather["bytes"] < 3e11
    assert bench.profiled_traffic("gsa_dense_attn", "c9") is None
    # every figure names the summary it came from and the kernel source digest it
    # was measured on; source_matches compares that digest with today's file
    for prof, kernel in ((dense, "gsa_dense_attn"), (idx, "gsa_indexer_select"), (gather, "gsa_sparse_attn")):
        assert prof["source"].startswith("profiles/") and os.path.exists(os.path.join(ROOT, prof["source"]))
        assert prof["kernel_source"] == f"{bench.KERNEL_SOURCES[kernel]}@{bench.source_digest(kernel)}"
        assert prof["source_matches"] == (prof["measured_on_source"] == prof["kernel_source"])
