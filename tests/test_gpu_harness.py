"""The benchmark harness on the GPU: verification of the drop-in layer against
the oracle layer (tests/oracle_layer.py) through the harness's own verify, the
sweep and its JSON report, and both rocprofv3 capture-window modes.

At the verification length T=512 (k_max clipped to T, so k_eff = T) every row
attends to all of its causal keys, so the selection cannot differ between the
oracle and the kernels and the fp32 bar is 1e-4."""

import json
import os

import pytest
import torch

from gsa_gdn_benchmarkstudy_amd import GatedSparseAttention, harness

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_LAYER = os.path.join(HERE, "oracle_layer.py")


def _log(msg):
    print(msg, flush=True)


@pytest.mark.parametrize("dtype,atol,rtol,rel", [(torch.bfloat16, 2e-2, 1e-2, 2e-2),
                                                 (torch.float32, 1e-4, 1e-4, 1e-4)])
@pytest.mark.parametrize("attn", ["auto", "gather"])
def test_harness_verify_against_oracle_layer(dev, dtype, atol, rtol, rel, attn):
    if attn == "auto" and dtype == torch.float32:
        pytest.skip("auto is the gather kernel in fp32")
    _log(f"harness verify T=512 {dtype} attn={attn}")
    ref_cls = harness.load_layer_class(ORACLE_LAYER)
    res = harness.verify(ref_cls, GatedSparseAttention, dev, dtype, T=512, atol=atol, rtol=rtol,
                         attn_impl=None if attn == "auto" else attn, out=_log)
    assert res.passed, res
    assert res.rel_l2 < rel, res


def test_harness_sweep_and_json(dev, tmp_path):
    path = tmp_path / "sweep.json"
    _log("harness main --skip-verify --T 512,2048")
    rc = harness.main(["--skip-verify", "--T", "512,2048", "--warmup", "1", "--iters", "2",
                       "--json", str(path)], out=_log)
    assert rc == 0
    rep = json.loads(path.read_text())
    assert rep["verify"] == "skipped" and rep["ref"] == []
    rows = rep["opt"]
    assert [r["T"] for r in rows] == [512, 2048]
    for r in rows:
        assert r["status"] == "ok", r
        assert r["ms"] > 0 and r["mem_mb"] > 0
        assert r["tok_per_s"] == pytest.approx(r["B"] * r["T"] / (r["ms"] / 1e3))


def test_harness_main_verifies_and_summarises(dev, tmp_path):
    path = tmp_path / "full.json"
    lines = []

    def out(msg):
        lines.append(msg)
        _log(msg)

    rc = harness.main(["--ref", ORACLE_LAYER, "--T", "512", "--warmup", "1", "--iters", "1",
                       "--json", str(path)], out=out)
    assert rc == 0
    rep = json.loads(path.read_text())
    assert rep["verify"]["passed"] and rep["verify"]["T"] == 512
    assert rep["ref"][0]["status"] == "ok" and rep["opt"][0]["status"] == "ok"
    assert any("Summary" in ln for ln in lines)


@pytest.mark.parametrize("flags", [["--profile", "--profile-T", "1024", "--profile-opt-only"],
                                   ["--ncu", "--ncu-T", "1024", "--ncu-opt-only"]])
def test_harness_capture_modes(dev, flags):
    _log(f"harness main {' '.join(flags)}")
    assert harness.main(flags + ["--warmup", "1"], out=_log) == 0


def test_harness_sweep_graph(dev, tmp_path):
    path = tmp_path / "graph.json"
    _log("harness main --skip-verify --graph --T 512,1024")
    rc = harness.main(["--skip-verify", "--graph", "--T", "512,1024", "--warmup", "1", "--iters", "3",
                       "--json", str(path)], out=_log)
    assert rc == 0
    rep = json.loads(path.read_text())
    assert rep["graph"] is True
    assert [r["status"] for r in rep["opt"]] == ["ok", "ok"]
