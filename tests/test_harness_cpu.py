"""Host logic of the benchmark harness (gsa_gdn_benchmarkstudy_amd/harness.py),
without a GPU: failure classification, the sweep's OOM/ERR rows, the summary
table, the CLI (including the reference's flag names), loading a reference
layer from a file, verification plumbing on the CPU oracle layer, and the
ROCTx capture-window calls."""

import json
import os
import textwrap

import pytest
import torch

from gsa_gdn_benchmarkstudy_amd import harness, roctx

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_LAYER = os.path.join(HERE, "oracle_layer.py")


def _silent(_msg):
    pass


def test_classify_failure():
    assert harness.classify_failure(torch.OutOfMemoryError("HIP out of memory. Tried to allocate")) == "OOM"
    assert harness.classify_failure(RuntimeError("CUDA out of memory. Tried to allocate 2 GiB")) == "OOM"
    assert harness.classify_failure(RuntimeError("hipErrorOutOfMemory: Out Of Memory")) == "OOM"
    assert harness.classify_failure(RuntimeError("gsa_dense_attn: unsupported shape")) == "ERR"
    assert harness.classify_failure(ValueError("hidden size 512 != 2048")) == "ERR"


def test_layer_kwargs_clip_k_max_to_T():
    assert harness.layer_kwargs(512)["k_max"] == 512
    assert harness.layer_kwargs(16384)["k_max"] == 4096
    kw = harness.layer_kwargs(4096, D=1024)
    assert kw["hidden_size"] == 1024 and kw["k_base"] == 2048 and kw["k_min"] == 256
    assert kw["num_heads"] == 16 and kw["d_indexer"] == 64 and kw["n_idx_heads"] == 4


class _TinyLayer(torch.nn.Module):
    """Stand-in layer: fails with OOM at T=64 and with a shape error at T=96."""

    def __init__(self, hidden_size, num_heads, k_max, d_indexer, n_idx_heads, k_base, k_min):
        super().__init__()
        self.lin = torch.nn.Linear(hidden_size, hidden_size, bias=False)
        self.k_max = k_max

    def forward(self, x):
        T = x.shape[1]
        if T == 64:
            raise torch.OutOfMemoryError("HIP out of memory. Tried to allocate 9.00 GiB")
        if T == 96:
            raise RuntimeError("gsa_indexer_select: unsupported shape")
        return self.lin(x)


def test_sweep_rows_ok_oom_err():
    pts = [(1, 32, 64), (1, 64, 64), (2, 96, 64), (2, 128, 64)]
    rows = harness.sweep(_TinyLayer, "tiny", pts, "cpu", torch.float32, warmup=1, iters=2,
                         timer=harness.wall_timer, out=_silent)
    assert [r.status for r in rows] == ["ok", "OOM", "ERR", "ok"]
    assert [r.key for r in rows] == pts
    for r in (rows[0], rows[3]):
        assert r.ms > 0 and r.tok_per_s == pytest.approx(r.B * r.T / (r.ms / 1e3))
        assert r.error == ""
    assert rows[1].ms is None and rows[1].tok_per_s is None and "out of memory" in rows[1].error
    assert rows[2].ms is None and "unsupported shape" in rows[2].error
    lines = [harness.format_row(r) for r in rows]
    assert "OOM" in lines[1] and "ERR" in lines[2] and "unsupported" in lines[2]


def test_summary_pairs_points_and_ratios():
    R, O = harness.Row, "ok"
    ref = [R(1, 512, 2048, O, 10.0, 51200.0, 400.0),
           R(1, 1024, 2048, "OOM", error="out of memory"),
           R(1, 2048, 2048, O, 30.0, 1.0, 900.0)]
    opt = [R(1, 512, 2048, O, 2.5, 204800.0, 100.0),
           R(1, 1024, 2048, O, 3.0, 1.0, 120.0),
           R(1, 2048, 2048, "ERR", error="boom"),
           R(1, 4096, 2048, O, 4.0, 1.0, 200.0)]
    lines = harness.summary_lines(ref, opt)
    body = lines[5:]
    assert len(body) == 4
    assert "10.00" in body[0] and "2.50" in body[0] and "4.00x" in body[0]
    assert "400" in body[0] and "100" in body[0]
    assert "OOM" in body[1] and "N/A" in body[1]
    assert "ERR" in body[2] and "N/A" in body[2]
    assert body[3].split("|")[1].strip() == "-" and "N/A" in body[3]


def test_cli_defaults_and_reference_flag_names():
    a = harness.parse_args([])
    assert a.dtype == "bf16" and (a.atol, a.rtol) == (2e-2, 1e-2)
    assert a.T == list(harness.DEFAULT_T) and a.B == 1 and a.verify_T == 512
    assert not a.profile and not a.counters and a.ref is None
    a = harness.parse_args(["--dtype", "fp32"])
    assert (a.atol, a.rtol) == (1e-4, 1e-4)
    a = harness.parse_args(["--ncu", "--ncu-T", "4096", "--ncu-opt-only", "--T", "512,2048",
                            "--skip-verify", "--atol", "0.1"])
    assert a.counters and a.counters_T == 4096 and a.counters_opt_only
    assert a.T == [512, 2048] and a.skip_verify and a.atol == 0.1
    a = harness.parse_args(["--profile", "--profile-T", "16384", "--profile-ref-only"])
    assert a.profile and a.profile_T == 16384 and a.profile_ref_only
    with pytest.raises(SystemExit):
        harness.parse_args(["--profile-ref-only", "--profile-opt-only"])
    with pytest.raises(SystemExit):
        harness.parse_args(["--T", "0"])


def test_main_needs_a_gpu():
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    msgs = []
    assert harness.main(["--skip-verify"], out=msgs.append) == 1
    assert "GPU is required" in msgs[0]


def test_load_layer_class_from_file_and_module(tmp_path):
    (tmp_path / "sibling_helper.py").write_text("VALUE = 7\n")
    (tmp_path / "my_ref.py").write_text(textwrap.dedent("""
        import sibling_helper
        class GatedSparseAttention:
            tag = sibling_helper.VALUE
    """))
    cls = harness.load_layer_class(str(tmp_path / "my_ref.py"))
    assert cls.tag == 7
    assert harness.load_layer_class("tests.oracle_layer").__name__ == "GatedSparseAttention"
    (tmp_path / "empty.py").write_text("X = 1\n")
    with pytest.raises(AttributeError):
        harness.load_layer_class(str(tmp_path / "empty.py"))
    with pytest.raises(FileNotFoundError):
        harness.load_layer_class(str(tmp_path / "missing.py"))


def test_verify_plumbing_on_the_oracle_layer():
    """Reference and candidate both the oracle layer on the CPU: identical weights
    (strict state-dict copy) and input give a zero difference; a candidate whose
    output is shifted by more than the tolerance fails."""
    ref_cls = harness.load_layer_class(ORACLE_LAYER)

    class Shifted(ref_cls):
        def forward(self, x, attention_mask=None):
            return super().forward(x) + 0.05

    kw = dict(hidden_size=256, num_heads=2)
    orig = harness.layer_kwargs
    harness.layer_kwargs = lambda T, D=256: {**orig(T, D), **kw}
    try:
        ok = harness.verify(ref_cls, ref_cls, "cpu", torch.float32, T=48, atol=1e-4, rtol=1e-4,
                            out=_silent)
        bad = harness.verify(ref_cls, Shifted, "cpu", torch.float32, T=48, atol=1e-2, rtol=1e-2,
                             out=_silent)
    finally:
        harness.layer_kwargs = orig
    assert ok.passed and ok.max_diff == 0.0 and ok.mean_diff == 0.0
    assert not bad.passed and bad.max_diff == pytest.approx(0.05, rel=1e-3)


def test_json_report_round_trip(tmp_path):
    rows = [harness.Row(1, 512, 2048, "ok", 1.0, 512000.0, 10.0),
            harness.Row(1, 1024, 2048, "OOM", error="out of memory")]
    path = tmp_path / "sub" / "r.json"
    harness._write_json(str(path), {"opt": [harness.asdict(r) for r in rows]})
    back = json.loads(path.read_text())
    assert back["opt"][1]["status"] == "OOM" and back["opt"][1]["ms"] is None
    assert back["opt"][0]["tok_per_s"] == 512000.0


def test_roctx_calls_are_safe_without_a_profiler():
    assert roctx.range_push("harness/test") in (0, 1)
    assert roctx.range_pop() in (0, -1)
    roctx.mark("harness/mark")
    assert roctx.profiler_resume() == 0 and roctx.profiler_pause() == 0
    with roctx.region("harness/region"):
        pass
