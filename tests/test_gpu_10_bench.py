"""bench.py runs and prints its one-line JSON contract (run with -m gpu).

Short runs of the default workload and of the optional feed-forward, router
and separate-shared-expert modes, each in a child process as the driver runs
it, so a broken code path in bench.py fails here rather than at the end of a
round.
"""
import json
import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
if not torch.cuda.is_available():
    pytest.skip("needs a GPU", allow_module_level=True)

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
KEYS = {"metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better", "scaling",
        "vs_baseline", "dtype", "data", "config", "roofline", "cpu_baseline"}


def run_bench(*args):
    cmd = [sys.executable, os.path.join(ROOT, "bench.py"), "--steps", "3", "--warmup", "1", *args]
    print("[bench]", " ".join(args), flush=True)
    r = subprocess.run(cmd, cwd=ROOT, capture_output=True, text=True, timeout=240)
    assert r.returncode == 0, r.stderr[-3000:]
    lines = [l for l in r.stdout.splitlines() if l.strip()]
    assert len(lines) == 1, r.stdout[-2000:]
    return json.loads(lines[0])


@pytest.mark.parametrize("args", [(), ("--workload", "c2", "--with-norm", "--with-router", "--no-cpu-baseline"),
                                  ("--workload", "c5d", "--weight-layout", "row_major", "--no-cpu-baseline"),
                                  ("--workload", "c4", "--no-cpu-baseline")])
def test_bench_prints_the_contract(args):
    d = run_bench(*args)
    assert KEYS <= set(d)
    assert d["value"] > 0 and d["ms_per_step"] > 0 and d["n_gpus"] == 1
    rf = d["roofline"]
    assert rf["bound"] in ("hbm", "mfma") and 0 < rf["frac"] < 1
    if not args:  # the default run: decode headline, c3 prefill sub-object, CPU baselines, timing rounds
        assert d["cpu_baseline"]["value"] > 0 and d["cpu_baseline"]["cores"] >= 1
        assert d["cpu_baseline"]["nproc"] >= d["cpu_baseline"]["cores"]
        assert rf["bound"] == "hbm" and rf["kernel"] == "gate_up_fused"
        assert d["config"]["weight_banks"] >= 4
        t = d["timing"]
        assert t["rounds"] == 7 and len(t["rotating_eager_rounds_ms"]) == 7
        assert t["hot_eager_ms"] > 0 and t["rotating_graph_ms"] > 0 and t["hot_graph_ms"] > 0
        p = d["prefill"]
        assert p["config"]["workload"] == "c3_30b_a3b_prefill" and p["config"]["tile_rows"] >= 64
        assert p["value"] > 0 and p["roofline"]["bound"] in ("hbm", "mfma") and 0 < p["roofline"]["frac"] < 1
        assert 0 < p["layer_roofline"]["mfma_frac"] < 1 and p["cpu_baseline"]["value"] > 0


def test_bench_rejects_more_than_one_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], cwd=ROOT,
                       capture_output=True, text=True, timeout=120)
    assert r.returncode != 0 and "one GPU" in r.stderr
