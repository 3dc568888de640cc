"""bench.py's output contract: one JSON line with the metric, the value and
its unit, the run's shape, the roofline object of the attention kernel (its
achieved rate from HIP events against the dense bf16 peak, and its HBM bytes
per launch from the committed counter measurement), and a refusal of more
than one GPU.  The GPU case runs a short bench (AWA layers only) in a child
process."""
import json
import math
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120, cwd=ROOT)
    assert r.returncode == 2 and "one GPU" in r.stderr and not r.stdout.strip()


@pytest.mark.gpu
def test_json_line_contract():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--steps", "2", "--warmup", "1", "--no-dit",
                        "--no-configs", "--no-cpu-baseline"], capture_output=True, text=True, timeout=300, cwd=ROOT)
    assert r.returncode == 0, r.stderr[-3000:]
    lines = [l for l in r.stdout.strip().split("\n") if l.strip()]
    assert len(lines) == 1, r.stdout[-2000:]
    d = json.loads(lines[0])
    for k in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better",
              "scaling", "vs_baseline", "dtype", "data", "config", "roofline"):
        assert k in d, k
    assert d["n_gpus"] == 1 and d["steps"] == 2 and d["warmup"] == 1
    assert d["higher_is_better"] is False and d["scaling"] in ("weak", "strong")
    assert d["value"] == d["ms_per_step"] and 0 < d["value"] < 10
    assert d["dtype"] == "bf16" and "synthetic" in d["data"]
    assert d["config"]["workload"] and "model" not in d["config"]
    rf = d["roofline"]
    for k in ("bound", "achieved", "peak", "unit", "frac", "traffic"):
        assert k in rf, k
    assert rf["bound"] == "mfma" and rf["unit"] == "TFLOP/s" and rf["peak"] == 2500.0
    assert 0 < rf["frac"] < 1 and math.isclose(rf["frac"], rf["achieved"] / rf["peak"], rel_tol=1e-3, abs_tol=1e-4)
    assert rf["traffic"] is None or rf["traffic"] > 0
