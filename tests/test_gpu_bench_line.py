"""bench.py's JSON line on the GPU: one line with the driver's keys, the metric and workload of
BASELINE.json's configuration (config 2, event mode), the roofline object of the dominant
kernel and the CPU baseline of the oracle, from a short run (2 timed steps, a 30-tick CPU
sample); and the op-level line of `bench.py --op`."""
import json
import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_bench_json_line():
    r = subprocess.run([sys.executable, os.path.join(HERE, "bench.py"), "--steps", "2", "--warmup", "1"],
                       cwd=HERE, capture_output=True, text=True, timeout=240)
    assert r.returncode == 0, r.stderr[-2000:]
    lines = [ln for ln in r.stdout.strip().splitlines() if ln.startswith("{")]
    assert len(lines) == 1
    d = json.loads(lines[0])
    for k in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better",
              "scaling", "vs_baseline", "dtype", "data", "config", "roofline", "cpu_baseline"):
        assert k in d, k
    assert d["n_gpus"] == 1 and d["steps"] == 2 and d["warmup"] == 1 and d["higher_is_better"] is True
    assert d["unit"] == "neuron-timesteps/s" and d["dtype"] == "f32" and d["data"] == "synthetic"
    assert d["config"]["neurons"] == 66000 and d["config"]["batch"] == 5 and d["config"]["seq_len"] == 500
    assert "config 2" in d["config"]["workload"]
    # value is the whole job's rate: B * N * T neuron-timesteps per step
    assert abs(d["value"] - 5 * 66000 * 500 / (d["ms_per_step"] / 1000)) <= 1e-3 * d["value"]
    rf = d["roofline"]
    for k in ("bound", "achieved", "peak", "unit", "frac", "traffic"):
        assert k in rf, k
    assert rf["peak"] == 8000.0 and rf["unit"] == "GB/s" and 0 < rf["frac"] < 1
    assert abs(rf["frac"] - rf["achieved"] / rf["peak"]) < 1e-3
    cb = d["cpu_baseline"]
    assert cb["value"] > 0 and cb["cores"] >= 1 and cb["kind"] in ("port", "reference") and cb["sample"]


@pytest.mark.parametrize("table,batch", [("rec", 5), ("lgn", 32), ("bkg", 5)])
def test_bench_op_line(table, batch):
    """bench.py --op on each config-2 table: one JSON line naming the table and batch, with the
    three per-call timings (forward in both modes, custom gradient) positive."""
    r = subprocess.run([sys.executable, os.path.join(HERE, "bench.py"), "--op", "--op-table", table,
                        "--op-batch", str(batch), "--steps", "2", "--warmup", "1"],
                       cwd=HERE, capture_output=True, text=True, timeout=240)
    assert r.returncode == 0, r.stderr[-2000:]
    lines = [ln for ln in r.stdout.strip().splitlines() if ln.startswith("{")]
    assert len(lines) == 1
    d = json.loads(lines[0])
    assert d["config"]["table"] == table and d["config"]["batch"] == batch
    assert d["higher_is_better"] is False and d["n_gpus"] == 1
    us = d["us_per_call"]
    assert set(us) == {"fwd_event", "fwd_deterministic", "bwd"} and all(v > 0 for v in us.values())
    assert abs(d["value"] - (us["fwd_event"] + us["bwd"])) <= 0.02
