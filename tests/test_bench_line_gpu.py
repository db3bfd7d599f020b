"""bench.py's result line (the driver parses the last stdout line): a short run in a child process must end with
one compact JSON object holding the headline fields, the roofline and the CPU baseline, with the dominant
launch timed inside the timed region (avg_launch_us <= ms_per_step * 1000), and the detail record on stderr."""
import json
import subprocess
import sys
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu
ROOT = Path(__file__).resolve().parent.parent


def test_bench_result_line_is_compact_and_consistent(cuda):
    print("running bench.py --steps 5 --warmup 2 --no-extras --no-decode", flush=True)
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--steps", "5", "--warmup", "2", "--no-extras",
                        "--no-decode"], capture_output=True, text=True, timeout=240, cwd=str(ROOT))
    assert r.returncode == 0, r.stderr[-3000:]
    last = r.stdout.strip().splitlines()[-1]
    assert len(last) < 4096, f"result line of {len(last)} characters"
    d = json.loads(last)
    for key in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better", "scaling",
                "vs_baseline", "dtype", "data", "config", "roofline", "cpu_baseline"):
        assert key in d, key
    assert d["n_gpus"] == 1 and d["steps"] == 5 and d["config"]["workload"]
    rf = d["roofline"]
    assert rf["bound"] == "hbm" and rf["unit"] == "GB/s" and rf["peak"] == 8000.0
    assert 0 < rf["frac"] < 1 and abs(rf["frac"] - rf["achieved"] / rf["peak"]) < 1e-3
    assert rf["avg_launch_us"] <= d["ms_per_step"] * 1000 * 1.0001
    cb = d["cpu_baseline"]
    assert cb["kind"] == "port" and cb["cores"] >= 1 and cb["value"] > 0 and cb["sample"]
    assert "bench-detail: {" in r.stderr
    detail = json.loads(r.stderr.split("bench-detail: ", 1)[1].splitlines()[0])
    assert "batched_per_class" in detail and "cpu_baseline" in detail
