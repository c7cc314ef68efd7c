"""The measurement script's contract, checked on the CPU: the multi-GPU
request is refused with a message, the roofline's HBM traffic figure is read
from the committed rocprofv3 summary, and the JSON line carries every field
the driver reads."""
import json
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))

import bench  # noqa: E402


def test_more_than_one_gpu_is_refused_with_a_message():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode != 0
    assert "one GPU" in r.stderr and r.stdout.strip() == ""


def test_traffic_figure_comes_from_the_committed_profile():
    t = bench._profiled_traffic()
    text = bench.TRAFFIC_PROFILE.read_text()
    assert t is not None and f"traffic_bytes_per_launch = {t}" in text
    assert 1e8 < t < 1e10  # bytes per GEMM launch of the GPT-2 small step


def test_json_line_has_the_driver_fields():
    class A:
        steps, warmup, dtype = 10, 2, "float32"
    roof = {"bound": "mfma", "achieved": 1.0, "peak": 157.3, "unit": "TFLOP/s", "frac": 1.0 / 157.3, "traffic": None}
    cpu = {"value": 1.0, "unit": "tokens/s", "cores": 1, "kind": "port", "sample": "s"}
    line = bench._line("m", 2.0, "tokens/s", A(), 3.0, {"workload": "w"}, roof, cpu)
    d = json.loads(json.dumps(line))
    for k in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better", "scaling",
              "vs_baseline", "dtype", "data", "config", "roofline", "cpu_baseline"):
        assert k in d, k
    assert d["n_gpus"] == 1 and d["dtype"] == "f32" and d["vs_baseline"] is None
    assert set(roof) <= set(d["roofline"]) and set(cpu) <= set(d["cpu_baseline"])
