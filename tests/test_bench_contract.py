"""bench.py's output contract: one JSON line with the fields the driver reads
(GPU: a short run end to end), and a refusal of more than one GPU (CPU)."""

import json
import pathlib
import subprocess
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=300, cwd=str(ROOT))
    assert r.returncode != 0
    assert "single GPU" in r.stderr + r.stdout


@pytest.mark.gpu
def test_short_run_prints_one_json_line_with_the_contract_fields():
    r = subprocess.run([sys.executable, "-u", str(ROOT / "bench.py"), "--steps", "2", "--warmup",
                        "1", "--latency-chunks", "3", "--no-cpu", "--no-configs"],
                       capture_output=True, text=True, timeout=280, cwd=str(ROOT))
    assert r.returncode == 0, r.stderr[-2000:]
    lines = [ln for ln in r.stdout.splitlines() if ln.strip()]
    assert len(lines) == 1, r.stdout[-2000:]
    b = json.loads(lines[0])
    for k in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step",
              "higher_is_better", "scaling", "vs_baseline", "dtype", "config", "roofline",
              "cpu_baseline", "latency_bs1", "output_check"):
        assert k in b, k
    assert b["unit"] == "chunks/s" and b["n_gpus"] == 1 and b["dtype"] == "bf16"
    assert b["steps"] == 2 and b["warmup"] == 1 and b["higher_is_better"] is True
    assert b["value"] > 0 and b["ms_per_step"] > 0
    assert abs(b["value"] - b["config"]["global_batch"] / b["ms_per_step"] * 1e3) < 0.01 * b["value"]
    assert "workload" in b["config"] and b["config"]["global_batch"] == 32
    ro = b["roofline"]
    for k in ("bound", "achieved", "peak", "unit", "frac", "traffic"):
        assert k in ro, k
    assert 0 < ro["frac"] <= 1 and abs(ro["achieved"] / ro["peak"] - ro["frac"]) < 1e-3
    assert b["output_check"]["finite"] is True
    assert b["latency_bs1"]["ms_per_chunk_median"] > 0
