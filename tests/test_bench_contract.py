"""bench.py's output contract: one JSON line with the headline metric of BASELINE.json, the
roofline object of the timed backward call and the CPU baseline; one GPU only."""
import json
import os
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
BENCH = ROOT / "bench.py"
F_FWD_BWD = 3.5 * 2.0 * 8 * 12 * 1024 * 1024 * 64  # 45.097 GFLOP, causal FlashAttention convention


def run_bench(*args, env=None, timeout=600):
    e = dict(os.environ)
    e.update(env or {})
    return subprocess.run([sys.executable, str(BENCH), *map(str, args)], capture_output=True, text=True,
                          timeout=timeout, cwd=str(ROOT), env=e)


def last_json(stdout):
    lines = [l for l in stdout.splitlines() if l.startswith("{")]
    assert lines, "no JSON line printed"
    return json.loads(lines[-1])


@pytest.mark.parametrize("args,env", [(["--gpus", "2"], {}), (["--gpus", "1"], {"WORLD_SIZE": "4"})])
def test_bench_refuses_more_than_one_gpu(args, env):
    """More than one GPU exits with status 2 and a JSON error before touching a device."""
    r = run_bench(*args, env=env, timeout=120)
    assert r.returncode == 2, r.stdout + r.stderr
    assert "one GPU" in last_json(r.stdout)["error"]


@pytest.mark.gpu
def test_bench_json_line():
    """A short run: every field of the contract, values consistent with each other."""
    print("[case] bench.py short run", flush=True)
    r = run_bench("--steps", 3, "--warmup", 1, "--clock-warmup-s", 0.05, "--cpu-heads", 1, "--cpu-c4-rows", 8,
                  "--no-decode", "--no-extras")
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    d = last_json(r.stdout)
    baseline = json.loads((ROOT / "BASELINE.json").read_text())
    assert d["metric"] == baseline["metric"]
    assert d["unit"] == "TFLOP/s" and d["n_gpus"] == 1 and d["steps"] == 3 and d["warmup"] == 1
    assert d["higher_is_better"] is True and d["scaling"] in ("weak", "strong") and d["dtype"] == "f32"
    assert d["vs_baseline"] is None and d["data"].startswith("synthetic")
    assert d["config"]["B"] == 8 and d["config"]["H"] == 12 and d["config"]["T"] == 1024 and d["config"]["D"] == 64
    # value is the whole step's FLOPs over the measured step time
    assert d["value"] > 0 and abs(d["value"] - F_FWD_BWD / (d["ms_per_step"] * 1e-3) / 1e12) <= 0.01 * d["value"]
    ro = d["roofline"]
    assert ro["bound"] == "mfma" and ro["unit"] == "TFLOP/s" and ro["peak"] == 157.3
    assert abs(ro["frac"] - ro["achieved"] / ro["peak"]) <= 1e-3
    assert ro["traffic"] > 0 and ro["achieved"] > 0
    assert abs(ro["achieved"] - ro["algorithmic_flop_per_launch"] / (ro["avg_launch_ms"] * 1e-3) / 1e12) <= 0.01 * ro["achieved"]
    cb = d["cpu_baseline"]
    assert cb["kind"] in ("port", "reference") and cb["cores"] == 1 and cb["value"] > 0 and cb["unit"] == "TFLOP/s"
    assert cb["sample"]
