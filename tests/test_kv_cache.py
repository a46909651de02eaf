"""Incremental decoding with KV caches (MultiHeadAttention::forward_cached,
GPTModel::forward_cached in inferno_amd/app/gpt.cpp) against the full causal
forward of the same tokens: the logits at every position must agree.

This pins the cache bookkeeping (slot positions, the end-aligned causal mask
of a chunked prefill, the single-query decode path, the positional table
offset): an off-by-one in any of them changes the logits at that position by
far more than the tolerance.  Bar: max|inc - full| / max|full| <= 1e-4 (fp32).
"""
import subprocess
from pathlib import Path

import numpy as np
import pytest

from oracle import gpt as ogpt

ROOT = Path(__file__).resolve().parents[1]
APP = ROOT / "inferno_amd" / "gpt"


def run_check(tmp_path, device, L, C, H, T, V, B, P):
    if not APP.exists():
        pytest.skip("inferno_amd/gpt not built")
    params = ogpt.init_params(L, C, V, seed=5)
    (tmp_path / "config.txt").write_text(f"{L} {C} {H} {T} {V} {B}\n")
    rng = np.random.default_rng(11)
    rng.integers(0, V, size=(B, T), dtype=np.int32).tofile(tmp_path / "tokens.bin")
    for name, val in params.items():
        np.ascontiguousarray(val, np.float32).tofile(tmp_path / f"{name}.bin")
    r = subprocess.run([str(APP), "decode-check", str(tmp_path), device, "--prefill", str(P)],
                       capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stdout + r.stderr
    full = np.fromfile(tmp_path / "logits_full.bin", np.float32).reshape(B, T, V)
    inc = np.fromfile(tmp_path / "logits_inc.bin", np.float32).reshape(B, T, V)
    err = np.abs(inc.astype(np.float64) - full).max(axis=(0, 2)) / np.abs(full).max()
    assert err.max() <= 1e-4, err


def test_kv_cache_cpu(tmp_path):
    run_check(tmp_path, "cpu", L=2, C=32, H=1, T=12, V=40, B=2, P=5)


@pytest.mark.gpu
@pytest.mark.parametrize("P", [1, 7, 33])
def test_kv_cache_hip(tmp_path, P):
    print(f"[case] kv cache hip prefill {P}", flush=True)
    run_check(tmp_path, "hip", L=2, C=128, H=2, T=70, V=96, B=3, P=P)
