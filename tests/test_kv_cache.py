"""Incremental decoding with KV caches (MultiHeadAttention::forward_cached,
GPTModel::forward_cached in inferno_amd/app/gpt.cpp) against the oracle.

The reference has no generation loop, only the commented-out select of the last
position's logits (InfernoApp/main.cpp:1173-1177); its parity bar is its own
CPU forward.  So the oracle's causal forward of the whole token sequence
(oracle/gpt.py gpt_logits: the reference chain per layer) is the reference for
the logits at every position, whether they were produced by one full forward,
by a prefill of P tokens or by single-token steps through the caches.  An
off-by-one in the slot positions, the end-aligned causal mask of a chunked
prefill, the single-query decode path or the positional table offset changes
the logits at that position by far more than the tolerance.

Bar: max|x - ref| / max|ref| <= 1e-4 (fp32) per position.  Greedy generation:
every picked token is an argmax of the oracle's logits at its position, up to
ties within that tolerance.
"""
import subprocess
from pathlib import Path

import numpy as np
import pytest

from oracle import gpt as ogpt

ROOT = Path(__file__).resolve().parents[1]
APP = ROOT / "inferno_amd" / "gpt"
TOL = 1e-4


def write_case(tmp_path, L, C, H, T, V, B, seed=5):
    params = ogpt.init_params(L, C, V, seed=seed)
    (tmp_path / "config.txt").write_text(f"{L} {C} {H} {T} {V} {B}\n")
    for name, val in params.items():
        np.ascontiguousarray(val, np.float32).tofile(tmp_path / f"{name}.bin")
    return params


def run_app(*args):
    if not APP.exists():
        pytest.skip("inferno_amd/gpt not built")
    r = subprocess.run([str(APP), *map(str, args)], capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stdout + r.stderr


def per_position_err(x, ref):
    return np.abs(x.astype(np.float64) - ref).max(axis=(0, 2)) / np.abs(ref).max()


def run_check(tmp_path, device, L, C, H, T, V, B, P):
    params = write_case(tmp_path, L, C, H, T, V, B)
    rng = np.random.default_rng(11)
    tokens = rng.integers(0, V, size=(B, T), dtype=np.int32)
    tokens.tofile(tmp_path / "tokens.bin")
    run_app("decode-check", tmp_path, device, "--prefill", P)
    ref = ogpt.gpt_logits(params, tokens, L, C, H)
    full = np.fromfile(tmp_path / "logits_full.bin", np.float32).reshape(B, T, V)
    inc = np.fromfile(tmp_path / "logits_inc.bin", np.float32).reshape(B, T, V)
    e_full, e_inc = per_position_err(full, ref), per_position_err(inc, ref)
    assert e_full.max() <= TOL, ("full forward", e_full)
    assert e_inc.max() <= TOL, ("prefill", P, "then cached steps", e_inc)


def test_kv_cache_cpu(tmp_path):
    run_check(tmp_path, "cpu", L=2, C=32, H=1, T=12, V=40, B=2, P=5)


@pytest.mark.gpu
@pytest.mark.parametrize("P", [1, 7, 33])
def test_kv_cache_hip(tmp_path, P):
    print(f"[case] kv cache hip prefill {P}", flush=True)
    run_check(tmp_path, "hip", L=2, C=128, H=2, T=70, V=96, B=3, P=P)


def check_generation(tmp_path, device, L, C, H, T, V, B, P, N):
    params = write_case(tmp_path, L, C, H, T, V, B, seed=21)
    rng = np.random.default_rng(12)
    prompt = rng.integers(0, V, size=(B, P), dtype=np.int32)
    prompt.tofile(tmp_path / "tokens.bin")
    run_app("generate-check", tmp_path, device, "--prompt", P, "--new", N)
    gen = np.fromfile(tmp_path / "generated.bin", np.int32).reshape(B, N)
    glog = np.fromfile(tmp_path / "gen_logits.bin", np.float32).reshape(B, N, V)
    # the oracle's logits over the sequence the app generated (teacher forcing on its picks)
    seq = np.concatenate([prompt, gen[:, :-1]], axis=1)
    ref = ogpt.gpt_logits(params, seq, L, C, H)[:, P - 1:]  # [B, N, V]: the positions picks were made at
    scale = np.abs(ref).max()
    assert per_position_err(glog, ref).max() <= TOL
    rows = np.arange(B)[:, None]
    picked = ref[rows, np.arange(N)[None, :], gen]
    best = ref.max(axis=2)
    assert (picked >= best - TOL * scale).all(), "a pick is not an argmax of the oracle's logits"
    # where the oracle's top two are separated by more than the tolerance the pick is exact
    top2 = np.sort(ref, axis=2)[:, :, -2:]
    clear = top2[:, :, 1] - top2[:, :, 0] > 2 * TOL * scale
    assert clear.mean() > 0.9
    assert (gen[clear] == ref.argmax(axis=2)[clear]).all()


def test_generation_cpu(tmp_path):
    check_generation(tmp_path, "cpu", L=2, C=32, H=2, T=24, V=40, B=2, P=6, N=10)


@pytest.mark.gpu
@pytest.mark.parametrize("P", [1, 9])
def test_generation_hip(tmp_path, P):
    """Greedy generation on the device (argmax picked on HIP, one token per cached step)."""
    print(f"[case] generation hip prompt {P}", flush=True)
    check_generation(tmp_path, "hip", L=2, C=128, H=2, T=64, V=96, B=3, P=P, N=24)
