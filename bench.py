"""Benchmark: causal attention fwd+bwd on one MI355X.

A step is one forward plus one backward pass of the fused causal attention
through the C-ABI (inf_attn_fwd + inf_attn_bwd) over the config-2 batch:
B=8 H=12 T=1024 D=64, fp32, Q/K/V/dO ~ N(0,1) from the seeded generator,
scale 1/sqrt(64), all inputs resident in HBM before timing.  Work is counted
with the FlashAttention causal convention: F_fwd = 2*B*H*T^2*D,
F_fwd+bwd = 3.5*F_fwd = 45.097 GFLOP.

Prints one JSON line.  Timing: untimed steps for a fixed 0.3 s (the GPU's
clocks ramp up over the first ~30 ms of sustained load, so a short warm-up
would time the ramp), then W untimed warm-up steps, then K steps between two
torch.cuda.synchronize() calls; per-entry-point durations come from HIP events
recorded on the launch stream around every call in a second pass of K steps.
The CPU baseline is the restated reference CPU path (oracle/liboracle.so, one
core) on a bounded sample of heads of the same workload.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

MFMA_FP32_PEAK_TFLOPS = 157.3   # MI355X dense fp32 matrix
MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 matrix
HBM_PEAK_GBS = 8000.0

# HBM bytes per launch (read + written) of the backward call's kernels at config 2, from
# rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE runs of this script, scaled by what the same
# counters read for a plain device copy (FETCH_SIZE x2.00, WRITE_SIZE x1.00).  fp32 bwd_main
# runs the split plan (partial dK / dV written and read back); the bf16 call adds the dQ
# conversion pass, and its pre pass only zeroes the dQ accumulator (the bf16 main kernel forms
# delta from O and dO itself).
BWD_TRAFFIC = {
    "f32": {"bwd_pre": 50.39e6 + 25.56e6, "bwd_main": 200.84e6 + 201.37e6},
    "bf16": {"bwd_zero": 0.03e6 + 25.17e6, "bwd_main": 83.94e6 + 107.60e6, "bwd_cvt": 25.20e6 + 12.58e6},
}
# where the figures above were measured (they are constants: re-measure after a kernel change)
BWD_TRAFFIC_SOURCE = "profiles/attn_c2_hbm_traffic.md (rocprofv3 --pmc FETCH_SIZE, WRITE_SIZE of bench.py at config 2)"

METRIC = "causal attn fwd+bwd TFLOP/s (B8 H12 T1024 D64 fp32) + % of MFMA peak"

# per-config lines that --only runs alone: (B, H, T, D, Q/K sigma, dtype, deterministic-dQ mode)
ONLY_CONFIGS = {
    "c2_bf16": (8, 12, 1024, 64, 1.0, "bf16", False),
    "c4_f32": (1, 16, 8192, 128, 3.0, "f32", False),
    "c4_bf16": (1, 16, 8192, 128, 3.0, "bf16", False),
    "c2_f32_deterministic": (8, 12, 1024, 64, 1.0, "f32", True),
    "c2_bf16_deterministic": (8, 12, 1024, 64, 1.0, "bf16", True),
}


def flops_fwd(B, H, T, D):
    return 2.0 * B * H * T * T * D  # 4*B*H*T^2*D / 2 (causal)


def _host_cpu():
    model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return model


def cpu_baseline(B, H, T, D, heads: int, c4_rows: int = 256, c4_heads: int = 0):
    """Time the restated reference CPU path on one pinned core: `heads` heads of config 2
    (fwd+bwd), the whole config-5 decode step, a row sample of config 4, and an estimate of the
    config-3 step.

    Config 4 (B1 H16 T8192 D128): the reference chain computes every entry of the T x T score
    square whatever the mask (cpu_matmul, then masked_fill), so its work per query row is the
    same for every row; the last `c4_rows` rows of one head against all 8192 keys (end-aligned
    causal, which the oracle takes as Tq < Tk) are timed and scaled by 8192 / c4_rows rows and
    16 heads.  With c4_heads > 0, whole heads are timed instead (over a minute each).

    Config 3 (the GPT step) would take hours on one core: it is estimated from the oracle's
    GEMM rate, timed on one of the step's products, times the step's GEMM FLOPs, plus its 12
    layers x 96 heads of attention at the per-head time of the config-2 sample.
    """
    import numpy as np

    import oracle

    prev = os.sched_getaffinity(0)
    core = min(prev)
    os.sched_setaffinity(0, {core})
    try:
        Hs = min(heads, B * H)
        q, k, v, do = oracle.attn_inputs(1, Hs, T, D, seed=42)
        t0 = time.perf_counter()
        oracle.attn_fwd(q, k, v)
        oracle.attn_bwd(q, k, v, do)
        dt = time.perf_counter() - t0
        f = 3.5 * flops_fwd(1, Hs, T, D)
        # config 5: one decode step, B32 H12 Tk2048 D64 (query sees every cached key)
        Bd, Hd, Tk = 32, 12, 2048
        kc, vc = oracle.randn(500, (Bd, Hd, Tk, D)), oracle.randn(501, (Bd, Hd, Tk, D))
        qd = oracle.randn(502, (Bd, Hd, 1, D))
        t1 = time.perf_counter()
        oracle.attn_fwd(qd, kc, vc)
        dt5 = time.perf_counter() - t1
        nbytes5 = 2 * Bd * Hd * Tk * D * 4 + 2 * Bd * Hd * D * 4
        extra = {
            "c5_decode": {"seconds": round(dt5, 4), "us_per_step": round(dt5 * 1e6, 1),
                          "GBs": round(nbytes5 / dt5 / 1e9, 3), "sample": "the whole step, B32 H12 Tk2048 D64"},
        }
        T4, D4, H4 = 8192, 128, 16
        F4 = 3.5 * flops_fwd(1, H4, T4, D4)
        if c4_heads > 0:
            q4, k4, v4, do4 = oracle.attn_inputs(1, c4_heads, T4, D4, seed=42, qk_sigma=3.0)
            t2 = time.perf_counter()
            oracle.attn_fwd(q4, k4, v4)
            oracle.attn_bwd(q4, k4, v4, do4)
            dt4 = time.perf_counter() - t2
            est = dt4 * H4 / c4_heads
            sample4 = f"{c4_heads} whole head(s) of 16, x{H4 / c4_heads:g} (extrapolated)"
        else:
            r = min(c4_rows, T4)
            q4 = oracle.randn(42, (1, 1, r, D4), 3.0)
            k4 = oracle.randn(43, (1, 1, T4, D4), 3.0)
            v4 = oracle.randn(44, (1, 1, T4, D4), 1.0)
            do4 = oracle.randn(45, (1, 1, r, D4), 1.0)
            t2 = time.perf_counter()
            oracle.attn_fwd(q4, k4, v4)
            oracle.attn_bwd(q4, k4, v4, do4)
            dt4 = time.perf_counter() - t2
            est = dt4 * (T4 / r) * H4
            sample4 = (f"the last {r} of 8192 query rows of one head against all 8192 keys, "
                       f"x{T4 / r:g} rows x16 heads (extrapolated: the reference computes the full score "
                       f"square, so every row costs the same)")
        extra["c4"] = {"seconds_timed": round(dt4, 3), "sample": sample4,
                       "extrapolated_s_for_config4": round(est, 1),
                       "TFLOPs": F4 / est / 1e12}
        # config 3: GEMM rate of the oracle's cpu_matmul on a Wqkv-shaped product, 256 rows
        a = oracle.randn(600, (256, 768))
        w = oracle.randn(601, (768, 2304))
        t3 = time.perf_counter()
        oracle.matmul(a, w)
        dt3 = time.perf_counter() - t3
        gemm_rate = 2.0 * 256 * 768 * 2304 / dt3
        L3, C3, V3, N3 = 12, 768, 8192, 8 * 1024
        # per layer: Wqkv (C x 3C), W_out (C x C), ff1 (C x 4C), ff2 (4C x C), forward + 2 backward
        # products each; plus the tied logits (C x V) forward and its 2 backward products
        gemm_flops = 3 * 2.0 * N3 * (L3 * (3 * C3 * C3 + C3 * C3 + 8 * C3 * C3) + C3 * V3)
        attn_s = L3 * 96 * (dt / Hs)
        step_s = gemm_flops / gemm_rate + attn_s
        extra["c3_gpt"] = {"estimated_s_per_step": round(step_s, 1), "tokens_per_s": round(N3 / step_s, 3),
                           "sample": f"estimated, not run: {gemm_flops / 1e12:.2f} TFLOP of GEMMs at the oracle's "
                                     f"{gemm_rate / 1e9:.2f} GFLOP/s (one 256x768x2304 product timed) plus "
                                     f"12 layers x 96 heads of attention at {dt / Hs:.2f} s per head "
                                     f"(the config-2 sample); element-wise work not counted"}
    finally:
        os.sched_setaffinity(0, prev)
    return {
        "value": f / dt / 1e12,
        "unit": "TFLOP/s",
        "cores": 1,
        "kind": "port",
        "sample": f"{Hs} of {B * H} heads (T={T}, D={D}) fwd+bwd through the restated reference "
                  f"CPU chain, {dt:.2f} s on one core pinned to CPU {core} of {os.cpu_count()} "
                  f"({_host_cpu()}); the backward recomputes the forward as the reference chain "
                  f"would; FLOPs counted with the causal convention",
        "seconds": dt,
        "host": {"cpu": _host_cpu(), "nproc": os.cpu_count(), "pinned_core": core},
        "configs": extra,
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    # The GPU's clocks ramp up over the first ~30 ms of sustained load (kernel
    # times fall by ~15% over that span): --clock-warmup-s of untimed steps run
    # before the W warm-up steps, so the timed steps see the clocks a long job sees.
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--clock-warmup-s", type=float, default=0.3,
                    help="seconds of untimed steps before the W warm-up steps (clock ramp)")
    ap.add_argument("--dtype", choices=["f32", "bf16"], default="f32")
    ap.add_argument("--cpu-heads", type=int, default=12, help="heads in the CPU-baseline sample (0 = skip)")
    ap.add_argument("--cpu-c4-rows", type=int, default=256, help="config-4 query rows timed on the CPU")
    ap.add_argument("--cpu-c4-heads", type=int, default=0,
                    help="time whole config-4 heads on the CPU instead of a row sample (over a minute each)")
    ap.add_argument("--deterministic", action="store_true",
                    help="run the main line's backward in the deterministic-dQ mode (inf_set_deterministic)")
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--no-extras", action="store_true", help="skip the config-2 bf16 and deterministic, config-3 and config-4 lines")
    ap.add_argument("--gpt-steps", type=int, default=5, help="timed steps of the config-3 GPT line")
    ap.add_argument("--only", choices=sorted(ONLY_CONFIGS) + ["shape", "c5_decode"],
                    help="run only this per-config line, with --steps timed steps (for profiling); "
                         "'shape' runs --shape / --dtype / --non-causal instead")
    ap.add_argument("--shape", default="8,12,1024,64", help="B,H,T,D for --only shape")
    ap.add_argument("--non-causal", action="store_true", help="--only shape without the causal mask")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run a plain 512 MiB device copy 5 times (HBM-counter calibration)")
    args = ap.parse_args()

    if args.calibrate_copy:
        import torch

        src = torch.ones(128 << 20, device="cuda:0")  # 512 MiB
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"calibration": "copy", "bytes_read": src.numel() * 4, "bytes_written": dst.numel() * 4}))
        return

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(json.dumps({"error": "this build measures one GPU only: every (b, h) head is independent, "
                                   "so the path shards by heads with no communication; run with --gpus 1"}))
        sys.exit(2)

    import numpy as np
    import torch

    import inferno_amd as ia
    import oracle

    if args.only:
        causal, det = True, False
        if args.only == "c5_decode":
            r = bench_decode(ia, oracle, torch, np, torch.device("cuda:0"))
            print(json.dumps({"decode": r}), flush=True)
            return
        if args.only == "shape":
            B, H, T, D = (int(x) for x in args.shape.split(","))
            sigma, dtype, causal = 1.0, args.dtype, not args.non_causal
        else:
            B, H, T, D, sigma, dtype, det = ONLY_CONFIGS[args.only]
        r = bench_attn(ia, oracle, torch, np, torch.device("cuda:0"), B, H, T, D, sigma, dtype, steps=args.steps,
                       deterministic=det, causal=causal)
        print(json.dumps({"configs": {args.only: r}}), flush=True)
        return

    B, H, T, D = 8, 12, 1024, 64
    dt = torch.float32 if args.dtype == "f32" else torch.bfloat16
    dev = torch.device("cuda:0")
    ia.set_deterministic(args.deterministic)  # before sizing the backward's workspace
    q, k, v, do = oracle.attn_inputs(B, H, T, D, seed=42)
    if args.dtype == "bf16":
        q, k, v, do = (oracle.bf16_to_f32(oracle.round_bf16(x)) for x in (q, k, v, do))
    Q, K, V, dO = (torch.from_numpy(x).to(dev, dt) for x in (q, k, v, do))
    O = torch.empty_like(Q)
    LSE = torch.empty((B, H, T), device=dev, dtype=torch.float32)
    dQ, dK, dV = torch.empty_like(Q), torch.empty_like(K), torch.empty_like(V)
    ws = torch.empty(max(ia.workspace_bytes(ia.OP_ATTN_BWD, B, H, T, T, D, ia.ops._dt(Q)), 1),
                     dtype=torch.uint8, device=dev)
    fws = torch.empty(max(ia.workspace_bytes(ia.OP_ATTN_FWD, B, H, T, T, D, ia.ops._dt(Q)), 1),
                      dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream()

    def step():
        ia.attn_fwd(Q, K, V, out=O, lse=LSE, workspace=fws, stream=stream)
        ia.attn_bwd(Q, K, V, O, dO, LSE, dq=dQ, dk=dK, dv=dV, workspace=ws, stream=stream)

    clock_steps = warm_up(step, torch, args.clock_warmup_s) if args.clock_warmup_s > 0 else 0
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    # `value`: K steps back to back, nothing else on the stream.
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        step()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    # Per-phase breakdown and the roofline's launch durations: the same K steps
    # again with HIP events around each call on the launch stream.
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(args.steps)]
    for i in range(args.steps):
        ev[i][0].record(stream)
        ia.attn_fwd(Q, K, V, out=O, lse=LSE, workspace=fws, stream=stream)
        ev[i][1].record(stream)
        ia.attn_bwd(Q, K, V, O, dO, LSE, dq=dQ, dk=dK, dv=dV, workspace=ws, stream=stream)
        ev[i][2].record(stream)
    torch.cuda.synchronize()
    fwd_all = np.array([e[0].elapsed_time(e[1]) for e in ev])
    bwd_all = np.array([e[1].elapsed_time(e[2]) for e in ev])
    step_all = np.array([e[0].elapsed_time(e[2]) for e in ev])
    fwd_ms = float(np.mean(fwd_all))
    bwd_ms = float(np.mean(bwd_all))
    ms_per_step = wall * 1e3 / args.steps

    def pct(a):
        return {"median_ms": round(float(np.median(a)), 4), "p10_ms": round(float(np.percentile(a, 10)), 4),
                "p90_ms": round(float(np.percentile(a, 90)), 4)}

    F_fwd = flops_fwd(B, H, T, D)
    F_bwd = 2.5 * F_fwd
    F_step = 3.5 * F_fwd
    peak = MFMA_FP32_PEAK_TFLOPS if args.dtype == "f32" else MFMA_BF16_PEAK_TFLOPS
    value = F_step / (ms_per_step * 1e-3) / 1e12
    bwd_tf = F_bwd / (bwd_ms * 1e-3) / 1e12
    fwd_tf = F_fwd / (fwd_ms * 1e-3) / 1e12

    out = {
        "metric": METRIC,
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "clock_warmup": {"seconds": args.clock_warmup_s, "steps": clock_steps,
                         "note": "untimed steps before the W warm-up steps, run whatever W is: the clocks "
                                 "ramp up over the first ~30 ms of load"},
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32" if args.dtype == "f32" else "bf16-in/f32-acc",
        "data": "synthetic: Q,K,V,dO iid N(0,1), MT19937-64 + Box-Muller, seed 42+{0,1,2,3}",
        "config": {"workload": "causal self-attention fwd+bwd, B=8 H=12 T=1024 D=64 (BASELINE config 2)",
                   "B": B, "H": H, "T": T, "D": D, "causal": True, "scale": ia.default_scale(D)},
        "frac_of_peak": round(value / peak, 4),
        "deterministic_dq": bool(args.deterministic),
        "timings": {"fwd": pct(fwd_all), "bwd": pct(bwd_all), "fwd+bwd": pct(step_all)},
        "roofline": {
            "bound": "mfma",
            "kernel": "bwd: " + " + ".join(BWD_TRAFFIC[args.dtype]) + " (one inf_attn_bwd call; bwd_main dominates)",
            "achieved": round(bwd_tf, 3),
            "peak": peak,
            "unit": "TFLOP/s",
            "frac": round(bwd_tf / peak, 4),
            # HBM bytes of the timed backward call's kernels, measured at this config by
            # rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE (x2.00 / x1.00 copy-kernel calibration)
            "traffic": round(sum(BWD_TRAFFIC[args.dtype].values()), -5),
            "traffic_by_kernel": BWD_TRAFFIC[args.dtype],
            "traffic_source": BWD_TRAFFIC_SOURCE,
            "algorithmic_flop_per_launch": F_bwd,
            "avg_launch_ms": round(bwd_ms, 4),
        },
        "roofline_fwd": {
            "bound": "mfma", "kernel": "attn_fwd_kernel", "achieved": round(fwd_tf, 3), "peak": peak,
            "unit": "TFLOP/s", "frac": round(fwd_tf / peak, 4), "algorithmic_flop_per_launch": F_fwd,
            "avg_launch_ms": round(fwd_ms, 4),
        },
    }

    if args.deterministic:
        # the query-major dQ pass replaces the atomic dQ product (and, for bf16, the conversion
        # pass); the counter-measured traffic above is the default mode's
        out["roofline"]["kernel"] = "bwd: bwd_pre + bwd_main (no dQ) + bwd_dq (one inf_attn_bwd call)"
        out["roofline"]["traffic"] = None
        del out["roofline"]["traffic_by_kernel"], out["roofline"]["traffic_source"]
        ia.set_deterministic(False)
    if not args.no_decode:
        out["decode"] = bench_decode(ia, oracle, torch, np, dev)
    if not args.no_extras:
        del Q, K, V, dO, O, dQ, dK, dV, ws, fws
        torch.cuda.empty_cache()
        out["configs"] = {
            "c2_bf16": bench_attn(ia, oracle, torch, np, dev, 8, 12, 1024, 64, 1.0, "bf16"),
            "c4_f32": bench_attn(ia, oracle, torch, np, dev, 1, 16, 8192, 128, 3.0, "f32", steps=5),
            "c4_bf16": bench_attn(ia, oracle, torch, np, dev, 1, 16, 8192, 128, 3.0, "bf16", steps=5),
            # the opt-in deterministic-dQ mode (query-major dQ pass, no atomics) at config 2
            "c2_f32_deterministic": bench_attn(ia, oracle, torch, np, dev, 8, 12, 1024, 64, 1.0, "f32",
                                               deterministic=True),
            "c2_bf16_deterministic": bench_attn(ia, oracle, torch, np, dev, 8, 12, 1024, 64, 1.0, "bf16",
                                                deterministic=True),
        }
        torch.cuda.empty_cache()
        out["configs"]["c3_gpt"] = bench_gpt(args.gpt_steps)
        out["configs"]["gpt_generate"] = bench_generate()

    if args.cpu_heads > 0:
        out["cpu_baseline"] = cpu_baseline(B, H, T, D, args.cpu_heads, args.cpu_c4_rows, args.cpu_c4_heads)
    print(json.dumps(out), flush=True)


def warm_up(fn, torch, seconds=0.2):
    """Run fn until `seconds` of back-to-back GPU work have passed (clock ramp-up)."""
    t0 = time.perf_counter()
    n = 0
    while True:
        fn()
        n += 1
        if n % 4 == 0:
            torch.cuda.synchronize()
            if time.perf_counter() - t0 >= seconds:
                return n


def bench_attn(ia, oracle, torch, np, dev, B, H, T, D, qk_sigma, dtype, steps=10, deterministic=False, causal=True):
    """One attention config: fwd+bwd throughput over `steps` back-to-back steps between two
    synchronizations (as `value`), and the fwd / bwd breakdown from HIP events recorded on the
    launch stream around each call in a second pass (the events add the launch gaps).  With
    `deterministic`, the backward runs in the deterministic-dQ mode (inf_set_deterministic)."""
    previous = ia.set_deterministic(deterministic)
    try:
        r = _bench_attn(ia, oracle, torch, np, dev, B, H, T, D, qk_sigma, dtype, steps, causal)
    finally:
        ia.set_deterministic(previous)
    if deterministic:
        r["deterministic_dq"] = True
    return r


def _bench_attn(ia, oracle, torch, np, dev, B, H, T, D, qk_sigma, dtype, steps, causal=True):
    tdt = torch.float32 if dtype == "f32" else torch.bfloat16
    q, k, v, do = oracle.attn_inputs(B, H, T, D, seed=42, qk_sigma=qk_sigma)
    Q, K, V, dO = (torch.from_numpy(x).to(dev, tdt) for x in (q, k, v, do))
    del q, k, v, do
    O = torch.empty_like(Q)
    LSE = torch.empty((B, H, T), device=dev, dtype=torch.float32)
    dQ, dK, dV = torch.empty_like(Q), torch.empty_like(K), torch.empty_like(V)
    ws = torch.empty(max(ia.workspace_bytes(ia.OP_ATTN_BWD, B, H, T, T, D, ia.ops._dt(Q)), 1),
                     dtype=torch.uint8, device=dev)
    fws = torch.empty(max(ia.workspace_bytes(ia.OP_ATTN_FWD, B, H, T, T, D, ia.ops._dt(Q)), 1),
                      dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream()

    def step():
        ia.attn_fwd(Q, K, V, causal=causal, out=O, lse=LSE, workspace=fws, stream=stream)
        ia.attn_bwd(Q, K, V, O, dO, LSE, causal=causal, dq=dQ, dk=dK, dv=dV, workspace=ws, stream=stream)

    warm_up(step, torch)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    step_ms = (time.perf_counter() - t0) * 1e3 / steps
    evs = []
    for i in range(steps):
        e = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
        e[0].record(stream)
        ia.attn_fwd(Q, K, V, causal=causal, out=O, lse=LSE, workspace=fws, stream=stream)
        e[1].record(stream)
        ia.attn_bwd(Q, K, V, O, dO, LSE, causal=causal, dq=dQ, dk=dK, dv=dV, workspace=ws, stream=stream)
        e[2].record(stream)
        evs.append(e)
    torch.cuda.synchronize()
    fwd_ms = float(np.mean([e[0].elapsed_time(e[1]) for e in evs]))
    bwd_ms = float(np.mean([e[1].elapsed_time(e[2]) for e in evs]))
    F = flops_fwd(B, H, T, D) * (1 if causal else 2)
    peak = MFMA_FP32_PEAK_TFLOPS if dtype == "f32" else MFMA_BF16_PEAK_TFLOPS
    tot = 3.5 * F / (step_ms * 1e-3) / 1e12
    # minimal HBM bytes: fwd Q,K,V in and O out (+ fp32 LSE); bwd Q,K,V,O,dO in and dQ,dK,dV out
    # (+ LSE); the second roof for the bf16 lines, whose forward sits near the bf16 ridge
    esz = 4 if dtype == "f32" else 2
    n = B * H * T * D
    fwd_bytes = 4 * n * esz + B * H * T * 4
    bwd_bytes = 8 * n * esz + B * H * T * 4
    roofs = {"fwd_hbm_bytes": fwd_bytes, "fwd_GBs": round(fwd_bytes / (fwd_ms * 1e-3) / 1e9, 1),
             "bwd_hbm_bytes": bwd_bytes, "bwd_GBs": round(bwd_bytes / (bwd_ms * 1e-3) / 1e9, 1),
             "hbm_peak_GBs": HBM_PEAK_GBS}
    return {
        "roofs": roofs,
        "shape": f"B{B} H{H} T{T} D{D}", "dtype": dtype if dtype == "f32" else "bf16-in/f32-acc",
        "qk_sigma": qk_sigma, "causal": causal, "ms_per_step": round(step_ms, 4), "fwd_ms": round(fwd_ms, 4), "bwd_ms": round(bwd_ms, 4),
        "fwd_tflops": round(F / (fwd_ms * 1e-3) / 1e12, 2),
        "bwd_tflops": round(2.5 * F / (bwd_ms * 1e-3) / 1e12, 2),
        "fwd_bwd_tflops": round(tot, 2), "peak_tflops": peak, "frac": round(tot / peak, 4),
    }


def bench_gpt(steps, warmup=2):
    """Config 3: the GPT training step on the C++ drop-in (inferno_amd/gpt, a child process).

    12 layers, d_model 768, 12 heads, ctx 1024, GELU MLP 4x, LayerNorm,
    vocab 8192, tied embedding; weights N(0, 0.02), tokens uniform in
    [0, 8192), targets shifted by one; batch 8; AdamW lr 3e-4.  A step is
    forward + cross-entropy + backward + AdamW + zero_grad; tokens/s counts the
    8192 tokens of a step.  The attention share is the fused attention
    forward + backward of one layer timed alone, times 12, over the step time.
    """
    import subprocess

    app = ROOT / "inferno_amd" / "gpt"
    r = subprocess.run([str(app), "bench", "--steps", str(steps), "--warmup", str(warmup)],
                       capture_output=True, text=True, timeout=600)
    if r.returncode != 0:
        raise RuntimeError(f"inferno_amd/gpt bench failed ({r.returncode}): {r.stderr[-2000:]}")
    line = [l for l in r.stdout.splitlines() if l.startswith("{")][-1]
    d = json.loads(line)
    d["unit"] = "tokens/s"
    d["dtype"] = "f32"
    return d


def bench_generate(batch=32, prompt=1024, new=64):
    """Greedy generation on the config-3 model with one KV cache per layer (inferno_amd/gpt generate).

    Prefill of a random prompt, then `new` tokens one at a time through the
    single-query decode kernel (the inference loop around BASELINE config 5's
    kernel); reports the per-token step time of the whole 12-layer model.
    """
    import subprocess

    app = ROOT / "inferno_amd" / "gpt"
    r = subprocess.run([str(app), "generate", "--batch", str(batch), "--prompt", str(prompt), "--new", str(new),
                        "--ctx", str(prompt + new)], capture_output=True, text=True, timeout=600)
    if r.returncode != 0:
        raise RuntimeError(f"inferno_amd/gpt generate failed ({r.returncode}): {r.stderr[-2000:]}")
    d = json.loads([l for l in r.stdout.splitlines() if l.startswith("{")][-1])
    d.pop("first_tokens", None)
    return d


def bench_decode(ia, oracle, torch, np, dev, reps=50):
    """Config 5: B32 H12 Tk2048 D64 fp32 decode, rotating two KV sets (> the 256 MB MALL)."""
    B, H, Tk, D = 32, 12, 2048, 64
    sets = []
    for s in range(3):
        kc = torch.from_numpy(oracle.randn(500 + 10 * s, (B, H, Tk, D))).to(dev)
        vc = torch.from_numpy(oracle.randn(501 + 10 * s, (B, H, Tk, D))).to(dev)
        q = torch.from_numpy(oracle.randn(502 + 10 * s, (B, H, 1, D))).to(dev)
        sets.append((q, kc, vc))
    out = torch.empty((B, H, 1, D), device=dev)
    ws = torch.zeros(ia.workspace_bytes(ia.OP_ATTN_DECODE, B, H, 1, Tk, D), dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream()
    it = [0]

    def one():
        q, kc, vc = sets[it[0] % 3]
        it[0] += 1
        ia.attn_decode(q, kc, vc, out=out, workspace=ws, stream=stream)

    warm_up(one, torch)
    evs = []
    for i in range(reps):
        q, kc, vc = sets[i % 3]
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        ia.attn_decode(q, kc, vc, out=out, workspace=ws, stream=stream)
        e1.record(stream)
        evs.append((e0, e1))
    torch.cuda.synchronize()
    ts = np.array([a.elapsed_time(b) for a, b in evs])
    nbytes = 2 * B * H * Tk * D * 4 + 2 * B * H * D * 4
    med = float(np.median(ts))
    return {
        "workload": "decode B32 H12 Tk2048 D64 fp32 (BASELINE config 5), 3 KV sets rotated",
        "median_us": round(med * 1e3, 2),
        "p10_us": round(float(np.percentile(ts, 10)) * 1e3, 2),
        "p90_us": round(float(np.percentile(ts, 90)) * 1e3, 2),
        "algorithmic_bytes": nbytes,
        "achieved_GBs": round(nbytes / (med * 1e-3) / 1e9, 1),
        "peak_GBs": HBM_PEAK_GBS,
        "frac": round(nbytes / (med * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
    }


if __name__ == "__main__":
    main()
