"""The C++ Tensor / autograd drop-in (libinferno.so) through tests/cpp/api_driver.

CPU-device runs must equal the oracle bit for bit (the CPU branch runs the
reference chain); HIP-device runs must be within the parity bar (1e-4 fp32,
2e-2 bf16 inputs) -- the device-parameterised pattern of the reference's tests.
"""
import subprocess
from pathlib import Path

import numpy as np
import pytest

import oracle

ROOT = Path(__file__).resolve().parents[1]
DRIVER = ROOT / "tests" / "cpp" / "api_driver"


def have_gpu():
    try:
        import torch

        return torch.cuda.is_available()
    except Exception:
        return False


def run(*args, timeout=300):
    if not DRIVER.exists():
        pytest.skip("api_driver not built (run __graft_entry__.build())")
    r = subprocess.run([str(DRIVER), *map(str, args)], capture_output=True, text=True, timeout=timeout)
    return r


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def write(d, **arrs):
    for k, v in arrs.items():
        np.ascontiguousarray(v, np.float32).tofile(d / f"{k}.bin")


def read(d, name, shape):
    return np.fromfile(d / f"{name}.bin", dtype=np.float32).reshape(shape)


def bf16_round(a):
    return oracle.bf16_to_f32(oracle.round_bf16(a))


def attn_case(tmp_path, B, H, T, D, dtype, device, causal=True, layout=None, seed=42):
    q, k, v, do = oracle.attn_inputs(B, H, T, D, seed=seed)
    if dtype == "bf16":
        q, k, v, do = (bf16_round(x) for x in (q, k, v, do))
    write(tmp_path, q=q, k=k, v=v, do=do)
    args = ["attn", tmp_path, B, H, T, D, dtype, device, int(causal)] + ([layout] if layout else [])
    r = run(*args)
    assert r.returncode == 0, r.stdout + r.stderr
    out = {n: read(tmp_path, n, (B, H, T, D)) for n in ("o", "dq", "dk", "dv")}
    out["lse"] = read(tmp_path, "lse", (B, H, T))
    o_r, lse_r = oracle.attn_fwd(q, k, v, causal=causal)
    dq_r, dk_r, dv_r = oracle.attn_bwd(q, k, v, do, causal=causal)
    return out, dict(o=o_r, lse=lse_r, dq=dq_r, dk=dk_r, dv=dv_r)


# ------------------------------------------------------------------ CPU device
def test_selftest_cpu():
    r = run("selftest", "cpu")
    assert r.returncode == 0, r.stdout + r.stderr
    assert "SELFTEST OK 0" in r.stdout


@pytest.mark.parametrize("B,H,T,D,causal", [(1, 4, 128, 32, True), (2, 1, 17, 8, True), (1, 2, 33, 16, False)])
def test_attention_cpu_equals_reference_chain_bitwise(tmp_path, B, H, T, D, causal):
    out, ref = attn_case(tmp_path, B, H, T, D, "f32", "cpu", causal)
    for n in ("o", "dq", "dk", "dv", "lse"):
        assert np.array_equal(bits(out[n]), bits(ref[n])), n


def test_attention_cpu_qkv_views_bitwise(tmp_path):
    """q, k, v sliced out of one [B, T, 3C] tensor (views all the way), grads back into it."""
    out, ref = attn_case(tmp_path, 2, 3, 20, 8, "f32", "cpu", True, layout="qkv")
    for n in ("o", "dq", "dk", "dv"):
        assert np.array_equal(bits(out[n]), bits(ref[n])), n


def test_attention_cpu_qkv_op_bitwise(tmp_path):
    """qkv_attention (the MultiHeadAttention op) on one [B, T, 3C] tensor: y and the gradient
    of qkv equal the oracle's O, dQ, dK, dV bit for bit."""
    out, ref = attn_case(tmp_path, 2, 3, 20, 8, "f32", "cpu", True, layout="qkvop")
    for n in ("o", "dq", "dk", "dv"):
        assert np.array_equal(bits(out[n]), bits(ref[n])), n


def test_softmax_cpu_bitwise(tmp_path):
    x = oracle.randn(7, (6, 50), 3.0)
    g = oracle.randn(8, (6, 50))
    write(tmp_path, x=x, g=g)
    r = run("softmax", tmp_path, 6, 50, "f32", "cpu", -1)
    assert r.returncode == 0, r.stderr
    y = read(tmp_path, "y", (6, 50))
    assert np.array_equal(bits(y), bits(oracle.softmax(x)))
    assert np.array_equal(bits(read(tmp_path, "dx", (6, 50))), bits(oracle.softmax_bwd(y, g)))


def test_softmax_f64_i32_cpu_bitwise(tmp_path):
    """Softmax of Float64 (-> Float64) and Int32 (-> Float32) tensors on the CPU device: the
    reference's cpu_softmax<double, double> / <int, float>, and the Float64 backward."""
    x = oracle.randn(21, (5, 37), 3.0).astype(np.float64) * (1 + 1e-9)
    g = oracle.randn(22, (5, 37)).astype(np.float64) / 3
    x.tofile(tmp_path / "x.bin")
    g.tofile(tmp_path / "g.bin")
    r = run("softmax-typed", tmp_path, 5, 37, "f64", "cpu", -1)
    assert r.returncode == 0, r.stderr
    y = np.fromfile(tmp_path / "y.bin", np.float64).reshape(5, 37)
    assert np.array_equal(y.view(np.uint64), oracle.softmax_f64(x).view(np.uint64))
    dx = np.fromfile(tmp_path / "dx.bin", np.float64).reshape(5, 37)
    assert np.array_equal(dx.view(np.uint64), oracle.softmax_bwd_f64(y, g).view(np.uint64))

    xi = (oracle.randn(23, (4, 29), 4.0) * 3).astype(np.int32)
    xi.tofile(tmp_path / "x.bin")
    r = run("softmax-typed", tmp_path, 4, 29, "i32", "cpu", -1)
    assert r.returncode == 0, r.stderr
    yi = np.fromfile(tmp_path / "y.bin", np.float32).reshape(4, 29)
    assert np.array_equal(bits(yi), bits(oracle.softmax_i32(xi)))


def test_decode_cpu(tmp_path):
    q = oracle.randn(1, (2, 3, 1, 16))
    kc = oracle.randn(2, (2, 3, 40, 16))
    vc = oracle.randn(3, (2, 3, 40, 16))
    write(tmp_path, q=q, kc=kc, vc=vc)
    r = run("decode", tmp_path, 2, 3, 40, 16, "f32", "cpu")
    assert r.returncode == 0, r.stderr
    assert np.array_equal(bits(read(tmp_path, "o", (2, 3, 1, 16))), bits(oracle.attn_decode(q, kc, vc)))


def test_error_paths_cpu(tmp_path):
    r = run("attn", tmp_path, 1, 1, 4, 8, "f32", "cpu", 1)  # missing input files
    assert r.returncode == 3 and "cannot read" in r.stderr


def pattern(shape, step, base):
    n = int(np.prod(shape))
    return (np.arange(n, dtype=np.float32) * np.float32(step) + np.float32(base)).reshape(shape)


def mask_expected():
    """Expected bytes of every `api_driver mask` case: np.triu / np.where on the driver's inputs."""
    a = pattern((2, 3, 5, 7), 0.5, -10.0)
    at = np.swapaxes(a, 2, 3)
    exp = {}
    for dg in (-2, 0, 1, 3):
        exp[f"triu_f32_{dg + 2}"] = np.triu(a, dg)
        exp[f"triu_f32t_{dg + 2}"] = np.triu(at, dg)
    exp["triu_i32"] = np.triu(np.ones((1, 1, 6, 9), np.int32), 1)
    exp["triu_bf16"] = np.triu(oracle.round_bf16(pattern((4, 6), 0.25, -3.0)), -1)
    m57 = np.triu(np.ones((5, 7), np.int32), 1)
    exp["mf_f32"] = np.where(m57 != 0, np.float32(-1e9), a)
    exp["mf_f32t"] = np.where(np.triu(np.ones((7, 5), np.int32), 0) != 0, np.float32(2.5), at)
    m_i8 = pattern((1, 7), 1.0, -3.0).astype(np.int8)
    exp["mf_i8"] = np.where(m_i8 != 0, np.float32(7.0), a)
    m_bool = pattern((3, 1, 1), 1.0, 0.0) != 0
    exp["mf_bool"] = np.where(m_bool, np.float32(-1.0), a)
    every3 = (np.arange(70) % 3 == 0).astype(np.int32).reshape(2, 1, 5, 7)
    xb = oracle.round_bf16(pattern((2, 3, 5, 7), 0.25, -7.0))
    fill_b = oracle.round_bf16(np.array([-1e9], np.float32))[0]
    exp["mf_bf16"] = np.where(every3 != 0, fill_b, xb)
    xi = pattern((4, 6), 3.0, -20.0).astype(np.int32)
    exp["mf_i32"] = np.where(pattern((6,), 1.0, -2.0) != 0, np.int32(-3), xi)  # static_cast<int>(-3.7f)
    return {k: np.ascontiguousarray(v).tobytes() for k, v in exp.items()}


def test_mask_ops_cpu_match_numpy(tmp_path):
    """triu / masked_fill (ops.cpp:1235-1398) on CPU tensors: dtypes f32, bf16, i32; strided views;
    Int32 / Int8 / Bool masks broadcast from the right -- against np.triu and np.where."""
    r = run("mask", tmp_path, "cpu")
    assert r.returncode == 0, r.stdout + r.stderr
    for name, want in mask_expected().items():
        assert (tmp_path / f"{name}.bin").read_bytes() == want, name


def test_mask_ops_pin_against_oracle():
    """The causal mask and the -1e9 fill equal the oracle's restatement (itself pinned bit for bit to
    the reference's cpu_triu / cpu_masked_fill in tests/test_oracle.py)."""
    T = 9
    assert np.array_equal(np.triu(np.ones((T, T), np.int32), 1), oracle.triu_ones(T, T, 1))
    s = oracle.randn(3, (T, T))
    assert np.array_equal(bits(np.where(np.triu(np.ones((T, T)), 1) != 0, np.float32(-1e9), s)),
                          bits(oracle.masked_fill(s, oracle.triu_ones(T, T, 1), -1e9)))


@pytest.mark.parametrize("B,H,T,D", [(1, 2, 33, 16), (2, 1, 64, 8)])
def test_reference_chain_cpu_bitwise(tmp_path, B, H, T, D):
    """The reference's unfused attention chain (main.cpp:732-754: transpose, contiguous, matmul,
    * scale, triu, masked_fill, Softmax, matmul) through this API equals the oracle bit for bit."""
    q, k, v, _ = oracle.attn_inputs(B, H, T, D, seed=9)
    write(tmp_path, q=q, k=k, v=v)
    r = run("chain", tmp_path, B, H, T, D, "cpu")
    assert r.returncode == 0, r.stdout + r.stderr
    o_r, _ = oracle.attn_fwd(q, k, v)
    assert np.array_equal(bits(read(tmp_path, "y", (B, H, T, D))), bits(o_r))
    assert (tmp_path / "mask.bin").read_bytes() == np.triu(np.ones((T, T), np.int32), 1).tobytes()


# ------------------------------------------------------------------ HIP device
gpu = pytest.mark.gpu


@gpu
def test_mask_ops_hip_equal_cpu(tmp_path):
    if not have_gpu():
        pytest.skip("no GPU")
    print("[case] api_driver mask hip", flush=True)
    r = run("mask", tmp_path, "hip")
    assert r.returncode == 0, r.stdout + r.stderr
    for name, want in mask_expected().items():
        assert (tmp_path / f"{name}.bin").read_bytes() == want, name


@gpu
def test_reference_chain_hip(tmp_path):
    """The unfused chain on HIP tensors: the causal mask bit-exact, y within the fp32 bar."""
    if not have_gpu():
        pytest.skip("no GPU")
    print("[case] api_driver chain hip", flush=True)
    B, H, T, D = 2, 3, 130, 64
    q, k, v, _ = oracle.attn_inputs(B, H, T, D, seed=9)
    write(tmp_path, q=q, k=k, v=v)
    r = run("chain", tmp_path, B, H, T, D, "hip")
    assert r.returncode == 0, r.stdout + r.stderr
    o_r, _ = oracle.attn_fwd(q, k, v)
    assert oracle.rel_err(read(tmp_path, "y", (B, H, T, D)), o_r) <= 1e-4
    assert (tmp_path / "mask.bin").read_bytes() == np.triu(np.ones((T, T), np.int32), 1).tobytes()


@gpu
def test_selftest_hip():
    if not have_gpu():
        pytest.skip("no GPU")
    print("[case] api_driver selftest hip", flush=True)
    r = run("selftest", "hip")
    assert r.returncode == 0, r.stdout + r.stderr
    assert "SELFTEST OK 0" in r.stdout


@gpu
@pytest.mark.parametrize("B,H,T,D,dtype,layout", [
    (1, 4, 128, 32, "f32", None),
    (2, 3, 200, 64, "f32", None),
    (1, 2, 129, 128, "f32", None),
    (2, 3, 150, 64, "f32", "qkv"),
    (1, 4, 128, 32, "bf16", None),
])
def test_attention_hip_parity(tmp_path, B, H, T, D, dtype, layout):
    if not have_gpu():
        pytest.skip("no GPU")
    print(f"[case] api_driver attn hip B{B} H{H} T{T} D{D} {dtype} {layout}", flush=True)
    out, ref = attn_case(tmp_path, B, H, T, D, dtype, "hip", True, layout)
    tol = 1e-4 if dtype == "f32" else 2e-2
    for n in ("o", "dq", "dk", "dv"):
        e = oracle.rel_err(out[n], ref[n])
        assert e <= tol, f"{n} rel err {e:.3e}"


@gpu
@pytest.mark.parametrize("B,H,T,D,dtype,layout", [
    (1, 2, 70, 16, "f32", None),      # zero-padded to 32
    (2, 2, 100, 48, "f32", None),     # padded to 64
    (1, 3, 90, 96, "f32", "qkv"),     # padded to 128, q / k / v as views of [B, T, 3C]
    (2, 3, 77, 48, "f32", "qkvop"),   # padded, through qkv_attention (the MultiHeadAttention op)
    (1, 2, 80, 80, "bf16", None),     # padded to 128, bf16 inputs
    (1, 2, 70, 160, "f32", None),     # above 128: the composed chain on HIP ops
    (2, 2, 50, 256, "f32", "qkvop"),  # composed, through qkv_attention
])
def test_attention_hip_other_head_dims(tmp_path, B, H, T, D, dtype, layout):
    """Head dims the fused kernels are not built for, through the C++ layer on HIP: up to 128 the
    kernels on zero-padded copies, above 128 the reference's composed chain on the HIP ops.
    O, dQ, dK, dV (and the LSE where the op returns it) against the oracle."""
    if not have_gpu():
        pytest.skip("no GPU")
    print(f"[case] api_driver attn hip other head dim B{B} H{H} T{T} D{D} {dtype} {layout}", flush=True)
    out, ref = attn_case(tmp_path, B, H, T, D, dtype, "hip", True, layout)
    tol = 1e-4 if dtype == "f32" else 2e-2
    for n in ("o", "dq", "dk", "dv"):
        e = oracle.rel_err(out[n], ref[n])
        assert e <= tol, f"{n} rel err {e:.3e}"
    if layout != "qkvop":
        assert oracle.rel_err(out["lse"], ref["lse"]) <= (1e-5 if dtype == "f32" else 1e-3)


@gpu
@pytest.mark.parametrize("D,dtype", [(48, "f32"), (80, "bf16"), (160, "f32")])
def test_decode_hip_other_head_dims(tmp_path, D, dtype):
    """attention_decode at head dims the decode kernel is not built for (padded up to 128,
    composed above), against the oracle's decode."""
    if not have_gpu():
        pytest.skip("no GPU")
    print(f"[case] api_driver decode hip D{D} {dtype}", flush=True)
    B, H, Tk = 2, 3, 300
    q, kc, vc = oracle.randn(31, (B, H, 1, D)), oracle.randn(32, (B, H, Tk, D)), oracle.randn(33, (B, H, Tk, D))
    if dtype == "bf16":
        q, kc, vc = (bf16_round(x) for x in (q, kc, vc))
    write(tmp_path, q=q, kc=kc, vc=vc)
    r = run("decode", tmp_path, B, H, Tk, D, dtype, "hip")
    assert r.returncode == 0, r.stdout + r.stderr
    e = oracle.rel_err(read(tmp_path, "o", (B, H, 1, D)), oracle.attn_decode(q, kc, vc))
    assert e <= (1e-4 if dtype == "f32" else 2e-2), f"rel err {e:.3e}"


@gpu
def test_softmax_f64_i32_hip_parity(tmp_path):
    """Softmax of Float64 and Int32 tensors on HIP through the C++ drop-in (forward), against the
    reference-exact oracle: Float64 within 1e-12 of max|ref| (exp on the device differs from
    the host's in the last bits), Int32 -> Float32 within 1e-4."""
    if not have_gpu():
        pytest.skip("no GPU")
    print("[case] api_driver softmax f64 / i32 hip", flush=True)
    x = oracle.randn(24, (33, 1000), 3.0).astype(np.float64)
    x.tofile(tmp_path / "x.bin")
    for axis in (-1, 0):
        r = run("softmax-typed", tmp_path, 33, 1000, "f64", "hip", axis)
        assert r.returncode == 0, r.stderr
        y = np.fromfile(tmp_path / "y.bin", np.float64).reshape(33, 1000)
        y_r = oracle.softmax_f64(x) if axis == -1 else oracle.softmax_f64(np.ascontiguousarray(x.T)).T
        assert oracle.rel_err(y, y_r) <= 1e-12
    xi = (oracle.randn(25, (16, 4096), 4.0) * 3).astype(np.int32)
    xi.tofile(tmp_path / "x.bin")
    r = run("softmax-typed", tmp_path, 16, 4096, "i32", "hip", -1)
    assert r.returncode == 0, r.stderr
    yi = np.fromfile(tmp_path / "y.bin", np.float32).reshape(16, 4096)
    assert oracle.rel_err(yi, oracle.softmax_i32(xi)) <= 1e-4


@gpu
def test_softmax_hip_parity(tmp_path):
    if not have_gpu():
        pytest.skip("no GPU")
    print("[case] api_driver softmax hip", flush=True)
    x = oracle.randn(7, (64, 1024), 3.0)
    g = oracle.randn(8, (64, 1024))
    write(tmp_path, x=x, g=g)
    for axis in (-1, 0):
        r = run("softmax", tmp_path, 64, 1024, "f32", "hip", axis)
        assert r.returncode == 0, r.stderr
        xr = x if axis == -1 else np.ascontiguousarray(x.T)
        gr = g if axis == -1 else np.ascontiguousarray(g.T)
        y_r = oracle.softmax(xr)
        dx_r = oracle.softmax_bwd(y_r, gr)
        if axis == 0:
            y_r, dx_r = y_r.T, dx_r.T
        assert oracle.rel_err(read(tmp_path, "y", (64, 1024)), y_r) <= 1e-4
        assert oracle.rel_err(read(tmp_path, "dx", (64, 1024)), dx_r) <= 1e-4


@gpu
def test_decode_hip_parity(tmp_path):
    if not have_gpu():
        pytest.skip("no GPU")
    print("[case] api_driver decode hip", flush=True)
    q = oracle.randn(1, (4, 12, 1, 64))
    kc = oracle.randn(2, (4, 12, 700, 64))
    vc = oracle.randn(3, (4, 12, 700, 64))
    write(tmp_path, q=q, kc=kc, vc=vc)
    r = run("decode", tmp_path, 4, 12, 700, 64, "f32", "hip")
    assert r.returncode == 0, r.stderr
    assert oracle.rel_err(read(tmp_path, "o", (4, 12, 1, 64)), oracle.attn_decode(q, kc, vc)) <= 1e-4
