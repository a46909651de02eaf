"""CPU oracle for Inferno's causal-attention path.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this package, and only as the
checker (or the timed CPU baseline).  The product package ``inferno_amd`` never
imports it and never falls back to it.

``liboracle.so`` (built from ``oracle.c`` by ``oracle/Makefile``) restates the
reference's CPU kernels literally; ``_ref/libinferno_ref.so`` (built from the
reference's own headers where ``/root/reference`` exists) is the real reference
arithmetic used to pin the restatement.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"
REF_PATH = HERE / "_ref" / "libinferno_ref.so"

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(dtype=np.uint16, flags="C_CONTIGUOUS")
_i64 = ctypes.c_int64
_vp = ctypes.c_void_p

_lib = None
_ref = None


def build() -> None:
    """Compile the oracle (and the reference build when the reference tree exists)."""
    import subprocess

    subprocess.run(["make", "-s", "-C", str(HERE), "all"], check=True)


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} missing: run `make -C oracle`")
        L = ctypes.CDLL(str(LIB_PATH))
        L.orc_randn_f32.argtypes = [ctypes.c_uint64, ctypes.c_double, _f32p, ctypes.c_size_t]
        L.orc_randn_f32.restype = None
        L.orc_mt64_seed.argtypes = [_vp, ctypes.c_uint64]
        L.orc_mt64_next.argtypes = [_vp]
        L.orc_mt64_next.restype = ctypes.c_uint64
        L.orc_round_bf16.argtypes = [_f32p, _u16p, ctypes.c_size_t]
        L.orc_bf16_to_f32.argtypes = [_u16p, _f32p, ctypes.c_size_t]
        L.orc_matmul_f32.argtypes = [_vp, _i64, _i64, _vp, _i64, _i64, _f32p, _i64, _i64, _i64]
        L.orc_scale_f32.argtypes = [_f32p, ctypes.c_float, _f32p, _i64]
        L.orc_triu_ones_i32.argtypes = [_i32p, _i64, _i64, ctypes.c_int]
        L.orc_masked_fill_f32.argtypes = [_f32p, _i32p, ctypes.c_float, _f32p, _i64, _i64]
        L.orc_softmax_f32.argtypes = [_f32p, _f32p, _i64, _i64]
        L.orc_softmax_bwd_f32.argtypes = [_f32p, _f32p, _f32p, _i64, _i64]
        _f64p = np.ctypeslib.ndpointer(dtype=np.float64, flags="C_CONTIGUOUS")
        L.orc_softmax_f64.argtypes = [_f64p, _f64p, _i64, _i64]
        L.orc_softmax_i32.argtypes = [_i32p, _f32p, _i64, _i64]
        L.orc_softmax_bwd_f64.argtypes = [_f64p, _f64p, _f64p, _i64, _i64]
        L.orc_attn_fwd_f32.argtypes = [_f32p, _f32p, _f32p, _i64, _i64, _i64, _i64, _i64,
                                       ctypes.c_float, ctypes.c_int, _f32p, _vp, _vp]
        L.orc_attn_bwd_f32.argtypes = [_f32p, _f32p, _f32p, _f32p, _i64, _i64, _i64, _i64, _i64,
                                       ctypes.c_float, ctypes.c_int, _f32p, _f32p, _f32p, _vp]
        L.orc_attn_decode_f32.argtypes = [_f32p, _f32p, _f32p, _i64, _i64, _i64, _i64,
                                          ctypes.c_float, _f32p]
        _lib = L
    return _lib


def ref_lib():
    """The reference's own kernels (oracle/_ref), or None where they were not built."""
    global _ref
    if _ref is None and REF_PATH.exists():
        R = ctypes.CDLL(str(REF_PATH), mode=os.RTLD_LAZY)
        i64p = ctypes.POINTER(ctypes.c_int64)
        R.ref_matmul4_f32.argtypes = [_f32p, i64p, _f32p, i64p, _f32p, _i64, _i64, _i64, _i64, _i64]
        R.ref_scale_f32.argtypes = [_f32p, _i64, ctypes.c_float, _f32p]
        R.ref_triu_ones_i32.argtypes = [_i64, _i64, ctypes.c_int, _i32p]
        R.ref_masked_fill_f32.argtypes = [_f32p, _i64, _i64, _i64, _i64, _i32p, ctypes.c_float, _f32p]
        R.ref_softmax_f32.argtypes = [_f32p, _i64, _i64, _f32p]
        R.ref_softmax_f64.argtypes = [np.ctypeslib.ndpointer(dtype=np.float64, flags="C_CONTIGUOUS"), _i64, _i64,
                                      np.ctypeslib.ndpointer(dtype=np.float64, flags="C_CONTIGUOUS")]
        R.ref_softmax_i32.argtypes = [_i32p, _i64, _i64, _f32p]
        R.ref_transpose_contig_f32.argtypes = [_f32p, _i64, _i64, _i64, _i64, _f32p]
        R.ref_attn_fwd_f32.argtypes = [_f32p, _f32p, _f32p, _i64, _i64, _i64, _i64, ctypes.c_float,
                                       ctypes.c_int, _f32p, _vp]
        R.ref_attn_bwd_stages_f32.argtypes = [_f32p, _f32p, _f32p, _f32p, _f32p, _f32p, _i64, _i64,
                                              _i64, _i64, ctypes.c_float, _f32p, _f32p, _f32p, _f32p]
        _ref = R
    return _ref


def _ptr(a):
    return None if a is None else a.ctypes.data_as(_vp)


# ---------------------------------------------------------------- generator --
def randn(seed: int, shape, sigma: float = 1.0) -> np.ndarray:
    """N(0, sigma^2) fp32 draws from MT19937-64 + Box-Muller (seeded, deterministic)."""
    n = int(np.prod(shape)) if len(shape) else 1
    out = np.empty(n, dtype=np.float32)
    lib().orc_randn_f32(seed, sigma, out, n)
    return out.reshape(shape)


def round_bf16(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bit patterns (uint16), round to nearest even."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().orc_round_bf16(x.reshape(-1), out.reshape(-1), x.size)
    return out


def triu_ones(rows: int, cols: int, diagonal: int) -> np.ndarray:
    """triu(ones[rows, cols], diagonal) as Int32 (cpu_triu, cpuops.h:617-656)."""
    out = np.empty((rows, cols), dtype=np.int32)
    lib().orc_triu_ones_i32(out, rows, cols, int(diagonal))
    return out


def masked_fill(x: np.ndarray, mask: np.ndarray, fill: float) -> np.ndarray:
    """(mask != 0) ? fill : x for a [rows, cols] fp32 x and Int32 mask (cpu_masked_fill)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    mask = np.ascontiguousarray(mask, dtype=np.int32)
    out = np.empty_like(x)
    lib().orc_masked_fill_f32(x, mask, np.float32(fill), out, x.shape[0], x.shape[1])
    return out


def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    b = np.ascontiguousarray(b, dtype=np.uint16)
    out = np.empty(b.shape, dtype=np.float32)
    lib().orc_bf16_to_f32(b.reshape(-1), out.reshape(-1), b.size)
    return out


def attn_inputs(B, H, T, D, seed=42, qk_sigma=1.0, Tk=None):
    """Q, K, V, dO for one config: seed+0..3, Q,K ~ N(0, qk_sigma^2), V, dO ~ N(0,1)."""
    Tk = T if Tk is None else Tk
    q = randn(seed + 0, (B, H, T, D), qk_sigma)
    k = randn(seed + 1, (B, H, Tk, D), qk_sigma)
    v = randn(seed + 2, (B, H, Tk, D), 1.0)
    do = randn(seed + 3, (B, H, T, D), 1.0)
    return q, k, v, do


# ------------------------------------------------------------- attention -----
def _c(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def attn_fwd(q, k, v, scale=None, causal=True, want_p=False):
    """Returns (O, LSE[, P]) through the reference chain (InfernoApp/main.cpp:737-754)."""
    q, k, v = _c(q), _c(k), _c(v)
    B, H, Tq, D = q.shape
    Tk = k.shape[2]
    if scale is None:
        scale = float(np.float32(1.0) / np.sqrt(np.float32(D)))
    o = np.empty((B, H, Tq, D), np.float32)
    lse = np.empty((B, H, Tq), np.float32)
    p = np.empty((B, H, Tq, Tk), np.float32) if want_p else None
    lib().orc_attn_fwd_f32(q, k, v, B, H, Tq, Tk, D, scale, int(causal), o, _ptr(lse), _ptr(p))
    return (o, lse, p) if want_p else (o, lse)


def attn_bwd(q, k, v, do, scale=None, causal=True, want_ds=False):
    """Returns (dQ, dK, dV[, dS]) through MMBackward/SoftmaxBackward/MultiplyBackward."""
    q, k, v, do = _c(q), _c(k), _c(v), _c(do)
    B, H, Tq, D = q.shape
    Tk = k.shape[2]
    if scale is None:
        scale = float(np.float32(1.0) / np.sqrt(np.float32(D)))
    dq = np.empty_like(q)
    dk = np.empty_like(k)
    dv = np.empty_like(v)
    ds = np.empty((B, H, Tq, Tk), np.float32) if want_ds else None
    lib().orc_attn_bwd_f32(q, k, v, do, B, H, Tq, Tk, D, scale, int(causal), dq, dk, dv, _ptr(ds))
    return (dq, dk, dv, ds) if want_ds else (dq, dk, dv)


def attn_decode(q, kc, vc, scale=None):
    q, kc, vc = _c(q), _c(kc), _c(vc)
    B, H, _, D = q.shape
    Tk = kc.shape[2]
    if scale is None:
        scale = float(np.float32(1.0) / np.sqrt(np.float32(D)))
    o = np.empty((B, H, 1, D), np.float32)
    lib().orc_attn_decode_f32(q, kc, vc, B, H, Tk, D, scale, o)
    return o


def softmax(x):
    x = _c(x)
    rows, cols = int(np.prod(x.shape[:-1])), x.shape[-1]
    y = np.empty_like(x)
    lib().orc_softmax_f32(x.reshape(-1), y.reshape(-1), rows, cols)
    return y


def softmax_f64(x):
    """cpu_softmax<double, double> over the last axis (Softmax of a Float64 tensor)."""
    x = np.ascontiguousarray(x, dtype=np.float64)
    rows, cols = int(np.prod(x.shape[:-1])), x.shape[-1]
    y = np.empty_like(x)
    lib().orc_softmax_f64(x.reshape(-1), y.reshape(-1), rows, cols)
    return y


def softmax_i32(x):
    """cpu_softmax<int, float> over the last axis (Softmax of an Int32 tensor -> Float32)."""
    x = np.ascontiguousarray(x, dtype=np.int32)
    rows, cols = int(np.prod(x.shape[:-1])), x.shape[-1]
    y = np.empty(x.shape, np.float32)
    lib().orc_softmax_i32(x.reshape(-1), y.reshape(-1), rows, cols)
    return y


def softmax_bwd_f64(y, g):
    """cpu_softmax_backward with RT = double (Float64 operands; Float32 ones widen exactly)."""
    y, g = np.ascontiguousarray(y, np.float64), np.ascontiguousarray(g, np.float64)
    rows, cols = int(np.prod(y.shape[:-1])), y.shape[-1]
    dx = np.empty_like(y)
    lib().orc_softmax_bwd_f64(y.reshape(-1), g.reshape(-1), dx.reshape(-1), rows, cols)
    return dx


def softmax_bwd(y, g):
    y, g = _c(y), _c(g)
    rows, cols = int(np.prod(y.shape[:-1])), y.shape[-1]
    dx = np.empty_like(y)
    lib().orc_softmax_bwd_f32(y.reshape(-1), g.reshape(-1), dx.reshape(-1), rows, cols)
    return dx


def matmul(a, b):
    """Dense 2-D a @ b through the restated cpu_matmul."""
    a, b = _c(a), _c(b)
    M, K = a.shape
    N = b.shape[1]
    out = np.empty((M, N), np.float32)
    lib().orc_matmul_f32(_ptr(a), K, 1, _ptr(b), N, 1, out, M, K, N)
    return out


def rel_err(x, ref, floor: float = 1e-30) -> float:
    """max|x - ref| / max(max|ref|, floor), the parity metric.

    `floor` only matters where the reference is (near) zero everywhere, e.g.
    dQ and dK at T = 1, which the reference computes as exactly 0.
    """
    x = np.asarray(x, np.float64)
    ref = np.asarray(ref, np.float64)
    den = max(float(np.max(np.abs(ref))) if ref.size else 0.0, floor)
    return float(np.max(np.abs(x - ref))) / den if ref.size else 0.0
