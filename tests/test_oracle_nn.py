"""Pins the oracle's model ops (oracle/oracle_nn.c) -- CPU only.

Where the reference's own header kernel compiles here (oracle/_ref), the
restatement must equal it bit for bit.  Where it does not (LayerNorm backward,
cross-entropy backward: their headers pull <cuda_runtime.h>), the restatement
is pinned by fp64 central differences of an independent fp64 forward, by the
invariants the mathematics fixes, and by brute force on exactly representable
inputs.
"""
import numpy as np
import pytest

import oracle
from oracle import nn as onn

need_ref = pytest.mark.skipif(not oracle.REF_PATH.exists(), reason="oracle/_ref not built (no reference tree)")


def rnd(seed, shape, sigma=1.0):
    return oracle.randn(seed, shape, sigma)


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


# ------------------------------------------------------------------ LayerNorm
@need_ref
@pytest.mark.parametrize("rows,dim", [(1, 4), (7, 33), (16, 768), (3, 1000)])
def test_layernorm_bit_exact_vs_reference(rows, dim):
    x = rnd(1, (rows, dim), 2.0) + 0.5
    g = rnd(2, (dim,)) + 1.0
    b = rnd(3, (dim,))
    y, m, s = onn.layernorm(x, g, b)
    yr, mr, sr = onn.ref_layernorm(x, g, b)
    assert np.array_equal(bits(y), bits(yr))
    assert np.array_equal(bits(m), bits(mr)) and np.array_equal(bits(s), bits(sr))


def ln64(x, g, b, eps=1e-5):
    x = x.astype(np.float64)
    mu = x.mean(-1, keepdims=True)
    var = ((x - mu) ** 2).mean(-1, keepdims=True)
    return (x - mu) / np.sqrt(var + eps) * g + b


def test_layernorm_closed_form():
    x = rnd(4, (9, 64), 3.0) - 1.0
    g = rnd(5, (64,)) + 1.0
    b = rnd(6, (64,))
    y, m, s = onn.layernorm(x, g, b)
    assert np.max(np.abs(y - ln64(x, g, b))) < 2e-5 * np.max(np.abs(y))
    assert np.allclose(m, x.astype(np.float64).mean(-1), atol=1e-6)
    # constant row: xhat = 0 -> y = beta
    yc, _, _ = onn.layernorm(np.full((2, 8), 3.25, np.float32), g[:8], b[:8])
    assert np.array_equal(yc, np.broadcast_to(b[:8], (2, 8)))


def test_layernorm_bwd_finite_differences():
    rows, dim = 3, 16
    x = rnd(7, (rows, dim), 1.5)
    g = rnd(8, (dim,)) + 1.0
    b = rnd(9, (dim,))
    G = rnd(10, (rows, dim))
    _, m, s = onn.layernorm(x, g, b)
    dx, dg, db = onn.layernorm_bwd(x, G, g, m, s)
    L = lambda xx, gg, bb: float(np.sum(ln64(xx, gg, bb) * G))
    h = 1e-6
    x64, g64, b64 = x.astype(np.float64), g.astype(np.float64), b.astype(np.float64)
    num_dx = np.zeros_like(x64)
    for i in range(rows):
        for j in range(dim):
            e = np.zeros_like(x64)
            e[i, j] = h
            num_dx[i, j] = (L(x64 + e, g64, b64) - L(x64 - e, g64, b64)) / (2 * h)
    num_dg = np.array([(L(x64, g64 + h * np.eye(dim)[j], b64) - L(x64, g64 - h * np.eye(dim)[j], b64)) / (2 * h)
                       for j in range(dim)])
    num_db = G.astype(np.float64).sum(0)
    assert oracle.rel_err(dx, num_dx) < 1e-4
    assert oracle.rel_err(dg, num_dg) < 1e-4
    assert oracle.rel_err(db, num_db) < 1e-6
    # invariants of the closed form: each dx row sums to 0 and is orthogonal to xhat
    xhat = (x64 - m[:, None]) * s[:, None]
    assert np.max(np.abs(dx.astype(np.float64).sum(1))) < 1e-4 * np.max(np.abs(dx))
    assert np.max(np.abs((dx * xhat).sum(1))) < 1e-3 * np.max(np.abs(dx))


# ----------------------------------------------------------------------- GELU
@need_ref
def test_gelu_fwd_bwd_bit_exact_vs_reference():
    x = np.concatenate([rnd(11, (4096,), 3.0), np.array([0.0, -0.0, 10.0, -10.0, 1e-30, 30.0], np.float32)])
    g = rnd(12, x.shape)
    assert np.array_equal(bits(onn.gelu(x)), bits(onn.ref_gelu(x)))
    assert np.array_equal(bits(onn.gelu_bwd(x, g)), bits(onn.ref_gelu_bwd(x, g)))


def test_gelu_closed_form_and_derivative():
    x = rnd(13, (512,), 2.0).astype(np.float64)
    f64 = lambda t: 0.5 * t * (1 + np.tanh(np.sqrt(2 / np.pi) * (t + 0.044715 * t ** 3)))
    assert np.max(np.abs(onn.gelu(x) - f64(x))) < 1e-6
    h = 1e-6
    num = (f64(x + h) - f64(x - h)) / (2 * h)
    assert np.max(np.abs(onn.gelu_bwd(x, np.ones_like(x)) - num)) < 1e-5
    assert onn.gelu(np.array([0.0], np.float32))[0] == 0.0


# -------------------------------------------------------------- cross-entropy
@need_ref
@pytest.mark.parametrize("rows,vocab", [(1, 3), (17, 100), (64, 8192)])
def test_cross_entropy_bit_exact_vs_reference(rows, vocab):
    logits = rnd(14, (rows, vocab), 3.0)
    t = (np.arange(rows) * 7919 % vocab).astype(np.int32)
    assert np.array_equal(bits(np.float32(onn.cross_entropy(logits, t))),
                          bits(np.float32(onn.ref_cross_entropy(logits, t))))


def test_cross_entropy_closed_forms():
    V = 64
    assert abs(onn.cross_entropy(np.zeros((5, V), np.float32), np.arange(5, dtype=np.int32)) - np.log(V)) < 1e-6
    assert np.isnan(onn.cross_entropy(np.zeros((2, V), np.float32), np.array([0, V], np.int32)))


def test_cross_entropy_bwd_finite_differences():
    rows, V = 4, 11
    x = rnd(15, (rows, V), 2.0)
    t = np.array([0, 10, 3, 3], np.int32)
    up = 0.75
    g = onn.cross_entropy_bwd(x, t, up)

    def L(z):
        z = z.astype(np.float64)
        mx = z.max(1, keepdims=True)
        lse = mx[:, 0] + np.log(np.exp(z - mx).sum(1))
        return up * float(np.mean(lse - z[np.arange(rows), t]))

    h = 1e-6
    num = np.zeros((rows, V))
    for i in range(rows):
        for j in range(V):
            e = np.zeros((rows, V))
            e[i, j] = h
            num[i, j] = (L(x + e) - L(x - e)) / (2 * h)
    assert oracle.rel_err(g, num) < 1e-5
    assert np.max(np.abs(g.astype(np.float64).sum(1))) < 1e-6


# ------------------------------------------------------------------ embedding
@need_ref
def test_embedding_bit_exact_vs_reference():
    table = rnd(16, (50, 24))
    ids = np.array([[3, 0, 49, 3], [7, 7, 1, 2]], np.int32)
    assert np.array_equal(onn.embedding(ids, table), onn.ref_embedding(ids, table))


def test_embedding_bwd_brute_force():
    vocab, dim = 20, 8
    ids = np.array([1, 5, 1, 19, 0, 1, 5], np.int32)
    gout = (np.arange(ids.size * dim).reshape(ids.size, dim) % 13 - 6).astype(np.float32)
    dt = onn.embedding_bwd(ids, gout, vocab)
    want = np.zeros((vocab, dim))
    for t, i in enumerate(ids):
        want[i] += gout[t]
    assert np.array_equal(dt, want.astype(np.float32))


# ---------------------------------------------------------------------- AdamW
@need_ref
@pytest.mark.parametrize("step", [1, 2, 10])
def test_adamw_bit_exact_vs_reference(step):
    n = 1000
    p, g = rnd(17, (n,)), rnd(18, (n,), 0.1)
    m, v = rnd(19, (n,), 0.01), np.abs(rnd(20, (n,), 0.001))
    a = onn.adamw(p, g, m, v, step)
    b = onn.ref_adamw(p, g, m, v, step)
    for x, y in zip(a, b):
        assert np.array_equal(bits(x), bits(y))


def test_adamw_first_step_closed_form():
    # step 1 from zero moments: m_hat = g, v_hat = g^2 -> update = g/(|g| + eps) + wd p
    p = rnd(21, (64,))
    g = rnd(22, (64,))
    z = np.zeros(64, np.float32)
    p1, m1, v1 = onn.adamw(p, g, z, z, 1, lr=0.01, weight_decay=0.1)
    want = p.astype(np.float64) - 0.01 * (np.sign(g) + 0.1 * p.astype(np.float64))
    assert np.max(np.abs(p1 - want)) < 1e-5
    assert onn.bias_correction(0.9, 1) == np.float32(1.0) - np.float32(0.9)


def test_sum_rows_brute_force():
    x = (np.arange(37 * 9).reshape(37, 9) % 11 - 5).astype(np.float32)
    assert np.array_equal(onn.sum_rows(x), x.astype(np.float64).sum(0).astype(np.float32))
