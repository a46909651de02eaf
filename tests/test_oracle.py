"""Pins the CPU oracle (oracle/oracle.c) before anything is checked against it.

Each oracle function is checked by something that would catch a plausible
mistake in it (a dropped term, a wrong sign, a transposed operand, a wrong
rounding point):
  - bit-exact equality with the reference's own header kernels compiled from
    /root/reference into oracle/_ref (skipped where that tree is absent);
  - the committed golden fixtures (tests/golden/*.npz) bit for bit;
  - closed forms, invariants and fp64 finite differences computed here
    independently of the oracle's code.
"""
import ctypes
from pathlib import Path

import numpy as np
import pytest

import oracle

GOLDEN = Path(__file__).resolve().parent / "golden"
# The reference build is loaded by a fixture, only by the tests that use it, so
# a run that deselects them (`-m gpu`) never maps it.
needs_ref = pytest.mark.skipif(not oracle.REF_PATH.exists(), reason="oracle/_ref not built (reference tree absent)")


@pytest.fixture(scope="module")
def REF():
    return oracle.ref_lib()


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def scale_of(D):
    return float(np.float32(1) / np.sqrt(np.float32(D)))


# ------------------------------------------------------------------ generator
def test_mt19937_64_standard_value():
    """The C++ standard fixes the 10000th output of mt19937_64 seeded with 5489."""
    L = oracle.lib()
    state = ctypes.create_string_buffer(312 * 8 + 8)
    L.orc_mt64_seed(state, 5489)
    x = 0
    for _ in range(10000):
        x = L.orc_mt64_next(state)
    assert x == 9981545732273789042


def test_randn_moments_and_determinism():
    a = oracle.randn(42, (200000,), 3.0)
    b = oracle.randn(42, (200000,), 3.0)
    assert np.array_equal(a, b)
    assert abs(a.mean()) < 0.03 and abs(a.std() - 3.0) < 0.03
    assert not np.array_equal(a, oracle.randn(43, (200000,), 3.0))


def test_bf16_rounding_known_values():
    x = np.array([1.0, 1.00390625, 1.01171875, -2.5, 0.0, 3.0e38, 1e-40], np.float32)
    # 1 + 2^-8 is a tie -> even (1.0); 1 + 3*2^-8 is a tie -> even (1 + 2^-6)
    expect = np.array([0x3F80, 0x3F80, 0x3F82, 0xC020, 0x0000], np.uint16)
    got = oracle.round_bf16(x)
    assert np.array_equal(got[:5], expect)
    torch = pytest.importorskip("torch")
    y = oracle.randn(9, (10000,), 10.0)
    t = torch.from_numpy(y).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(oracle.round_bf16(y), t)


# ------------------------------------------------ bit-exact vs the reference
@needs_ref
@pytest.mark.parametrize("M,K,N", [(1, 1, 1), (3, 5, 7), (17, 64, 33), (128, 32, 128)])
def test_matmul_bitwise_vs_reference(REF, M, K, N):
    a = oracle.randn(1, (1, 1, M, K))
    b = oracle.randn(2, (1, 1, K, N))
    ref = np.empty((1, 1, M, N), np.float32)
    sa = (ctypes.c_int64 * 4)(M * K, M * K, K, 1)
    sb = (ctypes.c_int64 * 4)(K * N, K * N, N, 1)
    REF.ref_matmul4_f32(a, sa, b, sb, ref, 1, 1, M, K, N)
    assert np.array_equal(bits(oracle.matmul(a[0, 0], b[0, 0])), bits(ref[0, 0]))


@needs_ref
def test_elementwise_kernels_bitwise_vs_reference(REF):
    L = oracle.lib()
    x = oracle.randn(3, (2, 3, 40, 40), 4.0)
    s = np.float32(0.17677669)
    out, ref = np.empty_like(x), np.empty_like(x)
    L.orc_scale_f32(x.reshape(-1), s, out.reshape(-1), x.size)
    REF.ref_scale_f32(x.reshape(-1), x.size, s, ref.reshape(-1))
    assert np.array_equal(bits(out), bits(ref))
    for diag in (0, 1, 5):
        m, mr = np.empty((40, 40), np.int32), np.empty((40, 40), np.int32)
        L.orc_triu_ones_i32(m, 40, 40, diag)
        REF.ref_triu_ones_i32(40, 40, diag, mr)
        assert np.array_equal(m, mr)
        assert np.array_equal(m, np.triu(np.ones((40, 40), np.int32), diag))
    m = np.triu(np.ones((40, 40), np.int32), 1)
    for bh in range(6):
        xs = x.reshape(6, 40, 40)[bh].copy()
        o = np.empty_like(xs)
        L.orc_masked_fill_f32(xs, m, np.float32(-1e9), o, 40, 40)
        assert (o[m == 1] == np.float32(-1e9)).all() and np.array_equal(o[m == 0], xs[m == 0])
    full = np.empty_like(x)
    REF.ref_masked_fill_f32(x, 2, 3, 40, 40, m, np.float32(-1e9), full)
    mine = np.stack([np.where(m == 1, np.float32(-1e9), x.reshape(6, 40, 40)[i]) for i in range(6)])
    assert np.array_equal(bits(full.reshape(6, 40, 40)), bits(mine))


@needs_ref
@pytest.mark.parametrize("rows,cols", [(1, 1), (5, 7), (64, 128), (3, 1000)])
def test_softmax_bitwise_vs_reference(REF, rows, cols):
    x = oracle.randn(4, (rows, cols), 5.0)
    ref = np.empty_like(x)
    REF.ref_softmax_f32(x, rows, cols, ref)
    assert np.array_equal(bits(oracle.softmax(x)), bits(ref))


@needs_ref
@pytest.mark.parametrize("rows,cols", [(1, 1), (5, 7), (64, 128), (3, 1000)])
def test_softmax_f64_and_i32_bitwise_vs_reference(REF, rows, cols):
    """Softmax's Float64 and Int32 instantiations (cpu_softmax<double, double>, <int, float>)."""
    x = oracle.randn(14, (rows, cols), 5.0).astype(np.float64) * (1 + 1e-9)
    ref = np.empty_like(x)
    REF.ref_softmax_f64(x, rows, cols, ref)
    assert np.array_equal(oracle.softmax_f64(x).view(np.uint64), ref.view(np.uint64))
    # ints spanning both exact and rounded int -> float conversions (|x| > 2^24)
    xi = (oracle.randn(15, (rows, cols), 4.0) * np.float32(3)).astype(np.int32)
    xi.reshape(-1)[:: 3] += np.int32(1 << 25) + 1
    refi = np.empty(xi.shape, np.float32)
    REF.ref_softmax_i32(xi, rows, cols, refi)
    assert np.array_equal(bits(oracle.softmax_i32(xi)), bits(refi))


def test_softmax_f64_i32_closed_forms():
    x = oracle.randn(16, (6, 50), 2.0).astype(np.float64)
    y = oracle.softmax_f64(x)
    e = np.exp(x - x.max(-1, keepdims=True))
    np.testing.assert_allclose(y, e / e.sum(-1, keepdims=True), rtol=1e-14, atol=0)
    xi = np.array([[0, 1, 2, -3], [5, 5, 5, 5]], np.int32)
    yi = oracle.softmax_i32(xi)
    ei = np.exp(xi.astype(np.float64) - xi.max(-1, keepdims=True))
    np.testing.assert_allclose(yi, ei / ei.sum(-1, keepdims=True), rtol=1e-6)
    assert yi.dtype == np.float32 and (yi[1] == np.float32(0.25)).all()


def test_softmax_bwd_f64_closed_form_and_finite_differences():
    x = oracle.randn(17, (3, 11), 1.5).astype(np.float64)
    g = oracle.randn(18, (3, 11)).astype(np.float64)
    y = oracle.softmax_f64(x)
    dx = oracle.softmax_bwd_f64(y, g)
    yl, gl = y.astype(np.longdouble), g.astype(np.longdouble)
    closed = yl * (gl - (gl * yl).sum(-1, keepdims=True))
    assert np.max(np.abs(dx - closed)) <= 1e-15
    assert np.max(np.abs(dx.sum(-1))) <= 1e-15

    def L(xx):
        ee = np.exp(xx - xx.max(-1, keepdims=True))
        return float((g * ee / ee.sum(-1, keepdims=True)).sum())

    h = 1e-5
    fd = np.zeros_like(x)
    for idx in np.ndindex(x.shape):
        xp, xm = x.copy(), x.copy()
        xp[idx] += h
        xm[idx] -= h
        fd[idx] = (L(xp) - L(xm)) / (2 * h)
    np.testing.assert_allclose(dx, fd, atol=1e-9)


@needs_ref
@pytest.mark.parametrize("B,H,T,D", [(1, 4, 128, 32), (2, 1, 17, 8), (1, 1, 1, 4), (1, 2, 65, 64)])
def test_attention_chain_bitwise_vs_reference(REF, B, H, T, D):
    q, k, v, do = oracle.attn_inputs(B, H, T, D, seed=42)
    sc = scale_of(D)
    o, _, p = oracle.attn_fwd(q, k, v, want_p=True)
    o_r, p_r = np.empty_like(o), np.empty_like(p)
    REF.ref_attn_fwd_f32(q, k, v, B, H, T, D, sc, 1, o_r, p_r.ctypes.data_as(ctypes.c_void_p))
    assert np.array_equal(bits(o), bits(o_r)) and np.array_equal(bits(p), bits(p_r))
    dq, dk, dv, ds = oracle.attn_bwd(q, k, v, do, want_ds=True)
    dp_r, dv_r, dq_r, dk_r = np.empty_like(p), np.empty_like(v), np.empty_like(q), np.empty_like(k)
    REF.ref_attn_bwd_stages_f32(q, k, v, p_r, do, ds, B, H, T, D, sc, dp_r, dv_r, dq_r, dk_r)
    for a, b in ((dv, dv_r), (dq, dq_r), (dk, dk_r)):
        assert np.array_equal(bits(a), bits(b))
    # the dS handed to the reference stages is SoftmaxBackward of (P, dP)
    ds64 = p_r.astype(np.float64) * (dp_r - (dp_r.astype(np.float64) * p_r).sum(-1, keepdims=True))
    assert np.max(np.abs(ds - ds64)) <= 1e-5 * max(1.0, np.max(np.abs(ds64)))


# ------------------------------------------------------------ golden fixtures
def test_golden_config1_bitwise():
    g = np.load(GOLDEN / "config1.npz")
    q, k, v, do = oracle.attn_inputs(1, 4, 128, 32, seed=42)
    for name, a in (("q", q), ("k", k), ("v", v), ("do", do)):
        assert np.array_equal(bits(a), bits(g[name])), name
    o, lse = oracle.attn_fwd(q, k, v)
    dq, dk, dv = oracle.attn_bwd(q, k, v, do)
    for name, a in (("o", o), ("lse", lse), ("dq", dq), ("dk", dk), ("dv", dv)):
        assert np.array_equal(bits(a), bits(g[name])), name


def test_golden_decode_and_softmax_bitwise():
    g = np.load(GOLDEN / "decode.npz")
    assert np.array_equal(bits(oracle.attn_decode(g["q"], g["kc"], g["vc"])), bits(g["o"]))
    s = np.load(GOLDEN / "softmax.npz")
    y = oracle.softmax(s["x"])
    assert np.array_equal(bits(y), bits(s["y"]))
    assert np.array_equal(bits(oracle.softmax_bwd(y, s["g"])), bits(s["dx"]))
    mask = np.triu(np.ones((8, 100), bool), 1)
    assert (y[mask] == 0).all()


# ------------------------------------------------- closed forms / invariants
def np_attention64(q, k, v, scale, causal=True):
    """Independent fp64 attention (vectorised formula, not the oracle's loops)."""
    q, k, v = (np.asarray(x, np.float64) for x in (q, k, v))
    s = np.einsum("bhid,bhjd->bhij", q, k) * scale
    Tq, Tk = s.shape[-2:]
    if causal:
        vis = np.arange(Tk)[None, :] <= np.arange(Tq)[:, None] + (Tk - Tq)
        s = np.where(vis, s, -np.inf)
    m = s.max(-1, keepdims=True)
    e = np.exp(s - m)
    l = e.sum(-1, keepdims=True)
    return np.einsum("bhij,bhjd->bhid", e / l, v), (m + np.log(l))[..., 0]


def test_softmax_closed_forms():
    x = oracle.randn(5, (6, 50), 2.0)
    y = oracle.softmax(x)
    assert np.all(y >= 0)
    np.testing.assert_allclose(y.sum(-1), 1.0, atol=1e-6)
    assert np.array_equal(oracle.softmax(np.zeros((1, 1), np.float32)), np.ones((1, 1), np.float32))
    np.testing.assert_allclose(oracle.softmax(x + np.float32(3.0)), y, atol=1e-6)
    # constant row over a visible prefix of i+1 entries -> 1/(i+1)
    T = 9
    c = np.where(np.triu(np.ones((T, T), bool), 1), np.float32(-1e9), np.float32(0.7))
    yc = oracle.softmax(c)
    for i in range(T):
        np.testing.assert_allclose(yc[i, : i + 1], 1.0 / (i + 1), rtol=1e-6)
        assert (yc[i, i + 1:] == 0).all()


def test_softmax_bwd_closed_form_and_finite_differences():
    x = oracle.randn(6, (4, 13), 1.5)
    g = oracle.randn(7, (4, 13))
    y = oracle.softmax(x)
    dx = oracle.softmax_bwd(y, g)
    y64, g64 = y.astype(np.float64), g.astype(np.float64)
    np.testing.assert_allclose(dx, y64 * (g64 - (g64 * y64).sum(-1, keepdims=True)), atol=1e-6)
    np.testing.assert_allclose(dx.sum(-1), 0.0, atol=1e-6)

    # d/dx of L = sum(g * softmax(x)) by fp64 central differences
    def L(xx):
        e = np.exp(xx - xx.max(-1, keepdims=True))
        return float((g64 * e / e.sum(-1, keepdims=True)).sum())

    x64, h = x.astype(np.float64), 1e-6
    fd = np.zeros_like(x64)
    for idx in np.ndindex(x64.shape):
        xp, xm = x64.copy(), x64.copy()
        xp[idx] += h
        xm[idx] -= h
        fd[idx] = (L(xp) - L(xm)) / (2 * h)
    np.testing.assert_allclose(dx, fd, atol=2e-6)


@pytest.mark.parametrize("B,H,T,D", [(1, 4, 128, 32), (2, 2, 37, 16), (1, 1, 1, 8)])
def test_attention_fwd_matches_fp64_formula(B, H, T, D):
    q, k, v, _ = oracle.attn_inputs(B, H, T, D, seed=9)
    o, lse = oracle.attn_fwd(q, k, v)
    o64, lse64 = np_attention64(q, k, v, scale_of(D))
    assert oracle.rel_err(o, o64) < 1e-5
    assert oracle.rel_err(lse, lse64) < 1e-6


def test_attention_fwd_closed_forms():
    B, H, T, D = 1, 2, 33, 8
    q, k, v, _ = oracle.attn_inputs(B, H, T, D, seed=1)
    # V == c  =>  O == c
    vc = np.full_like(v, np.float32(0.625))
    o, _ = oracle.attn_fwd(q, k, vc)
    np.testing.assert_allclose(o, 0.625, rtol=1e-6)
    # T == 1  =>  O == V exactly
    o1, lse1 = oracle.attn_fwd(q[:, :, :1], k[:, :, :1], v[:, :, :1])
    assert np.array_equal(o1, v[:, :, :1])
    np.testing.assert_allclose(lse1[..., 0], (q[:, :, 0] * k[:, :, 0]).sum(-1) * scale_of(D), rtol=1e-6)
    # Q == 0  =>  O_i = mean(V_0..V_i), the causal running mean
    o0, _ = oracle.attn_fwd(np.zeros_like(q), k, v)
    run_mean = np.cumsum(v.astype(np.float64), axis=2) / np.arange(1, T + 1)[None, None, :, None]
    np.testing.assert_allclose(o0, run_mean, atol=1e-6)
    # one dominant key per row => O_i ~= V of that key (row i sees key 0 only when strongly aligned)
    kd = np.zeros_like(k)
    kd[:, :, 0] = 50.0
    qd = np.ones_like(q)
    od, _ = oracle.attn_fwd(qd, kd, v)
    np.testing.assert_allclose(od, np.broadcast_to(v[:, :, :1], od.shape), atol=1e-5)


def test_lse_invariant():
    q, k, v, _ = oracle.attn_inputs(1, 2, 40, 16, seed=2, qk_sigma=3.0)
    o, lse, p = oracle.attn_fwd(q, k, v, want_p=True)
    s = np.einsum("bhid,bhjd->bhij", q.astype(np.float64), k.astype(np.float64)) * scale_of(16)
    vis = np.tril(np.ones((40, 40), bool))
    pp = np.where(vis, np.exp(s - lse[..., None].astype(np.float64)), 0.0)
    np.testing.assert_allclose(p, pp, atol=1e-5)  # fp32 LSE at |s| ~ 30: ulp ~ 2e-6


@pytest.mark.parametrize("causal", [True, False])
def test_attention_bwd_finite_differences(causal):
    """fp64 central differences of L = sum(O * dO) against the oracle's dQ, dK, dV."""
    B, H, T, D = 1, 1, 6, 4
    q, k, v, do = oracle.attn_inputs(B, H, T, D, seed=21)
    sc = scale_of(D)
    dq, dk, dv = oracle.attn_bwd(q, k, v, do, causal=causal)
    do64 = do.astype(np.float64)

    def L(qq, kk, vv):
        return float((np_attention64(qq, kk, vv, sc, causal)[0] * do64).sum())

    base = [x.astype(np.float64) for x in (q, k, v)]
    h = 1e-6
    for which, g in enumerate((dq, dk, dv)):
        fd = np.zeros_like(base[which])
        for idx in np.ndindex(fd.shape):
            plus = [x.copy() for x in base]
            minus = [x.copy() for x in base]
            plus[which][idx] += h
            minus[which][idx] -= h
            fd[idx] = (L(*plus) - L(*minus)) / (2 * h)
        np.testing.assert_allclose(g, fd, atol=5e-6, err_msg=f"input {which}")


def test_attention_bwd_invariants():
    B, H, T, D = 1, 2, 20, 8
    q, k, v, do = oracle.attn_inputs(B, H, T, D, seed=4)
    _, dk0, _ = oracle.attn_bwd(np.zeros_like(q), k, v, do)
    assert (dk0 == 0).all()  # Q = 0  =>  dK = 0 exactly
    dq, dk, dv, ds = oracle.attn_bwd(q, k, v, do, want_ds=True)
    np.testing.assert_allclose(ds.sum(-1), 0.0, atol=1e-5)  # rows of dS sum to 0
    assert (ds[..., np.triu(np.ones((T, T), bool), 1)] == 0).all()  # masked dS exactly 0
    _, _, p = oracle.attn_fwd(q, k, v, want_p=True)
    dv64 = np.einsum("bhij,bhid->bhjd", p.astype(np.float64), do.astype(np.float64))
    np.testing.assert_allclose(dv, dv64, atol=1e-5)  # dV = P^T dO


def test_decode_equals_last_prefill_row():
    q, k, v, _ = oracle.attn_inputs(2, 2, 50, 16, seed=8)
    o, _ = oracle.attn_fwd(q, k, v)
    od = oracle.attn_decode(q[:, :, -1:], k, v)
    assert oracle.rel_err(od, o[:, :, -1:]) < 1e-6
