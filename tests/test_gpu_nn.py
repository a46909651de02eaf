"""GPU parity of the model ops around the attention path (GEMM, LayerNorm,
GELU, cross-entropy, embedding, AdamW, column sums, broadcast add) through
the C-ABI, against the CPU oracle (oracle/oracle_nn.c, pinned in
tests/test_oracle_nn.py).

Bar: max|x - ref| / max|ref| <= 1e-4 for fp32 (the reductions run in a
different order than the reference's sequential loops); bit-exact where the
arithmetic is exact (embedding gather, integer-valued scatter and sums).
Shapes: the GPT-2-small step (rows = 8 x 1024 tokens, C = 768, 4C = 3072,
vocab 8192) and ragged edges.
"""
import numpy as np
import pytest

import oracle
from oracle import nn as onn

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

TOL = 1e-4


@pytest.fixture(scope="module")
def ia():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import inferno_amd

    inferno_amd.lib()
    return inferno_amd


def dev(a, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a)).to("cuda")
    return t if dtype is None else t.to(dtype)


def host(t):
    return t.float().cpu().numpy()


def rnd(seed, shape, sigma=1.0):
    return oracle.randn(seed, shape, sigma)


# ----------------------------------------------------------------------- GEMM
@pytest.mark.parametrize("M,K,N", [(64, 32, 48), (129, 77, 33), (1, 768, 768), (1024, 768, 2304)])
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_gemm_parity(ia, M, K, N, ta, tb):
    print(f"[case] gemm M{M} K{K} N{N} ta{ta} tb{tb}", flush=True)
    a = rnd(1, (K, M) if ta else (M, K))
    b = rnd(2, (N, K) if tb else (K, N))
    bias = rnd(3, (N,))
    A = a.T if ta else a
    Bm = b.T if tb else b
    want = A.astype(np.float64) @ Bm.astype(np.float64) + bias
    got = ia.gemm(dev(a), dev(b), trans_a=bool(ta), trans_b=bool(tb), bias=dev(bias))
    torch.cuda.synchronize()
    assert oracle.rel_err(host(got), want) < TOL
    # without bias, and against the restated cpu_matmul
    got2 = ia.gemm(dev(a), dev(b), trans_a=bool(ta), trans_b=bool(tb))
    assert oracle.rel_err(host(got2), oracle.matmul(A, Bm)) < TOL


def test_gemm_beta_accumulate_and_ld(ia):
    """C = 2 A B + 0.5 C on views with leading dimensions larger than their widths."""
    M, K, N = 40, 24, 20
    a_full = dev(rnd(4, (M, K + 8)))
    b_full = dev(rnd(5, (K, N + 12)))
    c_full = dev(rnd(6, (M, N + 4)))
    c0 = host(c_full)[:, :N].astype(np.float64)
    a, b, c = a_full[:, :K], b_full[:, :N], c_full[:, :N]
    ia.gemm(a, b, alpha=2.0, beta=0.5, out=c)
    want = 2 * host(a).astype(np.float64) @ host(b).astype(np.float64) + 0.5 * c0
    assert oracle.rel_err(host(c_full)[:, :N], want) < TOL
    assert np.array_equal(host(c_full)[:, N:], host(c_full)[:, N:])  # untouched columns stay


def test_gemm_batched_strided(ia):
    import ctypes

    Bt, M, K, N = 3, 33, 20, 17
    a, b = rnd(7, (Bt, M, K)), rnd(8, (Bt, K, N))
    A, B_, C = dev(a), dev(b), torch.zeros((Bt, M, N), device="cuda")
    ws = torch.empty(ia.nn_workspace_bytes(ia.OP_GEMM), dtype=torch.uint8, device="cuda")
    st = ia.lib().inf_gemm(0, 0, M, N, K, 1.0, A.data_ptr(), K, M * K, B_.data_ptr(), N, K * N, 0.0,
                           C.data_ptr(), N, M * N, Bt, None, 0, ws.data_ptr(), ws.numel(),
                           torch.cuda.current_stream().cuda_stream)
    assert st == 0
    want = np.einsum("bmk,bkn->bmn", a.astype(np.float64), b.astype(np.float64))
    assert oracle.rel_err(host(C), want) < TOL


# ------------------------------------------------------------------ LayerNorm
@pytest.mark.parametrize("rows,dim", [(8192, 768), (5, 64), (3, 1000), (7, 2048), (2, 33)])
def test_layernorm_parity(ia, rows, dim):
    print(f"[case] layernorm rows{rows} dim{dim}", flush=True)
    x = rnd(10, (rows, dim), 2.0) + 0.3
    g, b = rnd(11, (dim,)) + 1.0, rnd(12, (dim,))
    y, m, s = ia.layernorm_fwd(dev(x), dev(g), dev(b))
    yr, mr, sr = onn.layernorm(x, g, b)
    assert oracle.rel_err(host(y), yr) < TOL
    assert oracle.rel_err(host(m), mr) < TOL and oracle.rel_err(host(s), sr) < TOL
    if dim % 4 == 0 and dim <= 2048:
        G = rnd(13, (rows, dim))
        dx, dg, db = ia.layernorm_bwd(dev(x), dev(G), dev(g), m, s)
        dxr, dgr, dbr = onn.layernorm_bwd(x, G, g, mr, sr)
        assert oracle.rel_err(host(dx), dxr) < TOL
        assert oracle.rel_err(host(dg), dgr) < TOL
        assert oracle.rel_err(host(db), dbr) < TOL


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("rows,dim", [(32, 768), (257, 770), (8, 4096)])
def test_add_layernorm_equals_add_then_layernorm(ia, dtype, rows, dim):
    """inf_add_layernorm_fwd gives bit for bit what an add followed by inf_layernorm_fwd gives
    (register kernel for dim % 4 == 0, scalar kernel otherwise), also with h written over x."""
    print(f"[case] add_layernorm {dtype} rows{rows} dim{dim}", flush=True)
    x, r = dev(rnd(40, (rows, dim), 2.0), dtype), dev(rnd(41, (rows, dim)), dtype)
    g, b = dev(rnd(42, (dim,)) + 1.0), dev(rnd(43, (dim,)))
    h_ref = x + r  # torch rounds the fp32 sum to the tensor dtype, as the fused kernel does
    y_ref, _, _ = ia.layernorm_fwd(h_ref, g, b)
    h, y = ia.add_layernorm_fwd(x, r, g, b)
    torch.cuda.synchronize()
    assert torch.equal(h, h_ref) and torch.equal(y, y_ref)
    xi = x.clone()
    h2, y2 = ia.add_layernorm_fwd(xi, r, g, b, h=xi)  # residual stream updated in place
    torch.cuda.synchronize()
    assert torch.equal(xi, h_ref) and torch.equal(y2, y_ref)


# ----------------------------------------------------------------------- GELU
@pytest.mark.parametrize("n", [8192 * 3072, 1, 4099])
def test_gelu_parity(ia, n):
    x = rnd(14, (n,), 3.0)
    g = rnd(15, (n,))
    assert oracle.rel_err(host(ia.gelu_fwd(dev(x))), onn.gelu(x)) < TOL
    assert oracle.rel_err(host(ia.gelu_bwd(dev(x), dev(g))), onn.gelu_bwd(x, g)) < TOL


# -------------------------------------------------------------- cross-entropy
@pytest.mark.parametrize("rows,vocab", [(8192, 8192), (3, 5), (17, 22197)])
def test_cross_entropy_parity(ia, rows, vocab):
    print(f"[case] cross_entropy rows{rows} vocab{vocab}", flush=True)
    x = rnd(16, (rows, vocab), 2.0)
    t = ((np.arange(rows) * 7919 + 13) % vocab).astype(np.int32)
    loss, lse = ia.cross_entropy_fwd(dev(x), dev(t))
    ref = onn.cross_entropy(x, t)
    assert abs(float(host(loss)[0]) - ref) <= TOL * abs(ref)
    up = dev(np.array([0.5], np.float32))
    g = ia.cross_entropy_bwd(dev(x), dev(t), lse, up)
    assert oracle.rel_err(host(g), onn.cross_entropy_bwd(x, t, 0.5)) < TOL


def test_cross_entropy_bad_target_is_nan(ia):
    x = rnd(17, (2, 8))
    loss, _ = ia.cross_entropy_fwd(dev(x), dev(np.array([1, 8], np.int32)))
    assert np.isnan(host(loss)[0])


# ------------------------------------------------------------------ embedding
def test_embedding_parity(ia):
    vocab, dim, n = 8192, 768, 8192
    table = rnd(18, (vocab, dim), 0.02)
    ids = ((np.arange(n) * 2654435761) % vocab).astype(np.int32)
    ids[:64] = 5  # repeated ids collide in the scatter
    out = ia.embedding_fwd(dev(ids), dev(table))
    assert np.array_equal(host(out), onn.embedding(ids, table))
    # scatter-add of integer-valued gradients is exact in any order
    gout = ((np.arange(n * dim) % 7) - 3).astype(np.float32).reshape(n, dim)
    dt = ia.embedding_bwd(dev(ids), dev(gout), vocab)
    assert np.array_equal(host(dt), onn.embedding_bwd(ids, gout, vocab))


@pytest.mark.parametrize("vocab,dim,n", [(8192, 768, 8192), (1000, 100, 3000), (37, 16384, 50)])
def test_embedding_bwd_deterministic(ia, vocab, dim, n):
    """The deterministic mode's embedding backward sums each row in token order, as the
    oracle's CPU loop does: bit-identical to the oracle for arbitrary fp32 gradients (repeated
    ids and ids outside [0, vocab) included), and, accumulating into an existing dtable, to the
    same sequential sum started from that table."""
    print(f"[case] embedding bwd deterministic vocab{vocab} dim{dim} n{n}", flush=True)
    rng = np.random.default_rng(vocab + dim)
    ids = rng.integers(0, vocab, n).astype(np.int32)
    ids[: n // 4] = 3                       # one row collects a quarter of the tokens
    ids[n // 4 : n // 4 + 5] = [-1, vocab, vocab + 7, -100, 2 ** 31 - 1]  # skipped
    gout = rng.standard_normal((n, dim)).astype(np.float32)
    I, G = dev(ids), dev(gout)
    prev = ia.set_deterministic(True)
    try:
        dt = ia.embedding_bwd(I, G, vocab)
        dt2 = ia.embedding_bwd(I, G, vocab)
        base = rng.standard_normal((vocab, dim)).astype(np.float32)
        acc = dev(base)
        st = ia.lib().inf_embedding_bwd(I.data_ptr(), n, G.data_ptr(), vocab, dim, acc.data_ptr(), 0,
                                        torch.cuda.current_stream().cuda_stream)
        assert st == 0
        torch.cuda.synchronize()
    finally:
        ia.set_deterministic(prev)
    assert torch.equal(dt, dt2)
    ok = (ids >= 0) & (ids < vocab)  # the oracle's loop takes valid ids only
    assert np.array_equal(host(dt), onn.embedding_bwd(ids[ok], gout[ok], vocab))
    want = base.copy()
    for t in range(n):  # the same fp32 additions in token order
        if 0 <= ids[t] < vocab:
            want[ids[t]] += gout[t]
    assert np.array_equal(host(acc), want)


# ---------------------------------------------------------------------- AdamW
@pytest.mark.parametrize("step", [1, 3])
def test_adamw_parity(ia, step):
    n = 768 * 3072 + 3
    p, g = rnd(19, (n,), 0.02), rnd(20, (n,), 0.01)
    m, v = rnd(21, (n,), 0.001), np.abs(rnd(22, (n,), 1e-5))
    P, G, Mm, V = dev(p), dev(g), dev(m), dev(v)
    ia.adamw_step(P, G, Mm, V, step)
    pr, mr, vr = onn.adamw(p, g, m, v, step)
    assert oracle.rel_err(host(P), pr) < TOL
    assert oracle.rel_err(host(Mm), mr) < TOL and oracle.rel_err(host(V), vr) < TOL


@pytest.mark.parametrize("bf16", [False, True])
def test_adamw_multi_matches_single(ia, bf16):
    """The multi-tensor step equals the per-tensor step bit for bit: 60 tensors (two launches of
    at most 48), sizes with ragged tails, one tensor larger than a 1024-element group."""
    print(f"[case] adamw multi bf16={bf16}", flush=True)
    dt = torch.bfloat16 if bf16 else torch.float32
    sizes = [1, 3, 4, 5, 1023, 1024, 1025, 768 * 2304 + 7] + [17 * (i + 1) for i in range(52)]
    a, b = [], []
    for i, n in enumerate(sizes):
        p, g = rnd(100 + i, (n,), 0.02), rnd(200 + i, (n,), 0.01)
        m, v = rnd(300 + i, (n,), 0.001), np.abs(rnd(400 + i, (n,), 1e-5))
        a.append((dev(p).to(dt), dev(g).to(dt), dev(m), dev(v)))
        b.append(tuple(t.clone() for t in a[-1]))
    for step in (1, 2):
        for P, G, M, V in a:
            ia.adamw_step(P, G, M, V, step)
        ia.adamw_step_multi(b, step)
    torch.cuda.synchronize()
    for (P, _, M, V), (P2, _, M2, V2) in zip(a, b):
        assert torch.equal(P, P2) and torch.equal(M, M2) and torch.equal(V, V2)


@pytest.mark.parametrize("rows,cols,dt", [(32, 8192, "f32"), (5, 1, "f32"), (3, 1000, "bf16"), (7, 65, "f32")])
def test_argmax_rows(ia, rows, cols, dt):
    """Row argmax = numpy's argmax (first index on ties): random rows, plus rows of ties and a
    maximum in the last column; bf16 values compared after rounding."""
    print(f"[case] argmax {rows}x{cols} {dt}", flush=True)
    x = rnd(31, (rows, cols))
    x[0, :] = 1.0                      # all equal: index 0
    if cols > 3:
        x[1, 2] = x[1, 3] = 50.0       # tie: first of the two
        x[2 % rows, -1] = 60.0         # maximum in the last column
    tdt = torch.bfloat16 if dt == "bf16" else torch.float32
    X = dev(x).to(tdt)
    got = host(ia.argmax_rows(X)).astype(np.int64)
    want = np.argmax(X.float().cpu().numpy(), axis=1)
    assert np.array_equal(got, want)
    # a strided row view (every other row of a wider buffer)
    W = torch.zeros((2 * rows, cols + 3), dtype=tdt, device="cuda")
    W[::2, :cols] = X
    assert np.array_equal(host(ia.argmax_rows(W[::2, :cols])).astype(np.int64), want)


# ----------------------------------------------------------- reductions, bcast
@pytest.mark.parametrize("rows,cols", [(8192, 768), (1, 5), (300, 3072)])
def test_col_sum_parity(ia, rows, cols):
    x = rnd(23, (rows, cols))
    assert oracle.rel_err(host(ia.col_sum(dev(x))), onn.sum_rows(x)) < TOL
    xi = ((np.arange(rows * cols) % 9) - 4).astype(np.float32).reshape(rows, cols)
    assert np.array_equal(host(ia.col_sum(dev(xi))), onn.sum_rows(xi))


@pytest.mark.parametrize("n,nb", [(8 * 1024 * 768, 1024 * 768), (30, 3), (16, 16)])
def test_binary_bcast(ia, n, nb):
    a, b = rnd(24, (n,)), rnd(25, (nb,))
    got = host(ia.binary_bcast(0, dev(a), dev(b)))
    want = (a.reshape(-1, nb) + b).reshape(-1)
    assert np.array_equal(got, want)
    got = host(ia.binary_bcast(1, dev(a), dev(b)))
    assert np.array_equal(got, (a.reshape(-1, nb) * b).reshape(-1))
