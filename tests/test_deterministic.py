"""The deterministic-dQ mode (inf_set_deterministic): every attention backward takes dQ from the
query-major pass (fp32 and bf16, D in {32, 64, 128}) instead of fp32 atomics.

Checks, on seeded inputs: O, LSE, dQ, dK, dV against the CPU oracle at the dtype's bar; dQ
bit-identical between calls (a fixed summation order), with the output buffers NaN-filled
before each call so every element must be written; dK and dV bit-identical to the default
mode's (the same main kernel computes them); and a HIP-graph replay equal to the eager call.
"""
import numpy as np
import pytest

import oracle

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

TOL_F32 = 1e-4
TOL_BF16 = 2e-2


@pytest.fixture(scope="module")
def ia():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import inferno_amd

    inferno_amd.lib()
    return inferno_amd


@pytest.fixture(autouse=True)
def default_mode_after(ia):
    yield
    ia.set_deterministic(False)


def dev(a, dtype):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda", dtype=dtype)


def host(t):
    return t.float().cpu().numpy()


def bf16_round(a):
    return oracle.bf16_to_f32(oracle.round_bf16(a))


def nan_like(t):
    return torch.full_like(t, float("nan"))


def bwd(ia, Q, K, V, o, dO, lse, causal):
    dq, dk, dv = nan_like(Q), nan_like(K), nan_like(V)
    ia.attn_bwd(Q, K, V, o, dO, lse, causal=causal, dq=dq, dk=dk, dv=dv)
    return dq, dk, dv


CASES = [
    # (dtype, causal, B, H, Tq, Tk, D)
    ("f32", True, 1, 4, 128, 128, 32),      # config 1
    ("f32", True, 2, 3, 333, 333, 64),
    ("f32", True, 1, 2, 300, 300, 128),
    ("f32", True, 1, 3, 250, 400, 64),      # end-aligned causal, Tq < Tk
    ("f32", False, 2, 2, 150, 260, 32),
    ("f32", False, 1, 2, 97, 45, 128),
    ("f32", True, 1, 4, 1024, 1024, 64),    # a backward split plan
    ("bf16", True, 1, 4, 128, 128, 32),
    ("bf16", True, 2, 3, 333, 333, 64),
    ("bf16", True, 1, 2, 300, 300, 128),
    ("bf16", True, 1, 3, 250, 400, 32),
    ("bf16", False, 2, 2, 150, 260, 64),
    ("bf16", False, 1, 2, 97, 45, 128),
    ("bf16", True, 1, 4, 1024, 1024, 64),
    ("f32", True, 1, 1, 1, 1, 64),          # a single query and key
    ("bf16", True, 2, 1, 17, 17, 32),
]


@pytest.mark.parametrize("dt,causal,B,H,Tq,Tk,D", CASES, ids=[f"{c[0]}-{'c' if c[1] else 'nc'}-B{c[2]}H{c[3]}Tq{c[4]}Tk{c[5]}D{c[6]}" for c in CASES])
def test_deterministic_parity(ia, dt, causal, B, H, Tq, Tk, D):
    print(f"[case] deterministic {dt} causal={causal} B{B} H{H} Tq{Tq} Tk{Tk} D{D}", flush=True)
    bf = dt == "bf16"
    dtype = torch.bfloat16 if bf else torch.float32
    q, k, v, do = oracle.attn_inputs(B, H, Tq, D, seed=900 + Tq + 3 * Tk + D, Tk=Tk)
    if bf:
        q, k, v, do = (bf16_round(x) for x in (q, k, v, do))
    o_r, lse_r = oracle.attn_fwd(q, k, v, causal=causal)
    dq_r, dk_r, dv_r = oracle.attn_bwd(q, k, v, do, causal=causal)
    Q, K, V, dO = (dev(x, dtype) for x in (q, k, v, do))
    o, lse = ia.attn_fwd(Q, K, V, causal=causal)
    base = bwd(ia, Q, K, V, o, dO, lse, causal)          # default mode
    assert ia.set_deterministic(True) is False
    first = bwd(ia, Q, K, V, o, dO, lse, causal)
    second = bwd(ia, Q, K, V, o, dO, lse, causal)
    torch.cuda.synchronize()
    tol = TOL_BF16 if bf else TOL_F32
    assert oracle.rel_err(host(lse), lse_r) <= (1e-3 if bf else TOL_F32), "LSE"
    assert oracle.rel_err(host(o), o_r, floor=1e-2) <= tol, "O"
    for name, x, r in zip(("dQ", "dK", "dV"), first, (dq_r, dk_r, dv_r)):
        assert torch.isfinite(x.float()).all(), f"{name} not fully written"
        e = oracle.rel_err(host(x), r, floor=1e-2)
        assert e <= tol, f"{name} rel err {e:.3e}"
    assert torch.equal(first[0], second[0]), "dQ differs between two deterministic calls"
    assert torch.equal(first[1], base[1]) and torch.equal(first[2], base[2]), "dK / dV changed with the mode"
    # the two modes sum dQ in different orders: equal within rounding
    assert oracle.rel_err(host(first[0]), host(base[0]), floor=1e-2) <= (1e-2 if bf else 1e-5)


def _random_cases(n=16, seed=77):
    """Seeded draws: B, H, ragged Tq <= Tk (causal, end-aligned) or any Tq, Tk (non-causal),
    D in {32, 64, 128}, fp32 and bf16 alternating."""
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        causal = bool(rng.integers(0, 4))
        D = int(rng.choice([32, 64, 128]))
        B, H = int(rng.integers(1, 3)), int(rng.integers(1, 4))
        Tq = int(rng.integers(1, 600))
        Tk = Tq + int(rng.integers(0, 300)) if causal else int(rng.integers(1, 700))
        cases.append(("bf16" if i % 2 else "f32", causal, B, H, Tq, Tk, D))
    return cases


@pytest.mark.parametrize("dt,causal,B,H,Tq,Tk,D", _random_cases())
def test_deterministic_random_shapes(ia, dt, causal, B, H, Tq, Tk, D):
    """The mode at seeded random shapes: dQ against the oracle and bit-identical on a second call."""
    print(f"[case] deterministic random {dt} causal={causal} B{B} H{H} Tq{Tq} Tk{Tk} D{D}", flush=True)
    bf = dt == "bf16"
    dtype = torch.bfloat16 if bf else torch.float32
    q, k, v, do = oracle.attn_inputs(B, H, Tq, D, seed=1300 + Tq + 5 * Tk + D, Tk=Tk)
    if bf:
        q, k, v, do = (bf16_round(x) for x in (q, k, v, do))
    dq_r, dk_r, dv_r = oracle.attn_bwd(q, k, v, do, causal=causal)
    Q, K, V, dO = (dev(x, dtype) for x in (q, k, v, do))
    ia.set_deterministic(True)
    o, lse = ia.attn_fwd(Q, K, V, causal=causal)
    first = bwd(ia, Q, K, V, o, dO, lse, causal)
    second = bwd(ia, Q, K, V, o, dO, lse, causal)
    torch.cuda.synchronize()
    tol = TOL_BF16 if bf else TOL_F32
    for name, x, r in zip(("dQ", "dK", "dV"), first, (dq_r, dk_r, dv_r)):
        e = oracle.rel_err(host(x), r, floor=1e-2)
        assert e <= tol, f"{name} rel err {e:.3e}"
    assert torch.equal(first[0], second[0]), "dQ differs between two deterministic calls"


@pytest.mark.parametrize("dt,D,T", [("f32", 64, 150), ("bf16", 64, 150), ("f32", 128, 97), ("bf16", 32, 211),
                                    ("bf16", 128, 130)])
def test_deterministic_strided_qkv_view(ia, dt, D, T):
    """The mode on q/k/v read straight out of a [B, T, 3, H, D] projection buffer and dq/dk/dv
    written into a gradient buffer of the same layout (the C++ layer's qkv_attention)."""
    print(f"[case] deterministic strided views {dt} D{D} T{T}", flush=True)
    dtype = torch.bfloat16 if dt == "bf16" else torch.float32
    B, H = 2, 3
    q, k, v, do = oracle.attn_inputs(B, H, T, D, seed=31)
    if dt == "bf16":
        q, k, v, do = (bf16_round(x) for x in (q, k, v, do))
    buf = torch.empty((B, T, 3, H, D), device="cuda", dtype=dtype)
    gbuf = torch.full((B, T, 3, H, D), float("nan"), device="cuda", dtype=dtype)
    for i, x in enumerate((q, k, v)):
        buf[:, :, i] = dev(x, dtype).transpose(1, 2)
    Q, K, V = (buf[:, :, i].permute(0, 2, 1, 3) for i in range(3))
    dQ, dK, dV = (gbuf[:, :, i].permute(0, 2, 1, 3) for i in range(3))
    ia.set_deterministic(True)
    o, lse = ia.attn_fwd(Q, K, V)
    ia.attn_bwd(Q, K, V, o, dev(do, dtype), lse, dq=dQ, dk=dK, dv=dV)
    torch.cuda.synchronize()
    dq_r, dk_r, dv_r = oracle.attn_bwd(q, k, v, do)
    tol = TOL_BF16 if dt == "bf16" else TOL_F32
    for name, x, r in (("dQ", dQ, dq_r), ("dK", dK, dk_r), ("dV", dV, dv_r)):
        e = oracle.rel_err(host(x), r)
        assert e <= tol, f"{name} rel err {e:.3e}"


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_deterministic_config2_full_size(ia, dt):
    """Config 2 (B8 H12 T1024 D64) in the mode: three heads against the oracle, dQ of every head
    bit-identical on a second call, sum_j dV_j = sum_i dO_i."""
    print(f"[case] deterministic config2 full size {dt}", flush=True)
    bf = dt == "bf16"
    dtype = torch.bfloat16 if bf else torch.float32
    B, H, T, D = 8, 12, 1024, 64
    q, k, v, do = oracle.attn_inputs(B, H, T, D, seed=42)
    if bf:
        q, k, v, do = (bf16_round(x) for x in (q, k, v, do))
    Q, K, V, dO = (dev(x, dtype) for x in (q, k, v, do))
    ia.set_deterministic(True)
    o_t, lse_t = ia.attn_fwd(Q, K, V)
    first = bwd(ia, Q, K, V, o_t, dO, lse_t, True)
    second = bwd(ia, Q, K, V, o_t, dO, lse_t, True)
    torch.cuda.synchronize()
    assert torch.equal(first[0], second[0]), "dQ differs between two deterministic calls"
    dq, dk, dv = (host(x) for x in first)
    assert np.isfinite(dq).all() and np.isfinite(dk).all() and np.isfinite(dv).all()
    tol = TOL_BF16 if bf else TOL_F32
    for (b, h) in ((0, 0), (3, 7), (7, 11)):
        sl = (slice(b, b + 1), slice(h, h + 1))
        dq_r, dk_r, dv_r = oracle.attn_bwd(q[sl], k[sl], v[sl], do[sl])
        for name, x, r in (("dQ", dq, dq_r), ("dK", dk, dk_r), ("dV", dv, dv_r)):
            e = oracle.rel_err(x[sl], r)
            assert e <= tol, f"head {(b, h)} {name} rel err {e:.3e}"
    assert oracle.rel_err(dv.astype(np.float64).sum(axis=2), do.astype(np.float64).sum(axis=2)) <= tol


@pytest.mark.parametrize("dt,D", [("f32", 64), ("bf16", 64), ("f32", 128)])
def test_deterministic_graph_replay(ia, dt, D):
    """Forward + backward captured into a HIP graph in the mode: three replays, inputs rewritten
    and outputs NaN-filled before each, every output bit-identical to the same eager calls."""
    print(f"[case] deterministic graph {dt} D{D}", flush=True)
    dtype = torch.bfloat16 if dt == "bf16" else torch.float32
    B, H, T = 2, 3, 700
    mk = lambda: torch.empty((B, H, T, D), device="cuda", dtype=dtype)  # noqa: E731
    q, k, v, do = mk(), mk(), mk(), mk()
    gen = torch.Generator(device="cuda").manual_seed(5)

    def refill():
        for t in (q, k, v, do):
            t.copy_(torch.randn(t.shape, device="cuda", generator=gen))

    refill()
    ia.set_deterministic(True)
    dti = ia.INF_BF16 if dt == "bf16" else ia.INF_F32

    def bufs():
        lse = torch.empty((B, H, T), device="cuda", dtype=torch.float32)
        fws = torch.empty(max(ia.workspace_bytes(ia.OP_ATTN_FWD, B, H, T, T, D, dti), 256), device="cuda",
                          dtype=torch.uint8)
        bws = torch.empty(max(ia.workspace_bytes(ia.OP_ATTN_BWD, B, H, T, T, D, dti), 256), device="cuda",
                          dtype=torch.uint8)
        return mk(), lse, mk(), mk(), mk(), fws, bws

    def step(bb):
        o, lse, dq, dk, dv, fws, bws = bb
        ia.attn_fwd(q, k, v, out=o, lse=lse, workspace=fws)
        ia.attn_bwd(q, k, v, o, do, lse, dq=dq, dk=dk, dv=dv, workspace=bws)

    gb, eb = bufs(), bufs()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step(gb)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step(gb)
    torch.cuda.synchronize()
    for rep in range(3):
        refill()
        step(eb)
        for t in gb[:5]:
            t.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for name, a, b in zip(("O", "LSE", "dQ", "dK", "dV"), gb[:5], eb[:5]):
            assert torch.equal(a, b), f"replay {rep}: {name} differs from the eager call"
