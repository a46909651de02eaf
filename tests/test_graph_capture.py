"""HIP graph capture of the C-ABI entry points: a caller may record inf_attn_fwd / inf_attn_bwd,
inf_attn_decode, inf_attn_decode_static and the softmax pair into a graph and replay it.

The library issues kernels only (no memset / memcpy / allocation / synchronisation calls; the
backward's accumulator and delta are cleared by its own pre-pass kernel), so capture records the
same launches as an eager call.  Each case captures once, then replays three times; before each
replay the inputs are rewritten in place with new values, the same calls run eagerly into other
buffers, and the graph's outputs are filled with NaN, so every replay must recompute everything
from the current inputs.  Outputs with one writer per element (O, LSE, dK, dV, decode, softmax,
and dQ of the query-major pass) must match the eager ones bit for bit; dQ summed by fp32 atomics
(order-dependent) within 1e-5 (fp32) or one bf16 step (bf16).
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ia():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import inferno_amd

    inferno_amd.lib()
    return inferno_amd


def _rel(a, b):
    a, b = a.float(), b.float()
    return float((a - b).abs().max() / b.abs().max().clamp_min(1e-30))


def _capture(fn):
    """Warm up on a side stream (plans and caches), then record fn into a graph."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    torch.cuda.synchronize()
    return g


def _replays(g, inputs, refill, eager, graph_outs, eager_outs, check, reps=3):
    gen = torch.Generator(device="cuda").manual_seed(1234)
    for rep in range(reps):
        for t in inputs:
            refill(t, gen)
        eager()
        for t in graph_outs:
            t.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        check(rep, graph_outs, eager_outs)


def _randn_(t, gen, sigma=1.0):
    t.copy_(torch.randn(t.shape, device="cuda", generator=gen) * sigma)


ATTN_CASES = [
    # name, dtype, B, H, T, D, causal, dq deterministic
    ("f32 B2 H4 T512 D64 causal", torch.float32, 2, 4, 512, 64, True, False),
    ("bf16 B2 H4 T512 D64 causal", torch.bfloat16, 2, 4, 512, 64, True, False),
    ("f32 split plans B1 H2 T2048 D64", torch.float32, 1, 2, 2048, 64, True, False),
    ("bf16 split plans B1 H2 T2048 D128", torch.bfloat16, 1, 2, 2048, 128, True, False),
    ("bf16 query-major dQ B2 H8 T4096 D128", torch.bfloat16, 2, 8, 4096, 128, True, True),
    ("f32 non-causal ragged B1 H3 T300 D32", torch.float32, 1, 3, 300, 32, False, False),
]


@pytest.mark.parametrize("name,dtype,B,H,T,D,causal,dq_exact", ATTN_CASES, ids=[c[0] for c in ATTN_CASES])
def test_attention_fwd_bwd_graph(ia, name, dtype, B, H, T, D, causal, dq_exact):
    print(f"[case] graph fwd+bwd {name}", flush=True)
    mk = lambda: torch.empty((B, H, T, D), device="cuda", dtype=dtype)  # noqa: E731
    q, k, v, do = mk(), mk(), mk(), mk()
    gen = torch.Generator(device="cuda").manual_seed(7)
    for t in (q, k, v, do):
        _randn_(t, gen)
    dt = ia.ops._dt(q)

    def bufs():
        o = mk()
        lse = torch.empty((B, H, T), device="cuda", dtype=torch.float32)
        fws = torch.empty(max(ia.workspace_bytes(ia.OP_ATTN_FWD, B, H, T, T, D, dt), 256), device="cuda",
                          dtype=torch.uint8)
        bws = torch.empty(max(ia.workspace_bytes(ia.OP_ATTN_BWD, B, H, T, T, D, dt), 256), device="cuda",
                          dtype=torch.uint8)
        return o, lse, mk(), mk(), mk(), fws, bws

    def step(b):
        o, lse, dq, dk, dv, fws, bws = b
        ia.attn_fwd(q, k, v, causal=causal, out=o, lse=lse, workspace=fws)
        ia.attn_bwd(q, k, v, o, do, lse, causal=causal, dq=dq, dk=dk, dv=dv, workspace=bws)

    gb, eb = bufs(), bufs()
    g = _capture(lambda: step(gb))
    tol_dq = 0.0 if dq_exact else (1e-5 if dtype == torch.float32 else 1e-2)

    def check(rep, gouts, eouts):
        for nm, a, b in zip(("O", "LSE", "dQ", "dK", "dV"), gouts[:5], eouts[:5]):
            assert torch.isfinite(a.float()).all(), f"replay {rep}: {nm} not fully written"
            if nm == "dQ" and tol_dq > 0:
                e = _rel(a, b)
                assert e <= tol_dq, f"replay {rep}: dQ differs from eager by {e:.2e}"
            else:
                assert torch.equal(a, b), f"replay {rep}: {nm} differs from the eager call"

    _replays(g, (q, k, v, do), _randn_, lambda: step(eb), list(gb[:5]), list(eb[:5]), check)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_decode_graph(ia, dtype):
    """inf_attn_decode (caller workspace) and inf_attn_decode_static (library scratch) in one graph."""
    print(f"[case] graph decode {dtype}", flush=True)
    B, H, Tk, D = 4, 6, 1500, 64
    q = torch.empty((B, H, 1, D), device="cuda", dtype=dtype)
    kc = torch.empty((B, H, Tk, D), device="cuda", dtype=dtype)
    vc = torch.empty_like(kc)
    gen = torch.Generator(device="cuda").manual_seed(3)
    for t in (q, kc, vc):
        _randn_(t, gen)
    dt = ia.ops._dt(q)
    s = ia.Strides

    def st(t):
        x = t.stride()
        return s(x[0], x[1], x[2], x[3])

    def static_call(out):
        r = ia.lib().inf_attn_decode_static(q.data_ptr(), st(q), kc.data_ptr(), st(kc), vc.data_ptr(), st(vc),
                                            out.data_ptr(), st(out), B, H, Tk, D, ia.default_scale(D), dt,
                                            torch.cuda.current_stream().cuda_stream)
        assert r == 0, (r, ia.lib().inf_last_error_detail())

    ws_g = torch.empty(max(ia.workspace_bytes(ia.OP_ATTN_DECODE, B, H, 1, Tk, D, dt), 256), device="cuda",
                       dtype=torch.uint8)
    ws_e = torch.empty_like(ws_g)
    go1, go2, eo1, eo2 = (torch.empty_like(q) for _ in range(4))

    def graph_step():
        ia.attn_decode(q, kc, vc, out=go1, workspace=ws_g)
        static_call(go2)

    def eager_step():
        ia.attn_decode(q, kc, vc, out=eo1, workspace=ws_e)
        static_call(eo2)

    g = _capture(graph_step)

    def check(rep, gouts, eouts):
        for nm, a, b in zip(("decode", "decode_static"), gouts, eouts):
            assert torch.equal(a, b), f"replay {rep}: {nm} differs from the eager call"
        assert torch.equal(gouts[0], gouts[1]), f"replay {rep}: the two decode entry points differ"

    _replays(g, (q, kc, vc), _randn_, eager_step, [go1, go2], [eo1, eo2], check)


@pytest.mark.parametrize("cols", [1000, 6000], ids=["wave-rows", "block-rows"])
def test_softmax_graph(ia, cols):
    print(f"[case] graph softmax cols={cols}", flush=True)
    rows = 96
    x = torch.empty((rows, cols), device="cuda")
    dy = torch.empty_like(x)
    gen = torch.Generator(device="cuda").manual_seed(5)
    for t in (x, dy):
        _randn_(t, gen, 3.0)
    gy, gdx, ey, edx = (torch.empty_like(x) for _ in range(4))

    def step(y, dx):
        ia.softmax_fwd(x, out=y)
        ia.softmax_bwd(y, dy, out=dx)

    g = _capture(lambda: step(gy, gdx))

    def check(rep, gouts, eouts):
        for nm, a, b in zip(("y", "dx"), gouts, eouts):
            assert torch.equal(a, b), f"replay {rep}: softmax {nm} differs from the eager call"

    _replays(g, (x, dy), lambda t, gen: _randn_(t, gen, 3.0), lambda: step(ey, edx), [gy, gdx], [ey, edx], check)
    assert np.isfinite(gy.cpu().numpy()).all()
