"""inf_attn_decode_static, the decode entry point that allocates nothing (its split partials
live in the library's static device scratch), through the C-ABI against inf_attn_decode
(workspace from the caller): the same kernels and plan, so the outputs must be bit-identical.
Two calls in a row per dtype, the second on a smaller input with fewer splits, so partials
the first call left in the scratch must not leak into the second; a last check against the
oracle on the rounded inputs.
"""
import numpy as np
import pytest

import oracle

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ia():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import inferno_amd

    inferno_amd.lib()
    return inferno_amd


def dev(a, dtype):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda", dtype=dtype)


def decode_static(ia, q, kc, vc, out):
    B, H, _, D = q.shape
    Tk = kc.shape[2]
    s = ia.ops.strides_of
    st = ia.lib().inf_attn_decode_static(q.data_ptr(), s(q), kc.data_ptr(), s(kc), vc.data_ptr(), s(vc),
                                         out.data_ptr(), s(out), B, H, Tk, D, ia.default_scale(D),
                                         ia.ops._dt(q), None)
    return st


@pytest.mark.parametrize("dtype,D", [(torch.float32, 64), (torch.bfloat16, 64), (torch.float32, 128)])
def test_static_decode_equals_workspace_decode(ia, dtype, D):
    shapes = [(32, 12, 2048), (3, 5, 700)]  # config 5, then a smaller input with fewer splits
    for i, (B, H, Tk) in enumerate(shapes):
        print(f"[case] decode static {dtype} B{B} H{H} Tk{Tk} D{D} call {i}", flush=True)
        q = oracle.randn(900 + i, (B, H, 1, D))
        kc = oracle.randn(910 + i, (B, H, Tk, D))
        vc = oracle.randn(920 + i, (B, H, Tk, D))
        if dtype == torch.bfloat16:
            q, kc, vc = (oracle.bf16_to_f32(oracle.round_bf16(x)) for x in (q, kc, vc))
        Q, K, V = dev(q, dtype), dev(kc, dtype), dev(vc, dtype)
        assert ia.workspace_bytes(ia.OP_ATTN_DECODE, B, H, 1, Tk, D, ia.ops._dt(Q)) > 0  # splits: scratch used
        out = torch.full((B, H, 1, D), float("nan"), dtype=dtype, device="cuda")
        torch.cuda.synchronize()
        st = decode_static(ia, Q, K, V, out)
        assert st == 0, ia.status_string(st)
        torch.cuda.synchronize()
        ref = ia.attn_decode(Q, K, V)
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"call {i}: differs from inf_attn_decode"
        tol = 1e-4 if dtype == torch.float32 else 2e-2
        assert oracle.rel_err(out.float().cpu().numpy(), oracle.attn_decode(q, kc, vc)) <= tol
