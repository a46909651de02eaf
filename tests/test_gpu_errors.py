"""An error that an earlier, unrelated HIP call left pending on the calling thread is reported
by the next attention entry point (INF_ERR_HIP, named in inf_last_error_detail, nothing
launched) instead of being cleared by the planners' device queries; once reported it is
consumed, and the following call succeeds.

The pending error comes from hipSetDevice with an ordinal past the device count, which fails
on the host and changes nothing else."""
import ctypes

import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

INF_ERR_HIP = 9


@pytest.fixture(scope="module")
def ia():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import inferno_amd

    inferno_amd.lib()
    return inferno_amd


def leave_pending_error():
    hip = ctypes.CDLL("libamdhip64.so.7")  # the runtime torch and the library already share
    n = ctypes.c_int(0)
    assert hip.hipGetDeviceCount(ctypes.byref(n)) == 0
    assert hip.hipSetDevice(n.value + 7) != 0


@pytest.mark.parametrize("op", ["fwd", "bwd"])
def test_workspace_query_reports_pending_error(ia, op):
    print(f"[case] pending error workspace {op}", flush=True)
    L = ia.lib()
    code = ia.OP_ATTN_FWD if op == "fwd" else ia.OP_ATTN_BWD
    size = ctypes.c_size_t(0)
    leave_pending_error()
    assert L.inf_attn_workspace_bytes(code, 1, 2, 512, 512, 64, ia.INF_F32, ctypes.byref(size)) == INF_ERR_HIP
    detail = L.inf_last_error_detail()
    assert b"pending from an earlier call" in detail and b"hipErrorInvalidDevice" in detail
    assert L.inf_attn_workspace_bytes(code, 1, 2, 512, 512, 64, ia.INF_F32, ctypes.byref(size)) == 0


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_attention_calls_report_pending_error(ia, dtype):
    """inf_attn_fwd / inf_attn_bwd with every output and the workspace allocated beforehand, so
    that the pending error is left right before the C-ABI call (torch's own calls would report
    it first)."""
    print(f"[case] pending error attention {dtype}", flush=True)
    B, H, T, D = 1, 2, 256, 64
    dt = ia.INF_BF16 if dtype == torch.bfloat16 else ia.INF_F32
    q, k, v, do = (torch.randn(B, H, T, D, device="cuda").to(dtype) for _ in range(4))
    fws = torch.empty(max(ia.workspace_bytes(ia.OP_ATTN_FWD, B, H, T, T, D, dt), 256),
                      dtype=torch.uint8, device="cuda")
    bws = torch.empty(max(ia.workspace_bytes(ia.OP_ATTN_BWD, B, H, T, T, D, dt), 256),
                      dtype=torch.uint8, device="cuda")
    o, lse = ia.attn_fwd(q, k, v, workspace=fws)
    o2, lse2 = torch.empty_like(o), torch.empty_like(lse)
    grads = [torch.empty_like(x) for x in (q, k, v)]
    torch.cuda.synchronize()
    leave_pending_error()
    with pytest.raises(ia.InfernoError) as ex:
        ia.attn_fwd(q, k, v, out=o2, lse=lse2, workspace=fws)
    assert ex.value.status == INF_ERR_HIP
    ia.attn_fwd(q, k, v, out=o2, lse=lse2, workspace=fws)
    leave_pending_error()
    with pytest.raises(ia.InfernoError) as ex:
        ia.attn_bwd(q, k, v, o, do, lse, dq=grads[0], dk=grads[1], dv=grads[2], workspace=bws)
    assert ex.value.status == INF_ERR_HIP
    ia.attn_bwd(q, k, v, o, do, lse, dq=grads[0], dk=grads[1], dv=grads[2], workspace=bws)
    torch.cuda.synchronize()
    assert torch.equal(o, o2) and torch.equal(lse, lse2)
