"""Torch-facing helpers over the C-ABI (device memory and streams come from torch).

Each helper validates nothing itself: the C-ABI validates on the host and a
non-zero status raises InfernoError.  Tensors must live on the GPU; the
launches go to torch's current stream.
"""
from __future__ import annotations

import torch

from . import INF_BF16, INF_F32, INF_F64, INF_I32, OP_ATTN_BWD, OP_ATTN_DECODE, OP_ATTN_FWD, InfernoError, Strides, default_scale, lib, workspace_bytes


def _dt(t: torch.Tensor) -> int:
    if t.dtype == torch.float32:
        return INF_F32
    if t.dtype == torch.bfloat16:
        return INF_BF16
    if t.dtype == torch.float64:
        return INF_F64
    if t.dtype == torch.int32:
        return INF_I32
    raise TypeError(f"unsupported dtype {t.dtype}")


def strides_of(t: torch.Tensor) -> Strides:
    """inf_strides of a 4-D [B, H, T, D] tensor view."""
    if t.dim() != 4:
        raise ValueError("expected a 4-D [B, H, T, D] tensor")
    s = t.stride()
    return Strides(s[0], s[1], s[2], s[3])


def _stream(stream) -> int:
    if stream is None:
        return torch.cuda.current_stream().cuda_stream
    return stream.cuda_stream if hasattr(stream, "cuda_stream") else int(stream)


def _check(st: int, where: str) -> None:
    if st:
        raise InfernoError(st, where)


def attn_fwd(q, k, v, causal=True, scale=None, out=None, lse=None, workspace=None, stream=None):
    """O, LSE = causal attention forward of [B,H,T,D] views (fp32 or bf16)."""
    B, H, Tq, D = q.shape
    Tk = k.shape[2]
    scale = default_scale(D) if scale is None else float(scale)
    if out is None:
        out = torch.empty((B, H, Tq, D), dtype=q.dtype, device=q.device)
    if lse is None:
        lse = torch.empty((B, H, Tq), dtype=torch.float32, device=q.device)
    # a caller-supplied workspace is passed as is (the C-ABI checks its size):
    # no sizing round trip on that path
    if workspace is None and causal:
        nbytes = workspace_bytes(OP_ATTN_FWD, B, H, Tq, Tk, D, _dt(q))
        if nbytes:
            workspace = torch.empty(nbytes, dtype=torch.uint8, device=q.device)
    ws_ptr = workspace.data_ptr() if workspace is not None else None
    ws_len = workspace.numel() * workspace.element_size() if workspace is not None else 0
    st = lib().inf_attn_fwd(
        q.data_ptr(), strides_of(q), k.data_ptr(), strides_of(k), v.data_ptr(), strides_of(v),
        out.data_ptr(), strides_of(out), lse.data_ptr(), ws_ptr, ws_len, B, H, Tq, Tk, D, scale,
        int(bool(causal)), _dt(q), _stream(stream),
    )
    _check(st, "inf_attn_fwd")
    return out, lse


def attn_bwd(q, k, v, o, dout, lse, causal=True, scale=None, dq=None, dk=None, dv=None,
             workspace=None, stream=None):
    """dQ, dK, dV of causal attention (recompute from q, k, v, o, lse)."""
    B, H, Tq, D = q.shape
    Tk = k.shape[2]
    scale = default_scale(D) if scale is None else float(scale)
    dq = torch.empty_like(q, memory_format=torch.contiguous_format) if dq is None else dq
    dk = torch.empty_like(k, memory_format=torch.contiguous_format) if dk is None else dk
    dv = torch.empty_like(v, memory_format=torch.contiguous_format) if dv is None else dv
    if workspace is None:
        nbytes = workspace_bytes(OP_ATTN_BWD, B, H, Tq, Tk, D, _dt(q))
        workspace = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=q.device)
    st = lib().inf_attn_bwd(
        q.data_ptr(), strides_of(q), k.data_ptr(), strides_of(k), v.data_ptr(), strides_of(v),
        o.data_ptr(), strides_of(o), dout.data_ptr(), strides_of(dout), lse.data_ptr(),
        dq.data_ptr(), strides_of(dq), dk.data_ptr(), strides_of(dk), dv.data_ptr(), strides_of(dv),
        workspace.data_ptr(), workspace.numel(), B, H, Tq, Tk, D, scale, int(bool(causal)), _dt(q),
        _stream(stream),
    )
    _check(st, "inf_attn_bwd")
    return dq, dk, dv


def attn_decode(q, kcache, vcache, scale=None, out=None, workspace=None, stream=None):
    """Single-query attention: q [B,H,1,D] against caches [B,H,Tk,D]."""
    B, H, _, D = q.shape
    Tk = kcache.shape[2]
    scale = default_scale(D) if scale is None else float(scale)
    if out is None:
        out = torch.empty((B, H, 1, D), dtype=q.dtype, device=q.device)
    if workspace is None:
        nbytes = workspace_bytes(OP_ATTN_DECODE, B, H, 1, Tk, D, _dt(q))
        workspace = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=q.device)
    st = lib().inf_attn_decode(
        q.data_ptr(), strides_of(q), kcache.data_ptr(), strides_of(kcache), vcache.data_ptr(),
        strides_of(vcache), out.data_ptr(), strides_of(out), B, H, Tk, D, scale, _dt(q),
        workspace.data_ptr(), workspace.numel(), _stream(stream),
    )
    _check(st, "inf_attn_decode")
    return out


def _rows(t: torch.Tensor):
    cols = t.shape[-1]
    if t.stride(-1) != 1:
        raise ValueError("last axis must have unit stride")
    t2 = t.reshape(-1, cols) if t.dim() != 2 else t
    if t2.data_ptr() != t.data_ptr():
        raise ValueError("rows must be addressable with one row stride")
    return t2, t2.shape[0], cols, t2.stride(0) if t2.shape[0] > 1 else cols


def softmax_fwd(x, out=None, stream=None):
    """Row softmax over the last axis."""
    x2, rows, cols, sx = _rows(x)
    odt = torch.float32 if x.dtype == torch.int32 else x.dtype  # Int32 input -> Float32 output
    out = torch.empty((rows, cols), dtype=odt, device=x.device) if out is None else out.reshape(rows, cols)
    st = lib().inf_softmax_fwd(x2.data_ptr(), out.data_ptr(), rows, cols, sx,
                               out.stride(0) if rows > 1 else cols, _dt(x), _stream(stream))
    _check(st, "inf_softmax_fwd")
    return out.reshape(x.shape)


def softmax_bwd(y, dy, out=None, stream=None):
    """dx = y * (dy - sum(dy * y)) per row."""
    y2, rows, cols, sy = _rows(y)
    g2, _, _, sg = _rows(dy)
    out = torch.empty_like(y2) if out is None else out.reshape(rows, cols)
    st = lib().inf_softmax_bwd(y2.data_ptr(), g2.data_ptr(), out.data_ptr(), rows, cols, sy, sg,
                               out.stride(0) if rows > 1 else cols, _dt(y), _stream(stream))
    _check(st, "inf_softmax_bwd")
    return out.reshape(y.shape)


def softmax_axis_fwd(x, axis, stream=None):
    """Softmax along `axis` of a strided view, on its own strides (no copies); the output is
    dense in x's shape (Int32 input -> Float32 output)."""
    odt = torch.float32 if x.dtype == torch.int32 else x.dtype
    out = torch.empty(x.shape, dtype=odt, device=x.device)
    st = lib().inf_softmax_fwd_axis(x.data_ptr(), _i64(x.stride()), out.data_ptr(), _i64(out.stride()), x.dim(),
                                    _i64(x.shape), int(axis), _dt(x), _stream(stream))
    _check(st, "inf_softmax_fwd_axis")
    return out


def softmax_axis_bwd(y, dy, axis, stream=None):
    """dx = y * (dy - sum(dy * y)) along `axis` of strided views; dx dense in y's shape."""
    out = torch.empty(y.shape, dtype=y.dtype, device=y.device)
    st = lib().inf_softmax_bwd_axis(y.data_ptr(), _i64(y.stride()), dy.data_ptr(), _i64(dy.stride()),
                                    out.data_ptr(), _i64(out.stride()), y.dim(), _i64(y.shape), int(axis), _dt(y),
                                    _stream(stream))
    _check(st, "inf_softmax_bwd_axis")
    return out


def _i64(vals):
    import ctypes

    return (ctypes.c_int64 * max(len(vals), 1))(*vals)


def triu(a, diagonal, stream=None):
    """Dense triu of any [..., R, C] view (any dtype; elements copied bit for bit)."""
    out = torch.empty(a.shape, dtype=a.dtype, device=a.device)
    st = lib().inf_triu(a.data_ptr(), _i64(a.stride()), out.data_ptr(), a.dim(), _i64(a.shape), int(diagonal),
                        a.element_size(), _stream(stream))
    _check(st, "inf_triu")
    return out


def masked_fill(x, mask, value, stream=None):
    """Dense out = mask != 0 ? value : x, the integer mask broadcast from the right."""
    import numpy as np

    out = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    fill = torch.tensor([value], dtype=torch.float32).to(x.dtype)  # static_cast<AT>(value)
    bits = int(np.frombuffer(fill.view(torch.uint8).numpy().tobytes() + bytes(8), dtype=np.uint64, count=1)[0])
    st = lib().inf_masked_fill(x.data_ptr(), _i64(x.stride()), mask.data_ptr(), _i64(mask.shape),
                               _i64(mask.stride()), mask.dim(), mask.element_size(), out.data_ptr(), x.dim(),
                               _i64(x.shape), bits, x.element_size(), _stream(stream))
    _check(st, "inf_masked_fill")
    return out
