"""Torch-facing helpers over the model-op C-ABI (GEMM, LayerNorm, GELU,
cross-entropy, embedding, AdamW, column sums, broadcast add / multiply).

As in ``ops``: the C-ABI validates on the host and a non-zero status raises
InfernoError; tensors live on the GPU and launches go to torch's current
stream (or ``stream``).  Used by the GPU parity tests; the C++ layer
(libinferno.so) calls the same entry points directly.
"""
from __future__ import annotations

import torch

from . import (INF_F32, OP_COL_SUM, OP_CROSS_ENTROPY, OP_GEMM, OP_LAYERNORM_BWD, lib, nn_workspace_bytes)
from .ops import _check, _dt, _stream


def _ws(nbytes: int, device) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)


def _ld(t: torch.Tensor) -> int:
    """Row stride of a 2-D row-major view (unit column stride)."""
    if t.dim() != 2 or (t.shape[1] > 1 and t.stride(1) != 1):
        raise ValueError("expected a 2-D view with unit column stride")
    return t.stride(0) if t.shape[0] > 1 else max(t.shape[1], 1)


def gemm(a, b, trans_a=False, trans_b=False, bias=None, alpha=1.0, beta=0.0, out=None, workspace=None,
         stream=None):
    """Row-major out = alpha * op(a) @ op(b) + beta * out (+ bias per row), 2-D operands."""
    M = a.shape[1] if trans_a else a.shape[0]
    K = a.shape[0] if trans_a else a.shape[1]
    N = b.shape[0] if trans_b else b.shape[1]
    if out is None:
        out = torch.zeros((M, N), dtype=a.dtype, device=a.device)
    if workspace is None:
        workspace = _ws(nn_workspace_bytes(OP_GEMM), a.device)
    st = lib().inf_gemm(int(trans_a), int(trans_b), M, N, K, float(alpha), a.data_ptr(), _ld(a), 0, b.data_ptr(),
                        _ld(b), 0, float(beta), out.data_ptr(), _ld(out), 0, 1,
                        bias.data_ptr() if bias is not None else None, _dt(a), workspace.data_ptr(),
                        workspace.numel(), _stream(stream))
    _check(st, "inf_gemm")
    return out


def layernorm_fwd(x, gamma, beta, eps=1e-5, stream=None):
    """y, mean, invstd of LayerNorm over the last axis of a 2-D view."""
    rows, dim = x.shape
    y = torch.empty((rows, dim), dtype=x.dtype, device=x.device)
    mean = torch.empty(rows, dtype=torch.float32, device=x.device)
    invstd = torch.empty(rows, dtype=torch.float32, device=x.device)
    st = lib().inf_layernorm_fwd(x.data_ptr(), _ld(x), y.data_ptr(), _ld(y), gamma.data_ptr(), beta.data_ptr(),
                                 mean.data_ptr(), invstd.data_ptr(), rows, dim, float(eps), _dt(x), _stream(stream))
    _check(st, "inf_layernorm_fwd")
    return y, mean, invstd


def add_layernorm_fwd(x, r, gamma, beta, eps=1e-5, h=None, stream=None):
    """h = x + r and y = LayerNorm(h) in one pass (inf_add_layernorm_fwd); h may be x or r."""
    rows, dim = x.shape
    h = torch.empty((rows, dim), dtype=x.dtype, device=x.device) if h is None else h
    y = torch.empty((rows, dim), dtype=x.dtype, device=x.device)
    st = lib().inf_add_layernorm_fwd(x.data_ptr(), _ld(x), r.data_ptr(), _ld(r), h.data_ptr(), _ld(h), y.data_ptr(),
                                     _ld(y), gamma.data_ptr(), beta.data_ptr(), None, None, rows, dim, float(eps),
                                     _dt(x), _stream(stream))
    _check(st, "inf_add_layernorm_fwd")
    return h, y


def layernorm_bwd(x, dy, gamma, mean, invstd, stream=None):
    """dx, dgamma, dbeta of LayerNorm from the saved statistics."""
    rows, dim = x.shape
    dx = torch.empty_like(x)
    dgamma = torch.empty(dim, dtype=torch.float32, device=x.device)
    dbeta = torch.empty(dim, dtype=torch.float32, device=x.device)
    ws = _ws(nn_workspace_bytes(OP_LAYERNORM_BWD, rows, dim), x.device)
    st = lib().inf_layernorm_bwd(x.data_ptr(), _ld(x), dy.data_ptr(), _ld(dy), gamma.data_ptr(), mean.data_ptr(),
                                 invstd.data_ptr(), dx.data_ptr(), _ld(dx), dgamma.data_ptr(), dbeta.data_ptr(), 0,
                                 rows, dim, _dt(x), ws.data_ptr(), ws.numel(), _stream(stream))
    _check(st, "inf_layernorm_bwd")
    return dx, dgamma, dbeta


def gelu_fwd(x, stream=None):
    y = torch.empty_like(x)
    _check(lib().inf_gelu_fwd(x.data_ptr(), y.data_ptr(), x.numel(), _dt(x), _stream(stream)), "inf_gelu_fwd")
    return y


def gelu_bwd(x, dy, stream=None):
    dx = torch.empty_like(x)
    _check(lib().inf_gelu_bwd(x.data_ptr(), dy.data_ptr(), dx.data_ptr(), x.numel(), _dt(x), _stream(stream)),
           "inf_gelu_bwd")
    return dx


def cross_entropy_fwd(logits, targets, stream=None):
    """(mean loss [1], per-row lse [rows]) of logits [rows, vocab] and int32 targets."""
    rows, vocab = logits.shape
    loss = torch.empty(1, dtype=torch.float32, device=logits.device)
    lse = torch.empty(rows, dtype=torch.float32, device=logits.device)
    ws = _ws(nn_workspace_bytes(OP_CROSS_ENTROPY, rows, vocab), logits.device)
    st = lib().inf_cross_entropy_fwd(logits.data_ptr(), _ld(logits), targets.data_ptr(), loss.data_ptr(),
                                     lse.data_ptr(), rows, vocab, _dt(logits), ws.data_ptr(), ws.numel(),
                                     _stream(stream))
    _check(st, "inf_cross_entropy_fwd")
    return loss, lse


def cross_entropy_bwd(logits, targets, lse, upstream, stream=None):
    rows, vocab = logits.shape
    g = torch.empty_like(logits)
    st = lib().inf_cross_entropy_bwd(logits.data_ptr(), _ld(logits), targets.data_ptr(), lse.data_ptr(),
                                     upstream.data_ptr(), g.data_ptr(), _ld(g), rows, vocab, _dt(logits),
                                     _stream(stream))
    _check(st, "inf_cross_entropy_bwd")
    return g


def embedding_fwd(ids, table, stream=None):
    n = ids.numel()
    vocab, dim = table.shape
    out = torch.empty((n, dim), dtype=table.dtype, device=table.device)
    st = lib().inf_embedding_fwd(ids.data_ptr(), n, table.data_ptr(), vocab, dim, out.data_ptr(), _dt(table),
                                 _stream(stream))
    _check(st, "inf_embedding_fwd")
    return out


def embedding_bwd(ids, dout, vocab, stream=None):
    n, dim = dout.shape
    dtable = torch.empty((vocab, dim), dtype=torch.float32, device=dout.device)
    st = lib().inf_embedding_bwd(ids.data_ptr(), n, dout.data_ptr(), vocab, dim, dtable.data_ptr(), 1,
                                 _stream(stream))
    _check(st, "inf_embedding_bwd")
    return dtable


def adamw_step(p, g, m, v, step, lr=3e-4, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1, stream=None):
    """In-place AdamW update; bias corrections as the reference computes them (fp32 pow)."""
    import numpy as np

    bc1 = float(np.float32(1.0) - np.power(np.float32(beta1), np.float32(step)))
    bc2 = float(np.float32(1.0) - np.power(np.float32(beta2), np.float32(step)))
    st = lib().inf_adamw_step(p.data_ptr(), g.data_ptr(), m.data_ptr(), v.data_ptr(), p.numel(), float(lr),
                              float(beta1), float(beta2), float(eps), float(weight_decay), bc1, bc2, _dt(p),
                              _stream(stream))
    _check(st, "inf_adamw_step")


def adamw_step_multi(params, step, lr=3e-4, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1, stream=None):
    """In-place AdamW update of a list of (p, g, m, v) tensors through one multi-tensor call."""
    import ctypes

    import numpy as np

    from . import AdamWTensor

    bc1 = float(np.float32(1.0) - np.power(np.float32(beta1), np.float32(step)))
    bc2 = float(np.float32(1.0) - np.power(np.float32(beta2), np.float32(step)))
    dts = {_dt(p) for p, _, _, _ in params}
    if len(dts) > 1:
        raise ValueError("adamw_step_multi: all parameters must share one dtype")
    table = (AdamWTensor * max(len(params), 1))()
    for i, (p, g, m, v) in enumerate(params):
        table[i] = AdamWTensor(p.data_ptr(), g.data_ptr(), m.data_ptr(), v.data_ptr(), p.numel())
    dt = dts.pop() if dts else 0
    st = lib().inf_adamw_step_multi(ctypes.cast(table, ctypes.POINTER(AdamWTensor)), len(params), float(lr),
                                    float(beta1), float(beta2), float(eps), float(weight_decay), bc1, bc2, dt,
                                    _stream(stream))
    _check(st, "inf_adamw_step_multi")


def col_sum(x, out=None, accumulate=False, stream=None):
    rows, cols = x.shape
    out = torch.empty(cols, dtype=torch.float32, device=x.device) if out is None else out
    ws = _ws(nn_workspace_bytes(OP_COL_SUM, rows, cols), x.device)
    st = lib().inf_col_sum(x.data_ptr(), rows, cols, _ld(x), out.data_ptr(), int(accumulate), _dt(x),
                           ws.data_ptr(), ws.numel(), _stream(stream))
    _check(st, "inf_col_sum")
    return out


def binary_bcast(op, a, b, stream=None):
    out = torch.empty_like(a)
    st = lib().inf_binary_bcast(int(op), a.data_ptr(), b.data_ptr(), out.data_ptr(), a.numel(), b.numel(), _dt(a),
                                _stream(stream))
    _check(st, "inf_binary_bcast")
    return out


__all__ = ["gemm", "layernorm_fwd", "layernorm_bwd", "gelu_fwd", "gelu_bwd", "cross_entropy_fwd",
           "cross_entropy_bwd", "embedding_fwd", "embedding_bwd", "adamw_step", "col_sum", "binary_bcast",
           "INF_F32"]


def argmax_rows(x, stream=None):
    """Int32 index of each row's largest element (first on ties) of a [rows, cols] tensor."""
    rows, cols = x.shape
    out = torch.empty(rows, dtype=torch.int32, device=x.device)
    st = lib().inf_argmax_rows(x.data_ptr(), rows, cols, x.stride(0), out.data_ptr(), _dt(x), _stream(stream))
    _check(st, "inf_argmax_rows")
    return out
