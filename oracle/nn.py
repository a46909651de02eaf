"""Oracle wrappers for the model ops around the attention path (oracle_nn.c).

TEST INFRASTRUCTURE ONLY (see the package docstring): the checker for the HIP
path.  Each function returns numpy arrays computed by the restated reference
loops; the ``ref_*`` functions call the reference's own header kernels built
into ``oracle/_ref`` (None when that library is absent).
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _f32p, _i32p, _i64, lib, ref_lib

_f = ctypes.c_float
_done = set()


def _L():
    L = lib()
    if "nn" not in _done:
        L.orc_layernorm_f32.argtypes = [_f32p, _f32p, _f32p, _f32p, _f32p, _f32p, _i64, _i64, _f]
        L.orc_layernorm_bwd_f32.argtypes = [_f32p, _f32p, _f32p, _f32p, _f32p, _f32p, _f32p, _f32p, _i64, _i64]
        L.orc_gelu_f32.argtypes = [_f32p, _f32p, _i64]
        L.orc_gelu_bwd_f32.argtypes = [_f32p, _f32p, _f32p, _i64]
        L.orc_cross_entropy_f32.argtypes = [_f32p, _i32p, _f32p, _i64, _i64]
        L.orc_cross_entropy_bwd_f32.argtypes = [_f32p, _i32p, _f32p, _f32p, _i64, _i64]
        L.orc_embedding_f32.argtypes = [_i32p, _f32p, _f32p, _i64, _i64]
        L.orc_embedding_bwd_f32.argtypes = [_i32p, _f32p, _f32p, _i64, _i64, _i64]
        L.orc_adamw_f32.argtypes = [_f32p, _f32p, _f32p, _f32p, _i64, _f, _f, _f, _f, _f, _f, _f]
        L.orc_adamw_bias_correction.argtypes = [_f, _i64]
        L.orc_adamw_bias_correction.restype = _f
        L.orc_sum_rows_f32.argtypes = [_f32p, _f32p, _i64, _i64]
        _done.add("nn")
    return L


def _R():
    R = ref_lib()
    if R is not None and "ref" not in _done:
        R.ref_layernorm_f32.argtypes = [_f32p, _f32p, _f32p, _f32p, _f32p, _f32p, _i64, _i64, _f]
        R.ref_gelu_f32.argtypes = [_f32p, _f32p, _i64]
        R.ref_gelu_bwd_f32.argtypes = [_f32p, _f32p, _f32p, _i64]
        R.ref_cross_entropy_f32.argtypes = [_f32p, _i32p, _f32p, _i64, _i64]
        R.ref_embedding_f32.argtypes = [_i32p, _f32p, _f32p, _i64, _i64]
        R.ref_adamw_f32.argtypes = [_f32p, _f32p, _f32p, _f32p, _i64, _f, _f, _f, _f, _f, _f, _f]
        _done.add("ref")
    return R


def _c(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _ci(a):
    return np.ascontiguousarray(a, dtype=np.int32)


def _rows(x):
    x = _c(x)
    return x, int(np.prod(x.shape[:-1])), x.shape[-1]


# ---------------------------------------------------------------- LayerNorm --
def layernorm(x, gamma, beta, eps=1e-5, impl=None):
    """(y, mean, invstd) over the last axis."""
    x, rows, dim = _rows(x)
    y = np.empty_like(x)
    mean = np.empty(rows, np.float32)
    invstd = np.empty(rows, np.float32)
    name = "ref_layernorm_f32" if impl is not None else "orc_layernorm_f32"
    getattr(impl or _L(), name)(x.reshape(-1), _c(gamma), _c(beta), y.reshape(-1), mean, invstd, rows, dim, eps)
    return y, mean, invstd


def ref_layernorm(x, gamma, beta, eps=1e-5):
    R = _R()
    return None if R is None else layernorm(x, gamma, beta, eps, impl=R)


def layernorm_bwd(x, gout, gamma, mean, invstd):
    """(dx, dgamma, dbeta)."""
    x, rows, dim = _rows(x)
    gx = np.empty_like(x)
    gg = np.empty(dim, np.float32)
    gb = np.empty(dim, np.float32)
    _L().orc_layernorm_bwd_f32(x.reshape(-1), _c(gout).reshape(-1), _c(gamma), _c(mean), _c(invstd),
                               gx.reshape(-1), gg, gb, rows, dim)
    return gx, gg, gb


# --------------------------------------------------------------------- GELU --
def gelu(x):
    x = _c(x)
    y = np.empty_like(x)
    _L().orc_gelu_f32(x.reshape(-1), y.reshape(-1), x.size)
    return y


def gelu_bwd(x, g):
    x, g = _c(x), _c(g)
    dx = np.empty_like(x)
    _L().orc_gelu_bwd_f32(x.reshape(-1), g.reshape(-1), dx.reshape(-1), x.size)
    return dx


def ref_gelu(x):
    R = _R()
    if R is None:
        return None
    x = _c(x)
    y = np.empty_like(x)
    R.ref_gelu_f32(x.reshape(-1), y.reshape(-1), x.size)
    return y


def ref_gelu_bwd(x, g):
    R = _R()
    if R is None:
        return None
    x, g = _c(x), _c(g)
    dx = np.empty_like(x)
    R.ref_gelu_bwd_f32(x.reshape(-1), g.reshape(-1), dx.reshape(-1), x.size)
    return dx


# ------------------------------------------------------------ cross-entropy --
def cross_entropy(logits, targets, impl=None):
    logits, rows, vocab = _rows(logits)
    out = np.empty(1, np.float32)
    if impl is None:
        _L().orc_cross_entropy_f32(logits.reshape(-1), _ci(targets).reshape(-1), out, rows, vocab)
    else:
        impl.ref_cross_entropy_f32(logits.reshape(-1), _ci(targets).reshape(-1), out, rows, vocab)
    return float(out[0])


def ref_cross_entropy(logits, targets):
    R = _R()
    return None if R is None else cross_entropy(logits, targets, impl=R)


def cross_entropy_bwd(logits, targets, upstream=1.0):
    logits, rows, vocab = _rows(logits)
    g = np.empty_like(logits)
    _L().orc_cross_entropy_bwd_f32(logits.reshape(-1), _ci(targets).reshape(-1),
                                   np.array([upstream], np.float32), g.reshape(-1), rows, vocab)
    return g


# ---------------------------------------------------------------- embedding --
def embedding(ids, table, impl=None):
    ids = _ci(ids)
    table = _c(table)
    n = ids.size
    out = np.empty((n, table.shape[1]), np.float32)
    name = "ref_embedding_f32" if impl is not None else "orc_embedding_f32"
    getattr(impl or _L(), name)(ids.reshape(-1), table.reshape(-1), out.reshape(-1), n, table.shape[1])
    return out.reshape(ids.shape + (table.shape[1],))


def ref_embedding(ids, table):
    R = _R()
    return None if R is None else embedding(ids, table, impl=R)


def embedding_bwd(ids, gout, vocab):
    ids = _ci(ids)
    gout = _c(gout)
    dim = gout.shape[-1]
    dt = np.empty((vocab, dim), np.float32)
    _L().orc_embedding_bwd_f32(ids.reshape(-1), gout.reshape(-1), dt.reshape(-1), ids.size, vocab, dim)
    return dt


# -------------------------------------------------------------------- AdamW --
def bias_correction(beta, step):
    return float(_L().orc_adamw_bias_correction(beta, step))


def adamw(p, g, m, v, step, lr=3e-4, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1, impl=None):
    """Returns updated copies (p, m, v) after one step (defaults of adamw.h:15-21)."""
    p, g, m, v = _c(p).copy(), _c(g), _c(m).copy(), _c(v).copy()
    bc1, bc2 = bias_correction(beta1, step), bias_correction(beta2, step)
    name = "ref_adamw_f32" if impl is not None else "orc_adamw_f32"
    getattr(impl or _L(), name)(p.reshape(-1), g.reshape(-1), m.reshape(-1), v.reshape(-1), p.size, lr, beta1,
                                beta2, eps, weight_decay, bc1, bc2)
    return p, m, v


def ref_adamw(p, g, m, v, step, **kw):
    R = _R()
    return None if R is None else adamw(p, g, m, v, step, impl=R, **kw)


# -------------------------------------------------------------- reductions --
def sum_rows(x):
    x, rows, cols = _rows(x)
    out = np.empty(cols, np.float32)
    _L().orc_sum_rows_f32(x.reshape(-1), out, rows, cols)
    return out
