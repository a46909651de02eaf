"""inferno_amd -- MI355X-native causal self-attention for Inferno.

``libinferno_hip.so`` (built in-tree by ``inferno_amd.build``) is the product:
the C-ABI launch layer declared in ``include/inferno_hip.h`` and its gfx950
kernels.  This module binds that ABI with ctypes and offers thin helpers that
take torch tensors as device-memory handles (torch is plumbing here: storage
and streams).  There is no fallback: if the library is missing, every call
raises.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

PKG = Path(__file__).resolve().parent
LIB_PATH = PKG / "libinferno_hip.so"

INF_F32 = 0
INF_BF16 = 1
INF_F64 = 2  # softmax entry points only
INF_I32 = 3  # softmax forward input only (fp32 output)
OP_ATTN_FWD, OP_ATTN_BWD, OP_ATTN_DECODE = 0, 1, 2

STATUS = {
    0: "INF_OK",
    1: "INF_ERR_NULL_POINTER",
    2: "INF_ERR_BAD_SHAPE",
    3: "INF_ERR_BAD_STRIDE",
    4: "INF_ERR_BAD_DTYPE",
    5: "INF_ERR_UNSUPPORTED",
    6: "INF_ERR_WORKSPACE",
    7: "INF_ERR_ALIGNMENT",
    8: "INF_ERR_BAD_SCALE",
    9: "INF_ERR_HIP",
}

# Every symbol include/inferno_hip.h declares.
EXPORTS = (
    "inf_status_string",
    "inf_version",
    "inf_attn_workspace_bytes",
    "inf_attn_fwd",
    "inf_attn_bwd",
    "inf_softmax_fwd",
    "inf_softmax_bwd",
    "inf_softmax_fwd_axis",
    "inf_softmax_bwd_axis",
    "inf_attn_decode",
    "inf_fill",
    "inf_binary",
    "inf_copy_strided",
    "inf_triu",
    "inf_masked_fill",
    "inf_nn_workspace_bytes",
    "inf_gemm",
    "inf_layernorm_fwd",
    "inf_add_layernorm_fwd",
    "inf_layernorm_bwd",
    "inf_gelu_fwd",
    "inf_gelu_bwd",
    "inf_cross_entropy_fwd",
    "inf_cross_entropy_bwd",
    "inf_embedding_fwd",
    "inf_embedding_bwd",
    "inf_adamw_step",
    "inf_adamw_step_multi",
    "inf_col_sum",
    "inf_binary_bcast",
    "inf_argmax_rows",
    "inf_attn_decode_static",
    "inf_set_deterministic",
    "inf_get_deterministic",
    "inf_last_error_detail",
)


class Strides(ctypes.Structure):
    """inf_strides: element strides of a [B, H, T, D] view."""

    _fields_ = [("b", ctypes.c_int64), ("h", ctypes.c_int64), ("t", ctypes.c_int64), ("d", ctypes.c_int64)]


class AdamWTensor(ctypes.Structure):
    """inf_adamw_tensor: one parameter tensor of a multi-tensor AdamW step."""

    _fields_ = [("p", ctypes.c_void_p), ("g", ctypes.c_void_p), ("m", ctypes.c_void_p), ("v", ctypes.c_void_p),
                ("n", ctypes.c_int64)]


class InfernoError(RuntimeError):
    def __init__(self, status: int, where: str):
        self.status = status
        super().__init__(f"{where}: {STATUS.get(status, status)} ({status_string(status)})")


_lib = None


def lib() -> ctypes.CDLL:
    """Load libinferno_hip.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -m inferno_amd.build` "
                "(there is no CPU fallback)"
            )
        L = ctypes.CDLL(str(LIB_PATH))
        vp, i32, i64, f32 = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_float
        S = Strides
        L.inf_status_string.argtypes = [i32]
        L.inf_status_string.restype = ctypes.c_char_p
        L.inf_version.argtypes = []
        L.inf_version.restype = i32
        L.inf_attn_workspace_bytes.argtypes = [i32, i32, i32, i32, i32, i32, i32, ctypes.POINTER(ctypes.c_size_t)]
        L.inf_attn_workspace_bytes.restype = i32
        L.inf_attn_fwd.argtypes = [vp, S, vp, S, vp, S, vp, S, vp, vp, ctypes.c_size_t, i32, i32, i32, i32, i32, f32, i32, i32, vp]
        L.inf_attn_fwd.restype = i32
        L.inf_attn_bwd.argtypes = [vp, S, vp, S, vp, S, vp, S, vp, S, vp, vp, S, vp, S, vp, S, vp,
                                   ctypes.c_size_t, i32, i32, i32, i32, i32, f32, i32, i32, vp]
        L.inf_attn_bwd.restype = i32
        L.inf_softmax_fwd.argtypes = [vp, vp, i64, i64, i64, i64, i32, vp]
        L.inf_softmax_fwd.restype = i32
        L.inf_softmax_bwd.argtypes = [vp, vp, vp, i64, i64, i64, i64, i64, i32, vp]
        L.inf_softmax_bwd.restype = i32
        i64p = ctypes.POINTER(ctypes.c_int64)
        L.inf_softmax_fwd_axis.argtypes = [vp, i64p, vp, i64p, i32, i64p, i32, i32, vp]
        L.inf_softmax_fwd_axis.restype = i32
        L.inf_softmax_bwd_axis.argtypes = [vp, i64p, vp, i64p, vp, i64p, i32, i64p, i32, i32, vp]
        L.inf_softmax_bwd_axis.restype = i32
        L.inf_attn_decode.argtypes = [vp, S, vp, S, vp, S, vp, S, i32, i32, i32, i32, f32, i32, vp,
                                      ctypes.c_size_t, vp]
        L.inf_attn_decode.restype = i32
        L.inf_fill.argtypes = [vp, i64, i32, ctypes.c_uint32, vp]
        L.inf_fill.restype = i32
        L.inf_binary.argtypes = [i32, vp, vp, vp, i64, i32, i32, i32, vp]
        L.inf_binary.restype = i32
        i64p = ctypes.POINTER(ctypes.c_int64)
        L.inf_copy_strided.argtypes = [vp, i64p, vp, i64p, i32, i64p, i32, vp]
        L.inf_copy_strided.restype = i32
        L.inf_triu.argtypes = [vp, i64p, vp, i32, i64p, i32, i32, vp]
        L.inf_triu.restype = i32
        L.inf_masked_fill.argtypes = [vp, i64p, vp, i64p, i64p, i32, i32, vp, i32, i64p, ctypes.c_uint64, i32, vp]
        L.inf_masked_fill.restype = i32
        sz = ctypes.c_size_t
        L.inf_nn_workspace_bytes.argtypes = [i32, i64, i64, ctypes.POINTER(sz)]
        L.inf_gemm.argtypes = [i32, i32, i64, i64, i64, f32, vp, i64, i64, vp, i64, i64, f32, vp, i64, i64, i64,
                               vp, i32, vp, sz, vp]
        L.inf_layernorm_fwd.argtypes = [vp, i64, vp, i64, vp, vp, vp, vp, i64, i64, f32, i32, vp]
        L.inf_add_layernorm_fwd.argtypes = [vp, i64, vp, i64, vp, i64, vp, i64, vp, vp, vp, vp, i64, i64, f32, i32, vp]
        L.inf_layernorm_bwd.argtypes = [vp, i64, vp, i64, vp, vp, vp, vp, i64, vp, vp, i32, i64, i64, i32, vp, sz,
                                        vp]
        L.inf_gelu_fwd.argtypes = [vp, vp, i64, i32, vp]
        L.inf_gelu_bwd.argtypes = [vp, vp, vp, i64, i32, vp]
        L.inf_cross_entropy_fwd.argtypes = [vp, i64, vp, vp, vp, i64, i64, i32, vp, sz, vp]
        L.inf_cross_entropy_bwd.argtypes = [vp, i64, vp, vp, vp, vp, i64, i64, i64, i32, vp]
        L.inf_embedding_fwd.argtypes = [vp, i64, vp, i64, i64, vp, i32, vp]
        L.inf_embedding_bwd.argtypes = [vp, i64, vp, i64, i64, vp, i32, vp]
        L.inf_adamw_step.argtypes = [vp, vp, vp, vp, i64, f32, f32, f32, f32, f32, f32, f32, i32, vp]
        L.inf_adamw_step_multi.argtypes = [ctypes.POINTER(AdamWTensor), i32, f32, f32, f32, f32, f32, f32, f32, i32,
                                           vp]
        L.inf_col_sum.argtypes = [vp, i64, i64, i64, vp, i32, i32, vp, sz, vp]
        L.inf_binary_bcast.argtypes = [i32, vp, vp, vp, i64, i64, i32, vp]
        L.inf_argmax_rows.argtypes = [vp, i64, i64, i64, vp, i32, vp]
        L.inf_attn_decode_static.argtypes = [vp, S, vp, S, vp, S, vp, S, i32, i32, i32, i32, f32, i32, vp]
        L.inf_set_deterministic.argtypes = [i32]
        L.inf_get_deterministic.argtypes = []
        for name in EXPORTS[11:-1]:
            getattr(L, name).restype = i32
        L.inf_last_error_detail.argtypes = []
        L.inf_last_error_detail.restype = ctypes.c_char_p
        _lib = L
    return _lib


def status_string(status: int) -> str:
    return lib().inf_status_string(int(status)).decode()


def workspace_bytes(op: int, B: int, H: int, Tq: int, Tk: int, D: int, dtype: int = INF_F32) -> int:
    out = ctypes.c_size_t(0)
    st = lib().inf_attn_workspace_bytes(op, B, H, Tq, Tk, D, dtype, ctypes.byref(out))
    if st:
        raise InfernoError(st, "inf_attn_workspace_bytes")
    return int(out.value)


OP_GEMM, OP_LAYERNORM_BWD, OP_COL_SUM, OP_CROSS_ENTROPY = 3, 4, 5, 6


def nn_workspace_bytes(op: int, rows: int = 0, cols: int = 0) -> int:
    out = ctypes.c_size_t(0)
    st = lib().inf_nn_workspace_bytes(op, rows, cols, ctypes.byref(out))
    if st:
        raise InfernoError(st, "inf_nn_workspace_bytes")
    return int(out.value)


def set_deterministic(enable: bool) -> bool:
    """Process-wide switch (inf_set_deterministic): every later attention backward takes dQ
    from the query-major pass and every embedding backward sums its rows in token order, bitwise
    the same on every run.  Returns the previous setting."""
    return bool(lib().inf_set_deterministic(1 if enable else 0))


def deterministic() -> bool:
    """Whether the attention backward runs in the deterministic-dQ mode."""
    return bool(lib().inf_get_deterministic())


def default_scale(D: int) -> float:
    """1.0f / std::sqrt((float)D), as InfernoApp/main.cpp:743 computes it (fp32)."""
    import numpy as np

    return float(np.float32(1.0) / np.sqrt(np.float32(D)))


from .ops import (  # noqa: E402  (torch-facing helpers need lib())
    attn_bwd,
    attn_decode,
    attn_fwd,
    masked_fill,
    softmax_axis_bwd,
    softmax_axis_fwd,
    softmax_bwd,
    softmax_fwd,
    strides_of,
    triu,
)
from .nn import (  # noqa: E402
    add_layernorm_fwd,
    adamw_step,
    adamw_step_multi,
    argmax_rows,
    col_sum,
    cross_entropy_bwd,
    cross_entropy_fwd,
    embedding_bwd,
    embedding_fwd,
    gelu_bwd,
    gelu_fwd,
    gemm,
    layernorm_bwd,
    layernorm_fwd,
    binary_bcast,
)

__all__ = [
    "lib",
    "attn_fwd",
    "attn_bwd",
    "attn_decode",
    "softmax_fwd",
    "softmax_bwd",
    "softmax_axis_fwd",
    "softmax_axis_bwd",
    "strides_of",
    "workspace_bytes",
    "set_deterministic",
    "deterministic",
    "default_scale",
    "InfernoError",
    "EXPORTS",
]
