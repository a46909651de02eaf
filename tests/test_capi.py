"""The C-ABI boundary without a GPU: exports, status strings, workspace sizing and
host-side argument validation (every call here carries at least one invalid
argument, so it returns before any HIP call)."""
import ctypes
import re
from pathlib import Path

import pytest

import inferno_amd as ia
from inferno_amd import Strides

HEADER = Path(__file__).resolve().parents[1] / "include" / "inferno_hip.h"
FAKE = 0x10000  # never dereferenced: each call below fails validation first


def declared_functions():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\*?\s+\**(inf_\w+)\(", text, re.M)))


def test_library_exports_every_declared_symbol():
    names = declared_functions()
    assert len(names) >= 8
    L = ia.lib()
    for n in names:
        assert hasattr(L, n), n
    assert set(names) == set(ia.EXPORTS)


def test_version_and_status_strings():
    assert ia.lib().inf_version() >= 100
    for code in range(10):
        s = ia.status_string(code)
        assert s and s != "unknown status"
    assert ia.status_string(12345) == "unknown status"


def dense(B, H, T, D):
    return Strides(H * T * D, T * D, D, 1)


def fwd(**kw):
    a = dict(q=FAKE, sq=dense(1, 1, 8, 64), k=FAKE, sk=dense(1, 1, 8, 64), v=FAKE, sv=dense(1, 1, 8, 64),
             o=FAKE, so=dense(1, 1, 8, 64), lse=FAKE, ws=None, ws_bytes=0, B=1, H=1, Tq=8, Tk=8, D=64,
             scale=0.125, causal=1, dt=ia.INF_F32)
    a.update(kw)
    return ia.lib().inf_attn_fwd(a["q"], a["sq"], a["k"], a["sk"], a["v"], a["sv"], a["o"], a["so"], a["lse"],
                                 a["ws"], a["ws_bytes"], a["B"], a["H"], a["Tq"], a["Tk"], a["D"], a["scale"],
                                 a["causal"], a["dt"], None)


@pytest.mark.parametrize("kw,status", [
    (dict(q=None), 1),
    (dict(o=None), 1),
    (dict(D=48), 5),
    (dict(D=256), 5),
    (dict(B=0), 2),
    (dict(Tq=0), 2),
    (dict(Tq=9, Tk=8), 2),            # causal needs Tq <= Tk
    (dict(dt=7), 4),
    (dict(scale=0.0), 8),
    (dict(scale=-1.0), 8),
    (dict(scale=float("inf")), 8),
    (dict(scale=float("nan")), 8),
    (dict(sq=Strides(512, 512, 64, 2)), 3),   # head-dim stride must be 1
    (dict(sk=Strides(-1, 512, 64, 1)), 3),
    (dict(sv=Strides(512, 512, 66, 1)), 7),   # row stride not 4-element aligned
    (dict(sk=Strides(0, 0, (1 << 22) + 4, 1)), 3),  # row stride above 2^22 (32-bit tile offsets)
    (dict(so=Strides(0, 0, 1 << 23, 1)), 3),
    (dict(q=FAKE + 4), 7),                    # 16-byte alignment for fp32
])
def test_fwd_validation(kw, status):
    assert fwd(**kw) == status


def test_bf16_alignment_is_8_bytes():
    # an 8-byte aligned bf16 base passes the alignment check; fails later on D
    assert fwd(q=FAKE + 8, dt=ia.INF_BF16, D=48) == 5
    assert fwd(q=FAKE + 4, dt=ia.INF_BF16) == 7


def test_fwd_workspace():
    # one small head: nothing to balance, no workspace
    assert ia.workspace_bytes(ia.OP_ATTN_FWD, 1, 1, 8, 8, 64) == 0
    assert ia.workspace_bytes(ia.OP_ATTN_FWD, 1, 1, 8, 8, 64, ia.INF_BF16) == 0
    # a causal grid of few workgroups per CU splits its heaviest query tiles:
    # whole (tile, head) partials of 128 rows x (D + 2) floats, 256-byte rounded
    B, H, T, D = 4, 12, 1024, 64
    ws = ia.workspace_bytes(ia.OP_ATTN_FWD, B, H, T, T, D)
    assert ws > 0 and ws % 256 == 0
    per_slot = B * H * 128 * (D + 2) * 4
    assert ws >= 2 * per_slot and ws < per_slot * (T // 128) * 16
    sq = dense(B, H, T, D)
    args = dict(sq=sq, sk=sq, sv=sq, so=sq, B=B, H=H, Tq=T, Tk=T, D=D)
    assert fwd(**args) == 6                                  # workspace missing
    assert fwd(ws=FAKE, ws_bytes=ws - 256, **args) == 6      # too small
    assert fwd(ws=FAKE + 16, ws_bytes=ws, **args) == 7       # misaligned


def test_workspace_sizes():
    ws = ia.workspace_bytes(ia.OP_ATTN_BWD, 8, 12, 1024, 1024, 64)
    assert ws >= 8 * 12 * 1024 * 4 and ws % 256 == 0        # delta (+ split partials)
    wsb = ia.workspace_bytes(ia.OP_ATTN_BWD, 8, 12, 1024, 1024, 64, ia.INF_BF16)
    assert wsb >= 8 * 12 * 1024 * 4 + 8 * 12 * 1024 * 64 * 4 and wsb % 256 == 0  # + fp32 dQ accumulator
    # a causal grid far below the device's slots splits its heaviest key blocks: partials + counters
    small = ia.workspace_bytes(ia.OP_ATTN_BWD, 1, 4, 1024, 1024, 64)
    assert small > 4 * 1024 * 4 + 2 * 64 * 128 * 4 * 4
    wd = ia.workspace_bytes(ia.OP_ATTN_DECODE, 32, 12, 1, 2048, 64)
    assert wd >= 32 * 12 * 2 * 66 * 4 and wd % 256 == 0  # >= 2 splits of (o[64], m, l) per row
    assert ia.workspace_bytes(ia.OP_ATTN_DECODE, 1, 1, 1, 64, 64) == 0  # one split: no workspace
    with pytest.raises(ia.InfernoError):
        ia.workspace_bytes(ia.OP_ATTN_BWD, 1, 1, 8, 8, 40)
    with pytest.raises(ia.InfernoError):
        ia.workspace_bytes(9, 1, 1, 8, 8, 64)


def test_deterministic_switch_and_workspace():
    """inf_set_deterministic returns the previous setting; in the mode, bf16 needs no fp32 dQ
    accumulator (dq comes from the query-major pass), fp32 the same delta / split workspace."""
    L = ia.lib()
    assert not ia.deterministic()
    shapes = [(8, 12, 1024, 1024, 64), (1, 4, 1024, 1024, 64), (2, 3, 300, 300, 32), (1, 2, 500, 700, 128)]
    before = {(dt, s): ia.workspace_bytes(ia.OP_ATTN_BWD, *s, dt) for dt in (ia.INF_F32, ia.INF_BF16) for s in shapes}
    try:
        assert ia.set_deterministic(True) is False
        assert ia.deterministic() and L.inf_get_deterministic() == 1
        assert L.inf_set_deterministic(7) == 1 and L.inf_get_deterministic() == 1  # any non-zero value: on
        for (dt, s), n in before.items():
            B, H, Tq = s[0], s[1], s[2]
            det = ia.workspace_bytes(ia.OP_ATTN_BWD, *s, dt)
            acc = (B * H * Tq * s[4] * 4 + 255) // 256 * 256
            assert det == (n - acc if dt == ia.INF_BF16 else n), (dt, s, n, det)
        # validation is unchanged in the mode (no GPU call is reached)
        st = dense(1, 1, 8, 64)
        args = [FAKE, st] * 5 + [FAKE] + [FAKE, st] * 3
        assert L.inf_attn_bwd(*args, None, 0, 1, 1, 8, 8, 64, 0.125, 1, ia.INF_F32, None) == 6
        assert L.inf_attn_bwd(*args, FAKE, 1 << 20, 1, 1, 8, 8, 96, 0.125, 1, ia.INF_F32, None) == 5
    finally:
        assert ia.set_deterministic(False) is True
    assert not ia.deterministic()
    assert all(ia.workspace_bytes(ia.OP_ATTN_BWD, *s, dt) == n for (dt, s), n in before.items())


@pytest.mark.parametrize("dt,B,H,T,D,splits", [
    (ia.INF_F32, 8, 12, 1024, 64, False),    # config 2: more workgroups than resident slots
    (ia.INF_F32, 4, 12, 1024, 64, True),
    (ia.INF_F32, 1, 2, 8192, 128, True),
    (ia.INF_F32, 1, 16, 8192, 128, False),   # config 4
    (ia.INF_BF16, 8, 12, 1024, 64, False),   # config 2 bf16: measured 48% slower split
    (ia.INF_BF16, 4, 12, 1024, 64, False),   # bf16 query tiles under 2048 keys never split
    (ia.INF_BF16, 1, 12, 2048, 64, True),
    (ia.INF_BF16, 1, 2, 8192, 128, True),
    (ia.INF_BF16, 1, 16, 8192, 128, False),  # config 4 bf16
])
def test_forward_split_decisions(dt, B, H, T, D, splits):
    """The forward split plan (a non-zero forward workspace) where it was measured to pay, and
    none where it was measured to lose, on an MI355X's occupancy (the CPU build assumes it)."""
    assert (ia.workspace_bytes(ia.OP_ATTN_FWD, B, H, T, T, D, dt) > 0) == splits


def test_adamw_multi_validation():
    L = ia.lib()
    T = ia.AdamWTensor
    args = (1e-3, 0.9, 0.95, 1e-8, 0.1, 0.1, 0.05)

    def call(entries, dt=ia.INF_F32, bc=args):
        table = (T * max(len(entries), 1))(*entries)
        return L.inf_adamw_step_multi(ctypes.cast(table, ctypes.POINTER(T)), len(entries), *bc, dt, None)

    ok = T(FAKE, FAKE, FAKE, FAKE, 10)
    assert call([]) == 0                                            # nothing to do
    assert L.inf_adamw_step_multi(None, 1, *args, ia.INF_F32, None) == 1
    assert call([ok, T(FAKE, None, FAKE, FAKE, 10)]) == 1          # null gradient
    assert call([ok, T(FAKE, FAKE, FAKE, FAKE, -1)]) == 2          # negative size
    assert call([ok], dt=7) == 4
    assert call([T(FAKE + 4, FAKE, FAKE, FAKE, 10)]) == 7          # fp32 p needs 16 bytes
    assert call([T(FAKE, FAKE, FAKE + 8, FAKE, 10)]) == 7          # m needs 16 bytes
    assert call([T(FAKE, FAKE + 4, FAKE, FAKE, 10)], dt=ia.INF_BF16) == 7  # bf16 g needs 8 bytes
    assert call([ok], bc=args[:5] + (0.0, 0.05)) == 8              # bias correction must be > 0


def test_triu_masked_fill_validation():
    L = ia.lib()
    i64 = lambda *v: (ctypes.c_int64 * len(v))(*v)  # noqa: E731
    sh, st = i64(3, 4), i64(4, 1)
    assert L.inf_triu(FAKE, st, FAKE, 1, i64(4), 0, 4, None) == 2       # rank < 2
    assert L.inf_triu(FAKE, st, FAKE, 2, sh, 0, 3, None) == 4           # element size
    assert L.inf_triu(FAKE, i64(4, -1), FAKE, 2, sh, 0, 4, None) == 3   # negative stride
    assert L.inf_triu(None, st, FAKE, 2, sh, 0, 4, None) == 1
    assert L.inf_triu(None, st, None, 2, i64(0, 4), 0, 4, None) == 0     # empty: nothing to do
    ms, mst = i64(1, 4), i64(4, 1)
    args = lambda **k: dict(dict(inp=FAKE, ist=st, mask=FAKE, msh=ms, mst=mst, mrank=2, mbytes=4, out=FAKE,  # noqa
                                 rank=2, shape=sh, fill=0, eb=4), **k)
    call = lambda a: L.inf_masked_fill(a["inp"], a["ist"], a["mask"], a["msh"], a["mst"], a["mrank"],  # noqa
                                       a["mbytes"], a["out"], a["rank"], a["shape"], a["fill"], a["eb"], None)
    assert call(args(msh=i64(2, 4))) == 2            # mask dim 2 vs input 3: does not broadcast
    assert call(args(mrank=3, msh=i64(1, 1, 4), mst=i64(4, 4, 1))) == 2  # mask rank > input rank
    assert call(args(mbytes=2)) == 4                 # mask element size
    assert call(args(eb=5)) == 4
    assert call(args(mst=i64(4, -1))) == 3
    assert call(args(mask=None)) == 1
    assert call(args(shape=i64(3, 0), msh=i64(1, 0))) == 0  # empty


def test_bwd_validation():
    L = ia.lib()
    s = dense(1, 1, 8, 64)
    args = [FAKE, s] * 5 + [FAKE] + [FAKE, s] * 3
    # no workspace -> INF_ERR_WORKSPACE
    assert L.inf_attn_bwd(*args, None, 0, 1, 1, 8, 8, 64, 0.125, 1, ia.INF_F32, None) == 6
    # too small
    assert L.inf_attn_bwd(*args, FAKE, 16, 1, 1, 8, 8, 64, 0.125, 1, ia.INF_F32, None) == 6
    # null lse
    a2 = list(args)
    a2[10] = None
    assert L.inf_attn_bwd(*a2, FAKE, 1 << 20, 1, 1, 8, 8, 64, 0.125, 1, ia.INF_F32, None) == 1
    # misaligned workspace
    assert L.inf_attn_bwd(*args, FAKE + 16, 1 << 20, 1, 1, 8, 8, 64, 0.125, 1, ia.INF_F32, None) == 7
    # bad head dim
    assert L.inf_attn_bwd(*args, FAKE, 1 << 20, 1, 1, 8, 8, 96, 0.125, 1, ia.INF_F32, None) == 5


@pytest.mark.parametrize("which", ["dq", "dk", "dv"])
@pytest.mark.parametrize("st,B,H,T,ok", [
    (Strides(2 * 8 * 64, 8 * 64, 64, 1), 2, 2, 8, True),     # dense [B, H, T, D]
    (Strides(8 * 2 * 3 * 64, 64, 2 * 3 * 64, 1), 2, 2, 8, True),  # a [B, T, 3, H, D] gradient buffer
    (Strides(2 * 8 * 64, 8 * 64, 0, 1), 2, 2, 8, False),     # every row of a head on one address
    (Strides(2 * 8 * 64, 0, 64, 1), 2, 2, 8, False),         # both heads on one buffer
    (Strides(0, 8 * 64, 64, 1), 2, 2, 8, False),             # both batches on one buffer
    (Strides(2 * 8 * 64, 8 * 64, 32, 1), 2, 2, 8, False),    # rows overlap by half a row
    (Strides(2 * 8 * 64, 4 * 64, 64, 1), 2, 2, 8, False),    # heads overlap
    (Strides(0, 0, 0, 1), 1, 1, 1, True),                     # one row: strides never used
    (Strides(64, 0, 0, 1), 2, 1, 1, True),                    # B x 1 x 1 rows 64 apart
])
def test_bwd_rejects_overlapping_outputs(which, st, B, H, T, ok):
    """Output views (dq, dk, dv) that map two elements onto one address are rejected before
    launch; overlap-free ones pass the view checks (and fail on the missing workspace)."""
    L = ia.lib()
    s = dense(B, H, T, 64)
    views = {"dq": s, "dk": s, "dv": s}
    views[which] = st
    args = [FAKE, s] * 5 + [FAKE] + [FAKE, views["dq"], FAKE, views["dk"], FAKE, views["dv"]]
    r = L.inf_attn_bwd(*args, None, 0, B, H, T, T, 64, 0.125, 1, ia.INF_F32, None)
    assert r == (6 if ok else 3)


def test_fwd_and_decode_reject_overlapping_outputs():
    assert fwd(so=Strides(8 * 64, 8 * 64, 0, 1)) == 3
    assert fwd(so=Strides(8 * 64, 0, 64, 1), H=2) == 3
    L = ia.lib()
    s, kv = dense(2, 2, 1, 64), dense(2, 2, 100, 64)
    # [B, H, 1, D] outputs: the head stride must keep heads apart
    assert L.inf_attn_decode(FAKE, s, FAKE, kv, FAKE, kv, FAKE, Strides(128, 0, 64, 1), 2, 2, 100, 64, 0.125,
                             ia.INF_F32, None, 0, None) == 3
    assert L.inf_attn_decode(FAKE, s, FAKE, kv, FAKE, kv, FAKE, Strides(128, 64, 0, 1), 2, 2, 100, 64, 0.125,
                             ia.INF_F32, None, 0, None) == 6


def test_static_decode_validation():
    """inf_attn_decode_static validates like inf_attn_decode and rejects, before any HIP call,
    a shape whose split partials exceed its 4 MiB static scratch."""
    L = ia.lib()
    s, kv = dense(2, 2, 1, 64), dense(2, 2, 100, 64)
    assert L.inf_attn_decode_static(None, s, FAKE, kv, FAKE, kv, FAKE, s, 2, 2, 100, 64, 0.125, ia.INF_F32, None) == 1
    assert L.inf_attn_decode_static(FAKE, s, FAKE, kv, FAKE, kv, FAKE, s, 2, 2, 100, 48, 0.125, ia.INF_F32, None) == 5
    assert L.inf_attn_decode_static(FAKE, s, FAKE, kv, FAKE, kv, FAKE, Strides(128, 0, 64, 1), 2, 2, 100, 64, 0.125,
                                    ia.INF_F32, None) == 3
    # B*H = 4095 rows of D = 128 take 2 splits: 4095 * 2 * 130 * 4 bytes > 4 MiB
    B, H, Tk, D = 1, 4095, 64, 128
    assert ia.workspace_bytes(ia.OP_ATTN_DECODE, B, H, 1, Tk, D) > 4 << 20
    sq, skv = dense(B, H, 1, D), dense(B, H, Tk, D)
    assert L.inf_attn_decode_static(FAKE, sq, FAKE, skv, FAKE, skv, FAKE, sq, B, H, Tk, D, 0.125, ia.INF_F32,
                                    None) == 6
    assert b"static scratch" in L.inf_last_error_detail()
    # 4032 rows: 4032 * 2 * 130 * 4 bytes fit; 4033 rows (8066 partial rows of 130 floats) do not
    assert ia.workspace_bytes(ia.OP_ATTN_DECODE, 1, 4032, 1, Tk, D) <= 4 << 20
    assert ia.workspace_bytes(ia.OP_ATTN_DECODE, 1, 4033, 1, Tk, D) > 4 << 20
    sq, skv = dense(1, 4033, 1, D), dense(1, 4033, Tk, D)
    assert L.inf_attn_decode_static(FAKE, sq, FAKE, skv, FAKE, skv, FAKE, sq, 1, 4033, Tk, D, 0.125, ia.INF_F32,
                                    None) == 6


def test_add_layernorm_validation():
    """inf_add_layernorm_fwd checks its arguments on the host before any HIP call."""
    L = ia.lib()
    F = FAKE
    ok = (F, 64, F, 64, F, 64, F, 64, F, F, None, None, 4, 64, 1e-5, ia.INF_F32, None)
    assert L.inf_add_layernorm_fwd(*ok[:12], 0, *ok[13:]) == 0  # no rows: nothing to do
    args = list(ok); args[2] = None
    assert L.inf_add_layernorm_fwd(*args) == 1  # r missing
    args = list(ok); args[4] = None
    assert L.inf_add_layernorm_fwd(*args) == 1  # h missing
    args = list(ok); args[5] = 32
    assert L.inf_add_layernorm_fwd(*args) == 3  # h rows shorter than dim
    args = list(ok); args[15] = 7
    assert L.inf_add_layernorm_fwd(*args) == 4  # dtype


def test_decode_and_softmax_validation():
    L = ia.lib()
    s = dense(2, 2, 1, 64)
    kv = dense(2, 2, 100, 64)
    assert L.inf_attn_decode(FAKE, s, FAKE, kv, FAKE, kv, FAKE, s, 2, 2, 100, 64, 0.125, ia.INF_F32,
                             None, 0, None) == 6
    assert L.inf_attn_decode(FAKE, s, FAKE, kv, FAKE, kv, FAKE, s, 2, 2, 0, 64, 0.125, ia.INF_F32,
                             FAKE, 1 << 20, None) == 2
    assert L.inf_softmax_fwd(None, FAKE, 4, 4, 4, 4, ia.INF_F32, None) == 1
    assert L.inf_softmax_fwd(FAKE, FAKE, 0, 4, 4, 4, ia.INF_F32, None) == 2
    assert L.inf_softmax_fwd(FAKE, FAKE, 4, 8, 4, 8, ia.INF_F32, None) == 3  # row stride < cols
    assert L.inf_softmax_bwd(FAKE, FAKE, FAKE, 4, 4, 4, 4, 4, 3, None) == 4


def test_softmax_axis_validation():
    """inf_softmax_{fwd,bwd}_axis reject bad ranks, axes, shapes, strides, dtypes and null
    pointers on the host (no device needed); empty views succeed without launching."""
    L = ia.lib()
    I64 = ctypes.c_int64 * 8

    def a(*v):
        return I64(*v)

    shape, st = a(4, 5, 6), a(30, 6, 1)
    assert L.inf_softmax_fwd_axis(FAKE, st, FAKE, st, 0, shape, 0, ia.INF_F32, None) == 2      # rank 0
    assert L.inf_softmax_fwd_axis(FAKE, st, FAKE, st, 9, shape, 0, ia.INF_F32, None) == 5      # rank > 8
    assert L.inf_softmax_fwd_axis(FAKE, st, FAKE, st, 3, shape, 3, ia.INF_F32, None) == 2      # axis
    assert L.inf_softmax_fwd_axis(FAKE, st, FAKE, st, 3, shape, -4, ia.INF_F32, None) == 2
    assert L.inf_softmax_fwd_axis(FAKE, st, FAKE, st, 3, a(4, -1, 6), 1, ia.INF_F32, None) == 2
    assert L.inf_softmax_fwd_axis(FAKE, a(30, -6, 1), FAKE, st, 3, shape, 1, ia.INF_F32, None) == 3
    assert L.inf_softmax_fwd_axis(FAKE, st, FAKE, a(30, 6, 0), 3, shape, 1, ia.INF_F32, None) == 3  # y overlaps
    assert L.inf_softmax_fwd_axis(FAKE, st, FAKE, a(6, 1, 1), 3, shape, 0, ia.INF_F32, None) == 3
    assert L.inf_softmax_fwd_axis(None, st, FAKE, st, 3, shape, 1, ia.INF_F32, None) == 1
    assert L.inf_softmax_fwd_axis(FAKE, None, FAKE, st, 3, shape, 1, ia.INF_F32, None) == 1
    assert L.inf_softmax_fwd_axis(FAKE, st, FAKE, st, 3, shape, 1, 7, None) == 4
    assert L.inf_softmax_fwd_axis(None, st, None, st, 3, a(4, 0, 6), 1, ia.INF_F32, None) == 0  # empty
    assert L.inf_softmax_bwd_axis(FAKE, st, FAKE, st, FAKE, st, 3, shape, 1, ia.INF_I32, None) == 4
    assert L.inf_softmax_bwd_axis(FAKE, st, FAKE, None, FAKE, st, 3, shape, 1, ia.INF_F32, None) == 1
    assert L.inf_softmax_bwd_axis(FAKE, st, None, st, FAKE, st, 3, shape, 1, ia.INF_F32, None) == 1
    assert L.inf_softmax_bwd_axis(FAKE, st, FAKE, st, FAKE, a(30, 0, 1), 3, shape, 1, ia.INF_F32, None) == 3


def test_product_does_not_reference_oracle():
    """The product (package + C sources) never loads the CPU oracle: there is no fallback."""
    pkg = Path(ia.__file__).parent
    files = list(pkg.glob("*.py")) + list((pkg / "csrc").glob("*"))
    for f in files:
        text = f.read_text()
        assert "import oracle" not in text and "from oracle" not in text, f
        assert "liboracle" not in text and "orc_" not in text, f
