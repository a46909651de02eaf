"""Write the committed golden fixtures (small, config-1 sized) from the CPU oracle.

The oracle is first checked bit-for-bit against the reference's own compiled
kernels (oracle/_ref) where those were built, then its outputs are stored:

  config1.npz  B1 H4 T128 D32 causal, scale 1/sqrt(32): q, k, v, do (inputs,
               seed 42+{0,1,2,3}) and o, lse, dq, dk, dv (outputs)
  decode.npz   B2 H3 Tk100 D32: q, kc, vc, o
  softmax.npz  8 rows x 100 with a causal -1e9 fill: x, g, y, dx

Run from the repository root: python tests/golden/make_golden.py
"""
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
import oracle  # noqa: E402

OUT = Path(__file__).resolve().parent


def main():
    B, H, T, D = 1, 4, 128, 32
    q, k, v, do = oracle.attn_inputs(B, H, T, D, seed=42)
    o, lse, p = oracle.attn_fwd(q, k, v, want_p=True)
    dq, dk, dv, ds = oracle.attn_bwd(q, k, v, do, want_ds=True)
    R = oracle.ref_lib()
    if R is not None:
        import ctypes

        scale = float(np.float32(1) / np.sqrt(np.float32(D)))
        o_r = np.empty_like(o)
        p_r = np.empty_like(p)
        R.ref_attn_fwd_f32(q, k, v, B, H, T, D, scale, 1, o_r, p_r.ctypes.data_as(ctypes.c_void_p))
        assert np.array_equal(o.view(np.uint32), o_r.view(np.uint32))
        assert np.array_equal(p.view(np.uint32), p_r.view(np.uint32))
        dp_r, dv_r, dq_r, dk_r = (np.empty_like(p), np.empty_like(v), np.empty_like(q), np.empty_like(k))
        R.ref_attn_bwd_stages_f32(q, k, v, p_r, do, ds, B, H, T, D, scale, dp_r, dv_r, dq_r, dk_r)
        for a, b in ((dv, dv_r), (dq, dq_r), (dk, dk_r)):
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
        print("oracle == reference kernels (bitwise) on config 1")
    np.savez(OUT / "config1.npz", q=q, k=k, v=v, do=do, o=o, lse=lse, dq=dq, dk=dk, dv=dv)

    qd = oracle.randn(100, (2, 3, 1, 32))
    kc = oracle.randn(101, (2, 3, 100, 32))
    vc = oracle.randn(102, (2, 3, 100, 32))
    np.savez(OUT / "decode.npz", q=qd, kc=kc, vc=vc, o=oracle.attn_decode(qd, kc, vc))

    x = oracle.randn(300, (8, 100), 2.0)
    x[np.triu(np.ones((8, 100), bool), 1)] = np.float32(-1e9)
    g = oracle.randn(301, (8, 100))
    y = oracle.softmax(x)
    np.savez(OUT / "softmax.npz", x=x, g=g, y=y, dx=oracle.softmax_bwd(y, g))
    for f in sorted(OUT.glob("*.npz")):
        print(f.name, f.stat().st_size)


if __name__ == "__main__":
    main()
