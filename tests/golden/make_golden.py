"""Writes the known-answer vectors of the int8 linear path (tests/golden/*.npz).

The reference ships no test vectors for this path and cannot be built here
(its library needs ggml, fetched at configure time). These vectors are
therefore computed from the mathematics: every fp32 operation of the path is
evaluated on exact rationals and rounded once (tests/exact_fp32.py), following
  quantize_row      src/nexterabert.cpp:378-403
  build_i8_weight   src/nexterabert.cpp:1030-1042
  i8_kernel_*       src/nexterabert.cpp:881-964 (per-block int sums, fma chain)
No part of the oracle or of the engine is used to make them.

Run from the repository root:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent))
import exact_fp32 as X  # noqa: E402


def sx_flat(sxm: np.ndarray) -> np.ndarray:
    """[T][n_blk] -> the reference's flat [(T+3)//4][n_blk][4] layout."""
    T, nb = sxm.shape
    out = np.zeros(((T + 3) // 4) * nb * 4, np.float32)
    for t in range(T):
        for B in range(nb):
            out[((t // 4) * nb + B) * 4 + t % 4] = sxm[t, B]
    return out


def make_case(name: str, T: int, n_in: int, n_out: int, act_max: int, seed: int) -> None:
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((T, n_in)).astype(np.float32)
    wf = (0.02 * rng.standard_normal((n_out, n_in))).astype(np.float32)
    res = rng.standard_normal((T, n_out)).astype(np.float32)
    # edge rows: an all-zero activation row (amax 0 -> q = ACT_OFF, scale 0) and a
    # row whose block maximum is act_max so that inv = 1 and x*inv = k + 0.5 ties
    # exercise round-half-even.
    x[0, :] = 0.0
    if T > 1:
        x[1, :] = np.float32(0.25) * np.round(rng.standard_normal(n_in) * 8).astype(np.float32)
        x[1, ::7] = np.float32(2.5)
        x[1, 3::7] = np.float32(-3.5)
        for B in range(0, n_in, 256):
            x[1, B] = np.float32(act_max)
    # a weight row with amax 127 so that inv = 1 and lround's ties away from zero show
    wf[0, :] = np.float32(0.5) * np.round(rng.standard_normal(n_in) * 6).astype(np.float32)
    wf[0, ::5] = np.float32(2.5)
    wf[0, 1::5] = np.float32(-4.5)
    for B in range(0, n_in, 256):
        wf[0, B] = np.float32(127.0)

    nb = (n_in + 255) // 256
    act_off = act_max + 1
    # activations
    q = np.zeros((T, n_in), np.uint8)
    sxm = np.zeros((T, nb), np.float32)
    for t in range(T):
        for B in range(nb):
            i0, i1 = B * 256, min(n_in, (B + 1) * 256)
            qq, s = X.quantize_block([float(v) for v in x[t, i0:i1]], act_max)
            q[t, i0:i1] = qq
            sxm[t, B] = s
    # weights
    w8 = np.zeros((n_out, n_in), np.int8)
    sw = np.zeros((nb, n_out), np.float32)
    off = np.zeros((nb, n_out), np.int32)
    for r in range(n_out):
        for B in range(nb):
            i0, i1 = B * 256, min(n_in, (B + 1) * 256)
            qq, s, tot = X.expand_block([float(v) for v in wf[r, i0:i1]])
            w8[r, i0:i1] = qq
            sw[B, r] = s
            off[B, r] = -act_off * tot
    # outputs
    y = np.zeros((T, n_out), np.float32)
    yr = np.zeros((T, n_out), np.float32)
    sums = np.zeros((nb, T, n_out), np.int32)
    for t in range(T):
        for r in range(n_out):
            y[t, r] = X.linear_point(w8[r], sw[:, r], off[:, r], q[t], [float(v) for v in sxm[t]])
            yr[t, r] = X.linear_point(w8[r], sw[:, r], off[:, r], q[t], [float(v) for v in sxm[t]],
                                      res=float(res[t, r]))
            for B in range(nb):
                i0, i1 = B * 256, min(n_in, (B + 1) * 256)
                sums[B, t, r] = int(np.dot(w8[r, i0:i1].astype(np.int64), q[t, i0:i1].astype(np.int64))) + off[B, r]
    np.savez_compressed(HERE / f"{name}.npz", x=x, wf=wf, res=res, q=q, sx=sx_flat(sxm), w8=w8, sw=sw,
                        off=off, sums=sums, y=y, y_res=yr, act_max=np.int32(act_max))
    print(f"wrote {name}.npz: T={T} n_in={n_in} n_out={n_out} act_max={act_max}")


if __name__ == "__main__":
    make_case("linear_vnni_t6_k320_n20", 6, 320, 20, 127, seed=11)
    make_case("linear_vnni_t9_k64_n8", 9, 64, 8, 127, seed=12)
    make_case("linear_avx2_t5_k512_n12", 5, 512, 12, 63, seed=13)
