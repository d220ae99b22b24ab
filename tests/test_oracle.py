"""Pins the CPU oracle (oracle/nx_oracle.cpp) before it is trusted as the checker.

Each check is chosen so that a plausible mistake fails it: exact rational
arithmetic (tests/exact_fp32.py) for every fp32 rounding, constructed ties that
tell RNE from lround, closed forms for the NaN/Inf/zero special cases, the
scale-index formula, numpy int64 brute force for the integer sums, and the
known-answer vectors in tests/golden/.
"""
from __future__ import annotations

import glob
import os

import numpy as np
import pytest

import exact_fp32 as X

GOLDEN = sorted(glob.glob(os.path.join(os.path.dirname(__file__), "golden", "*.npz")))


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


# --- the exact checker itself --------------------------------------------------

def test_exact_checker_matches_ieee_float32_ops():
    rng = np.random.default_rng(0)
    a = (rng.standard_normal(400) * 10.0 ** rng.integers(-30, 30, 400)).astype(np.float32)
    b = (rng.standard_normal(400) * 10.0 ** rng.integers(-8, 8, 400)).astype(np.float32)
    with np.errstate(over="ignore", under="ignore"):
        for x, y in zip(a, b):
            assert X.mul(x, y) == float(np.float32(x) * np.float32(y))
            assert X.div(x, y) == float(np.float32(x) / np.float32(y))
            assert X.add(x, y) == float(np.float32(x) + np.float32(y))
    # subnormal results and overflow
    assert X.mul(1e-30, 1e-15) == float(np.float32(1e-30) * np.float32(1e-15))
    assert X.mul(3e38, 10.0) == float("inf")
    # fma rounds once: (1 + 2^-23)(1 - 2^-23) - 1 = -2^-46 exactly
    e = 2.0 ** -23
    assert X.fma(1 + e, 1 - e, -1.0) == -(2.0 ** -46)
    assert X.rne_int(2.5) == 2 and X.rne_int(3.5) == 4 and X.rne_int(-2.5) == -2
    assert X.lround(2.5) == 3 and X.lround(-2.5) == -3 and X.lround(0.49999997) == 0


# --- quantize_row -------------------------------------------------------------

@pytest.mark.parametrize("act_max", [127, 63])
@pytest.mark.parametrize("n_in", [32, 256, 96 + 256, 1024])
def test_quantize_matches_exact_arithmetic(orc, act_max, n_in):
    rng = np.random.default_rng(n_in + act_max)
    T = 5
    x = (rng.standard_normal((T, n_in)) * np.exp(rng.standard_normal((T, 1)) * 3)).astype(np.float32)
    q, sx = orc.quantize_rows(x, act_max)
    sxm = orc.sx_matrix(sx, T, n_in)
    for t in range(T):
        for B in range(orc.n_blocks(n_in)):
            i0, i1 = B * 256, min(n_in, (B + 1) * 256)
            qq, s = X.quantize_block([float(v) for v in x[t, i0:i1]], act_max)
            assert list(q[t, i0:i1]) == qq
            assert float(sxm[t, B]) == s


def test_quantize_round_half_even_ties(orc):
    # amax = 127 -> inv = 127/127 = 1 exactly, so q = RNE(x) + 128
    x = np.zeros((1, 256), np.float32)
    x[0, 0] = 127.0
    x[0, 1:9] = [0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 3.5, -126.5]
    q, sx = orc.quantize_rows(x)
    got = q[0, 1:9].astype(int) - 128
    assert list(got) == [0, 2, 2, 0, -2, -2, 4, -126]      # lround would give 1, 2, 3, -1, -2, -3, 4, -127
    assert sx[0] == np.float32(1.0)
    assert q[0, 0] == 255


def test_quantize_zero_block_and_scale_index(orc):
    T, n_in = 7, 768
    nb = 3
    x = np.zeros((T, n_in), np.float32)
    for t in range(T):
        for B in range(nb):
            if (t + B) % 3:
                x[t, B * 256 + (t * 5 + B) % 256] = np.float32((t + 1) * 10 + B)
    q, sx = orc.quantize_rows(x)
    for t in range(T):
        for B in range(nb):
            amax = (t + 1) * 10 + B if (t + B) % 3 else 0
            assert sx[orc.sx_index(t, B, nb)] == np.float32(np.float32(amax) / np.float32(127))
            blk = q[t, B * 256:(B + 1) * 256]
            if amax == 0:
                assert (blk == 128).all()
            else:
                assert blk.max() == 255 and (np.sort(blk)[:-1] == 128).all()


def test_quantize_inf_closed_form(orc):
    x = np.random.default_rng(3).standard_normal((2, 256)).astype(np.float32)
    x[0, 17] = np.inf
    x[1, 200] = -np.inf
    q, sx = orc.quantize_rows(x)
    # amax = inf -> inv = 0 -> finite x*0 = 0 -> 128; inf*0 = NaN -> 0x80000000 -> saturates to 0
    for t, p in ((0, 17), (1, 200)):
        assert q[t, p] == 0
        assert (np.delete(q[t], p) == 128).all()
        assert np.isinf(orc.sx_matrix(sx, 2, 256)[t, 0])


def test_quantize_nan_closed_forms(orc):
    rng = np.random.default_rng(4)
    base = rng.uniform(-1, 1, 256).astype(np.float32)
    base[100] = 2.0   # unique maximum, lane 4 position 12
    # NaN as the last element of its lane's sequence: it survives every MAXPS -> amax NaN
    x = np.stack([base, base, base])
    x[0, 255] = np.nan
    # NaN at the first element of lane 0: the next element of that lane replaces it
    x[1, 0] = np.nan
    # NaN in the same lane as the maximum but before it: forgotten, amax = 2
    x[2, 4] = np.nan
    q, sx = orc.quantize_rows(x)
    sxm = orc.sx_matrix(sx, 3, 256)
    assert np.isnan(sxm[0, 0])
    assert q[0, 255] == 0 and (q[0, :255] == 128).all()     # inv = 0 (NaN > 0 is false)
    for t, p in ((1, 0), (2, 4)):
        assert sxm[t, 0] == np.float32(np.float32(2.0) / np.float32(127))
        assert q[t, p] == 0                                     # NaN*inv -> indefinite -> 0
        assert q[t, 100] == 255
    # NaN after the maximum in the same lane wipes the maximum: amax = max of the others
    x2 = base.copy()
    x2[108] = np.nan
    q2, sx2 = orc.quantize_rows(x2[None])
    others = np.abs(np.delete(base, [100, 108]))
    lane4_tail = np.abs(base[116::8])   # lane 4's elements after the NaN
    expect = max(np.max(np.abs(np.delete(base, np.r_[4:256:8]))), lane4_tail.max())
    assert sx2[0] == np.float32(np.float32(expect) / np.float32(127))
    assert others.max() >= expect


def test_quantize_scalar_matches_simd_on_adversarial_rows(orc):
    rng = np.random.default_rng(5)
    T, n_in = 64, 512 + 96
    x = rng.standard_normal((T, n_in)).astype(np.float32)
    specials = np.array([np.nan, np.inf, -np.inf, 0.0, -0.0, 1e-40, -1e-42, 3e38, -3e38, 1e-38],
                        np.float32)
    for t in range(T):
        k = rng.integers(0, 6)
        pos = rng.integers(0, n_in, k)
        x[t, pos] = specials[rng.integers(0, len(specials), k)]
    x[5] = 1e-41          # all-subnormal row: inv overflows to inf
    x[6] = 0.0
    x[7, :] = -0.0
    x[8] *= np.float32(1e-38)
    for act_max in (127, 63):
        q1, s1 = orc.quantize_rows(x, act_max, simd=False)
        q2, s2 = orc.quantize_rows(x, act_max, simd=True)
        assert (q1 == q2).all()
        assert (bits(s1) == bits(s2)).all()


def test_quantize_subnormal_row_maps_to_zero(orc):
    # amax ~1e-41 -> 127/amax = inf -> x*inf = +-inf -> indefinite -> u8 0 (q_s = -128)
    x = np.full((1, 64), np.float32(1e-41))
    x[0, ::2] *= -1
    q, sx = orc.quantize_rows(x)
    assert (q == 0).all()
    assert sx[0] == np.float32(np.float32(1e-41) / np.float32(127))


# --- op_relu_sqr ----------------------------------------------------------------

def test_relu2_closed_form(orc):
    # MAXPS(x, 0) returns the second operand for NaN and for -0 (not greater): both 0.
    x = np.array([np.nan, -np.nan, np.inf, -np.inf, 0.0, -0.0, -1.0, -1e-40, 1e-40, 1e-20, 3e38,
                  1.5, 2.0 ** 64], np.float32)
    y = orc.relu2(x)
    zero = [0, 1, 3, 4, 5, 6, 7, 8]              # NaN, -inf, +-0, negatives, 1e-40^2 underflow
    assert (bits(y[zero]) == 0).all()            # all +0
    assert y[2] == np.inf and y[10] == np.inf and y[12] == np.inf   # inf, 3e38^2, 2^128
    assert y[11] == np.float32(2.25)
    # 1e-20^2 = 1e-40 is an f32 subnormal: RNE of the exact square
    assert y[9] == np.float32(np.float64(np.float32(1e-20)) ** 2) and y[9] > 0


def test_relu2_is_the_exact_square_rounded_once(orc):
    # the product of two f32 is exact in f64 (48 significant bits), so f32(f64(r)^2)
    # is the single RNE rounding of r*r; subnormal and overflow ranges included
    rng = np.random.default_rng(11)
    x = (rng.standard_normal(20000) * 10.0 ** rng.integers(-25, 22, 20000)).astype(np.float32)
    y = orc.relu2(x)
    r = np.where(x > 0, x, 0).astype(np.float64)
    with np.errstate(over="ignore"):
        want = (r * r).astype(np.float32)
    assert (bits(y) == bits(want)).all()


# --- op_rms_norm -----------------------------------------------------------------

def _exact_dot_avx2(x):
    """dot_f32(x, x) in the AVX2 build's order (src/nexterabert.cpp:124-149), every
    operation rounded once by exact arithmetic."""
    s = [[0.0] * 8 for _ in range(4)]
    n = len(x)
    i = 0
    while i + 32 <= n:
        for k in range(4):
            for j in range(8):
                e = float(x[i + 8 * k + j])
                s[k][j] = X.fma(e, e, s[k][j])
        i += 32
    while i + 8 <= n:
        for j in range(8):
            e = float(x[i + j])
            s[0][j] = X.fma(e, e, s[0][j])
        i += 8
    v = [X.add(X.add(s[0][j], s[1][j]), X.add(s[2][j], s[3][j])) for j in range(8)]
    h = [X.add(v[j], v[j + 4]) for j in range(4)]
    return X.add(X.add(h[0], h[2]), X.add(h[1], h[3]))


def _exact_rms_norm(x, g, eps):
    C = len(x)
    inv = X.div(1.0, X.sqrt(X.add(X.div(_exact_dot_avx2(x), float(C)), float(np.float32(eps)))))
    return np.array([X.mul(X.mul(float(x[i]), inv), float(g[i])) for i in range(C)], np.float32)


@pytest.mark.parametrize("C", [32, 64, 96, 136])
def test_rms_norm_matches_exact_arithmetic(orc, C):
    rng = np.random.default_rng(C)
    x = (rng.standard_normal((3, C)) * 10.0 ** rng.integers(-3, 4, (3, C))).astype(np.float32)
    g = (1.0 + 0.1 * rng.standard_normal(C)).astype(np.float32)
    for eps in (1e-8, 1e-5, 0.0):
        y = orc.rms_norm(x, g, eps)
        for t in range(3):
            assert (bits(y[t]) == bits(_exact_rms_norm(x[t], g, eps))).all()


def test_rms_norm_follows_the_avx2_accumulation_order(orc):
    # one large square among small ones: where the small ones are absorbed depends on
    # which accumulator chain and combine step they meet the large one in
    C = 64
    x = np.full(C, np.float32(3e-4), np.float32)
    x[5] = np.float32(1.0)
    x[37] = np.float32(-1.0)
    exact_order = _exact_dot_avx2(x)
    seq = 0.0
    for e in x:
        seq = X.fma(float(e), float(e), seq)
    assert exact_order != seq            # the check below can tell the two orders apart
    g = np.ones(C, np.float32)
    y = orc.rms_norm(x[None, :], g, 0.0)[0]
    assert (bits(y) == bits(_exact_rms_norm(x, g, 0.0))).all()


def test_rms_norm_closed_forms(orc):
    C = 64
    g = np.full(C, np.float32(2.0), np.float32)
    # zero row, eps 0: inv = 1/0 = inf, 0 * inf = NaN
    assert np.isnan(orc.rms_norm(np.zeros((1, C), np.float32), g, 0.0)).all()
    # zero row, eps > 0: 0
    assert (orc.rms_norm(np.zeros((1, C), np.float32), g, 1e-8) == 0).all()
    # constant row a = 2: dot = 256 exactly, mean 4, inv 0.5, out (2 * 0.5) * 2 = 2
    assert (orc.rms_norm(np.full((1, C), np.float32(2.0)), g, 0.0) == 2.0).all()
    # a NaN or an Inf anywhere makes inv NaN or 0
    x = np.ones((2, C), np.float32)
    x[0, 7] = np.nan
    x[1, 9] = np.inf
    y = orc.rms_norm(x, g, 0.0)
    assert np.isnan(y[0]).all()
    assert np.isnan(y[1, 9]) and (y[1, np.arange(C) != 9] == 0).all()


# --- build_i8_weight ----------------------------------------------------------

@pytest.mark.parametrize("n_in", [64, 256 + 32, 1024])
def test_expand_matches_exact_arithmetic(orc, n_in):
    rng = np.random.default_rng(n_in)
    rows = (0.02 * rng.standard_normal((6, n_in))).astype(np.float32)
    rows[1] = 0.0
    w, scale, off = orc.expand_rows(rows)
    for r in range(6):
        for B in range(orc.n_blocks(n_in)):
            i0, i1 = B * 256, min(n_in, (B + 1) * 256)
            qq, s, tot = X.expand_block([float(v) for v in rows[r, i0:i1]])
            assert list(w[r, i0:i1]) == qq
            assert float(scale[B, r]) == s
            assert off[B, r] == -128 * tot


def test_expand_lround_ties_away_from_zero(orc):
    rows = np.zeros((1, 32), np.float32)
    rows[0, 0] = 127.0                       # inv = 1
    rows[0, 1:7] = [0.5, 1.5, 2.5, -0.5, -1.5, -2.5]
    w, scale, off = orc.expand_rows(rows, act_off=64)
    assert list(w[0, 1:7]) == [1, 2, 3, -1, -2, -3]   # RNE would give 0, 2, 2, 0, -2, -2
    assert off[0, 0] == -64 * int(w[0].astype(int).sum())
    assert scale[0, 0] == np.float32(1.0)


def test_q8_0_dequant_is_exact(orc):
    rng = np.random.default_rng(7)
    nblk = 16
    d = (rng.uniform(1e-4, 1e-2, nblk)).astype(np.float16)
    qs = rng.integers(-127, 128, (nblk, 32)).astype(np.int8)
    raw = np.zeros((nblk, 34), np.uint8)
    raw[:, 0:2] = d.view(np.uint8).reshape(nblk, 2)
    raw[:, 2:] = qs.view(np.uint8)
    out = orc.dequant_q8_0(raw.reshape(-1), nblk * 32)
    expect = (d.astype(np.float64)[:, None] * qs.astype(np.float64)).astype(np.float32).reshape(-1)
    assert (bits(out) == bits(expect)).all()


# --- int8 GEMM ----------------------------------------------------------------

def _case(rng, T, n_in, n_out, act_max=127):
    x = rng.standard_normal((T, n_in)).astype(np.float32)
    rows = (0.02 * rng.standard_normal((n_out, n_in))).astype(np.float32)
    q, sx = _quant(x, act_max)
    w, scale, off = _expand(rows, act_max + 1)
    return x, q, sx, w, scale, off


def _quant(x, act_max):
    from oracle import oracle as o
    return o.quantize_rows(x, act_max)


def _expand(rows, act_off):
    from oracle import oracle as o
    return o.expand_rows(rows, act_off)


@pytest.mark.parametrize("n_in", [64, 256, 320, 1024])
def test_block_sums_equal_signed_int64_matmul(orc, n_in):
    rng = np.random.default_rng(n_in + 1)
    T, n_out = 9, 13
    _, q, sx, w, scale, off = _case(rng, T, n_in, n_out)
    sums = orc.block_sums(w, off, q)
    qs = q.astype(np.int64) - 128
    for B in range(orc.n_blocks(n_in)):
        i0, i1 = B * 256, min(n_in, (B + 1) * 256)
        ref = qs[:, i0:i1] @ w[:, i0:i1].astype(np.int64).T
        assert (sums[B] == ref).all()


def test_linear_scalar_matches_exact_arithmetic(orc):
    rng = np.random.default_rng(8)
    T, n_in, n_out = 3, 512 + 64, 5
    _, q, sx, w, scale, off = _case(rng, T, n_in, n_out)
    res = rng.standard_normal((T, n_out)).astype(np.float32)
    y = orc.linear(w, scale, off, q, sx)
    yr = orc.linear(w, scale, off, q, sx, res=res)
    sxm = orc.sx_matrix(sx, T, n_in)
    for t in range(T):
        for r in range(n_out):
            args = (w[r], scale[:, r], off[:, r], q[t], [float(v) for v in sxm[t]])
            assert float(y[t, r]) == X.linear_point(*args)
            assert float(yr[t, r]) == X.linear_point(*args, res=float(res[t, r]))


def test_linear_single_block_closed_form(orc):
    # one block: y = RN(RN(s * sx) * sw), since fma(p, sw, 0) rounds p*sw once
    rng = np.random.default_rng(9)
    _, q, sx, w, scale, off = _case(rng, 4, 256, 6)
    y = orc.linear(w, scale, off, q, sx)
    s = (q.astype(np.int64) - 128) @ w.astype(np.int64).T
    p = s.astype(np.float32) * orc.sx_matrix(sx, 4, 256)[:, 0:1]
    assert (bits(y) == bits(p * scale[0][None, :])).all()


def test_linear_unit_scales_is_integer_matmul(orc):
    rng = np.random.default_rng(10)
    T, n_in, n_out = 6, 768, 7
    q = rng.integers(1, 256, (T, n_in)).astype(np.uint8)
    w = rng.integers(-127, 128, (n_out, n_in)).astype(np.int8)
    nb = 3
    off = (-128 * w.reshape(n_out, nb, 256).astype(np.int64).sum(-1)).T.astype(np.int32).copy()
    scale = np.ones((nb, n_out), np.float32)
    sx = np.ones(orc.sx_len(T, n_in), np.float32)
    y = orc.linear(w, scale, off, q, sx)
    ref = (q.astype(np.int64) - 128) @ w.astype(np.int64).T
    assert (y == ref.astype(np.float32)).all()


def test_linear_float64_tolerance_crosscheck(orc):
    rng = np.random.default_rng(11)
    T, n_in, n_out = 8, 1024, 16
    _, q, sx, w, scale, off = _case(rng, T, n_in, n_out)
    y = orc.linear(w, scale, off, q, sx)
    sxm = orc.sx_matrix(sx, T, n_in).astype(np.float64)
    qs = q.astype(np.float64) - 128
    ref = np.zeros((T, n_out))
    for B in range(4):
        sl = slice(B * 256, (B + 1) * 256)
        ref += (qs[:, sl] @ w[:, sl].astype(np.float64).T) * sxm[:, B:B + 1] * scale[B][None, :]
    assert np.allclose(y, ref, rtol=1e-5, atol=1e-6 * np.abs(ref).max())


@pytest.mark.parametrize("T,n_in,n_out", [(1, 1024, 4), (37, 1024, 100), (10, 2304, 25), (64, 64, 12)])
def test_linear_simd_matches_scalar(orc, T, n_in, n_out):
    if not orc.vnni_flavour():
        pytest.skip("no VNNI on this CPU")
    rng = np.random.default_rng(T * n_in + n_out)
    _, q, sx, w, scale, off = _case(rng, T, n_in, n_out)
    res = rng.standard_normal((T, n_out)).astype(np.float32)
    for r in (None, res):
        a = orc.linear(w, scale, off, q, sx, res=r)
        for nt in (1, 3):
            b = orc.linear(w, scale, off, q, sx, res=r, simd=True, n_threads=nt)
            assert (bits(a) == bits(b)).all()


def test_linear_batch_invariance(orc):
    # a row's result does not depend on where it sits in the packed batch
    if not orc.vnni_flavour():
        pytest.skip("no VNNI on this CPU")
    rng = np.random.default_rng(12)
    x = rng.standard_normal((23, 512)).astype(np.float32)
    rows = (0.02 * rng.standard_normal((10, 512))).astype(np.float32)
    w, scale, off = orc.expand_rows(rows)
    q, sx = orc.quantize_rows(x)
    full = orc.linear(w, scale, off, q, sx, simd=True, n_threads=2)
    for t in (0, 5, 22):
        q1, sx1 = orc.quantize_rows(x[t:t + 1])
        one = orc.linear(w, scale, off, q1, sx1, simd=True)
        assert (bits(one[0]) == bits(full[t])).all()


# --- known-answer vectors -------------------------------------------------------

@pytest.mark.parametrize("path", GOLDEN, ids=lambda p: os.path.basename(p))
def test_golden_vectors(orc, path):
    g = np.load(path)
    act_max = int(g["act_max"])
    q, sx = orc.quantize_rows(g["x"], act_max)
    assert (q == g["q"]).all()
    assert (bits(sx) == bits(g["sx"])).all()
    w, scale, off = orc.expand_rows(g["wf"], act_max + 1)
    assert (w == g["w8"]).all() and (bits(scale) == bits(g["sw"])).all() and (off == g["off"]).all()
    assert (orc.block_sums(w, off, q) == g["sums"]).all()
    assert (bits(orc.linear(w, scale, off, q, sx)) == bits(g["y"])).all()
    assert (bits(orc.linear(w, scale, off, q, sx, res=g["res"])) == bits(g["y_res"])).all()
    if orc.vnni_flavour() and act_max == 127 and g["x"].shape[1] % 32 == 0:
        y2 = orc.linear(w, scale, off, q, sx, res=g["res"], simd=True, n_threads=2)
        assert (bits(y2) == bits(g["y_res"])).all()
