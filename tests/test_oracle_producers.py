"""CPU: pins of the oracle's mixer producers -- exp256 / op_gate, op_dwconv,
op_lily_state and op_block_mean (src/nexterabert.cpp:81-122, 507-578, 638-659).

Each is checked against (a) exact binary32 arithmetic, one correctly rounded
operation at a time (tests/exact_fp32.py), which tells fused from unfused steps and
any other rounding difference, (b) closed forms that hold whatever the inputs (clamps,
one-hot taps, single-row documents, block sizes whose reciprocal is exact), and, for
exp, (c) the same steps on AVX2 + FMA themselves and the true exponential (which the
Cephes constants must approximate to a few units in the last place)."""
from __future__ import annotations

import math

import numpy as np
import pytest

import exact_fp32 as X


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def f32(v):
    return float(np.float32(v))


# --- exp256 ---------------------------------------------------------------------

P = [1.9875691500e-4, 1.3981999507e-3, 8.3334519073e-3, 4.1665795894e-2, 1.6666665459e-1, 5.0000001201e-1]


def exact_exp(x: float) -> float:
    """exp256 for one finite lane, each operation rounded once."""
    hi, lo = f32(88.3762626647949), f32(-87.3)
    x = x if x < hi else hi
    x = x if x > lo else lo
    n = X.rne_int(X.mul(x, f32(1.44269504088896341)))
    r = X.fma(-n, f32(0.693359375), x)
    r = X.fma(-n, f32(-2.12194440e-4), r)
    r2 = X.mul(r, r)
    p = f32(P[0])
    for c in P[1:]:
        p = X.fma(p, r, f32(c))
    p = X.fma(p, r2, X.add(r, 1.0))
    return X.mul(p, math.ldexp(1.0, n))


def test_exp_matches_exact_arithmetic(orc):
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.uniform(-95, 95, 300), rng.uniform(-2, 2, 100), [0.0, -0.0, 1e-30, -1e-30]]).astype(np.float32)
    y = orc.exp_cephes(x)
    ref = np.array([exact_exp(float(v)) for v in x], np.float32)
    assert (bits(y) == bits(ref)).all()


def tie_points(k_range):
    """f32 x with x * log2(e) rounding to exactly k + 0.5 (n's ties-to-even case)."""
    L = np.float32(1.44269504088896341)
    out = []
    for k in k_range:
        x = np.float32((k + 0.5) / float(L))
        for _ in range(64):
            if np.float32(x * L) == np.float32(k + 0.5):
                out.append(x)
                break
            x = np.nextafter(x, np.float32(np.inf) if np.float32(x * L) < k + 0.5 else np.float32(-np.inf))
    return np.array(out, np.float32)


def test_exp_scalar_equals_avx2_fma(orc):
    rng = np.random.default_rng(2)
    specials = np.array([np.nan, np.inf, -np.inf, 0.0, -0.0, 88.3762626647949, 88.38, -87.3, -87.31, 1e-38, -1e-45,
                         3.4e38, -3.4e38], np.float32)
    ties = tie_points(range(-120, 120, 7))
    assert ties.size > 20
    x = np.concatenate([rng.uniform(-100, 100, 200_000).astype(np.float32), specials, ties])
    x = np.concatenate([x, np.zeros((-x.size) % 8, np.float32)])
    try:
        s = orc.exp_cephes(x, simd=True)
    except RuntimeError:
        pytest.skip("no AVX2/FMA on this CPU")
    assert (bits(orc.exp_cephes(x)) == bits(s)).all()


def test_exp_approximates_the_exponential(orc):
    x = np.linspace(-87.0, 88.3, 400_001, dtype=np.float32)
    y = orc.exp_cephes(x).astype(np.float64)
    ref = np.exp(x.astype(np.float64))
    assert np.max(np.abs(y - ref) / ref) < 4 * 2.0 ** -24


def test_exp_closed_forms(orc):
    e = lambda v: orc.exp_cephes(np.array([v], np.float32))[0]
    assert e(0.0) == 1.0 and e(-0.0) == 1.0 and e(1e-30) == 1.0
    top, bottom = e(88.3762626647949), e(-87.3)
    # clamps, MINPS/MAXPS returning the bound for a NaN
    for v in (88.38, 100.0, 3e38, np.inf, np.nan):
        assert bits(e(v)) == bits(top)
    for v in (-87.31, -100.0, -3e38, -np.inf):
        assert bits(e(v)) == bits(bottom)
    assert np.isfinite(top) and top > 2.0 ** 127 and 2.0 ** -126 <= bottom < 2.0 ** -125


# --- op_gate --------------------------------------------------------------------

def test_gate_matches_exact_arithmetic(orc):
    rng = np.random.default_rng(3)
    g = (rng.standard_normal((4, 32)) * 6).astype(np.float32)
    y = rng.standard_normal((4, 32)).astype(np.float32)
    out = orc.gate(g, y)
    for t in range(4):
        for i in range(32):
            e = exact_exp(X.add(0.0, -float(g[t, i])))
            ref = X.mul(X.div(1.0, X.add(1.0, e)), float(y[t, i]))
            assert bits(np.float32(ref)) == bits(out[t, i])


def test_gate_closed_forms(orc):
    y = np.array([[1.5, -2.25, 3e-3, -7e10] * 8], np.float32)
    assert (bits(orc.gate(np.zeros_like(y), y)) == bits(0.5 * y)).all()            # sigmoid(0) = 1/2
    assert (bits(orc.gate(np.full_like(y, 100.0), y)) == bits(y)).all()            # 1 / (1 + ~6e-39) = 1
    # very negative and NaN g: exp clamps at its upper bound, 1 / (1 + 2.4e38)
    lo = orc.gate(np.full_like(y, -100.0), y)
    assert (bits(orc.gate(np.full_like(y, np.nan), y)) == bits(lo)).all()
    top = float(orc.exp_cephes(np.array([88.3762626647949], np.float32))[0])
    s = X.div(1.0, X.add(1.0, top))                                               # ~4.2e-39, subnormal
    assert 0 < s < 2.0 ** -126
    assert (bits(lo) == bits(np.array([X.mul(s, float(v)) for v in y[0]], np.float32))).all()


# --- op_dwconv / op_lily_state ----------------------------------------------------

def packed(rng, lengths, C):
    cu = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
    return cu, rng.standard_normal((int(cu[-1]), C)).astype(np.float32)


def exact_dwconv(x, r, taps, cu):
    T, C = x.shape
    k = taps.shape[0]
    out = np.zeros_like(x)
    for d in range(len(cu) - 1):
        lo, hi = int(cu[d]), int(cu[d + 1])
        for t in range(lo, hi):
            for i in range(C):
                o = float(r[t, i]) if r is not None else 0.0
                for j in range(k):
                    tt = t + j - k // 2
                    if lo <= tt < hi:
                        o = X.fma(float(taps[j, i]), float(x[tt, i]), o)
                out[t, i] = o
    return out


@pytest.mark.parametrize("k", [3, 4, 5])
@pytest.mark.parametrize("with_r", [False, True])
def test_dwconv_matches_exact_arithmetic(orc, k, with_r):
    rng = np.random.default_rng(10 * k + with_r)
    cu, x = packed(rng, [1, 4, 6, 2], 32)
    r = rng.standard_normal(x.shape).astype(np.float32) if with_r else None
    taps = rng.standard_normal((k, 32)).astype(np.float32)
    assert (bits(orc.dwconv(x, taps, cu, r)) == bits(exact_dwconv(x, r, taps, cu))).all()


def test_dwconv_closed_forms(orc):
    rng = np.random.default_rng(11)
    cu, x = packed(rng, [1, 7, 3], 64)
    r = rng.standard_normal(x.shape).astype(np.float32)
    one_hot = np.zeros((5, 64), np.float32)
    one_hot[2] = 1.0                                                    # the centre tap, j = k/2
    assert (bits(orc.dwconv(x, one_hot, cu, r)) == bits(x + r)).all()
    assert (bits(orc.dwconv(x, np.zeros((5, 64), np.float32), cu, r)) == bits(r)).all()
    # a one-row document sees only its own row: fma(taps[k/2], x, 0)
    taps = rng.standard_normal((5, 64)).astype(np.float32)
    y = orc.dwconv(x, taps, cu)
    assert (bits(y[0]) == bits(taps[2] * x[0])).all()
    # documents do not see each other: one alone gives the same rows
    alone = orc.dwconv(x[1:8], taps, [0, 7])
    assert (bits(alone) == bits(y[1:8])).all()


def exact_lily(a, x, b, taps, cu):
    T, C = x.shape
    k = taps.shape[0]
    out = np.zeros_like(x)
    for d in range(len(cu) - 1):
        lo, hi = int(cu[d]), int(cu[d + 1])
        for t in range(lo, hi):
            j0, j1 = max(0, lo - (t - k // 2)), min(k, hi - (t - k // 2))
            for i in range(C):
                acc = 0.0
                for j in range(j0, j1):
                    tt = t + j - k // 2
                    acc = X.fma(float(taps[j, i]), X.mul(float(a[tt, i]), float(x[tt, i])), acc)
                out[t, i] = X.mul(acc, float(b[t, i]))
    return out


@pytest.mark.parametrize("k", [3, 5])
def test_lily_state_matches_exact_arithmetic(orc, k):
    rng = np.random.default_rng(20 + k)
    cu, x = packed(rng, [2, 5, 1, 4], 32)
    a = rng.standard_normal(x.shape).astype(np.float32)
    b = rng.standard_normal(x.shape).astype(np.float32)
    taps = rng.standard_normal((k, 32)).astype(np.float32)
    assert (bits(orc.lily_state(a, x, b, taps, cu)) == bits(exact_lily(a, x, b, taps, cu))).all()


def test_lily_state_closed_forms(orc):
    rng = np.random.default_rng(23)
    cu, x = packed(rng, [6, 1, 3], 64)
    a = rng.standard_normal(x.shape).astype(np.float32)
    b = rng.standard_normal(x.shape).astype(np.float32)
    one_hot = np.zeros((5, 64), np.float32)
    one_hot[2] = 1.0
    assert (bits(orc.lily_state(a, x, b, one_hot, cu)) == bits((a * x) * b)).all()
    assert (bits(orc.lily_state(a, x, b, np.zeros((5, 64), np.float32), cu)) == bits(np.float32(0.0) * b)).all()
    taps = rng.standard_normal((5, 64)).astype(np.float32)
    y = orc.lily_state(a, x, b, taps, cu)
    assert (bits(orc.lily_state(a[6:7], x[6:7], b[6:7], taps, [0, 1])) == bits(y[6:7])).all()
    assert (bits(y[6]) == bits((taps[2] * (a[6] * x[6])) * b[6])).all()


# --- op_block_mean --------------------------------------------------------------

def exact_block_mean(h, g, cu, block):
    rows = []
    for d in range(len(cu) - 1):
        lo, n_tok = int(cu[d]), int(cu[d + 1] - cu[d])
        for bi in range((n_tok + block - 1) // block):
            ts, n = lo + bi * block, min(block, n_tok - bi * block)
            o = [0.0] * h.shape[1]
            for u in range(n):
                for i in range(h.shape[1]):
                    hv = float(h[ts + u, i])
                    o[i] = X.fma(hv, float(g[ts + u, i]), o[i]) if g is not None else X.add(o[i], hv)
            inv = X.div(1.0, float(n))
            rows.append([X.mul(v, inv) for v in o])
    return np.array(rows, np.float32)


@pytest.mark.parametrize("block", [1, 3, 4])
@pytest.mark.parametrize("with_g", [False, True])
def test_block_mean_matches_exact_arithmetic(orc, block, with_g):
    rng = np.random.default_rng(30 + block + with_g)
    cu, h = packed(rng, [1, 5, 8, 3], 32)
    g = rng.standard_normal(h.shape).astype(np.float32) if with_g else None
    y = orc.block_mean(h, cu, block, g)
    assert y.shape[0] == sum((n + block - 1) // block for n in np.diff(cu))
    assert (bits(y) == bits(exact_block_mean(h, g, cu, block))).all()


def test_block_mean_closed_forms(orc):
    rng = np.random.default_rng(33)
    cu, h = packed(rng, [4, 2, 1], 64)
    g = rng.standard_normal(h.shape).astype(np.float32)
    assert (bits(orc.block_mean(h, cu, 1, g)) == bits(h * g)).all()                # block 1: one product per row
    y = orc.block_mean(h, cu, 2)                                                   # 1/2 is exact
    assert (bits(y[0]) == bits((h[0] + h[1]) * np.float32(0.5))).all()
    assert (bits(y[2]) == bits((h[4] + h[5]) * np.float32(0.5))).all()
    assert (bits(y[3]) == bits(h[6])).all()                                        # a one-token run: itself
