"""CPU: pins of the oracle's op_attention (head_dim 64, src/nexterabert.cpp:704-852) and of
the restated C-library expf that the GPU uses for softmax_exp's last n % 8 keys.

  * expf: the restatement equals the host's expf on every 97th float bit pattern and on
    the whole range softmax arguments take near 0 and near underflow (the full 2^32 check
    was run once on the host: 0 mismatches);
  * scores: the lane-wise statement of scores_d64 equals the same steps on AVX2 + FMA
    (HADDPS / VPERM2F128 for groups of 8 keys, hsum256 for the rest);
  * attention: one key gives v itself; equal scores give the exact-arithmetic mean chain;
    it is attention (a float64 softmax within a few float ulps); GQA heads of one group
    share their keys; a band at least as wide as the document is the full attention;
    documents do not see each other; per-document scales apply per document."""
from __future__ import annotations

import numpy as np
import pytest

import exact_fp32 as X


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def test_expf_restatement_equals_the_c_library(orc):
    n, bad = orc.expf_restated_mismatches(0, 97, 2 ** 32 // 97 + 1)
    assert n == 0, [hex(b) for b in bad]
    # [-104, 0]: softmax's arguments, through the subnormal results to the underflow cut
    lo, hi = 0x80000000, 0xC2D00000          # -0.0 .. -104.0 as bit patterns
    n, bad = orc.expf_restated_mismatches(lo, 7, (hi - lo) // 7 + 1)
    assert n == 0, [hex(b) for b in bad]


@pytest.mark.parametrize("n", [1, 7, 8, 9, 16, 63, 100])
def test_scores_lane_statement_equals_avx2(orc, n):
    rng = np.random.default_rng(n)
    q = rng.standard_normal(64).astype(np.float32)
    k = (rng.standard_normal((n, 64)) * np.exp(rng.uniform(-4, 4, (n, 1)))).astype(np.float32)
    try:
        s = orc.scores_d64(q, k, 0.125, simd=True)
    except RuntimeError:
        pytest.skip("no AVX2/FMA")
    assert (bits(orc.scores_d64(q, k, 0.125)) == bits(s)).all()


def sequential_softmax(s):
    """softmax_exp's weights (exp256 for the 8-groups, expf for the tail, as the oracle) but
    summed one by one in index order: a plausible wrong order the pin must reject."""
    import oracle.oracle as o
    w, _ = o.softmax_exp(s)
    total = np.float32(0)
    for x in w:
        total = np.float32(total + x)
    return w, total


@pytest.mark.parametrize("n", list(range(1, 101)))
def test_softmax_exp_order_equals_avx2(orc, n):
    """softmax_exp's lane statement (8 lane sums of the 8-groups, hsum256, then the tail one by
    one) equals the reference's instructions on AVX2 + FMA bit for bit, weights and sum, on
    scores spread over +-30 (so the weights span many binades)."""
    rng = np.random.default_rng(1000 + n)
    s = (rng.standard_normal(n) * rng.uniform(0.1, 10)).astype(np.float32)
    try:
        w_simd, sum_simd = orc.softmax_exp(s, simd=True)
    except RuntimeError:
        pytest.skip("no AVX2/FMA")
    w, total = orc.softmax_exp(s)
    assert (bits(w) == bits(w_simd)).all()
    assert bits(np.float32(total)) == bits(np.float32(sum_simd))
    assert w.max() == np.float32(1.0)                   # exp(max - max)


def test_softmax_exp_order_is_pinned(orc):
    """A constructed row whose sequential sum differs from the lane order's: the statement
    follows the reference's instructions there too, so a wrong order fails the test above."""
    try:
        orc.softmax_exp(np.zeros(8, np.float32), simd=True)
    except RuntimeError:
        pytest.skip("no AVX2/FMA")
    # one weight of 1 (the max) among weights e^-15 .. e^-18, around half an ulp of 1: summed
    # one by one many of them round away, in 8 lanes they add up before meeting the 1
    found = None
    rng = np.random.default_rng(77)
    for trial in range(2000):
        n = int(rng.integers(9, 40))
        s = np.concatenate([[0.0], rng.uniform(-18, -15, n - 1)]).astype(np.float32)
        rng.shuffle(s)
        w, total = orc.softmax_exp(s)
        _, seq = sequential_softmax(s)
        if bits(np.float32(total)) != bits(np.float32(seq)):
            found = s
            break
    assert found is not None, "no row where the orders differ"
    w, total = orc.softmax_exp(found)
    w_simd, sum_simd = orc.softmax_exp(found, simd=True)
    assert bits(np.float32(total)) == bits(np.float32(sum_simd))
    assert bits(np.float32(sequential_softmax(found)[1])) != bits(np.float32(sum_simd))


def rand_qkv(rng, T, H, G):
    q = rng.standard_normal((T, H * 64)).astype(np.float32)
    k = rng.standard_normal((G, T, 64)).astype(np.float32)
    v = rng.standard_normal((G, T, 64)).astype(np.float32)
    return q, k, v


def attention64(q, k, v, cu, scale, H, G, half=-1):
    """float64 softmax attention inside each document (no particular order)."""
    T = q.shape[0]
    out = np.zeros((T, H * 64))
    rep = H // G
    for d in range(len(cu) - 1):
        for t in range(cu[d], cu[d + 1]):
            lo, hi = cu[d], cu[d + 1]
            if half >= 0:
                lo, hi = max(lo, t - half), min(hi, t + half + 1)
            for h in range(H):
                g = h // rep
                s = k[g, lo:hi].astype(np.float64) @ q[t, h * 64:(h + 1) * 64].astype(np.float64) * scale[d]
                w = np.exp(s - s.max())
                out[t, h * 64:(h + 1) * 64] = (w / w.sum()) @ v[g, lo:hi].astype(np.float64)
    return out


def test_attention_is_attention(orc):
    rng = np.random.default_rng(1)
    H, G = 4, 2
    cu = np.array([0, 5, 13, 40], np.int32)
    q, k, v = rand_qkv(rng, 40, H, G)
    scale = np.array([0.125, 0.2, 0.09], np.float32)
    for half in (-1, 3):
        y = orc.attention(q, k, v, cu, scale, H, G, half)
        ref = attention64(q, k, v, cu, scale, H, G, half)
        assert np.max(np.abs(y - ref)) < 2e-6 * max(1.0, np.max(np.abs(ref)))


def test_attention_closed_forms(orc):
    rng = np.random.default_rng(2)
    H, G = 4, 2
    cu = np.array([0, 1, 9, 25], np.int32)          # a one-token document, 8 and 16 keys
    q, k, v = rand_qkv(rng, 25, H, G)
    scale = np.full(3, 0.125, np.float32)
    y = orc.attention(q, k, v, cu, scale, H, G)
    # one key: softmax weight 1 (expf(0) = 1, 1/1), out = fma(1, v, 0) = v
    for h in range(H):
        assert (bits(y[0, h * 64:(h + 1) * 64]) == bits(v[h // 2, 0])).all()
    # equal keys: every weight exp256(0) = 1, sum n, out = fma(1/n, v_j, out) in key order
    k2 = k.copy()
    k2[:, 1:9] = k[:, 1:2]
    y2 = orc.attention(q, k2, v, cu, scale, H, G)
    inv = X.div(1.0, 8.0)
    for h in range(H):
        acc = [0.0] * 64
        for j in range(1, 9):
            acc = [X.fma(inv, float(v[h // 2, j, e]), acc[e]) for e in range(64)]
        assert (bits(y2[1, h * 64:(h + 1) * 64]) == bits(np.array(acc, np.float32))).all()
    # GQA: heads 0 and 1 share kv head 0 -- with the same query they give the same output
    q3 = q.copy()
    q3[:, 64:128] = q3[:, 0:64]
    y3 = orc.attention(q3, k, v, cu, scale, H, G)
    assert (bits(y3[:, 0:64]) == bits(y3[:, 64:128])).all()
    # a band as wide as the longest document is the full attention
    assert (bits(orc.attention(q, k, v, cu, scale, H, G, half=16)) == bits(y)).all()


def test_attention_documents_and_scales(orc):
    rng = np.random.default_rng(3)
    H, G = 2, 1
    cu = np.array([0, 11, 30, 37], np.int32)
    q, k, v = rand_qkv(rng, 37, H, G)
    scale = np.array([0.125, 0.3, 0.05], np.float32)
    y = orc.attention(q, k, v, cu, scale, H, G)
    lo, hi = 11, 30
    alone = orc.attention(q[lo:hi], k[:, lo:hi], v[:, lo:hi], [0, hi - lo], scale[1:2], H, G)
    assert (bits(alone) == bits(y[lo:hi])).all()
    # the scale is the document's own: another scale changes only that document
    s2 = scale.copy()
    s2[1] = 0.7
    y2 = orc.attention(q, k, v, cu, s2, H, G)
    assert (bits(y2[:lo]) == bits(y[:lo])).all() and (bits(y2[hi:]) == bits(y[hi:])).all()
    assert not (bits(y2[lo:hi]) == bits(y[lo:hi])).all()


def test_attention_scales_helper(nxg):
    import math
    cu = [0, 1, 5, 1029]
    base = np.float32(1.0) / np.float32(math.sqrt(64.0))
    assert (nxg.attention_scales(cu, 64, nxg.SSMAX_NONE) == base).all()
    s = nxg.attention_scales(cu, 64, nxg.SSMAX_SSMAX, s=0.5)
    ln = np.log(np.array([1, 4, 1024], np.float32))
    assert np.allclose(s, base * (np.float32(0.5) * ln), rtol=0, atol=1e-7)
    s3 = nxg.attention_scales(cu, 64, nxg.SSMAX_SSSMAX, s=0.5, b=-1.0, ssmax_base=0.1)
    assert s3[0] == base * np.float32(0.1)           # ln 1 = 0, max(b, 0) = 0


# --- tanh256 / op_qk_prep / build_rope ---------------------------------------------

def test_tanh_scalar_equals_avx2_and_is_tanh(orc):
    import math
    rng = np.random.default_rng(11)
    specials = [0.0, -0.0, 0.1, -0.1, 0.09999999, -0.09999999, np.nan, np.inf, -np.inf, 20.0, -20.0, 1e-30, 3e38, -3e38]
    x = np.concatenate([rng.standard_normal(200_000) * 3, specials]).astype(np.float32)
    x = np.concatenate([x, np.zeros((-x.size) % 8, np.float32)])
    y = orc.tanh_ref(x)
    try:
        ys = orc.tanh_ref(x, simd=True)
    except RuntimeError:
        ys = None
    if ys is not None:
        nan = np.isnan(y) & np.isnan(ys)
        assert ((bits(y) == bits(ys)) | nan).all()
    fin = np.isfinite(x)
    assert (bits(orc.tanh_ref(-x[fin])) == bits(-y[fin])).all()          # odd, bit for bit
    t = np.abs(x) < 15
    ref = np.tanh(x[t].astype(np.float64))
    assert np.max(np.abs(y[t] - ref) / np.maximum(np.abs(ref), 1e-30)) < 8 * 2.0 ** -24   # (1-t)/(1+t) near 0.1
    assert bits(orc.tanh_ref(np.array([-0.0], np.float32)))[0] == 0x80000000
    assert orc.tanh_ref(np.array([20.0], np.float32))[0] == 1.0
    # MINPS returns its second operand for a NaN, so exp256 clamps NaN to 88.38: t = inf-ish,
    # (1 - t) / (1 + t) = -1, and the NaN's sign bit is ORed in (NaN is not < 0.1: big is taken)
    assert orc.tanh_ref(np.array([np.nan], np.float32))[0] == -1.0
    assert not math.isnan(orc.tanh_ref(np.array([np.nan], np.float32))[0])


def test_rope_table(nxg):
    c, s = nxg.rope_table(300, 10000.0, 64)
    assert c.shape == s.shape == (300, 32)
    assert (c[0] == 1.0).all() and (s[0] == 0.0).all()
    inv = 1.0 / (10000.0 ** (np.arange(32) * 2 / 64.0))
    a = np.arange(300)[:, None] * inv[None, :]
    assert np.max(np.abs(c - np.cos(a))) < 1e-4 and np.max(np.abs(s - np.sin(a))) < 1e-4


def test_qk_prep_closed_forms(orc, nxg):
    rng = np.random.default_rng(12)
    H, D = 4, 64
    cu = np.array([0, 3, 40], np.int32)
    x = rng.standard_normal((40, H * D)).astype(np.float32)
    alpha = rng.uniform(0.2, 2.0, D).astype(np.float32)
    beta = rng.uniform(0.5, 1.5, D).astype(np.float32)
    c, s = nxg.rope_table(64, 10000.0, D)
    y = orc.qk_prep(x, alpha, beta, c, s, cu, H)
    # DyT terms
    a = beta[None, :32] * orc.tanh_ref(alpha[None, :32] * x.reshape(40, H, D)[:, :, :32])
    b = beta[None, 32:] * orc.tanh_ref(alpha[None, 32:] * x.reshape(40, H, D)[:, :, 32:])
    yr = y.reshape(40, H, D)
    # position 0 of each document: cos 1, sin 0 -> (a, b) exactly
    for t in (0, 3):
        assert (bits(yr[t, :, :32]) == bits(a[t])).all() and (bits(yr[t, :, 32:]) == bits(b[t])).all()
    # any position: y1 = fma(a, cos, b sin), y2 = fma(-a, sin, b cos), each rounded once
    t, pos = 17, 14
    for h in range(H):
        for i in range(32):
            ai, bi, ci, si = float(a[t, h, i]), float(b[t, h, i]), float(c[pos, i]), float(s[pos, i])
            assert bits(np.float32(X.fma(ai, ci, X.mul(bi, si)))) == bits(yr[t, h, i])
            assert bits(np.float32(X.fma(-ai, si, X.mul(bi, ci)))) == bits(yr[t, h, 32 + i])
    # a rotation: each pair keeps its length (up to rounding)
    n0 = a ** 2 + b ** 2
    n1 = yr[:, :, :32].astype(np.float64) ** 2 + yr[:, :, 32:].astype(np.float64) ** 2
    assert np.max(np.abs(n1 - n0) / n0) < 1e-5
    # head-major is the same values, [H][T][D]
    yh = orc.qk_prep(x, alpha, beta, c, s, cu, H, head_major=True)
    assert (bits(yh) == bits(yr.transpose(1, 0, 2))).all()
