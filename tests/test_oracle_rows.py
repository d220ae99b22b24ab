"""CPU: pins of the oracle's fp32 row ops around the encoder's int8 linears.

  * upsample_add (src/nexterabert.cpp:675-690): each token row is its block row plus r, one
    fp32 addition (numpy float32 addition rounds the same way);
  * layer_norm (ggml_norm * w + b, :1290-1291): ggml is not in the reference's tree, so the
    order of its double sums is unpinned; pinned here: it is a LayerNorm (float64 within a
    few float ulps), w and b are applied as two separately rounded operations after the
    normalisation, a constant row gives exactly b, a row of +-a gives +-a / sqrt(a^2 + eps);
  * doc_mean (:1913-1925, :659-672): the document's rows summed one at a time in float32,
    times 1 / n; normalized, times 1 / sqrt(dot) with dot_f32's order (pinned against
    AVX2 by the RMSNorm tests): a unit vector along the sum, zero for a zero sum."""
from __future__ import annotations

import numpy as np


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def test_upsample_add_closed_form(orc):
    rng = np.random.default_rng(1)
    lens, block, C = [1, 4, 5, 9, 3], 4, 64
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    nb = [(n + block - 1) // block for n in lens]
    cub = np.concatenate([[0], np.cumsum(nb)])
    yb = rng.standard_normal((int(cub[-1]), C)).astype(np.float32)
    r = rng.standard_normal((int(cu[-1]), C)).astype(np.float32)
    out = orc.upsample_add(yb, r, cu, block)
    for d, n in enumerate(lens):
        for i in range(n):
            t = cu[d] + i
            assert (bits(out[t]) == bits(yb[cub[d] + i // block] + r[t])).all()


def test_layer_norm_is_layer_norm(orc):
    rng = np.random.default_rng(2)
    x = (rng.standard_normal((64, 1024)) * np.exp(rng.uniform(-5, 5, (64, 1))) + rng.normal(0, 3, (64, 1))).astype(np.float32)
    y = orc.layer_norm(x, eps=1e-5)
    xd = x.astype(np.float64)
    ref = (xd - xd.mean(1, keepdims=True)) / np.sqrt(xd.var(1, keepdims=True) + 1e-5)
    assert np.max(np.abs(y - ref)) < 4e-6 * max(1.0, np.max(np.abs(ref)))


def test_layer_norm_affine_and_closed_forms(orc):
    rng = np.random.default_rng(3)
    C = 96
    x = rng.standard_normal((8, C)).astype(np.float32)
    w = rng.uniform(0.5, 2, C).astype(np.float32)
    b = rng.standard_normal(C).astype(np.float32)
    y = orc.layer_norm(x, eps=1e-5)
    assert (bits(orc.layer_norm(x, w, b, 1e-5)) == bits((y * w) + b)).all()      # two roundings, in order
    assert (bits(orc.layer_norm(x, w, None, 1e-5)) == bits(y * w)).all()
    # a constant row: mean exact, v = 0 -> y = 0 -> out = b
    xc = np.full((1, C), 3.25, np.float32)
    assert (bits(orc.layer_norm(xc, w, b, 1e-5)[0]) == bits(np.float32(0) * w + b)).all()
    # +-a: mean 0, variance a^2 (exact), y = +-a * (1 / sqrt(a^2 + eps)) in float32
    a = np.float32(1.5)
    xa = np.tile(np.array([a, -a], np.float32), C // 2)[None, :]
    scale = np.float32(1.0) / np.sqrt(np.float32(a * a) + np.float32(1e-5))
    assert (bits(orc.layer_norm(xa, eps=1e-5)[0]) == bits(xa[0] * scale)).all()


def test_doc_mean_closed_forms(orc):
    rng = np.random.default_rng(4)
    lens, C = [1, 7, 30], 128
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    x = (rng.standard_normal((int(cu[-1]), C)) * 4).astype(np.float32)
    m = orc.doc_mean(x, cu)
    u = orc.doc_mean(x, cu, normalize=True)
    for d in range(len(lens)):
        acc = np.zeros(C, np.float32)
        for t in range(cu[d], cu[d + 1]):
            acc = acc + x[t]
        assert (bits(m[d]) == bits(acc * (np.float32(1) / np.float32(lens[d])))).all()
        nrm = np.linalg.norm(acc.astype(np.float64))
        assert abs(np.linalg.norm(u[d].astype(np.float64)) - 1.0) < 1e-6
        assert np.max(np.abs(u[d] - acc / nrm)) < 1e-6
        dot = np.float32(np.sum(acc.astype(np.float64) ** 2))
        # the scale is 1 / sqrtf(dot) for a dot within float rounding of the exact one
        s = u[d][acc != 0] / acc[acc != 0]
        assert np.allclose(s, np.float32(1) / np.sqrt(dot), rtol=2e-7, atol=0)
    z = orc.doc_mean(np.zeros((3, 32), np.float32), [0, 3], normalize=True)
    assert (bits(z) == 0).all()
