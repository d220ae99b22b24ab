"""GPU: one launch of a weight fused along n_out from several projections of the same input
(nxg_linear_i8_rows_split) writes each projection's columns to its own buffer with the bits
of a separate linear of that projection and of the oracle's linear (every row up to 1,024
rows, else a sample around the tile boundaries and at random), through the few-row kernels
and the 128 x 128 tiles; bad segment layouts are refused before any launch."""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


@pytest.fixture(scope="module")
def torch():
    import torch as t
    assert t.cuda.is_available(), "no GPU"
    return t


@pytest.fixture(scope="module")
def dev(torch, nxg):
    nxg.init()
    return torch.device("cuda:0")


def parts(nxg, rng, n_in, cols):
    out = []
    for i, c in enumerate(cols):
        rows = (0.02 * rng.standard_normal((c, n_in))).astype(np.float32)
        t = (8, 12, 14)[i % 3] if n_in % 256 == 0 else 8          # Q8_0, Q4_K, Q6_K
        out.append(nxg.expand_weight(t, nxg.quantize_weight(t, rows), n_in, c))
    return out


def fuse(nxg, ws):
    return nxg.I8Weight(w=np.concatenate([w.w for w in ws]), scale=np.concatenate([w.scale for w in ws], axis=1),
                        off=np.concatenate([w.off for w in ws], axis=1))


# (T, n_in, cols): the encoder's groups (lily in_proj | A | x_proj | B_proj, q | k | v, HRA
# qkv_in | qkv_gate | c_C) at few rows and at many, plus a last segment not a multiple of 64
SPLITS = [
    (1000, 1024, [64, 64, 1024, 1024]),
    (1024, 1024, [1024, 512, 512]),
    (8192, 1024, [1024, 512, 512]),
    (5000, 1024, [64, 64, 1024, 1024]),
    (300, 512, [128, 192]),
    (777, 256, [64, 60]),
    (3000, 256, [256]),
]


def rows_checked(rng, T):
    if T <= 1024:
        return np.arange(T)
    fixed = [0, 1, 127, 128, 255, 256, T - 129, T - 128, T - 2, T - 1]
    return np.unique(np.concatenate([fixed, rng.choice(T, 200, replace=False)]))


@pytest.mark.parametrize("T,n_in,cols", SPLITS)
def test_split_equals_separate_linears(nxg, orc, torch, dev, T, n_in, cols):
    say(f"linear_split T={T} n_in={n_in} cols={cols}")
    rng = np.random.default_rng(T + n_in + len(cols))
    ws = parts(nxg, rng, n_in, cols)
    fused = nxg.DeviceWeight(fuse(nxg, ws))
    x = torch.from_numpy(rng.standard_normal((T, n_in)).astype(np.float32)).cuda()
    qa = nxg.quantize_rows(x)
    outs = [torch.full((T, c), float("nan"), device="cuda") for c in cols]
    nxg.linear_i8_split(fused, qa, cols, outs=outs)
    torch.cuda.synchronize()
    pick = rows_checked(rng, T)
    q_ref, sx_ref = orc.quantize_rows(x.cpu().numpy()[pick])
    for k, w in enumerate(ws):
        ref = nxg.linear_i8(nxg.DeviceWeight(w), qa)
        torch.cuda.synchronize()
        got = outs[k].cpu().numpy()
        assert (bits(got) == bits(ref.cpu().numpy())).all(), f"segment {k}"
        y_ref = orc.linear(w.w, w.scale, w.off, q_ref, sx_ref, simd=bool(orc.vnni_flavour()), n_threads=8)
        assert (bits(got[pick]) == bits(y_ref)).all(), f"segment {k} against the oracle"


def test_split_refusals(nxg, torch, dev):
    rng = np.random.default_rng(3)
    qa = nxg.quantize_rows(torch.zeros(64, 1024, device="cuda"))
    w = nxg.DeviceWeight(fuse(nxg, parts(nxg, rng, 1024, [96, 96])))
    with pytest.raises(ValueError, match="multiples of 64"):
        nxg.linear_i8_split(w, qa, [96, 96])                   # boundary at 96
    with pytest.raises(ValueError, match="cover"):
        nxg.linear_i8_split(w, qa, [64, 64])                   # 128 of 192 columns
    w2 = nxg.DeviceWeight(fuse(nxg, parts(nxg, rng, 320, [64, 64])))
    with pytest.raises(ValueError, match="n_in % 256"):
        nxg.linear_i8_split(w2, nxg.quantize_rows(torch.zeros(64, 320, device="cuda")), [64, 64])
