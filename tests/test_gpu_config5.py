"""GPU: the long-context linear path's launches at their full size, M = 65,536 packed rows of
one document, each against the oracle on a sample of rows (rows are independent, so a sample
checks a full-size launch: every row tile position the sample hits, first and last rows
included), plus a second launch for determinism:

  * the MLP's c_fc -> relu^2 -> int8 (1,024 -> 2,304), the fused kernel of the step;
  * the projections that share an input, fused along n_out into one launch: QKV (1,024 ->
    1,024 + 512 + 512), SnowLily's in_proj / A / x_proj / B_proj (-> 64 + 64 + 1,024 + 1,024)
    and HRA's qkv_in / qkv_gate / c_C (-> 3 x 1,024);
  * HRA's q / k / v on the 16,384 block rows of the document;
  * attn.c_proj with its residual (1,024 -> 1,024) and SnowLily's out_proj (64 -> 1,024).
"""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

T = 65536


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


def make_weight(nxg, rng, n_in, n_out):
    rows = (0.02 * rng.standard_normal((n_out, n_in))).astype(np.float32)
    return nxg.expand_weight(8, nxg.quantize_weight(8, rows), n_in, n_out)


def concat(nxg, parts):
    return nxg.I8Weight(np.concatenate([p.w for p in parts]), np.concatenate([p.scale for p in parts], 1),
                        np.concatenate([p.off for p in parts], 1))


def sample(rng, rows):
    """First and last rows, both sides of every 128-row tile boundary near the ends, and a
    random sample."""
    fixed = [0, 1, 127, 128, 255, 256, rows - 129, rows - 128, rows - 2, rows - 1]
    return np.unique(np.concatenate([fixed, rng.choice(rows, 160, replace=False)]))


def oracle_linear(orc, W, x, res=None):
    q, sx = orc.quantize_rows(x)
    return orc.linear(W.w, W.scale, W.off, q, sx, res=res, simd=bool(orc.vnni_flavour()), n_threads=8)


def sx_of_rows(sx_flat, rows, n_blk):
    """Scales of `rows` from the [row/4][block][row%4] layout, as [len(rows)][n_blk]."""
    rows = np.asarray(rows)
    idx = ((rows[:, None] // 4) * n_blk + np.arange(n_blk)[None, :]) * 4 + rows[:, None] % 4
    return np.asarray(sx_flat)[idx]


def test_relu2_q8_full_size(nxg, orc, torch, dev):
    say("config5 relu2_q8 65536 x 1024 -> 2304")
    rng = np.random.default_rng(51)
    W = make_weight(nxg, rng, 1024, 2304)
    dw = nxg.DeviceWeight(W)
    xd = torch.randn(T, 1024, device="cuda", generator=torch.Generator("cuda").manual_seed(51))
    qa = nxg.quantize_rows(xd)
    r1 = nxg.linear_i8_relu2_q8(dw, qa)
    r2 = nxg.linear_i8_relu2_q8(dw, qa, cu_offsets=[0, T])
    torch.cuda.synchronize()
    assert torch.equal(r1.q, r2.q) and torch.equal(r1.sx.view(torch.int32), r2.sx.view(torch.int32))
    u8, sx = nxg.export_qact(r1)
    pick = sample(rng, T)
    y_ref = oracle_linear(orc, W, xd[torch.from_numpy(pick).cuda()].cpu().numpy())
    r_ref, rsx_ref = orc.quantize_rows(orc.relu2(y_ref))
    assert (u8[torch.from_numpy(pick).cuda()].cpu().numpy() == r_ref).all()
    nb = 2304 // 256
    got = sx_of_rows(sx.cpu().numpy(), pick, nb)
    want = sx_of_rows(rsx_ref, np.arange(pick.size), nb)
    assert (bits(got) == bits(want)).all()
    del xd, qa, r1, r2, u8, sx


SPLITS = {"qkv": [1024, 512, 512], "lily_in": [64, 64, 1024, 1024], "hra_in": [1024, 1024, 1024]}


@pytest.mark.parametrize("group,rows", [("qkv", T), ("lily_in", T), ("hra_in", T), ("qkv", T // 4)])
def test_fused_projections_full_size(nxg, orc, torch, dev, group, rows):
    cols = SPLITS[group]
    say(f"config5 split {group} {rows} x 1024 -> {cols}")
    rng = np.random.default_rng(len(group) + rows)
    parts = [make_weight(nxg, rng, 1024, c) for c in cols]
    W = concat(nxg, parts)
    dw = nxg.DeviceWeight(W)
    xd = torch.randn(rows, 1024, device="cuda", generator=torch.Generator("cuda").manual_seed(rows + len(cols)))
    qa = nxg.quantize_rows(xd)
    outs = nxg.linear_i8_split(dw, qa, cols)
    again = nxg.linear_i8_split(dw, qa, cols)
    torch.cuda.synchronize()
    pick = sample(rng, rows)
    pick_d = torch.from_numpy(pick).cuda()
    x = xd[pick_d].cpu().numpy()
    for k, (o, o2, part) in enumerate(zip(outs, again, parts)):
        assert torch.equal(o.view(torch.int32), o2.view(torch.int32)), f"segment {k} not deterministic"
        y_ref = oracle_linear(orc, part, x)
        assert (bits(o[pick_d].cpu().numpy()) == bits(y_ref)).all(), f"segment {k} ({cols[k]} columns) differs"
    del xd, qa, outs, again


@pytest.mark.parametrize("n_in,n_out,resid", [(1024, 1024, True), (64, 1024, False)])
def test_residual_and_lily_out_full_size(nxg, orc, torch, dev, n_in, n_out, resid):
    say(f"config5 linear {T} x {n_in} -> {n_out} residual={resid}")
    rng = np.random.default_rng(n_in + n_out)
    W = make_weight(nxg, rng, n_in, n_out)
    dw = nxg.DeviceWeight(W)
    xd = torch.randn(T, n_in, device="cuda", generator=torch.Generator("cuda").manual_seed(n_in))
    resd = torch.randn(T, n_out, device="cuda") if resid else None
    qa = nxg.quantize_rows(xd)
    y = nxg.linear_i8(dw, qa, residual=resd, cu_offsets=[0, T])
    torch.cuda.synchronize()
    pick = sample(rng, T)
    pick_d = torch.from_numpy(pick).cuda()
    res = resd[pick_d].cpu().numpy() if resid else None
    y_ref = oracle_linear(orc, W, xd[pick_d].cpu().numpy(), res)
    assert (bits(y[pick_d].cpu().numpy()) == bits(y_ref)).all()
    del xd, resd, qa, y
