"""GPU: the int8 linear path captured once in a HIP graph and replayed gives the oracle's bits
on every replay: quantize_row -> linear (fp32 out), c_fc -> relu^2 -> int8 from a qact and from
fp32 rows (the row-tile kernel quantizing its own input rows), and c_proj + residual, at few rows
(every row checked) and at 16,400 rows (a row sample: rows are computed independently, so the
oracle runs on the sampled rows alone). Eager launches of the same entry points on other inputs
run between the replays, and the outputs are overwritten before each replay."""
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


def make_weight(nxg, rng, n_in, n_out, std=0.02):
    rows = (std * rng.standard_normal((n_out, n_in))).astype(np.float32)
    return nxg.expand_weight(8, nxg.quantize_weight(8, rows), n_in, n_out)


def rows_checked(rng, T):
    if T <= 1024:
        return np.arange(T)
    fixed = [0, 1, 63, 64, 255, 256, T - 65, T - 64, T - 2, T - 1]
    return np.unique(np.concatenate([fixed, rng.choice(T, 120, replace=False)]))


@pytest.mark.parametrize("T", [300, 16400])
def test_graph_replays_equal_oracle(nxg, orc, torch, dev, T):
    C, H = 1024, 2304
    rng = np.random.default_rng(T + 5)
    h = rng.standard_normal((T, C)).astype(np.float32)
    x = rng.standard_normal((T, C)).astype(np.float32)
    W_g, W_fc, W_pr = make_weight(nxg, rng, C, C), make_weight(nxg, rng, C, H), make_weight(nxg, rng, H, C)
    d_g, d_fc, d_pr = nxg.DeviceWeight(W_g), nxg.DeviceWeight(W_fc), nxg.DeviceWeight(W_pr)
    say(f"graph T={T}: {nxg.gemm_kernel_name(T, C, C)}, {nxg.gemm_kernel_name(T, C, H, relu2=True)}, "
        f"{nxg.gemm_kernel_name(T, C, H, relu2=True, f32_in=True)}, {nxg.gemm_kernel_name(T, H, C, residual=True)}")
    if T > 16000:
        assert nxg.gemm_kernel_name(T, C, H, relu2=True, f32_in=True).endswith("true>")
    hd, xd = torch.from_numpy(h).cuda(), torch.from_numpy(x).cuda()
    qa, ws = nxg.qact_alloc(T, C), nxg.qact_alloc(T, C)
    r, r2 = nxg.qact_alloc(T, H), nxg.qact_alloc(T, H)
    g = torch.empty(T, C, device="cuda")
    y = torch.empty(T, C, device="cuda")

    def step():
        nxg.quantize_rows(hd, out=qa)
        nxg.linear_i8(d_g, qa, out=g)
        nxg.linear_i8_relu2_q8(d_fc, qa, out=r)
        nxg.linear_f32_relu2_q8(d_fc, hd, out=r2, workspace=ws)
        nxg.linear_i8(d_pr, r2, residual=xd, out=y)

    # the oracle on the checked rows
    pick = rows_checked(rng, T)
    simd, nt = bool(orc.vnni_flavour()), orc.default_threads()
    q_ref, sx_ref = orc.quantize_rows(h[pick])
    g_ref = orc.linear(W_g.w, W_g.scale, W_g.off, q_ref, sx_ref, simd=simd, n_threads=nt)
    u = orc.linear(W_fc.w, W_fc.scale, W_fc.off, q_ref, sx_ref, simd=simd, n_threads=nt)
    r_ref, rsx_ref = orc.quantize_rows(orc.relu2(u))
    y_ref = orc.linear(W_pr.w, W_pr.scale, W_pr.off, r_ref, rsx_ref, res=x[pick], simd=simd, n_threads=nt)
    rsm = orc.sx_matrix(rsx_ref, len(pick), H)

    # warm up eagerly (and on a side stream, as capture does), then capture
    step()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    torch.cuda.synchronize()

    other = torch.randn(T, C, device="cuda")
    for rep in range(3):
        g.fill_(float("nan"))
        y.fill_(float("nan"))
        for a in (r, r2):
            a.q.fill_(0)
            a.sx.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        say(f"graph T={T}: replay {rep}")
        assert (bits(g.cpu().numpy()[pick]) == bits(g_ref)).all(), f"replay {rep}: fp32 linear"
        assert (bits(y.cpu().numpy()[pick]) == bits(y_ref)).all(), f"replay {rep}: c_proj + residual"
        for name, a in (("from a qact", r), ("from fp32 rows", r2)):
            u8, sx = nxg.export_qact(a)
            sxm = orc.sx_matrix(sx.cpu().numpy(), T, H)
            assert (u8.cpu().numpy()[pick] == r_ref).all(), f"replay {rep}: relu^2 int8 {name}"
            assert (bits(sxm[pick]) == bits(rsm)).all(), f"replay {rep}: relu^2 scales {name}"
        # eager launches of the same entry points on other inputs between replays
        qo = nxg.quantize_rows(other)
        nxg.linear_i8(d_g, qo)
        nxg.linear_f32_relu2_q8(d_fc, other)
        torch.cuda.synchronize()
