"""GPU: the mixers' producers quantized for an int8 consumer, bit for bit against the
oracle chain (the producer's rows, then quantize_row):

  op_gate        -> c_proj of the gated mixers      nxg_gate_quantize_rows
  op_dwconv      -> SnowLily ltc_conv.out_proj      nxg_dwconv_quantize_rows
  op_lily_state  -> SnowLily c_proj                 nxg_lily_state_quantize_rows
  op_block_mean  -> HRA c_q / c_k / c_v             nxg_block_mean_quantize_rows

over packed batches with one-row and short documents, k odd and even, and NaN / Inf /
huge / subnormal inputs."""
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


def cuda(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()


def check(nxg, orc, qa, rows_ref, act_max):
    u8, sx = nxg.export_qact(qa)
    q_ref, sx_ref = orc.quantize_rows(rows_ref, act_max)
    assert (u8.cpu().numpy() == q_ref).all(), "int8 activations differ"
    assert (bits(sx.cpu().numpy()) == bits(sx_ref)).all(), "scales differ"


def with_specials(rng, x, frac=0.01):
    x = x.copy()
    specials = np.array([np.nan, np.inf, -np.inf, 0.0, -0.0, 1e-40, -3e-39, 3e38, -2e38, 1e30], np.float32)
    n = max(1, int(frac * x.size))
    x.flat[rng.integers(0, x.size, n)] = specials[rng.integers(0, len(specials), n)]
    return x


LENGTHS = [1, 50, 7, 200, 3, 2]


@pytest.mark.parametrize("C", [64, 96, 1024])
@pytest.mark.parametrize("act_max", [127, 63])
def test_gate_quantize(nxg, orc, torch, dev, C, act_max):
    say(f"gate_quantize C={C} act_max={act_max}")
    rng = np.random.default_rng(C + act_max)
    T = 333
    g = (rng.standard_normal((T, C)) * np.exp(rng.uniform(-3, 4, (T, 1)))).astype(np.float32)
    y = (rng.standard_normal((T, C)) * np.exp(rng.uniform(-8, 8, (T, 1)))).astype(np.float32)
    g, y = with_specials(rng, g), with_specials(rng, y, 0.002)
    g[5] = 0.0                                    # sigmoid(0) = 1/2 exactly
    g[6] = 100.0                                  # sigmoid = 1
    qa = nxg.gate_quantize_rows(cuda(torch, g), cuda(torch, y), act_max)
    check(nxg, orc, qa, orc.gate(g, y), act_max)


@pytest.mark.parametrize("C,k", [(64, 5), (64, 4), (1024, 3), (96, 1)])
@pytest.mark.parametrize("with_r", [False, True])
def test_dwconv_quantize(nxg, orc, torch, dev, C, k, with_r):
    say(f"dwconv_quantize C={C} k={k} r={with_r}")
    rng = np.random.default_rng(C * 10 + k + with_r)
    cu = nxg.cu_offsets_of(LENGTHS)
    T = int(cu[-1])
    x = with_specials(rng, rng.standard_normal((T, C)).astype(np.float32), 0.001)
    r = rng.standard_normal((T, C)).astype(np.float32) if with_r else None
    taps = rng.standard_normal((k, C)).astype(np.float32)
    for act_max in (127, 63):
        qa = nxg.dwconv_quantize_rows(cuda(torch, x), cuda(torch, taps), cu,
                                      r=cuda(torch, r) if with_r else None, act_max=act_max)
        check(nxg, orc, qa, orc.dwconv(x, taps, cu, r), act_max)


@pytest.mark.parametrize("C,k", [(1024, 5), (64, 3), (96, 2)])
def test_lily_state_quantize(nxg, orc, torch, dev, C, k):
    say(f"lily_state_quantize C={C} k={k}")
    rng = np.random.default_rng(C + 7 * k)
    cu = nxg.cu_offsets_of(LENGTHS)
    T = int(cu[-1])
    a = rng.standard_normal((T, C)).astype(np.float32)
    x = with_specials(rng, rng.standard_normal((T, C)).astype(np.float32), 0.001)
    b = rng.standard_normal((T, C)).astype(np.float32)
    taps = rng.standard_normal((k, C)).astype(np.float32)
    for act_max in (127, 63):
        qa = nxg.lily_state_quantize_rows(cuda(torch, a), cuda(torch, x), cuda(torch, b), cuda(torch, taps), cu,
                                          act_max=act_max)
        check(nxg, orc, qa, orc.lily_state(a, x, b, taps, cu), act_max)


@pytest.mark.parametrize("block", [4, 3, 1])
@pytest.mark.parametrize("with_g", [True, False])
def test_block_mean_quantize(nxg, orc, torch, dev, block, with_g):
    say(f"block_mean_quantize block={block} g={with_g}")
    rng = np.random.default_rng(block * 2 + with_g)
    cu = nxg.cu_offsets_of(LENGTHS)
    T, C = int(cu[-1]), 1024
    h = with_specials(rng, rng.standard_normal((T, C)).astype(np.float32), 0.001)
    g = rng.standard_normal((T, C)).astype(np.float32) if with_g else None
    for act_max in (127, 63):
        qa = nxg.block_mean_quantize_rows(cuda(torch, h), cu, block, g=cuda(torch, g) if with_g else None,
                                          act_max=act_max)
        ref = orc.block_mean(h, cu, block, g)
        assert qa.T == ref.shape[0]
        check(nxg, orc, qa, ref, act_max)


def test_producers_batch_invariance(nxg, torch, dev):
    """A document gives the same int8 rows alone and inside a packed batch."""
    say("producers: document alone vs in a batch")
    rng = np.random.default_rng(99)
    C = 64
    cu = nxg.cu_offsets_of(LENGTHS)
    T = int(cu[-1])
    x, a, b = (rng.standard_normal((T, C)).astype(np.float32) for _ in range(3))
    taps = rng.standard_normal((5, C)).astype(np.float32)
    lo, hi = int(cu[3]), int(cu[4])
    full = nxg.export_qact(nxg.lily_state_quantize_rows(cuda(torch, a), cuda(torch, x), cuda(torch, b),
                                                        cuda(torch, taps), cu))[0]
    alone = nxg.export_qact(nxg.lily_state_quantize_rows(cuda(torch, a[lo:hi]), cuda(torch, x[lo:hi]),
                                                         cuda(torch, b[lo:hi]), cuda(torch, taps), [0, hi - lo]))[0]
    torch.cuda.synchronize()
    assert torch.equal(full[lo:hi], alone)
    full = nxg.export_qact(nxg.dwconv_quantize_rows(cuda(torch, x), cuda(torch, taps), cu))[0]
    alone = nxg.export_qact(nxg.dwconv_quantize_rows(cuda(torch, x[lo:hi]), cuda(torch, taps), [0, hi - lo]))[0]
    torch.cuda.synchronize()
    assert torch.equal(full[lo:hi], alone)


def test_producers_bad_arguments(nxg, torch, dev):
    say("producers: bad arguments")
    x = torch.zeros(4, 64, device="cuda")
    taps = torch.zeros(0, 64, device="cuda")
    with pytest.raises(ValueError):
        nxg.dwconv_quantize_rows(x, taps, [0, 4])                  # k = 0
    with pytest.raises(ValueError):
        nxg.gate_quantize_rows(x, torch.zeros(4, 32, device="cuda"))
    with pytest.raises(ValueError):
        nxg.block_mean_quantize_rows(x, [0, 3], 4)                 # offsets must end at T
    with pytest.raises(ValueError):
        nxg.gate_quantize_rows(torch.zeros(4, 48, device="cuda"), torch.zeros(4, 48, device="cuda"))  # n_in % 32


# --- the reference builder's int8 chains through the producers ------------------------

def _weights(nxg, rng, shapes):
    host, dev = {}, {}
    for name, (n_in, n_out) in shapes.items():
        rows = (0.05 * rng.standard_normal((n_out, n_in))).astype(np.float32)
        W = nxg.expand_weight(nxg.TYPE_Q8_0, nxg.quantize_weight(nxg.TYPE_Q8_0, rows), n_in, n_out)
        host[name], dev[name] = W, nxg.DeviceWeight(W)
    return host, dev


def _lin(orc, W, x, res=None):
    q, sx = orc.quantize_rows(x)
    simd = bool(orc.vnni_flavour()) and W.w.shape[1] % 32 == 0
    return orc.linear(W.w, W.scale, W.off, q, sx, res=res, simd=simd, n_threads=orc.default_threads())


def test_builder_gated_out(nxg, orc, torch, dev):
    """x + c_proj(sigmoid(c_gate(y)) * z) (src/nexterabert.cpp:1208-1213) against the oracle chain."""
    say("Builder.gated_out")
    rng = np.random.default_rng(41)
    C, pre = 256, "blocks.0.attn."
    host, devw = _weights(nxg, rng, {pre + "c_gate.weight": (C, C), pre + "c_proj.weight": (C, C)})
    cu = nxg.cu_offsets_of([100, 50])
    y, z, x = (rng.standard_normal((150, C)).astype(np.float32) for _ in range(3))
    b = nxg.Builder(devw)
    out = b.gated_out(pre, cuda(torch, y), cuda(torch, z), cuda(torch, x), cu_offsets=cu).cpu().numpy()
    gl = _lin(orc, host[pre + "c_gate.weight"], y)
    ref = _lin(orc, host[pre + "c_proj.weight"], orc.gate(gl, z), res=x)
    assert (bits(out) == bits(ref)).all()


def test_builder_lily(nxg, orc, torch, dev):
    """SnowLily's linears and producers (src/nexterabert.cpp:1231-1243) against the oracle chain."""
    say("Builder.lily")
    rng = np.random.default_rng(42)
    C, R, pre = 256, 64, "blocks.0.attn."
    shapes = {pre + "ltc_conv.in_proj.weight": (C, R), pre + "ltc_conv.A.weight": (C, R),
              pre + "ltc_conv.out_proj.weight": (R, C), pre + "x_proj.weight": (C, C),
              pre + "B_proj.weight": (C, C), pre + "c_proj.weight": (C, C)}
    host, devw = _weights(nxg, rng, shapes)
    lengths = [100, 3, 47]
    cu = nxg.cu_offsets_of(lengths)
    T = int(cu[-1])
    h, x = (rng.standard_normal((T, C)).astype(np.float32) for _ in range(2))
    ltc = rng.standard_normal((5, R)).astype(np.float32)
    st_taps = rng.standard_normal((3, C)).astype(np.float32)
    b = nxg.Builder(devw)
    out = b.lily(pre, cuda(torch, h), cuda(torch, x), cuda(torch, ltc), cuda(torch, st_taps), cu).cpu().numpy()
    W = lambda n: host[pre + n]
    z, r = _lin(orc, W("ltc_conv.in_proj.weight"), h), _lin(orc, W("ltc_conv.A.weight"), h)
    a = _lin(orc, W("ltc_conv.out_proj.weight"), orc.dwconv(z, ltc, cu, r))
    xp, bb = _lin(orc, W("x_proj.weight"), h), _lin(orc, W("B_proj.weight"), h)
    ref = _lin(orc, W("c_proj.weight"), orc.lily_state(a, xp, bb, st_taps, cu), res=x)
    assert (bits(out) == bits(ref)).all()


def test_builder_hra_block_qkv(nxg, orc, torch, dev):
    """HRA's block means -> c_q / c_k / c_v on block rows (src/nexterabert.cpp:1251-1256)."""
    say("Builder.hra_block_qkv")
    rng = np.random.default_rng(43)
    C, pre = 256, "blocks.0.attn."
    host, devw = _weights(nxg, rng, {pre + "c_q.weight": (C, C), pre + "c_k.weight": (C, 128),
                                     pre + "c_v.weight": (C, 128)})
    lengths = [9, 1, 30]
    cu = nxg.cu_offsets_of(lengths)
    T = int(cu[-1])
    ci, gt = (rng.standard_normal((T, C)).astype(np.float32) for _ in range(2))
    b = nxg.Builder(devw)
    q, k, v = (t.cpu().numpy() for t in b.hra_block_qkv(pre, cuda(torch, ci), cuda(torch, gt), cu, 4))
    hb = orc.block_mean(ci, cu, 4, gt)
    assert q.shape == (hb.shape[0], C) and hb.shape[0] == 3 + 1 + 8
    for got, n in ((q, "c_q.weight"), (k, "c_k.weight"), (v, "c_v.weight")):
        assert (bits(got) == bits(_lin(orc, host[pre + n], hb))).all(), n
