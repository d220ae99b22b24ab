"""GPU parity of the int8 linear path against the CPU oracle (bit for bit).

int32 block sums, quantized activations, scales and fp32 outputs are compared by
bits: the engine's results must be the reference's exactly. Every case prints its
name, shape and seed before it touches the GPU.
"""
from __future__ import annotations

import glob
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

GOLDEN = sorted(glob.glob(os.path.join(os.path.dirname(__file__), "golden", "*.npz")))


def say(msg):
    print(msg, flush=True)


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def same_f32(a, b):
    """Bit equality, with any NaN equal to any NaN."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    na, nb = np.isnan(a), np.isnan(b)
    return bool((na == nb).all() and (bits(a)[~na] == bits(b)[~nb]).all())


@pytest.fixture(scope="module")
def torch():
    import torch as t
    assert t.cuda.is_available(), "no GPU"
    return t


@pytest.fixture(scope="module")
def dev(torch, nxg):
    nxg.init()
    return torch.device("cuda:0")


def gpu_quant(nxg, torch, x, act_max=127):
    qa = nxg.quantize_rows(torch.from_numpy(np.ascontiguousarray(x, np.float32)).cuda(), act_max)
    u8, sx = nxg.export_qact(qa)
    torch.cuda.synchronize()
    return qa, u8.cpu().numpy(), sx.cpu().numpy()


def make_weight(nxg, rng, n_in, n_out, wtype=8, std=0.02):
    rows = (std * rng.standard_normal((n_out, n_in))).astype(np.float32)
    data = nxg.quantize_weight(wtype, rows)
    return nxg.expand_weight(wtype, data, n_in, n_out)


# --- known-answer vectors -------------------------------------------------------

@pytest.mark.parametrize("path", GOLDEN, ids=lambda p: os.path.basename(p))
def test_golden_vectors_on_gpu(nxg, torch, dev, path):
    say(f"golden {os.path.basename(path)}")
    g = np.load(path)
    act_max = int(g["act_max"])
    qa, u8, sx = gpu_quant(nxg, torch, g["x"], act_max)
    assert (u8 == g["q"]).all()
    assert (bits(sx) == bits(g["sx"])).all()
    W = nxg.I8Weight(g["w8"], g["sw"], g["off"])
    dw = nxg.DeviceWeight(W)
    s = nxg.block_sums(dw, qa).cpu().numpy()
    assert (s == g["sums"]).all()
    y = nxg.linear_i8(dw, qa).cpu().numpy()
    yr = nxg.linear_i8(dw, qa, residual=torch.from_numpy(g["res"]).cuda()).cpu().numpy()
    assert (bits(y) == bits(g["y"])).all()
    assert (bits(yr) == bits(g["y_res"])).all()


# --- quantize -------------------------------------------------------------------

@pytest.mark.parametrize("T,n_in", [(1, 32), (15, 64), (16, 96), (17, 320), (100, 1024), (1000, 2304), (33, 4096)])
@pytest.mark.parametrize("act_max", [127, 63])
def test_quantize_matches_oracle(nxg, orc, torch, dev, T, n_in, act_max):
    say(f"quantize T={T} n_in={n_in} act_max={act_max}")
    rng = np.random.default_rng(T * 7 + n_in)
    x = (rng.standard_normal((T, n_in)) * np.exp(rng.standard_normal((T, 1)) * 4)).astype(np.float32)
    _, u8, sx = gpu_quant(nxg, torch, x, act_max)
    q_ref, sx_ref = orc.quantize_rows(x, act_max)
    assert (u8 == q_ref).all()
    assert (bits(sx) == bits(sx_ref)).all()


@pytest.mark.parametrize("act_max", [127, 63])
def test_quantize_special_values(nxg, orc, torch, dev, act_max):
    say(f"quantize specials act_max={act_max}")
    rng = np.random.default_rng(5)
    T, n_in = 96, 512 + 96
    x = rng.standard_normal((T, n_in)).astype(np.float32)
    specials = np.array([np.nan, np.inf, -np.inf, 0.0, -0.0, 1e-40, -1e-42, 3e38, -3e38, 1e-38], np.float32)
    for t in range(T):
        k = rng.integers(0, 6)
        x[t, rng.integers(0, n_in, k)] = specials[rng.integers(0, len(specials), k)]
    x[5] = 1e-41
    x[6] = 0.0
    x[7] = -0.0
    x[8] *= np.float32(1e-38)
    x[9, 255] = np.nan           # NaN last in its MAXPS lane: amax NaN
    x[10, 0] = np.nan            # NaN replaced by the next element of its lane
    x[11, 100] = 50.0
    x[11, 108] = np.nan          # NaN after the maximum in the same lane
    x[12, 3::8] = np.nan         # one lane all NaN
    _, u8, sx = gpu_quant(nxg, torch, x, act_max)
    q_ref, sx_ref = orc.quantize_rows(x, act_max)
    assert (u8 == q_ref).all()
    assert same_f32(sx, sx_ref)


def test_quantize_padding_is_zero(nxg, torch, dev):
    say("quantize padding T=5 n_in=96")
    T, n_in = 5, 96
    x = torch.randn(T, n_in, device="cuda")
    qa = nxg.qact_alloc(T, n_in)
    qa.q.fill_(0x55)
    qa.sx.fill_(7.0)
    nxg.quantize_rows(x, out=qa)
    q = qa.q.cpu().numpy().reshape(1, 2, 64, 16)      # 1 row group, KS = 2
    torch.cuda.synchronize()
    # rows 5..15 and inputs 96..127 are padding
    lanes = np.arange(64)
    rows, chunk = lanes % 16, lanes // 16
    for ks in range(2):
        for ln in range(64):
            k0 = ks * 64 + chunk[ln] * 16
            if rows[ln] >= T or k0 >= n_in:
                assert (q[0, ks, ln] == 0).all()
    sx = qa.sx.cpu().numpy()
    assert (sx[T:16] == 0).all()


# --- GEMM -----------------------------------------------------------------------

@pytest.mark.parametrize("T,n_in,n_out", [(1, 32, 4), (16, 64, 16), (37, 320, 100), (130, 1024, 260),
                                          (64, 2304, 1024), (200, 1024, 2304), (300, 96, 12)])
def test_block_sums_equal_int64_matmul(nxg, torch, dev, T, n_in, n_out):
    say(f"block_sums T={T} n_in={n_in} n_out={n_out}")
    rng = np.random.default_rng(T + n_in + n_out)
    x = rng.standard_normal((T, n_in)).astype(np.float32)
    W = make_weight(nxg, rng, n_in, n_out)
    qa, u8, _ = gpu_quant(nxg, torch, x)
    s = nxg.block_sums(nxg.DeviceWeight(W), qa).cpu().numpy()
    qs = u8.astype(np.int64) - 128
    for B in range((n_in + 255) // 256):
        sl = slice(B * 256, min(n_in, (B + 1) * 256))
        ref = qs[:, sl] @ W.w[:, sl].astype(np.int64).T
        assert (s[B] == ref).all(), f"block {B}"


@pytest.mark.parametrize("T,n_in,n_out", [(1, 1024, 4), (37, 320, 100), (128, 1024, 1024), (64, 2304, 1024),
                                          (257, 64, 1024), (300, 1024, 64), (129, 96, 12)])
def test_linear_matches_oracle(nxg, orc, torch, dev, T, n_in, n_out):
    say(f"linear T={T} n_in={n_in} n_out={n_out}")
    rng = np.random.default_rng(3 * T + n_in + 7 * n_out)
    x = rng.standard_normal((T, n_in)).astype(np.float32)
    res = rng.standard_normal((T, n_out)).astype(np.float32)
    W = make_weight(nxg, rng, n_in, n_out)
    qa, u8, sx = gpu_quant(nxg, torch, x)
    dw = nxg.DeviceWeight(W)
    y = nxg.linear_i8(dw, qa).cpu().numpy()
    yr = nxg.linear_i8(dw, qa, residual=torch.from_numpy(res).cuda()).cpu().numpy()
    q_ref, sx_ref = orc.quantize_rows(x)
    assert (u8 == q_ref).all()
    simd = bool(orc.vnni_flavour()) and n_in % 32 == 0
    y_ref = orc.linear(W.w, W.scale, W.off, q_ref, sx_ref, simd=simd, n_threads=8)
    yr_ref = orc.linear(W.w, W.scale, W.off, q_ref, sx_ref, res=res, simd=simd, n_threads=8)
    assert (bits(y) == bits(y_ref)).all()
    assert (bits(yr) == bits(yr_ref)).all()


def test_config1_single_linear(nxg, orc, torch, dev):
    """M=128, K=N=1024; weights N(0, 0.02) seed 0 -> Q8_0 -> int8; activations N(0, 1) seed 2."""
    say("config1 M=128 K=1024 N=1024")
    w = (0.02 * np.random.default_rng(0).standard_normal((1024, 1024))).astype(np.float32)
    x = np.random.default_rng(2).standard_normal((128, 1024)).astype(np.float32)
    W = nxg.expand_weight(nxg.TYPE_Q8_0, nxg.quantize_weight(nxg.TYPE_Q8_0, w), 1024, 1024)
    qa, u8, sx = gpu_quant(nxg, torch, x)
    dw = nxg.DeviceWeight(W)
    s = nxg.block_sums(dw, qa).cpu().numpy()
    y = nxg.linear_i8(dw, qa, cu_offsets=[0, 128]).cpu().numpy()
    q_ref, sx_ref = orc.quantize_rows(x)
    assert (u8 == q_ref).all() and (bits(sx) == bits(sx_ref)).all()
    assert (s == orc.block_sums(W.w, W.off, q_ref)).all()
    assert (bits(y) == bits(orc.linear(W.w, W.scale, W.off, q_ref, sx_ref))).all()
    # Tolerance cross-check against float64: the fp32 chain rounds each of the 4 block terms
    # twice and the running sum once per block, so its error is bounded by a few units of
    # 2^-24 of the sum of the terms' magnitudes (not of |y|, which can cancel to ~0).
    ref64 = np.zeros_like(y, dtype=np.float64)
    mag = np.zeros_like(y, dtype=np.float64)
    sxm = orc.sx_matrix(sx_ref, 128, 1024).astype(np.float64)
    for B in range(4):
        term = s[B].astype(np.float64) * sxm[:, B:B + 1] * W.scale[B].astype(np.float64)[None, :]
        ref64 += term
        mag += np.abs(term)
    assert np.max(np.abs(y - ref64) / np.maximum(mag, 1e-30)) < 1e-6


def test_batch_invariance(nxg, torch, dev):
    """A sequence's rows give the same bits alone and at any offset of a packed batch."""
    say("batch invariance")
    rng = np.random.default_rng(21)
    n_in, n_out = 1024, 300
    W = make_weight(nxg, rng, n_in, n_out)
    dw = nxg.DeviceWeight(W)
    seq = rng.standard_normal((45, n_in)).astype(np.float32)
    alone = nxg.linear_i8(dw, nxg.quantize_rows(torch.from_numpy(seq).cuda())).cpu().numpy()
    for pre in (0, 3, 16, 77, 130):
        other = rng.standard_normal((pre, n_in)).astype(np.float32)
        tail = rng.standard_normal((19, n_in)).astype(np.float32)
        batch = np.concatenate([other, seq, tail])
        cu = nxg.cu_offsets_of([n for n in (pre, 45, 19) if n > 0])
        y = nxg.linear_i8(dw, nxg.quantize_rows(torch.from_numpy(batch).cuda()), cu_offsets=cu).cpu().numpy()
        assert (bits(y[pre:pre + 45]) == bits(alone)).all(), f"offset {pre}"


def test_layer_config2(nxg, orc, torch, dev):
    """One attention layer's projections at T=512 (fused QKV, c_gate, c_proj+res, c_fc, mlp.c_proj+res)."""
    say("config2 T=512")
    import nexterabert_cpp_amd.model as M
    rng = np.random.default_rng(2)
    T = 512
    for g in M.layer_groups(9, "swa"):
        W = make_weight(nxg, rng, g.n_in, g.n_out)
        x = rng.standard_normal((T, g.n_in)).astype(np.float32)
        res = rng.standard_normal((T, g.n_out)).astype(np.float32) if g.residual else None
        qa, u8, sx = gpu_quant(nxg, torch, x)
        y = nxg.linear_i8(nxg.DeviceWeight(W), qa,
                          residual=torch.from_numpy(res).cuda() if res is not None else None).cpu().numpy()
        q_ref, sx_ref = orc.quantize_rows(x)
        y_ref = orc.linear(W.w, W.scale, W.off, q_ref, sx_ref, res=res, simd=bool(orc.vnni_flavour()), n_threads=8)
        assert (bits(y) == bits(y_ref)).all(), g.name


CFG3_LENGTHS = [977, 1056, 1551, 1948, 86, 309, 1689, 1944, 522, 649, 1782, 876, 571, 1698, 538, 847, 1324,
                1133, 190, 72, 1775, 1547, 1719, 1110, 1678, 686, 936, 1618, 267, 632, 268, 937]


def test_config3_lengths_pinned():
    lens = np.random.default_rng(1).integers(16, 2048, 32, endpoint=True)
    assert list(lens) == CFG3_LENGTHS and int(lens.sum()) == 32935


def test_ragged_batch_config3(nxg, orc, torch, dev):
    """32 documents packed into M=32,935 rows; Q4_K_M weights (Q4_K / Q6_K) expanded to int8.
    The oracle checks every sequence's first and last rows plus a random sample (rows are
    independent, so a row subset checks the full-size launch)."""
    say("config3 M=32935")
    import nexterabert_cpp_amd.model as M
    rng = np.random.default_rng(3)
    cu = nxg.cu_offsets_of(CFG3_LENGTHS)
    T = int(cu[-1])
    pick = np.unique(np.concatenate([cu[:-1], cu[1:] - 1, rng.choice(T, 256, replace=False)]))
    for g in M.layer_groups(9, "swa"):
        parts = [nxg.expand_weight(M.file_type_of(s.name, s.n_in, "Q4_K_M"),
                                   nxg.quantize_weight(M.file_type_of(s.name, s.n_in, "Q4_K_M"),
                                                       (0.02 * rng.standard_normal((s.n_out, s.n_in))).astype(np.float32)),
                                   s.n_in, s.n_out) for s in g.specs]
        W = nxg.I8Weight(np.concatenate([p.w for p in parts]), np.concatenate([p.scale for p in parts], 1),
                         np.concatenate([p.off for p in parts], 1))
        xd = torch.randn(T, g.n_in, device="cuda", generator=torch.Generator("cuda").manual_seed(7))
        resd = torch.randn(T, g.n_out, device="cuda") if g.residual else None
        y = nxg.linear_i8(nxg.DeviceWeight(W), nxg.quantize_rows(xd), residual=resd, cu_offsets=cu)
        torch.cuda.synchronize()
        x = xd.cpu().numpy()[pick]
        res = resd.cpu().numpy()[pick] if resd is not None else None
        q_ref, sx_ref = orc.quantize_rows(x)
        y_ref = orc.linear(W.w, W.scale, W.off, q_ref, sx_ref, res=res, simd=bool(orc.vnni_flavour()), n_threads=8)
        assert (bits(y.cpu().numpy()[pick]) == bits(y_ref)).all(), g.name


def test_long_context_rows_config5(nxg, orc, torch, dev):
    """M=65,536 rows through the largest projections; a row sample against the oracle and
    a second launch for determinism."""
    say("config5 M=65536")
    rng = np.random.default_rng(5)
    T = 65536
    for n_in, n_out, resid in ((1024, 2304, False), (2304, 1024, True)):
        W = make_weight(nxg, rng, n_in, n_out)
        dw = nxg.DeviceWeight(W)
        xd = torch.randn(T, n_in, device="cuda")
        resd = torch.randn(T, n_out, device="cuda") if resid else None
        qa = nxg.quantize_rows(xd)
        y1 = nxg.linear_i8(dw, qa, residual=resd, cu_offsets=[0, T])
        y2 = nxg.linear_i8(dw, qa, residual=resd)
        torch.cuda.synchronize()
        assert torch.equal(y1.view(torch.int32), y2.view(torch.int32))
        pick = np.unique(np.concatenate([[0, 1, T - 2, T - 1], rng.choice(T, 192, replace=False)]))
        x = xd.cpu().numpy()[pick]
        res = resd.cpu().numpy()[pick] if resd is not None else None
        q_ref, sx_ref = orc.quantize_rows(x)
        y_ref = orc.linear(W.w, W.scale, W.off, q_ref, sx_ref, res=res, simd=bool(orc.vnni_flavour()), n_threads=8)
        assert (bits(y1.cpu().numpy()[pick]) == bits(y_ref)).all()
        del xd, resd, qa, y1, y2


def test_builder_shares_quantized_input(nxg, orc, torch, dev):
    """builder::linear: linears that read one f32 tensor quantize it once."""
    say("builder qcache")
    rng = np.random.default_rng(8)
    Wq, Wk = make_weight(nxg, rng, 1024, 64), make_weight(nxg, rng, 1024, 32)
    b = nxg.Builder({"q": nxg.DeviceWeight(Wq), "k": nxg.DeviceWeight(Wk)})
    x = torch.from_numpy(rng.standard_normal((10, 1024)).astype(np.float32)).cuda()
    yq = b.linear("q", x)
    yk = b.linear("k", x)
    assert len(b.qcache) == 1
    q_ref, sx_ref = orc.quantize_rows(x.cpu().numpy())
    assert (bits(yq.cpu().numpy()) == bits(orc.linear(Wq.w, Wq.scale, Wq.off, q_ref, sx_ref))).all()
    assert (bits(yk.cpu().numpy()) == bits(orc.linear(Wk.w, Wk.scale, Wk.off, q_ref, sx_ref))).all()
    with pytest.raises(KeyError):
        b.linear("missing", x)


def test_bad_inputs_raise(nxg, torch, dev):
    say("bad inputs")
    W = nxg.DeviceWeight(make_weight(nxg, np.random.default_rng(0), 64, 8))
    qa = nxg.quantize_rows(torch.randn(6, 64, device="cuda"))
    with pytest.raises(ValueError):
        nxg.linear_i8(W, qa, cu_offsets=[0, 3, 3, 6])          # empty sequence
    with pytest.raises(ValueError):
        nxg.linear_i8(W, qa, cu_offsets=[0, 5])                # does not cover T
    with pytest.raises(ValueError):
        nxg.quantize_rows(torch.randn(6, 48, device="cuda"))   # n_in % 32
    with pytest.raises(ValueError):
        nxg.quantize_rows(torch.randn(6, 64, device="cuda"), act_max=100)
    with pytest.raises(ValueError):
        nxg.linear_i8(nxg.DeviceWeight(make_weight(nxg, np.random.default_rng(0), 128, 8)), qa)
