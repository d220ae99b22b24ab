"""GPU: the few-row GEMMs (gemm_fsk with 64 x 64 and 64 x 32 tiles, gemm_small with 32 x 32
and 32 x 64 pieces, gemm_relu2_small) give the reference's bits, and a sequence's rows are the
same whichever kernel a batch size selects.

The kernel is chosen per launch: for n_in % 256 == 0 and at most 9 blocks, gemm_fsk (one
wave per 256-input block) while its 64-row tiles number at most 2 per CU; else one-wave
pieces, 32 x 32 while they number at most 4 per CU, 32 x 64 while those do, else the
128 x 128 tiles; for c_fc -> relu^2 -> int8, the few-row kernel while its workgroups fit
one per CU. The shapes below are picked for MI355X's 256 CUs (noted per case); on another
device they still run, through whichever kernel it selects."""
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


def quant(nxg, torch, orc, x):
    qa = nxg.quantize_rows(torch.from_numpy(np.ascontiguousarray(x, np.float32)).cuda())
    q_ref, sx_ref = orc.quantize_rows(x)
    u8, _ = nxg.export_qact(qa)
    assert (u8.cpu().numpy() == q_ref).all()
    return qa, q_ref, sx_ref


def oracle_linear(orc, W, q_ref, sx_ref, res=None):
    simd = bool(orc.vnni_flavour()) and W.w.shape[1] % 32 == 0
    return orc.linear(W.w, W.scale, W.off, q_ref, sx_ref, res=res, simd=simd, n_threads=orc.default_threads())


# (T, n_in, n_out): route on 256 CUs
FEW_ROW_SHAPES = [
    (1000, 1024, 1024),   # gemm_fsk 64 x 64 tiles (256), 4 blocks
    (1000, 1024, 1000),   # gemm_fsk, last column tile partly past n_out
    (333, 768, 260),      # gemm_fsk, 3 blocks (a fold-only wave), ragged rows and columns
    (1000, 256, 1024),    # gemm_fsk, one block
    (300, 512, 520),      # gemm_fsk, 2 blocks, a last column tile of 8
    (700, 1280, 1000),    # gemm_fsk 64 x 32 tiles, 5 blocks
    (1000, 2304, 512),    # gemm_fsk 64 x 32 tiles, 9 blocks
    (2000, 1024, 1024),   # gemm_fsk, 512 tiles: 2 per CU
    (1000, 1024, 2048),   # gemm_fsk, 512 tiles
    (1000, 320, 1024),    # gemm_small 32 x 32, n_in % 256 != 0: last block of one k-step
    (1000, 2304, 2000),   # gemm_small 32 x 64, 9 blocks (1008 gemm_fsk tiles), last piece partly past n_out
    (1000, 96, 2048),     # gemm_small 32 x 64, one partial block of 2 k-steps
    (5, 64, 4),           # gemm_small, one piece, one k-step
    (1, 4096, 64),        # gemm_small, 16 blocks: the most whose sw the few-row kernels keep in LDS
    (100, 4352, 256),     # 17 blocks: the 128 x 128 kernel
]


@pytest.mark.parametrize("T,n_in,n_out", FEW_ROW_SHAPES)
def test_few_row_linear_matches_oracle(nxg, orc, torch, dev, T, n_in, n_out):
    say(f"few-row linear T={T} n_in={n_in} n_out={n_out}")
    rng = np.random.default_rng(5 * T + 3 * n_in + n_out)
    x = rng.standard_normal((T, n_in)).astype(np.float32)
    res = rng.standard_normal((T, n_out)).astype(np.float32)
    W = make_weight(nxg, rng, n_in, n_out)
    qa, q_ref, sx_ref = quant(nxg, torch, orc, x)
    dw = nxg.DeviceWeight(W)
    y = nxg.linear_i8(dw, qa).cpu().numpy()
    yr = nxg.linear_i8(dw, qa, residual=torch.from_numpy(res).cuda()).cpu().numpy()
    y_ref = oracle_linear(orc, W, q_ref, sx_ref)
    assert (bits(y) == bits(y_ref)).all()
    assert (bits(yr) == bits(oracle_linear(orc, W, q_ref, sx_ref, res=res))).all()


# (T, n_in, n_out) for c_fc -> relu^2 -> int8: route on 256 CUs
FEW_ROW_RELU2_SHAPES = [
    (1000, 1024, 2304),   # the MLP's c_fc at ~1k tokens: 1152 waves, few-row kernel
    (1000, 512, 320),     # few-row, the last 256-column block a quarter full (KSo = 5)
    (333, 2304, 1024),    # few-row, 9 blocks
    (3000, 1024, 2304),   # 3392 waves: the 128 x 256 kernel
]


@pytest.mark.parametrize("T,n_in,n_out", FEW_ROW_RELU2_SHAPES)
def test_few_row_relu2_q8(nxg, orc, torch, dev, T, n_in, n_out):
    rng = np.random.default_rng(7 * T + n_in + n_out)
    x = rng.standard_normal((T, n_in)).astype(np.float32)
    W = make_weight(nxg, rng, n_in, n_out, std=0.05)
    qa, q_ref, sx_ref = quant(nxg, torch, orc, x)
    dw = nxg.DeviceWeight(W)
    y_ref = oracle_linear(orc, W, q_ref, sx_ref)
    for act_max in (127, 63):
        say(f"few-row linear_relu2_q8 T={T} n_in={n_in} n_out={n_out} act_max={act_max}")
        fused = nxg.linear_i8_relu2_q8(dw, qa, act_max)
        two = nxg.quantize_rows_relu2(nxg.linear_i8(dw, qa), act_max)
        torch.cuda.synchronize()
        assert torch.equal(fused.q, two.q), "activation tiles (padding included) differ from the two-step path"
        assert torch.equal(fused.sx.view(torch.int32), two.sx.view(torch.int32)), "scales differ from the two-step path"
        r_ref, rsx_ref = orc.quantize_rows(orc.relu2(y_ref), act_max)
        u8, sx = nxg.export_qact(fused)
        assert (u8.cpu().numpy() == r_ref).all()
        assert (bits(sx.cpu().numpy()) == bits(rsx_ref)).all()


@pytest.mark.parametrize("n_out", [1024, 2048])
def test_sequence_same_bits_across_kernels(nxg, orc, torch, dev, n_out):
    """45 rows alone (a few-row kernel) and inside a 20,000-row batch (the 128 x 128
    kernel) give the same bits: outputs depend on a row's own inputs only."""
    say(f"sequence alone vs in a large batch, n_out={n_out}")
    rng = np.random.default_rng(n_out)
    n_in = 1024
    W = make_weight(nxg, rng, n_in, n_out)
    dw = nxg.DeviceWeight(W)
    seq = rng.standard_normal((45, n_in)).astype(np.float32)
    res = rng.standard_normal((45, n_out)).astype(np.float32)
    alone = nxg.linear_i8(dw, nxg.quantize_rows(torch.from_numpy(seq).cuda()),
                          residual=torch.from_numpy(res).cuda()).cpu().numpy()
    pre, post = 12_345, 20_000 - 12_345 - 45
    batch = np.concatenate([rng.standard_normal((pre, n_in)).astype(np.float32), seq,
                            rng.standard_normal((post, n_in)).astype(np.float32)])
    bres = np.concatenate([np.zeros((pre, n_out), np.float32), res, np.zeros((post, n_out), np.float32)])
    cu = nxg.cu_offsets_of([pre, 45, post])
    y = nxg.linear_i8(dw, nxg.quantize_rows(torch.from_numpy(batch).cuda()), cu_offsets=cu,
                      residual=torch.from_numpy(bres).cuda()).cpu().numpy()
    assert (bits(y[pre:pre + 45]) == bits(alone)).all()
    # and the fused relu^2 output likewise
    qa_alone = nxg.quantize_rows(torch.from_numpy(seq).cuda())
    qa_batch = nxg.quantize_rows(torch.from_numpy(batch).cuda())
    a = nxg.linear_i8_relu2_q8(dw, qa_alone)
    b = nxg.linear_i8_relu2_q8(dw, qa_batch, cu_offsets=cu)
    ua, sa = nxg.export_qact(a)
    ub, sb = nxg.export_qact(b)
    torch.cuda.synchronize()
    assert torch.equal(ua, ub[pre:pre + 45])
    sa_m = orc.sx_matrix(sa.cpu().numpy(), 45, n_out)
    sb_m = orc.sx_matrix(sb.cpu().numpy(), 20_000, n_out)
    assert (bits(sa_m) == bits(sb_m[pre:pre + 45])).all()
