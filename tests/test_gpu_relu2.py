"""GPU parity at shapes with many tiles, and of the fused c_fc -> relu^2 -> int8 path.

The fp32 GEMM is checked in full against the oracle at shapes of at least 256 tiles
(persistent workgroups walking several tiles each: full, ragged and partial tiles, one
and several 256-input blocks). The relu^2 output runs on 64 x 256 tiles over an
LDS-resident row tile (n_in 256 or 1024) or on 128 x 256 tiles; it is compared
bit for bit with the CPU oracle (linear, then relu^2, then quantize_row) and, raw buffers
with padding included, with the two-step GPU path (fp32 linear, then relu^2 quantize).
"""
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


# (T, n_in, n_out): at least 256 tiles of 128 x 128
LARGE_SHAPES = [(8192, 512, 1024),     # full tiles, 2 blocks
               (8000, 256, 1152),     # last row tile half, last column tile half
               (16384, 256, 512)]     # one block per tile (4 blocks: the relu^2 tests)


@pytest.mark.parametrize("T,n_in,n_out", LARGE_SHAPES)
def test_large_linear_matches_oracle(nxg, orc, torch, dev, T, n_in, n_out):
    say(f"large linear T={T} n_in={n_in} n_out={n_out}")
    rng = np.random.default_rng(T + n_in + n_out)
    x = rng.standard_normal((T, n_in)).astype(np.float32)
    res = rng.standard_normal((T, n_out)).astype(np.float32)
    W = make_weight(nxg, rng, n_in, n_out)
    qa, q_ref, sx_ref = quant(nxg, torch, orc, x)
    dw = nxg.DeviceWeight(W)
    y = nxg.linear_i8(dw, qa).cpu().numpy()
    yr = nxg.linear_i8(dw, qa, residual=torch.from_numpy(res).cuda()).cpu().numpy()
    y_ref = orc.linear(W.w, W.scale, W.off, q_ref, sx_ref, simd=bool(orc.vnni_flavour()),
                       n_threads=orc.default_threads())
    assert (bits(y) == bits(y_ref)).all()
    # y = res + f (src/nexterabert.cpp:957-958): one f32 add on the oracle-checked f
    assert (bits(yr) == bits(res + y_ref)).all()


@pytest.mark.parametrize("act_max", [127, 63])
def test_quantize_relu2_matches_oracle(nxg, orc, torch, dev, act_max):
    say(f"quantize_relu2 act_max={act_max}")
    rng = np.random.default_rng(21 + act_max)
    T, n_in = 333, 2304 + 32
    x = (rng.standard_normal((T, n_in)) * np.exp(rng.standard_normal((T, 1)) * 3)).astype(np.float32)
    specials = np.array([np.nan, np.inf, -np.inf, 0.0, -0.0, 1e-30, -1e-30, 2e19, -3e38], np.float32)
    for t in range(0, T, 3):
        k = rng.integers(1, 5)
        x[t, rng.integers(0, n_in, k)] = specials[rng.integers(0, len(specials), k)]
    x[4] = -1.0                      # whole row non-positive: amax 0
    qa = nxg.quantize_rows_relu2(torch.from_numpy(x).cuda(), act_max)
    u8, sx = nxg.export_qact(qa)
    q_ref, sx_ref = orc.quantize_rows(orc.relu2(x), act_max)
    assert (u8.cpu().numpy() == q_ref).all()
    assert (bits(sx.cpu().numpy()) == bits(sx_ref)).all()


# (T, n_in, n_out) for c_fc -> relu^2 -> int8; n_out % 32 == 0, n_in % 256 == 0
RELU2_SHAPES = [(20000, 1024, 2304),  # the MLP's c_fc, a 32-row last row tile, spans across row tiles
                (33000, 256, 1216),   # one block; a 40-row last row tile, 192-column last tile
                (4096, 1024, 2304),   # the MLP's c_fc, 4 blocks, 9 column tiles (64 x 256 row-tile kernel)
                (5000, 1024, 1216),   # row-tile kernel: a partial last row tile (8 rows), a 192-column last tile
                (20000, 1024, 320),   # row-tile kernel: spans that start inside a row tile, 2 column tiles
                (9000, 512, 1216),    # 2 blocks (128 x 256 kernel), ragged rows, a 192-column last tile
                (9000, 256, 1216),    # one block (row-tile kernel, its 1-block instance)
                (777, 512, 320),      # ragged rows, a 64-column last tile, KSo = 5
                (33, 256, 96),        # one row tile, n_out % 64 = 32
                (1, 1024, 256)]


@pytest.mark.parametrize("T,n_in,n_out", RELU2_SHAPES)
def test_linear_relu2_q8(nxg, orc, torch, dev, T, n_in, n_out):
    rng = np.random.default_rng(T * 3 + n_in + n_out)
    x = rng.standard_normal((T, n_in)).astype(np.float32)
    W = make_weight(nxg, rng, n_in, n_out, std=0.05)
    qa, q_ref, sx_ref = quant(nxg, torch, orc, x)
    dw = nxg.DeviceWeight(W)
    # the oracle: linear, relu^2, quantize_row
    y_ref = orc.linear(W.w, W.scale, W.off, q_ref, sx_ref, simd=bool(orc.vnni_flavour()),
                       n_threads=orc.default_threads())
    for act_max in (127, 63):
        say(f"linear_relu2_q8 T={T} n_in={n_in} n_out={n_out} act_max={act_max}")
        fused = nxg.linear_i8_relu2_q8(dw, qa, act_max)
        # two steps on the GPU: fp32 rows, then relu^2 + quantize
        two = nxg.quantize_rows_relu2(nxg.linear_i8(dw, qa), act_max)
        torch.cuda.synchronize()
        assert torch.equal(fused.q, two.q), "activation tiles (padding included) differ from the two-step path"
        assert torch.equal(fused.sx.view(torch.int32), two.sx.view(torch.int32)), "scales differ from the two-step path"
        r_ref, rsx_ref = orc.quantize_rows(orc.relu2(y_ref), act_max)
        u8, sx = nxg.export_qact(fused)
        assert (u8.cpu().numpy() == r_ref).all()
        assert (bits(sx.cpu().numpy()) == bits(rsx_ref)).all()


@pytest.mark.parametrize("lengths", [[300, 17, 1000, 129],       # few-row kernel
                                     [3000, 17, 5000, 129]])     # row-tile kernel; sequence 2 alone: few-row
def test_linear_relu2_q8_packed_batch(nxg, orc, torch, dev, lengths):
    say(f"linear_relu2_q8 with cu_offsets {lengths}")
    rng = np.random.default_rng(8)
    cu = nxg.cu_offsets_of(lengths)
    T, n_in, n_out = int(cu[-1]), 1024, 512
    x = rng.standard_normal((T, n_in)).astype(np.float32)
    W = make_weight(nxg, rng, n_in, n_out)
    qa, _, _ = quant(nxg, torch, orc, x)
    dw = nxg.DeviceWeight(W)
    a = nxg.linear_i8_relu2_q8(dw, qa, cu_offsets=cu)
    b = nxg.linear_i8_relu2_q8(dw, qa)
    torch.cuda.synchronize()
    assert torch.equal(a.q, b.q) and torch.equal(a.sx.view(torch.int32), b.sx.view(torch.int32))
    # each sequence alone gives the same rows
    s0, s1 = int(cu[2]), int(cu[3])
    qs, _, _ = quant(nxg, torch, orc, x[s0:s1])
    c = nxg.linear_i8_relu2_q8(dw, qs)
    uc, sc = nxg.export_qact(c)
    ua, sa = nxg.export_qact(a)
    torch.cuda.synchronize()
    assert torch.equal(uc, ua[s0:s1])
    n_blk = (n_out + 255) // 256
    sa_m = orc.sx_matrix(sa.cpu().numpy(), T, n_out)
    sc_m = orc.sx_matrix(sc.cpu().numpy(), s1 - s0, n_out)
    assert (bits(sa_m[s0:s1]) == bits(sc_m)).all() and sa_m.shape[1] == n_blk


@pytest.mark.parametrize("n_in,T,n_out", [(1024, 20000, 2304), (1024, 8200, 512), (512, 8200, 512)])
def test_linear_relu2_q8_overflowing_rows(nxg, orc, torch, dev, n_in, T, n_out):
    """Rows whose fp32 sums overflow: relu^2 gives +Inf, the row maximum is infinite and the
    quantization takes the reference's NaN path (x * 0 for the infinite values). Waves that
    hold such a row use the full CVTPS2DQ statement, the others the packed conversion; both
    against the oracle chain, on the many-row kernels (T >= 8192): the row-tile kernel
    (n_in 1024, at 20,000 x 2,304 and 8,200 x 512) and the 128 x 256 one (n_in 512)."""
    say(f"linear_relu2_q8 with overflowing rows, n_in={n_in} T={T} n_out={n_out}")
    rng = np.random.default_rng(11)
    x = rng.standard_normal((T, n_in)).astype(np.float32)
    x[5, :] *= np.float32(3e37)          # every block of the row: sums reach the fp32 limit
    x[4100, ::3] = np.float32(-2e38)     # a row of mixed signs in another tile
    x[8199, 17] = np.float32(3e38)       # the last, partial row tile
    W = make_weight(nxg, rng, n_in, n_out, std=0.05)
    qa, q_ref, sx_ref = quant(nxg, torch, orc, x)
    dw = nxg.DeviceWeight(W)
    y_ref = orc.linear(W.w, W.scale, W.off, q_ref, sx_ref, simd=bool(orc.vnni_flavour()),
                       n_threads=orc.default_threads())
    r = orc.relu2(y_ref)
    assert np.isinf(r).any(), "the case needs an infinite relu^2 value"
    for act_max in (127, 63):
        fused = nxg.linear_i8_relu2_q8(dw, qa, act_max)
        r_ref, rsx_ref = orc.quantize_rows(r, act_max)
        u8, sx = nxg.export_qact(fused)
        torch.cuda.synchronize()
        assert (u8.cpu().numpy() == r_ref).all(), f"act_max={act_max}"
        s = sx.cpu().numpy()
        assert ((bits(s) == bits(rsx_ref)) | (np.isnan(s) & np.isnan(rsx_ref))).all(), f"act_max={act_max}"


@pytest.mark.parametrize("n_in,T,n_out", [(1024, 20000, 2304), (1024, 8200, 512), (512, 8200, 512)])
def test_linear_relu2_q8_tiny_row_maxima(nxg, orc, torch, dev, n_in, T, n_out):
    """Rows whose relu^2 maximum is positive but below ACT_MAX / FLT_MAX (normal and
    denormal), so that inv = ACT_MAX / amax overflows to +Inf: the reference's CVTPS2DQ then
    gives 0x80000000 for every value of the row (u8 0). Rows are scaled by powers of two, which
    scale the quantized activations' sx and every fold step exactly, so the maxima land where
    chosen (2^-62: just above the bound, inv finite; 2^-64, 2^-65: normal maxima below it;
    2^-70: a denormal maximum; 2^-80: relu^2 underflows to 0). T >= 8192 keeps the many-row
    kernels (the row-tile one at n_in 1024, the 128 x 256 one at 512); checked against the
    oracle chain and against the two-step path."""
    say(f"linear_relu2_q8 with tiny row maxima, n_in={n_in} T={T} n_out={n_out}")
    rng = np.random.default_rng(12)
    x = rng.standard_normal((T, n_in)).astype(np.float32)
    scaled = {5: -62, 6: -65, 70: -64, 3000: -70, 3001: -62, 6000: -80, 8195: -65}
    for t, e in scaled.items():
        x[t] *= np.float32(2.0 ** e)
    W = make_weight(nxg, rng, n_in, n_out, std=0.05)
    qa, q_ref, sx_ref = quant(nxg, torch, orc, x)
    dw = nxg.DeviceWeight(W)
    y_ref = orc.linear(W.w, W.scale, W.off, q_ref, sx_ref, simd=bool(orc.vnni_flavour()),
                       n_threads=orc.default_threads())
    r = orc.relu2(y_ref)
    rmax = r[list(scaled)].max(axis=1)
    assert (rmax[[1, 2, 3, 6]] > 0).all() and (rmax[[1, 2, 3, 6]] < 63 / np.finfo(np.float32).max).all()
    assert rmax[3] < np.finfo(np.float32).tiny, "the case needs a denormal row maximum"
    assert rmax[0] > 127 / np.finfo(np.float32).max and rmax[5] == 0
    for act_max in (127, 63):
        fused = nxg.linear_i8_relu2_q8(dw, qa, act_max)
        two = nxg.quantize_rows_relu2(nxg.linear_i8(dw, qa), act_max)
        r_ref, rsx_ref = orc.quantize_rows(r, act_max)
        u8, sx = nxg.export_qact(fused)
        torch.cuda.synchronize()
        assert (r_ref[[6, 70, 3000, 8195]] == 0).all(), "the oracle maps these rows to u8 0"
        assert (u8.cpu().numpy() == r_ref).all(), f"act_max={act_max}"
        assert (bits(sx.cpu().numpy()) == bits(rsx_ref)).all(), f"act_max={act_max}"
        assert torch.equal(fused.q, two.q) and torch.equal(fused.sx.view(torch.int32), two.sx.view(torch.int32))


# (T, n_in, n_out) from fp32 rows: the row-tile kernel quantizing each row tile in LDS (n_in
# 1024 and 256, ragged last row tiles), and shapes that quantize into the workspace first
F32_SHAPES = [(20000, 1024, 2304),   # c_fc at 20k rows, fused (5.5 tiles per workgroup): a 32-row last row tile
              (40000, 256, 1216),    # one block, fused: a 192-column last tile
              (8250, 256, 1216),     # 1.3 tiles per workgroup: the rows quantized first
              (4100, 1024, 2304),
              (700, 1024, 2304),     # few rows: gemm_relu2_small after a quantization
              (9000, 512, 1216)]     # 2 blocks: the 128 x 256 kernel after a quantization


@pytest.mark.parametrize("T,n_in,n_out", F32_SHAPES)
def test_linear_f32_relu2_q8(nxg, orc, torch, dev, T, n_in, n_out):
    """nxg_linear_f32_relu2_q8_rows equals quantize_rows then linear_i8_relu2_q8, raw buffers
    with padding, bit for bit, on rows that take every branch of quantize_row: NaN (alone and
    among values), +-Inf, denormals, zero rows, maxima whose ACT_MAX / amax overflows, and
    ordinary rows; and the oracle chain on the rows without NaN."""
    rng = np.random.default_rng(T + n_in + 7 * n_out)
    x = rng.standard_normal((T, n_in)).astype(np.float32)
    special = {3: np.nan, 4: np.inf, 5: -np.inf, 6: 0.0, 7: 1e-40, 8: 3e-39, T - 1: np.nan}
    for t, v in special.items():
        if t in (6, 7, 8):
            x[t] = v
        else:
            x[t, 17] = v
    x[9, 200:] = np.float32(2.0 ** -126) * np.float32(0.25)       # a block of denormals after normal values
    x[10, :] *= np.float32(2.0 ** -130)                            # amax below ACT_MAX / FLT_MAX: inv overflows
    x[11, ::5] = np.float32(3e38)
    W = make_weight(nxg, rng, n_in, n_out, std=0.05)
    dw = nxg.DeviceWeight(W)
    xd = torch.from_numpy(x).cuda()
    for act_max in (127, 63):
        say(f"linear_f32_relu2_q8 T={T} n_in={n_in} n_out={n_out} act_max={act_max} "
            f"-> {nxg.gemm_kernel_name(T, n_in, n_out, relu2=True, act_max=act_max, f32_in=True)}")
        fused = nxg.linear_f32_relu2_q8(dw, xd, act_max)
        two = nxg.linear_i8_relu2_q8(dw, nxg.quantize_rows(xd, act_max), act_max)
        torch.cuda.synchronize()
        assert torch.equal(fused.q, two.q), "activation tiles (padding included) differ from quantize + GEMM"
        assert torch.equal(fused.sx.view(torch.int32), two.sx.view(torch.int32)), "scales differ from quantize + GEMM"
    # the oracle chain (act_max 127) on the rows without NaN or Inf
    q_ref, sx_ref = orc.quantize_rows(x)
    y_ref = orc.linear(W.w, W.scale, W.off, q_ref, sx_ref, simd=bool(orc.vnni_flavour()),
                       n_threads=orc.default_threads())
    r_ref, rsx_ref = orc.quantize_rows(orc.relu2(y_ref))
    fused = nxg.linear_f32_relu2_q8(dw, xd, 127)
    u8, sx = nxg.export_qact(fused)
    u8 = u8.cpu().numpy()
    sxm = orc.sx_matrix(sx.cpu().numpy(), T, n_out)
    rsm = orc.sx_matrix(rsx_ref, T, n_out)
    ok = np.isfinite(x).all(axis=1)
    assert (u8[ok] == r_ref[ok]).all()
    assert (bits(sxm[ok]) == bits(rsm[ok])).all()


def _f32_sweep_shapes():
    rng = np.random.default_rng(20261202)
    out = []
    for i in range(8):
        n_in = (256, 1024)[i % 2]
        n_out = 32 * int(rng.integers(8, 129))             # 256 .. 4,096, any multiple of 32
        T = int(rng.integers(12000, 70000))
        out.append((T, n_in, n_out, (127, 63)[(i // 2) % 2]))
    return out


@pytest.mark.parametrize("T,n_in,n_out,act_max", _f32_sweep_shapes())
def test_linear_f32_relu2_q8_sweep(nxg, torch, dev, T, n_in, n_out, act_max):
    """Seeded shapes (ragged row tiles, column tiles past n_out, fused or not by the workgroup
    count): nxg_linear_f32_relu2_q8 equals quantize_rows then linear_i8_relu2_q8 bit for bit,
    raw buffers with padding (that path is oracle-checked in the tests above)."""
    name = nxg.gemm_kernel_name(T, n_in, n_out, relu2=True, act_max=act_max, f32_in=True)
    say(f"linear_f32_relu2_q8 sweep T={T} n_in={n_in} n_out={n_out} act_max={act_max} -> {name}")
    g = torch.Generator(device="cuda")
    g.manual_seed(T + n_out)
    x = torch.randn(T, n_in, device="cuda", generator=g)
    rng = np.random.default_rng(T)
    dw = nxg.DeviceWeight(make_weight(nxg, rng, n_in, n_out, std=0.05))
    fused = nxg.linear_f32_relu2_q8(dw, x, act_max)
    two = nxg.linear_i8_relu2_q8(dw, nxg.quantize_rows(x, act_max), act_max)
    torch.cuda.synchronize()
    assert torch.equal(fused.q, two.q)
    assert torch.equal(fused.sx.view(torch.int32), two.sx.view(torch.int32))


@pytest.mark.parametrize("lengths,n_in", [([10000, 7000, 3000], 1024), ([5, 700, 33], 1024), ([30000, 12000], 256)])
def test_linear_f32_relu2_q8_packed(nxg, orc, torch, dev, lengths, n_in):
    """nxg_linear_f32_relu2_q8 over a packed batch (cu_offsets) equals the rows entry point on the
    same rows, bit for bit (fused and quantize-first sizes), and every row equals the oracle chain
    on a sample of rows."""
    rng = np.random.default_rng(sum(lengths) + n_in)
    cu = nxg.cu_offsets_of(lengths)
    T, n_out = int(cu[-1]), 2304
    say(f"linear_f32_relu2_q8 packed {lengths} n_in={n_in} -> "
        f"{nxg.gemm_kernel_name(T, n_in, n_out, relu2=True, f32_in=True)}")
    x = rng.standard_normal((T, n_in)).astype(np.float32)
    W = make_weight(nxg, rng, n_in, n_out, std=0.05)
    dw = nxg.DeviceWeight(W)
    xd = torch.from_numpy(x).cuda()
    packed = nxg.linear_f32_relu2_q8(dw, xd, 127, cu_offsets=cu)
    rows = nxg.linear_f32_relu2_q8(dw, xd, 127)
    torch.cuda.synchronize()
    assert torch.equal(packed.q, rows.q)
    assert torch.equal(packed.sx.view(torch.int32), rows.sx.view(torch.int32))
    pick = np.unique(np.concatenate([cu[:-1], cu[1:] - 1, rng.choice(T, 64, replace=False)]))
    q_ref, sx_ref = orc.quantize_rows(x[pick])
    y_ref = orc.linear(W.w, W.scale, W.off, q_ref, sx_ref, simd=bool(orc.vnni_flavour()),
                       n_threads=orc.default_threads())
    r_ref, rsx_ref = orc.quantize_rows(orc.relu2(y_ref))
    u8, sx = nxg.export_qact(packed)
    assert (u8.cpu().numpy()[pick] == r_ref).all()
    assert (bits(orc.sx_matrix(sx.cpu().numpy(), T, n_out)[pick]) == bits(orc.sx_matrix(rsx_ref, len(pick), n_out))).all()


@pytest.mark.parametrize("n_in_fc", [1024, 96])
def test_builder_mlp(nxg, orc, torch, dev, n_in_fc):
    """x + c_proj(relu(c_fc(h))^2): fused when n_in % 256 == 0, fp32 then quantize otherwise."""
    say(f"builder mlp n_in={n_in_fc}")
    rng = np.random.default_rng(n_in_fc)
    T, n_hidden = 400, 2304
    h = rng.standard_normal((T, n_in_fc)).astype(np.float32)
    x = rng.standard_normal((T, n_in_fc)).astype(np.float32)
    W_fc = make_weight(nxg, rng, n_in_fc, n_hidden)
    W_proj = make_weight(nxg, rng, n_hidden, n_in_fc)
    b = nxg.Builder({"fc": nxg.DeviceWeight(W_fc), "proj": nxg.DeviceWeight(W_proj)})
    y = b.mlp("fc", "proj", torch.from_numpy(h).cuda(), torch.from_numpy(x).cuda()).cpu().numpy()
    qh, sh = orc.quantize_rows(h)
    simd = bool(orc.vnni_flavour())
    u = orc.linear(W_fc.w, W_fc.scale, W_fc.off, qh, sh, simd=simd, n_threads=orc.default_threads())
    qr, sr = orc.quantize_rows(orc.relu2(u))
    y_ref = orc.linear(W_proj.w, W_proj.scale, W_proj.off, qr, sr, res=x, simd=simd, n_threads=orc.default_threads())
    assert (bits(y) == bits(y_ref)).all()


def test_relu2_q8_bad_shapes_raise(nxg, torch, dev):
    rng = np.random.default_rng(0)
    x = torch.randn(64, 96, device="cuda")
    qa = nxg.quantize_rows(x)
    dw = nxg.DeviceWeight(make_weight(nxg, rng, 96, 64))      # n_in % 256 != 0
    with pytest.raises(ValueError, match="n_in % 256"):
        nxg.linear_i8_relu2_q8(dw, qa)
    x2 = torch.randn(64, 256, device="cuda")
    dw2 = nxg.DeviceWeight(make_weight(nxg, rng, 256, 100))   # n_out % 32 != 0
    # the wrapper refuses to size such an output; the C entry point refuses the shape
    with pytest.raises(ValueError, match="multiple of 32"):
        nxg.linear_i8_relu2_q8(dw2, nxg.quantize_rows(x2))
    with pytest.raises(ValueError, match="n_out % 32"):
        nxg.linear_i8_relu2_q8(dw2, nxg.quantize_rows(x2), out=nxg.qact_alloc(64, 128))


@pytest.mark.parametrize("T,n_in", [(333, 1024), (100, 2304), (17, 32), (50, 96), (1, 4096),
                                    (1000, 256), (45, 512), (70, 2048), (4111, 1024), (8200, 1024)])
@pytest.mark.parametrize("act_max", [127, 63])
def test_rmsnorm_quantize_matches_oracle(nxg, orc, torch, dev, T, n_in, act_max):
    """op_rms_norm feeding an int8 linear: the oracle's RMSNorm (AVX2 dot order), then
    quantize_row; rows of very different scales, eps 1e-8 and 0, NaN/Inf/zero rows. n_in of
    whole 256-blocks up to 2,048 take the register-resident kernel, one workgroup per (16 rows,
    block) below 2 row groups per CU and one per 16 rows from there (8,200 rows on 256 CUs)."""
    say(f"rmsnorm_quantize T={T} n_in={n_in} act_max={act_max}")
    rng = np.random.default_rng(T + n_in + act_max)
    x = (rng.standard_normal((T, n_in)) * 10.0 ** rng.integers(-6, 6, (T, 1))).astype(np.float32)
    g = (1.0 + 0.2 * rng.standard_normal(n_in)).astype(np.float32)
    if T > 1000:
        x[-1, 9] = np.nan                # a NaN in the last row group only
    if T > 8:
        x[1] = 0.0                       # eps 0: inv = inf, 0 * inf = NaN everywhere
        x[2, 5] = np.nan
        x[3, 7] = np.inf
        x[4] = 1e-30                     # dot underflows to tiny values
        x[5, ::3] = -0.0
    for eps in (1e-8, 0.0):
        qa = nxg.rmsnorm_quantize_rows(torch.from_numpy(x).cuda(), torch.from_numpy(g).cuda(), eps, act_max)
        u8, sx = nxg.export_qact(qa)
        y = orc.rms_norm(x, g, eps)
        q_ref, sx_ref = orc.quantize_rows(y, act_max)
        assert (u8.cpu().numpy() == q_ref).all(), f"eps={eps}"
        s = sx.cpu().numpy()
        assert ((bits(s) == bits(sx_ref)) | (np.isnan(s) & np.isnan(sx_ref))).all(), f"eps={eps}"
