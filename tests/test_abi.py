"""CPU tests of libnxg.so: exported symbols, argument checking before any device work,
the host half (load-time expansion, GGUF block decoders, placement rule), and the
model's linear inventory. No test here launches GPU work."""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
HEADERS = sorted((ROOT / "include").glob("*.h"))


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def declared_symbols():
    text = "".join(h.read_text() for h in HEADERS)
    return sorted(set(re.findall(r"NXG_API\s+[^;(]*?\b(nxg_\w+)\s*\(", text)))


def test_header_declares_the_path():
    names = declared_symbols()
    for n in ("nxg_quantize_rows", "nxg_linear_i8", "nxg_weight_create", "nxg_expand_weight",
              "nxg_weight_is_int8", "nxg_linear_i8_block_sums", "nxg_qact_export",
              "nxg_linear_i8_relu2_q8", "nxg_quantize_rows_relu2", "nxg_gguf_open", "nxg_gguf_weight_create"):
        assert n in names


def test_library_exports_every_declared_symbol(nxg):
    L = nxg.load_library()
    missing = [n for n in declared_symbols() if not hasattr(L, n)]
    assert not missing, missing


def test_library_exports_nothing_undeclared(nxg):
    import subprocess
    out = subprocess.run(["nm", "-D", "--defined-only", str(nxg.LIB_PATH)], capture_output=True, text=True).stdout
    exported = {l.split()[-1] for l in out.splitlines() if " T " in l and l.split()[-1].startswith("nxg_")}
    assert exported == set(declared_symbols())


def test_qact_sizes(nxg):
    L = nxg.load_library()
    assert L.nxg_qact_q_bytes(5, 96) == 16 * 128          # rows to 16, inputs to 64
    assert L.nxg_qact_sx_bytes(5, 96) == 16 * 1 * 4
    assert L.nxg_qact_q_bytes(65536, 2304) == 65536 * 2304
    assert L.nxg_qact_sx_bytes(65536, 2304) == 65536 * 9 * 4
    assert L.nxg_qact_q_bytes(5, 48) == 0 and L.nxg_qact_q_bytes(-1, 64) == 0


def test_arguments_checked_before_device_work(nxg):
    L = nxg.load_library()
    assert L.nxg_quantize_rows(None, 4, 48, 127, None, None, None) == nxg.NXG_EINVAL
    assert b"multiple of 32" in L.nxg_last_error()
    assert L.nxg_quantize_rows(None, 4, 64, 100, None, None, None) == nxg.NXG_EINVAL
    assert L.nxg_quantize_rows(None, -1, 64, 127, None, None, None) == nxg.NXG_EINVAL
    assert L.nxg_quantize_rows(None, 0, 64, 127, None, None, None) == nxg.NXG_OK      # nothing to do
    cu = (ctypes.c_int32 * 4)(0, 3, 3, 6)
    assert L.nxg_linear_i8(None, None, None, cu, 3, None, None, None) == nxg.NXG_EINVAL
    assert b"empty" in L.nxg_last_error()
    cu2 = (ctypes.c_int32 * 2)(1, 6)
    assert L.nxg_linear_i8(None, None, None, cu2, 1, None, None, None) == nxg.NXG_EINVAL
    assert L.nxg_linear_i8_rows(None, None, None, 4, None, None, None) == nxg.NXG_EINVAL
    w = np.zeros((4, 48), np.int8)
    s = np.zeros((1, 4), np.float32)
    h = ctypes.c_void_p()
    assert L.nxg_weight_create(w.ctypes.data, s.ctypes.data, 48, 4, ctypes.byref(h)) == nxg.NXG_EINVAL
    assert h.value is None
    # the split GEMM and the fused q/k/v preparation check their arguments first too
    cols = (ctypes.c_int32 * 2)(64, 64)
    assert L.nxg_linear_i8_rows_split(None, None, None, 4, 2, cols, None, None) == nxg.NXG_EINVAL
    assert L.nxg_linear_i8_rows_split(None, None, None, 4, 0, cols, None, None) == nxg.NXG_EINVAL
    assert L.nxg_qkv_prep(*([None] * 9), 1, None, 1, 4, 16, 8, 63, None, None, None, None) == nxg.NXG_EINVAL
    assert b"head_dim=63" in L.nxg_last_error()
    # RMSNorm's vector loads: x and gain must be 16-byte aligned (no pointer is dereferenced)
    assert L.nxg_rmsnorm_quantize_rows(4, 16, ctypes.c_float(1e-6), 16, 256, 127, 16, 16, None) == nxg.NXG_EINVAL
    assert b"aligned" in L.nxg_last_error()
    assert L.nxg_rmsnorm_quantize_rows(16, 16, ctypes.c_float(1e-6), 16, 256, 127, 20, 16, None) == nxg.NXG_EINVAL
    assert b"aligned" in L.nxg_last_error()
    # every quantizer and producer reads and writes 16 bytes per lane: misaligned buffers are refused
    assert L.nxg_quantize_rows(4, 16, 256, 127, 16, 16, None) == nxg.NXG_EINVAL
    assert b"aligned" in L.nxg_last_error()
    assert L.nxg_quantize_rows(16, 16, 256, 127, 16, 24, None) == nxg.NXG_EINVAL
    assert L.nxg_quantize_rows_relu2(16, 16, 256, 127, 8, 16, None) == nxg.NXG_EINVAL
    assert L.nxg_gate_quantize_rows(16, 36, 16, 256, 127, 16, 16, None) == nxg.NXG_EINVAL
    assert b"aligned" in L.nxg_last_error()
    assert L.nxg_gate_quantize_rows(16, 16, 16, 256, 127, 16, 4, None) == nxg.NXG_EINVAL
    assert b"aligned" in L.nxg_last_error()
    # attention's workspace: a size without memory, a negative size or a misaligned one is refused
    args = (None, None, None, None, 1, None, 8, 2, 1, -1, 8, None)
    assert L.nxg_attention_ws(*args, None, 64, None) == nxg.NXG_EINVAL
    assert L.nxg_attention_ws(*args, 16, -1, None) == nxg.NXG_EINVAL
    assert L.nxg_attention_ws(*args, 18, 64, None) == nxg.NXG_EINVAL
    assert b"workspace" in L.nxg_last_error()
    assert L.nxg_attention_workspace_bytes(8, 3, 2, 8) == nxg.NXG_EINVAL
    assert L.nxg_attention_workspace_bytes(0, 2, 1, 8) == 0


def test_gemm_kernel_name(nxg):
    """The launch plan's kernel choice on a 256-CU device, as the profiler names it: the
    encoder's shapes at 65,536 rows, few-row shapes, refusals."""
    k = lambda *a, **kw: nxg.gemm_kernel_name(*a, cus=256, **kw)
    assert k(65536, 1024, 2048) == "gemm_k256<false>"
    assert k(65536, 2304, 1024, residual=True) == "gemm_k256<true>"
    assert k(65536, 64, 1024, residual=True) == "gemm_kernel<true, false, false>"
    assert k(65536, 1024, 2304, relu2=True) == "gemm_relu2_rt<127, 4, false>"
    assert k(65536, 1024, 2304, relu2=True, act_max=63) == "gemm_relu2_rt<63, 4, false>"
    assert k(65536, 256, 512, relu2=True) == "gemm_relu2_rt<127, 1, false>"
    assert k(65536, 1024, 2304, relu2=True, f32_in=True) == "gemm_relu2_rt<127, 4, true>"
    assert k(65536, 256, 512, relu2=True, act_max=63, f32_in=True) == "gemm_relu2_rt<63, 1, true>"
    assert k(65536, 512, 2304, relu2=True, f32_in=True) == "gemm_relu2_q8<127>"      # after the quantize kernel
    assert k(16384, 1024, 2304, relu2=True, f32_in=True) == "gemm_relu2_rt<127, 4, true>"    # 4.5 tiles per workgroup
    assert k(8192, 1024, 2304, relu2=True, f32_in=True) == "gemm_relu2_rt<127, 4, false>"    # 2.25: quantize first
    assert k(65536, 512, 2304, relu2=True) == "gemm_relu2_q8<127>"
    assert k(65536, 2304, 1024, relu2=True, act_max=63) == "gemm_relu2_q8<63>"
    assert k(768, 1024, 2304, relu2=True) == "gemm_relu2_small<127>"     # 216 workgroups: one per CU
    assert k(1024, 1024, 2304, relu2=True) == "gemm_relu2_rt<127, 4, false>"    # 288 would be: the row tiles
    assert k(1024, 1024, 1024) == "gemm_fsk<64, 4, false>"               # 256 tiles of 64 x 64
    assert k(1024, 2304, 1024, residual=True) == "gemm_fsk<32, 9, true>"  # 9 blocks: 64 x 32 tiles
    assert k(1024, 1024, 3072) == "gemm_k256<false>"                      # 768 tiles: more than 2 per CU
    assert k(1024, 320, 1024) == "gemm_small<2, false, false>"           # n_in % 256 != 0
    assert k(1024, 320, 64, sums=True) == "gemm_kernel<false, true, false>"
    L = nxg.load_library()
    assert L.nxg_gemm_kernel_name(64, 1024, 2304, nxg.GEMM_RELU2 | nxg.GEMM_RESIDUAL, 256) is None
    assert L.nxg_gemm_kernel_name(64, 96, 2304, nxg.GEMM_RELU2, 256) is None      # n_in % 256
    assert L.nxg_gemm_kernel_name(64, 48, 64, 0, 256) is None
    assert L.nxg_gemm_kernel_name(64, 1024, 2304, nxg.GEMM_F32_IN, 256) is None     # fp32 input: relu^2 only
    assert L.nxg_gemm_kernel_name(0, 64, 64, 0, 256) is None


def test_device_calls_fail_loudly_without_gpu(nxg):
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    L = nxg.load_library()
    assert L.nxg_init() == nxg.NXG_EDEVICE
    with pytest.raises(RuntimeError):
        nxg.init()


# --- placement rule and row sizes --------------------------------------------------

def test_weight_is_int8_rule(nxg):
    f = nxg.weight_is_int8
    assert f("blocks.0.mlp.c_fc.weight", 2, nxg.TYPE_Q4_K, 1024, 2304)
    assert f("blocks.0.attn.ltc_conv.out_proj.weight", 2, nxg.TYPE_Q5_0, 64, 1024)
    assert not f("blocks.0.mlp.c_fc.weight", 2, nxg.TYPE_Q4_K, 1024, 2304, use_int8=False)
    assert not f("blocks.0.mlp.c_fc.weight", 2, nxg.TYPE_F32, 1024, 2304)      # not quantized
    assert not f("blocks.0.mlp.c_fc.weight", 2, nxg.TYPE_F16, 1024, 2304)
    assert not f("embedding.weight", 2, nxg.TYPE_Q8_0, 1024, 50368)
    assert not f("mlm.decoder.weight", 2, nxg.TYPE_Q8_0, 1024, 50368)
    assert not f("token_type_embeddings.weight", 2, nxg.TYPE_Q8_0, 1024, 4)
    assert not f("blocks.0.x.weight", 1, nxg.TYPE_Q8_0, 1024, 1)              # 1-D
    assert not f("blocks.0.x.weight", 2, nxg.TYPE_Q8_0, 1056 + 16, 8)         # ne0 % 32
    assert not f("blocks.0.x.weight", 2, nxg.TYPE_Q8_0, 1024, 6)              # ne1 % 4
    assert f("mlm.dense.weight", 2, nxg.TYPE_Q6_K, 1024, 1024)


def test_row_bytes(nxg):
    rb = nxg.row_bytes
    assert rb(nxg.TYPE_F32, 64) == 256 and rb(nxg.TYPE_F16, 64) == 128 and rb(nxg.TYPE_BF16, 64) == 128
    assert rb(nxg.TYPE_Q8_0, 1024) == 32 * 34 and rb(nxg.TYPE_Q4_0, 64) == 36 and rb(nxg.TYPE_Q4_1, 64) == 40
    assert rb(nxg.TYPE_Q5_0, 64) == 44 and rb(nxg.TYPE_Q5_1, 64) == 48
    assert rb(nxg.TYPE_Q2_K, 256) == 84 and rb(nxg.TYPE_Q3_K, 256) == 110 and rb(nxg.TYPE_Q4_K, 512) == 288
    assert rb(nxg.TYPE_Q5_K, 256) == 176 and rb(nxg.TYPE_Q6_K, 2304) == 9 * 210
    assert rb(nxg.TYPE_Q4_K, 64) == 0 and rb(99, 64) == 0


# --- block decoders, from hand-built blocks of the published formats -----------------

def f16(v):
    return np.array([v], np.float16).view(np.uint8)


def test_decode_q8_0_and_q4_0_q4_1(nxg):
    qs = np.arange(-16, 16, dtype=np.int8)
    blk = np.concatenate([f16(0.5), qs.view(np.uint8)])
    assert (nxg.dequantize_rows(nxg.TYPE_Q8_0, blk, 32, 1)[0] == 0.5 * qs).all()
    nib = np.arange(16, dtype=np.uint8)
    b4 = np.concatenate([f16(2.0), (nib | ((15 - nib) << 4)).astype(np.uint8)])
    y = nxg.dequantize_rows(nxg.TYPE_Q4_0, b4, 32, 1)[0]
    assert (y[:16] == 2.0 * (nib.astype(np.float32) - 8)).all()           # low nibbles: values 0..15
    assert (y[16:] == 2.0 * ((15 - nib).astype(np.float32) - 8)).all()    # high nibbles: values 16..31
    b41 = np.concatenate([f16(0.25), f16(-1.0), (nib | (nib << 4)).astype(np.uint8)])
    y = nxg.dequantize_rows(nxg.TYPE_Q4_1, b41, 32, 1)[0]
    assert (y[:16] == 0.25 * nib - 1.0).all() and (y[16:] == 0.25 * nib - 1.0).all()


def test_decode_q5_0_q5_1(nxg):
    nib = np.arange(16, dtype=np.uint8)
    qh = np.uint32(0xA5A50F0F)        # bit j: fifth bit of value j
    b = np.concatenate([f16(1.0), np.array([qh], "<u4").view(np.uint8), (nib | (nib << 4)).astype(np.uint8)])
    y = nxg.dequantize_rows(nxg.TYPE_Q5_0, b, 32, 1)[0]
    hb = np.array([(int(qh) >> j) & 1 for j in range(32)])
    q = np.concatenate([nib, nib]).astype(int) | (hb << 4)
    assert (y == (q - 16).astype(np.float32)).all()
    b1 = np.concatenate([f16(0.5), f16(2.0), np.array([qh], "<u4").view(np.uint8), (nib | (nib << 4)).astype(np.uint8)])
    y1 = nxg.dequantize_rows(nxg.TYPE_Q5_1, b1, 32, 1)[0]
    assert (y1 == 0.5 * q + 2.0).all()


def pack_scale_min_k4(sc, mn):
    """12 bytes holding 8 (6-bit scale, 6-bit min) pairs: pairs 0-3 in the low 6 bits of
    bytes 0-3 / 4-7; pairs 4-7 as nibbles of bytes 8-11 with their top 2 bits in the top
    2 bits of bytes 0-3 (scales) and 4-7 (mins)."""
    s = np.zeros(12, np.uint8)
    for j in range(8):
        if j < 4:
            s[j] |= sc[j] & 63
            s[j + 4] |= mn[j] & 63
        else:
            s[j + 4] = (sc[j] & 15) | ((mn[j] & 15) << 4)
            s[j - 4] |= (sc[j] >> 4) << 6
            s[j] |= (mn[j] >> 4) << 6
    return s


def test_decode_q4_k(nxg):
    sc = np.array([1, 2, 3, 63, 17, 40, 5, 33])
    mn = np.array([0, 1, 2, 3, 60, 7, 18, 63])
    q = (np.arange(256) * 7 % 16).astype(np.uint8)
    qs = np.zeros(128, np.uint8)
    for j in range(4):      # run j: 32 bytes; low nibbles are values 64j..64j+31, high nibbles 64j+32..
        qs[32 * j:32 * j + 32] = q[64 * j:64 * j + 32] | (q[64 * j + 32:64 * j + 64] << 4)
    blk = np.concatenate([f16(0.5), f16(0.25), pack_scale_min_k4(sc, mn), qs])
    y = nxg.dequantize_rows(nxg.TYPE_Q4_K, blk, 256, 1)[0]
    sub = np.arange(256) // 32
    expect = (np.float32(0.5) * sc[sub].astype(np.float32)) * q.astype(np.float32) - np.float32(0.25) * mn[sub].astype(np.float32)
    assert (bits(y) == bits(expect.astype(np.float32))).all()


def test_decode_q6_k(nxg):
    q = (np.arange(256) * 11 % 64).astype(np.int64)
    sc = np.arange(-8, 8, dtype=np.int8) * 3
    ql = np.zeros(128, np.uint8)
    qh = np.zeros(64, np.uint8)
    for h in range(2):        # each half of 128 values: runs of 32 in ql[64h..], qh[32h..]
        b = 128 * h
        for l in range(32):
            q1, q2, q3, q4 = q[b + l], q[b + l + 32], q[b + l + 64], q[b + l + 96]
            ql[64 * h + l] = (q1 & 15) | ((q3 & 15) << 4)
            ql[64 * h + l + 32] = (q2 & 15) | ((q4 & 15) << 4)
            qh[32 * h + l] = (q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4) | ((q4 >> 4) << 6)
    blk = np.concatenate([ql, qh, sc.view(np.uint8), f16(0.125)])
    y = nxg.dequantize_rows(nxg.TYPE_Q6_K, blk, 256, 1)[0]
    expect = (np.float32(0.125) * sc[np.arange(256) // 16].astype(np.float32)) * (q - 32).astype(np.float32)
    assert (bits(y) == bits(expect.astype(np.float32))).all()


def test_decode_q2_k_q3_k_structure(nxg):
    # Q2_K: scales byte (min << 4 | scale) per 16 values; 2-bit values 4 per byte
    q = (np.arange(256) % 4).astype(np.uint8)
    scb = np.array([(m << 4) | s for s, m in zip(range(1, 17), range(16))], np.uint8)
    qs = np.zeros(64, np.uint8)
    for half in range(2):
        for sh in range(4):
            for part in range(2):
                for l in range(16):
                    idx = 128 * half + 32 * sh + 16 * part + l
                    qs[32 * half + 16 * part + l] |= q[idx] << (2 * sh)
    blk = np.concatenate([scb, qs, f16(1.0), f16(0.5)])
    y = nxg.dequantize_rows(nxg.TYPE_Q2_K, blk, 256, 1)[0]
    sub = np.arange(256) // 16
    expect = (scb[sub] & 15).astype(np.float32) * q - np.float32(0.5) * (scb[sub] >> 4).astype(np.float32)
    assert (y == expect).all()
    # Q3_K: all high bits set -> value = 2-bit value; scales 6-bit biased by 32
    sc6 = (np.arange(16) * 4 + 1) % 64
    s12 = np.zeros(12, np.uint8)
    for j in range(16):
        low, high = sc6[j] & 15, sc6[j] >> 4
        if j < 8:
            s12[j] |= low
        else:
            s12[j - 8] |= low << 4
        s12[8 + (j & 3)] |= high << (2 * (j >> 2))
    blk3 = np.concatenate([np.full(32, 255, np.uint8), qs, s12, f16(1.0)])
    y3 = nxg.dequantize_rows(nxg.TYPE_Q3_K, blk3, 256, 1)[0]
    assert (y3 == (sc6[sub] - 32).astype(np.float32) * q).all()


def test_encoders_round_trip(nxg):
    rng = np.random.default_rng(0)
    x = (0.02 * rng.standard_normal((8, 1024))).astype(np.float32)
    for t, tol in ((nxg.TYPE_Q8_0, 0.006), (nxg.TYPE_Q6_K, 0.03), (nxg.TYPE_Q4_K, 0.12)):
        y = nxg.dequantize_rows(t, nxg.quantize_weight(t, x), 1024, 8)
        assert np.linalg.norm(y - x) / np.linalg.norm(x) < tol, t


# --- load-time expansion -------------------------------------------------------------

@pytest.mark.parametrize("wtype", [0, 1, 8, 12, 14])
@pytest.mark.parametrize("act_off", [128, 64])
def test_expand_weight_matches_oracle(nxg, orc, wtype, act_off):
    rng = np.random.default_rng(wtype + act_off)
    n_in, n_out = 1024, 36
    x = (0.02 * rng.standard_normal((n_out, n_in))).astype(np.float32)
    if wtype == 0:
        data = x.view(np.uint8).reshape(-1)
    elif wtype == 1:
        data = x.astype(np.float16).view(np.uint8).reshape(-1)
    else:
        data = nxg.quantize_weight(wtype, x)
    W = nxg.expand_weight(wtype, data, n_in, n_out, act_off=act_off, n_threads=3)
    rows = nxg.dequantize_rows(wtype, data, n_in, n_out)
    w, scale, off = orc.expand_rows(rows, act_off)
    assert (W.w == w).all() and (bits(W.scale) == bits(scale)).all() and (W.off == off).all()


def test_q8_0_decoder_matches_oracle(nxg, orc):
    x = (0.02 * np.random.default_rng(3).standard_normal((4, 256))).astype(np.float32)
    data = nxg.quantize_weight(nxg.TYPE_Q8_0, x)
    assert (bits(nxg.dequantize_rows(nxg.TYPE_Q8_0, data, 256, 4).reshape(-1))
            == bits(orc.dequant_q8_0(data, 1024))).all()


# --- the model's linears -------------------------------------------------------------

def test_model_linear_inventory(nxg):
    import nexterabert_cpp_amd.model as M
    lin = M.encoder_linears()
    assert len(lin) == 140                       # + mlm.dense = the 141 int8 linears of the file
    assert M.linear_ops_per_token() == 313_524_224
    groups = [g for l, k in enumerate(M.BLOCK_TYPES) for g in M.layer_groups(l, k)]
    assert len(groups) == 92
    assert sum(len(M.layer_groups(l, k, fuse=False)) for l, k in enumerate(M.BLOCK_TYPES)) == 140
    params = sum(s.n_in * s.n_out for s in lin)
    assert params == 160_956_416 - 1024 * 1024   # int8 weights of the file minus mlm.dense
    assert M.file_type_of("blocks.3.attn.c_v.weight", 1024, "Q4_K_M") == M.Q6_K
    assert M.file_type_of("blocks.3.attn.c_q.weight", 1024, "Q4_K_M") == M.Q4_K
    assert M.file_type_of("blocks.0.attn.ltc_conv.out_proj.weight", 64, "Q4_K_M") == M.Q5_0
