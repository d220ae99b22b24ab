"""The oracle's GGUF reader and ggml block decoders (oracle/ggml_blocks.py), CPU.

Three kinds of checks:
  - known-answer blocks packed here from ggml's published block layouts (ggml-common.h
    of ggml v0.9.9, the version the reference's CMakeLists.txt fetches) with values
    whose decoded floats are exact, so that a transposed nibble, a wrong run order or a
    misread scale field gives a different number;
  - random blocks (every bit pattern with a finite fp16 scale) decoded by the oracle and
    by the engine's separately written C decoders (nxg_dequantize_rows), bit for bit;
  - a GGUF file assembled byte by byte here, and a synthetic model file read by both the
    oracle's reader and the engine's.
Parity with ggml's own compiled decoders is not pinned beyond the layouts: ggml is not
vendored with the reference, and a build that contracts `d * q - m` into an fma would
differ in the last bit for the types with a min.
"""
import struct

import numpy as np
import pytest

from oracle import ggml_blocks as gb

F16 = np.float16


def h16(x: float) -> bytes:
    return np.array([x], F16).tobytes()


def _decode(t, raw, n):
    return gb.dequantize(t, bytes(raw), n)


# --- known answers -----------------------------------------------------------------------

def test_q8_0_known():
    q = np.arange(-128, 128, 8).astype(np.int8)            # 32 values
    raw = h16(0.5) + q.tobytes()
    np.testing.assert_array_equal(_decode(gb.Q8_0, raw, 32), q.astype(np.float32) * 0.5)


def test_q4_0_known():
    q = (np.arange(32) % 16) - 8                            # -8..7
    qs = bytes(((q[j] + 8) | ((q[j + 16] + 8) << 4)) for j in range(16))
    np.testing.assert_array_equal(_decode(gb.Q4_0, h16(0.25) + qs, 32), q.astype(np.float32) * 0.25)


def test_q5_0_and_q5_1_known():
    u = (np.arange(32) * 7) % 32                            # 0..31, every fifth bit pattern
    qh = sum(int(u[j] >> 4) << j for j in range(32))
    qs = bytes(((u[j] & 15) | ((u[j + 16] & 15) << 4)) for j in range(16))
    np.testing.assert_array_equal(_decode(gb.Q5_0, h16(2.0) + struct.pack("<I", qh) + qs, 32),
                                  (u - 16).astype(np.float32) * 2.0)
    np.testing.assert_array_equal(_decode(gb.Q5_1, h16(0.5) + h16(-3.0) + struct.pack("<I", qh) + qs, 32),
                                  u.astype(np.float32) * 0.5 - 3.0)


def _k4_scale_bytes(sc, mn):
    """12 bytes holding 8 six-bit (scale, min) pairs, as ggml's quantize_row_q4_K packs them."""
    b = bytearray(12)
    for j in range(8):
        if j < 4:
            b[j] = sc[j]
            b[j + 4] = mn[j]
        else:
            b[j + 4] = (sc[j] & 0x0F) | ((mn[j] & 0x0F) << 4)
            b[j - 4] |= (sc[j] >> 4) << 6
            b[j] |= (mn[j] >> 4) << 6
    return bytes(b)


def test_q4_k_known():
    sc = [8 * k + 5 for k in range(8)]                      # 5..61: top bits used by pairs 4..7
    mn = [63 - 8 * k for k in range(8)]
    d, dmin = 1.0 / 64, 1.0 / 128
    q = (np.arange(256) * 5) % 16                           # sub-block k = values 32k..32k+31
    qs = bytearray(128)
    for r in range(4):                                      # run r: low nibbles sub-block 2r, high 2r+1
        for l in range(32):
            qs[32 * r + l] = q[64 * r + l] | (q[64 * r + 32 + l] << 4)
    raw = h16(d) + h16(dmin) + _k4_scale_bytes(sc, mn) + bytes(qs)
    k = np.arange(256) // 32
    want = (np.array(sc)[k] * d) * q - np.array(mn)[k] * dmin       # exact in float32
    np.testing.assert_array_equal(_decode(gb.Q4_K, raw, 256), want.astype(np.float32))


def test_q5_k_known():
    sc = [61 - 7 * k for k in range(8)]
    mn = [3 + 8 * k for k in range(8)]
    d, dmin = 1.0 / 32, 1.0 / 256
    u = (np.arange(256) * 11) % 32
    ql, qh = bytearray(128), bytearray(32)
    for r in range(4):
        for l in range(32):
            lo, hi = u[64 * r + l], u[64 * r + 32 + l]
            ql[32 * r + l] = (lo & 15) | ((hi & 15) << 4)
            qh[l] |= ((lo >> 4) << (2 * r)) | ((hi >> 4) << (2 * r + 1))
    raw = h16(d) + h16(dmin) + _k4_scale_bytes(sc, mn) + bytes(qh) + bytes(ql)
    k = np.arange(256) // 32
    want = (np.array(sc)[k] * d) * u - np.array(mn)[k] * dmin
    np.testing.assert_array_equal(_decode(gb.Q5_K, raw, 256), want.astype(np.float32))


def test_q6_k_known():
    q = ((np.arange(256) * 13) % 64) - 32                   # -32..31
    sc = np.array([(-1) ** j * (j + 1) for j in range(16)], np.int8)   # scale of values 16j..16j+15
    d = 0.125
    ql, qh = bytearray(128), bytearray(64)
    for h in range(2):
        for i in range(32):
            u = [q[128 * h + 32 * k + i] + 32 for k in range(4)]       # 6-bit values of the 4 quarters
            ql[64 * h + i] = (u[0] & 15) | ((u[2] & 15) << 4)
            ql[64 * h + 32 + i] = (u[1] & 15) | ((u[3] & 15) << 4)
            qh[32 * h + i] = (u[0] >> 4) | ((u[1] >> 4) << 2) | ((u[2] >> 4) << 4) | ((u[3] >> 4) << 6)
    raw = bytes(ql) + bytes(qh) + sc.tobytes() + h16(d)
    want = (d * sc[np.arange(256) // 16].astype(np.float32)) * q
    np.testing.assert_array_equal(_decode(gb.Q6_K, raw, 256), want.astype(np.float32))


def test_q2_k_known():
    sc = [(s % 16) | ((15 - s % 16) << 4) for s in range(16)]          # scale, min nibbles
    u = (np.arange(256) * 3 + np.arange(256) // 7) % 4
    qs = bytearray(64)
    # value h*128 + 32p + 16part + l: byte h*32 + 16part + l, bits 2p; scale byte h*8 + 2p + part
    for v in range(256):
        h, r = divmod(v, 128)
        p, r = divmod(r, 32)
        part, l = divmod(r, 16)
        qs[32 * h + 16 * part + l] |= int(u[v]) << (2 * p)
    d, dmin = 0.5, 0.25
    raw = bytes(sc) + bytes(qs) + h16(d) + h16(dmin)
    s = np.array(sc)[(np.arange(256) // 128) * 8 + ((np.arange(256) % 128) // 32) * 2 + (np.arange(256) % 32) // 16]
    want = (d * (s & 15)).astype(np.float32) * u - (dmin * (s >> 4)).astype(np.float32)
    np.testing.assert_array_equal(_decode(gb.Q2_K, raw, 256), want.astype(np.float32))


def _q3_k_scales_ggml(s12: bytes) -> np.ndarray:
    """The 16 six-bit scales of a Q3_K block as ggml's dequantize_row_q3_K unpacks them:
    three 32-bit words, masks 0x03030303 / 0x0f0f0f0f, bytes of the four results."""
    a0, a1, tmp = struct.unpack("<III", s12)
    k1, k2 = 0x03030303, 0x0F0F0F0F
    aux = [(a0 & k2) | (((tmp >> 0) & k1) << 4), (a1 & k2) | (((tmp >> 2) & k1) << 4),
           ((a0 >> 4) & k2) | (((tmp >> 4) & k1) << 4), ((a1 >> 4) & k2) | (((tmp >> 6) & k1) << 4)]
    return np.frombuffer(struct.pack("<IIII", *aux), np.int8).astype(np.int32)


def test_q3_k_scales_match_ggml_word_form():
    rng = np.random.default_rng(3)
    for _ in range(200):
        s12 = rng.integers(0, 256, 12, dtype=np.uint8).tobytes()
        want = _q3_k_scales_ggml(s12) - 32
        raw = bytes(32) + bytes(64) + s12 + h16(1.0)       # hmask 0, q 0: value = -4 * scale
        got = _decode(gb.Q3_K, raw, 256)
        idx = (np.arange(256) // 128) * 8 + ((np.arange(256) % 128) // 32) * 2 + (np.arange(256) % 32) // 16
        np.testing.assert_array_equal(got, (want[idx] * -4).astype(np.float32))


def test_q3_k_known_values():
    # all scales 33 (biased: 1), d = 1: value = u - 4 unless its hmask bit is set
    s12 = bytes([0x11] * 8 + [0xAA] * 4)                    # low 4 bits 1, top 2 bits 2: 1 + 32 = 33
    u = (np.arange(256) * 5) % 4
    hbit = (np.arange(256) // 3) % 2
    qs, hm = bytearray(64), bytearray(32)
    for v in range(256):
        h, r = divmod(v, 128)
        p, r = divmod(r, 32)
        part, l = divmod(r, 16)
        qs[32 * h + 16 * part + l] |= int(u[v]) << (2 * p)
        hm[16 * part + l] |= int(hbit[v]) << (4 * h + p)
    raw = bytes(hm) + bytes(qs) + s12 + h16(1.0)
    want = (u - np.where(hbit == 1, 0, 4)).astype(np.float32)
    assert (_q3_k_scales_ggml(s12) == 33).all()
    np.testing.assert_array_equal(_decode(gb.Q3_K, raw, 256), want)


def test_float_types_known():
    x = np.array([0.0, -0.0, 1.5, -2.25, 65504.0, 6.1035156e-05, 5.9604645e-08, np.inf], np.float32)
    np.testing.assert_array_equal(_decode(gb.F16, x.astype(F16).tobytes(), 8), x)
    np.testing.assert_array_equal(_decode(gb.F32, x.tobytes(), 8), x)
    bf = (x.view(np.uint32) >> 16).astype(np.uint16)          # truncated: the top 16 bits
    np.testing.assert_array_equal(_decode(gb.BF16, bf.tobytes(), 8), (bf.astype(np.uint32) << 16).view(np.float32))
    assert _decode(gb.BF16, bf.tobytes(), 8)[4] == 65280.0


# --- against the engine's decoders -------------------------------------------------------

HALF_FIELDS = {gb.Q4_0: [0], gb.Q4_1: [0, 2], gb.Q5_0: [0], gb.Q5_1: [0, 2], gb.Q8_0: [0], gb.Q2_K: [80, 82],
               gb.Q3_K: [108], gb.Q4_K: [0, 2], gb.Q5_K: [0, 2], gb.Q6_K: [208]}


@pytest.mark.parametrize("t", sorted(gb.BLOCK))
def test_random_blocks_match_engine_decoders(nxg, t):
    rng = np.random.default_rng(100 + t)
    qk, nbytes = gb.BLOCK[t]
    nblk = 4096 // qk * 4
    b = rng.integers(0, 256, size=(nblk, nbytes), dtype=np.uint8)
    # finite scales: the top exponent bit of each fp16 (or bf16 / f32 value) cleared
    for p in HALF_FIELDS.get(t, []):
        b[:, p + 1] &= 0x3F
    if t in (gb.F16, gb.BF16):
        b[:, 1] &= 0x3F
    if t == gb.F32:
        b[:, 3] &= 0x3F
    n = nblk * qk
    mine = gb.dequantize(t, b.tobytes(), n)
    theirs = nxg.dequantize_rows(t, b.tobytes(), n, 1).reshape(-1)
    np.testing.assert_array_equal(mine.view(np.uint32), theirs.view(np.uint32))


# --- GGUF -----------------------------------------------------------------------------------

def _gguf_string(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def test_gguf_assembled_by_hand(tmp_path):
    """v3 file: 3 KV pairs (u32, string array, f32), two tensors at 64-byte alignment."""
    kv = (_gguf_string("general.alignment") + struct.pack("<II", 4, 64)
          + _gguf_string("x.names") + struct.pack("<IIQ", 9, 8, 2) + _gguf_string("a") + _gguf_string("bc")
          + _gguf_string("x.eps") + struct.pack("<If", 6, 0.25))
    t0 = np.arange(12, dtype=np.float32).reshape(3, 4)
    q8 = h16(0.5) + np.arange(-16, 16, dtype=np.int8).tobytes()          # one Q8_0 block
    infos = (_gguf_string("t0") + struct.pack("<IQQIQ", 2, 4, 3, gb.F32, 0)
             + _gguf_string("t1") + struct.pack("<IQIQ", 1, 32, gb.Q8_0, 64))
    head = b"GGUF" + struct.pack("<IQQ", 3, 2, 3) + kv + infos
    pad = (-len(head)) % 64
    body = t0.tobytes() + bytes(64 - t0.nbytes) + q8
    path = tmp_path / "hand.gguf"
    path.write_bytes(head + bytes(pad) + body)
    meta, tensors = gb.read_gguf(path)
    assert meta == {"general.alignment": 64, "x.names": ["a", "bc"], "x.eps": 0.25}
    (n0, ty0, ne0, r0), (n1, ty1, ne1, r1) = tensors
    assert (n0, ty0, ne0, n1, ty1, ne1) == ("t0", gb.F32, (4, 3), "t1", gb.Q8_0, (32,))
    np.testing.assert_array_equal(gb.dequantize(ty0, r0, 12).reshape(3, 4), t0)
    np.testing.assert_array_equal(gb.dequantize(ty1, r1, 32), np.arange(-16, 16, dtype=np.float32) * 0.5)


def test_gguf_synthetic_model_matches_engine_reader(nxg, tmp_path):
    path = tmp_path / "m.gguf"
    from nexterabert_cpp_amd import synth
    d = synth.Dims(n_vocab=300, n_embd=128, n_inter=256, n_head=2, n_kv_head=1, lily_rank=64, swa_window=8,
                   block_types=["lily", "swa", "attn", "hra"], n_types=2)
    synth.write_random_model(nxg, path, preset="Q4_K_M", seed=5, dims=d)
    meta, tensors = gb.read_gguf(path)
    with nxg.GGUF(path) as g:
        assert sorted(meta) == sorted(g.keys())
        for k, v in meta.items():
            w = g.get(k)
            if isinstance(v, float):
                assert np.float32(v) == np.float32(w), k
            else:
                assert v == w, k
        by_name = {t.name: t for t in g.tensors()}
        assert [n for n, *_ in tensors] == list(by_name)
        for name, t, ne, raw in tensors:
            info = by_name[name]
            assert t == info.type and ne == tuple(int(x) for x in info.ne[:info.n_dims])
            assert bytes(raw) == bytes(g.tensor_bytes(name))
