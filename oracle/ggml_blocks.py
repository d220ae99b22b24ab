"""GGUF reading and ggml block decoding for the oracle (test infrastructure).

The oracle's own path from a model file to float tensors, independent of the engine's
GGUF reader and codecs: only tests, smoke() and the benchmark's CPU baseline use it.

The reference loads models through ggml (CMakeLists.txt fetches ggml at tag v0.9.9;
it is not vendored): gguf_init_from_file reads the file, and build_i8_weight
(src/nexterabert.cpp:1010-1049) turns each weight row into floats with ggml's to_float
for its type, the dequantize_row_* functions of ggml/src/ggml-quants.c, on the block
layouts of ggml/src/ggml-common.h. Those are restated here from the published formats,
vectorised over blocks with numpy, in float32 with one rounding per operation in
ggml's evaluation order (a compiler that fuses ggml's `d * q - m` into one fma would
round once less for the types with a min: Q4_1, Q5_1, Q2_K, Q4_K, Q5_K -- that
difference is not pinned here).
"""
from __future__ import annotations

import mmap
import struct
from pathlib import Path
from typing import Dict, List, Tuple

import numpy as np

# ggml_type values (ggml.h)
F32, F16, Q4_0, Q4_1, Q5_0, Q5_1, Q8_0 = 0, 1, 2, 3, 6, 7, 8
Q2_K, Q3_K, Q4_K, Q5_K, Q6_K = 10, 11, 12, 13, 14
BF16 = 30

# (values per block, bytes per block)
BLOCK = {F32: (1, 4), F16: (1, 2), BF16: (1, 2), Q4_0: (32, 18), Q4_1: (32, 20), Q5_0: (32, 22),
         Q5_1: (32, 24), Q8_0: (32, 34), Q2_K: (256, 84), Q3_K: (256, 110), Q4_K: (256, 144),
         Q5_K: (256, 176), Q6_K: (256, 210)}

f32 = np.float32


def _half(b: np.ndarray) -> np.ndarray:
    """Little-endian fp16 in two byte columns -> float32 (exact)."""
    return np.ascontiguousarray(b).view("<f2").astype(f32).reshape(-1)


def _blocks(raw, n: int, t: int) -> np.ndarray:
    qk, nbytes = BLOCK[t]
    if n % qk:
        raise ValueError(f"type {t}: {n} values are not whole blocks of {qk}")
    b = np.frombuffer(raw, np.uint8, count=(n // qk) * nbytes)
    return b.reshape(n // qk, nbytes)


def _nibbles(qs: np.ndarray) -> Tuple[np.ndarray, np.ndarray]:
    return (qs & 0x0F).astype(np.int32), (qs >> 4).astype(np.int32)


def _q4_0(b):      # d, qs[16]: value j = low nibble of byte j, value j + 16 = its high nibble
    d = _half(b[:, 0:2])[:, None]
    lo, hi = _nibbles(b[:, 2:18])
    return np.concatenate([(lo - 8).astype(f32) * d, (hi - 8).astype(f32) * d], axis=1)


def _q4_1(b):      # d, m, qs[16]; x * d + m
    d, m = _half(b[:, 0:2])[:, None], _half(b[:, 2:4])[:, None]
    lo, hi = _nibbles(b[:, 4:20])
    return np.concatenate([lo.astype(f32) * d + m, hi.astype(f32) * d + m], axis=1)


def _fifth_bits(qh_bytes: np.ndarray) -> np.ndarray:
    """qh as 32 bits, bit i = the fifth bit of value i."""
    qh = np.ascontiguousarray(qh_bytes).view("<u4").reshape(-1, 1)
    return ((qh >> np.arange(32, dtype=np.uint32)) & 1).astype(np.int32)


def _q5_0(b):      # d, qh (u32), qs[16]; q = (nibble | fifth bit << 4) - 16
    d = _half(b[:, 0:2])[:, None]
    h = _fifth_bits(b[:, 2:6])
    lo, hi = _nibbles(b[:, 6:22])
    q = np.concatenate([lo | (h[:, :16] << 4), hi | (h[:, 16:] << 4)], axis=1) - 16
    return q.astype(f32) * d


def _q5_1(b):      # d, m, qh, qs[16]; q * d + m
    d, m = _half(b[:, 0:2])[:, None], _half(b[:, 2:4])[:, None]
    h = _fifth_bits(b[:, 4:8])
    lo, hi = _nibbles(b[:, 8:24])
    q = np.concatenate([lo | (h[:, :16] << 4), hi | (h[:, 16:] << 4)], axis=1)
    return q.astype(f32) * d + m


def _q8_0(b):      # d, qs[32] (s8)
    d = _half(b[:, 0:2])[:, None]
    return b[:, 2:34].view(np.int8).astype(f32) * d


def _q2_k(b):
    """scales[16] (low nibble scale, high nibble min), qs[64], d, dmin. The 256 values are
    two halves of 128; in half h, 2-bit plane p (bits 2p..2p+1 of 32 bytes) gives values
    h*128 + 32p + i for byte i, with (scale, min) byte h*8 + 2p + i // 16."""
    nb = b.shape[0]
    sc = b[:, 0:16].astype(np.int32)
    d, dmin = _half(b[:, 80:82]).reshape(nb, 1, 1, 1, 1), _half(b[:, 82:84]).reshape(nb, 1, 1, 1, 1)
    qs = b[:, 16:80].reshape(nb, 2, 1, 32).astype(np.int32)                  # [half][.][byte]
    planes = (qs >> (2 * np.arange(4).reshape(1, 1, 4, 1))) & 3               # [half][plane][byte]
    s = sc.reshape(nb, 2, 4, 2, 1)                                            # [half][plane][part]
    dl = d * (s & 0x0F).astype(f32)
    ml = dmin * (s >> 4).astype(f32)
    v = planes.reshape(nb, 2, 4, 2, 16).astype(f32)
    return (dl * v - ml).reshape(nb, 256)


def _q3_k(b):
    """hmask[32], qs[64], scales[12] (16 six-bit scales, biased by 32), d. Value
    h*128 + 32p + i (i < 32): 2 bits from plane p of byte i of half h, minus 4 unless bit
    4h + p of hmask byte i is set; scale j = h*8 + 2p + i // 16."""
    nb = b.shape[0]
    d = _half(b[:, 108:110])[:, None, None, None, None]
    s = b[:, 96:108].astype(np.int32)
    j = np.arange(16)
    low = np.where(j < 8, s[:, j % 8] & 0x0F, s[:, j % 8] >> 4)               # scales 0-7 low nibbles, 8-15 high
    high = (s[:, 8 + (j % 4)] >> (2 * (j // 4))) & 3
    scales = ((low | (high << 4)) - 32).astype(f32)                           # [16]
    qs = b[:, 32:96].reshape(nb, 2, 1, 32).astype(np.int32)
    planes = (qs >> (2 * np.arange(4).reshape(1, 1, 4, 1))) & 3               # [half][plane][byte]
    hm = b[:, 0:32].astype(np.int32).reshape(nb, 1, 1, 32)
    bit = (hm >> (4 * np.arange(2).reshape(1, 2, 1, 1) + np.arange(4).reshape(1, 1, 4, 1))) & 1
    v = (planes - np.where(bit == 1, 0, 4)).reshape(nb, 2, 4, 2, 16).astype(f32)
    dl = d * scales.reshape(nb, 2, 4, 2, 1)
    return (dl * v).reshape(nb, 256)


def _k4_scales(s: np.ndarray) -> Tuple[np.ndarray, np.ndarray]:
    """The 8 (scale, min) pairs of 12 bytes (get_scale_min_k4): pairs 0-3 are the low 6
    bits of bytes 0-3 / 4-7; pairs 4-7 take 4 bits from bytes 8-11 (low / high nibble)
    and their top 2 bits from the top bits of bytes 0-3 / 4-7."""
    s = s.astype(np.int32)
    sc = np.concatenate([s[:, 0:4] & 63, (s[:, 8:12] & 0x0F) | ((s[:, 0:4] >> 6) << 4)], axis=1)
    mn = np.concatenate([s[:, 4:8] & 63, (s[:, 8:12] >> 4) | ((s[:, 4:8] >> 6) << 4)], axis=1)
    return sc.astype(f32), mn.astype(f32)


def _q4_k(b):
    """d, dmin, scales[12], qs[128]: 4 runs of 32 bytes, run r giving 64 values (low
    nibbles, sub-block 2r, then high nibbles, sub-block 2r + 1)."""
    nb = b.shape[0]
    d, dmin = _half(b[:, 0:2])[:, None], _half(b[:, 2:4])[:, None]
    sc, mn = _k4_scales(b[:, 4:16])
    dl, ml = (d * sc)[..., None], (dmin * mn)[..., None]                      # [8][1]
    q = b[:, 16:144].reshape(nb, 4, 32)
    v = np.stack([q & 0x0F, q >> 4], axis=2).reshape(nb, 8, 32).astype(f32)   # sub-block 2r, 2r+1
    return (dl * v - ml).reshape(nb, 256)


def _q5_k(b):
    """As Q4_K with qh[32] before qs: sub-block k's values add 16 where bit k of qh[i] is set."""
    nb = b.shape[0]
    d, dmin = _half(b[:, 0:2])[:, None], _half(b[:, 2:4])[:, None]
    sc, mn = _k4_scales(b[:, 4:16])
    dl, ml = (d * sc)[..., None], (dmin * mn)[..., None]
    qh = b[:, 16:48].astype(np.int32).reshape(nb, 1, 32)
    q = b[:, 48:176].reshape(nb, 4, 32).astype(np.int32)
    lo4 = np.stack([q & 0x0F, q >> 4], axis=2).reshape(nb, 8, 32)
    fifth = (qh >> np.arange(8).reshape(1, 8, 1)) & 1
    v = (lo4 + 16 * fifth).astype(f32)
    return (dl * v - ml).reshape(nb, 256)


def _q6_k(b):
    """ql[128], qh[64], scales[16] (s8), d. Half h (128 values): for byte i < 32 of its
    64 ql bytes and 32 qh bytes, values 32k + i (k = 0..3) take the low nibble of ql[i]
    (k = 0), of ql[32 + i] (k = 1), the high nibbles (k = 2, 3), with bits 2k..2k+1 of
    qh[i] on top, minus 32; scale 8h + 2k + i // 16; y = d * scale * q."""
    nb = b.shape[0]
    d = _half(b[:, 208:210])[:, None, None, None]
    ql = b[:, 0:128].reshape(nb, 2, 2, 32).astype(np.int32)                  # [half][lo/hi 32][byte]
    qh = b[:, 128:192].reshape(nb, 2, 1, 32).astype(np.int32)
    sc = b[:, 192:208].view(np.int8).astype(f32).reshape(nb, 2, 8)
    low4 = np.stack([ql[:, :, 0] & 0x0F, ql[:, :, 1] & 0x0F, ql[:, :, 0] >> 4, ql[:, :, 1] >> 4], axis=2)
    high2 = (qh >> (2 * np.arange(4).reshape(1, 1, 4, 1))) & 3
    q = ((low4 | (high2 << 4)) - 32).astype(f32)                              # [half][k][byte]
    s = np.stack([sc[:, :, 0:8:2], sc[:, :, 1:8:2]], axis=3)                  # [half][k][i // 16]
    s = np.repeat(s, 16, axis=3)                                              # [half][k][byte]
    return ((d * s) * q).reshape(nb, 256)


_DECODERS = {Q4_0: _q4_0, Q4_1: _q4_1, Q5_0: _q5_0, Q5_1: _q5_1, Q8_0: _q8_0, Q2_K: _q2_k, Q3_K: _q3_k,
             Q4_K: _q4_k, Q5_K: _q5_k, Q6_K: _q6_k}


def row_bytes(t: int, n: int) -> int:
    qk, nbytes = BLOCK[t]
    return (n // qk) * nbytes


def dequantize(t: int, raw, n: int) -> np.ndarray:
    """n values of ggml type t from their bytes (ggml's to_float), as float32."""
    if t == F32:
        return np.frombuffer(raw, "<f4", count=n).astype(f32)
    if t == F16:
        return np.frombuffer(raw, "<f2", count=n).astype(f32)
    if t == BF16:
        u = np.frombuffer(raw, "<u2", count=n).astype(np.uint32) << 16
        return u.view(f32)
    if t not in _DECODERS:
        raise ValueError(f"ggml type {t} is not decoded here")
    return np.ascontiguousarray(_DECODERS[t](_blocks(raw, n, t)), dtype=f32).reshape(-1)


# --- GGUF (v2, v3) ---------------------------------------------------------------------

_SCALAR = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?", 10: "<Q", 11: "<q", 12: "<d"}
GGUF_STRING, GGUF_ARRAY = 8, 9


class _Cursor:
    def __init__(self, buf):
        self.buf, self.pos = buf, 0

    def take(self, fmt: str):
        v = struct.unpack_from(fmt, self.buf, self.pos)[0]
        self.pos += struct.calcsize(fmt)
        return v

    def string(self) -> str:
        n = self.take("<Q")
        s = bytes(self.buf[self.pos:self.pos + n]).decode("utf-8", errors="surrogateescape")
        self.pos += n
        return s

    def value(self, vt: int):
        if vt == GGUF_STRING:
            return self.string()
        if vt == GGUF_ARRAY:
            et, n = self.take("<I"), self.take("<Q")
            return [self.value(et) for _ in range(n)]
        v = self.take(_SCALAR[vt])
        return float(v) if vt in (6, 12) else (bool(v) if vt == 7 else int(v))


def read_gguf(path) -> Tuple[Dict[str, object], List[Tuple[str, int, Tuple[int, ...], np.ndarray]]]:
    """Metadata and tensors of a GGUF file: (meta, [(name, ggml type, ne, raw bytes)])."""
    with open(Path(path), "rb") as fh:
        buf = mmap.mmap(fh.fileno(), 0, access=mmap.ACCESS_READ)
    c = _Cursor(buf)
    if bytes(buf[0:4]) != b"GGUF":
        raise ValueError(f"{path}: not a GGUF file")
    c.pos = 4
    version = c.take("<I")
    if version not in (2, 3):
        raise ValueError(f"{path}: GGUF version {version}")
    n_tensors, n_kv = c.take("<Q"), c.take("<Q")
    meta = {}
    for _ in range(n_kv):
        key = c.string()
        meta[key] = c.value(c.take("<I"))
    infos = []
    for _ in range(n_tensors):
        name = c.string()
        nd = c.take("<I")
        ne = tuple(c.take("<Q") for _ in range(nd))
        infos.append((name, ne, c.take("<I"), c.take("<Q")))
    align = int(meta.get("general.alignment", 32))
    data = (c.pos + align - 1) // align * align
    whole = np.frombuffer(buf, np.uint8)
    tensors = []
    for name, ne, t, off in infos:
        n = int(np.prod(ne))
        nbytes = row_bytes(t, int(ne[0])) * (n // int(ne[0]))
        tensors.append((name, t, ne, whole[data + off:data + off + nbytes]))
    return meta, tensors
