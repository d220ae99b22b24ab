"""A small GGUF writer: the published container format (version 3 by default),
little-endian. Makes synthetic model files (synth.py) for the reader in include/nxg_gguf.h.

    write_gguf(path, kvs, tensors, alignment=None, version=3)
      kvs      [(key, gguf_type, value)]; arrays as (GGUF_ARRAY, (elem_type, [values]))
      tensors  [(name, ggml_type, ne (tuple, ne[0] = row length), data bytes)]
"""
from __future__ import annotations

import struct

(UINT8, INT8, UINT16, INT16, UINT32, INT32, FLOAT32, BOOL, STRING, ARRAY, UINT64, INT64, FLOAT64) = range(13)

_FMT = {UINT8: "<B", INT8: "<b", UINT16: "<H", INT16: "<h", UINT32: "<I", INT32: "<i", FLOAT32: "<f",
        BOOL: "<?", UINT64: "<Q", INT64: "<q", FLOAT64: "<d"}


def _string(s) -> bytes:
    b = s.encode() if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


def _scalar(t: int, v) -> bytes:
    if t == STRING:
        return _string(v)
    return struct.pack(_FMT[t], v)


def encode_kv(key: str, t: int, v) -> bytes:
    out = _string(key) + struct.pack("<I", t)
    if t == ARRAY:
        et, vals = v
        out += struct.pack("<IQ", et, len(vals)) + b"".join(_scalar(et, x) for x in vals)
    else:
        out += _scalar(t, v)
    return out


def header_and_table(kvs, tensors, alignment: int, version: int = 3):
    """Bytes up to the data section, and each tensor's offset within it."""
    head = b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(kvs))
    head += b"".join(encode_kv(k, t, v) for k, t, v in kvs)
    offsets, pos = [], 0
    for name, ttype, ne, data in tensors:
        offsets.append(pos)
        pos += (len(data) + alignment - 1) // alignment * alignment
    for (name, ttype, ne, data), off in zip(tensors, offsets):
        head += _string(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", n) for n in ne)
        head += struct.pack("<IQ", ttype, off)
    return head, offsets


def write_gguf(path, kvs, tensors, alignment=None, version: int = 3) -> dict:
    al = 32
    for k, t, v in kvs:
        if k == "general.alignment":
            al = v
    if alignment is not None and alignment != al:
        raise ValueError("pass the alignment as the general.alignment key")
    head, offsets = header_and_table(kvs, tensors, al, version)
    data_start = (len(head) + al - 1) // al * al
    with open(path, "wb") as f:
        f.write(head)
        f.write(b"\0" * (data_start - len(head)))
        for (name, ttype, ne, data), off in zip(tensors, offsets):
            f.seek(data_start + off)
            f.write(bytes(data))
        end = data_start + (offsets[-1] + len(tensors[-1][3]) if tensors else 0)
        f.truncate(end)
    return {"data_offset": data_start, "offsets": offsets}
