"""CPU tests of the GGUF reader (include/nxg_gguf.h) on files written by nexterabert.cpp_amd/gguf_writer.py
from the published format: every metadata value type, tensor table and bytes, alignment,
the int8 placement of the reference's loader, and malformed files. No GPU work."""
from __future__ import annotations

import struct

import numpy as np
import pytest

from nexterabert_cpp_amd import gguf_writer as W


def f16_bytes(x):
    return np.asarray(x, np.float16).tobytes()


@pytest.fixture(scope="module")
def model_file(tmp_path_factory, nxg):
    """A NexteraBERT-shaped file: the hparams keys nextera_load reads
    (src/nexterabert.cpp:1562-1633) and one tensor of each kind."""
    rng = np.random.default_rng(0)
    path = tmp_path_factory.mktemp("gguf") / "model.gguf"
    mats = {}

    def quant(name, ttype, n_out, n_in):
        rows = (0.02 * rng.standard_normal((n_out, n_in))).astype(np.float32)
        data = nxg.quantize_weight(ttype, rows)
        mats[name] = (ttype, n_in, n_out, data.tobytes())
        return (name, ttype, (n_in, n_out), data.tobytes())

    tensors = [
        ("embedding.weight", nxg.TYPE_Q8_0, (256, 64), nxg.quantize_weight(nxg.TYPE_Q8_0,
         rng.standard_normal((64, 256)).astype(np.float32)).tobytes()),
        ("blocks.0.attn_norm.weight", nxg.TYPE_F32, (1024,), rng.standard_normal(1024).astype(np.float32).tobytes()),
        quant("blocks.0.attn.c_q.weight", nxg.TYPE_Q8_0, 1024, 1024),
        quant("blocks.0.mlp.c_fc.weight", nxg.TYPE_Q4_K, 2304, 1024),
        quant("blocks.0.mlp.c_proj.weight", nxg.TYPE_Q6_K, 1024, 2304),
        ("blocks.0.attn.c_gate.weight", nxg.TYPE_F16, (512, 8), f16_bytes(rng.standard_normal((8, 512)))),
        quant("blocks.0.attn.odd.weight", nxg.TYPE_Q8_0, 6, 256),         # ne1 % 4 != 0: not int8
    ]
    kvs = [
        ("general.architecture", W.STRING, "nexterabert"),
        ("general.file_type", W.UINT32, 15),
        ("nexterabert.vocab_size", W.UINT32, 50368),
        ("nexterabert.embedding_length", W.UINT32, 1024),
        ("nexterabert.block_count", W.UINT32, 2),
        ("nexterabert.rope.freq_base", W.FLOAT32, 100000.0),
        ("nexterabert.rms_norm_epsilon", W.FLOAT32, 1e-8),
        ("nexterabert.mlm_head", W.BOOL, True),
        ("nexterabert.block_types", W.ARRAY, (W.STRING, ["lily", "attn"])),
        ("tokenizer.ggml.cls_token_id", W.UINT32, 50281),
        ("test.u8", W.UINT8, 250), ("test.i8", W.INT8, -5), ("test.u16", W.UINT16, 65000),
        ("test.i16", W.INT16, -30000), ("test.i32", W.INT32, -2_000_000_000),
        ("test.u64", W.UINT64, 2 ** 40 + 3), ("test.i64", W.INT64, -(2 ** 50)),
        ("test.f64", W.FLOAT64, 0.1), ("test.empty", W.STRING, ""),
        ("test.utf8", W.STRING, "größe ✓"),
        ("test.arr_f32", W.ARRAY, (W.FLOAT32, [1.5, -2.25, 3e-8])),
        ("test.arr_u32", W.ARRAY, (W.UINT32, [1, 2, 4_000_000_000])),
        ("test.arr_bool", W.ARRAY, (W.BOOL, [True, False])),
        ("test.arr_empty", W.ARRAY, (W.INT32, [])),
    ]
    layout = W.write_gguf(path, kvs, tensors)
    return path, kvs, tensors, mats, layout


def test_metadata_round_trip(nxg, model_file):
    path, kvs, tensors, _, layout = model_file
    with nxg.GGUF(path) as g:
        assert g.version == 3 and g.alignment == 32 and g.data_offset == layout["data_offset"]
        assert g.keys() == [k for k, _, _ in kvs]
        assert g.get("general.architecture") == "nexterabert"
        assert g.get("nexterabert.vocab_size") == 50368
        assert g.get("nexterabert.rope.freq_base") == 100000.0
        assert g.get("nexterabert.rms_norm_epsilon") == float(np.float32(1e-8))
        assert g.get("nexterabert.mlm_head") is True
        assert g.get("nexterabert.block_types") == ["lily", "attn"]
        assert (g.get("test.u8"), g.get("test.i8"), g.get("test.u16"), g.get("test.i16")) == (250, -5, 65000, -30000)
        assert (g.get("test.i32"), g.get("test.u64"), g.get("test.i64")) == (-2_000_000_000, 2 ** 40 + 3, -(2 ** 50))
        assert g.get("test.f64") == 0.1 and g.get("test.empty") == "" and g.get("test.utf8") == "größe ✓"
        assert g.get("test.arr_f32") == [1.5, -2.25, float(np.float32(3e-8))]
        assert g.get("test.arr_u32") == [1, 2, 4_000_000_000]
        assert g.get("test.arr_bool") == [True, False] and g.get("test.arr_empty") == []
        assert g.get("missing.key", 7) == 7


def test_tensor_table_and_bytes(nxg, model_file):
    path, _, tensors, _, layout = model_file
    with nxg.GGUF(path) as g:
        infos = g.tensors()
        assert [t.name for t in infos] == [t[0] for t in tensors]
        for info, (name, ttype, ne, data), off in zip(infos, tensors, layout["offsets"]):
            assert info.type == ttype and info.n_dims == len(ne)
            assert info.ne == tuple(ne) + (1,) * (4 - len(ne))
            assert info.offset == off and info.offset % 32 == 0 and info.nbytes == len(data)
            assert g.tensor_bytes(name).tobytes() == data
        with pytest.raises(KeyError):
            g.tensor_bytes("nope")


def test_int8_placement_is_the_reference_rule(nxg, model_file):
    path, *_ = model_file
    with nxg.GGUF(path) as g:
        # embeddings stay plain; F32/F16 are not quantized types; ne1 % 4 != 0 is refused
        assert g.int8_names() == ["blocks.0.attn.c_q.weight", "blocks.0.mlp.c_fc.weight", "blocks.0.mlp.c_proj.weight"]


def test_expanded_bytes_match_the_direct_expansion(nxg, model_file):
    """The bytes the loader expands are the ones written: expansion from the file equals
    expansion of the original encoding."""
    path, _, _, mats, _ = model_file
    with nxg.GGUF(path) as g:
        for name, (ttype, n_in, n_out, data) in mats.items():
            if name not in g.int8_names():
                continue
            a = nxg.expand_weight(ttype, g.tensor_bytes(name), n_in, n_out)
            b = nxg.expand_weight(ttype, np.frombuffer(data, np.uint8), n_in, n_out)
            assert (a.w == b.w).all() and (a.scale.view(np.uint32) == b.scale.view(np.uint32)).all()


def test_custom_alignment_and_version_2(nxg, tmp_path):
    data = np.arange(96, dtype=np.float32).tobytes()
    for version, al in ((2, 64), (3, 256)):
        p = tmp_path / f"v{version}.gguf"
        lay = W.write_gguf(p, [("general.alignment", W.UINT32, al)],
                           [("a", 0, (24,), data), ("b", 0, (3, 4), data[:48])], version=version)
        with nxg.GGUF(p) as g:
            assert g.version == version and g.alignment == al
            assert g.data_offset == lay["data_offset"] and g.data_offset % al == 0
            assert [t.offset for t in g.tensors()] == [0, (len(data) + al - 1) // al * al] == lay["offsets"]
            assert g.tensor_bytes("b").tobytes() == data[:48]


def _good(tmp_path):
    p = tmp_path / "good.gguf"
    W.write_gguf(p, [("k", W.UINT32, 1)], [("t", 0, (8,), np.ones(8, np.float32).tobytes())])
    return p.read_bytes()


def _expect_error(nxg, tmp_path, blob, pattern):
    p = tmp_path / "bad.gguf"
    p.write_bytes(blob)
    with pytest.raises(ValueError, match=pattern):
        nxg.GGUF(p)


def test_malformed_files_are_refused(nxg, tmp_path):
    good = _good(tmp_path)
    _expect_error(nxg, tmp_path, b"GGML" + good[4:], "not a GGUF file")
    _expect_error(nxg, tmp_path, good[:4] + struct.pack("<I", 1) + good[8:], "unsupported GGUF version 1")
    _expect_error(nxg, tmp_path, good[:4] + struct.pack(">I", 3) + good[8:], "unsupported GGUF version")
    for cut in (20, 30, 45, 60, len(good) - 1):
        _expect_error(nxg, tmp_path, good[:cut], "truncated|too short|past the end|implausible")
    # a tensor whose data runs past the end of the file
    head, _ = W.header_and_table([], [("t", 0, (1024,), b"")], 32)
    _expect_error(nxg, tmp_path, head + b"\0" * 64, "past the end|larger than the file")
    # offset not a multiple of the alignment
    head, _ = W.header_and_table([], [("t", 0, (8,), b"")], 32)
    blob = bytearray(head)
    blob[-8:] = struct.pack("<Q", 4)
    _expect_error(nxg, tmp_path, bytes(blob) + b"\0" * 96, "not a multiple of the alignment")
    # unsupported tensor type, bad dimensions, duplicates, bad alignment key
    head, _ = W.header_and_table([], [("t", 99, (8,), b"")], 32)
    _expect_error(nxg, tmp_path, head + b"\0" * 64, "unsupported type 99")
    head, _ = W.header_and_table([], [("t", 0, (1, 2, 3, 4, 5), b"")], 32)
    _expect_error(nxg, tmp_path, head + b"\0" * 512, "5 dimensions")
    head, _ = W.header_and_table([("k", W.UINT32, 1), ("k", W.UINT32, 2)], [], 32)
    _expect_error(nxg, tmp_path, head + b"\0" * 32, "duplicate key 'k'")
    head, _ = W.header_and_table([], [("t", 0, (8,), b"\0" * 32), ("t", 0, (8,), b"\0" * 32)], 32)
    _expect_error(nxg, tmp_path, head + b"\0" * 128, "duplicate tensor 't'")
    head, _ = W.header_and_table([("general.alignment", W.UINT32, 48)], [], 32)
    _expect_error(nxg, tmp_path, head + b"\0" * 64, "power-of-two")
    with pytest.raises(ValueError, match="cannot open"):
        nxg.GGUF(tmp_path / "does_not_exist.gguf")


def test_metadata_type_errors(nxg, model_file):
    path, *_ = model_file
    L = nxg.load_library()
    with nxg.GGUF(path) as g:
        import ctypes
        i = L.nxg_gguf_find_key(g._h, b"general.architecture")
        v = ctypes.c_int64()
        assert L.nxg_gguf_get_i64(g._h, i, ctypes.byref(v)) == nxg.NXG_EINVAL
        assert b"not a number" in L.nxg_last_error()
        assert L.nxg_gguf_get_i64(g._h, 10 ** 6, ctypes.byref(v)) == nxg.NXG_EINVAL
        j = L.nxg_gguf_find_key(g._h, b"test.arr_u32")
        assert L.nxg_gguf_arr_i64(g._h, j, 3, ctypes.byref(v)) == nxg.NXG_EINVAL     # out of range
        assert L.nxg_gguf_find_tensor(g._h, b"nope") == -1


def test_weight_create_refuses_non_int8_tensors_before_device_work(nxg, model_file):
    path, *_ = model_file
    L = nxg.load_library()
    import ctypes
    with nxg.GGUF(path) as g:
        h = ctypes.c_void_p()
        for name in ("embedding.weight", "blocks.0.attn_norm.weight", "blocks.0.attn.odd.weight"):
            i = L.nxg_gguf_find_tensor(g._h, name.encode())
            assert L.nxg_gguf_weight_create(g._h, i, 1, ctypes.byref(h)) == nxg.NXG_EINVAL
            assert b"not an int8 linear weight" in L.nxg_last_error()
