"""CPU: nxg_encoder_load's checks of a file's metadata (nextera_load's, src/nexterabert.cpp:
1557-1631, plus the GPU kernels' own: head_dim 64, widths multiples of 32), all made before
the GPU is touched; a valid file on a machine without the GPU fails with NXG_EDEVICE."""
from __future__ import annotations

import numpy as np
import pytest


@pytest.fixture(scope="module")
def synth(nxg):
    from nexterabert_cpp_amd import synth as S
    return S


def write(nxg, synth, path, meta_edit=None, type_of=None, **dims):
    d = synth.Dims(n_vocab=100, n_embd=128, n_inter=256, n_head=2, n_kv_head=1, lily_rank=64,
                   block_types=["lily", "attn"], **dims)
    import nexterabert_cpp_amd.gguf_writer as W
    t = synth.model_tensors(d, seed=0)
    meta = synth.metadata(d, "Q8_0")
    if meta_edit:
        meta = meta_edit(meta)
    entries = []
    for name in sorted(t):
        ty = (type_of or {}).get(name, synth.file_type_of(name, t[name], "Q8_0"))
        ne = tuple(reversed(t[name].shape)) if t[name].ndim == 2 else (t[name].size,)
        data = (np.ascontiguousarray(t[name], np.float16).tobytes() if ty == synth.F16
                else synth.encode_tensor(nxg, t[name], ty))
        entries.append((name, ty, ne, data))
    W.write_gguf(path, meta, entries)
    return path


def load_error(nxg, path):
    with pytest.raises((ValueError, nxg.NxgError)) as ei:
        nxg.Encoder(path)
    return ei


def replace(meta, key, t, v):
    return [(k, t, v) if k == key else (k, tt, vv) for k, tt, vv in meta]


def test_rejects_other_architectures(nxg, synth, tmp_path):
    import nexterabert_cpp_amd.gguf_writer as W
    p = write(nxg, synth, tmp_path / "a.gguf", lambda m: replace(m, "general.architecture", W.STRING, "bert"))
    ei = load_error(nxg, p)
    assert ei.type is ValueError and "not a nexterabert GGUF" in str(ei.value)


def test_rejects_block_type_errors(nxg, synth, tmp_path):
    import nexterabert_cpp_amd.gguf_writer as W
    p = write(nxg, synth, tmp_path / "b.gguf",
              lambda m: replace(m, "nexterabert.block_types", W.ARRAY, (W.STRING, ["lily"])))
    assert "block_types has 1 entries, expected 2" in str(load_error(nxg, p).value)
    p = write(nxg, synth, tmp_path / "c.gguf",
              lambda m: replace(m, "nexterabert.block_types", W.ARRAY, (W.STRING, ["lily", "mamba"])))
    assert "unsupported block type 'mamba'" in str(load_error(nxg, p).value)


def test_rejects_missing_keys_and_head_layouts(nxg, synth, tmp_path):
    p = write(nxg, synth, tmp_path / "d.gguf", lambda m: [e for e in m if e[0] != "nexterabert.vocab_size"])
    assert "missing key 'nexterabert.vocab_size'" in str(load_error(nxg, p).value)
    import nexterabert_cpp_amd.gguf_writer as W
    p = write(nxg, synth, tmp_path / "e.gguf", lambda m: replace(m, "nexterabert.attention.head_count_kv", W.UINT32, 3))
    assert "unsupported head layout" in str(load_error(nxg, p).value)
    p = write(nxg, synth, tmp_path / "f.gguf", lambda m: replace(m, "nexterabert.attention.head_count", W.UINT32, 4))
    assert "head_dim 64" in str(load_error(nxg, p).value)


def test_missing_file_and_no_gpu(nxg, synth, tmp_path):
    assert load_error(nxg, tmp_path / "none.gguf").type is ValueError
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    p = write(nxg, synth, tmp_path / "g.gguf")
    ei = load_error(nxg, p)
    assert ei.type is nxg.NxgError          # NXG_EDEVICE: the metadata passed, no gfx950 GPU here


@pytest.mark.parametrize("linear,type_name", [("blocks.1.mlp.c_fc.weight", "F16"), ("blocks.0.attn.x_proj.weight", "F32")])
def test_refuses_linears_off_the_int8_path(nxg, synth, tmp_path, linear, type_name):
    """An F16 or F32 encoder linear (which the reference would run on ggml_mul_mat,
    src/nexterabert.cpp:1140-1142) is refused from the tensor table, before the GPU is
    touched, with the reason."""
    ty = getattr(synth, type_name)
    p = write(nxg, synth, tmp_path / "h.gguf", type_of={linear: ty})
    ei = load_error(nxg, p)
    assert ei.type is ValueError
    msg = str(ei.value)
    assert f"'{linear}' (ggml type {ty}) is not on the int8 path" in msg and "no ggml_mul_mat fallback" in msg
