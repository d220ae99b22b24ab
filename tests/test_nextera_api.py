"""CPU tests of the reference's public C API as this build serves it (include/nexterabert.h,
libnexterabert.so): the header declares exactly the reference's functions and struct
(src/nexterabert.h:28-123, checked against the reference's own header where its tree is
present), the library exports exactly what the header declares, and nextera_load's refusals
(bad path, wrong architecture, use_int8 = 0, unsupported classifier task, missing head
tensors, no GPU) return NULL with the reason on stderr. No test here launches GPU work."""
from __future__ import annotations

import ctypes
import re
import subprocess
from pathlib import Path

import numpy as np
import pytest

import nextera_api as api

REF_HEADER = Path("/root/reference/src/nexterabert.h")
REF_CLI_SRC = Path("/root/reference/tools/cli.cpp")
REF_CPP = Path("/root/reference/src/nexterabert.cpp")
DEBUG = ("nextera_debug_set_layers", "nextera_debug_profile", "nextera_debug_profile_print")


@pytest.fixture(scope="module")
def lib(nxg):
    nxg.load_library()
    return api.bind()


def test_header_declares_the_c_api():
    d = api.declarations(api.HEADER.read_text())
    assert len(d) == 30
    assert d["nextera_load"] == ("struct nextera_context *", ["const char *", "struct nextera_params"])
    assert d["nextera_encode_segments"] == ("int32_t", ["struct nextera_context *", "const int32_t *",
                                                        "const int32_t *", "const int32_t *", "int32_t",
                                                        "float *", "float *", "int32_t"])
    assert api.struct_fields(api.HEADER.read_text()) == ["int32_t n_threads", "int32_t use_int8",
                                                         "int32_t use_repack", "int32_t verbosity"]
    assert ctypes.sizeof(api.Params) == 16


@pytest.mark.skipif(not REF_HEADER.is_file(), reason="the reference's tree is not present")
def test_declarations_are_the_references():
    """Every function of the reference's header, and its struct, with the same types; the three
    diagnostics as the reference's CLI and library declare them."""
    ours = api.declarations(api.HEADER.read_text())
    ref = api.declarations(REF_HEADER.read_text())
    assert len(ref) == 27
    assert {k: ours[k] for k in ref} == ref
    assert api.struct_fields(REF_HEADER.read_text()) == api.struct_fields(api.HEADER.read_text())
    cli = api.declarations(REF_CLI_SRC.read_text())
    assert cli == {k: ours[k] for k in ("nextera_debug_profile", "nextera_debug_profile_print")}
    text = REF_CPP.read_text()
    m = re.search(r"void\s+nextera_debug_set_layers\s*\(([^)]*)\)", text)
    assert m and [" ".join(a.split()[:-1]) for a in m.group(1).split(",")] == \
        ours["nextera_debug_set_layers"][1]
    assert set(ours) == set(ref) | set(DEBUG)


def test_library_exports_exactly_the_header(lib):
    out = subprocess.run(["nm", "-D", "--defined-only", str(api.LIB)], capture_output=True, text=True,
                         check=True).stdout
    exported = {l.split()[-1] for l in out.splitlines() if " T " in l}
    assert exported == set(api.declarations(api.HEADER.read_text()))


def test_library_links_the_engine_next_to_it():
    out = subprocess.run(["ldd", str(api.LIB)], capture_output=True, text=True, check=True).stdout
    line = next(l for l in out.splitlines() if "libnxg.so" in l)
    assert str(api.LIB.parent) in line.replace("/./", "/")


def test_default_params(lib):
    p = lib.nextera_default_params()
    assert (p.n_threads, p.use_int8, p.use_repack, p.verbosity) == (0, 1, 1, 0)


def _model(nxg, path, extra_metadata=None, extra_tensors=None):
    from nexterabert_cpp_amd import synth
    d = synth.Dims(n_vocab=64, n_embd=128, n_inter=256, n_head=2, n_kv_head=1, lily_rank=64, swa_window=8,
                   block_types=["lily", "attn"])
    synth.write_random_model(nxg, path, "Q8_0", seed=3, dims=d, extra_metadata=extra_metadata,
                             extra_tensors=extra_tensors)
    return d


def _load(lib, path, **kw):
    p = lib.nextera_default_params()
    for k, v in kw.items():
        setattr(p, k, v)
    return lib.nextera_load(str(path).encode(), p)


def test_load_refusals_return_null_with_a_reason(nxg, lib, tmp_path, capfd):
    from nexterabert_cpp_amd import gguf_writer as W
    assert not _load(lib, tmp_path / "missing.gguf")
    assert "failed to open" in capfd.readouterr().err

    other = tmp_path / "other.gguf"
    W.write_gguf(other, [("general.architecture", W.STRING, "llama")], [])
    assert not _load(lib, other)
    assert "is not a nexterabert GGUF (general.architecture = 'llama')" in capfd.readouterr().err

    good = tmp_path / "m.gguf"
    _model(nxg, good)
    assert not _load(lib, good, use_int8=0)
    assert "use_int8 = 0" in capfd.readouterr().err

    # an F16 encoder linear: refused with the reason, before any device work (also without a GPU)
    from nexterabert_cpp_amd import synth as S
    f16 = tmp_path / "f16.gguf"
    d = S.Dims(n_vocab=100, n_embd=128, n_inter=256, n_head=2, n_kv_head=1, lily_rank=64, block_types=["lily", "attn"])
    t = S.model_tensors(d, seed=0)
    entries = []
    for name in sorted(t):
        ty = S.F16 if name == "blocks.1.attn.c_q.weight" else S.file_type_of(name, t[name], "Q8_0")
        ne = tuple(reversed(t[name].shape)) if t[name].ndim == 2 else (t[name].size,)
        data = np.ascontiguousarray(t[name], np.float16).tobytes() if ty == S.F16 else S.encode_tensor(nxg, t[name], ty)
        entries.append((name, ty, ne, data))
    W.write_gguf(f16, S.metadata(d, "Q8_0"), entries)
    assert not _load(lib, f16)
    err = capfd.readouterr().err
    assert "'blocks.1.attn.c_q.weight' (ggml type 1) is not on the int8 path" in err, err

    bad_task = tmp_path / "task.gguf"
    _model(nxg, bad_task, extra_metadata=[("nexterabert.classifier.task", W.STRING, "regression")])
    assert not _load(lib, bad_task)
    assert "unsupported classifier task 'regression'" in capfd.readouterr().err

    no_head = tmp_path / "mlm.gguf"
    _model(nxg, no_head, extra_metadata=[("nexterabert.mlm_head", W.BOOL, True)])
    assert not _load(lib, no_head)
    assert "has no tensor 'mlm.dense.weight'" in capfd.readouterr().err

    cls_no_pooler = tmp_path / "cls.gguf"
    C = 128
    _model(nxg, cls_no_pooler, extra_metadata=[("nexterabert.classifier.task", W.STRING, "sequence-classification")],
           extra_tensors={"classifier.weight": np.zeros((3, C), np.float32),
                          "classifier.bias": np.zeros(3, np.float32)})
    assert not _load(lib, cls_no_pooler)
    assert "has no tensor 'pooler.dense.weight'" in capfd.readouterr().err


def test_load_without_a_gpu_fails_loudly(nxg, lib, tmp_path, capfd):
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    good = tmp_path / "m.gguf"
    _model(nxg, good)
    assert not _load(lib, good)
    err = capfd.readouterr().err
    assert err.startswith("nexterabert: ") and ("gfx950" in err or "device" in err.lower() or "HIP" in err)
