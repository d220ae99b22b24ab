"""GPU: the reference's public C API (include/nexterabert.h) on libnexterabert.so, bound with
ctypes from the header's own declarations (tests/nextera_api.py), on a random-init model file
that carries every head's metadata:

  * the getters return the file's metadata (nextera_load's keys and defaults);
  * nextera_encode / nextera_encode_segments give hidden rows and pooled vectors bit for bit
    equal to the oracle's restatement of the forward pass (oracle/encoder.py), with either
    output optional; nextera_debug_set_layers returns the residual stream after block k;
  * nextera_debug_profile / _print report the three kinds and the rest of the wall time;
  * bad ids, empty sequences and the heads return 1 with the reason on stderr;
  * the reference's own CLI (tools/cli.cpp, compiled unchanged against this header, see
    oracle/Makefile) loads the file, prints --info, the pooled embedding of --ids sequences
    equal to the oracle's, and runs --bench --profile.
"""
from __future__ import annotations

import ctypes
import re
import subprocess

import numpy as np
import pytest

import nextera_api as api

pytestmark = pytest.mark.gpu

P_I32 = ctypes.POINTER(ctypes.c_int32)
P_F32 = ctypes.POINTER(ctypes.c_float)
LABELS = ["neg", "pos", "mid"]
TOKENIZER = '{"version": "1.0", "model": {"type": "BPE"}}'


def say(msg):
    print(msg, flush=True)


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def ptr(a, t):
    return None if a is None else a.ctypes.data_as(t)


@pytest.fixture(scope="module")
def torch():
    import torch as t
    assert t.cuda.is_available(), "no GPU"
    return t


@pytest.fixture(scope="module")
def lib(nxg, torch):
    nxg.load_library()
    return api.bind()


@pytest.fixture(scope="module")
def model(nxg, tmp_path_factory):
    from nexterabert_cpp_amd import gguf_writer as W
    from nexterabert_cpp_amd import synth
    from oracle import encoder as E
    d = synth.Dims(n_vocab=1200, n_embd=128, n_inter=256, n_head=2, n_kv_head=1, lily_rank=64, swa_window=8,
                   n_types=2, block_types=["lily", "swa", "attn", "hra"])
    C, rng = d.n_embd, np.random.default_rng(11)
    heads = {"classifier.weight": rng.standard_normal((3, C), dtype=np.float32),
             "classifier.bias": rng.standard_normal(3, dtype=np.float32),
             "pooler.dense.weight": (0.02 * rng.standard_normal((C, C))).astype(np.float32),
             "pooler.norm.weight": np.ones(C, np.float32),
             "mlm.dense.weight": (0.02 * rng.standard_normal((C, C))).astype(np.float32),
             "mlm.norm.weight": np.ones(C, np.float32),
             "mlm.bias": np.zeros(d.n_vocab, np.float32)}
    meta = [("nexterabert.classifier.task", W.STRING, "sequence-classification"),
            ("nexterabert.classifier.labels", W.ARRAY, (W.STRING, LABELS)),
            ("nexterabert.mlm_head", W.BOOL, True),
            ("tokenizer.huggingface.json", W.STRING, TOKENIZER),
            ("tokenizer.ggml.cls_token_id", W.UINT32, 1), ("tokenizer.ggml.seperator_token_id", W.UINT32, 2),
            ("tokenizer.ggml.padding_token_id", W.UINT32, 3), ("tokenizer.ggml.mask_token_id", W.UINT32, 4)]
    path = tmp_path_factory.mktemp("api") / "heads.gguf"
    synth.write_random_model(nxg, path, "Q4_K_M", seed=21, dims=d, extra_metadata=meta, extra_tensors=heads)
    return path, d, E.from_gguf(path)


@pytest.fixture(scope="module")
def ctx(lib, model):
    path = model[0]
    p = lib.nextera_default_params()
    p.n_threads = 3
    c = lib.nextera_load(str(path).encode(), p)
    assert c, "nextera_load returned NULL"
    yield c
    lib.nextera_free(c)


def test_getters(lib, ctx, model):
    say("nextera getters")
    _, d, _ = model
    assert (lib.nextera_n_embd(ctx), lib.nextera_n_vocab(ctx), lib.nextera_n_layer(ctx)) == (128, 1200, 4)
    assert lib.nextera_n_token_types(ctx) == 2
    assert lib.nextera_has_mlm_head(ctx) == 1 and lib.nextera_has_pooler(ctx) == 1
    assert lib.nextera_classifier_task(ctx) == b"sequence-classification"
    assert lib.nextera_n_labels(ctx) == 3
    assert [lib.nextera_label(ctx, i) for i in range(-1, 4)] == [b"", b"neg", b"pos", b"mid", b""]
    assert [lib.nextera_token_cls(ctx), lib.nextera_token_sep(ctx), lib.nextera_token_pad(ctx),
            lib.nextera_token_mask(ctx)] == [1, 2, 3, 4]
    assert lib.nextera_tokenizer_json(ctx).decode() == TOKENIZER
    assert lib.nextera_ftype(ctx) == b"Q4_K_M"
    info = lib.nextera_system_info(ctx).decode()
    assert "gfx950" in info and "int8" in info
    assert lib.nextera_get_n_threads(ctx) == 3
    lib.nextera_set_n_threads(ctx, 5)
    assert lib.nextera_get_n_threads(ctx) == 5


@pytest.mark.parametrize("lengths", [[1], [3, 1, 9, 33, 2], [70, 5]])
def test_encode_matches_oracle(nxg, lib, ctx, model, lengths):
    _, d, m = model
    from oracle import encoder as E
    say(f"nextera_encode lengths={lengths}")
    T = sum(lengths)
    rng = np.random.default_rng(T)
    tok = rng.integers(0, d.n_vocab, T).astype(np.int32)
    typ = rng.integers(0, 2, T).astype(np.int32)
    lens = np.asarray(lengths, np.int32)
    for types in (None, typ):
        for normalize in (0, 1):
            hidden = np.full((T, d.n_embd), np.nan, np.float32)
            pooled = np.full((len(lengths), d.n_embd), np.nan, np.float32)
            if types is None:
                rc = lib.nextera_encode(ctx, ptr(tok, P_I32), ptr(lens, P_I32), len(lengths), ptr(hidden, P_F32),
                                        ptr(pooled, P_F32), normalize)
            else:
                rc = lib.nextera_encode_segments(ctx, ptr(tok, P_I32), ptr(types, P_I32), ptr(lens, P_I32),
                                                 len(lengths), ptr(hidden, P_F32), ptr(pooled, P_F32), normalize)
            assert rc == 0
            hr, pr = E.encode(m, tok, lengths, types, normalize=bool(normalize))
            assert (bits(hidden) == bits(hr)).all(), f"hidden differs (types={types is not None})"
            assert (bits(pooled) == bits(pr)).all(), f"pooled differs (normalize={normalize})"
            assert lib.nextera_last_ms(ctx) > 0
    # either output may be NULL
    pooled = np.zeros((len(lengths), d.n_embd), np.float32)
    assert lib.nextera_encode(ctx, ptr(tok, P_I32), ptr(lens, P_I32), len(lengths), None, ptr(pooled, P_F32), 0) == 0
    assert (bits(pooled) == bits(E.encode(m, tok, lengths)[1])).all()
    hidden = np.zeros((T, d.n_embd), np.float32)
    assert lib.nextera_encode(ctx, ptr(tok, P_I32), ptr(lens, P_I32), len(lengths), ptr(hidden, P_F32), None, 0) == 0
    assert (bits(hidden) == bits(E.encode(m, tok, lengths)[0])).all()


def test_debug_set_layers(lib, ctx, model):
    _, d, m = model
    from oracle import encoder as E
    say("nextera_debug_set_layers")
    lengths = [12, 30]
    tok = np.random.default_rng(2).integers(0, d.n_vocab, sum(lengths)).astype(np.int32)
    lens = np.asarray(lengths, np.int32)
    outs = []
    E.encode(m, tok, lengths, layer_outputs=outs)
    for k in (1, 3):
        lib.nextera_debug_set_layers(ctx, k)
        hidden = np.zeros((sum(lengths), d.n_embd), np.float32)
        assert lib.nextera_encode(ctx, ptr(tok, P_I32), ptr(lens, P_I32), 2, ptr(hidden, P_F32), None, 0) == 0
        assert (bits(hidden) == bits(outs[k - 1])).all()
    lib.nextera_debug_set_layers(ctx, -1)
    hidden = np.zeros((sum(lengths), d.n_embd), np.float32)
    assert lib.nextera_encode(ctx, ptr(tok, P_I32), ptr(lens, P_I32), 2, ptr(hidden, P_F32), None, 0) == 0
    assert (bits(hidden) == bits(E.encode(m, tok, lengths)[0])).all()


def parse_profile(err):
    rows = {}
    for name in ("int8 linear", "attention", "norm / conv / gate / quantize", "everything else"):
        m = re.search(re.escape(name) + r"\s+(-?[\d.]+)\s+(-?[\d.]+)%", err)
        assert m, f"no profile row '{name}' in:\n{err}"
        rows[name] = (float(m.group(1)), float(m.group(2)))
    m = re.search(r"\n\s+total\s+([\d.]+)", err)
    assert m, err
    rows["total"] = float(m.group(1))
    return rows


def test_debug_profile(lib, ctx, model, capfd):
    _, d, _ = model
    say("nextera_debug_profile")
    lengths = [64, 64]
    tok = np.random.default_rng(4).integers(0, d.n_vocab, 128).astype(np.int32)
    lens = np.asarray(lengths, np.int32)
    pooled = np.zeros((2, d.n_embd), np.float32)
    capfd.readouterr()
    lib.nextera_debug_profile_print(ctx)             # nothing profiled yet: prints nothing
    assert capfd.readouterr().err == ""
    lib.nextera_debug_profile(ctx, 1)
    for _ in range(3):
        assert lib.nextera_encode(ctx, ptr(tok, P_I32), ptr(lens, P_I32), 2, None, ptr(pooled, P_F32), 1) == 0
    lib.nextera_debug_profile_print(ctx)
    err = capfd.readouterr().err
    assert "profile over 3 forward passes" in err
    rows = parse_profile(err)
    for k in ("int8 linear", "attention", "norm / conv / gate / quantize"):
        assert rows[k][0] > 0, err
    assert rows["everything else"][0] >= 0
    parts = sum(rows[k][0] for k in ("int8 linear", "attention", "norm / conv / gate / quantize", "everything else"))
    assert abs(parts - rows["total"]) <= 0.01 + 1e-3 * rows["total"]
    lib.nextera_debug_profile(ctx, 0)
    lib.nextera_debug_profile_print(ctx)
    assert capfd.readouterr().err == ""


def test_bad_input_and_heads(lib, ctx, model, capfd):
    _, d, _ = model
    say("nextera bad input and heads")
    tok = np.array([0, d.n_vocab], np.int32)
    lens = np.array([2], np.int32)
    out = np.zeros((2, 8), np.float32)
    capfd.readouterr()
    assert lib.nextera_encode(ctx, ptr(tok, P_I32), ptr(lens, P_I32), 1, None, ptr(out, P_F32), 0) == 1
    assert "token id 1200 out of range" in capfd.readouterr().err
    tok = np.array([0, 1], np.int32)
    lens = np.array([2, 0], np.int32)
    assert lib.nextera_encode(ctx, ptr(tok, P_I32), ptr(lens, P_I32), 2, None, ptr(out, P_F32), 0) == 1
    assert "empty sequence" in capfd.readouterr().err
    lens = np.array([2], np.int32)
    assert lib.nextera_pooler_output(ctx, ptr(tok, P_I32), None, ptr(lens, P_I32), 1, ptr(out, P_F32)) == 1
    assert lib.nextera_classify(ctx, ptr(tok, P_I32), None, ptr(lens, P_I32), 1, ptr(out, P_F32)) == 1
    pos = np.array([0], np.int32)
    assert lib.nextera_mlm_logits(ctx, ptr(tok, P_I32), 2, ptr(pos, P_I32), 1, ptr(out, P_F32)) == 1
    err = capfd.readouterr().err
    assert err.count("which this engine does not run") == 3


def test_reference_cli_on_the_engine(nxg, model, tmp_path):
    from oracle import oracle as orc
    from oracle import encoder as E
    if not orc.REF_CLI.is_file():
        pytest.skip("the reference's CLI was not built (oracle/Makefile, needs the reference's tree)")
    path, d, m = model
    say("reference tools/cli.cpp on libnexterabert.so: --info, --ids, --bench --profile")
    run = lambda *a: subprocess.run([str(orc.REF_CLI), "-m", str(path), *a], capture_output=True, text=True,
                                    timeout=120)
    r = run("--info")
    assert r.returncode == 0, r.stderr
    assert "file type  : Q4_K_M" in r.stdout and "n_layer    : 4" in r.stdout and "segments   : 2" in r.stdout
    assert "classifier : sequence-classification, 3 labels (neg, pos, mid)" in r.stdout
    assert f"tokenizer  : {len(TOKENIZER)} bytes" in r.stdout and "gfx950" in r.stdout
    seqs = [[1, 17, 400, 99, 2], [1, 1100, 2]]
    r = run("--ids", ",".join(map(str, seqs[0])), "--ids", ",".join(map(str, seqs[1])))
    assert r.returncode == 0, r.stderr
    tok = np.array(seqs[0] + seqs[1], np.int32)
    _, pr = E.encode(m, tok, [len(s) for s in seqs], normalize=True)
    for i, s in enumerate(seqs):
        want = f"[{i}] ({len(s)} tokens)" + "".join(f" {v:.6f}" for v in pr[i, :8]) + " ..."
        assert want in r.stdout, (want, r.stdout)
    r = run("--bench", "48", "--batch", "2", "--reps", "4", "--profile")
    assert r.returncode == 0, r.stderr
    assert re.search(r"bench: Q4_K_M  T=48  batch=2  threads=\d+  median [\d.]+ ms", r.stdout), r.stdout
    assert "profile over 4 forward passes" in r.stderr
    parse_profile(r.stderr)
