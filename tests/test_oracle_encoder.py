"""CPU: the oracle's full encoder forward (oracle/encoder.py) on small random-init models
written by the package's synth.py -- the pins of its composition (each op is pinned in
its own test file):

  * a sequence alone gives the bits it gets inside a packed batch (nexterabert.h:72-76),
    for every block type and with segment embeddings;
  * n_layers = k returns the residual stream after block k (nextera_debug_set_layers);
  * with every linear that writes the residual stream at zero (mixer and MLP c_proj), each
    block adds exactly 0, so the output is out_norm of the embedding rows;
  * the metadata defaults are nextera_load's (:1574-1612);
  * the pooled vectors are the mean of the output rows of each sequence.
"""
from __future__ import annotations

import numpy as np
import pytest


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


@pytest.fixture(scope="module")
def synth(nxg):
    from nexterabert_cpp_amd import synth as S
    return S


@pytest.fixture(scope="module")
def enc():
    from oracle import encoder as E
    return E


def tiny_dims(S, **kw):
    d = dict(n_vocab=300, n_embd=128, n_inter=256, n_head=2, n_kv_head=1, lily_rank=64, swa_window=8,
             block_types=["lily", "swa", "attn", "hra"])
    d.update(kw)
    return S.Dims(**d)


def test_batch_invariance_and_layers(nxg, synth, enc, tmp_path):
    d = tiny_dims(synth, n_types=2)
    path = tmp_path / "tiny.gguf"
    synth.write_random_model(nxg, path, "Q4_K_M", seed=3, dims=d)
    m = enc.from_gguf(path)
    assert m.n_types == 2 and len(m.lin) == 4 * 2 + 6 + 5 + 5 + 8
    rng = np.random.default_rng(0)
    lens = [5, 17, 1, 40]
    cu = np.concatenate([[0], np.cumsum(lens)])
    tok = rng.integers(0, d.n_vocab, cu[-1])
    typ = rng.integers(0, 2, cu[-1])
    outs = []
    h, p = enc.encode(m, tok, lens, typ, layer_outputs=outs)
    assert len(outs) == 4
    for i, n in enumerate(lens):
        hi, pi = enc.encode(m, tok[cu[i]:cu[i + 1]], [n], typ[cu[i]:cu[i + 1]])
        assert (bits(hi) == bits(h[cu[i]:cu[i + 1]])).all() and (bits(pi) == bits(p[i:i + 1])).all()
    for k in (1, 3):
        hk, _ = enc.encode(m, tok, lens, typ, n_layers=k)
        assert (bits(hk) == bits(outs[k - 1])).all()
    # segment ids change the result (the file has segment embeddings)
    h0, _ = enc.encode(m, tok, lens, np.zeros_like(typ))
    assert not (bits(h0) == bits(h)).all()
    # pooled: the rows' mean per sequence
    for i in range(len(lens)):
        assert np.allclose(p[i], h[cu[i]:cu[i + 1]].astype(np.float64).mean(0), atol=1e-5)


def test_zero_residual_writers_leave_the_embedding(nxg, synth, enc, orc, tmp_path):
    d = tiny_dims(synth)
    t = synth.model_tensors(d, seed=4)
    for name in t:
        if name.endswith("attn.c_proj.weight") or name.endswith("mlp.c_proj.weight"):
            t[name] = np.zeros_like(t[name])
    path = tmp_path / "zero.gguf"
    synth.write_random_model(nxg, path, "Q8_0", dims=d, tensors=t)
    m = enc.from_gguf(path)
    tok = np.random.default_rng(1).integers(0, d.n_vocab, 50)
    h, _ = enc.encode(m, tok, [20, 30])
    emb = m.f["embedding.weight"].reshape(-1, d.n_embd)[tok]
    ref = orc.layer_norm(emb, m.f["out_norm.weight"], m.f["out_norm.bias"], m.hp.ln_eps)
    assert (bits(h) == bits(ref)).all()


def test_metadata_defaults(enc):
    meta = {"nexterabert.vocab_size": 10, "nexterabert.embedding_length": 128, "nexterabert.block_count": 1,
            "nexterabert.feed_forward_length": 256, "nexterabert.attention.head_count": 2,
            "nexterabert.attention.head_count_kv": 1, "nexterabert.block_types": ["lily"]}
    hp = enc.HParams.from_metadata(meta)
    assert (hp.head_dim, hp.lily_rank, hp.hra_block, hp.swa_window, hp.ntk_train_len) == (64, 64, 4, 256, 0)
    assert (hp.rope_base, hp.swa_rope_base, hp.ssmax) == (100000.0, 10000.0, 2)
    assert hp.rms_eps == float(np.float32(1e-8)) and hp.ln_eps == float(np.float32(1e-5))
    assert hp.ssmax_base == float(np.float32(0.1))


def test_file_types_follow_the_quantizer(synth):
    d = synth.Dims()
    t = {"blocks.0.attn.c_v.weight": np.zeros((512, 1024), np.float32),
         "blocks.0.attn.c_q.weight": np.zeros((1024, 1024), np.float32),
         "blocks.0.attn.ltc_conv.out_proj.weight": np.zeros((1024, 64), np.float32),
         "blocks.0.mlp.c_proj.weight": np.zeros((1024, 2304), np.float32),
         "blocks.0.attn.state_conv.depthwise.weight": np.zeros((1024, 5), np.float32),
         "embedding.weight": np.zeros((50368, 1024), np.float32),
         "token_type_embeddings.weight": np.zeros((2, 1024), np.float32)}
    got = {n: synth.file_type_of(n, a, "Q4_K_M") for n, a in t.items()}
    assert got == {"blocks.0.attn.c_v.weight": synth.Q6_K, "blocks.0.attn.c_q.weight": synth.Q4_K,
                   "blocks.0.attn.ltc_conv.out_proj.weight": synth.Q5_0, "blocks.0.mlp.c_proj.weight": synth.Q6_K,
                   "blocks.0.attn.state_conv.depthwise.weight": synth.F32, "embedding.weight": synth.Q4_K,
                   "token_type_embeddings.weight": synth.F32}
    assert synth.file_type_of("x.attn.c_proj.weight", np.zeros((1024, 64), np.float32), "Q4_K_M") == synth.Q8_0
