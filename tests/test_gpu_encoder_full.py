"""GPU: the whole encoder forward (include/nxg_encoder.h) bit for bit against the oracle's
restatement (oracle/encoder.py) on random-init GGUF files written by synth.py:

  * small models with every block type (SnowLily, sliding-window and full attention, HRA)
    at n_embd 128 (the MLP's c_fc through fp32 rows, K-quants falling back to Q5_0) and 256
    (c_fc -> relu^2 -> int8 fused), Q4_K_M and Q8_0, with segment embeddings, ragged
    batches, one-token sequences and sequences shorter than an HRA block: hidden rows and
    pooled vectors (mean and L2-normalised);
  * a sequence alone gives its bits inside the batch; nxg_encoder_set_layers returns the
    residual stream after the given block; the device-buffer entry point equals the host
    one; bad ids and empty sequences are refused;
  * the 213M-parameter model (18 blocks, Q4_K_M) on one 1,024-token sequence: hidden bit for
    bit, and token cosine >= 0.99999 against the oracle.
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
def synth(nxg):
    from nexterabert_cpp_amd import synth as S
    return S


@pytest.fixture(scope="module")
def enc():
    from oracle import encoder as E
    return E


SMALL = {
    "c128_q4km": dict(n_embd=128, n_inter=256, n_head=2, n_kv_head=1, preset="Q4_K_M"),
    "c256_q8": dict(n_embd=256, n_inter=512, n_head=4, n_kv_head=2, preset="Q8_0"),
}


@pytest.fixture(scope="module")
def small_models(nxg, synth, enc, tmp_path_factory):
    out = {}
    for key, cfg in SMALL.items():
        cfg = dict(cfg)
        preset = cfg.pop("preset")
        d = synth.Dims(n_vocab=500, lily_rank=64, swa_window=8, n_types=2,
                       block_types=["lily", "swa", "attn", "hra", "lily", "hra"], **cfg)
        path = tmp_path_factory.mktemp("enc") / f"{key}.gguf"
        synth.write_random_model(nxg, path, preset, seed=len(key), dims=d)
        out[key] = (path, d, enc.from_gguf(path))
    return out


BATCHES = [[1], [7], [3, 1, 9, 33, 2], [130, 5, 64]]


@pytest.mark.parametrize("key", list(SMALL))
@pytest.mark.parametrize("lengths", BATCHES)
def test_encoder_matches_oracle(nxg, enc, torch, small_models, key, lengths):
    path, d, m = small_models[key]
    say(f"encoder {key} lengths={lengths}")
    rng = np.random.default_rng(sum(lengths))
    T = sum(lengths)
    tok = rng.integers(0, d.n_vocab, T).astype(np.int32)
    typ = rng.integers(0, 2, T).astype(np.int32)
    with nxg.Encoder(path) as e:
        assert (e.n_embd, e.n_layer, e.n_vocab, e.n_token_types) == (d.n_embd, len(d.block_types), d.n_vocab, 2)
        for types in (None, typ):
            for normalize in (False, True):
                h, p = e.encode(tok, lengths, types, pooled=True, normalize=normalize)
                hr, pr = enc.encode(m, tok, lengths, types, normalize=normalize)
                assert (bits(h) == bits(hr)).all(), f"hidden differs: types={types is not None}"
                assert (bits(p) == bits(pr)).all(), f"pooled differs: normalize={normalize}"


def test_encoder_long_document_matches_oracle(nxg, enc, torch, small_models):
    """One 2,700-token document: its full-attention layer has more keys per query than the tile
    kernel's LDS holds, so the encoder's attention keeps the scores in its workspace."""
    path, d, m = small_models["c128_q4km"]
    say("encoder c128_q4km one 2,700-token document")
    tok = np.random.default_rng(27).integers(0, d.n_vocab, 2700).astype(np.int32)
    with nxg.Encoder(path) as e:
        h, p = e.encode(tok, [2700], pooled=True)
    hr, pr = enc.encode(m, tok, [2700])
    assert (bits(h) == bits(hr)).all()
    assert (bits(p) == bits(pr)).all()


def test_encoder_work_limit_shrinks_the_attention_workspace(nxg, enc, torch, small_models):
    """nxg_encoder_set_work_limit: under a cap that leaves no room for the score workspace the
    long document's attention recomputes its scores, with the same bits; a cap below the
    activations fails with NXG_ENOMEM and leaves the context usable."""
    path, d, m = small_models["c128_q4km"]
    say("encoder work limit, one 2,700-token document")
    tok = np.random.default_rng(27).integers(0, d.n_vocab, 2700).astype(np.int32)
    with nxg.Encoder(path) as e:
        weights = e.device_bytes
        h0, p0 = e.encode(tok, [2700], pooled=True)
        ws, work = e.attention_workspace, e.device_bytes - weights
        assert ws > 0 and work > ws
        e.set_work_limit(work - ws + 4096)           # the activations (and alignment), no room for a score slot
        h1, p1 = e.encode(tok, [2700], pooled=True)
        assert e.attention_workspace == 0 and e.device_bytes - weights <= work - ws + 4096
        assert (bits(h1) == bits(h0)).all() and (bits(p1) == bits(p0)).all()
        e.set_work_limit(work - ws - (1 << 20))      # not even the activations
        with pytest.raises(Exception, match="exceed the limit"):
            e.encode(tok, [2700], pooled=True)
        e.set_work_limit(0)
        h2, p2 = e.encode(tok, [2700], pooled=True)
        assert e.attention_workspace == ws
        assert (bits(h2) == bits(h0)).all() and (bits(p2) == bits(p0)).all()
    hr, pr = enc.encode(m, tok, [2700])
    assert (bits(h0) == bits(hr)).all() and (bits(p0) == bits(pr)).all()


def test_encoder_batch_invariance_and_layers(nxg, enc, torch, small_models):
    path, d, m = small_models["c256_q8"]
    say("encoder batch invariance, set_layers, device entry point")
    lengths = [40, 1, 17, 5]
    cu = np.concatenate([[0], np.cumsum(lengths)])
    rng = np.random.default_rng(5)
    tok = rng.integers(0, d.n_vocab, cu[-1]).astype(np.int32)
    with nxg.Encoder(path) as e:
        h, p = e.encode(tok, lengths, pooled=True)
        for i, n in enumerate(lengths):
            hi, pi = e.encode(tok[cu[i]:cu[i + 1]], [n], pooled=True)
            assert (bits(hi) == bits(h[cu[i]:cu[i + 1]])).all() and (bits(pi) == bits(p[i:i + 1])).all()
        outs = []
        enc.encode(m, tok, lengths, layer_outputs=outs)
        for k in (1, 4):
            e.set_layers(k)
            hk, _ = e.encode(tok, lengths)
            assert (bits(hk) == bits(outs[k - 1])).all()
        e.set_layers(-1)
        # the device entry point, on torch's stream
        td = torch.from_numpy(tok).cuda()
        hd = torch.empty((int(cu[-1]), d.n_embd), dtype=torch.float32, device="cuda")
        pd = torch.empty((len(lengths), d.n_embd), dtype=torch.float32, device="cuda")
        e.forward(td, lengths, hidden=hd, pooled=pd)
        torch.cuda.synchronize()
        assert (bits(hd.cpu().numpy()) == bits(h)).all() and (bits(pd.cpu().numpy()) == bits(p)).all()
        with pytest.raises(ValueError):
            e.encode(np.array([0, d.n_vocab], np.int32), [2])          # id out of range
        with pytest.raises(ValueError):
            e.encode(np.array([0, 1], np.int32), [2, 0])               # an empty sequence
        assert e.last_ms > 0 and e.device_bytes > 0


def test_encoder_full_model_1024(nxg, synth, enc, torch, tmp_path):
    """The 213M-parameter model, Q4_K_M, one 1,024-token sequence of uniform random ids."""
    say("encoder: full model (18 blocks, Q4_K_M), 1,024 tokens")
    path = tmp_path / "full_q4km.gguf"
    synth.write_random_model(nxg, path, "Q4_K_M", seed=0)
    tok = np.random.default_rng(0).integers(0, 50368, 1024).astype(np.int32)
    with nxg.Encoder(path) as e:
        h, p = e.encode(tok, [1024], pooled=True)
    say("encoder: oracle forward")
    m = enc.from_gguf(path)
    hr, pr = enc.encode(m, tok, [1024])
    cos = np.sum(h.astype(np.float64) * hr, 1) / (np.linalg.norm(h.astype(np.float64), axis=1) * np.linalg.norm(hr, axis=1))
    say(f"encoder: min token cosine {cos.min():.9f}")
    assert cos.min() >= 0.99999
    assert (bits(h) == bits(hr)).all() and (bits(p) == bits(pr)).all()


def test_cli_encode_bench(nxg, torch, small_models, capsys):
    """--bench --encode in both drivers: the reference CLI's encode benchmark on nxg_encoder."""
    import importlib.util
    import subprocess
    from pathlib import Path
    root = Path(__file__).resolve().parent.parent
    path, d, _ = small_models["c256_q8"]
    spec = importlib.util.spec_from_file_location("nxg_cli", root / "nexterabert.cpp_amd" / "cli.py")
    cli = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(cli)
    say("cli --bench 48 --batch 2 --reps 3 --encode")
    assert cli.main(["--bench", "48", "--batch", "2", "--reps", "3", "--encode", "-m", str(path)]) == 0
    line = next(l for l in capsys.readouterr().out.splitlines() if l.startswith("bench: "))
    assert line.startswith("bench: Q8_0  T=48  batch=2  encoder  median") and "tokens/s" in line
    say("nxg-cli --bench 48 --batch 2 --reps 3 --encode")
    r = subprocess.run([str(root / "nexterabert.cpp_amd" / "nxg-cli"), "--bench", "48", "--batch", "2", "--reps", "3",
                        "--encode", "-m", str(path)], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr
    line = next(l for l in r.stdout.splitlines() if l.startswith("bench: "))
    assert line.startswith("bench: Q8_0  T=48  batch=2  encoder  median") and "tokens/s" in line
    # --profile: the reference's report of where the time goes, the timed passes only
    import re
    say("cli / nxg-cli --bench 48 --batch 2 --reps 3 --encode --profile")
    assert cli.main(["--bench", "48", "--batch", "2", "--reps", "3", "--encode", "--profile", "-m", str(path)]) == 0
    outs = [capsys.readouterr().out]
    r = subprocess.run([str(root / "nexterabert.cpp_amd" / "nxg-cli"), "--bench", "48", "--batch", "2", "--reps", "3",
                        "--encode", "--profile", "-m", str(path)], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr
    outs.append(r.stdout)
    for out in outs:
        assert "profile over 3 forward passes" in out, out
        rows = {}
        for k in ("int8 linear", "attention", "norm / conv / gate / quantize", "everything else"):
            m = re.search(re.escape(k) + r"\s+(-?[\d.]+)\s+(-?[\d.]+)%", out)
            assert m, (k, out)
            rows[k] = float(m.group(1))
        total = float(re.search(r"\n\s+total\s+([\d.]+)", out).group(1))
        assert all(rows[k] > 0 for k in ("int8 linear", "attention", "norm / conv / gate / quantize")), out
        assert abs(sum(rows.values()) - total) <= 0.01 + 1e-3 * total, out


BRANCH_BLOCKS = ["lily", "swa", "attn", "hra"]


@pytest.mark.parametrize("variant", ["ntk", "ssmax_none", "ssmax", "act63"])
def test_encoder_branches_match_oracle(nxg, synth, enc, torch, tmp_path, variant):
    """Branches of the forward pass the default synthetic file does not take, each against the
    oracle bit for bit: dynamic-NTK RoPE for a single sequence longer than
    rope.ntk_train_length (src/nexterabert.cpp:1356-1366; a batch of such sequences is refused,
    one of shorter sequences keeps the base), Scalable-Softmax modes "none" and "ssmax"
    (:1196-1201), and the AVX2-only build's 7-bit activations (ACT_MAX 63, :53-70)."""
    say(f"encoder branch {variant}")
    kw = dict(n_vocab=300, n_embd=256, n_inter=512, n_head=4, n_kv_head=2, lily_rank=64, swa_window=8,
              block_types=BRANCH_BLOCKS)
    if variant == "ntk":
        kw["ntk_train_len"] = 24
    elif variant.startswith("ssmax"):
        kw["ssmax_mode"] = {"ssmax_none": "none", "ssmax": "ssmax"}[variant]
    d = synth.Dims(**kw)
    path = tmp_path / f"{variant}.gguf"
    synth.write_random_model(nxg, path, "Q8_0", seed=7, dims=d)
    act_max = 63 if variant == "act63" else 127
    m = enc.from_gguf(path, act_max=act_max)
    rng = np.random.default_rng(3)
    cases = [[61]] if variant == "ntk" else [[61], [19, 1, 40]]
    if variant == "ntk":
        cases.append([24, 9])                      # every sequence within the trained length: no NTK
    with nxg.Encoder(path, act_max=act_max) as e:
        for lengths in cases:
            tok = rng.integers(0, d.n_vocab, sum(lengths)).astype(np.int32)
            h, p = e.encode(tok, lengths, pooled=True, normalize=True)
            hr, pr = enc.encode(m, tok, lengths, normalize=True)
            assert (bits(h) == bits(hr)).all(), f"hidden differs, lengths={lengths}"
            assert (bits(p) == bits(pr)).all(), f"pooled differs, lengths={lengths}"
        if variant == "ntk":
            with pytest.raises(ValueError, match="one at a time"):
                e.encode(rng.integers(0, d.n_vocab, 70).astype(np.int32), [30, 40])
    if variant == "ntk":                           # the stretched base is in use: the bits differ without it
        d0 = synth.Dims(**{**kw, "ntk_train_len": 0})
        p0 = tmp_path / "ntk0.gguf"
        synth.write_random_model(nxg, p0, "Q8_0", seed=7, dims=d0)
        tok = np.random.default_rng(3).integers(0, d.n_vocab, 61).astype(np.int32)
        with nxg.Encoder(p0) as e0, nxg.Encoder(path) as e1:
            assert not (bits(e0.encode(tok, [61])[0]) == bits(e1.encode(tok, [61])[0])).all()
