"""GPU: the encoder's linear path (EncoderLinearPath) and the command line's --bench.

  * the path has the reference's linears: 140 projections as 92 GEMMs (18 of them
    c_fc -> relu^2 -> int8) and 74 quantizations per layer stack, 313,524,224 int8 ops
    per token with HRA q/k/v on T/4 block rows;
  * a packed batch gives every sequence the bits it gets alone (fp32 rows and int8
    activations, through the batch's cu_offsets);
  * weights read from a GGUF file give the same path as the same weights made in memory;
  * cli.py --bench prints the reference CLI's line (median, min, tokens/s).
"""
from __future__ import annotations

import importlib.util
from pathlib import Path

import numpy as np
import pytest

from nexterabert_cpp_amd import gguf_writer as W

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parent.parent


def say(msg):
    print(msg, flush=True)


@pytest.fixture(scope="module")
def torch():
    import torch as t
    assert t.cuda.is_available(), "no GPU"
    return t


@pytest.fixture(scope="module")
def enc(torch, nxg):
    nxg.init()
    import nexterabert_cpp_amd.encoder as e
    return e


def run_and_collect(path, torch):
    path.step()
    torch.cuda.synchronize()
    outs = {k: v.cpu().numpy() for k, v in path.outs.items()}
    qacts = {k: tuple(a.cpu().numpy() for a in path.nxg.export_qact(v)) for k, v in path.qacts.items()}
    return outs, qacts


def test_path_counts_and_ops(nxg, enc):
    say("encoder path counts, M=1024")
    p = enc.EncoderLinearPath(nxg, [1024])
    assert (p.n_gemm, p.n_relu2, p.n_quant) == (92, 18, 74)
    assert p.ops == 313_524_224 * 1024
    assert sum(len(g.specs) for steps in p.layers for (_, _, _, _, _, g, _) in steps) == 140


def test_packed_batch_equals_sequences_alone(nxg, orc, enc, torch):
    lengths = [40, 7, 101]               # HRA block rows 10, 2, 26: never equal to the token rows
    say(f"encoder path packed {lengths} vs each alone")
    batch = enc.EncoderLinearPath(nxg, lengths)
    cu = np.concatenate([[0], np.cumsum(lengths)])
    blk = [(n + 3) // 4 for n in lengths]
    cub = np.concatenate([[0], np.cumsum(blk)])
    M, MB = int(cu[-1]), int(cub[-1])
    b_outs, b_q = run_and_collect(batch, torch)
    for s, n in enumerate(lengths):
        alone = enc.EncoderLinearPath(nxg, [n], weights=batch.dev_weights)
        tok, bl = slice(int(cu[s]), int(cu[s + 1])), slice(int(cub[s]), int(cub[s + 1]))
        # the same inputs: this sequence's rows of the batch's synthetic rows and residual
        for (name, n_in, rows), x in alone.inputs.items():
            block = rows != n
            x.copy_(batch.inputs[(name, n_in, MB if block else M)][bl if block else tok])
        alone.residual.copy_(batch.residual[tok])
        a_outs, a_q = run_and_collect(alone, torch)
        for (n_out, rows), y in a_outs.items():
            block = rows != n
            ref = b_outs[(n_out, MB if block else M)][bl if block else tok]
            assert (y.view(np.uint32) == ref.view(np.uint32)).all(), f"sequence {s}: fp32 rows, n_out {n_out}"
        for (name, n_in, rows), (u8, sx) in a_q.items():
            block = rows != n
            bu8, bsx = b_q[(name, n_in, MB if block else M)]
            assert (u8 == bu8[bl if block else tok]).all(), f"sequence {s}: int8 activations {name}"
            sa = orc.sx_matrix(sx, rows, n_in)
            sb = orc.sx_matrix(bsx, MB if block else M, n_in)[bl if block else tok]
            assert (sa.view(np.uint32) == sb.view(np.uint32)).all(), f"sequence {s}: scales {name}"


def test_gguf_weights_equal_weights_made_in_memory(nxg, enc, torch, tmp_path):
    """The random path draws N(0, 0.02) rows in group order and encodes them as Q8_0; a
    GGUF file holding the same blocks must give the same expanded weights and outputs."""
    import nexterabert_cpp_amd.model as model
    say("encoder path from a GGUF file (140 Q8_0 tensors)")
    rng = np.random.default_rng(0)
    tensors = []
    for l, kind in enumerate(model.BLOCK_TYPES):
        for g in model.layer_groups(l, kind, True):
            for s in g.specs:
                rows = (0.02 * rng.standard_normal((s.n_out, s.n_in))).astype(np.float32)
                tensors.append((s.name, nxg.TYPE_Q8_0, (s.n_in, s.n_out), nxg.quantize_weight(nxg.TYPE_Q8_0, rows).tobytes()))
    path = tmp_path / "enc.gguf"
    W.write_gguf(path, [("general.architecture", W.STRING, "nexterabert"), ("general.file_type", W.UINT32, 7)], tensors)
    del tensors
    mem = enc.EncoderLinearPath(nxg, [96])
    with nxg.GGUF(path) as gg:
        assert len(gg.int8_names()) == 140
        fil = enc.EncoderLinearPath(nxg, [96], gguf=gg)
    for k, Wm in mem.host_weights.items():
        Wf = fil.host_weights[k]
        assert np.array_equal(Wm.w, Wf.w) and np.array_equal(Wm.scale.view(np.uint32), Wf.scale.view(np.uint32))
    m_outs, m_q = run_and_collect(mem, torch)
    f_outs, f_q = run_and_collect(fil, torch)
    for k in m_outs:
        assert (m_outs[k].view(np.uint32) == f_outs[k].view(np.uint32)).all()
    for k in m_q:
        assert (m_q[k][0] == f_q[k][0]).all()


@pytest.mark.parametrize("extra", [[], ["--graph", "--profile"]])
def test_cli_bench(nxg, enc, capsys, extra):
    spec = importlib.util.spec_from_file_location("nxg_cli", ROOT / "nexterabert.cpp_amd" / "cli.py")
    cli = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(cli)
    say(f"cli --bench 64 --batch 3 --reps 3 {' '.join(extra)}")
    assert cli.main(["--bench", "64", "--batch", "3", "--reps", "3"] + extra) == 0
    out = capsys.readouterr().out
    line = next(l for l in out.splitlines() if l.startswith("bench: "))
    assert "T=64  batch=3" in line and "median" in line and "tokens/s" in line
    if "--profile" in extra:
        assert "quantize" in out and "GEMM fp32 out" in out and "GEMM relu^2 -> int8" in out


@pytest.mark.parametrize("extra", [[], ["--graph", "--profile"]])
def test_cxx_cli_bench(nxg, extra):
    """The C++ driver (nxg-cli) runs the same pass through the C ABI alone."""
    import subprocess
    cli = ROOT / "nexterabert.cpp_amd" / "nxg-cli"
    say(f"nxg-cli --bench 64 --batch 3 --reps 3 {' '.join(extra)}")
    r = subprocess.run([str(cli), "--bench", "64", "--batch", "3", "--reps", "3"] + extra,
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr
    line = next(l for l in r.stdout.splitlines() if l.startswith("bench: "))
    assert "T=64  batch=3" in line and "tokens/s" in line
    assert "92 GEMMs (18 relu^2 -> int8) + 74 quantizations" in r.stdout
    if "--profile" in extra:
        assert "GEMM fp32 out" in r.stdout and "quantize" in r.stdout
