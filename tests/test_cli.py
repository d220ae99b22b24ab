"""CPU: the command line's arguments, --info on a GGUF file, and the file-type names of
the reference (src/nexterabert.cpp:1390-1410)."""
from __future__ import annotations

import importlib.util
from pathlib import Path

import pytest

from nexterabert_cpp_amd import gguf_writer as W

ROOT = Path(__file__).resolve().parent.parent


@pytest.fixture(scope="module")
def cli(nxg):
    spec = importlib.util.spec_from_file_location("nxg_cli", ROOT / "nexterabert.cpp_amd" / "cli.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_bench_defaults_follow_the_reference_cli(cli):
    a = cli.parse_args(["--bench", "128"])
    assert (a.bench, a.batch, a.reps, a.profile, a.graph) == (128, 1, 20, False, False)
    a = cli.parse_args(["--bench", "64", "--batch", "8", "--reps", "5", "--profile", "--graph", "-m", "x.gguf"])
    assert (a.bench, a.batch, a.reps, a.profile, a.graph, a.model) == (64, 8, 5, True, True, "x.gguf")


@pytest.mark.parametrize("argv", [["--bench", "-1"], ["--bench", "8", "--batch", "0"], ["--bench", "8", "--reps", "0"]])
def test_bad_arguments_exit(cli, argv):
    with pytest.raises(SystemExit):
        cli.parse_args(argv)


def test_ftype_names(cli):
    assert cli.ftype_name(7) == "Q8_0" and cli.ftype_name(15) == "Q4_K_M" and cli.ftype_name(18) == "Q6_K"
    assert cli.ftype_name(4) == "unknown" and cli.ftype_name(None) == "unknown"


def test_info_on_a_gguf_file(cli, nxg, tmp_path, capsys):
    import numpy as np
    rows = (0.02 * np.random.default_rng(0).standard_normal((8, 64))).astype(np.float32)
    tensors = [("blocks.0.attn.c_q.weight", nxg.TYPE_Q8_0, (64, 8), nxg.quantize_weight(nxg.TYPE_Q8_0, rows).tobytes()),
               ("embedding.weight", nxg.TYPE_Q8_0, (64, 8), nxg.quantize_weight(nxg.TYPE_Q8_0, rows).tobytes())]
    path = tmp_path / "m.gguf"
    W.write_gguf(path, [("general.architecture", W.STRING, "nexterabert"), ("general.file_type", W.UINT32, 15)], tensors)
    assert cli.main(["--info", "-m", str(path)]) == 0
    out = capsys.readouterr().out
    assert "libnxg.so" in out
    assert "GGUF v3, Q4_K_M, architecture nexterabert, 2 tensors, 1 int8 linears" in out


# --- the C++ driver (nexterabert.cpp_amd/nxg-cli) ----------------------------------

CXX_CLI = ROOT / "nexterabert.cpp_amd" / "nxg-cli"


def test_cxx_cli_help_and_info(nxg, tmp_path):
    import subprocess
    import numpy as np
    assert CXX_CLI.exists(), "nxg-cli is built by nexterabert.cpp_amd/build.py"
    r = subprocess.run([str(CXX_CLI), "--help"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0 and "--bench T" in r.stderr
    r = subprocess.run([str(CXX_CLI), "--bench", "8", "--nonsense"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 1
    rows = (0.02 * np.random.default_rng(1).standard_normal((8, 64))).astype(np.float32)
    tensors = [("blocks.0.attn.c_q.weight", nxg.TYPE_Q8_0, (64, 8), nxg.quantize_weight(nxg.TYPE_Q8_0, rows).tobytes())]
    path = tmp_path / "m.gguf"
    W.write_gguf(path, [("general.file_type", W.UINT32, 7)], tensors)
    r = subprocess.run([str(CXX_CLI), "--info", "-m", str(path)], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stderr
    assert "model: GGUF v3, Q8_0, 1 tensors" in r.stdout
