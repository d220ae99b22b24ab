"""GPU: int8 linear weights loaded from a GGUF file (nxg_gguf_weight_create) give the
reference's outputs: the oracle expands the same file bytes (build_i8_weight) and runs
op_linear_i8 on the same quantized activations."""
from __future__ import annotations

import numpy as np
import pytest

from nexterabert_cpp_amd import gguf_writer as W
from oracle import ggml_blocks as gb

pytestmark = pytest.mark.gpu


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


@pytest.fixture(scope="module")
def torch():
    import torch as t
    assert t.cuda.is_available(), "no GPU"
    return t


def test_linear_from_gguf_matches_oracle(nxg, orc, torch, tmp_path):
    nxg.init()
    rng = np.random.default_rng(4)
    shapes = {"blocks.0.attn.c_q.weight": (nxg.TYPE_Q8_0, 1024, 1024),
              "blocks.0.mlp.c_fc.weight": (nxg.TYPE_Q4_K, 1024, 2304),
              "blocks.0.mlp.c_proj.weight": (nxg.TYPE_Q6_K, 2304, 1024)}
    tensors = []
    for name, (ttype, n_in, n_out) in shapes.items():
        rows = (0.02 * rng.standard_normal((n_out, n_in))).astype(np.float32)
        tensors.append((name, ttype, (n_in, n_out), nxg.quantize_weight(ttype, rows).tobytes()))
    path = tmp_path / "m.gguf"
    W.write_gguf(path, [("general.architecture", W.STRING, "nexterabert")], tensors)
    T = 333
    ref_tensors = {name: (t, raw) for name, t, _, raw in gb.read_gguf(path)[1]}
    with nxg.GGUF(path) as g:
        dev = g.load_int8_weights()
        assert sorted(dev) == sorted(shapes)
        for name, (ttype, n_in, n_out) in shapes.items():
            print(f"gguf linear {name}", flush=True)
            d = dev[name]
            assert (d.n_in, d.n_out) == (n_in, n_out)
            x = rng.standard_normal((T, n_in)).astype(np.float32)
            qa = nxg.quantize_rows(torch.from_numpy(x).cuda())
            y = nxg.linear_i8(d, qa).cpu().numpy()
            # the oracle's side: its own GGUF reader, ggml block decoder and build_i8_weight
            w_ref, scale_ref, off_ref = orc.expand_rows(
                gb.dequantize(ref_tensors[name][0], ref_tensors[name][1], n_in * n_out).reshape(n_out, n_in))
            q_ref, sx_ref = orc.quantize_rows(x)
            y_ref = orc.linear(w_ref, scale_ref, off_ref, q_ref, sx_ref, simd=bool(orc.vnni_flavour()),
                               n_threads=orc.default_threads())
            assert (bits(y) == bits(y_ref)).all()
