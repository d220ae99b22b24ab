"""GPU: int8 linear weights loaded from a GGUF file (nxg_gguf_weight_create) give the
reference's outputs: the oracle expands the same file bytes (build_i8_weight) and runs
op_linear_i8 on the same quantized activations."""
from __future__ import annotations

import numpy as np
import pytest

import gguf_writer as W

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
            E = nxg.expand_weight(ttype, g.tensor_bytes(name), n_in, n_out)
            q_ref, sx_ref = orc.quantize_rows(x)
            y_ref = orc.linear(E.w, E.scale, E.off, q_ref, sx_ref, simd=bool(orc.vnni_flavour()),
                               n_threads=orc.default_threads())
            assert (bits(y) == bits(y_ref)).all()
