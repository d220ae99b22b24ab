"""CPU restatement of the NexteraBERT encoder's forward pass: nextera_load's preparation of
the tensors (src/nexterabert.cpp:1549-1712) and builder::encoder (:1206-1292) with
prepare_batch (:1341-1371) and run_forward's pooling (:1913-1925), composed from the
oracle's restated ops (oracle.py over nx_oracle.cpp).

TEST INFRASTRUCTURE ONLY: the checker that the GPU encoder (include/nxg_encoder.h) is
compared against. Only the test suite, the smoke check and the benchmark's CPU-baseline leg
use it; nothing in the product imports it.

Inputs are decoded tensors: from_gguf reads the GGUF file and decodes each tensor's blocks
to float32 with the oracle's own reader and decoders (ggml_blocks.py, pinned by known-answer
blocks and against the engine's separately written decoders; their parity with a compiled
ggml is pinned only up to its block layouts). From there this module restates everything
the reference does:
the metadata defaults, the int8 placement rule and build_i8_weight (orc_expand_rows), the
conv kernels re-laid out one row per tap, and each op of the graph in order.

Each op's own pins are in tests/test_oracle_*.py; the composition is pinned by the
structure tests in tests/test_oracle_encoder.py (a sequence alone equals it inside a
batch, layer by layer equality with the ops called one at a time, closed forms at zero
weights).
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Dict, List, Optional, Sequence

import numpy as np

from . import ggml_blocks as gb
from . import oracle as orc

MIXERS = ("lily", "swa", "attn", "hra")
_FLOAT_TYPES = (0, 1, 30)      # F32, F16, BF16: not "quantized" for the int8 rule


@dataclass
class HParams:
    """nextera_load's hyperparameters and defaults (src/nexterabert.cpp:1574-1626)."""
    n_vocab: int
    n_embd: int
    n_layer: int
    n_inter: int
    n_head: int
    n_kv_head: int
    head_dim: int
    lily_rank: int
    hra_block: int
    swa_window: int
    ntk_train_len: int
    rope_base: float
    swa_rope_base: float
    ssmax_base: float
    rms_eps: float
    ln_eps: float
    ssmax: int                 # 0 none, 1 ssmax, 2 sssmax
    block_types: List[str] = field(default_factory=list)

    @classmethod
    def from_metadata(cls, meta: Dict[str, object]) -> "HParams":
        k = "nexterabert."
        f32 = lambda key, d: float(np.float32(meta.get(key, d)))
        n_embd, n_head = int(meta[k + "embedding_length"]), int(meta[k + "attention.head_count"])
        head_dim = n_embd // n_head
        mode = str(meta.get(k + "ssmax.mode", "sssmax"))
        types = [str(t) for t in meta[k + "block_types"]]
        assert all(t in MIXERS for t in types)
        return cls(n_vocab=int(meta[k + "vocab_size"]), n_embd=n_embd, n_layer=int(meta[k + "block_count"]),
                   n_inter=int(meta[k + "feed_forward_length"]), n_head=n_head,
                   n_kv_head=int(meta[k + "attention.head_count_kv"]), head_dim=head_dim,
                   lily_rank=int(meta.get(k + "lily.low_rank", head_dim)),
                   hra_block=int(meta.get(k + "hra.block_size", 4)), swa_window=int(meta.get(k + "swa.window", 256)),
                   ntk_train_len=int(meta.get(k + "rope.ntk_train_length", 0)),
                   rope_base=f32(k + "rope.freq_base", 100000.0), swa_rope_base=f32(k + "swa.rope.freq_base", 10000.0),
                   ssmax_base=f32(k + "ssmax.base", 0.1), rms_eps=f32(k + "rms_norm_epsilon", 1e-8),
                   ln_eps=f32(k + "layer_norm_epsilon", 1e-5),
                   ssmax=0 if mode == "none" else 1 if mode == "ssmax" else 2, block_types=types)


def is_int8(name: str, n_dims: int, ggml_type: int, ne0: int, ne1: int) -> bool:
    """The placement rule of nextera_load (src/nexterabert.cpp:1658-1667), use_int8 on."""
    if name in ("embedding.weight", "mlm.decoder.weight", "token_type_embeddings.weight"):
        return False
    return n_dims == 2 and ggml_type not in _FLOAT_TYPES and ne0 % 32 == 0 and ne1 % 4 == 0


@dataclass
class Linear:
    w: np.ndarray       # int8 [n_out][n_in]
    scale: np.ndarray   # [n_blk][n_out]
    off: np.ndarray     # [n_blk][n_out]


class Model:
    """tensors: name -> (ggml type, ne tuple, decoded float32 array, [ne1][ne0] for 2-D)."""

    def __init__(self, meta: Dict[str, object], tensors: Dict[str, tuple], act_max: int = 127):
        self.hp = HParams.from_metadata(meta)
        self.act_max = act_max
        self.lin: Dict[str, Linear] = {}
        self.f: Dict[str, np.ndarray] = {}
        for name, (ggml_type, ne, arr) in tensors.items():
            nd = len(ne)
            if is_int8(name, nd, ggml_type, ne[0], ne[1] if nd > 1 else 1):
                w, sc, off = orc.expand_rows(arr.reshape(ne[1], ne[0]), act_off=act_max + 1)
                self.lin[name] = Linear(w, sc, off)
                continue
            a = np.ascontiguousarray(arr, np.float32)
            if name.endswith(".depthwise.weight") or name.endswith(".kernel"):
                a = np.ascontiguousarray(a.reshape(ne[1], ne[0]).T)     # [C][k] -> one row per tap [k][C]
            self.f[name] = a
        self.n_types = self.f["token_type_embeddings.weight"].shape[0] if "token_type_embeddings.weight" in self.f else 0


def from_gguf(path, act_max: int = 127) -> Model:
    """A Model from a GGUF file, read and block-decoded by the oracle's own GGUF reader and
    ggml decoders (ggml_blocks.py), not the engine's."""
    meta, raw = gb.read_gguf(path)
    tensors = {}
    for name, t, ne, data in raw:
        n = int(np.prod(ne))
        arr = gb.dequantize(t, data, n)
        tensors[name] = (t, ne, arr.reshape(ne[1], ne[0]) if len(ne) == 2 else arr.reshape(-1))
    return Model(meta, tensors, act_max)


class Forward:
    """One forward pass of builder::encoder over a packed batch."""

    def __init__(self, m: Model, lengths: Sequence[int], n_threads: Optional[int] = None):
        self.m, hp = m, m.hp
        self.lengths = [int(n) for n in lengths]
        assert self.lengths and min(self.lengths) > 0
        self.cu = np.concatenate([[0], np.cumsum(self.lengths)]).astype(np.int32)
        nb = [(n + hp.hra_block - 1) // hp.hra_block for n in self.lengths]
        self.cub = np.concatenate([[0], np.cumsum(nb)]).astype(np.int32)
        self.T = int(self.cu[-1])
        self.threads = n_threads or orc.default_threads()
        max_len = max(self.lengths)
        base = hp.rope_base
        if hp.ntk_train_len > 0 and max_len > hp.ntk_train_len:      # dynamic NTK (:1356-1366)
            assert len(self.lengths) == 1, "sequences beyond rope.ntk_train_length are encoded one at a time"
            d = float(hp.head_dim)
            base = float(np.float32(float(base) * (max_len / hp.ntk_train_len) ** (d / (d - 2.0))))
        self.rope = [orc.rope_table(max_len, base, hp.head_dim), orc.rope_table(max_len, hp.swa_rope_base, hp.head_dim)]

    # builder::linear (src/nexterabert.cpp:1121-1143) on the int8 path: quantize_row, op_linear_i8
    def linear(self, name: str, x: np.ndarray, res: Optional[np.ndarray] = None) -> np.ndarray:
        L = self.m.lin[name]
        q, sx = orc.quantize_rows(x, self.m.act_max, simd=True, n_threads=self.threads)
        return orc.linear(L.w, L.scale, L.off, q, sx, res, simd=True, n_threads=self.threads)

    def scales(self, pre: str, cu: np.ndarray, mode: int) -> np.ndarray:
        f = self.m.f
        s = float(f[pre + "scalable_factor.s"][0]) if mode else 0.0
        b = float(f[pre + "scalable_factor.b"][0]) if mode == 2 else 0.0
        return np.array([orc.attention_scale(int(n), self.m.hp.head_dim, mode, s, b, self.m.hp.ssmax_base)
                         for n in np.diff(cu)], np.float32)

    # builder::attention (:1184-1204)
    def attention(self, pre: str, h: np.ndarray, cu: np.ndarray, rope, half: int, scale: np.ndarray) -> np.ndarray:
        hp, f = self.m.hp, self.m.f
        G, D = hp.n_kv_head, hp.head_dim
        T = h.shape[0]
        c, s = rope
        q = orc.qk_prep(self.linear(pre + "c_q.weight", h), f[pre + "q_norm.alpha"], f[pre + "q_norm.beta"], c, s, cu,
                        hp.n_head)
        k = orc.qk_prep(self.linear(pre + "c_k.weight", h), f[pre + "k_norm.alpha"], f[pre + "k_norm.beta"], c, s, cu,
                        G, head_major=True)
        v = np.ascontiguousarray(self.linear(pre + "c_v.weight", h).reshape(T, G, D).transpose(1, 0, 2))
        return orc.attention(q, k, v, cu, scale, hp.n_head, G, half)

    # builder::gated_out (:1206-1213)
    def gated_out(self, pre: str, y: np.ndarray, z: np.ndarray, x: np.ndarray) -> np.ndarray:
        gl = self.linear(pre + "c_gate.weight", y)
        return self.linear(pre + "c_proj.weight", orc.gate(gl, z), x)

    def block(self, l: int, x: np.ndarray) -> np.ndarray:
        hp, f = self.m.hp, self.m.f
        blk = f"blocks.{l}."
        pre = blk + "attn."
        kind = hp.block_types[l]
        h = orc.rms_norm(x, f[blk + "attn_norm.weight"], hp.rms_eps)
        if kind in ("attn", "swa"):                                     # mix_attn (:1215-1222)
            swa = kind == "swa"
            half = max(1, hp.swa_window // 2) if swa else -1
            y = self.attention(pre, h, self.cu, self.rope[1 if swa else 0], half,
                               self.scales(pre, self.cu, 0 if swa else hp.ssmax))
            x = self.gated_out(pre, y, y, x)
        elif kind == "lily":                                            # mix_lily (:1224-1244)
            z = self.linear(pre + "ltc_conv.in_proj.weight", h)
            r = self.linear(pre + "ltc_conv.A.weight", h)
            lr = orc.dwconv(z, f[pre + "ltc_conv.kernel"], self.cu, r=r)
            a = self.linear(pre + "ltc_conv.out_proj.weight", lr)
            xp = self.linear(pre + "x_proj.weight", h)
            b = self.linear(pre + "B_proj.weight", h)
            st = orc.lily_state(a, xp, b, f[pre + "state_conv.depthwise.weight"], self.cu)
            x = self.linear(pre + "c_proj.weight", st, x)
        else:                                                           # mix_hra (:1246-1268)
            i = self.linear(pre + "qkv_in.weight", h)
            ci = orc.dwconv(i, f[pre + "qkv_conv.depthwise.weight"], self.cu)
            gt = self.linear(pre + "qkv_gate.weight", h)
            hb = orc.block_mean(ci, self.cu, hp.hra_block, g=gt)
            yb = self.attention(pre, hb, self.cub, self.rope[0], -1, self.scales(pre, self.cub, hp.ssmax))
            y = orc.upsample_add(yb, self.linear(pre + "c_C.weight", h), self.cu, hp.hra_block)
            co = orc.dwconv(y, f[pre + "c_o.depthwise.weight"], self.cu)
            x = self.gated_out(pre, y, co, x)
        # x + c_proj(relu(c_fc(norm(x)))^2) (:1284-1289)
        h = orc.rms_norm(x, f[blk + "mlp_norm.weight"], hp.rms_eps)
        u = self.linear(blk + "mlp.c_fc.weight", h)
        return self.linear(blk + "mlp.c_proj.weight", orc.relu2(u), x)

    def embed(self, tokens: np.ndarray, types: Optional[np.ndarray]) -> np.ndarray:
        f = self.m.f
        x = f["embedding.weight"].reshape(-1, self.m.hp.n_embd)[tokens]
        if types is not None and self.m.n_types > 0:
            x = (x + f["token_type_embeddings.weight"][types]).astype(np.float32)
        return np.ascontiguousarray(x, np.float32)


def encode(m: Model, tokens, lengths, token_types=None, n_layers: int = -1, normalize: bool = False,
           n_threads: Optional[int] = None, layer_outputs: Optional[list] = None):
    """nextera_encode_segments (hidden, pooled). n_layers >= 0: the first n_layers blocks
    and the residual stream before out_norm (nextera_debug_set_layers). layer_outputs, if a
    list, receives the residual stream after each block."""
    fw = Forward(m, lengths, n_threads)
    tokens = np.asarray(tokens, np.int32)
    types = None if token_types is None else np.asarray(token_types, np.int32)
    assert tokens.size == fw.T and ((tokens >= 0) & (tokens < m.hp.n_vocab)).all()
    x = fw.embed(tokens, types)
    n = m.hp.n_layer if n_layers < 0 else min(n_layers, m.hp.n_layer)
    for l in range(n):
        x = fw.block(l, x)
        if layer_outputs is not None:
            layer_outputs.append(x)
    if n_layers < 0:
        x = orc.layer_norm(x, m.f["out_norm.weight"], m.f["out_norm.bias"], m.hp.ln_eps)
    return x, orc.doc_mean(x, fw.cu, normalize=normalize)
