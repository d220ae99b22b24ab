"""Random-init NexteraBERT GGUF files: every tensor builder::encoder reads
(src/nexterabert.cpp:1206-1292), under the metadata keys the converter writes
(python/convert_hf_to_gguf.py:178-209), with the block types tools/quantize.cpp gives each
tensor (:70-98, :165-182): matrices (2-D ".weight", both sides >= 32) at the preset's base
type, the ones feeding the residual stream, c_v and c_gate at its "more bits" type, rows
that do not divide into K-quant super-blocks at the fallback type; norms, DyT curves, conv
kernels and scalars stay F32.

Values: linear weights N(0, 0.02) (the benchmarks' synthetic weights), embeddings N(0, 1),
norm gains and DyT beta U(0.8, 1.2), DyT alpha U(0.3, 1), conv taps U(-0.5, 0.5),
Scalable-Softmax s U(0.2, 0.5) and b U(-0.1, 0.3) (a negative b exercises max(b, 0)),
out_norm bias N(0, 0.02). The default dimensions are the 213M-parameter checkpoint's.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Dict, List, Optional

import numpy as np

from . import gguf_writer as W
from . import model

F32, F16, Q4_0, Q5_0, Q8_0, Q4_K, Q6_K = 0, 1, 2, 6, 8, 12, 14
_BLCK = {F32: 1, F16: 1, Q5_0: 32, Q8_0: 32, Q4_K: 256, Q6_K: 256}
# preset -> (general.file_type, base type, "more bits" type) (tools/quantize.cpp's presets)
PRESETS = {"Q8_0": (7, Q8_0, Q8_0), "Q4_K_M": (15, Q4_K, Q6_K), "Q6_K": (18, Q6_K, Q6_K)}


@dataclass
class Dims:
    n_vocab: int = 50368
    n_embd: int = model.N_EMBD
    n_inter: int = model.N_INTER
    n_head: int = model.N_HEAD
    n_kv_head: int = model.N_KV_HEAD
    lily_rank: int = model.LILY_RANK
    lily_kernel: int = 5
    hra_kernel: int = 3
    hra_block: int = model.HRA_BLOCK
    swa_window: int = 256
    block_types: List[str] = field(default_factory=lambda: list(model.BLOCK_TYPES))
    n_types: int = 0                  # rows of token_type_embeddings (0: none in the file)
    ssmax_mode: str = "sssmax"
    rope_base: float = 100000.0
    swa_rope_base: float = 10000.0
    ntk_train_len: int = 0

    @property
    def head_dim(self) -> int:
        return self.n_embd // self.n_head


def wants_more_bits(name: str) -> bool:
    """tools/quantize.cpp:78-82."""
    return (name.endswith(".attn.c_proj.weight") or name.endswith(".mlp.c_proj.weight")
            or name.endswith(".attn.c_v.weight") or name.endswith(".attn.c_gate.weight")
            or name in ("mlm.dense.weight", "head.dense.weight", "pooler.dense.weight"))


def fallback_for_row(t: int, n_per_row: int) -> int:
    """tools/quantize.cpp:86-98: K-quants need rows of whole 256-blocks."""
    if n_per_row % _BLCK[t] == 0:
        return t
    t = {Q4_K: Q5_0, Q6_K: Q8_0}.get(t, t)
    return t if n_per_row % _BLCK[t] == 0 else F32


def model_tensors(d: Dims, seed: int = 0) -> Dict[str, np.ndarray]:
    """name -> float32 array in numpy order ([ne1][ne0] for matrices; conv kernels [C][k])."""
    rng = np.random.default_rng(seed)
    C, KV, R, I, D = d.n_embd, d.n_kv_head * d.head_dim, d.lily_rank, d.n_inter, d.head_dim

    def lin(n_in, n_out):
        return (rng.standard_normal((n_out, n_in), dtype=np.float32) * np.float32(0.02)).astype(np.float32)

    def unif(lo, hi, *shape):
        return rng.uniform(lo, hi, shape).astype(np.float32)

    t: Dict[str, np.ndarray] = {"embedding.weight": rng.standard_normal((d.n_vocab, C), dtype=np.float32)}
    if d.n_types > 0:
        t["token_type_embeddings.weight"] = rng.standard_normal((d.n_types, C), dtype=np.float32)
    for l, kind in enumerate(d.block_types):
        blk = f"blocks.{l}."
        pre = blk + "attn."
        t[blk + "attn_norm.weight"] = unif(0.8, 1.2, C)

        def attn(scalars: bool):
            t[pre + "c_q.weight"] = lin(C, C)
            t[pre + "c_k.weight"] = lin(C, KV)
            t[pre + "c_v.weight"] = lin(C, KV)
            for n in ("q_norm", "k_norm"):
                t[pre + n + ".alpha"] = unif(0.3, 1.0, D)
                t[pre + n + ".beta"] = unif(0.8, 1.2, D)
            if scalars:
                t[pre + "scalable_factor.s"] = unif(0.2, 0.5, 1)
                t[pre + "scalable_factor.b"] = unif(-0.1, 0.3, 1)
            t[pre + "c_gate.weight"] = lin(C, C)
            t[pre + "c_proj.weight"] = lin(C, C)

        if kind in ("attn", "swa"):
            attn(kind == "attn")
        elif kind == "lily":
            t[pre + "ltc_conv.in_proj.weight"] = lin(C, R)
            t[pre + "ltc_conv.A.weight"] = lin(C, R)
            t[pre + "ltc_conv.kernel"] = unif(-0.5, 0.5, R, d.lily_kernel)
            t[pre + "ltc_conv.out_proj.weight"] = lin(R, C)
            t[pre + "x_proj.weight"] = lin(C, C)
            t[pre + "B_proj.weight"] = lin(C, C)
            t[pre + "state_conv.depthwise.weight"] = unif(-0.5, 0.5, C, d.lily_kernel)
            t[pre + "c_proj.weight"] = lin(C, C)
        elif kind == "hra":
            t[pre + "qkv_in.weight"] = lin(C, C)
            t[pre + "qkv_conv.depthwise.weight"] = unif(-0.5, 0.5, C, d.hra_kernel)
            t[pre + "qkv_gate.weight"] = lin(C, C)
            t[pre + "c_C.weight"] = lin(C, C)
            t[pre + "c_o.depthwise.weight"] = unif(-0.5, 0.5, C, d.hra_kernel)
            attn(True)
        else:
            raise ValueError(f"unsupported block type {kind!r}")
        t[blk + "mlp_norm.weight"] = unif(0.8, 1.2, C)
        t[blk + "mlp.c_fc.weight"] = lin(C, I)
        t[blk + "mlp.c_proj.weight"] = lin(I, C)
    t["out_norm.weight"] = unif(0.8, 1.2, C)
    t["out_norm.bias"] = (rng.standard_normal(C, dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    return t


def file_type_of(name: str, arr: np.ndarray, preset: str) -> int:
    """The block type tools/quantize.cpp:165-182 gives a tensor under `preset`."""
    _, base, more = PRESETS[preset]
    is_matrix = (arr.ndim == 2 and name.endswith(".weight") and name != "classifier.weight"
                 and arr.shape[1] >= 32 and arr.shape[0] >= 32)
    if not is_matrix:
        return F32
    return fallback_for_row(more if wants_more_bits(name) else base, arr.shape[1])


def encode_tensor(nxg, arr: np.ndarray, type_: int) -> bytes:
    if type_ == F32:
        return np.ascontiguousarray(arr, np.float32).tobytes()
    return nxg.quantize_weight(type_, arr.reshape(-1, arr.shape[-1])).tobytes()


def metadata(d: Dims, preset: str) -> list:
    k = "nexterabert."
    return [
        ("general.architecture", W.STRING, "nexterabert"),
        ("general.name", W.STRING, "nexterabert-random"),
        ("general.file_type", W.UINT32, PRESETS[preset][0]),
        ("general.quantization_version", W.UINT32, 2),
        (k + "vocab_size", W.UINT32, d.n_vocab),
        (k + "embedding_length", W.UINT32, d.n_embd),
        (k + "block_count", W.UINT32, len(d.block_types)),
        (k + "feed_forward_length", W.UINT32, d.n_inter),
        (k + "attention.head_count", W.UINT32, d.n_head),
        (k + "attention.head_count_kv", W.UINT32, d.n_kv_head),
        (k + "block_types", W.ARRAY, (W.STRING, list(d.block_types))),
        (k + "lily.low_rank", W.UINT32, d.lily_rank),
        (k + "lily.kernel_size", W.UINT32, d.lily_kernel),
        (k + "hra.block_size", W.UINT32, d.hra_block),
        (k + "swa.window", W.UINT32, d.swa_window),
        (k + "rope.freq_base", W.FLOAT32, d.rope_base),
        (k + "swa.rope.freq_base", W.FLOAT32, d.swa_rope_base),
        (k + "rope.ntk_train_length", W.UINT32, d.ntk_train_len),
        (k + "ssmax.mode", W.STRING, d.ssmax_mode),
        (k + "ssmax.base", W.FLOAT32, 0.1),
        (k + "rms_norm_epsilon", W.FLOAT32, 1e-8),
        (k + "layer_norm_epsilon", W.FLOAT32, 1e-5),
        (k + "mlm_head", W.BOOL, False),
        ("tokenizer.ggml.cls_token_id", W.UINT32, 50281),
        ("tokenizer.ggml.seperator_token_id", W.UINT32, 50282),
        ("tokenizer.ggml.padding_token_id", W.UINT32, 50283),
        ("tokenizer.ggml.mask_token_id", W.UINT32, 50284),
    ]


def write_random_model(nxg, path, preset: str = "Q4_K_M", seed: int = 0, dims: Optional[Dims] = None,
                       tensors: Optional[Dict[str, np.ndarray]] = None, extra_metadata: Optional[list] = None,
                       extra_tensors: Optional[Dict[str, np.ndarray]] = None) -> dict:
    """Writes a random-init model file (or the given tensors, model_tensors' layout);
    returns {"n_params", "types": {name: block type}}. extra_metadata: (key, type, value)
    entries added to the converter's keys (replacing one of the same key); extra_tensors:
    more tensors (heads, for instance), typed by the same rule."""
    d = dims or Dims()
    if preset not in PRESETS:
        raise ValueError(f"preset must be one of {sorted(PRESETS)}")
    if tensors is None:
        tensors = model_tensors(d, seed)
    if extra_tensors:
        tensors = {**tensors, **extra_tensors}
    meta = metadata(d, preset)
    if extra_metadata:
        keys = {k for k, _, _ in extra_metadata}
        meta = [m for m in meta if m[0] not in keys] + list(extra_metadata)
    entries, types = [], {}
    for name in sorted(tensors):                 # the converter writes tensors sorted by name
        arr = tensors[name]
        t = file_type_of(name, arr, preset)
        ne = tuple(reversed(arr.shape)) if arr.ndim == 2 else (arr.size,)
        entries.append((name, t, ne, encode_tensor(nxg, arr, t)))
        types[name] = t
    W.write_gguf(path, meta, entries)
    return {"n_params": int(sum(a.size for a in tensors.values())), "types": types}
