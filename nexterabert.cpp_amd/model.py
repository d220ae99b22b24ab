"""The int8 linears of the NexteraBERT encoder, per layer, as the reference's graph builder
emits them (src/nexterabert.cpp:1185-1289), with the file-type rule that picks each
weight's GGUF block type (tools/quantize.cpp:79-98).

Model dimensions are those of the 213M-parameter checkpoint: n_embd 1024, 18 layers, FFN
2304, 16 query / 8 KV heads of 64, SnowLily rank 64, HRA block 4. The order of the 18
blocks (8 lily, 5 swa, 3 attn, 2 hra) is not stored in the reference's sources; the
order used here does not change any linear's shape.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Dict, List

N_EMBD = 1024
N_LAYER = 18
N_INTER = 2304
N_HEAD = 16
N_KV_HEAD = 8
HEAD_DIM = 64
LILY_RANK = 64
HRA_BLOCK = 4
BLOCK_TYPES = ["lily"] * 8 + ["swa"] * 5 + ["attn"] * 3 + ["hra"] * 2

# ggml type ids
Q8_0, Q5_0, Q4_K, Q6_K = 8, 6, 12, 14


@dataclass
class LinearSpec:
    name: str            # GGUF tensor name
    n_in: int
    n_out: int
    input: str           # which activation of the layer it reads (linears that share one share its qact)
    residual: bool = False     # + residual stream (c_proj of the mixer and of the MLP)
    block_rows: bool = False   # HRA q/k/v: run on ceil(len/4) block rows per sequence
    relu2_into: str = ""       # the output only feeds relu^2 into this input (the MLP's c_fc)


@dataclass
class LinearGroup:
    """Linears that read the same activation, run as one GEMM over the weights concatenated
    along the output dimension (exact per output column)."""
    input: str
    specs: List[LinearSpec] = field(default_factory=list)

    @property
    def n_in(self) -> int:
        return self.specs[0].n_in

    @property
    def n_out(self) -> int:
        return sum(s.n_out for s in self.specs)

    @property
    def residual(self) -> bool:
        return any(s.residual for s in self.specs)

    @property
    def block_rows(self) -> bool:
        return self.specs[0].block_rows

    @property
    def relu2_into(self) -> str:
        return self.specs[0].relu2_into if len(self.specs) == 1 else ""

    @property
    def name(self) -> str:
        return "+".join(s.name.rsplit(".", 2)[-2] for s in self.specs) if len(self.specs) > 1 else self.specs[0].name


def layer_linears(l: int, kind: str) -> List[LinearSpec]:
    """The int8 linears of block l, in graph order (src/nexterabert.cpp:1217-1289)."""
    blk = f"blocks.{l}."
    pre = blk + "attn."
    C, kv = N_EMBD, N_KV_HEAD * HEAD_DIM
    out: List[LinearSpec] = []
    if kind in ("attn", "swa"):
        # mix_attn :1217 -> attention :1185-1188 -> gated_out :1208-1213
        out += [LinearSpec(pre + "c_q.weight", C, C, "h"),
                LinearSpec(pre + "c_k.weight", C, kv, "h"),
                LinearSpec(pre + "c_v.weight", C, kv, "h"),
                LinearSpec(pre + "c_gate.weight", C, C, "attn_out"),
                LinearSpec(pre + "c_proj.weight", C, C, "gate_out", residual=True)]
    elif kind == "lily":
        # mix_lily :1226-1244
        r = LILY_RANK
        out += [LinearSpec(pre + "ltc_conv.in_proj.weight", C, r, "h"),
                LinearSpec(pre + "ltc_conv.A.weight", C, r, "h"),
                LinearSpec(pre + "ltc_conv.out_proj.weight", r, C, "conv_out"),
                LinearSpec(pre + "x_proj.weight", C, C, "h"),
                LinearSpec(pre + "B_proj.weight", C, C, "h"),
                LinearSpec(pre + "c_proj.weight", C, C, "state_out", residual=True)]
    elif kind == "hra":
        # mix_hra :1246-1268
        out += [LinearSpec(pre + "qkv_in.weight", C, C, "h"),
                LinearSpec(pre + "qkv_gate.weight", C, C, "h"),
                LinearSpec(pre + "c_q.weight", C, C, "block_mean", block_rows=True),
                LinearSpec(pre + "c_k.weight", C, kv, "block_mean", block_rows=True),
                LinearSpec(pre + "c_v.weight", C, kv, "block_mean", block_rows=True),
                LinearSpec(pre + "c_C.weight", C, C, "h"),
                LinearSpec(pre + "c_gate.weight", C, C, "attn_out"),
                LinearSpec(pre + "c_proj.weight", C, C, "gate_out", residual=True)]
    else:
        raise ValueError(kind)
    # MLP :1284-1289
    out += [LinearSpec(blk + "mlp.c_fc.weight", C, N_INTER, "mlp_in", relu2_into="relu_out"),
            LinearSpec(blk + "mlp.c_proj.weight", N_INTER, C, "relu_out", residual=True)]
    return out


def layer_groups(l: int, kind: str, fuse: bool = True) -> List[LinearGroup]:
    """The layer's linears grouped by shared input (fuse=False: one group per linear)."""
    groups: Dict[str, LinearGroup] = {}
    order: List[LinearGroup] = []
    for s in layer_linears(l, kind):
        if fuse and s.input in groups:
            groups[s.input].specs.append(s)
            continue
        g = LinearGroup(s.input, [s])
        order.append(g)
        if fuse:
            groups[s.input] = g
    return order


def encoder_linears() -> List[LinearSpec]:
    return [s for l, k in enumerate(BLOCK_TYPES) for s in layer_linears(l, k)]


def wants_more_bits(name: str) -> bool:
    """The "_M" presets' rule (tools/quantize.cpp:79-83)."""
    return (name.endswith(".attn.c_proj.weight") or name.endswith(".mlp.c_proj.weight")
            or name.endswith(".attn.c_v.weight") or name.endswith(".attn.c_gate.weight")
            or name in ("mlm.dense.weight", "head.dense.weight", "pooler.dense.weight"))


def file_type_of(name: str, n_in: int, preset: str) -> int:
    """Block type of a weight in a Q8_0 or Q4_K_M file, with the K-quant row fallback
    (tools/quantize.cpp:87-98,172-182)."""
    if preset == "Q8_0":
        return Q8_0
    if preset != "Q4_K_M":
        raise ValueError(preset)
    t = Q6_K if wants_more_bits(name) else Q4_K
    if n_in % 256:
        t = {Q4_K: Q5_0, Q6_K: Q8_0}[t]
    return t


def linear_ops_per_token() -> int:
    """int8 ops (2 per MAC) of the encoder's linears per token; HRA q/k/v count 1/4."""
    tot = 0
    for s in encoder_linears():
        macs = s.n_in * s.n_out
        tot += 2 * macs // (HRA_BLOCK if s.block_rows else 1)
    return tot
