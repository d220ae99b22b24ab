"""The encoder's int8 linear path over one packed batch, on one GPU.

Every int8 projection of the 18 layers, in the order the reference's graph builder
emits them (src/nexterabert.cpp:1185-1289). Per layer each distinct activation a linear
reads is quantized once (builder::linear's qcache, :1121-1143); projections that read the
same activation run as one GEMM over their weights concatenated along N (exact per output
column); the MLP's c_fc writes c_proj's int8 activations through the fused relu^2
epilogue (op_relu_sqr feeding an int8 linear, :484-505, :1284-1289). HRA q/k/v run on
each sequence's ceil(len / 4) block rows. Rows are the packed batch: every GEMM gets the
batch's cumulative offsets (prepare_batch, :1341-1354).

The producers of the activations (norms, attention, convolutions, the SnowLily state,
block means) are not on this path: their outputs are synthetic fp32 rows, N(0, 1), made
on the GPU once. Weights are random N(0, 0.02) encoded as Q8_0, or read from a GGUF
file; either way they are expanded on the host as build_i8_weight does (:1010-1049) and
uploaded once.
"""
from __future__ import annotations

from typing import Dict, List, Optional, Sequence

import numpy as np

from . import model


def gemm_bytes(rows: int, n_in: int, n_out: int, relu2: bool, residual: bool) -> int:
    """Algorithmic HBM bytes of one GEMM launch: int8 activations and their scales, int8
    weights and their scales, then the output -- fp32 rows (+ the fp32 residual read), or
    for the relu^2 -> int8 epilogue the next linear's int8 activations and scales."""
    nb, nb_out = (n_in + 255) // 256, (n_out + 255) // 256
    b = rows * n_in + 4 * rows * nb + n_out * n_in + 4 * n_out * nb
    if relu2:
        return b + rows * n_out + 4 * rows * nb_out
    return b + 4 * rows * n_out * (2 if residual else 1)


def gemm_f32_relu2_bytes(rows: int, n_in: int, n_out: int) -> int:
    """Algorithmic HBM bytes of the relu^2 GEMM that quantizes its fp32 input rows itself:
    the fp32 rows, int8 weights and their scales, the next linear's int8 activations and
    scales."""
    nb, nb_out = (n_in + 255) // 256, (n_out + 255) // 256
    return 4 * rows * n_in + n_out * n_in + 4 * n_out * nb + rows * n_out + 4 * rows * nb_out


def quantize_bytes(rows: int, n_in: int) -> int:
    """Algorithmic HBM bytes of one quantize_row pass: fp32 in, int8 and the scales out."""
    return 5 * rows * n_in + 4 * rows * ((n_in + 255) // 256)


class EncoderLinearPath:
    """Device buffers and the launch sequence of one forward of the linear path.

    lengths   sequence lengths of the packed batch (rows = their sum)
    fuse      run linears that share an input as one GEMM
    fuse_mlp  c_fc -> relu^2 -> int8 in one kernel (else fp32 rows, then
              quantize_rows_relu2)
    fuse_quant  c_fc reads its fp32 input rows and quantizes them itself
              (linear_f32_relu2_q8: quantize_row inside the GEMM, for the shapes where the
              library's row-tile kernel does so) instead of a quantize_rows launch before it
    weights   device weights from an earlier path (same fuse setting), reused
    gguf      an open nxg.GGUF holding the encoder's int8 tensors (else random weights)
    kinds     the block kind of each layer to run (default: the 18 blocks of the model);
              e.g. ["attn"] for the linears of one attention layer
    preset    block types of the random weights: "Q8_0" everywhere, or the "Q4_K_M" mix
              (Q4_K, Q6_K where the _M rule wants more bits; tools/quantize.cpp:79-98)
    """

    def __init__(self, nxg, lengths: Sequence[int], fuse: bool = True, weights=None, seed: int = 0,
                 fuse_mlp: bool = True, gguf=None, kinds: Optional[Sequence[str]] = None,
                 preset: str = "Q8_0", fuse_quant: bool = True):
        import torch
        lengths = [int(n) for n in lengths]
        if not lengths or min(lengths) <= 0:
            raise ValueError("lengths: need at least one sequence, each of at least one token")
        self.nxg, self.torch = nxg, torch
        self.lengths = lengths
        self.M = sum(lengths)
        block_lengths = [(n + model.HRA_BLOCK - 1) // model.HRA_BLOCK for n in lengths]
        rows_block = sum(block_lengths)
        single = len(lengths) == 1
        self.cu = None if single else nxg.cu_offsets_of(lengths)
        self.cu_block = None if single else nxg.cu_offsets_of(block_lengths)
        rng = np.random.default_rng(seed)
        gen = torch.Generator(device="cuda").manual_seed(seed)
        types = {t.name: t for t in gguf.tensors()} if gguf is not None else {}
        self.layers = []
        self.host_weights: Dict[str, object] = {}
        self.dev_weights = {} if weights is None else weights
        self.inputs, self.qacts, self.outs = {}, {}, {}
        self.residual = torch.randn(self.M, model.N_EMBD, device="cuda", generator=gen)
        self.ops = 0
        self.ops_fp32 = self.ops_relu2 = 0
        self.gemm_bytes = 0       # algorithmic HBM bytes of the fp32-output GEMMs
        self.relu2_bytes = 0      # ... of the c_fc -> relu^2 -> int8 GEMMs
        self.quant_bytes = 0      # ... of the standalone quantizations
        self.relu2_f32_bytes = 0  # ... of the relu^2 GEMMs quantizing their fp32 input rows
        self.fuse_quant = fuse_quant and fuse_mlp
        M = self.M
        self.preset = preset
        for l, kind in enumerate(model.BLOCK_TYPES if kinds is None else kinds):
            steps = []
            seen = set()
            made = set()          # qact keys produced by a GEMM of this layer (relu^2 -> int8)
            for g in model.layer_groups(l, kind, fuse):
                rows = rows_block if g.block_rows else M
                key = (g.input, g.n_in, rows)
                if key not in self.qacts:
                    self.qacts[key] = nxg.qact_alloc(rows, g.n_in)
                if key not in made and key not in self.inputs:
                    self.inputs[key] = torch.randn(rows, g.n_in, device="cuda", generator=gen)
                okey = (g.n_out, rows)
                gkind = "fp32"
                if g.relu2_into:
                    # c_fc: its output only feeds relu^2 into the next linear's qact
                    gkind = "relu2" if fuse_mlp else "relu2_unfused"
                    rkey = (g.relu2_into, g.n_out, rows)
                    if rkey not in self.qacts:
                        self.qacts[rkey] = nxg.qact_alloc(rows, g.n_out)
                    made.add(rkey)
                    okey = rkey if fuse_mlp else okey
                if gkind != "relu2" and okey not in self.outs:      # fp32 rows out
                    self.outs[okey] = torch.empty(rows, g.n_out, device="cuda")
                wname = g.name if len(g.specs) == 1 else f"blocks.{l}.{g.name}"
                if wname not in self.dev_weights:
                    parts = [self._expand(nxg, s, rng, gguf, types, preset) for s in g.specs]
                    W = parts[0] if len(parts) == 1 else nxg.I8Weight(
                        np.concatenate([p.w for p in parts]),
                        np.ascontiguousarray(np.concatenate([p.scale for p in parts], 1)),
                        np.ascontiguousarray(np.concatenate([p.off for p in parts], 1)))
                    self.host_weights[wname] = W
                    self.dev_weights[wname] = nxg.DeviceWeight(W)
                first = key not in seen and key not in made
                seen.add(key)
                res = g.residual
                if (gkind == "relu2" and first and self.fuse_quant
                        and nxg.gemm_kernel_name(rows, g.n_in, g.n_out, relu2=True,
                                                 f32_in=True).endswith("true>")):
                    gkind = "relu2_f32"
                steps.append((key, first, wname, okey, res, g, gkind))
                ops = 2 * rows * g.n_in * g.n_out
                self.ops += ops
                if gkind == "relu2_f32":
                    self.ops_relu2 += ops
                    self.relu2_f32_bytes += gemm_f32_relu2_bytes(rows, g.n_in, g.n_out)
                elif gkind == "relu2":
                    self.ops_relu2 += ops
                    self.relu2_bytes += gemm_bytes(rows, g.n_in, g.n_out, relu2=True, residual=False)
                else:
                    self.ops_fp32 += ops
                    self.gemm_bytes += gemm_bytes(rows, g.n_in, g.n_out, relu2=False, residual=res)
                if gkind == "relu2_unfused":      # fp32 rows, then relu^2 + quantize_row
                    self.quant_bytes += quantize_bytes(rows, g.n_out)
                if first and gkind != "relu2_f32":
                    self.quant_bytes += quantize_bytes(rows, g.n_in)
            self.layers.append(steps)
        self.n_gemm = sum(len(s) for s in self.layers)
        self.n_relu2 = sum(1 for s in self.layers for st in s if st[6] in ("relu2", "relu2_f32"))
        self.n_relu2_f32 = sum(1 for s in self.layers for st in s if st[6] == "relu2_f32")
        self.n_quant = sum(1 for s in self.layers for st in s
                           if (st[1] and st[6] != "relu2_f32") or st[6] == "relu2_unfused")

    @staticmethod
    def _expand(nxg, spec, rng, gguf, types, preset):
        if gguf is None:
            rows_f = (0.02 * rng.standard_normal((spec.n_out, spec.n_in))).astype(np.float32)
            t = model.file_type_of(spec.name, spec.n_in, preset)
            return nxg.expand_weight(t, nxg.quantize_weight(t, rows_f), spec.n_in, spec.n_out)
        info = types.get(spec.name)
        if info is None:
            raise KeyError(f"{spec.name}: not in the GGUF file")
        if info.n_dims != 2 or tuple(info.ne[:2]) != (spec.n_in, spec.n_out):
            raise ValueError(f"{spec.name}: ne {info.ne[:info.n_dims]} in the file, expected ({spec.n_in}, {spec.n_out})")
        return nxg.expand_weight(info.type, gguf.tensor_bytes(spec.name), spec.n_in, spec.n_out)

    def _timed(self, events, fn, *tag):
        if events is None:
            fn()
            return
        e = self.torch.cuda.Event(enable_timing=True)
        fn()
        e.record()
        events.append((self._mark, e) + tag)
        self._mark = e                         # this launch's end is the next one's start

    def step(self, gemm_events: Optional[List] = None, quant_events: Optional[List] = None) -> None:
        """One forward of the path on the current stream. With event lists, every GEMM and
        every quantization is bracketed by HIP events: one event before the first launch and
        one after each launch, so consecutive launches share the event between them. GEMM
        entries are (start, end, group, kind, rows, residual), quantization entries (start,
        end, rows, n_in, relu2)."""
        nxg = self.nxg
        if gemm_events is not None or quant_events is not None:
            if gemm_events is None or quant_events is None:
                raise ValueError("step: pass both event lists or neither")
            self._mark = self.torch.cuda.Event(enable_timing=True)
            self._mark.record()
        for steps in self.layers:
            for key, first, wname, okey, res, g, gkind in steps:
                qa = self.qacts[key]
                w = self.dev_weights[wname]
                cu = self.cu_block if g.block_rows else self.cu
                if gkind == "relu2_f32":
                    # quantize_row inside the GEMM (or into qa first where no fused kernel runs)
                    self._timed(gemm_events, lambda: nxg.linear_f32_relu2_q8(w, self.inputs[key], cu_offsets=cu,
                                                                             out=self.qacts[okey], workspace=qa),
                                g, "relu2_f32", qa.T, False)
                    continue
                if first:
                    self._timed(quant_events, lambda: nxg.quantize_rows(self.inputs[key], out=qa), qa.T, g.n_in, False)
                if gkind == "relu2":
                    self._timed(gemm_events, lambda: nxg.linear_i8_relu2_q8(w, qa, cu_offsets=cu, out=self.qacts[okey]),
                                g, gkind, qa.T, False)
                    continue
                self._timed(gemm_events, lambda: nxg.linear_i8(w, qa, residual=self.residual if res else None,
                                                               cu_offsets=cu, out=self.outs[okey]), g, gkind, qa.T, res)
                if gkind == "relu2_unfused":
                    rkey = (g.relu2_into, g.n_out, qa.T)
                    self._timed(quant_events, lambda: nxg.quantize_rows_relu2(self.outs[okey], out=self.qacts[rkey]),
                                qa.T, g.n_out, True)
