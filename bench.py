#!/usr/bin/env python3
"""Benchmark of the int8 linear path of NexteraBERT.cpp on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--rows M] [--no-cpu]

A step is one pass of the path over every int8 projection of the 18-layer encoder
for one packed batch of M rows (default 65,536: one long sequence): for each layer,
each distinct activation a linear reads is quantized once (the reference's
quantize_row), then every projection runs the W8A8 GEMM with the per-block fp32
epilogue (+ residual where the reference adds one). Projections that read the same
activation are concatenated along N into one GEMM (exact per output column), so
the 140 linears run as 92 GEMMs. HRA q/k/v run on M/4 block rows. The MLP's c_fc
reads its fp32 input rows and quantizes them itself where the library's row-tile
kernel does so (from 4 tiles per workgroup; --no-fuse-quant: a quantize launch
first, as for the other inputs); `quantize_first` times that variant of the step. Weights are
N(0, 0.02), Q8_0-encoded, expanded to int8 on the host; activations N(0, 1); all
inputs are resident in HBM before timing starts.

Output: one JSON line. `value` is int8 TOPS of the whole step (quantization
included, 2 ops per MAC of the GEMMs). HIP events around every launch of the timed
steps give `rooflines_by_kernel` (one roofline object per kernel the step launches:
algorithmic ops and bytes per launch, average launch time, the bound its intensity
selects and the fraction of it reached), `roofline` (the GEMM kernel with the largest
share of the step) and `shapes` (per GEMM shape, the fraction of its own roofline bound
min(MFMA peak, intensity x HBM peak)). `linear_path_8192` is the same path at 8,192
rows (one GPU's share of 65,536 rows over 8 GPUs) and `ragged_layer_32docs` one
attention layer's linears over 32 packed documents (M = 32,935, Q4_K_M weights,
cumulative offsets on every launch) beside the same rows as one sequence. `cpu_baseline` times the
CPU oracle (the same path on VPDPBUSD, the reference's instruction) on a row
sample on this host; `mfma_counters` gives each GEMM kind's MFMA-busy %, counted int8
ops and shader clock from a rocprofv3 --pmc pass over the same workload, run as a
child process before this one touches the GPU (--no-counters skips it). The 1,024-token encoder line is the same path at M=1024,
replayed from a HIP graph; `encoder` times the whole encoder forward (nxg_encoder:
embedding, every block, out_norm) on the 213M-parameter model at 1x1024 and 8x1024
tokens and on one 8,192- and one 65,536-token document, beside the reference's published CPU timings of
the same calls.
"""
from __future__ import annotations

import argparse
import json
import os
import shutil
import signal
import statistics
import subprocess
import sys
import tempfile
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "int8 linear TOPS (% of MFMA peak) + encoder tokens/s at 1,024-token seqs"
PEAK_INT8_TOPS = 5000.0   # MI355X dense int8 MFMA, 5.0 POPS
PEAK_HBM_GBS = 8000.0     # MI355X HBM3E, 8 TB/s


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def LinearPath(nxg, M: int, **kw):
    """The encoder's int8 linear path over one sequence of M rows (the package's
    EncoderLinearPath)."""
    from nexterabert_cpp_amd.encoder import EncoderLinearPath
    return EncoderLinearPath(nxg, [M], **kw)


def time_steps(path, steps: int, warmup: int):
    """W untimed steps, then K steps with HIP events around every launch (on the launching
    stream). Returns ms per step (events around the K steps), wall ms per step, GEMM ms per
    step by output kind, quantize ms per step, and the event lists."""
    torch = path.torch
    for _ in range(warmup):
        path.step()
    torch.cuda.synchronize()
    gemm_ev, quant_ev = [], []
    t0 = time.perf_counter()
    s0 = torch.cuda.Event(enable_timing=True)
    s1 = torch.cuda.Event(enable_timing=True)
    s0.record()
    for _ in range(steps):
        path.step(gemm_ev, quant_ev)
    s1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    total_ms = s0.elapsed_time(s1)
    gemm_ms = {}
    for a, b, g, kind, rows, res in gemm_ev:
        k = "relu2" if kind in ("relu2", "relu2_f32") else "fp32"
        gemm_ms[k] = gemm_ms.get(k, 0.0) + a.elapsed_time(b) / steps
    quant_ms = sum(e[0].elapsed_time(e[1]) for e in quant_ev)
    return total_ms / steps, wall / steps * 1e3, gemm_ms, quant_ms / steps, gemm_ev, quant_ev


RIDGE = PEAK_INT8_TOPS * 1e12 / (PEAK_HBM_GBS * 1e9)     # int8 ops per HBM byte


def roofline_of(kernel: str, n_launch: int, ms_total: float, ops: int, nbytes: int, steps: int) -> dict:
    """Roofline object of one kernel over n_launch launches taking ms_total together: the
    MFMA peak when its algorithmic intensity (ops / bytes per launch) is above the ridge,
    else HBM bandwidth. achieved = algorithmic ops (or bytes) per launch / average launch
    time."""
    avg_s = ms_total * 1e-3 / n_launch
    ops_pl, bytes_pl = ops / n_launch, nbytes / n_launch
    ai = ops / nbytes if nbytes else 0.0
    if ops and ai >= RIDGE:
        r = {"bound": "mfma", "achieved": round(ops_pl / avg_s / 1e12, 2), "peak": PEAK_INT8_TOPS, "unit": "TFLOP/s"}
    else:
        r = {"bound": "hbm", "achieved": round(bytes_pl / avg_s / 1e9, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s"}
    r["frac"] = round(r["achieved"] / r["peak"], 4)
    r["traffic"] = None
    r["kernel"] = kernel
    r["launches_per_step"] = round(n_launch / steps, 2)
    r["ms_per_step"] = round(ms_total / steps, 4)
    r["per_launch"] = {"algorithmic_ops": int(ops_pl), "algorithmic_bytes": int(bytes_pl),
                       "avg_us": round(avg_s * 1e6, 2), "arith_intensity": round(ai, 1),
                       "int8_tops": round(ops_pl / avg_s / 1e12, 2), "gb_per_s": round(bytes_pl / avg_s / 1e9, 1)}
    return r


def kernel_rooflines(nxg, gemm_ev, quant_ev, steps: int) -> list:
    """One roofline object per kernel the step launches (the GEMM kernel of each launch as
    the launch plan picks it, nxg_gemm_kernel_name; the quantize kernel), most time first."""
    from nexterabert_cpp_amd.encoder import gemm_bytes, gemm_f32_relu2_bytes, quantize_bytes
    acc = {}
    for a, b, g, kind, rows, res in gemm_ev:
        relu2, f32_in = kind in ("relu2", "relu2_f32"), kind == "relu2_f32"
        name = nxg.gemm_kernel_name(rows, g.n_in, g.n_out, residual=res, relu2=relu2, f32_in=f32_in)
        d = acc.setdefault(name, [0, 0.0, 0, 0])
        d[0] += 1
        d[1] += a.elapsed_time(b)
        d[2] += 2 * rows * g.n_in * g.n_out
        d[3] += (gemm_f32_relu2_bytes(rows, g.n_in, g.n_out) if f32_in
                 else gemm_bytes(rows, g.n_in, g.n_out, relu2, res))
    for a, b, rows, n_in, relu2 in quant_ev:
        d = acc.setdefault(f"quantize_kernel<127, {int(relu2)}>", [0, 0.0, 0, 0])
        d[0] += 1
        d[1] += a.elapsed_time(b)
        d[3] += quantize_bytes(rows, n_in)
    out = [roofline_of(k, n, ms, ops, nb, steps) for k, (n, ms, ops, nb) in acc.items()]
    return sorted(out, key=lambda r: -r["ms_per_step"])


def shape_table(gemm_ev, steps: int) -> list:
    """Per GEMM shape of the step: average launch time, int8 TOPS, and the shape's roofline
    bound min(MFMA peak, AI x HBM peak) with the fraction of it reached."""
    from nexterabert_cpp_amd.encoder import gemm_bytes, gemm_f32_relu2_bytes
    acc = {}
    for a, b, g, kind, rows, res in gemm_ev:
        relu2, f32_in = kind in ("relu2", "relu2_f32"), kind == "relu2_f32"
        k = (rows, g.n_in, g.n_out, bool(res), relu2, f32_in)
        d = acc.setdefault(k, [0, 0.0, g.name])
        d[0] += 1
        d[1] += a.elapsed_time(b)
    out = []
    for (rows, n_in, n_out, res, relu2, f32_in), (n, ms, name) in acc.items():
        ops = 2 * rows * n_in * n_out
        nb = gemm_f32_relu2_bytes(rows, n_in, n_out) if f32_in else gemm_bytes(rows, n_in, n_out, relu2, res)
        avg_us = ms * 1e3 / n
        tops = ops / (avg_us * 1e-6) / 1e12
        bound = min(PEAK_INT8_TOPS, ops / nb * PEAK_HBM_GBS / 1e3)
        out.append({"shape": f"{rows}x{n_in}->{n_out}" + (" +res" if res else "") + (" relu2->int8" if relu2 else "")
                    + (" from fp32 rows" if f32_in else ""),
                    "example": name.split(".")[-2] if "." in name else name,
                    "launches_per_step": round(n / steps, 2), "avg_us": round(avg_us, 2),
                    "int8_tops": round(tops, 1), "pct_of_mfma_peak": round(100 * tops / PEAK_INT8_TOPS, 2),
                    "bound_tops": round(bound, 1), "frac_of_bound": round(tops / bound, 4)})
    return sorted(out, key=lambda r: -r["avg_us"] * r["launches_per_step"])


def path_line(nxg, path, steps: int, warmup: int, workload: str) -> dict:
    """A linear-path workload other than the headline one: ms per step, int8 TOPS, tokens/s,
    the per-shape table and the per-kernel rooflines."""
    ms, wall_ms, gemm_ms, quant_ms, gemm_ev, quant_ev = time_steps(path, steps, warmup)
    tops = path.ops / (ms * 1e-3) / 1e12
    return {"workload": workload, "rows": path.M, "n_seqs": len(path.lengths), "gemm_launches": path.n_gemm,
            "quantize_launches": path.n_quant, "ms_per_step": round(ms, 4), "int8_tops": round(tops, 2),
            "pct_of_mfma_peak": round(100 * tops / PEAK_INT8_TOPS, 2),
            "tokens_per_s": round(path.M / (ms * 1e-3), 1),
            "gemm_ms_per_step": {k: round(v, 4) for k, v in gemm_ms.items()},
            "quantize_ms_per_step": round(quant_ms, 4),
            "shapes": shape_table(gemm_ev, steps), "kernels": kernel_rooflines(nxg, gemm_ev, quant_ev, steps)}


# The ragged batch of 32 documents (lengths numpy.random.default_rng(1).integers(16, 2048, 32,
# endpoint=True)), M = 32,935, through one attention layer's projections with Q4_K_M weights.
RAGGED_LENGTHS = [977, 1056, 1551, 1948, 86, 309, 1689, 1944, 522, 649, 1782, 876, 571, 1698, 538, 847,
                  1324, 1133, 190, 72, 1775, 1547, 1719, 1110, 1678, 686, 936, 1618, 267, 632, 268, 937]


def ragged_layer_line(nxg, steps: int, warmup: int) -> dict:
    """One attention layer's linears (fused QKV, c_gate, c_proj + residual, c_fc -> relu^2 ->
    int8, mlp.c_proj + residual) over the packed 32-document batch, cu_offsets on every
    launch, beside the same rows as one sequence with the same weights."""
    from nexterabert_cpp_amd.encoder import EncoderLinearPath
    lengths = [int(n) for n in np.random.default_rng(1).integers(16, 2048, 32, endpoint=True)]
    assert lengths == RAGGED_LENGTHS
    ragged = EncoderLinearPath(nxg, lengths, kinds=["attn"], preset="Q4_K_M")
    r = path_line(nxg, ragged, steps, warmup,
                  "one attention layer's 5 int8 linears (QKV fused) over 32 packed documents, Q4_K_M weights")
    one = EncoderLinearPath(nxg, [ragged.M], kinds=["attn"], preset="Q4_K_M", weights=ragged.dev_weights)
    # the packed batch against the same rows as one sequence: alternating, best of 3 each
    t_ragged, t_one = [r["ms_per_step"]], []
    for i in range(3):
        t_one.append(time_steps(one, steps, warmup)[0])
        if i < 2:
            t_ragged.append(time_steps(ragged, steps, warmup)[0])
    r["lengths"] = lengths
    r["weights"] = "random N(0, 0.02); c_q, c_k, c_fc Q4_K; c_v, c_gate, c_proj, mlp.c_proj Q6_K; expanded to int8"
    r["ragged_ms_best_of_3"] = round(min(t_ragged), 4)
    r["one_sequence_same_rows_ms_best_of_3"] = round(min(t_one), 4)
    r["ragged_over_one_sequence"] = round(min(t_ragged) / min(t_one), 4)
    del ragged, one
    return r


def time_graph(path, steps: int, warmup: int):
    """The step captured once in a HIP graph and replayed; checked against eager."""
    torch = path.torch
    path.step()
    torch.cuda.synchronize()
    eager = {k: v.clone() for k, v in path.outs.items()}
    eager_q = {k: (v.q.clone(), v.sx.view(torch.int32).clone()) for k, v in path.qacts.items()}
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        path.step()
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        path.step()
    # every replay against the eager result, with eager work between the replays
    for i in range(max(3, warmup)):
        g.replay()
        torch.cuda.synchronize()
        for k, v in path.outs.items():
            if not torch.equal(v.view(torch.int32), eager[k].view(torch.int32)):
                raise RuntimeError(f"graph replay {i} differs from eager execution (fp32 rows {k})")
        for k, v in path.qacts.items():
            if not (torch.equal(v.q, eager_q[k][0]) and torch.equal(v.sx.view(torch.int32), eager_q[k][1])):
                raise RuntimeError(f"graph replay {i} differs from eager execution (activations {k})")
        path.step()
        torch.cuda.synchronize()
    s0 = torch.cuda.Event(enable_timing=True)
    s1 = torch.cuda.Event(enable_timing=True)
    s0.record()
    for _ in range(steps):
        g.replay()
    s1.record()
    torch.cuda.synchronize()
    return s0.elapsed_time(s1) / steps


def time_encoder(nxg, steps: int, warmup: int, preset: str = "Q4_K_M", long_tokens=(8192, 65536)):
    """The whole encoder (nxg_encoder) on the 213M-parameter model with random-init
    weights written to a temporary GGUF file: one 1,024-token sequence and a batch of
    8 of them, uniform random ids, then one document of each of `long_tokens` (best of 2
    passes after one warm-up). Timed with HIP events on the launching stream,
    launched eagerly and replayed from a HIP graph (each replay's output compared bit
    for bit with the eager one, eager work between replays). tokens/s = 1000 T B /
    median ms, the reference CLI's rule (tools/cli.cpp:188-203)."""
    import tempfile
    import torch
    from nexterabert_cpp_amd import synth
    out = {"model": f"NexteraBERT 213M (18 blocks: 8 lily, 5 swa, 3 attn, 2 hra), random init, {preset}",
           "data": "synthetic (uniform random token ids)"}
    with tempfile.TemporaryDirectory() as tmp:
        path = Path(tmp) / "nexterabert_random.gguf"
        t0 = time.perf_counter()
        info = synth.write_random_model(nxg, path, preset, seed=0)
        enc = nxg.Encoder(path)
        log(f"encoder model: {info['n_params']} parameters written and loaded in {time.perf_counter() - t0:.1f} s")
    out["n_params"] = info["n_params"]
    rng = np.random.default_rng(0)
    for B in (1, 8):
        lens = [1024] * B
        T = 1024 * B
        tok = torch.from_numpy(rng.integers(0, 50368, T).astype(np.int32)).cuda()
        h = torch.empty((T, 1024), dtype=torch.float32, device="cuda")
        for _ in range(warmup):
            enc.forward(tok, lens, hidden=h)
        torch.cuda.synchronize()
        ev = []
        for _ in range(steps):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            enc.forward(tok, lens, hidden=h)
            b.record()
            ev.append((a, b))
        torch.cuda.synchronize()
        ms = statistics.median(a.elapsed_time(b) for a, b in ev)
        ref = h.clone()
        g = torch.cuda.CUDAGraph()
        hg = torch.empty_like(h)
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            enc.forward(tok, lens, hidden=hg)                # layout uploaded before capture
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        with torch.cuda.graph(g):
            enc.forward(tok, lens, hidden=hg)
        gev, same = [], True
        for i in range(steps):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            hg.zero_()
            a.record()
            g.replay()
            b.record()
            torch.cuda.synchronize()
            gev.append(a.elapsed_time(b))
            same = same and bool(torch.equal(hg.view(torch.int32), ref.view(torch.int32)))
            if i % 4 == 0:
                enc.forward(tok, lens, hidden=h)             # eager work between replays
        gms = statistics.median(gev)
        out[f"{B}x1024"] = {"ms": round(ms, 4), "tokens_per_s": round(T / (ms * 1e-3), 1),
                            "graph_ms": round(gms, 4), "graph_tokens_per_s": round(T / (gms * 1e-3), 1),
                            "graph_replays_equal_eager": same}
        log(f"encoder {B}x1024: {ms:.3f} ms launched, {gms:.3f} ms from a graph -> "
            f"{T / (ms * 1e-3):.0f} / {T / (gms * 1e-3):.0f} tokens/s")
        del g
    for T in long_tokens:
        # one long document: the three-pass attention kernel on its full-attention layers
        tok = torch.from_numpy(rng.integers(0, 50368, T).astype(np.int32)).cuda()
        h = torch.empty((T, 1024), dtype=torch.float32, device="cuda")
        enc.forward(tok, [T], hidden=h)
        torch.cuda.synchronize()
        ms = []
        for _ in range(2):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            enc.forward(tok, [T], hidden=h)
            b.record()
            torch.cuda.synchronize()
            ms.append(a.elapsed_time(b))
        out[f"1x{T}"] = {"ms": round(min(ms), 2), "tokens_per_s": round(T / (min(ms) * 1e-3), 1),
                         "finite": bool(torch.isfinite(h).all())}
        log(f"encoder 1x{T}: {min(ms):.1f} ms -> {T / (min(ms) * 1e-3):.0f} tokens/s")
        del h, tok
        torch.cuda.empty_cache()
    enc.close()
    pub = {"1x1024_ms": 104.9, "8x1024_ms": 876.3, "1x8192_ms": 1716.76, "1x65536_ms": 98951.67,
           "source": "reference README.md:60,76, results/bench_short.json:224, results/bench.json:109-110 "
                     "(Intel Core Ultra 7 265K, 18 threads, AVX-VNNI int8 path, Q4_K_M)"}
    out["reference_published_cpu"] = pub
    for k in ("1x1024", "8x1024", "1x8192", "1x65536"):
        if k in out:
            out[f"speedup_vs_published_{k}"] = round(pub[f"{k}_ms"] / out[k]["ms"], 1)
    return out


def cpu_baseline(path, rows: int, reps: int):
    """The CPU oracle (VPDPBUSD GEMM + AVX2 quantizer, threaded like the reference's pool)
    over the same 92 GEMMs at `rows` rows (HRA block rows at rows/4)."""
    from oracle import oracle as orc
    import nexterabert_cpp_amd.model as model
    orc.build()
    if not orc.vnni_flavour():
        return None
    host = host_cpu()
    # the reference's default pool, hw - hw/10 (src/nexterabert.cpp:1519-1524), of the cores this
    # process may use: its affinity, capped at the 16-core share a one-GPU lease grants
    share = min(CPU_SHARE, host["affinity"])
    n_threads = max(1, share - share // 10)
    rng = np.random.default_rng(1)
    rb = (rows + 3) // 4
    xs = {}
    for steps in path.layers:
        for key, first, wname, okey, res, g, gkind in steps:
            r = rb if g.block_rows else rows
            k = (key[0], key[1], r)
            if first and k not in xs:
                xs[k] = rng.standard_normal((r, key[1])).astype(np.float32)
    resid = rng.standard_normal((rows, model.N_EMBD)).astype(np.float32)
    ops = 0

    def one_pass():
        nonlocal ops
        ops = 0
        for steps in path.layers:
            q = {}
            for key, first, wname, okey, res, g, gkind in steps:
                r = rb if g.block_rows else rows
                k = (key[0], key[1], r)
                if k not in q:
                    q[k] = orc.quantize_rows(xs[k], simd=True, n_threads=n_threads)
                W = path.host_weights[wname]
                y = orc.linear(W.w, W.scale, W.off, q[k][0], q[k][1], res=resid if res else None,
                               simd=True, n_threads=n_threads)
                if g.relu2_into:      # op_relu_sqr quantized for the next linear
                    q[(g.relu2_into, g.n_out, r)] = orc.quantize_rows(orc.relu2(y), simd=True, n_threads=n_threads)
                ops += 2 * r * g.n_in * g.n_out

    one_pass()
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        one_pass()
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    limited = host["affinity"] > CPU_SHARE
    return {
        "value": round(ops / med / 1e12, 4),
        "unit": "TOPS",
        "cores": n_threads,
        "kind": "port",
        "sample": (f"all 140 encoder int8 linears as 92 GEMMs + activation quantization (relu^2 between "
                   f"c_fc and c_proj) at {rows} rows "
                   f"(HRA q/k/v at {rb}), CPU oracle on {orc.vnni_flavour()}, median of {reps} passes "
                   f"after 1 warm-up, {med:.2f} s per pass"),
        "tokens_per_s": round(rows / med, 1),
        "cpu": host["model"],
        "nproc": host["nproc"],
        "affinity": host["affinity"],
        "threads_rule": (f"hw - hw/10 of {share} cores (the reference's default pool size)"
                         + (f"; the lease grants a {CPU_SHARE}-core share of the {host['affinity']} CPUs "
                            "in this process's affinity" if limited else "")),
        "vnni": orc.vnni_flavour(),
    }


CPU_SHARE = 16   # host cores a one-GPU lease grants


def host_cpu() -> dict:
    """The host CPU: model name, logical CPUs, CPUs in this process's affinity."""
    model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    try:
        aff = len(os.sched_getaffinity(0))
    except AttributeError:
        aff = os.cpu_count() or 1
    return {"model": model, "nproc": os.cpu_count() or 1, "affinity": aff}


TRAFFIC_FILE = ROOT / "profiles" / "gemm_traffic_config5.json"

# MFMA utilisation from hardware counters, one rocprofv3 --pmc pass (2 SQ + 1 GRBM counters).
MFMA_COUNTERS = ("SQ_VALU_MFMA_BUSY_CYCLES", "SQ_INSTS_VALU_MFMA_MOPS_I8", "GRBM_GUI_ACTIVE")
N_XCC = 8                      # GRBM_GUI_ACTIVE is summed over the 8 XCDs
INT8_OPS_PER_SIMD_CYCLE = 2048  # v_mfma_i32_32x32x32_i8: 65,536 ops in 32 cycles


def gemm_class(name: str):
    if "gemm_relu2_q8" in name or "gemm_relu2_small" in name or "gemm_relu2_rt" in name:
        return "relu2"
    if "gemm_k256" in name or "gemm_kernel" in name or "gemm_small" in name:
        return "fp32"
    return None


def counter_pass(args) -> int:
    """The child of mfma_counters: the same workload, one warm-up and two steps, under the
    profiler; prints the device's CU count for the parent."""
    import torch
    import __graft_entry__
    nxg = __graft_entry__.load_package()
    torch.cuda.set_device(0)
    nxg.init()
    path = LinearPath(nxg, args.rows, fuse=not args.no_fuse, fuse_mlp=not args.no_fuse_mlp,
                      fuse_quant=not args.no_fuse_quant)
    for _ in range(3):
        path.step()
    torch.cuda.synchronize()
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    print(json.dumps({"counter_pass": "done", "cus": cus, "gemms_per_step": path.n_gemm}), flush=True)
    return 0


def short_name(name: str) -> str:
    """A profiler kernel name without return type, namespace and arguments:
    "gemm_k256<true>", "quantize_kernel<127, 0>"."""
    n = name.replace("(anonymous namespace)::", "").replace("void ", "", 1)
    depth, out = 0, []
    for ch in n:
        if ch == "(" and depth == 0:
            break
        depth += ch == "<"
        depth -= ch == ">"
        out.append(ch)
    return "".join(out).strip()


def summarize_counters(csv_path: Path, cus: int, skip_first: int) -> dict:
    """Per GEMM kind, and per GEMM kernel under "by_kernel", from a counter_collection.csv of
    MFMA_COUNTERS: MFMA-busy % (the MfmaUtil metric: busy cycles summed over all SIMDs /
    (GUI-active cycles of an XCD x SIMDs)), the int8 ops the MFMAs counted (MOPS_I8 x 512),
    the shader clock (GUI-active cycles of an XCD / dispatch time) and the ops rate against
    the peak at that clock. Rates are sums over the dispatches (total ops / total time, total
    busy cycles / total cycles), not means of per-dispatch rates. The first skip_first
    dispatches of each kind (the warm-up step) are left out."""
    import csv
    disp = {}
    for row in csv.DictReader(open(csv_path)):
        kind = gemm_class(row["Kernel_Name"])
        if kind is None:
            continue
        d = disp.setdefault(int(row["Dispatch_Id"]), {"kind": kind, "name": short_name(row["Kernel_Name"])})
        d[row["Counter_Name"]] = float(row["Counter_Value"])
        d["ns"] = int(row["End_Timestamp"]) - int(row["Start_Timestamp"])
    simds = 4 * cus

    def summary(ds):
        cyc = sum(d["GRBM_GUI_ACTIVE"] / N_XCC for d in ds)          # shader cycles of one XCD
        ns = sum(d["ns"] for d in ds)
        ops = sum(d["SQ_INSTS_VALU_MFMA_MOPS_I8"] * 512 for d in ds)
        return {"dispatches": len(ds),
                "mfma_busy_pct": round(100.0 * sum(d["SQ_VALU_MFMA_BUSY_CYCLES"] for d in ds) / (cyc * simds), 2),
                "int8_ops_counted_per_launch": int(ops / len(ds)),
                "clock_ghz": round(cyc / ns, 3),
                "us_per_launch_profiled": round(ns / len(ds) / 1e3, 2),
                "int8_tops_profiled": round(ops / ns / 1e3, 1),
                "pct_of_peak_at_clock": round(100.0 * ops / (simds * INT8_OPS_PER_SIMD_CYCLE * cyc), 2)}

    res = {}
    for kind in ("fp32", "relu2"):
        ds = [disp[k] for k in sorted(disp) if disp[k]["kind"] == kind]
        ds = ds[skip_first * len(ds) // (skip_first + 2):] if ds else ds
        ds = [d for d in ds if all(c in d for c in MFMA_COUNTERS) and d["ns"] > 0]
        if not ds:
            continue
        r = summary(ds)
        r["kernels"] = sorted({d["name"] for d in ds})
        r["by_kernel"] = {n: summary([d for d in ds if d["name"] == n]) for n in r["kernels"]}
        res[kind] = r
    return res


def mfma_counters(args, timeout_s: int = 240) -> dict:
    """MFMA utilisation of the two GEMM kinds from hardware counters: a child process runs
    the same workload (one warm-up and two steps) under rocprofv3 --pmc MFMA_COUNTERS.
    Started before this process touches the GPU; on any failure the reason is returned
    instead of figures."""
    rocprof = shutil.which("rocprofv3") or "/opt/rocm/bin/rocprofv3"
    if not Path(rocprof).exists():
        return {"status": "not measured: rocprofv3 not found"}
    out = Path(tempfile.mkdtemp(prefix="nxg_pmc_", dir="/tmp"))
    child = [sys.executable, str(ROOT / "bench.py"), "--counter-pass", "--rows", str(args.rows)]
    if args.no_fuse:
        child.append("--no-fuse")
    if args.no_fuse_mlp:
        child.append("--no-fuse-mlp")
    if args.no_fuse_quant:
        child.append("--no-fuse-quant")
    cmd = [rocprof, "--pmc", *MFMA_COUNTERS, "--output-format", "csv", "-d", str(out), "-o", "pmc", "--", *child]
    res = {"command": "rocprofv3 --pmc " + " ".join(MFMA_COUNTERS) + " --output-format csv -d DIR -o pmc -- "
                      "python3 bench.py --counter-pass --rows " + str(args.rows)}
    t0 = time.perf_counter()
    try:
        proc = subprocess.Popen(cmd, cwd="/tmp", env=dict(os.environ, TMPDIR="/tmp"), stdout=subprocess.PIPE,
                                stderr=subprocess.STDOUT, text=True, start_new_session=True)
        try:
            text, _ = proc.communicate(timeout=timeout_s)
        except subprocess.TimeoutExpired:
            os.killpg(proc.pid, signal.SIGKILL)
            proc.communicate()
            res["status"] = f"not measured: the profiled pass did not finish in {timeout_s} s"
            return res
        info = None
        for line in text.splitlines():
            if line.startswith('{"counter_pass"'):
                info = json.loads(line)
        files = sorted(out.rglob("*counter_collection.csv"))
        # rocprofv3 may end with a signal after a complete run; the child's own line and
        # the CSV say whether the results are whole
        if info is None or not files:
            tail = " | ".join(text.strip().splitlines()[-3:])
            res["status"] = f"not measured: rocprofv3 exit {proc.returncode}: {tail[-300:]}"
            return res
        res.update(summarize_counters(files[0], info["cus"], skip_first=1))
        res["status"] = "ok"
        res["profiled_pass_s"] = round(time.perf_counter() - t0, 1)
        return res
    finally:
        shutil.rmtree(out, ignore_errors=True)


def pmc_summary(fetch_csv: str, write_csv: str, calib_mib: int, out_path: Path, merge: bool = False) -> dict:
    """HBM traffic per launch of each GEMM and quantize kernel from two rocprofv3 --pmc runs
    of this script (FETCH_SIZE, then WRITE_SIZE, KiB per dispatch), each scaled by what the
    same counter reads for the calibration copy of calib_mib MiB (a device to device copy,
    dispatched by the HIP runtime as its copy-buffer kernel). Per kernel name, and per class
    (gemm_fp32, gemm_relu2, quant) as the mean over the class's launches. merge: keep the
    existing file and add this run's entries for the kernels it does not have."""
    import csv

    def per_kernel(path, counter):
        vals, copies = {}, []
        for row in csv.DictReader(open(path)):
            if row["Counter_Name"] != counter:
                continue
            name, v = row["Kernel_Name"], float(row["Counter_Value"])
            if gemm_class(name) or "quantize_kernel" in name:
                vals.setdefault(short_name(name), []).append(v)
            elif "copy" in name.lower():
                copies.append(v)
        return vals, (max(copies) if copies else None)   # the calibration copy is the largest copy

    def cls(n):
        c = gemm_class(n)
        return {"fp32": "gemm_fp32", "relu2": "gemm_relu2"}.get(c, "quant")

    f, fc = per_kernel(fetch_csv, "FETCH_SIZE")
    w, wc = per_kernel(write_csv, "WRITE_SIZE")
    kib = calib_mib * 1024.0
    fs, ws = kib / fc, kib / wc
    res = {"fetch_scale": round(fs, 4), "write_scale": round(ws, 4),
           "calibration": f"plain device copy of {calib_mib} MiB (reads and writes {calib_mib} MiB)",
           "by_kernel": {}}

    def entry(fv, wv):
        fm, wm = sum(fv) / len(fv), sum(wv) / len(wv)
        return {"launches": len(fv), "fetch_bytes_per_launch": int(fm * fs * 1024),
                "write_bytes_per_launch": int(wm * ws * 1024), "hbm_bytes_per_launch": int((fm * fs + wm * ws) * 1024),
                "raw_fetch_kib": round(fm, 1), "raw_write_kib": round(wm, 1)}

    for n in sorted(set(f) & set(w)):
        res["by_kernel"][n] = entry(f[n], w[n])
    for c in ("gemm_fp32", "gemm_relu2", "quant"):
        fv = [v for n in f if cls(n) == c for v in f[n]]
        wv = [v for n in w if cls(n) == c for v in w[n]]
        if fv and wv:
            res[c] = entry(fv, wv)
    if merge and out_path.exists():
        # the existing file stays as it is; this run (e.g. --no-fuse-quant) adds the kernels it lacks
        old = json.loads(out_path.read_text())
        for n, e in res["by_kernel"].items():
            old.setdefault("by_kernel", {}).setdefault(n, e)
        res = old
    out_path.write_text(json.dumps(res, indent=2) + "\n")
    return res


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--rows", type=int, default=65536, help="packed rows M of the timed workload")
    ap.add_argument("--no-fuse", action="store_true", help="one GEMM per linear (140) instead of 92")
    ap.add_argument("--no-fuse-mlp", action="store_true",
                    help="c_fc writes fp32 rows, then relu^2 + quantize (instead of the int8 epilogue)")
    ap.add_argument("--no-fuse-quant", action="store_true",
                    help="every input quantized by its own launch (else c_fc quantizes its fp32 rows itself "
                         "where the library's row-tile kernel does so)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-rows", type=int, default=8192)
    ap.add_argument("--cpu-reps", type=int, default=3)
    ap.add_argument("--no-encoder1024", action="store_true")
    ap.add_argument("--no-encoder", action="store_true", help="skip the whole-encoder timing")
    ap.add_argument("--no-extra-lines", action="store_true",
                    help="skip the M=8192 linear-path line and the ragged 32-document layer line")
    ap.add_argument("--encoder-long", default="8192,65536", metavar="T1,T2",
                    help="also time the whole encoder on one document of each of these lengths ('': none)")
    ap.add_argument("--calib-copy-mib", type=int, default=0,
                    help="run one plain device copy of this many MiB first (PMC counter calibration)")
    ap.add_argument("--no-counters", action="store_true",
                    help="skip the rocprofv3 MFMA-counter pass (MFMA busy %% of both GEMM kinds)")
    ap.add_argument("--counter-pass", action="store_true", help=argparse.SUPPRESS)
    ap.add_argument("--pmc-merge", action="store_true",
                    help="with --pmc-summary: keep the existing file, adding this run's kernels it lacks")
    ap.add_argument("--pmc-summary", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                    help="summarize two rocprofv3 --pmc counter_collection.csv files of a run with "
                         "--calib-copy-mib into " + str(TRAFFIC_FILE.relative_to(ROOT)) + " and exit")
    args = ap.parse_args()
    if args.pmc_summary:
        res = pmc_summary(args.pmc_summary[0], args.pmc_summary[1], args.calib_copy_mib or 512, TRAFFIC_FILE,
                          merge=args.pmc_merge)
        print(json.dumps(res))
        return 0
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              "(the linear path shards by rows with no exchange; see the design notes)", file=sys.stderr)
        return 2
    if args.counter_pass:
        return counter_pass(args)
    counters = None
    if not args.no_counters:
        # before this process initialises the GPU: the profiler runs as a separate child
        counters = mfma_counters(args)
        log(f"MFMA counters: {counters}")

    import torch
    import __graft_entry__
    nxg = __graft_entry__.load_package()
    torch.cuda.set_device(0)
    nxg.init()

    if args.calib_copy_mib:
        n = args.calib_copy_mib * (1 << 20) // 4
        a = torch.empty(n, device="cuda")
        b = torch.empty(n, device="cuda")
        b.copy_(a)
        torch.cuda.synchronize()
        del a, b

    t0 = time.perf_counter()
    path = LinearPath(nxg, args.rows, fuse=not args.no_fuse, fuse_mlp=not args.no_fuse_mlp,
                      fuse_quant=not args.no_fuse_quant)
    torch.cuda.synchronize()
    log(f"setup {time.perf_counter() - t0:.1f} s: M={args.rows}, {path.n_gemm} GEMMs ({path.n_relu2} with the "
        f"relu^2 -> int8 output) + {path.n_quant} quantizations per step, {path.ops / 1e12:.3f} T int8 ops")

    ms, wall_ms, gemm_ms, quant_ms, gemm_ev, quant_ev = time_steps(path, args.steps, args.warmup)
    gemm_total = sum(gemm_ms.values())
    log(f"timed {args.steps} steps: {ms:.3f} ms/step (wall {wall_ms:.3f}), GEMMs {gemm_total:.3f} ms "
        f"({gemm_ms}), quantize {quant_ms:.3f} ms")

    value = path.ops / (ms * 1e-3) / 1e12
    gemm_tops = path.ops / (gemm_total * 1e-3) / 1e12

    # One roofline per kernel; `roofline` is the GEMM kernel with the largest share of the step.
    kernels = kernel_rooflines(nxg, gemm_ev, quant_ev, args.steps)
    tr = json.loads(TRAFFIC_FILE.read_text()) if TRAFFIC_FILE.exists() else {}
    use_traffic = args.rows == 65536 and not args.no_fuse and not args.no_fuse_mlp

    def annotate(rs):
        for r in rs:
            by = (tr.get("by_kernel") or {}).get(r["kernel"])
            if use_traffic and by:
                r["traffic"] = by["hbm_bytes_per_launch"]
                r["traffic_over_algorithmic"] = round(by["hbm_bytes_per_launch"] / r["per_launch"]["algorithmic_bytes"], 3)
            for kind in ("fp32", "relu2"):
                bk = ((counters or {}).get(kind) or {}).get("by_kernel", {}).get(r["kernel"])
                if bk:
                    r["mfma_busy_pct"] = bk["mfma_busy_pct"]
    annotate(kernels)
    roof = dict(next(r for r in kernels if not r["kernel"].startswith("quantize")))
    if roof.get("traffic") is not None:
        roof["traffic_source"] = (f"{TRAFFIC_FILE.relative_to(ROOT)}: rocprofv3 FETCH_SIZE x {tr['fetch_scale']} + "
                                  f"WRITE_SIZE x {tr['write_scale']} per launch of this kernel in this workload")
    roof_relu2 = next((r for r in kernels if r["kernel"].startswith("gemm_relu2")), None)
    shapes = shape_table(gemm_ev, args.steps)
    log(f"dominant kernel {roof['kernel']}: {roof['per_launch']['avg_us']} us/launch, frac {roof['frac']}")

    # The same step with c_fc reading a qact written by its own quantize launch: the relu^2
    # GEMM's roofline without the input quantization inside it.
    qfirst = None
    if not args.no_extra_lines and path.n_relu2_f32:
        pq = LinearPath(nxg, args.rows, fuse=not args.no_fuse, weights=path.dev_weights,
                        fuse_mlp=not args.no_fuse_mlp, fuse_quant=False)
        ql = path_line(nxg, pq, args.steps, args.warmup, "the same step, every input quantized by its own launch")
        qfirst = {k: ql[k] for k in ("workload", "ms_per_step", "int8_tops", "quantize_launches",
                                     "gemm_ms_per_step", "quantize_ms_per_step")}
        annotate(ql["kernels"])
        qfirst["roofline_relu2_q8"] = next((r for r in ql["kernels"] if r["kernel"].startswith("gemm_relu2")), None)
        log(f"quantize first: {qfirst['ms_per_step']} ms/step, relu2 kernel frac "
            f"{(qfirst['roofline_relu2_q8'] or {}).get('frac')}")
        del pq

    m8k = None
    if not args.no_extra_lines and args.rows != 8192:
        p8 = LinearPath(nxg, 8192, fuse=not args.no_fuse, weights=path.dev_weights, fuse_mlp=not args.no_fuse_mlp,
                        fuse_quant=not args.no_fuse_quant)
        m8k = path_line(nxg, p8, max(args.steps, 20), args.warmup,
                        "all 140 encoder int8 projections, one 8192-token sequence (one GPU's share of 65,536 "
                        "rows over 8 GPUs)")
        log(f"M=8192: {m8k['ms_per_step']} ms/step, {m8k['int8_tops']} TOPS")
        del p8
    ragged = None
    if not args.no_extra_lines:
        ragged = ragged_layer_line(nxg, max(args.steps, 20), args.warmup)
        log(f"ragged 32-document layer: {ragged['ms_per_step']} ms/step, {ragged['int8_tops']} TOPS, "
            f"x{ragged['ragged_over_one_sequence']} of one sequence")

    enc = None
    if not args.no_encoder1024:
        p1k = LinearPath(nxg, 1024, fuse=not args.no_fuse, weights=path.dev_weights, fuse_mlp=not args.no_fuse_mlp,
                         fuse_quant=not args.no_fuse_quant)
        p1k.host_weights = path.host_weights
        ms1k = time_graph(p1k, max(args.steps, 20), args.warmup)
        enc = {"tokens_per_s": round(1024 / (ms1k * 1e-3), 1), "ms_per_step": round(ms1k, 4),
               "int8_tops": round(p1k.ops / (ms1k * 1e-3) / 1e12, 2), "rows": 1024,
               "mode": "HIP graph replay of the step"}
        log(f"encoder linear path at 1024 tokens: {ms1k:.3f} ms -> {enc['tokens_per_s']:.0f} tokens/s")
        del p1k

    full = None
    if not args.no_encoder:
        long_tokens = [int(t) for t in args.encoder_long.split(",") if t.strip()]
        full = time_encoder(nxg, max(args.steps, 20), args.warmup, long_tokens=long_tokens)

    cpu = None
    if not args.no_cpu:
        t0 = time.perf_counter()
        cpu = cpu_baseline(path, args.cpu_rows, args.cpu_reps)
        log(f"cpu baseline {time.perf_counter() - t0:.1f} s: {cpu}")

    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (N(0,1) activations, N(0,0.02) weights -> Q8_0 -> int8)",
        "config": {"workload": f"all 140 encoder int8 projections, one {args.rows}-token sequence",
                   "rows": args.rows, "gemm_launches": path.n_gemm, "quantize_launches": path.n_quant,
                   "fused_shared_inputs": not args.no_fuse,
                   "mlp_relu2_int8_epilogue": path.n_relu2 > 0,
                   "c_fc_quantizes_fp32_rows": path.n_relu2_f32, "weights": "Q8_0 expanded to int8",
                   "parallelism": "single GPU"},
        "pct_of_mfma_peak": round(100 * value / PEAK_INT8_TOPS, 2),
        "mfma_counters": counters,
        "tokens_per_s": round(args.rows / (ms * 1e-3), 1),
        "gemm_only": {"int8_tops": round(gemm_tops, 2), "pct_of_mfma_peak": round(100 * gemm_tops / PEAK_INT8_TOPS, 2),
                      "ms_per_step": round(gemm_total, 4),
                      "ms_per_step_by_output": {k: round(v, 4) for k, v in gemm_ms.items()}},
        "quantize": {"ms_per_step": round(quant_ms, 4),
                     "gb_per_s": round(path.quant_bytes / (quant_ms * 1e-3) / 1e9, 1) if quant_ms else None},
        "encoder_1024": enc,
        "encoder": full,
        "roofline": roof,
        # the relu^2 GEMM from a qact (the quantize_first step) where the headline step's c_fc
        # quantizes its fp32 rows itself; that kernel's roofline is roofline_relu2_f32_in
        "roofline_relu2_q8": dict((qfirst or {}).get("roofline_relu2_q8") or {}, step="quantize_first")
                             if (qfirst or {}).get("roofline_relu2_q8") else roof_relu2,
        "roofline_relu2_f32_in": roof_relu2 if path.n_relu2_f32 else None,
        "quantize_first": qfirst,
        "rooflines_by_kernel": kernels,
        "shapes": shapes,
        "linear_path_8192": m8k,
        "ragged_layer_32docs": ragged,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
