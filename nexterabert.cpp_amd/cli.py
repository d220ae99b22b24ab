#!/usr/bin/env python3
"""Command line for the int8 linear path, with the reference CLI's --bench rule.

    python nexterabert.cpp_amd/cli.py --info [-m model.gguf]
    python nexterabert.cpp_amd/cli.py --bench T [--batch B] [--reps R] [--profile] [-m model.gguf]

--bench times forward passes of the encoder's int8 linear path (every projection of the
18 layers with its activation quantization, EncoderLinearPath) over B packed sequences
of T tokens, the way tools/cli.cpp:177-204 times nextera_encode: 3 untimed passes, then
R timed ones, each measured on the host clock around a pass that ends with a device
synchronization; it prints the median and the minimum and tokens/s = 1000 * T * B /
median_ms. The producers of the activations are not on the path and run as synthetic
rows (see encoder.py). Weights are random Q8_0 unless -m names a GGUF file holding the
encoder's tensors. --graph replays the pass from a HIP graph instead of launching it.
--profile adds the device time per kind of launch from HIP events on one extra pass.

    python nexterabert.cpp_amd/cli.py --bench T --encode [--batch B] [--reps R] [--profile] [-m model.gguf]

--encode times the whole encoder instead (nxg_encoder_encode, the counterpart of
nextera_encode, on host buffers), exactly as tools/cli.cpp:177-204 times nextera_encode:
ids uniform in [1000, min(vocab, 40000)) from a fixed seed with CLS first and SEP last in
each sequence, the pooled vectors L2-normalised as the only output. Without -m the model
is the 213M-parameter architecture with random-init weights, written as Q4_K_M to a
temporary file. With --profile the timed passes are profiled (nxg_encoder_profile) and the
reference's --profile report follows: ms per pass of the int8 linears, attention and row
ops (device time from HIP events), everything else, and the total wall time.
"""
from __future__ import annotations

import argparse
import statistics
import sys
import time
from pathlib import Path
from typing import List, Optional

_ROOT = Path(__file__).resolve().parent.parent

# ggml's file types (general.file_type), named as src/nexterabert.cpp:1390-1410 names them.
FTYPE_NAMES = {0: "F32", 1: "F16", 2: "Q4_0", 3: "Q4_1", 7: "Q8_0", 8: "Q5_0", 9: "Q5_1", 10: "Q2_K",
               11: "Q3_K_S", 12: "Q3_K_M", 13: "Q3_K_L", 14: "Q4_K_S", 15: "Q4_K_M", 16: "Q5_K_S",
               17: "Q5_K_M", 18: "Q6_K"}


def _package():
    if str(_ROOT) not in sys.path:
        sys.path.insert(0, str(_ROOT))
    import __graft_entry__
    return __graft_entry__.load_package()


def ftype_name(ft: Optional[int]) -> str:
    return FTYPE_NAMES.get(ft, "unknown") if ft is not None else "unknown"


def parse_args(argv: Optional[List[str]] = None) -> argparse.Namespace:
    ap = argparse.ArgumentParser(prog="cli.py", description="int8 linear path of NexteraBERT on one MI355X")
    ap.add_argument("-m", "--model", help="GGUF file with the encoder's weights (default: random Q8_0)")
    ap.add_argument("--info", action="store_true", help="print device / library / model info")
    ap.add_argument("--bench", type=int, default=0, metavar="T", help="time passes over random sequences of T tokens")
    ap.add_argument("--batch", type=int, default=1, metavar="B", help="sequences per pass in --bench (default 1)")
    ap.add_argument("--reps", type=int, default=20, metavar="R", help="timed repetitions in --bench (default 20)")
    ap.add_argument("--profile", action="store_true", help="with --bench: print where the time goes")
    ap.add_argument("--graph", action="store_true", help="with --bench: replay each pass from a HIP graph")
    ap.add_argument("--no-fuse-mlp", action="store_true", help="c_fc writes fp32 rows, then relu^2 + quantize")
    ap.add_argument("--encode", action="store_true", help="with --bench: time the whole encoder (nxg_encoder)")
    args = ap.parse_args(argv)
    if args.bench < 0 or args.batch < 1 or args.reps < 1:
        ap.error("--bench T >= 1, --batch B >= 1 and --reps R >= 1")
    return args


def info(nxg, gguf) -> List[str]:
    import torch
    lines = [f"library: {nxg.load_library()._name}"]
    if torch.cuda.is_available():
        p = torch.cuda.get_device_properties(0)
        lines.append(f"device: {p.name} ({getattr(p, 'gcnArchName', '?')}), {p.multi_processor_count} CUs, "
                     f"{p.total_memory / 2**30:.0f} GiB")
    else:
        lines.append("device: none (the int8 path needs a gfx950 GPU)")
    if gguf is not None:
        names = gguf.int8_names()
        lines.append(f"model: GGUF v{gguf.version}, {ftype_name(gguf.get('general.file_type'))}, "
                     f"architecture {gguf.get('general.architecture', '?')}, {len(gguf.tensors())} tensors, "
                     f"{len(names)} int8 linears")
    return lines


def bench(nxg, args, gguf) -> str:
    import torch
    from nexterabert_cpp_amd.encoder import EncoderLinearPath
    nxg.init()
    path = EncoderLinearPath(nxg, [args.bench] * args.batch, gguf=gguf, fuse_mlp=not args.no_fuse_mlp)
    ftype = ftype_name(gguf.get("general.file_type")) if gguf is not None else "Q8_0 (random weights)"
    run = path.step
    if args.graph:
        stream = torch.cuda.Stream()
        stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(stream):
            path.step()
        torch.cuda.current_stream().wait_stream(stream)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            path.step()
        run = g.replay
    ms = []
    for r in range(args.reps + 3):
        t0 = time.perf_counter()
        run()
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        if r >= 3:
            ms.append((t1 - t0) * 1e3)
    ms.sort()
    med = ms[len(ms) // 2]
    T, B = args.bench, args.batch
    lines = [f"bench: {ftype}  T={T}  batch={B}  {'graph' if args.graph else 'eager'}  "
             f"median {med:.3f} ms  min {ms[0]:.3f} ms  ({1000.0 * T * B / med:.0f} tokens/s)"]
    if args.profile:
        gemm_ev, quant_ev = [], []
        path.step(gemm_ev, quant_ev)
        torch.cuda.synchronize()
        per = {}
        for a, b, grp, kind, *_ in gemm_ev:
            k = f"GEMM {'relu^2 -> int8' if kind == 'relu2' else 'fp32 out'}"
            n, t = per.get(k, (0, 0.0))
            per[k] = (n + 1, t + a.elapsed_time(b))
        per["quantize"] = (len(quant_ev), sum(e[0].elapsed_time(e[1]) for e in quant_ev))
        total = sum(t for _, t in per.values())
        for k, (n, t) in per.items():
            lines.append(f"  {k:22s} {n:4d} launches  {t:8.3f} ms  {100 * t / total:5.1f}%")
        lines.append(f"  {path.ops / 1e9:.1f} G int8 ops per pass: {path.ops / (med * 1e-3) / 1e12:.1f} TOPS at the median")
    return "\n".join(lines)


def bench_encoder(nxg, args) -> str:
    """--bench --encode: the reference CLI's encode benchmark on nxg_encoder."""
    import tempfile
    import numpy as np
    with tempfile.TemporaryDirectory() as tmp:
        path = args.model
        if path is None:
            from nexterabert_cpp_amd import synth
            path = str(Path(tmp) / "nexterabert_random_q4km.gguf")
            synth.write_random_model(nxg, path, "Q4_K_M", seed=0)
        with nxg.GGUF(path) as g:
            ftype = ftype_name(g.get("general.file_type"))
            cls_id = int(g.get("tokenizer.ggml.cls_token_id", -1))
            sep_id = int(g.get("tokenizer.ggml.seperator_token_id", -1))
        enc = nxg.Encoder(path)
    T, B = args.bench, args.batch
    rng = np.random.default_rng(0)
    hi = min(enc.n_vocab, 40000)
    tok = rng.integers(min(1000, hi - 1), hi, T * B).astype(np.int32)      # a tiny vocabulary: from below 1000
    for b in range(B):
        if 0 <= cls_id < enc.n_vocab:
            tok[b * T] = cls_id
        if 0 <= sep_id < enc.n_vocab:
            tok[(b + 1) * T - 1] = sep_id
    lens = [T] * B
    ms = []
    try:
        for r in range(args.reps + 3):
            t0 = time.perf_counter()
            enc.encode(tok, lens, hidden=False, pooled=True, normalize=True)
            t1 = time.perf_counter()
            if r >= 3:
                ms.append((t1 - t0) * 1e3)
            if r == 2 and args.profile:          # the reference CLI profiles the timed passes (tools/cli.cpp:196)
                enc.profile(True)
        prof = enc.profile_read() if args.profile else None
    finally:
        enc.close()
    ms.sort()
    med = ms[len(ms) // 2]
    lines = [f"bench: {ftype}  T={T}  batch={B}  encoder  median {med:.3f} ms  min {ms[0]:.3f} ms  "
             f"({1000.0 * T * B / med:.0f} tokens/s)"]
    if prof:
        lines += profile_lines(prof)
    return "\n".join(lines)


def profile_lines(prof: dict) -> List[str]:
    """nextera_debug_profile_print's report (src/nexterabert.cpp:1828-1841) from an encoder
    profile: ms per pass and share of the wall time of the three kinds, the rest, the total."""
    n, total = max(prof["passes"], 1), max(prof["wall_ms"], 1e-9)
    out = [f"profile over {prof['passes']} forward passes (ms per pass, GPU time from HIP events):"]
    done = 0.0
    for k in ("int8 linear", "attention", "norm / conv / gate / quantize"):
        t = prof["kinds"][k]
        done += t
        out.append(f"  {k:22s} {t / n:8.3f}  {100 * t / total:5.1f}%")
    out.append(f"  {'everything else':22s} {(total - done) / n:8.3f}  {100 * (total - done) / total:5.1f}%"
               "   (embedding rows, out_norm, copies, launch gaps, host)")
    out.append(f"  {'total':22s} {total / n:8.3f}")
    return out


def main(argv: Optional[List[str]] = None) -> int:
    args = parse_args(argv)
    nxg = _package()
    gguf = nxg.GGUF(args.model) if args.model else None
    try:
        if args.info or not args.bench:
            print("\n".join(info(nxg, gguf)), flush=True)
        if args.bench:
            print(bench_encoder(nxg, args) if args.encode else bench(nxg, args, gguf), flush=True)
    finally:
        if gguf is not None:
            gguf.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
