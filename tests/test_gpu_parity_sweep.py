"""GPU parity over a seeded sweep of shapes (bit for bit against the CPU oracle).

Rows, inputs and outputs are drawn so that every kernel the launcher can pick is reached:
the few-row pieces (gemm_small, gemm_relu2_small), the 128 x 128 tiles with and without a
per-tile schedule (gemm_k256, gemm_kernel), the 128 x 256 relu^2 tiles (gemm_relu2_q8) and
the 64 x 256 relu^2 tiles over an LDS-resident row tile (gemm_relu2_rt), with ragged rows,
partial column tiles, residuals and both activation ranges; two relu^2 shapes of 17,000 to
30,000 rows give workgroups spans that cross row tiles. Each case prints
its index, shape and kernel before it touches the GPU.
"""
from __future__ import annotations

import ctypes
import shutil
import subprocess
from pathlib import Path

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parents[1]
KINDS = {0: "gemm_kernel", 2: "gemm_k256", 3: "gemm_small", 4: "gemm_relu2_q8", 5: "gemm_relu2_small",
         6: "gemm_relu2_rt", 7: "gemm_fsk"}


def say(msg):
    print(msg, flush=True)


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def _cases(n=24, seed=2024):
    """(T, n_in, n_out, relu2, residual, act_max): T log-uniform in [1, 700] (few-row kernels) or
    uniform in [2500, 9000] (tiled kernels), alternately; relu^2 cases need n_in % 256 == 0 and
    n_out % 32 == 0, fp32 cases n_in % 32 == 0 and (for a residual) any n_out."""
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        relu2 = i % 3 == 2
        T = int(np.exp(rng.uniform(0.0, np.log(700.0)))) if i % 2 == 0 else int(rng.integers(2500, 9001))
        if relu2:
            n_in = int(rng.choice([256, 512, 768, 1024, 1280, 2304]))
            n_out = 32 * int(rng.integers(1, 81))
        else:
            n_in = int(rng.choice([32, 64, 96, 256, 320, 512, 1024, 1280, 2304]))
            n_out = int(rng.choice([4 * int(rng.integers(1, 640)), int(rng.integers(1, 300))]))
        out.append((i, max(T, 1), n_in, n_out, relu2, bool(rng.integers(0, 2)), int(rng.choice([127, 63]))))
    # relu^2 at 17,000..30,000 rows: spans of several row tiles per workgroup
    for i in (n, n + 1):
        T = int(rng.integers(17000, 30001))
        n_in = int(rng.choice([256, 1024]))
        n_out = 32 * int(rng.integers(48, 81))
        out.append((i, T, n_in, n_out, True, False, int(rng.choice([127, 63]))))
    return out


@pytest.fixture(scope="module")
def torch():
    import torch as t
    assert t.cuda.is_available(), "no GPU"
    return t


@pytest.fixture(scope="module")
def dev(torch, nxg):
    nxg.init()
    return torch.device("cuda:0")


@pytest.fixture(scope="module")
def plan(tmp_path_factory):
    """The launcher's kernel choice for a shape (the host replay library's plan), for the case
    names and the coverage check."""
    if shutil.which("g++") is None:
        return None
    lib = tmp_path_factory.mktemp("plan") / "libgemm_replay.so"
    subprocess.run(["g++", "-O2", "-std=c++17", "-shared", "-fPIC", f"-I{ROOT / 'nexterabert.cpp_amd' / 'csrc'}",
                    f"-I{ROOT / 'include'}", str(ROOT / "tests" / "gemm_replay.cpp"), "-o", str(lib)], check=True)
    dll = ctypes.CDLL(str(lib))

    def kind(T, n_in, n_out, mode):
        k, acc = ctypes.c_int(-1), ctypes.c_longlong(0)
        err = ctypes.create_string_buffer(256)
        cols = (ctypes.c_int * 4)()
        dll.gemm_replay(T, n_in, n_out, mode, 0, cols, 256, ctypes.byref(k), ctypes.byref(acc), err, 256)
        return KINDS.get(k.value, str(k.value))
    return kind


@pytest.mark.parametrize("case", _cases(), ids=lambda c: f"{c[0]}")
def test_sweep_matches_oracle(nxg, orc, torch, dev, plan, case):
    i, T, n_in, n_out, relu2, residual, act_max = case
    kind = plan(T, n_in, n_out, 3 if relu2 else (1 if residual else 0)) if plan else "?"
    say(f"sweep {i}: T={T} n_in={n_in} n_out={n_out} {'relu2 act_max=%d' % act_max if relu2 else 'fp32'}"
        f"{' + residual' if residual and not relu2 else ''} -> {kind}")
    rng = np.random.default_rng(1000 + i)
    x = (rng.standard_normal((T, n_in)) * np.exp(rng.standard_normal((T, 1)))).astype(np.float32)
    rows = ((0.05 if relu2 else 0.02) * rng.standard_normal((n_out, n_in))).astype(np.float32)
    W = nxg.expand_weight(8, nxg.quantize_weight(8, rows), n_in, n_out)
    dw = nxg.DeviceWeight(W)
    qa = nxg.quantize_rows(torch.from_numpy(x).cuda())
    q_ref, sx_ref = orc.quantize_rows(x)
    simd = bool(orc.vnni_flavour()) and n_in % 32 == 0
    if relu2:
        out = nxg.linear_i8_relu2_q8(dw, qa, act_max)
        u8, sx = nxg.export_qact(out)
        torch.cuda.synchronize()
        y_ref = orc.linear(W.w, W.scale, W.off, q_ref, sx_ref, simd=simd, n_threads=orc.default_threads())
        r_ref, rsx_ref = orc.quantize_rows(orc.relu2(y_ref), act_max)
        assert (u8.cpu().numpy() == r_ref).all()
        assert (bits(sx.cpu().numpy()) == bits(rsx_ref)).all()
    else:
        res = rng.standard_normal((T, n_out)).astype(np.float32) if residual else None
        y = nxg.linear_i8(dw, qa, residual=torch.from_numpy(res).cuda() if residual else None).cpu().numpy()
        y_ref = orc.linear(W.w, W.scale, W.off, q_ref, sx_ref, res=res, simd=simd, n_threads=orc.default_threads())
        assert (bits(y) == bits(y_ref)).all()


def test_sweep_reached_every_kernel(plan):
    """The drawn shapes reach every GEMM kernel the launcher picks from."""
    if plan is None:
        pytest.skip("g++ not available for the plan")
    seen = {plan(T, n_in, n_out, 3 if relu2 else (1 if res else 0)) for _, T, n_in, n_out, relu2, res, _ in _cases()}
    assert set(KINDS.values()) <= seen, sorted(seen)
