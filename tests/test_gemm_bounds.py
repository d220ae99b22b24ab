"""Host replay of the int8 GEMM kernels' global and LDS addresses (CPU).

tests/gemm_replay.cpp walks every workgroup, wave and lane of the kernel that the
launcher's plan picks for a shape (plan_gemm in nexterabert.cpp_amd/csrc/nxg_gemm_plan.h,
the header the kernels include for their tile walk and address arithmetic), and checks
each load and store against the bytes its buffer holds as the C ABI sizes it, each LDS
access against the kernel's LDS arrays, and that every output word (padding of the int8
outputs included) is written exactly once. The planted-mistake tests compile the replay
against a copy of that header with one clamp removed and expect the replay to fail: a
schedule or address change that leaves a buffer shows up here, before a GPU runs it.
"""
import ctypes
import re
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
CSRC = ROOT / "nexterabert.cpp_amd" / "csrc"
SRC = ROOT / "tests" / "gemm_replay.cpp"

FP32, RESIDUAL, SUMS, RELU2, RELU2_F32 = 0, 1, 2, 3, 4
KINDS = {0: "gemm_kernel", 1: "gemm_kernel sums", 2: "gemm_k256", 3: "gemm_small", 4: "gemm_relu2_q8",
         5: "gemm_relu2_small", 6: "gemm_relu2_rt", 7: "gemm_fsk"}


def _build(out_dir: Path, header_text: str = None) -> ctypes.CDLL:
    inc = CSRC
    if header_text is not None:
        inc = out_dir / "inc"
        inc.mkdir(parents=True, exist_ok=True)
        (inc / "nxg_gemm_plan.h").write_text(header_text)
    lib = out_dir / "libgemm_replay.so"
    subprocess.run(["g++", "-O2", "-std=c++17", "-Wall", "-shared", "-fPIC", f"-I{inc}", f"-I{ROOT / 'include'}",
                    str(SRC), "-o", str(lib)], check=True)
    dll = ctypes.CDLL(str(lib))
    f = dll.gemm_replay
    f.argtypes = [ctypes.c_int] * 5 + [ctypes.POINTER(ctypes.c_int), ctypes.c_int, ctypes.POINTER(ctypes.c_int),
                                       ctypes.POINTER(ctypes.c_longlong), ctypes.c_char_p, ctypes.c_int]
    f.restype = ctypes.c_int
    return dll


def _run(dll, T, n_in, n_out, mode=FP32, segs=(), cus=256):
    kind, acc = ctypes.c_int(-1), ctypes.c_longlong(0)
    err = ctypes.create_string_buffer(1024)
    cols = (ctypes.c_int * 4)(*(list(segs) + [0] * (4 - len(segs))))
    rc = dll.gemm_replay(T, n_in, n_out, mode, len(segs), cols, cus, ctypes.byref(kind), ctypes.byref(acc), err, 1024)
    return rc, KINDS.get(kind.value), acc.value, err.value.decode()


@pytest.fixture(scope="module")
def replay(tmp_path_factory):
    if shutil.which("g++") is None:
        pytest.skip("g++ not available")
    return _build(tmp_path_factory.mktemp("replay"))


SEEN = set()


def _ok(dll, *args, **kw):
    rc, kind, acc, err = _run(dll, *args, **kw)
    assert rc == 0, f"{args} {kw}: {kind}: {err}"
    assert acc > 0
    SEEN.add(kind)
    return kind


@pytest.mark.parametrize("T", [1, 15, 17, 129, 32935])
@pytest.mark.parametrize("n_in", [64, 256, 320, 2304])
def test_fp32_rows_in_bounds(replay, T, n_in):
    for n_out in (4, 60, 260, 2304):
        for mode in (FP32, RESIDUAL):
            _ok(replay, T, n_in, n_out, mode)
    # columns not a multiple of 4: gemm_kernel's per-element stores
    for n_out in (1, 6, 30):
        _ok(replay, T, n_in, n_out, RESIDUAL)


@pytest.mark.parametrize("T", [1, 15, 17, 129, 4100])
def test_block_sums_in_bounds(replay, T):
    for n_in in (64, 256, 320, 2304):
        for n_out in (4, 6, 60, 260):
            assert _ok(replay, T, n_in, n_out, SUMS) == "gemm_kernel sums"


@pytest.mark.parametrize("T", [1, 15, 17, 129, 1000, 8191, 32935])
def test_relu2_int8_in_bounds(replay, T):
    for n_in in (256, 512, 1024, 2304):
        for n_out in (32, 96, 288, 2304):
            _ok(replay, T, n_in, n_out, RELU2)


@pytest.mark.parametrize("T", [1, 17, 1000, 8191, 8250, 32935])
def test_relu2_fp32_rows_in_bounds(replay, T):
    """nxg_linear_f32_relu2_q8_rows: the row-tile kernel reading and quantizing fp32 rows (n_in
    256 and 1024) at every shape that plans it, also those where the library quantizes into the
    workspace first for want of row tiles per workgroup; the other kernels after that quantization."""
    for n_in in (256, 512, 1024):
        for n_out in (32, 288, 2304):
            _ok(replay, T, n_in, n_out, RELU2_F32)


def test_relu2_fp32_rows_sweep_shapes_in_bounds(replay):
    """The seeded shapes of the GPU sweep of nxg_linear_f32_relu2_q8 (tests/test_gpu_relu2.py),
    replayed before any GPU runs them: ragged row tiles, a last column tile past n_out."""
    import numpy as np
    rng = np.random.default_rng(20261202)
    for i in range(8):
        n_in = (256, 1024)[i % 2]
        n_out = 32 * int(rng.integers(8, 129))
        T = int(rng.integers(12000, 70000))
        assert _ok(replay, T, n_in, n_out, RELU2_F32) == "gemm_relu2_rt"


def test_relu2_kernel_choice(replay):
    """n_in 256 and 1024 on the row-tile kernel, other block counts on the 128 x 256 one."""
    assert _ok(replay, 65536, 1024, 2304, RELU2) == "gemm_relu2_rt"
    assert _ok(replay, 9000, 256, 1216, RELU2) == "gemm_relu2_rt"
    assert _ok(replay, 9000, 512, 1216, RELU2) == "gemm_relu2_q8"
    assert _ok(replay, 9000, 2304, 1024, RELU2) == "gemm_relu2_q8"


@pytest.mark.parametrize("T", [1, 17, 129, 5000, 32935])
def test_split_outputs_in_bounds(replay, T):
    # segment boundaries at multiples of 64, each segment a multiple of 4 columns
    for n_in, segs in ((1024, (1024, 512, 512)), (256, (64, 60)), (2304, (128, 64, 64, 4)), (1024, (2048, 128))):
        _ok(replay, T, n_in, sum(segs), FP32, segs=segs)


def test_encoder_shapes_at_full_size(replay):
    """The 65,536-token batch's GEMMs (the benchmark workload) and a 16,384-row HRA pass."""
    for T, n_in, n_out, mode in ((65536, 1024, 2304, RELU2), (65536, 2304, 1024, RESIDUAL),
                                 (65536, 1024, 1024, RESIDUAL), (65536, 1024, 3072, FP32),
                                 (16384, 1024, 2048, FP32), (65536, 1024, 64, FP32)):
        _ok(replay, T, n_in, n_out, mode)
    _ok(replay, 65536, 1024, 2048, FP32, segs=(1024, 512, 512))
    _ok(replay, 65536, 1024, 2176, FP32, segs=(1024, 1024, 128))


@pytest.mark.parametrize("cus", [1, 7, 80, 255])
def test_other_grids(replay, cus):
    """Persistent grids of other sizes: walks of many tiles per workgroup, uneven XCDs."""
    for T, n_in, n_out, mode in ((4100, 1024, 2304, RELU2), (4100, 2304, 1024, RESIDUAL), (3000, 320, 260, FP32),
                                 (3000, 1024, 1000, SUMS), (300, 1024, 2048, FP32), (70, 2304, 2304, RELU2),
                                 (4100, 512, 2304, RELU2), (777, 256, 320, RELU2)):
        _ok(replay, T, n_in, n_out, mode, cus=cus)


def test_every_kernel_replayed(replay):
    for T, n_in, n_out, mode in ((5, 256, 64, FP32), (5, 256, 64, RELU2), (4100, 1024, 2304, RELU2),
                                 (4100, 512, 2304, RELU2), (4100, 1024, 1024, FP32), (300, 320, 6, FP32),
                                 (300, 320, 6, SUMS)):
        _ok(replay, T, n_in, n_out, mode)
    assert set(KINDS.values()) <= SEEN


def test_plan_refuses_nothing_valid(replay):
    rc, _, _, err = _run(replay, 0, 256, 64)
    assert rc == 3 and "no plan" in err


# --- planted mistakes: each removes one clamp from a copy of the shared header ----------

PLANTS = [
    # activation fragment rows past the last one
    ("a_frag", r"return imin\(mt \* \(BM / 16\) \+ i, MF - 1\);", "return mt * (BM / 16) + i;",
     (4100, 1024, 1024, FP32), "a bytes"),
    # few-row pieces' fragment rows
    ("small_a_frag", r"return imin\(mt \* SDT \+ j, MF - 1\);", "return mt * SDT + j;", (33, 320, 260, FP32), "past its"),
    # the split-block few-row tiles' fragment rows and sx groups
    ("fsk_a_frag", r"return imin\(mt \* 4 \+ i, MF - 1\);", "return mt * 4 + i;", (33, 1024, 260, RESIDUAL), "a bytes"),
    ("fsk_sx_group", r"imin\(mt \* 16 \+ g, MF \* 4 - 1\)", "(mt * 16 + g)", (33, 2304, 260, FP32), "sx bytes"),
    # the sx groups of a partial row tile
    ("sx_group_index", r"imin\(mt \* \(BM / 4\) \+ g, MF \* 4 - 1\)", "(mt * (BM / 4) + g)", (4100, 1024, 1024, FP32),
     "sx bytes"),
    # residual columns past N in the last column tile
    ("clamp_col4", r"return imin\(n, N - 4\);", "return n;", (4100, 1024, 1000, RESIDUAL), "res bytes"),
    # residual rows past T in the last row tile
    ("clamp_row", r"return imin\(t, T - 1\);", "return t;", (4100, 1024, 1024, RESIDUAL), "res bytes"),
    # the row-tile relu^2 kernel: fragment rows and sx groups past the last ones, spans that overlap
    ("a_frag_rt", r"return imin\(mt \* \(RM / 16\) \+ i, MF - 1\);", "return mt * (RM / 16) + i;",
     (4100, 1024, 2304, RELU2), "a bytes"),
    ("sx_group_index_rt", r"imin\(mt \* \(RM / 4\) \+ g, MF \* 4 - 1\)", "(mt * (RM / 4) + g)",
     (4100, 1024, 2304, RELU2), "sx bytes"),
    ("tile_span", r"count = \(int\) \(b - a\);", "count = (int) (b - a) + 1;", (4100, 1024, 2304, RELU2), "spans tiles"),
    # its fp32 input rows past T in a partial last row tile
    ("rt_x_row", r"return imin\(mt \* RM \+ r, T - 1\);", "return mt * RM + r;", (8250, 1024, 2304, RELU2_F32), "xf bytes"),
    # a split boundary off by one segment: columns land in the wrong buffer
    ("out_col_of", r"if \(n_seg > 1 && n >= seg_end\[0\]\)", "if (n_seg > 1 && n > seg_end[0])",
     (4100, 1024, 2048, FP32, (1024, 512, 512)), "seg"),
]


@pytest.mark.parametrize("name,pattern,repl,case,expect", PLANTS, ids=[p[0] for p in PLANTS])
def test_planted_mistake_is_caught(tmp_path, name, pattern, repl, case, expect):
    if shutil.which("g++") is None:
        pytest.skip("g++ not available")
    text = (CSRC / "nxg_gemm_plan.h").read_text()
    planted, n = re.subn(pattern, repl, text)
    assert n == 1, f"{name}: the pattern no longer matches the header"
    dll = _build(tmp_path, planted)
    T, n_in, n_out, mode, *rest = case
    rc, kind, _, err = _run(dll, T, n_in, n_out, mode, segs=rest[0] if rest else ())
    assert rc in (1, 2), f"{name}: the replay passed with the mistake planted ({kind})"
    assert expect in err, err
