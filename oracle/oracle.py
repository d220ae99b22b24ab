"""numpy front end of the CPU oracle (liboracle.so, built from nx_oracle.cpp).

TEST INFRASTRUCTURE ONLY: imported by the tests, the smoke check and the
CPU-baseline leg of bench.py, as the checker. The product never imports it.

Array conventions follow the reference's int8 path (src/nexterabert.cpp):
  activations  x   f32 [T][n_in]
  quantized    q   u8  [T][n_in]  (value + ACT_OFF)
               sx  f32 [(T+3)//4][n_blk][4]  flattened  (src/nexterabert.cpp:372-375)
  weights      w   s8  [n_out][n_in]
               scale f32 [n_blk][n_out], off i32 [n_blk][n_out]  (src/nexterabert.cpp:256-261)
  output       y   f32 [T][n_out]
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

from typing import Optional

import numpy as np

_HERE = Path(__file__).resolve().parent
_LIB_PATH = _HERE / "liboracle.so"
_lib = None

BLOCK = 256


def build(force: bool = False) -> Path:
    """Compile liboracle.so with the Makefile next to this file."""
    if force or not _LIB_PATH.exists():
        subprocess.run(["make", "-s", "-B" if force else "liboracle.so"], cwd=_HERE, check=True)
    return _LIB_PATH


REFERENCE = Path("/root/reference")
REF_CLI = _HERE / "_ref" / "nexterabert-cli"


def build_reference_cli() -> Optional[Path]:
    """The reference's command-line client (tools/cli.cpp), compiled unchanged where it lies
    against include/nexterabert.h and linked to libnexterabert.so (the Makefile's
    _ref/nexterabert-cli). Only where the reference's tree is present; None otherwise."""
    if not (REFERENCE / "tools" / "cli.cpp").is_file():
        return None
    subprocess.run(["make", "-s", "-B", "_ref/nexterabert-cli", f"REF={REFERENCE}"], cwd=_HERE, check=True)
    return REF_CLI


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(_LIB_PATH))
        P = ctypes.c_void_p
        i32 = ctypes.c_int
        L.orc_n_blocks.argtypes, L.orc_n_blocks.restype = [i32], i32
        L.orc_qact_bytes.argtypes, L.orc_qact_bytes.restype = [i32, i32], ctypes.c_size_t
        L.orc_quantize_rows_scalar.argtypes = [P, i32, i32, i32, P, P]
        L.orc_quantize_rows_scalar.restype = None
        L.orc_quantize_rows_simd.argtypes = [P, i32, i32, i32, P, P]
        L.orc_quantize_rows_simd.restype = i32
        L.orc_quantize_rows_simd_mt.argtypes = [P, i32, i32, i32, P, P, i32]
        L.orc_quantize_rows_simd_mt.restype = i32
        L.orc_expand_rows.argtypes = [P, i32, i32, i32, P, P, P]
        L.orc_expand_rows.restype = None
        L.orc_rms_norm_rows.argtypes = [P, P, ctypes.c_float, i32, i32, P]
        L.orc_rms_norm_rows.restype = None
        i64 = ctypes.c_int64
        L.orc_exp_cephes_rows.argtypes, L.orc_exp_cephes_rows.restype = [P, i64, P], None
        L.orc_exp_cephes_simd.argtypes, L.orc_exp_cephes_simd.restype = [P, i64, P], i32
        L.orc_gate_rows.argtypes, L.orc_gate_rows.restype = [P, P, i32, i32, P], None
        L.orc_dwconv_rows.argtypes, L.orc_dwconv_rows.restype = [P, P, P, i32, P, i32, i32, P], None
        L.orc_lily_state_rows.argtypes, L.orc_lily_state_rows.restype = [P, P, P, P, i32, P, i32, i32, P], None
        L.orc_block_mean_rows.argtypes, L.orc_block_mean_rows.restype = [P, P, P, i32, i32, i32, P], None
        L.orc_upsample_add.argtypes, L.orc_upsample_add.restype = [P, P, P, P, i32, i32, i32, P], None
        L.orc_layer_norm.argtypes = [P, P, P, ctypes.c_float, i32, i32, P]
        L.orc_layer_norm.restype = None
        L.orc_doc_mean.argtypes, L.orc_doc_mean.restype = [P, P, i32, i32, i32, P], None
        L.orc_attention_scale.argtypes = [i32, i32, i32, ctypes.c_float, ctypes.c_float, ctypes.c_float]
        L.orc_attention_scale.restype = ctypes.c_float
        L.orc_rope_table.argtypes, L.orc_rope_table.restype = [i32, ctypes.c_float, i32, P, P], None
        L.orc_attention.argtypes = [P, P, P, P, i32, P, i32, i32, i32, i32, P]
        L.orc_attention.restype = None
        L.orc_expf_rows.argtypes, L.orc_expf_rows.restype = [P, i64, P], None
        L.orc_tanh_rows.argtypes, L.orc_tanh_rows.restype = [P, i64, P], None
        L.orc_tanh_simd.argtypes, L.orc_tanh_simd.restype = [P, i64, P], i32
        L.orc_qk_prep.argtypes = [P, P, P, P, P, P, i32, i32, i32, i32, i32, P]
        L.orc_qk_prep.restype = None
        L.orc_expf_restated_check.argtypes = [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint64, P, i32]
        L.orc_expf_restated_check.restype = i64
        L.orc_scores_d64.argtypes, L.orc_scores_d64.restype = [P, P, i32, ctypes.c_float, P], None
        L.orc_softmax_exp.argtypes, L.orc_softmax_exp.restype = [P, i32, i32, P], i32
        L.orc_scores_d64_simd.argtypes, L.orc_scores_d64_simd.restype = [P, P, i32, ctypes.c_float, P], i32
        L.orc_dequant_q8_0.argtypes = [P, ctypes.c_int64, P]
        L.orc_dequant_q8_0.restype = None
        L.orc_block_sums.argtypes = [P, P, i32, i32, P, i32, P]
        L.orc_block_sums.restype = None
        L.orc_linear_scalar.argtypes = [P, P, P, i32, i32, P, P, i32, P, P]
        L.orc_linear_scalar.restype = None
        L.orc_linear_simd.argtypes = [P, P, P, i32, i32, P, P, i32, P, P, i32]
        L.orc_linear_simd.restype = i32
        L.orc_vnni_flavour.argtypes, L.orc_vnni_flavour.restype = [], ctypes.c_char_p
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data


def n_blocks(n_in: int) -> int:
    return (n_in + BLOCK - 1) // BLOCK


def sx_index(t: int, B: int, n_blk: int) -> int:
    return ((t // 4) * n_blk + B) * 4 + t % 4


def sx_len(T: int, n_in: int) -> int:
    return ((T + 3) // 4) * n_blocks(n_in) * 4


def sx_matrix(sx: np.ndarray, T: int, n_in: int) -> np.ndarray:
    """The flat [(T+3)//4][n_blk][4] scale layout as a [T][n_blk] matrix."""
    nb = n_blocks(n_in)
    g = sx.reshape((T + 3) // 4, nb, 4).transpose(0, 2, 1).reshape(-1, nb)
    return g[:T]


def quantize_rows(x: np.ndarray, act_max: int = 127, simd: bool = False, n_threads: int = 1):
    """quantize_row over every row of x (src/nexterabert.cpp:378-403). Returns (q u8, sx flat)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    T, n_in = x.shape
    assert n_in % 8 == 0
    q = np.empty((T, n_in), np.uint8)
    sx = np.zeros(sx_len(T, n_in), np.float32)
    if simd:
        if n_threads > 1:
            rc = lib().orc_quantize_rows_simd_mt(_p(x), T, n_in, act_max, _p(q), _p(sx), n_threads)
        else:
            rc = lib().orc_quantize_rows_simd(_p(x), T, n_in, act_max, _p(q), _p(sx))
        if rc != 0:
            raise RuntimeError("AVX2 not available on this CPU")
    else:
        lib().orc_quantize_rows_scalar(_p(x), T, n_in, act_max, _p(q), _p(sx))
    return q, sx


def relu2(x: np.ndarray) -> np.ndarray:
    """op_relu_sqr (src/nexterabert.cpp:484-505): r = x > 0 ? x : 0 (MAXPS with zero as
    the second operand, so a NaN gives 0), then r * r rounded to f32."""
    x = np.asarray(x, dtype=np.float32)
    with np.errstate(invalid="ignore", over="ignore"):
        r = np.where(x > np.float32(0), x, np.float32(0)).astype(np.float32)
        return (r * r).astype(np.float32)


def rms_norm(x: np.ndarray, gain: np.ndarray, eps: float) -> np.ndarray:
    """op_rms_norm (src/nexterabert.cpp:463-482) as the AVX2 build computes it:
    inv = 1 / sqrt(dot_f32(x, x) / C + eps) with dot_f32's accumulation order
    (src/nexterabert.cpp:124-149), out = (x * inv) * gain. C % 8 == 0."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    g = np.ascontiguousarray(gain, dtype=np.float32)
    T, C = x.shape
    assert C % 8 == 0 and g.shape == (C,)
    out = np.empty_like(x)
    lib().orc_rms_norm_rows(_p(x), _p(g), float(np.float32(eps)), T, C, _p(out))
    return out


def exp_cephes(x: np.ndarray, simd: bool = False) -> np.ndarray:
    """exp256 (src/nexterabert.cpp:81-100) element by element; simd: on AVX2 + FMA
    themselves (size % 8 == 0)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(x)
    if simd:
        if lib().orc_exp_cephes_simd(_p(x), x.size, _p(out)) != 0:
            raise RuntimeError("AVX2/FMA not available or size % 8 != 0")
    else:
        lib().orc_exp_cephes_rows(_p(x), x.size, _p(out))
    return out


def _f32_rows(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def gate(g: np.ndarray, y: np.ndarray) -> np.ndarray:
    """op_gate (src/nexterabert.cpp:507-522): sigmoid256(g) * y."""
    g, y = _f32_rows(g), _f32_rows(y)
    assert g.shape == y.shape and g.ndim == 2
    out = np.empty_like(g)
    lib().orc_gate_rows(_p(g), _p(y), g.shape[0], g.shape[1], _p(out))
    return out


def _cu(cu_offsets):
    return np.ascontiguousarray(cu_offsets, dtype=np.int32)


def dwconv(x: np.ndarray, taps: np.ndarray, cu_offsets, r: np.ndarray = None) -> np.ndarray:
    """op_dwconv (src/nexterabert.cpp:524-543) over a packed batch; taps [k][C]."""
    x, taps, cu = _f32_rows(x), _f32_rows(taps), _cu(cu_offsets)
    T, C = x.shape
    assert taps.shape[1] == C and cu[-1] == T
    if r is not None:
        r = _f32_rows(r)
        assert r.shape == x.shape
    out = np.empty_like(x)
    lib().orc_dwconv_rows(_p(x), _p(r), _p(taps), taps.shape[0], _p(cu), cu.size - 1, C, _p(out))
    return out


def lily_state(a: np.ndarray, x: np.ndarray, b: np.ndarray, taps: np.ndarray, cu_offsets) -> np.ndarray:
    """op_lily_state (src/nexterabert.cpp:545-578) over a packed batch; taps [k][C]."""
    a, x, b, taps, cu = _f32_rows(a), _f32_rows(x), _f32_rows(b), _f32_rows(taps), _cu(cu_offsets)
    T, C = x.shape
    assert a.shape == x.shape == b.shape and taps.shape[1] == C and cu[-1] == T
    out = np.empty_like(x)
    lib().orc_lily_state_rows(_p(a), _p(x), _p(b), _p(taps), taps.shape[0], _p(cu), cu.size - 1, C, _p(out))
    return out


def block_mean(h: np.ndarray, cu_offsets, block: int, g: np.ndarray = None) -> np.ndarray:
    """op_block_mean (src/nexterabert.cpp:638-659): ceil(len / block) rows per document."""
    h, cu = _f32_rows(h), _cu(cu_offsets)
    T, C = h.shape
    assert cu[-1] == T
    if g is not None:
        g = _f32_rows(g)
        assert g.shape == h.shape
    n_rows = int(sum((int(n) + block - 1) // block for n in np.diff(cu)))
    out = np.empty((n_rows, C), np.float32)
    lib().orc_block_mean_rows(_p(h), _p(g), _p(cu), cu.size - 1, block, C, _p(out))
    return out


def upsample_add(yb: np.ndarray, r: np.ndarray, cu_offsets, block: int) -> np.ndarray:
    """op_upsample_add (src/nexterabert.cpp:675-690): each token row gets its block row of yb
    (ceil(len / block) rows per document, in order) added to r."""
    yb, r, cu = _f32_rows(yb), _f32_rows(r), _cu(cu_offsets)
    T, C = r.shape
    lens = np.diff(cu)
    cub = np.concatenate([[0], np.cumsum((lens + block - 1) // block)]).astype(np.int32)
    assert cu[-1] == T and yb.shape == (int(cub[-1]), C)
    out = np.empty_like(r)
    lib().orc_upsample_add(_p(yb), _p(r), _p(cu), _p(cub), cu.size - 1, block, C, _p(out))
    return out


def layer_norm(x: np.ndarray, w: np.ndarray = None, b: np.ndarray = None, eps: float = 1e-5) -> np.ndarray:
    """ggml_norm, then * w and + b (src/nexterabert.cpp:1290-1291); sums in double in a fixed
    lane order (ggml's own order is not in the reference's tree)."""
    x = _f32_rows(x)
    T, C = x.shape
    w = None if w is None else np.ascontiguousarray(w, np.float32)
    b = None if b is None else np.ascontiguousarray(b, np.float32)
    out = np.empty_like(x)
    lib().orc_layer_norm(_p(x), _p(w), _p(b), eps, T, C, _p(out))
    return out


def doc_mean(x: np.ndarray, cu_offsets, normalize: bool = False) -> np.ndarray:
    """Per-document mean of the rows (or L2-normalised sum) as nextera_encode pools
    (src/nexterabert.cpp:1913-1925)."""
    x, cu = _f32_rows(x), _cu(cu_offsets)
    T, C = x.shape
    assert cu[-1] == T
    out = np.empty((cu.size - 1, C), np.float32)
    lib().orc_doc_mean(_p(x), _p(cu), cu.size - 1, C, 1 if normalize else 0, _p(out))
    return out


def attention_scale(n: int, head_dim: int, mode: int, s: float = 0.0, b: float = 0.0, ssmax_base: float = 0.1):
    """op_attention's scale for a document of n keys (src/nexterabert.cpp:1172-1201);
    mode 0 none / swa, 1 ssmax, 2 sssmax."""
    return np.float32(lib().orc_attention_scale(n, head_dim, mode, s, b, ssmax_base))


def rope_table(n_pos: int, base: float, head_dim: int):
    """build_rope (src/nexterabert.cpp:1322-1338): (cos, sin) [n_pos][head_dim / 2]."""
    c = np.empty((n_pos, head_dim // 2), np.float32)
    s = np.empty_like(c)
    lib().orc_rope_table(n_pos, base, head_dim, _p(c), _p(s))
    return c, s


def attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, cu_offsets, scale, n_head: int, n_kv_head: int,
              half: int = -1) -> np.ndarray:
    """op_attention with head_dim 64 (src/nexterabert.cpp:704-852): q [T][H*64] row-major,
    k / v [G][T][64] head-major, scale per document; half >= 0 restricts keys to the band."""
    q, k, v, cu = _f32_rows(q), np.ascontiguousarray(k, np.float32), np.ascontiguousarray(v, np.float32), _cu(cu_offsets)
    T = q.shape[0]
    assert q.shape[1] == n_head * 64 and k.shape == v.shape == (n_kv_head, T, 64) and cu[-1] == T
    sc = np.ascontiguousarray(scale, np.float32)
    assert sc.size == cu.size - 1
    out = np.empty_like(q)
    lib().orc_attention(_p(q), _p(k), _p(v), _p(cu), cu.size - 1, _p(sc), T, n_head, n_kv_head, half, _p(out))
    return out


def tanh_ref(x: np.ndarray, simd: bool = False) -> np.ndarray:
    """tanh256 (src/nexterabert.cpp:103-117) element by element; simd: on AVX2 + FMA (size % 8 == 0)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(x)
    if simd:
        if lib().orc_tanh_simd(_p(x), x.size, _p(out)) != 0:
            raise RuntimeError("AVX2/FMA not available or size % 8 != 0")
    else:
        lib().orc_tanh_rows(_p(x), x.size, _p(out))
    return out


def qk_prep(x, alpha, beta, cos_t, sin_t, cu_offsets, n_head: int, head_major: bool = False) -> np.ndarray:
    """op_qk_prep (src/nexterabert.cpp:590-632): DyT then RoPE; x [T][H*D]."""
    x, cu = _f32_rows(x), _cu(cu_offsets)
    T, width = x.shape
    D = width // n_head
    a, b = np.ascontiguousarray(alpha, np.float32), np.ascontiguousarray(beta, np.float32)
    c, s = _f32_rows(cos_t), _f32_rows(sin_t)
    assert a.shape == b.shape == (D,) and c.shape[1] == D // 2 and s.shape == c.shape and cu[-1] == T
    assert int(np.diff(cu).max()) <= c.shape[0]
    out = np.empty((n_head, T, D) if head_major else (T, width), np.float32)
    lib().orc_qk_prep(_p(x), _p(a), _p(b), _p(c), _p(s), _p(cu), cu.size - 1, T, n_head, D, int(head_major), _p(out))
    return out


def expf(x: np.ndarray) -> np.ndarray:
    """The C library's expf (the reference's std::exp on floats), element by element."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(x)
    lib().orc_expf_rows(_p(x), x.size, _p(out))
    return out


def expf_restated_mismatches(first: int, stride: int, count: int):
    """Inputs (as float bit patterns first, first + stride, ...) where the restated C-library
    expf differs from the host's expf: (count, first few patterns)."""
    bad = np.zeros(8, np.uint32)
    n = lib().orc_expf_restated_check(first, stride, count, _p(bad), bad.size)
    return int(n), bad[:min(int(n), bad.size)]


def scores_d64(q: np.ndarray, k: np.ndarray, scale: float, simd: bool = False) -> np.ndarray:
    """scores_d64 (src/nexterabert.cpp:704-731) of one query against n keys [n][64]."""
    q, k = np.ascontiguousarray(q, np.float32), np.ascontiguousarray(k, np.float32)
    n = k.shape[0]
    out = np.empty(n, np.float32)
    if simd:
        if lib().orc_scores_d64_simd(_p(q), _p(k), n, float(scale), _p(out)) != 0:
            raise RuntimeError("AVX2/FMA not available")
    else:
        lib().orc_scores_d64(_p(q), _p(k), n, float(scale), _p(out))
    return out


def softmax_exp(s: np.ndarray, simd: bool = False):
    """softmax_exp (src/nexterabert.cpp:177-197) of a row of scores: (weights exp(s - max),
    their sum in the reference's order). simd: on AVX2 + FMA, else the scalar statement."""
    w = np.array(s, dtype=np.float32, copy=True)
    total = ctypes.c_float()
    if lib().orc_softmax_exp(_p(w), w.size, 1 if simd else 0, ctypes.byref(total)) != 0:
        raise RuntimeError("AVX2/FMA not available")
    return w, np.float32(total.value)


def expand_rows(rows: np.ndarray, act_off: int = 128):
    """build_i8_weight on dequantized f32 rows (src/nexterabert.cpp:1030-1042)."""
    rows = np.ascontiguousarray(rows, dtype=np.float32)
    n_out, n_in = rows.shape
    nb = n_blocks(n_in)
    w = np.empty((n_out, n_in), np.int8)
    scale = np.empty((nb, n_out), np.float32)
    off = np.empty((nb, n_out), np.int32)
    lib().orc_expand_rows(_p(rows), n_in, n_out, act_off, _p(w), _p(scale), _p(off))
    return w, scale, off


def dequant_q8_0(data: np.ndarray, n: int) -> np.ndarray:
    data = np.ascontiguousarray(data, dtype=np.uint8)
    assert data.size == n // 32 * 34
    out = np.empty(n, np.float32)
    lib().orc_dequant_q8_0(_p(data), n, _p(out))
    return out


def block_sums(w, off, q) -> np.ndarray:
    """Per-block int32 sums [n_blk][T][n_out] = sum w8*u8 + off."""
    n_out, n_in = w.shape
    T = q.shape[0]
    s = np.empty((n_blocks(n_in), T, n_out), np.int32)
    lib().orc_block_sums(_p(w), _p(off), n_in, n_out, _p(q), T, _p(s))
    return s


def linear(w, scale, off, q, sx, res=None, simd: bool = False, n_threads: int = 1) -> np.ndarray:
    """op_linear_i8 (src/nexterabert.cpp:969-1007). Returns f32 [T][n_out]."""
    n_out, n_in = w.shape
    T = q.shape[0]
    out = np.empty((T, n_out), np.float32)
    if res is not None:
        res = np.ascontiguousarray(res, dtype=np.float32)
        assert res.shape == (T, n_out)
    args = (_p(w), _p(scale), _p(off), n_in, n_out, _p(q), _p(sx), T, _p(res), _p(out))
    if simd:
        rc = lib().orc_linear_simd(*args, n_threads)
        if rc != 0:
            raise RuntimeError(f"orc_linear_simd failed ({rc}): no VNNI on this CPU or n_in % 32 != 0")
    else:
        lib().orc_linear_scalar(*args)
    return out


def vnni_flavour() -> str:
    return lib().orc_vnni_flavour().decode()


def default_threads() -> int:
    """The reference's default pool size: all cores but ~10% (src/nexterabert.cpp:1519-1524)."""
    try:
        hw = len(os.sched_getaffinity(0))
    except AttributeError:  # pragma: no cover
        hw = os.cpu_count() or 1
    return max(1, hw - hw // 10)
