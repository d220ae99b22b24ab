"""nexterabert.cpp_amd -- the int8 linear-layer path of NexteraBERT.cpp on MI355X (gfx950).

Python side of libnxg.so (include/nxg_linear.h). It mirrors the reference's own
interface for the path, with torch tensors as device memory and torch's current
stream as the HIP stream:

  expand_weight(type, data, n_in, n_out)   build_i8_weight        src/nexterabert.cpp:1010-1049
  weight_is_int8(name, ...)                 placement rule         src/nexterabert.cpp:1658-1667
  quantize_rows(x)                          quantize_row / op_copy src/nexterabert.cpp:378-403,453-461
  linear_i8(weight, qact, residual)         op_linear_i8           src/nexterabert.cpp:969-1007
  Builder.linear(name, x, residual)         builder::linear        src/nexterabert.cpp:1121-1143

Errors follow the reference: bad input raises ValueError (rc 1), allocation
MemoryError (rc 2), device failures RuntimeError (rc 3). There is no CPU
fallback: without the built library or a gfx950 GPU every device call raises.
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass
from pathlib import Path
from typing import Dict, List, Optional, Sequence

import numpy as np

_PKG = Path(__file__).resolve().parent
LIB_PATH = _PKG / "libnxg.so"
BLOCK = 256

# ggml block types (GGUF numbering), include/nxg_linear.h
TYPE_F32, TYPE_F16, TYPE_Q4_0, TYPE_Q4_1 = 0, 1, 2, 3
TYPE_Q5_0, TYPE_Q5_1, TYPE_Q8_0 = 6, 7, 8
TYPE_Q2_K, TYPE_Q3_K, TYPE_Q4_K, TYPE_Q5_K, TYPE_Q6_K = 10, 11, 12, 13, 14
TYPE_BF16 = 30

# GGUF metadata value types, include/nxg_gguf.h
(GGUF_UINT8, GGUF_INT8, GGUF_UINT16, GGUF_INT16, GGUF_UINT32, GGUF_INT32, GGUF_FLOAT32, GGUF_BOOL,
 GGUF_STRING, GGUF_ARRAY, GGUF_UINT64, GGUF_INT64, GGUF_FLOAT64) = range(13)

NXG_OK, NXG_EINVAL, NXG_ENOMEM, NXG_EDEVICE = 0, 1, 2, 3

_lib: Optional[ctypes.CDLL] = None


class NxgError(RuntimeError):
    pass


class EncoderParams(ctypes.Structure):
    """struct nxg_encoder_params (include/nxg_encoder.h)."""
    _fields_ = [("act_max", ctypes.c_int32), ("load_threads", ctypes.c_int32), ("verbosity", ctypes.c_int32)]


def load_library(path: Optional[os.PathLike] = None) -> ctypes.CDLL:
    """Loads libnxg.so (built by build.py); raises if it is missing."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = Path(path) if path else LIB_PATH
    if not p.exists():
        raise FileNotFoundError(f"{p} is not built: run python nexterabert.cpp_amd/build.py "
                                "(or __graft_entry__.build())")
    L = ctypes.CDLL(str(p))
    P, i32, i64, sz = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_size_t
    sigs = {
        "nxg_last_error": ([], ctypes.c_char_p),
        "nxg_weight_is_int8": ([ctypes.c_char_p, i32, i32, i64, i64, i32], i32),
        "nxg_row_bytes": ([i32, i64], sz),
        "nxg_dequantize_rows": ([i32, P, i64, i64, P], i32),
        "nxg_expand_weight": ([i32, P, i32, i32, i32, i32, P, P, P], i32),
        "nxg_quantize_weight": ([i32, P, i64, i64, P], i32),
        "nxg_init": ([], i32),
        "nxg_qact_q_bytes": ([i32, i32], sz),
        "nxg_qact_sx_bytes": ([i32, i32], sz),
        "nxg_quantize_rows": ([P, i32, i32, i32, P, P, P], i32),
        "nxg_quantize_rows_relu2": ([P, i32, i32, i32, P, P, P], i32),
        "nxg_rmsnorm_quantize_rows": ([P, P, ctypes.c_float, i32, i32, i32, P, P, P], i32),
        "nxg_gate_quantize_rows": ([P, P, i32, i32, i32, P, P, P], i32),
        "nxg_dwconv_quantize_rows": ([P, P, P, i32, P, i32, i32, i32, i32, P, P, P], i32),
        "nxg_lily_state_quantize_rows": ([P, P, P, P, i32, P, i32, i32, i32, i32, P, P, P], i32),
        "nxg_block_mean_quantize_rows": ([P, P, P, P, i32, i32, i32, i32, i32, i32, P, P, P], i32),
        "nxg_attention": ([P, P, P, P, i32, P, i32, i32, i32, i32, i32, P, P], i32),
        "nxg_attention_ws": ([P, P, P, P, i32, P, i32, i32, i32, i32, i32, P, P, i64, P], i32),
        "nxg_attention_workspace_bytes": ([i32, i32, i32, i32], i64),
        "nxg_attention_scales": ([P, i32, i32, i32, ctypes.c_float, ctypes.c_float, ctypes.c_float, P], i32),
        "nxg_qk_prep": ([P, P, P, P, P, i32, P, i32, i32, i32, i32, i32, P, P], i32),
        "nxg_head_major": ([P, i32, i32, i32, P, P], i32),
        "nxg_qkv_prep": ([P, P, P, P, P, P, P, P, P, i32, P, i32, i32, i32, i32, i32, P, P, P, P], i32),
        "nxg_dwconv_rows": ([P, P, P, i32, P, i32, i32, i32, P, P], i32),
        "nxg_upsample_add": ([P, P, P, P, i32, i32, i32, i32, i32, P, P], i32),
        "nxg_embed_rows": ([P, i32, P, P, i32, P, i32, i32, P, P], i32),
        "nxg_layer_norm": ([P, P, P, ctypes.c_float, i32, i32, P, P], i32),
        "nxg_doc_mean": ([P, P, i32, i32, i32, i32, P, P], i32),
        "nxg_encoder_load": ([ctypes.c_char_p, ctypes.POINTER(EncoderParams), ctypes.POINTER(P)], i32),
        "nxg_encoder_free": ([P], None),
        "nxg_encoder_n_embd": ([P], i32),
        "nxg_encoder_n_vocab": ([P], i32),
        "nxg_encoder_n_layer": ([P], i32),
        "nxg_encoder_n_token_types": ([P], i32),
        "nxg_encoder_device_bytes": ([P], sz),
        "nxg_encoder_set_layers": ([P, i32], None),
        "nxg_encoder_encode": ([P, P, P, P, i32, P, P, i32], i32),
        "nxg_encoder_forward": ([P, P, P, P, i32, P, P, i32, P], i32),
        "nxg_encoder_last_ms": ([P], ctypes.c_double),
        "nxg_encoder_n_int8": ([P], i32),
        "nxg_encoder_profile": ([P, i32], None),
        "nxg_encoder_profile_read": ([P, P, P, P, P], i32),
        "nxg_encoder_set_work_limit": ([P, i64], i32),
        "nxg_encoder_attention_workspace": ([P], i64),
        "nxg_rope_table": ([i32, ctypes.c_float, i32, P, P], i32),
        "nxg_qact_export": ([P, P, i32, i32, i32, P, P, P], i32),
        "nxg_weight_create": ([P, P, i32, i32, ctypes.POINTER(P)], i32),
        "nxg_weight_destroy": ([P], None),
        "nxg_weight_n_in": ([P], i32),
        "nxg_weight_n_out": ([P], i32),
        "nxg_weight_device_bytes": ([P], sz),
        "nxg_linear_i8": ([P, P, P, P, i32, P, P, P], i32),
        "nxg_linear_i8_rows": ([P, P, P, i32, P, P, P], i32),
        "nxg_linear_i8_rows_split": ([P, P, P, i32, i32, P, P, P], i32),
        "nxg_linear_i8_block_sums": ([P, P, i32, P, P], i32),
        "nxg_linear_i8_relu2_q8": ([P, P, P, P, i32, i32, P, P, P], i32),
        "nxg_linear_i8_relu2_q8_rows": ([P, P, P, i32, i32, P, P, P], i32),
        "nxg_linear_f32_relu2_q8_rows": ([P, P, i32, i32, P, P, P, P, P], i32),
        "nxg_linear_f32_relu2_q8": ([P, P, P, i32, i32, P, P, P, P, P], i32),
        "nxg_gemm_kernel_name": ([i32, i32, i32, i32, i32], ctypes.c_char_p),
        # include/nxg_gguf.h
        "nxg_gguf_open": ([ctypes.c_char_p, ctypes.POINTER(P)], i32),
        "nxg_gguf_close": ([P], None),
        "nxg_gguf_version": ([P], ctypes.c_uint32),
        "nxg_gguf_data_offset": ([P], ctypes.c_uint64),
        "nxg_gguf_alignment": ([P], ctypes.c_uint32),
        "nxg_gguf_n_kv": ([P], i64),
        "nxg_gguf_find_key": ([P, ctypes.c_char_p], i64),
        "nxg_gguf_key": ([P, i64], ctypes.c_char_p),
        "nxg_gguf_kv_type": ([P, i64], i32),
        "nxg_gguf_get_i64": ([P, i64, ctypes.POINTER(i64)], i32),
        "nxg_gguf_get_f64": ([P, i64, ctypes.POINTER(ctypes.c_double)], i32),
        "nxg_gguf_get_str": ([P, i64, ctypes.POINTER(ctypes.c_void_p), ctypes.POINTER(ctypes.c_uint64)], i32),
        "nxg_gguf_arr_info": ([P, i64, ctypes.POINTER(i32), ctypes.POINTER(ctypes.c_uint64)], i32),
        "nxg_gguf_arr_i64": ([P, i64, ctypes.c_uint64, ctypes.POINTER(i64)], i32),
        "nxg_gguf_arr_f64": ([P, i64, ctypes.c_uint64, ctypes.POINTER(ctypes.c_double)], i32),
        "nxg_gguf_arr_str": ([P, i64, ctypes.c_uint64, ctypes.POINTER(ctypes.c_void_p), ctypes.POINTER(ctypes.c_uint64)], i32),
        "nxg_gguf_n_tensors": ([P], i64),
        "nxg_gguf_find_tensor": ([P, ctypes.c_char_p], i64),
        "nxg_gguf_tensor_name": ([P, i64], ctypes.c_char_p),
        "nxg_gguf_tensor_info": ([P, i64, ctypes.POINTER(i32), ctypes.POINTER(i32), ctypes.POINTER(i64),
                                  ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_uint64)], i32),
        "nxg_gguf_tensor_data": ([P, i64], P),
        "nxg_gguf_weight_create": ([P, i64, i32, ctypes.POINTER(P)], i32),
    }
    for name, (args, res) in sigs.items():
        fn = getattr(L, name)
        fn.argtypes, fn.restype = args, res
    if path is None:
        _lib = L
    return L


def _check(rc: int, what: str) -> None:
    if rc == NXG_OK:
        return
    msg = f"{what}: {load_library().nxg_last_error().decode()}"
    if rc == NXG_EINVAL:
        raise ValueError(msg)
    if rc == NXG_ENOMEM:
        raise MemoryError(msg)
    raise NxgError(msg)


def _np_ptr(a: Optional[np.ndarray]):
    return None if a is None else a.ctypes.data


# --- host side: load-time expansion ------------------------------------------------------------

def weight_is_int8(name: str, n_dims: int, type_: int, ne0: int, ne1: int, use_int8: bool = True) -> bool:
    """The reference's rule for putting a weight on the int8 GEMM (src/nexterabert.cpp:1658-1667)."""
    return bool(load_library().nxg_weight_is_int8(name.encode(), n_dims, type_, ne0, ne1, int(use_int8)))


def row_bytes(type_: int, n_in: int) -> int:
    return int(load_library().nxg_row_bytes(type_, n_in))


def dequantize_rows(type_: int, data: np.ndarray, n_in: int, n_rows: int) -> np.ndarray:
    data = np.ascontiguousarray(data)
    out = np.empty((n_rows, n_in), np.float32)
    _check(load_library().nxg_dequantize_rows(type_, _np_ptr(data), n_in, n_rows, _np_ptr(out)), "dequantize_rows")
    return out


def quantize_weight(type_: int, x: np.ndarray) -> np.ndarray:
    """Encodes f32 rows [n_rows][n_in] as GGUF blocks (Q8_0, Q5_0, Q4_K or Q6_K)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    n_rows, n_in = x.shape
    rb = row_bytes(type_, n_in)
    if rb == 0:
        raise ValueError(f"type {type_} cannot hold rows of {n_in}")
    out = np.zeros(rb * n_rows, np.uint8)
    _check(load_library().nxg_quantize_weight(type_, _np_ptr(x), n_in, n_rows, _np_ptr(out)), "quantize_weight")
    return out


@dataclass
class I8Weight:
    """The reference's i8_weight (src/nexterabert.cpp:256-261): s8 [n_out][n_in] with one
    float scale and one int32 offset per (256-input block, output row)."""
    w: np.ndarray        # int8 [n_out][n_in]
    scale: np.ndarray    # f32 [n_blk][n_out]
    off: np.ndarray      # i32 [n_blk][n_out]

    @property
    def n_in(self) -> int:
        return self.w.shape[1]

    @property
    def n_out(self) -> int:
        return self.w.shape[0]

    @property
    def n_blk(self) -> int:
        return (self.n_in + BLOCK - 1) // BLOCK


def expand_weight(type_: int, data: np.ndarray, n_in: int, n_out: int, act_off: int = 128,
                  n_threads: int = 0) -> I8Weight:
    """build_i8_weight: GGUF rows of `type_` -> I8Weight (src/nexterabert.cpp:1010-1049)."""
    data = np.ascontiguousarray(data)
    nb = (n_in + BLOCK - 1) // BLOCK
    w = np.empty((n_out, n_in), np.int8)
    scale = np.empty((nb, n_out), np.float32)
    off = np.empty((nb, n_out), np.int32)
    _check(load_library().nxg_expand_weight(type_, _np_ptr(data), n_in, n_out, act_off, n_threads,
                                            _np_ptr(w), _np_ptr(scale), _np_ptr(off)), "expand_weight")
    return I8Weight(w, scale, off)


# --- device side -------------------------------------------------------------------------------

def _torch():
    import torch
    return torch


def _stream_ptr(stream=None) -> Optional[int]:
    torch = _torch()
    s = stream if stream is not None else torch.cuda.current_stream()
    return s.cuda_stream or None


def _order_on(stream, *tensors) -> None:
    """Before a launch on `stream` that reads or writes tensors allocated here, on torch's
    current stream: the launch waits for the current stream's work (host-to-device copies
    of offsets and scales), and the caching allocator may not hand those tensors' memory to
    anything else before `stream` has finished with them. A no-op when `stream` is the
    current stream (or None)."""
    if stream is None:
        return
    torch = _torch()
    cur = torch.cuda.current_stream()
    if stream.cuda_stream == cur.cuda_stream:
        return
    stream.wait_stream(cur)
    for t in tensors:
        if t is not None:
            t.record_stream(stream)


def init() -> None:
    """Checks that the current device is a gfx950 GPU (raises otherwise)."""
    _check(load_library().nxg_init(), "init")


class DeviceWeight:
    """An I8Weight uploaded once into MFMA fragment tiles (nxg_weight)."""

    def __init__(self, weight: Optional[I8Weight], handle: Optional[ctypes.c_void_p] = None):
        L = load_library()
        if handle is None:
            w = np.ascontiguousarray(weight.w)
            s = np.ascontiguousarray(weight.scale)
            handle = ctypes.c_void_p()
            _check(L.nxg_weight_create(_np_ptr(w), _np_ptr(s), w.shape[1], w.shape[0], ctypes.byref(handle)),
                   "weight_create")
        self._h = handle
        self.n_in, self.n_out = int(L.nxg_weight_n_in(handle)), int(L.nxg_weight_n_out(handle))
        self.n_blk = (self.n_in + BLOCK - 1) // BLOCK
        self.device_bytes = int(L.nxg_weight_device_bytes(handle))

    @property
    def handle(self) -> ctypes.c_void_p:
        return self._h

    def close(self) -> None:
        if getattr(self, "_h", None) and self._h.value:
            load_library().nxg_weight_destroy(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


@dataclass
class QAct:
    """Quantized activations of T rows (the reference's qact buffer, src/nexterabert.cpp:368-375):
    q in MFMA fragment tiles (signed: u8 - ACT_OFF) and sx in the reference's scale layout."""
    q: object            # torch int8, nxg_qact_q_bytes(T, n_in)
    sx: object           # torch float32, nxg_qact_sx_bytes(T, n_in) / 4
    T: int
    n_in: int
    act_max: int = 127


def qact_alloc(T: int, n_in: int, act_max: int = 127, device="cuda") -> QAct:
    torch = _torch()
    L = load_library()
    qb, sb = int(L.nxg_qact_q_bytes(T, n_in)), int(L.nxg_qact_sx_bytes(T, n_in))
    if T > 0 and (qb == 0 or sb == 0):
        raise ValueError(f"n_in={n_in} must be a positive multiple of 32")
    return QAct(torch.empty(max(qb, 1), dtype=torch.int8, device=device),
                torch.empty(max(sb // 4, 1), dtype=torch.float32, device=device), T, n_in, act_max)


def _quantize(fn_name: str, x, act_max: int, out: Optional[QAct], stream) -> QAct:
    torch = _torch()
    if x.dtype != torch.float32 or x.dim() != 2 or not x.is_cuda or not x.is_contiguous():
        raise ValueError("x must be a contiguous 2-D float32 device tensor")
    T, n_in = x.shape
    qa = out if out is not None else qact_alloc(T, n_in, act_max, x.device)
    qa.T, qa.n_in, qa.act_max = T, n_in, act_max
    fn = getattr(load_library(), fn_name)
    _order_on(stream, qa.q, qa.sx)
    _check(fn(x.data_ptr(), T, n_in, act_max, qa.q.data_ptr(), qa.sx.data_ptr(), _stream_ptr(stream)), fn_name)
    return qa


def quantize_rows(x, act_max: int = 127, out: Optional[QAct] = None, stream=None) -> QAct:
    """quantize_row over every row of x (device f32 [T][n_in])."""
    return _quantize("nxg_quantize_rows", x, act_max, out, stream)


def quantize_rows_relu2(x, act_max: int = 127, out: Optional[QAct] = None, stream=None) -> QAct:
    """op_relu_sqr quantized for an int8 consumer: quantize_row of relu(x)^2 per row."""
    return _quantize("nxg_quantize_rows_relu2", x, act_max, out, stream)


def rmsnorm_quantize_rows(x, gain, eps: float, act_max: int = 127, out: Optional[QAct] = None, stream=None) -> QAct:
    """op_rms_norm quantized for an int8 consumer: quantize_row of (x * inv) * gain per row,
    inv = 1 / sqrt(mean(x^2) + eps) with the reference's dot_f32 order."""
    torch = _torch()
    if x.dtype != torch.float32 or x.dim() != 2 or not x.is_cuda or not x.is_contiguous():
        raise ValueError("x must be a contiguous 2-D float32 device tensor")
    T, n_in = x.shape
    if gain.dtype != torch.float32 or tuple(gain.shape) != (n_in,) or not gain.is_cuda or not gain.is_contiguous():
        raise ValueError(f"gain must be a contiguous float32 device tensor of shape ({n_in},)")
    qa = out if out is not None else qact_alloc(T, n_in, act_max, x.device)
    qa.T, qa.n_in, qa.act_max = T, n_in, act_max
    _order_on(stream, qa.q, qa.sx)
    _check(load_library().nxg_rmsnorm_quantize_rows(x.data_ptr(), gain.data_ptr(), float(eps), T, n_in, act_max,
                                                     qa.q.data_ptr(), qa.sx.data_ptr(), _stream_ptr(stream)),
           "rmsnorm_quantize_rows")
    return qa


def _rows_arg(t, name, shape=None):
    torch = _torch()
    if t.dtype != torch.float32 or t.dim() != 2 or not t.is_cuda or not t.is_contiguous():
        raise ValueError(f"{name} must be a contiguous 2-D float32 device tensor")
    if shape is not None and tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name} must have shape {tuple(shape)}, got {tuple(t.shape)}")
    return t


def _device_offsets(cu_offsets, device):
    """cu_offsets (host sequence or device int32 tensor) as a device int32 tensor."""
    torch = _torch()
    if isinstance(cu_offsets, torch.Tensor):
        t = cu_offsets.to(device=device, dtype=torch.int32).contiguous()
    else:
        t = torch.tensor(np.ascontiguousarray(cu_offsets, dtype=np.int32), device=device)
    if t.dim() != 1 or t.numel() < 2:
        raise ValueError("cu_offsets: need n_seqs + 1 >= 2 offsets")
    return t


def _produce_out(T, n_in, act_max, out, device):
    qa = out if out is not None else qact_alloc(T, n_in, act_max, device)
    qa.T, qa.n_in, qa.act_max = T, n_in, act_max
    return qa


def gate_quantize_rows(g, y, act_max: int = 127, out: Optional[QAct] = None, stream=None) -> QAct:
    """op_gate quantized for an int8 consumer: quantize_row of sigmoid(g) * y per row
    (the reference's exp256-based sigmoid)."""
    _rows_arg(g, "g")
    T, n_in = g.shape
    _rows_arg(y, "y", (T, n_in))
    qa = _produce_out(T, n_in, act_max, out, g.device)
    _order_on(stream, qa.q, qa.sx)
    _check(load_library().nxg_gate_quantize_rows(g.data_ptr(), y.data_ptr(), T, n_in, act_max, qa.q.data_ptr(),
                                                 qa.sx.data_ptr(), _stream_ptr(stream)), "gate_quantize_rows")
    return qa


def dwconv_quantize_rows(x, taps, cu_offsets, r=None, act_max: int = 127, out: Optional[QAct] = None,
                         stream=None) -> QAct:
    """op_dwconv quantized for an int8 consumer: r + the depthwise convolution of x with
    taps [k][n_in] inside each document of the packed batch (cu_offsets)."""
    _rows_arg(x, "x")
    T, n_in = x.shape
    _rows_arg(taps, "taps")
    if taps.shape[1] != n_in:
        raise ValueError(f"taps must be [k][{n_in}]")
    if r is not None:
        _rows_arg(r, "r", (T, n_in))
    cu = _device_offsets(cu_offsets, x.device)
    qa = _produce_out(T, n_in, act_max, out, x.device)
    _order_on(stream, cu, qa.q, qa.sx)
    _check(load_library().nxg_dwconv_quantize_rows(x.data_ptr(), r.data_ptr() if r is not None else None,
                                                   taps.data_ptr(), taps.shape[0], cu.data_ptr(), cu.numel() - 1,
                                                   T, n_in, act_max, qa.q.data_ptr(), qa.sx.data_ptr(),
                                                   _stream_ptr(stream)), "dwconv_quantize_rows")
    return qa


def lily_state_quantize_rows(a, x, b, taps, cu_offsets, act_max: int = 127, out: Optional[QAct] = None,
                             stream=None) -> QAct:
    """op_lily_state quantized for an int8 consumer: b * the depthwise convolution of a * x
    with taps [k][n_in] inside each document (cu_offsets)."""
    _rows_arg(x, "x")
    T, n_in = x.shape
    _rows_arg(a, "a", (T, n_in))
    _rows_arg(b, "b", (T, n_in))
    _rows_arg(taps, "taps")
    if taps.shape[1] != n_in:
        raise ValueError(f"taps must be [k][{n_in}]")
    cu = _device_offsets(cu_offsets, x.device)
    qa = _produce_out(T, n_in, act_max, out, x.device)
    _order_on(stream, cu, qa.q, qa.sx)
    _check(load_library().nxg_lily_state_quantize_rows(a.data_ptr(), x.data_ptr(), b.data_ptr(), taps.data_ptr(),
                                                       taps.shape[0], cu.data_ptr(), cu.numel() - 1, T, n_in,
                                                       act_max, qa.q.data_ptr(), qa.sx.data_ptr(),
                                                       _stream_ptr(stream)), "lily_state_quantize_rows")
    return qa


def block_offsets(cu_offsets: Sequence[int], block: int) -> np.ndarray:
    """The block rows' layout of a packed batch: ceil(len_d / block) rows per document."""
    cu = np.asarray(cu_offsets, dtype=np.int64)
    return cu_offsets_of([(int(n) + block - 1) // block for n in np.diff(cu)])


def block_mean_quantize_rows(h, cu_offsets: Sequence[int], block: int, g=None, act_max: int = 127,
                             out: Optional[QAct] = None, stream=None) -> QAct:
    """op_block_mean quantized for an int8 consumer: per document, the mean of each run of
    `block` tokens of h (* g), one row per run. cu_offsets: host offsets of the tokens."""
    _rows_arg(h, "h")
    T, n_in = h.shape
    if g is not None:
        _rows_arg(g, "g", (T, n_in))
    cu_host = np.ascontiguousarray(cu_offsets, dtype=np.int32)
    if cu_host.size < 2 or int(cu_host[-1]) != T:
        raise ValueError(f"cu_offsets must end at T={T}")
    cub_host = block_offsets(cu_host, block)
    n_blocks = int(cub_host[-1])
    cu, cub = _device_offsets(cu_host, h.device), _device_offsets(cub_host, h.device)
    qa = _produce_out(n_blocks, n_in, act_max, out, h.device)
    _order_on(stream, cu, cub, qa.q, qa.sx)
    _check(load_library().nxg_block_mean_quantize_rows(h.data_ptr(), g.data_ptr() if g is not None else None,
                                                       cu.data_ptr(), cub.data_ptr(), cu.numel() - 1, T, n_blocks,
                                                       block, n_in, act_max, qa.q.data_ptr(), qa.sx.data_ptr(),
                                                       _stream_ptr(stream)), "block_mean_quantize_rows")
    return qa


SSMAX_NONE, SSMAX_SSMAX, SSMAX_SSSMAX = 0, 1, 2   # nxg_attention_scales modes


def attention_scales(cu_offsets: Sequence[int], head_dim: int = 64, mode: int = SSMAX_NONE, s: float = 1.0,
                     b: float = 0.0, ssmax_base: float = 0.1) -> np.ndarray:
    """The per-document attention scales of src/nexterabert.cpp:1196-1201 (host, the C
    library's logf): 1/sqrt(head_dim) times 1, s ln n, or s ln n + ssmax_base + max(b, 0)."""
    cu = np.ascontiguousarray(cu_offsets, dtype=np.int32)
    out = np.empty(cu.size - 1, np.float32)
    _check(load_library().nxg_attention_scales(_np_ptr(cu), cu.size - 1, head_dim, mode, float(s), float(b),
                                                 float(ssmax_base), _np_ptr(out)), "attention_scales")
    return out


def attention_workspace_bytes(T: int, n_head: int, n_kv_head: int, max_keys: int) -> int:
    """nxg_attention_workspace_bytes: the workspace attention(..., workspace="auto") allocates
    (0 when the launch keeps its scores in LDS)."""
    n = int(load_library().nxg_attention_workspace_bytes(T, n_head, n_kv_head, max_keys))
    if n < 0:
        _check(n, "attention_workspace_bytes")
    return n


def attention(q, k, v, cu_offsets: Sequence[int], scale, n_head: int, n_kv_head: int, half: int = -1,
              out=None, stream=None, workspace=None):
    """op_attention with head_dim 64 inside each document: q [T][n_head*64], k / v
    [n_kv_head][T][64] head-major, scale per document (host or device floats).
    workspace: None (nxg_attention), a uint8 device tensor, or "auto" (one of
    attention_workspace_bytes) for nxg_attention_ws, which keeps the scores of documents too
    long for LDS in it instead of recomputing them."""
    torch = _torch()
    _rows_arg(q, "q")
    T = q.shape[0]
    if q.shape[1] != n_head * 64:
        raise ValueError(f"q must be [T][{n_head * 64}]")
    for name, t in (("k", k), ("v", v)):
        if t.dtype != torch.float32 or tuple(t.shape) != (n_kv_head, T, 64) or not t.is_cuda or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous float32 device tensor [{n_kv_head}][{T}][64]")
    cu_host = np.ascontiguousarray(cu_offsets, dtype=np.int32)
    if cu_host.size < 2 or int(cu_host[-1]) != T:
        raise ValueError(f"cu_offsets must end at T={T}")
    lens = np.diff(cu_host)
    max_keys = int(lens.max()) if half < 0 else int(min(lens.max(), 2 * half + 1))
    cu = _device_offsets(cu_host, q.device)
    sc = scale if isinstance(scale, torch.Tensor) else torch.tensor(np.asarray(scale, np.float32), device=q.device)
    sc = sc.to(device=q.device, dtype=torch.float32).contiguous()
    if out is None:
        out = torch.empty_like(q)
    if workspace is None:
        _order_on(stream, cu, sc, out)
        _check(load_library().nxg_attention(q.data_ptr(), k.data_ptr(), v.data_ptr(), cu.data_ptr(), cu.numel() - 1,
                                            sc.data_ptr(), T, n_head, n_kv_head, half, max(1, max_keys),
                                            out.data_ptr(), _stream_ptr(stream)), "attention")
        return out
    if isinstance(workspace, str):
        if workspace != "auto":
            raise ValueError('workspace must be None, "auto" or a uint8 device tensor')
        workspace = torch.empty(attention_workspace_bytes(T, n_head, n_kv_head, max(1, max_keys)),
                                dtype=torch.uint8, device=q.device)
    if workspace.dtype != torch.uint8 or not workspace.is_cuda or not workspace.is_contiguous():
        raise ValueError("workspace must be a contiguous uint8 device tensor")
    _order_on(stream, cu, sc, out, workspace)
    _check(load_library().nxg_attention_ws(q.data_ptr(), k.data_ptr(), v.data_ptr(), cu.data_ptr(), cu.numel() - 1,
                                           sc.data_ptr(), T, n_head, n_kv_head, half, max(1, max_keys),
                                           out.data_ptr(), workspace.data_ptr() if workspace.numel() else None,
                                           workspace.numel(), _stream_ptr(stream)), "attention")
    return out


def rope_table(n_pos: int, base: float, head_dim: int = 64):
    """build_rope (src/nexterabert.cpp:1322-1338) on the host: (cos, sin) [n_pos][head_dim/2]."""
    c = np.empty((n_pos, head_dim // 2), np.float32)
    s = np.empty_like(c)
    _check(load_library().nxg_rope_table(n_pos, float(base), head_dim, _np_ptr(c), _np_ptr(s)), "rope_table")
    return c, s


def qk_prep(x, alpha, beta, cos_t, sin_t, cu_offsets: Sequence[int], n_head: int, head_major: bool = False,
            out=None, stream=None):
    """op_qk_prep: DyT (beta * tanh(alpha * x)) then RoPE at each row's position in its
    document. x [T][n_head*D]; alpha, beta [D]; cos_t, sin_t [n_pos][D/2] (device tensors).
    Returns [T][n_head*D] or, head_major, [n_head][T][D]."""
    torch = _torch()
    _rows_arg(x, "x")
    T, width = x.shape
    D = width // n_head
    if D * n_head != width or D % 2:
        raise ValueError(f"x must be [T][n_head * head_dim] with an even head_dim")
    for name, t, n in (("alpha", alpha, D), ("beta", beta, D)):
        if t.dtype != torch.float32 or tuple(t.shape) != (n,) or not t.is_cuda or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous float32 device tensor [{n}]")
    _rows_arg(cos_t, "cos_t")
    _rows_arg(sin_t, "sin_t", cos_t.shape)
    if cos_t.shape[1] != D // 2:
        raise ValueError(f"cos_t / sin_t must be [n_pos][{D // 2}]")
    cu = _device_offsets(cu_offsets, x.device)
    if out is None:
        out = torch.empty((n_head, T, D) if head_major else (T, width), dtype=torch.float32, device=x.device)
    _order_on(stream, cu, out)
    _check(load_library().nxg_qk_prep(x.data_ptr(), alpha.data_ptr(), beta.data_ptr(), cos_t.data_ptr(),
                                      sin_t.data_ptr(), cos_t.shape[0], cu.data_ptr(), cu.numel() - 1, T, n_head, D,
                                      1 if head_major else 0, out.data_ptr(), _stream_ptr(stream)), "qk_prep")
    return out


def head_major(x, n_head: int, out=None, stream=None):
    """op_head_major: [T][n_head*D] -> [n_head][T][D]."""
    torch = _torch()
    _rows_arg(x, "x")
    T, width = x.shape
    D = width // n_head
    if out is None:
        out = torch.empty((n_head, T, D), dtype=torch.float32, device=x.device)
    _order_on(stream, out)
    _check(load_library().nxg_head_major(x.data_ptr(), T, n_head, D, out.data_ptr(), _stream_ptr(stream)), "head_major")
    return out


def qkv_prep(q, k, v, q_alpha, q_beta, k_alpha, k_beta, cos_t, sin_t, cu_offsets: Sequence[int], n_head: int,
             n_kv_head: int, stream=None):
    """qk_prep(q) (row-major), qk_prep(k) (head-major) and head_major(v) in one launch, each
    element as by the separate calls. Returns (q_out [T][n_head*D], k_out and v_out
    [n_kv_head][T][D])."""
    torch = _torch()
    for name, t in (("q", q), ("k", k), ("v", v)):
        _rows_arg(t, name)
    T, width = q.shape
    D = width // n_head
    if D * n_head != width or D % 2 or tuple(k.shape) != (T, n_kv_head * D) or tuple(v.shape) != (T, n_kv_head * D):
        raise ValueError("q must be [T][n_head * D], k and v [T][n_kv_head * D], D even")
    for name, t in (("q_alpha", q_alpha), ("q_beta", q_beta), ("k_alpha", k_alpha), ("k_beta", k_beta)):
        if t.dtype != torch.float32 or tuple(t.shape) != (D,) or not t.is_cuda or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous float32 device tensor [{D}]")
    _rows_arg(cos_t, "cos_t")
    _rows_arg(sin_t, "sin_t", cos_t.shape)
    if cos_t.shape[1] != D // 2:
        raise ValueError(f"cos_t / sin_t must be [n_pos][{D // 2}]")
    cu = _device_offsets(cu_offsets, q.device)
    qo = torch.empty((T, width), dtype=torch.float32, device=q.device)
    ko = torch.empty((n_kv_head, T, D), dtype=torch.float32, device=q.device)
    vo = torch.empty((n_kv_head, T, D), dtype=torch.float32, device=q.device)
    _order_on(stream, cu, qo, ko, vo)
    _check(load_library().nxg_qkv_prep(q.data_ptr(), k.data_ptr(), v.data_ptr(), q_alpha.data_ptr(), q_beta.data_ptr(),
                                       k_alpha.data_ptr(), k_beta.data_ptr(), cos_t.data_ptr(), sin_t.data_ptr(),
                                       cos_t.shape[0], cu.data_ptr(), cu.numel() - 1, T, n_head, n_kv_head, D,
                                       qo.data_ptr(), ko.data_ptr(), vo.data_ptr(), _stream_ptr(stream)), "qkv_prep")
    return qo, ko, vo


def dwconv_rows(x, taps, cu_offsets, r=None, out=None, stream=None):
    """op_dwconv as fp32 rows: r (or 0) + the depthwise convolution of x with taps [k][C]
    inside each document of the packed batch."""
    torch = _torch()
    _rows_arg(x, "x")
    T, C = x.shape
    _rows_arg(taps, "taps")
    if taps.shape[1] != C:
        raise ValueError(f"taps must be [k][{C}]")
    if r is not None:
        _rows_arg(r, "r", (T, C))
    cu = _device_offsets(cu_offsets, x.device)
    if out is None:
        out = torch.empty_like(x)
    _order_on(stream, cu, out)
    _check(load_library().nxg_dwconv_rows(x.data_ptr(), r.data_ptr() if r is not None else None, taps.data_ptr(),
                                          taps.shape[0], cu.data_ptr(), cu.numel() - 1, T, C, out.data_ptr(),
                                          _stream_ptr(stream)), "dwconv_rows")
    return out


def upsample_add(yb, r, cu_offsets, block: int, out=None, stream=None):
    """op_upsample_add: every token row of r plus its block's row of yb (ceil(len / block)
    block rows per document, in order)."""
    torch = _torch()
    _rows_arg(r, "r")
    T, C = r.shape
    _rows_arg(yb, "yb")
    cu_host = np.ascontiguousarray(cu_offsets, dtype=np.int32)
    cub_host = block_offsets(cu_host, block)
    if yb.shape != (int(cub_host[-1]), C):
        raise ValueError(f"yb must be [{int(cub_host[-1])}][{C}]")
    cu, cub = _device_offsets(cu_host, r.device), _device_offsets(cub_host, r.device)
    if out is None:
        out = torch.empty_like(r)
    _order_on(stream, cu, cub, out)
    _check(load_library().nxg_upsample_add(yb.data_ptr(), r.data_ptr(), cu.data_ptr(), cub.data_ptr(), cu.numel() - 1,
                                           T, yb.shape[0], block, C, out.data_ptr(), _stream_ptr(stream)),
           "upsample_add")
    return out


def embed_rows(table, ids, type_table=None, types=None, out=None, stream=None):
    """The encoder's input rows: table[ids] (+ type_table[types]). table [n_vocab][C] fp32,
    ids / types int32 device tensors [T]."""
    torch = _torch()
    _rows_arg(table, "table")
    n_vocab, C = table.shape
    if ids.dtype != torch.int32 or ids.dim() != 1 or not ids.is_cuda or not ids.is_contiguous():
        raise ValueError("ids must be a contiguous int32 device tensor [T]")
    T = ids.numel()
    n_types = 0
    if type_table is not None:
        _rows_arg(type_table, "type_table")
        n_types = type_table.shape[0]
        if type_table.shape[1] != C or types is None or types.dtype != torch.int32 or types.numel() != T:
            raise ValueError("type_table must be [n_types][C] with int32 types [T]")
    if out is None:
        out = torch.empty((T, C), dtype=torch.float32, device=table.device)
    _order_on(stream, out)
    _check(load_library().nxg_embed_rows(table.data_ptr(), n_vocab, ids.data_ptr(),
                                         type_table.data_ptr() if type_table is not None else None, n_types,
                                         types.data_ptr() if type_table is not None else None, T, C, out.data_ptr(),
                                         _stream_ptr(stream)), "embed_rows")
    return out


def layer_norm(x, w=None, b=None, eps: float = 1e-5, out=None, stream=None):
    """ggml_norm of each row, then * w and + b (either may be None)."""
    torch = _torch()
    _rows_arg(x, "x")
    T, C = x.shape
    for name, t in (("w", w), ("b", b)):
        if t is not None and (t.dtype != torch.float32 or tuple(t.shape) != (C,) or not t.is_cuda or not t.is_contiguous()):
            raise ValueError(f"{name} must be a contiguous float32 device tensor [{C}]")
    if out is None:
        out = torch.empty_like(x)
    _order_on(stream, out)
    _check(load_library().nxg_layer_norm(x.data_ptr(), w.data_ptr() if w is not None else None,
                                         b.data_ptr() if b is not None else None, eps, T, C, out.data_ptr(),
                                         _stream_ptr(stream)), "layer_norm")
    return out


def doc_mean(x, cu_offsets, normalize: bool = False, out=None, stream=None):
    """Per-document mean of the rows (normalize: the sum scaled to unit L2 norm), as
    nextera_encode's pooled output."""
    torch = _torch()
    _rows_arg(x, "x")
    T, C = x.shape
    cu = _device_offsets(cu_offsets, x.device)
    n = cu.numel() - 1
    if out is None:
        out = torch.empty((n, C), dtype=torch.float32, device=x.device)
    _order_on(stream, cu, out)
    _check(load_library().nxg_doc_mean(x.data_ptr(), cu.data_ptr(), n, T, C, 1 if normalize else 0, out.data_ptr(),
                                       _stream_ptr(stream)), "doc_mean")
    return out


def export_qact(qa: QAct, stream=None):
    """The qact in the reference's own format: (u8 [T][n_in], sx flat [(T+3)//4][n_blk][4])."""
    torch = _torch()
    nb = (qa.n_in + BLOCK - 1) // BLOCK
    u8 = torch.empty((qa.T, qa.n_in), dtype=torch.uint8, device=qa.q.device)
    sx = torch.empty(((qa.T + 3) // 4) * nb * 4, dtype=torch.float32, device=qa.q.device)
    _order_on(stream, u8, sx)
    _check(load_library().nxg_qact_export(qa.q.data_ptr(), qa.sx.data_ptr(), qa.T, qa.n_in, qa.act_max,
                                          u8.data_ptr(), sx.data_ptr(), _stream_ptr(stream)), "qact_export")
    return u8, sx


def _check_rows(t, T, n, name):
    torch = _torch()
    if t.dtype != torch.float32 or tuple(t.shape) != (T, n) or not t.is_contiguous() or not t.is_cuda:
        raise ValueError(f"{name} must be a contiguous float32 device tensor of shape ({T}, {n})")


def linear_i8(weight: DeviceWeight, qa: QAct, residual=None, cu_offsets: Optional[Sequence[int]] = None,
              out=None, stream=None):
    """op_linear_i8: f32 [T][n_out] = qact x weight^T with the per-block epilogue (+ residual).
    cu_offsets: the packed batch's cumulative row offsets (n_seqs + 1 entries); T = cu_offsets[-1]."""
    torch = _torch()
    if qa.n_in != weight.n_in:
        raise ValueError(f"n_in mismatch: activations {qa.n_in}, weight {weight.n_in}")
    T = qa.T
    if out is None:
        out = torch.empty((T, weight.n_out), dtype=torch.float32, device=qa.q.device)
    _check_rows(out, T, weight.n_out, "out")
    if residual is not None:
        _check_rows(residual, T, weight.n_out, "residual")
    L = load_library()
    res_ptr = residual.data_ptr() if residual is not None else None
    if cu_offsets is not None:
        cu = np.ascontiguousarray(cu_offsets, dtype=np.int32)
        if cu.size < 2 or int(cu[-1]) != T:
            raise ValueError(f"cu_offsets must end at T={T}")
        _order_on(stream, out)
        rc = L.nxg_linear_i8(weight.handle, qa.q.data_ptr(), qa.sx.data_ptr(), _np_ptr(cu), cu.size - 1,
                             res_ptr, out.data_ptr(), _stream_ptr(stream))
    else:
        _order_on(stream, out)
        rc = L.nxg_linear_i8_rows(weight.handle, qa.q.data_ptr(), qa.sx.data_ptr(), T, res_ptr,
                                  out.data_ptr(), _stream_ptr(stream))
    _check(rc, "linear_i8")
    return out


GEMM_RESIDUAL, GEMM_RELU2, GEMM_SUMS, GEMM_ACT63, GEMM_F32_IN = 1, 2, 4, 8, 16


def gemm_kernel_name(T: int, n_in: int, n_out: int, residual: bool = False, relu2: bool = False,
                     act_max: int = 127, sums: bool = False, cus: int = 0, f32_in: bool = False) -> str:
    """The kernel a GEMM of this shape launches, as the profiler names its template instance
    (nxg_gemm_kernel_name); cus = 0 asks the current device. f32_in: linear_f32_relu2_q8."""
    flags = ((GEMM_RESIDUAL if residual else 0) | (GEMM_RELU2 if relu2 else 0) | (GEMM_SUMS if sums else 0)
             | (GEMM_ACT63 if relu2 and act_max == 63 else 0) | (GEMM_F32_IN if f32_in else 0))
    name = load_library().nxg_gemm_kernel_name(T, n_in, n_out, flags, cus)
    if name is None:
        raise ValueError(f"gemm_kernel_name: no kernel for T={T} n_in={n_in} n_out={n_out} flags={flags}")
    return name.decode()


def linear_i8_split(weight: DeviceWeight, qa: QAct, cols: Sequence[int], outs=None, stream=None):
    """linear_i8 of a weight fused along n_out from several projections of the same input:
    one launch; columns [c_k, c_k + cols[k]) go to outs[k], a [T][cols[k]] float32 tensor
    (allocated when outs is None). Every boundary c_k must be a multiple of 64."""
    torch = _torch()
    if qa.n_in != weight.n_in:
        raise ValueError(f"n_in mismatch: activations {qa.n_in}, weight {weight.n_in}")
    cols = [int(c) for c in cols]
    T = qa.T
    if outs is None:
        outs = [torch.empty((T, c), dtype=torch.float32, device=qa.q.device) for c in cols]
    if len(outs) != len(cols):
        raise ValueError("one output per segment")
    for o, c in zip(outs, cols):
        _check_rows(o, T, c, "out")
    cols_a = np.ascontiguousarray(cols, dtype=np.int32)
    ptrs = (ctypes.c_void_p * len(outs))(*[o.data_ptr() for o in outs])
    _order_on(stream, *outs)
    _check(load_library().nxg_linear_i8_rows_split(weight.handle, qa.q.data_ptr(), qa.sx.data_ptr(), T, len(cols),
                                                   _np_ptr(cols_a), ctypes.cast(ptrs, ctypes.c_void_p),
                                                   _stream_ptr(stream)), "linear_i8_split")
    return outs


def linear_i8_relu2_q8(weight: DeviceWeight, qa: QAct, act_max: int = 127,
                       cu_offsets: Optional[Sequence[int]] = None, out: Optional[QAct] = None,
                       stream=None) -> QAct:
    """c_fc -> relu^2 -> int8 in one pass: the qact (T rows by n_out inputs) that
    quantize_rows_relu2 would make from linear_i8(weight, qa), without the fp32 rows."""
    if qa.n_in != weight.n_in:
        raise ValueError(f"n_in mismatch: activations {qa.n_in}, weight {weight.n_in}")
    T = qa.T
    res = out if out is not None else qact_alloc(T, weight.n_out, act_max, qa.q.device)
    res.T, res.n_in, res.act_max = T, weight.n_out, act_max
    L = load_library()
    if cu_offsets is not None:
        cu = np.ascontiguousarray(cu_offsets, dtype=np.int32)
        if cu.size < 2 or int(cu[-1]) != T:
            raise ValueError(f"cu_offsets must end at T={T}")
        _order_on(stream, res.q, res.sx)
        rc = L.nxg_linear_i8_relu2_q8(weight.handle, qa.q.data_ptr(), qa.sx.data_ptr(), _np_ptr(cu), cu.size - 1,
                                      act_max, res.q.data_ptr(), res.sx.data_ptr(), _stream_ptr(stream))
    else:
        _order_on(stream, res.q, res.sx)
        rc = L.nxg_linear_i8_relu2_q8_rows(weight.handle, qa.q.data_ptr(), qa.sx.data_ptr(), T, act_max,
                                           res.q.data_ptr(), res.sx.data_ptr(), _stream_ptr(stream))
    _check(rc, "linear_i8_relu2_q8")
    return res


def linear_f32_relu2_q8(weight: DeviceWeight, x, act_max: int = 127, cu_offsets: Optional[Sequence[int]] = None,
                        out: Optional[QAct] = None, workspace: Optional[QAct] = None, stream=None) -> QAct:
    """op_linear_i8 from fp32 rows for c_fc -> relu^2 -> int8 (nxg_linear_f32_relu2_q8): the
    same qact as linear_i8_relu2_q8(weight, quantize_rows(x, act_max), act_max). The row-tile
    kernel quantizes x inside the GEMM; other shapes quantize into `workspace` (a qact of x's
    shape, allocated when not given) first."""
    torch = _torch()
    if x.dtype != torch.float32 or x.dim() != 2 or not x.is_cuda or not x.is_contiguous():
        raise ValueError("x: a contiguous float32 CUDA tensor [T][n_in]")
    T, n_in = int(x.shape[0]), int(x.shape[1])
    if n_in != weight.n_in:
        raise ValueError(f"n_in mismatch: activations {n_in}, weight {weight.n_in}")
    res = out if out is not None else qact_alloc(T, weight.n_out, act_max, x.device)
    res.T, res.n_in, res.act_max = T, weight.n_out, act_max
    ws = workspace if workspace is not None else qact_alloc(T, n_in, act_max, x.device)
    _order_on(stream, res.q, res.sx, x, ws.q, ws.sx)
    L = load_library()
    if cu_offsets is not None:
        cu = np.ascontiguousarray(cu_offsets, dtype=np.int32)
        if cu.size < 2 or int(cu[-1]) != T:
            raise ValueError(f"cu_offsets must end at T={T}")
        rc = L.nxg_linear_f32_relu2_q8(weight.handle, x.data_ptr(), _np_ptr(cu), cu.size - 1, act_max, ws.q.data_ptr(),
                                       ws.sx.data_ptr(), res.q.data_ptr(), res.sx.data_ptr(), _stream_ptr(stream))
    else:
        rc = L.nxg_linear_f32_relu2_q8_rows(weight.handle, x.data_ptr(), T, act_max, ws.q.data_ptr(), ws.sx.data_ptr(),
                                            res.q.data_ptr(), res.sx.data_ptr(), _stream_ptr(stream))
    _check(rc, "linear_f32_relu2_q8")
    return res


def block_sums(weight: DeviceWeight, qa: QAct, stream=None):
    """int32 [n_blk][T][n_out]: the exact per-block sums of the GEMM."""
    torch = _torch()
    s = torch.empty((weight.n_blk, qa.T, weight.n_out), dtype=torch.int32, device=qa.q.device)
    _order_on(stream, s)
    _check(load_library().nxg_linear_i8_block_sums(weight.handle, qa.q.data_ptr(), qa.T, s.data_ptr(),
                                                   _stream_ptr(stream)), "block_sums")
    return s


@dataclass
class TensorInfo:
    name: str
    type: int
    n_dims: int
    ne: tuple            # ggml ne[0..3]: ne[0] is the row length
    offset: int          # from the start of the data section
    nbytes: int


class GGUF:
    """A GGUF model file (include/nxg_gguf.h): metadata, tensor table, tensor bytes, and
    the int8 load of the linear weights (the reference's nextera_load,
    src/nexterabert.cpp:1549-1712, for the tensors its int8 GEMM takes)."""

    def __init__(self, path: os.PathLike):
        L = load_library()
        h = ctypes.c_void_p()
        _check(L.nxg_gguf_open(os.fsencode(path), ctypes.byref(h)), "gguf_open")
        self._h, self.path = h, str(path)
        self.version = int(L.nxg_gguf_version(h))
        self.alignment = int(L.nxg_gguf_alignment(h))
        self.data_offset = int(L.nxg_gguf_data_offset(h))

    def close(self) -> None:
        if getattr(self, "_h", None) and self._h.value:
            load_library().nxg_gguf_close(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    # metadata
    def keys(self) -> List[str]:
        L = load_library()
        return [L.nxg_gguf_key(self._h, i).decode() for i in range(L.nxg_gguf_n_kv(self._h))]

    def _str(self, fn, *args) -> str:
        p, n = ctypes.c_void_p(), ctypes.c_uint64()
        _check(fn(self._h, *args, ctypes.byref(p), ctypes.byref(n)), "gguf metadata")
        return ctypes.string_at(p.value, n.value).decode("utf-8", errors="surrogateescape") if n.value else ""

    def get(self, key: str, default=None):
        """The value of `key` as int, float, bool, str or list; `default` if absent."""
        L = load_library()
        i = L.nxg_gguf_find_key(self._h, key.encode())
        if i < 0:
            return default
        t = L.nxg_gguf_kv_type(self._h, i)
        if t == GGUF_STRING:
            return self._str(L.nxg_gguf_get_str, i)
        if t == GGUF_ARRAY:
            et, n = ctypes.c_int32(), ctypes.c_uint64()
            _check(L.nxg_gguf_arr_info(self._h, i, ctypes.byref(et), ctypes.byref(n)), "gguf metadata")
            out = []
            for j in range(n.value):
                if et.value == GGUF_STRING:
                    out.append(self._str(L.nxg_gguf_arr_str, i, j))
                elif et.value in (GGUF_FLOAT32, GGUF_FLOAT64):
                    v = ctypes.c_double()
                    _check(L.nxg_gguf_arr_f64(self._h, i, j, ctypes.byref(v)), "gguf metadata")
                    out.append(v.value)
                else:
                    v = ctypes.c_int64()
                    _check(L.nxg_gguf_arr_i64(self._h, i, j, ctypes.byref(v)), "gguf metadata")
                    out.append(bool(v.value) if et.value == GGUF_BOOL else v.value)
            return out
        if t in (GGUF_FLOAT32, GGUF_FLOAT64):
            v = ctypes.c_double()
            _check(L.nxg_gguf_get_f64(self._h, i, ctypes.byref(v)), "gguf metadata")
            return v.value
        v = ctypes.c_int64()
        _check(L.nxg_gguf_get_i64(self._h, i, ctypes.byref(v)), "gguf metadata")
        return bool(v.value) if t == GGUF_BOOL else v.value

    def metadata(self) -> Dict[str, object]:
        return {k: self.get(k) for k in self.keys()}

    # tensors
    def tensors(self) -> List[TensorInfo]:
        L = load_library()
        out = []
        for i in range(L.nxg_gguf_n_tensors(self._h)):
            t, nd = ctypes.c_int32(), ctypes.c_int32()
            ne = (ctypes.c_int64 * 4)()
            off, nb = ctypes.c_uint64(), ctypes.c_uint64()
            _check(L.nxg_gguf_tensor_info(self._h, i, ctypes.byref(t), ctypes.byref(nd), ne, ctypes.byref(off),
                                          ctypes.byref(nb)), "gguf tensor_info")
            out.append(TensorInfo(L.nxg_gguf_tensor_name(self._h, i).decode(), t.value, nd.value, tuple(ne),
                                  off.value, nb.value))
        return out

    def _index(self, name: str) -> int:
        i = load_library().nxg_gguf_find_tensor(self._h, name.encode())
        if i < 0:
            raise KeyError(name)
        return i

    def tensor_bytes(self, name: str) -> np.ndarray:
        """A copy of the tensor's bytes as stored in the file."""
        L = load_library()
        i = self._index(name)
        info = self.tensors()[i]
        ptr = L.nxg_gguf_tensor_data(self._h, i)
        return np.frombuffer(ctypes.string_at(ptr, info.nbytes), dtype=np.uint8).copy()

    def int8_names(self) -> List[str]:
        """The tensors the reference runs on its int8 GEMM (src/nexterabert.cpp:1658-1667)."""
        L = load_library()
        return [t.name for t in self.tensors()
                if L.nxg_weight_is_int8(t.name.encode(), t.n_dims, t.type, t.ne[0], t.ne[1], 1)]

    def load_int8_weights(self, names: Optional[Sequence[str]] = None, n_threads: int = 0) -> Dict[str, DeviceWeight]:
        """Expands and uploads the int8 linear weights (all of them by default)."""
        L = load_library()
        out = {}
        for name in (self.int8_names() if names is None else names):
            h = ctypes.c_void_p()
            _check(L.nxg_gguf_weight_create(self._h, self._index(name), n_threads, ctypes.byref(h)),
                   f"gguf_weight_create({name})")
            out[name] = DeviceWeight(None, handle=h)
        return out


class Encoder:
    """The encoder on the GPU (include/nxg_encoder.h): nextera_load of a GGUF file, then
    nextera_encode / nextera_encode_segments of packed batches (src/nexterabert.cpp:1861-1935).

    encode() takes and returns host arrays; forward() runs on device tensors without
    synchronising (for timing and for callers that keep activations on the GPU)."""

    def __init__(self, path: os.PathLike, act_max: int = 127, load_threads: int = 0, verbosity: int = 0):
        L = load_library()
        self._h = None
        params = EncoderParams(act_max, load_threads, verbosity)
        h = ctypes.c_void_p()
        _check(L.nxg_encoder_load(os.fsencode(str(path)), ctypes.byref(params), ctypes.byref(h)), "encoder_load")
        self._h = h

    def close(self) -> None:
        if self._h is not None:
            load_library().nxg_encoder_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    @property
    def n_embd(self) -> int:
        return load_library().nxg_encoder_n_embd(self._h)

    @property
    def n_vocab(self) -> int:
        return load_library().nxg_encoder_n_vocab(self._h)

    @property
    def n_layer(self) -> int:
        return load_library().nxg_encoder_n_layer(self._h)

    @property
    def n_token_types(self) -> int:
        return load_library().nxg_encoder_n_token_types(self._h)

    @property
    def device_bytes(self) -> int:
        return int(load_library().nxg_encoder_device_bytes(self._h))

    @property
    def last_ms(self) -> float:
        return float(load_library().nxg_encoder_last_ms(self._h))

    @property
    def n_int8(self) -> int:
        return int(load_library().nxg_encoder_n_int8(self._h))

    PROFILE_KINDS = ("int8 linear", "attention", "norm / conv / gate / quantize", "other device work")

    def profile(self, enable: bool = True) -> None:
        """nxg_encoder_profile: clear the per-kind device times and turn profiling on or off."""
        load_library().nxg_encoder_profile(self._h, 1 if enable else 0)

    def profile_read(self) -> dict:
        """{"passes", "wall_ms", "device_ms", "kinds": {kind: ms}} summed over the profiled passes."""
        kinds = (ctypes.c_double * 4)()
        dev, wall, n = ctypes.c_double(), ctypes.c_double(), ctypes.c_int64()
        _check(load_library().nxg_encoder_profile_read(self._h, kinds, ctypes.byref(dev), ctypes.byref(wall),
                                                       ctypes.byref(n)), "encoder_profile_read")
        return {"passes": int(n.value), "wall_ms": wall.value, "device_ms": dev.value,
                "kinds": dict(zip(self.PROFILE_KINDS, list(kinds)))}

    def set_work_limit(self, nbytes: int) -> None:
        """nxg_encoder_set_work_limit: cap the work buffers (0: no cap); the attention's score
        workspace shrinks, down to none, to fit."""
        _check(load_library().nxg_encoder_set_work_limit(self._h, int(nbytes)), "encoder_set_work_limit")

    @property
    def attention_workspace(self) -> int:
        """Bytes of attention score workspace in the current work area."""
        return int(load_library().nxg_encoder_attention_workspace(self._h))

    def set_layers(self, n_layers: int) -> None:
        """Run only the first n_layers blocks, returning the residual stream (-1: all)."""
        load_library().nxg_encoder_set_layers(self._h, n_layers)

    def encode(self, tokens, lengths, token_types=None, hidden: bool = True, pooled: bool = False,
               normalize: bool = False):
        """Host arrays in, host arrays out: (hidden [sum(lengths)][n_embd] or None,
        pooled [n_seqs][n_embd] or None)."""
        tok = np.ascontiguousarray(tokens, dtype=np.int32)
        lens = np.ascontiguousarray(lengths, dtype=np.int32)
        typ = None if token_types is None else np.ascontiguousarray(token_types, dtype=np.int32)
        if typ is not None and typ.size != tok.size:
            raise ValueError("token_types must have one id per token")
        if lens.size == 0 or int(lens.sum()) != tok.size:
            raise ValueError("lengths must sum to the number of tokens")
        C = self.n_embd
        h = np.empty((tok.size, C), np.float32) if hidden else None
        p = np.empty((lens.size, C), np.float32) if pooled else None
        _check(load_library().nxg_encoder_encode(self._h, _np_ptr(tok), _np_ptr(typ), _np_ptr(lens), lens.size,
                                                 _np_ptr(h), _np_ptr(p), 1 if normalize else 0), "encoder_encode")
        return h, p

    def forward(self, tokens, lengths, token_types=None, hidden=None, pooled=None, normalize: bool = False,
                stream=None):
        """Device int32 tokens (and types) in; writes the device tensors hidden [T][n_embd]
        and / or pooled [n_seqs][n_embd] that are given."""
        torch = _torch()
        lens = np.ascontiguousarray(lengths, dtype=np.int32)
        T, C = int(lens.sum()), self.n_embd
        for name, t in (("tokens", tokens), ("token_types", token_types)):
            if t is not None and (t.dtype != torch.int32 or t.numel() != T or not t.is_cuda or not t.is_contiguous()):
                raise ValueError(f"{name} must be a contiguous int32 device tensor of {T} ids")
        if hidden is not None:
            _check_rows(hidden, T, C, "hidden")
        if pooled is not None:
            _check_rows(pooled, lens.size, C, "pooled")
        _check(load_library().nxg_encoder_forward(
            self._h, tokens.data_ptr(), token_types.data_ptr() if token_types is not None else None, _np_ptr(lens),
            lens.size, hidden.data_ptr() if hidden is not None else None,
            pooled.data_ptr() if pooled is not None else None, 1 if normalize else 0, _stream_ptr(stream)),
            "encoder_forward")


def cu_offsets_of(lengths: Sequence[int]) -> np.ndarray:
    """The packed batch's row offsets (the reference's layout::build, src/nexterabert.cpp:236-243)."""
    lens = np.asarray(lengths, dtype=np.int64)
    if lens.size == 0 or (lens <= 0).any():
        raise ValueError("empty sequence in batch")
    return np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)


class Builder:
    """builder::linear of the reference (src/nexterabert.cpp:1121-1143) over device weights.

    Weights registered under their GGUF names run on the int8 GEMM; an f32 input is
    quantized once and the quantized copy is shared by every linear that reads the
    same tensor (the reference's qcache, :1068,1125-1129). Weights that the placement
    rule keeps off the int8 path are not handled here.
    """

    def __init__(self, weights: Dict[str, DeviceWeight], act_max: int = 127):
        self.i8 = weights
        self.act_max = act_max
        self.qcache: Dict[int, QAct] = {}

    def int8_only(self, names: Sequence[str]) -> bool:
        return all(n in self.i8 for n in names)

    def quantized(self, x) -> QAct:
        key = x.data_ptr()
        qa = self.qcache.get(key)
        if qa is None or qa.T != x.shape[0] or qa.n_in != x.shape[1]:
            qa = quantize_rows(x, self.act_max)
            self.qcache[key] = qa
        return qa

    def linear(self, name: str, x, residual=None, cu_offsets=None, out=None):
        w = self.i8.get(name)
        if w is None:
            raise KeyError(f"{name} is not an int8 weight")
        qa = x if isinstance(x, QAct) else self.quantized(x)
        return linear_i8(w, qa, residual=residual, cu_offsets=cu_offsets, out=out)

    def rms_norm(self, x, gain, eps: float) -> QAct:
        """builder::rms_norm with int8 consumers (src/nexterabert.cpp:463-482, e.g. :1285):
        the normalized rows are quantized where they are made; the f32 rows are not kept."""
        return rmsnorm_quantize_rows(x, gain, eps, self.act_max)

    def mlp(self, fc: str, proj: str, h, x, cu_offsets=None, out=None):
        """x + c_proj(relu(c_fc(h))^2) (src/nexterabert.cpp:1284-1289). With both weights
        int8, relu^2 is quantized where c_fc's output is made (one fused pass when the
        shapes allow it, else c_fc in fp32 then quantize_rows_relu2)."""
        w_fc, w_proj = self.i8.get(fc), self.i8.get(proj)
        if w_fc is None or w_proj is None:
            raise KeyError(f"{fc} and {proj} must both be int8 weights")
        qa = h if isinstance(h, QAct) else self.quantized(h)
        if w_fc.n_in % 256 == 0 and w_fc.n_out % 32 == 0:
            r = linear_i8_relu2_q8(w_fc, qa, self.act_max, cu_offsets=cu_offsets)
        else:
            r = quantize_rows_relu2(linear_i8(w_fc, qa, cu_offsets=cu_offsets), self.act_max)
        return linear_i8(w_proj, r, residual=x, cu_offsets=cu_offsets, out=out)

    def gated_out(self, pre: str, y, z, x, cu_offsets=None, out=None):
        """x + c_proj(sigmoid(c_gate(y)) * z) (gated_out, src/nexterabert.cpp:1208-1213): y is
        quantized once (op_copy), c_gate runs in fp32 rows, and op_gate quantizes its rows for
        the int8 c_proj where it makes them."""
        gl = self.linear(pre + "c_gate.weight", y, cu_offsets=cu_offsets)
        gz = gate_quantize_rows(gl, z, self.act_max)
        return self.linear(pre + "c_proj.weight", gz, residual=x, cu_offsets=cu_offsets, out=out)

    def lily(self, pre: str, h, x, ltc_taps, state_taps, cu_offsets, out=None):
        """SnowLily's linears and their producers (mix_lily after its norm, src/nexterabert.cpp:
        1231-1243): z = in_proj(h), r = A(h), lr = dwconv(z; ltc taps) + r quantized for
        out_proj, a = out_proj(lr), xp = x_proj(h), b = B_proj(h), st = lily_state(a, xp, b)
        quantized for c_proj, x + c_proj(st). h: the norm's quantized rows (or f32 rows);
        taps [k][channels] as conv_params hands them over."""
        cu = cu_offsets if cu_offsets is not None else [0, (h.T if isinstance(h, QAct) else h.shape[0])]
        z = self.linear(pre + "ltc_conv.in_proj.weight", h, cu_offsets=cu)
        r = self.linear(pre + "ltc_conv.A.weight", h, cu_offsets=cu)
        lr = dwconv_quantize_rows(z, ltc_taps, cu, r=r, act_max=self.act_max)
        a = self.linear(pre + "ltc_conv.out_proj.weight", lr, cu_offsets=cu)
        xp = self.linear(pre + "x_proj.weight", h, cu_offsets=cu)
        b = self.linear(pre + "B_proj.weight", h, cu_offsets=cu)
        st = lily_state_quantize_rows(a, xp, b, state_taps, cu, act_max=self.act_max)
        return self.linear(pre + "c_proj.weight", st, residual=x, cu_offsets=cu, out=out)

    def hra_block_qkv(self, pre: str, ci, gt, cu_offsets, block: int = 4):
        """HRA's block attention inputs (mix_hra, src/nexterabert.cpp:1251-1256): the block
        means of ci * gt (op_block_mean, quantized for the int8 c_q / c_k / c_v, which share
        it) and the three projections on the block rows. Returns (q, k, v) fp32 rows."""
        hb = block_mean_quantize_rows(ci, cu_offsets, block, g=gt, act_max=self.act_max)
        cub = block_offsets(cu_offsets, block)
        return tuple(self.linear(pre + n, hb, cu_offsets=cub) for n in ("c_q.weight", "c_k.weight", "c_v.weight"))

    def reset(self) -> None:
        """Drops the quantized copies (the reference rebuilds its graph per forward)."""
        self.qcache.clear()
