"""GPU: nxg_attention_noalloc, the allocation-free variant of nxg_attention_ws (its workspace is
the library's static device array), called through the C ABI with ctypes: its outputs equal
nxg_attention_ws's (with a workspace of its own) bit for bit on two calls in a row, the second
with a smaller input, for documents long enough to keep their scores in the workspace and for
short ones; both calls are also checked against the oracle. A max_keys whose one slot would
not fit in the static array is refused before any device work."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

P, i32 = ctypes.c_void_p, ctypes.c_int32


def say(msg):
    print(msg, flush=True)


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


@pytest.fixture(scope="module")
def torch():
    import torch as t
    assert t.cuda.is_available(), "no GPU"
    return t


@pytest.fixture(scope="module")
def lib(nxg, torch):
    L = nxg.load_library()
    fn = L.nxg_attention_noalloc
    fn.argtypes = [P, P, P, P, i32, P, i32, i32, i32, i32, i32, P, P]
    fn.restype = i32
    nxg.init()
    return L


def call_noalloc(lib, torch, q, k, v, cu, sc, T, H, G, half, max_keys, out):
    rc = lib.nxg_attention_noalloc(q.data_ptr(), k.data_ptr(), v.data_ptr(), cu.data_ptr(), cu.numel() - 1,
                                   sc.data_ptr(), T, H, G, half, max_keys, out.data_ptr(),
                                   torch.cuda.current_stream().cuda_stream or None)
    assert rc == 0, lib.nxg_last_error()


@pytest.mark.parametrize("lengths,half,H,G", [([3000], -1, 2, 1), ([2700, 9, 400], 1300, 4, 2), ([300, 45], -1, 16, 8)])
def test_noalloc_equals_workspace_entry_point(nxg, orc, lib, torch, lengths, half, H, G):
    say(f"attention_noalloc lengths={lengths} half={half} H={H} G={G}")
    rng = np.random.default_rng(sum(lengths) + H)
    for call, lens in enumerate((lengths, [max(1, n * 3 // 4) for n in lengths])):   # the second call smaller
        cu_h = nxg.cu_offsets_of(lens)
        T = int(cu_h[-1])
        q = rng.standard_normal((T, H * 64)).astype(np.float32)
        k, v = (rng.standard_normal((G, T, 64)).astype(np.float32) for _ in range(2))
        scale = rng.uniform(0.05, 0.2, len(lens)).astype(np.float32)
        c = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()
        qd, kd, vd, sd = c(q), c(k), c(v), c(scale)
        cu = torch.from_numpy(cu_h.astype(np.int32)).cuda()
        diffs = np.diff(cu_h)
        max_keys = int(diffs.max()) if half < 0 else int(min(diffs.max(), 2 * half + 1))
        y_ws = nxg.attention(qd, kd, vd, cu_h, scale, H, G, half, workspace="auto")
        y = torch.full_like(qd, float("nan"))
        call_noalloc(lib, torch, qd, kd, vd, cu, sd, T, H, G, half, max_keys, y)
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int32), y_ws.view(torch.int32)), f"call {call}: differs from nxg_attention_ws"
        assert (bits(y.cpu().numpy()) == bits(orc.attention(q, k, v, cu_h, scale, H, G, half))).all(), \
            f"call {call}: differs from the oracle"


def test_noalloc_refuses_keys_beyond_the_scratch(nxg, lib, torch):
    say("attention_noalloc refuses max_keys beyond its static scratch")
    T, H, G = 8, 2, 1
    q = torch.zeros(T, H * 64, device="cuda")
    k = torch.zeros(G, T, 64, device="cuda")
    cu = torch.tensor([0, T], dtype=torch.int32, device="cuda")
    sc = torch.ones(1, device="cuda")
    out = torch.zeros_like(q)
    rc = lib.nxg_attention_noalloc(q.data_ptr(), k.data_ptr(), k.data_ptr(), cu.data_ptr(), 1, sc.data_ptr(), T, H, G,
                                   -1, 2_000_000, out.data_ptr(), None)
    assert rc == nxg.NXG_EINVAL
    assert b"static scratch" in lib.nxg_last_error()
