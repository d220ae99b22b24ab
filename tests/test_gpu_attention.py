"""GPU: op_attention (head_dim 64) bit for bit against the oracle (src/nexterabert.cpp:704-852):
documents of 1 to 4,000 tokens (key counts off multiples of 8 send the last keys through
hsum256 and the C library's expf), full and banded (swa) attention, 16 query / 8 KV heads,
per-document scales, and scores large enough to underflow exp in both its forms. The kernel
depends on the keys per query: the tile kernel up to ~2,400 (scores in LDS), the three-pass
kernel beyond (scores recomputed), the row kernel for head ratios that do not divide 16."""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


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
def dev(torch, nxg):
    nxg.init()
    return torch.device("cuda:0")


def run(nxg, torch, q, k, v, cu, scale, H, G, half, workspace=None):
    c = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()
    return nxg.attention(c(q), c(k), c(v), cu, scale, H, G, half, workspace=workspace).cpu().numpy()


CASES = [
    ([1, 7, 8, 9, 64, 111], -1),
    ([1, 7, 8, 9, 64, 111], 5),
    ([1, 7, 8, 9, 64, 111], 64),
    ([1024], -1),
    ([1024], 128),
    ([300, 2, 45], 0),
]


@pytest.mark.parametrize("lengths,half", CASES)
def test_attention_matches_oracle(nxg, orc, torch, dev, lengths, half):
    say(f"attention lengths={lengths} half={half}")
    rng = np.random.default_rng(sum(lengths) + half)
    H, G = 16, 8
    cu = nxg.cu_offsets_of(lengths)
    T = int(cu[-1])
    q = rng.standard_normal((T, H * 64)).astype(np.float32)
    k = rng.standard_normal((G, T, 64)).astype(np.float32)
    v = rng.standard_normal((G, T, 64)).astype(np.float32)
    scale = rng.uniform(0.05, 0.3, len(lengths)).astype(np.float32)
    y = run(nxg, torch, q, k, v, cu, scale, H, G, half)
    ref = orc.attention(q, k, v, cu, scale, H, G, half)
    assert (bits(y) == bits(ref)).all()


def test_attention_long_document(nxg, orc, torch, dev):
    say("attention one document of 2,500 tokens")
    rng = np.random.default_rng(7)
    H, G = 2, 1
    cu = nxg.cu_offsets_of([2500])
    q = rng.standard_normal((2500, H * 64)).astype(np.float32)
    k, v = (rng.standard_normal((G, 2500, 64)).astype(np.float32) for _ in range(2))
    scale = np.array([0.125], np.float32)
    assert (bits(run(nxg, torch, q, k, v, cu, scale, H, G, -1)) == bits(orc.attention(q, k, v, cu, scale, H, G))).all()


@pytest.mark.parametrize("lengths,half", [([4000], 1500), ([3000, 5, 700], -1)])
def test_attention_long_documents(nxg, orc, torch, dev, lengths, half):
    """Past the tile kernel's LDS: the three-pass kernel, banded and packed."""
    say(f"attention long lengths={lengths} half={half}")
    rng = np.random.default_rng(len(lengths) + 3)
    H, G = 2, 1
    cu = nxg.cu_offsets_of(lengths)
    T = int(cu[-1])
    q = rng.standard_normal((T, H * 64)).astype(np.float32)
    k, v = (rng.standard_normal((G, T, 64)).astype(np.float32) for _ in range(2))
    scale = rng.uniform(0.05, 0.2, len(lengths)).astype(np.float32)
    y = run(nxg, torch, q, k, v, cu, scale, H, G, half)
    assert (bits(y) == bits(orc.attention(q, k, v, cu, scale, H, G, half))).all()


@pytest.mark.parametrize("lengths,half,H,G", [([4000], 1500, 2, 1), ([3000, 5, 700], -1, 2, 1),
                                              ([2600, 1, 9], -1, 4, 2), ([2500], 1300, 1, 1)])
def test_attention_stored_scores(nxg, orc, torch, dev, lengths, half, H, G):
    """nxg_attention_ws past the tile kernel's LDS: the scores written once to the workspace and
    read back by the softmax and the values give the oracle's bits, with a slot for every
    resident workgroup and with 3 slots (each workgroup then takes many tiles in turn)."""
    say(f"attention stored scores lengths={lengths} half={half} H={H} G={G}")
    rng = np.random.default_rng(len(lengths) + 11 * H + half)
    cu = nxg.cu_offsets_of(lengths)
    T = int(cu[-1])
    q = rng.standard_normal((T, H * 64)).astype(np.float32)
    k, v = (rng.standard_normal((G, T, 64)).astype(np.float32) for _ in range(2))
    scale = rng.uniform(0.05, 0.2, len(lengths)).astype(np.float32)
    ref = orc.attention(q, k, v, cu, scale, H, G, half)
    lens = np.diff(cu)
    max_keys = int(lens.max()) if half < 0 else int(min(lens.max(), 2 * half + 1))
    full = nxg.attention_workspace_bytes(T, H, G, max_keys)
    slot = 16 * max_keys * 4
    assert full >= slot and full % slot == 0
    for ws in ("auto", torch.empty(3 * slot + 100, dtype=torch.uint8, device="cuda")):
        y = run(nxg, torch, q, k, v, cu, scale, H, G, half, workspace=ws)
        assert (bits(y) == bits(ref)).all()


@pytest.mark.parametrize("lengths", [[1536], [1024, 1024], [1100, 900, 48]])
def test_attention_stored_where_tiles_fit(nxg, orc, torch, dev, lengths):
    """Scores that fit in LDS with room for one workgroup per CU (1,536 keys), or for two in a
    launch of more than two rounds (2,048 tiles), go to the stored kernel when a workspace is
    given, to the tile kernel without one: both give the oracle's bits."""
    say(f"attention stored where tiles fit lengths={lengths}")
    rng = np.random.default_rng(sum(lengths) + 21)
    H, G = 16, 8
    cu = nxg.cu_offsets_of(lengths)
    T = int(cu[-1])
    assert nxg.attention_workspace_bytes(T, H, G, max(lengths)) > 0
    q = rng.standard_normal((T, H * 64)).astype(np.float32)
    k, v = (rng.standard_normal((G, T, 64)).astype(np.float32) for _ in range(2))
    scale = rng.uniform(0.05, 0.2, len(lengths)).astype(np.float32)
    ref = orc.attention(q, k, v, cu, scale, H, G, -1)
    for ws in ("auto", None):
        assert (bits(run(nxg, torch, q, k, v, cu, scale, H, G, -1, workspace=ws)) == bits(ref)).all(), ws


def test_attention_workspace_ignored_when_scores_fit(nxg, orc, torch, dev):
    """Short documents keep their scores in LDS: no workspace is asked for, and one given is unused."""
    say("attention workspace with short documents")
    assert nxg.attention_workspace_bytes(1024, 16, 8, 1024) == 0
    rng = np.random.default_rng(12)
    H, G = 4, 2
    cu = nxg.cu_offsets_of([100, 30])
    T = int(cu[-1])
    q = rng.standard_normal((T, H * 64)).astype(np.float32)
    k, v = (rng.standard_normal((G, T, 64)).astype(np.float32) for _ in range(2))
    scale = np.array([0.1, 0.2], np.float32)
    ws = torch.empty(4096, dtype=torch.uint8, device="cuda")
    y = run(nxg, torch, q, k, v, cu, scale, H, G, -1, workspace=ws)
    assert (bits(y) == bits(orc.attention(q, k, v, cu, scale, H, G))).all()


def test_attention_head_ratio_3(nxg, orc, torch, dev):
    """6 query heads over 2 KV heads (3 does not divide 16): the row kernel."""
    say("attention H=6 G=2")
    rng = np.random.default_rng(31)
    H, G = 6, 2
    cu = nxg.cu_offsets_of([17, 1, 64])
    T = int(cu[-1])
    q = rng.standard_normal((T, H * 64)).astype(np.float32)
    k, v = (rng.standard_normal((G, T, 64)).astype(np.float32) for _ in range(2))
    scale = np.array([0.1, 0.2, 0.15], np.float32)
    for half in (-1, 4):
        y = run(nxg, torch, q, k, v, cu, scale, H, G, half)
        assert (bits(y) == bits(orc.attention(q, k, v, cu, scale, H, G, half))).all()


def test_attention_extreme_scores(nxg, orc, torch, dev):
    """Scores spread over +-400: most exponentials underflow, in exp256 (clamped at -87.3)
    and in the C library's expf (to subnormals and to 0)."""
    say("attention with extreme scores")
    rng = np.random.default_rng(8)
    H, G = 4, 2
    cu = nxg.cu_offsets_of([13, 29, 5])
    T = int(cu[-1])
    q = (rng.standard_normal((T, H * 64)) * 6).astype(np.float32)
    k, v = (rng.standard_normal((G, T, 64)).astype(np.float32) for _ in range(2))
    scale = np.array([1.0, 0.5, 2.0], np.float32)
    y = run(nxg, torch, q, k, v, cu, scale, H, G, -1)
    assert (bits(y) == bits(orc.attention(q, k, v, cu, scale, H, G))).all()


@pytest.mark.parametrize("lengths,half,H,G,ws", [([40, 300, 25], -1, 16, 8, None), ([600], 100, 16, 8, None),
                                                 ([3000], 1300, 2, 1, "auto"), ([40, 2900, 25], -1, 2, 1, "auto"),
                                                 ([40, 2900, 25], -1, 2, 1, None)])
def test_attention_non_finite_values_outside_a_pair(nxg, orc, torch, dev, lengths, half, H, G, ws):
    """Inf and NaN values at keys that other pairs of the same staged tile do not attend to (a
    neighbour document, outside a band), on the tile, stored and recomputing kernels: value
    tiles that hold them take the per-key path, the others the broadcast path with zero weights
    outside a pair's keys; the pairs that do not see them stay finite and give the oracle's
    bits, the others its NaN / Inf pattern."""
    say(f"attention non-finite values lengths={lengths} half={half} H={H} G={G} ws={ws}")
    rng = np.random.default_rng(sum(lengths) + 31)
    cu = nxg.cu_offsets_of(lengths)
    T = int(cu[-1])
    q = rng.standard_normal((T, H * 64)).astype(np.float32)
    k, v = (rng.standard_normal((G, T, 64)).astype(np.float32) for _ in range(2))
    bad = [3, 30, T - 5] if len(lengths) > 1 else [5, T // 2, T - 3]
    v[:, bad[0], 5] = np.inf
    v[:, bad[1], 7] = np.nan
    v[:, bad[2], 9] = -np.inf
    scale = rng.uniform(0.05, 0.2, len(lengths)).astype(np.float32)
    y = run(nxg, torch, q, k, v, cu, scale, H, G, half, workspace=ws)
    ref = orc.attention(q, k, v, cu, scale, H, G, half)
    same = (bits(y) == bits(ref)) | (np.isnan(y) & np.isnan(ref))
    assert same.all()
    assert np.isfinite(ref).mean() > 0.5 and not np.isfinite(ref).all()


def test_attention_document_alone(nxg, torch, dev):
    say("attention: a document alone and in a batch")
    rng = np.random.default_rng(9)
    H, G = 16, 8
    lengths = [33, 100, 7]
    cu = nxg.cu_offsets_of(lengths)
    T = int(cu[-1])
    q = rng.standard_normal((T, H * 64)).astype(np.float32)
    k, v = (rng.standard_normal((G, T, 64)).astype(np.float32) for _ in range(2))
    scale = np.array([0.1, 0.2, 0.3], np.float32)
    y = run(nxg, torch, q, k, v, cu, scale, H, G, -1)
    lo, hi = 33, 133
    alone = run(nxg, torch, q[lo:hi], k[:, lo:hi], v[:, lo:hi], [0, 100], scale[1:2], H, G, -1)
    assert (bits(alone) == bits(y[lo:hi])).all()


@pytest.mark.parametrize("head_major", [False, True])
def test_qk_prep_matches_oracle(nxg, orc, torch, dev, head_major):
    say(f"qk_prep head_major={head_major}")
    rng = np.random.default_rng(20 + head_major)
    H, D = 16, 64
    lengths = [1, 7, 100, 33]
    cu = nxg.cu_offsets_of(lengths)
    T = int(cu[-1])
    x = (rng.standard_normal((T, H * D)) * np.exp(rng.uniform(-6, 3, (T, 1)))).astype(np.float32)
    x.flat[rng.integers(0, x.size, 50)] = np.array([0.0, -0.0, 0.1, -0.1, 30.0, -1e-30], np.float32)[rng.integers(0, 6, 50)]
    alpha = rng.uniform(0.2, 2.0, D).astype(np.float32)
    beta = rng.uniform(0.5, 1.5, D).astype(np.float32)
    c, s = nxg.rope_table(128, 10000.0, D)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()
    y = nxg.qk_prep(t(x), t(alpha), t(beta), t(c), t(s), cu, H, head_major=head_major).cpu().numpy()
    assert (bits(y) == bits(orc.qk_prep(x, alpha, beta, c, s, cu, H, head_major=head_major))).all()


@pytest.mark.parametrize("H,G", [(16, 8), (2, 1), (4, 4)])
def test_qkv_prep_equals_separate_calls(nxg, torch, dev, H, G):
    """nxg_qkv_prep: the queries' and keys' qk_prep and the values' head-major copy in one
    launch give the separate calls' bits (test_qk_prep_matches_oracle pins those)."""
    say(f"qkv_prep H={H} G={G}")
    rng = np.random.default_rng(H + G)
    D = 64
    cu = nxg.cu_offsets_of([1, 7, 100, 33])
    T = int(cu[-1])
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()
    q, k, v = (t(rng.standard_normal((T, n * D)) * 3) for n in (H, G, G))
    qa, qb, ka, kb = (t(rng.uniform(0.2, 2.0, D)) for _ in range(4))
    c, s = nxg.rope_table(128, 10000.0, D)
    c, s = t(c), t(s)
    qo, ko, vo = nxg.qkv_prep(q, k, v, qa, qb, ka, kb, c, s, cu, H, G)
    refs = (nxg.qk_prep(q, qa, qb, c, s, cu, H), nxg.qk_prep(k, ka, kb, c, s, cu, G, head_major=True),
            nxg.head_major(v, G))
    for got, ref in zip((qo, ko, vo), refs):
        assert (bits(got.cpu().numpy()) == bits(ref.cpu().numpy())).all()


def test_head_major(nxg, torch, dev):
    say("head_major")
    x = torch.randn(77, 8 * 64, device="cuda")
    y = nxg.head_major(x, 8)
    assert torch.equal(y, x.view(77, 8, 64).permute(1, 0, 2).contiguous())


def test_attention_workspace_16384_keys(nxg, torch, dev):
    """One 16,384-token document: nxg_attention_ws with a 3-slot workspace (few workgroups at a
    time, each over many query tiles; 3 MiB of slots, so pass 2 stores the exponentials for pass
    3) and with a slot per resident workgroup (512 MiB: pass 3 recomputes them) equals the
    recomputing kernel (no workspace) bit for bit."""
    say("attention 16,384 keys: 3-slot and full workspaces vs recomputing kernel")
    H, G, T = 2, 1, 16384
    g = torch.Generator("cuda").manual_seed(16)
    q = torch.randn(T, H * 64, device="cuda", generator=g)
    k = torch.randn(G, T, 64, device="cuda", generator=g)
    v = torch.randn(G, T, 64, device="cuda", generator=g)
    cu = [0, T]
    scale = np.array([0.125], np.float32)
    slot = 16 * T * 4
    y_rec = nxg.attention(q, k, v, cu, scale, H, G)
    y_ws = nxg.attention(q, k, v, cu, scale, H, G, workspace=torch.empty(3 * slot, dtype=torch.uint8, device="cuda"))
    y_full = nxg.attention(q, k, v, cu, scale, H, G, workspace="auto")
    torch.cuda.synchronize()
    assert torch.isfinite(y_rec).all()
    assert torch.equal(y_rec.view(torch.int32), y_ws.view(torch.int32))
    assert torch.equal(y_rec.view(torch.int32), y_full.view(torch.int32))


def test_attention_auto_workspace_on_a_side_stream(nxg, orc, torch, dev):
    """workspace="auto" with a caller's stream: the wrapper's temporaries (offsets, scales,
    workspace) allocated on torch's current stream stay reserved until the side stream's
    kernel is done, although the caller reuses memory on the current stream right away."""
    say("attention auto workspace on a side stream")
    rng = np.random.default_rng(31)
    H, G, T = 2, 1, 2600
    cu = nxg.cu_offsets_of([T])
    q = rng.standard_normal((T, H * 64)).astype(np.float32)
    k, v = (rng.standard_normal((G, T, 64)).astype(np.float32) for _ in range(2))
    scale = np.array([0.1], np.float32)
    ref = orc.attention(q, k, v, cu, scale, H, G)
    c = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()
    qd, kd, vd = c(q), c(k), c(v)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    y = nxg.attention(qd, kd, vd, cu, scale, H, G, stream=side, workspace="auto")
    junk = torch.full((nxg.attention_workspace_bytes(T, H, G, T) // 4 + 4096,), float("nan"), device="cuda")
    side.synchronize()
    torch.cuda.synchronize()
    assert (bits(y.cpu().numpy()) == bits(ref)).all()
    del junk
