"""GPU: the fp32 row ops around the encoder's int8 linears, bit for bit against the oracle
on packed batches of ragged documents: op_dwconv writing fp32 rows (HRA's qkv_conv / c_o,
src/nexterabert.cpp:524-543), op_upsample_add (:675-690), the embedding lookup with and
without segment rows (:1271-1272), the output LayerNorm (:1290-1291) and the pooled vectors
(:1913-1925), plus argument errors."""
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


def cuda(torch, a, dtype=np.float32):
    return torch.from_numpy(np.ascontiguousarray(a, dtype)).cuda()


LENGTHS = [[1], [1, 2, 3, 4, 5], [37, 1, 100, 6], [300]]


@pytest.mark.parametrize("lengths", LENGTHS)
@pytest.mark.parametrize("k,with_r", [(1, False), (3, False), (3, True), (5, True)])
def test_dwconv_rows(nxg, orc, torch, dev, lengths, k, with_r):
    say(f"dwconv_rows lengths={lengths} k={k} r={with_r}")
    rng = np.random.default_rng(len(lengths) * 10 + k)
    C = 1024
    cu = nxg.cu_offsets_of(lengths)
    T = int(cu[-1])
    x = rng.standard_normal((T, C)).astype(np.float32)
    r = rng.standard_normal((T, C)).astype(np.float32) if with_r else None
    taps = rng.standard_normal((k, C)).astype(np.float32)
    y = nxg.dwconv_rows(cuda(torch, x), cuda(torch, taps), cu, r=cuda(torch, r) if with_r else None).cpu().numpy()
    assert (bits(y) == bits(orc.dwconv(x, taps, cu, r=r))).all()


@pytest.mark.parametrize("lengths", LENGTHS)
@pytest.mark.parametrize("block", [1, 3, 4])
def test_upsample_add(nxg, orc, torch, dev, lengths, block):
    say(f"upsample_add lengths={lengths} block={block}")
    rng = np.random.default_rng(block + sum(lengths))
    C = 1024
    cu = nxg.cu_offsets_of(lengths)
    nb = int(nxg.block_offsets(cu, block)[-1])
    yb = rng.standard_normal((nb, C)).astype(np.float32)
    r = rng.standard_normal((int(cu[-1]), C)).astype(np.float32)
    y = nxg.upsample_add(cuda(torch, yb), cuda(torch, r), cu, block).cpu().numpy()
    assert (bits(y) == bits(orc.upsample_add(yb, r, cu, block))).all()


@pytest.mark.parametrize("C", [64, 96, 1024])
def test_embed_rows(nxg, torch, dev, C):
    say(f"embed_rows C={C}")
    rng = np.random.default_rng(C)
    table = rng.standard_normal((500, C)).astype(np.float32)
    types_t = rng.standard_normal((2, C)).astype(np.float32)
    ids = rng.integers(0, 500, 333).astype(np.int32)
    types = rng.integers(0, 2, 333).astype(np.int32)
    y = nxg.embed_rows(cuda(torch, table), cuda(torch, ids, np.int32)).cpu().numpy()
    assert (bits(y) == bits(table[ids])).all()
    y2 = nxg.embed_rows(cuda(torch, table), cuda(torch, ids, np.int32), cuda(torch, types_t),
                        cuda(torch, types, np.int32)).cpu().numpy()
    assert (bits(y2) == bits(table[ids] + types_t[types])).all()


@pytest.mark.parametrize("T,C", [(1, 1024), (333, 1024), (50, 96), (7, 64)])
def test_layer_norm(nxg, orc, torch, dev, T, C):
    say(f"layer_norm T={T} C={C}")
    rng = np.random.default_rng(T + C)
    x = (rng.standard_normal((T, C)) * np.exp(rng.uniform(-6, 6, (T, 1))) + rng.normal(0, 2, (T, 1))).astype(np.float32)
    x[0, : C // 2] = 0.0                      # a half-zero row
    if T > 2:
        x[1] = 2.5                            # a constant row
        x[2, 3] = np.nan                      # a NaN propagates through its row
    w = rng.uniform(0.5, 1.5, C).astype(np.float32)
    b = rng.standard_normal(C).astype(np.float32)
    for ww, bb in ((w, b), (w, None), (None, None)):
        y = nxg.layer_norm(cuda(torch, x), None if ww is None else cuda(torch, ww),
                           None if bb is None else cuda(torch, bb), eps=1e-5).cpu().numpy()
        ref = orc.layer_norm(x, ww, bb, 1e-5)
        assert ((bits(y) == bits(ref)) | (np.isnan(y) & np.isnan(ref))).all()


@pytest.mark.parametrize("lengths", LENGTHS)
@pytest.mark.parametrize("normalize", [False, True])
def test_doc_mean(nxg, orc, torch, dev, lengths, normalize):
    say(f"doc_mean lengths={lengths} normalize={normalize}")
    rng = np.random.default_rng(len(lengths) + normalize)
    C = 1024
    cu = nxg.cu_offsets_of(lengths)
    x = (rng.standard_normal((int(cu[-1]), C)) * 3).astype(np.float32)
    if normalize and len(lengths) > 1:
        x[: lengths[0]] = 0.0                 # a zero document: pooled vector 0
    y = nxg.doc_mean(cuda(torch, x), cu, normalize=normalize).cpu().numpy()
    assert (bits(y) == bits(orc.doc_mean(x, cu, normalize=normalize))).all()


@pytest.mark.parametrize("lengths,C", [([3000, 1, 257], 1024), ([513, 0, 40], 100), ([256, 255], 36), ([600], 2048)])
def test_doc_mean_long_and_narrow(nxg, orc, torch, dev, lengths, C):
    """Documents spanning several 256-row chunks (and exactly one), an empty document
    (mean 0 * (1 / 0): NaN, as the oracle), column counts that leave a partial 32-column slice."""
    say(f"doc_mean lengths={lengths} C={C}")
    rng = np.random.default_rng(C + len(lengths))
    cu = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)    # cu_offsets_of refuses empty ones
    x = (rng.standard_normal((int(cu[-1]), C)) * 3).astype(np.float32)
    for normalize in ([False, True] if C % 32 == 0 else [False]):
        y = nxg.doc_mean(cuda(torch, x), cu, normalize=normalize).cpu().numpy()
        ref = orc.doc_mean(x, cu, normalize=normalize)
        assert ((bits(y) == bits(ref)) | (np.isnan(y) & np.isnan(ref))).all(), f"normalize={normalize}"


def test_row_op_errors(nxg, torch, dev):
    x = torch.zeros(4, 1024, device="cuda")
    with pytest.raises(ValueError):
        nxg.dwconv_rows(x, torch.zeros(3, 512, device="cuda"), [0, 4])
    with pytest.raises(ValueError):
        nxg.upsample_add(torch.zeros(5, 1024, device="cuda"), x, [0, 4], 4)      # 1 block row, not 5
    with pytest.raises(ValueError):
        nxg.doc_mean(torch.zeros(4, 100, device="cuda"), [0, 4], normalize=True)  # C % 32 != 0
