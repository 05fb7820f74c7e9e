"""GPU parity of the paged decode (cqkv_decode_attention_paged): the reference's
attention_packed_blocks over a block table (candle-nn/src/turbo_quant.rs:1082-1114,
candle-core/src/accel/attention.rs:293-366), where the keys are the blocks' valid rows
concatenated in block order and masks are bottom-right aligned over that concatenation.

Checked against the oracle decode of the concatenated rows (max-abs 2e-2 / mean-abs 2e-3), and
against the dense decode of one cache holding the same rows: the reference's own claim is that
paged and dense agree up to the summation order, so the bar is each format's split invariance
(test_decode_split_invariance). Rows past a block's valid count hold large decoy values, which
must not reach the output."""
import numpy as np
import pytest
import torch

from tests.helpers import (assert_close_bf16, assert_decode_parity, exact_decode, exact_scores,
                           kv_source, oracle_decode, oracle_rows)

pytestmark = pytest.mark.gpu

FMTS = {"fp8": 5, "mxfp4": 2, "turbo4": 0, "nvfp4": 3, "mxfp8": 4}


def export_np(cq, side, tokens):
    return cq.rows_export(side, tokens).cpu().numpy().view(np.uint32)


def paged_case(cq, dev, fmt, b, hq, hkv, d, sizes, caps, lq=1, wl=-1, wr=-1, seed=0,
               outliers=True):
    f = FMTS[fmt]
    total = sum(sizes)
    q = kv_source(seed + 1, (b, hq, lq, d))
    k = kv_source(seed + 2, (b, hkv, total, d), outliers)
    v = kv_source(seed + 3, (b, hkv, total, d), outliers)
    blocks, off = [], 0
    for i, (n, cap) in enumerate(zip(sizes, caps)):
        kc = cq.CacheSide.empty(f, False, b, hkv, d, cap, dev, seed=42)
        vc = cq.CacheSide.empty(f, True, b, hkv, d, cap, dev, seed=44)
        if n:
            cq.quant_append(kc, k[:, :, off:off + n].to(dev), 0)
            cq.quant_append(vc, v[:, :, off:off + n].to(dev), 0)
        if cap > n:  # decoys past the valid rows
            junk = kv_source(seed + 100 + i, (b, hkv, cap - n, d)) * 50
            cq.quant_append(kc, junk.to(dev), n)
            cq.quant_append(vc, junk.to(dev), n)
        blocks.append((kc, vc, n))
        off += n
    scale = 1.0 / d ** 0.5
    got = cq.decode_attention_paged(q.to(dev), blocks, scale, window_left=wl, window_right=wr,
                                    out=torch.empty((b, hq, lq, d), dtype=torch.float32, device=dev))
    # the same rows in one dense cache
    cap = (total + 31) // 32 * 32
    dense = cq.TurboKvCache(f, f, b, hkv, d, cap, device=dev)
    dense.append(k.to(dev), v.to(dev))
    want_dense = cq.decode_attention(q.to(dev), dense.k, dense.v, total, scale, window_left=wl,
                                     window_right=wr,
                                     out=torch.empty((b, hq, lq, d), dtype=torch.float32,
                                                     device=dev))
    torch.cuda.synchronize()
    if f == 0:  # decode parity on the codes the GPU wrote (encoder flips are checked elsewhere)
        kr = np.concatenate([export_np(cq, kc, n) for kc, _, n in blocks if n], axis=2)
        vr = np.concatenate([export_np(cq, vc, n) for _, vc, n in blocks if n], axis=2)
    else:
        kr, vr = oracle_rows(f, k, 42), oracle_rows(f, v, 44)
    want = oracle_decode(f, q, kr, vr, total, scale, wl=wl, wr=wr)
    got = got.cpu().numpy()
    # one-operand P (MXFP4 bf16, TurboQuant-4 and NVFP4 f16): segments round P against other
    # maxima
    atol, rtol = {"mxfp4": (2e-3, 4e-3), "turbo4": (2e-3, 4e-3), "nvfp4": (2e-4, 2e-3)}.get(fmt, (1e-5, 1e-4))
    np.testing.assert_allclose(got, want_dense.cpu().numpy(), atol=atol, rtol=rtol)
    if exact_scores(f):
        exact = exact_decode(f, q, kr, vr, total, scale, wl=wl, wr=wr)
        assert_decode_parity(f, got, want, exact)
    else:
        assert_close_bf16(got, want)
    return got


@pytest.mark.parametrize("fmt", ["fp8", "mxfp4", "turbo4", "nvfp4", "mxfp8"])
def test_paged_blocks_of_uneven_sizes(cq, dev, fmt):
    """Blocks of 100, 37, 0, 256 and 5 rows with capacities 128, 64, 32, 256 and 32: tiles that
    cross a block's valid end, an empty block, a block filling its capacity."""
    paged_case(cq, dev, fmt, 2, 8, 2, 128, [100, 37, 0, 256, 5], [128, 64, 32, 256, 32])


@pytest.mark.parametrize("fmt", ["fp8", "turbo4"])
@pytest.mark.parametrize("wl,wr", [(40, 0), (-1, 0), (3, 1)])
def test_paged_multi_query_windows(cq, dev, fmt, wl, wr):
    """Windows bottom-right aligned over the concatenated keys, across block boundaries. No
    outlier channels, as in the dense window tests: a 3-key window averages a handful of rows, and
    bf16 P against x8 channels alone moves the reference path by ~3e-2 there."""
    paged_case(cq, dev, fmt, 1, 16, 4, 128, [33, 64, 20], [64, 64, 32], lq=4, wl=wl, wr=wr,
               seed=5, outliers=False)


def test_paged_more_blocks_than_the_reference_table(cq, dev):
    """150 blocks (the reference's table stops at 128 and concatenates beyond)."""
    rng = np.random.default_rng(3)
    sizes = [int(x) for x in rng.integers(1, 40, 150)]
    paged_case(cq, dev, "fp8", 1, 8, 8, 64, sizes, [64] * 150, seed=9, outliers=False)


@pytest.mark.parametrize("fmt", ["fp8", "turbo4"])
def test_paged_single_segment(cq, dev, fmt):
    """One short block: one segment, no combine pass (TurboQuant unrotates in the kernel)."""
    paged_case(cq, dev, fmt, 1, 8, 8, 64, [40], [64], seed=2)


def test_paged_caller_workspace(cq, dev):
    """With a caller-sized workspace the call allocates nothing and gives the same result."""
    b, hq, hkv, d = 2, 8, 2, 128
    blocks = []
    for n in (200, 300):
        kc = cq.CacheSide.empty(5, False, b, hkv, d, 320, dev)
        vc = cq.CacheSide.empty(5, True, b, hkv, d, 320, dev)
        x = kv_source(n, (b, hkv, n, d))
        cq.quant_append(kc, x.to(dev), 0)
        cq.quant_append(vc, x.to(dev), 0)
        blocks.append((kc, vc, n))
    q = kv_source(1, (b, hq, 1, d)).to(dev)
    nbytes = cq.decode_paged_workspace_bytes(blocks, b, hq, 1)
    assert nbytes > 0
    ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    a = cq.decode_attention_paged(q, blocks, 0.1, workspace=ws)
    c = cq.decode_attention_paged(q, blocks, 0.1)
    torch.cuda.synchronize()
    assert torch.equal(a, c)
    with pytest.raises(cq.CqkvError):
        cq.decode_attention_paged(q, blocks, 0.1, workspace=ws[:16])


def test_paged_decode_graph_capture_replays(cq, dev):
    """A paged decode captured into a HIP graph and replayed: its segment table travels in kernel
    arguments (captured by value), so every replay matches the eager result, with eager paged
    calls over other blocks between the replays (which rewrite the same workspace's table)."""
    b, hq, hkv, d = 2, 8, 2, 128
    blocks, others = [], []
    for n, store in ((70, blocks), (130, blocks), (40, blocks), (90, others), (33, others)):
        kc = cq.CacheSide.empty(5, False, b, hkv, d, 160, dev)
        vc = cq.CacheSide.empty(5, True, b, hkv, d, 160, dev)
        x = kv_source(n + 7, (b, hkv, n, d))
        cq.quant_append(kc, x.to(dev), 0)
        cq.quant_append(vc, (x * 0.5).to(dev), 0)
        store.append((kc, vc, n))
    q = kv_source(4, (b, hq, 1, d)).to(dev)
    nbytes = max(cq.decode_paged_workspace_bytes(blocks, b, hq, 1),
                 cq.decode_paged_workspace_bytes(others, b, hq, 1))
    ws = torch.zeros(nbytes, dtype=torch.uint8, device=dev)
    out = torch.empty_like(q)
    cq.decode_attention_paged(q, blocks, 0.1, out=out, workspace=ws)
    torch.cuda.synchronize()
    want = out.clone()
    s = torch.cuda.Stream(dev)
    s.wait_stream(torch.cuda.current_stream(dev))
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            cq.decode_attention_paged(q, blocks, 0.1, out=out, workspace=ws)
    torch.cuda.current_stream(dev).wait_stream(s)
    for i in range(4):
        other = cq.decode_attention_paged(q, others, 0.1, workspace=ws)  # rewrites the table
        out.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want), f"replay {i} differs from the eager result"
        assert not torch.equal(other, want)
