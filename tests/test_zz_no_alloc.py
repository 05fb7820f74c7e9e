"""cqkv_decode_attention_noalloc (no allocation: split partials in the library's per-GPU device
scratch array) against cqkv_decode_attention (partials in a workspace), through the C ABI.

Both run the same kernels over the same split count, so their outputs must be equal bit for bit.
Two calls in a row, the second smaller, show that the array's leftover contents from one call do
not leak into the next; a third case lowers the automatic split count to fit the array, and an
explicit split count that does not fit is refused."""
import ctypes

import numpy as np
import pytest
import torch

from tests.helpers import kv_source

pytestmark = pytest.mark.gpu


def make_cache(cq, dev, fmt, b, hkv, d, cap, n, seed):
    cache = cq.TurboKvCache(fmt, fmt, b, hkv, d, cap, device=dev)
    cache.append(kv_source(seed, (b, hkv, n, d), outliers=True).to(dev),
                 kv_source(seed + 1, (b, hkv, n, d), outliers=True).to(dev))
    return cache


def both(cq, q, cache, kv_len, kv_lens=None, splits=0, wl=-1, wr=-1):
    scale = 1.0 / q.shape[-1] ** 0.5
    want = cq.decode_attention(q, cache.k, cache.v, kv_len, scale, kv_lens=kv_lens, splits=splits,
                               window_left=wl, window_right=wr)
    got = torch.full_like(q, float("nan"))
    cq.decode_attention_noalloc(q, cache.k, cache.v, kv_len, scale, kv_lens=kv_lens,
                                window_left=wl, window_right=wr, out=got, splits=splits)
    torch.cuda.synchronize()
    return got, want


@pytest.mark.parametrize("fmt", [5, 0])  # FP8, TurboQuant-4 (combine with unrotation)
def test_noalloc_matches_workspace_entry_point_two_calls(cq, dev, fmt):
    # call 1: ragged lengths, automatic splits (> 1: the scratch array holds the partials)
    b, hq, hkv, d, cap = 8, 32, 8, 128, 4096
    c1 = make_cache(cq, dev, fmt, b, hkv, d, cap, cap, 11)
    lens = torch.tensor([4096, 1, 700, 3000, 33, 4095, 2048, 1500], dtype=torch.int32, device=dev)
    assert cq.decode_splits(b, hkv, cap, fmt, ragged=True) > 1
    q1 = kv_source(3, (b, hq, 1, d)).to(dev)
    got1, want1 = both(cq, q1, c1, cap, kv_lens=lens)
    assert torch.equal(got1, want1)
    # call 2: a smaller input (fewer rows, D = 64, two queries, a window, explicit splits)
    b2, hq2, hkv2, d2, cap2 = 2, 8, 2, 64, 704
    c2 = make_cache(cq, dev, fmt, b2, hkv2, d2, cap2, 700, 21)
    q2 = kv_source(4, (b2, hq2, 2, d2)).to(dev)
    got2, want2 = both(cq, q2, c2, 700, splits=5, wl=300, wr=0)
    assert torch.equal(got2, want2)
    assert torch.isfinite(got2).all()


def test_noalloc_lowers_automatic_splits_and_refuses_explicit_ones(cq, dev):
    """4096 query rows (B=64, 32 heads, 2 queries): each split's partials take 2,113,536 bytes, so
    at most 15 fit the 32 MiB array. The ragged split rule asks 16 for a 65,536-key capacity; the
    call lowers that to 15 (the same result as the workspace entry point with 15 splits), and an
    explicit 16 is refused."""
    b, hq, hkv, d, cap = 64, 32, 8, 128, 65536
    cache = cq.TurboKvCache(5, 5, b, hkv, d, cap, device=dev)  # zero codes past the first rows
    n = 320
    cq.quant_append(cache.k, kv_source(31, (b, hkv, n, d)).to(dev), 0)
    cq.quant_append(cache.v, kv_source(32, (b, hkv, n, d)).to(dev), 0)
    lens = torch.from_numpy(np.random.default_rng(5).integers(1, n + 1, b).astype(np.int32)).to(dev)
    assert cq.decode_splits(b, hkv, cap, 5, ragged=True) == 16
    per_split = 4096 * d * 4 + 4096 * 4
    assert 15 * per_split <= cq.DECODE_SCRATCH_BYTES < 16 * per_split
    q = kv_source(6, (b, hq, 2, d)).to(dev)
    scale = 1.0 / d ** 0.5
    want = cq.decode_attention(q, cache.k, cache.v, cap, scale, kv_lens=lens, splits=15)
    got = torch.full_like(q, float("nan"))
    cq.decode_attention_noalloc(q, cache.k, cache.v, cap, scale, kv_lens=lens, out=got)
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    with pytest.raises(cq.CqkvError) as e:
        cq.decode_attention_noalloc(q, cache.k, cache.v, cap, scale, kv_lens=lens, out=got,
                                    splits=16)
    assert e.value.code == cq.ERR_WORKSPACE and "scratch" in str(e.value)


def _pool_growth(dev, fn) -> int:
    """Bytes the device's default memory pool (the one hipMallocAsync draws from) rose above its
    level before fn(): the used-memory high-water mark, reset to the current use first
    (hipMemPoolAttrUsedMemHigh = 8, hipMemPoolAttrUsedMemCurrent = 7)."""
    hip = ctypes.CDLL("libamdhip64.so")
    pool = ctypes.c_void_p()
    assert hip.hipDeviceGetDefaultMemPool(ctypes.byref(pool), dev.index or 0) == 0
    zero, cur, high = ctypes.c_uint64(0), ctypes.c_uint64(0), ctypes.c_uint64(0)
    torch.cuda.synchronize()
    assert hip.hipMemPoolSetAttribute(pool, 8, ctypes.byref(zero)) == 0
    assert hip.hipMemPoolGetAttribute(pool, 7, ctypes.byref(cur)) == 0
    fn()
    torch.cuda.synchronize()
    assert hip.hipMemPoolGetAttribute(pool, 8, ctypes.byref(high)) == 0
    return high.value - cur.value


def test_noalloc_allocates_nothing(cq, dev):
    """The allocation-free entry point takes nothing from the stream-ordered pool, where the
    workspace-free cqkv_decode_attention call of the same split count does (the control)."""
    b, hq, hkv, d, cap = 4, 32, 8, 128, 2048
    cache = make_cache(cq, dev, 0, b, hkv, d, cap, cap, 41)  # TurboQuant-4: partials + combine
    q = kv_source(7, (b, hq, 1, d)).to(dev)
    out = torch.empty_like(q)
    scale = 1.0 / d ** 0.5
    assert _pool_growth(dev, lambda: cq.decode_attention(q, cache.k, cache.v, cap, scale, out=out,
                                                         splits=4)) > 0
    assert _pool_growth(dev, lambda: cq.decode_attention_noalloc(q, cache.k, cache.v, cap, scale,
                                                                 out=out, splits=4)) == 0
