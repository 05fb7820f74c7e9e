"""HIP-graph capture of the entry points a serving loop replays: every call below is captured with
a caller workspace (so nothing is allocated while capturing), then replayed several times with
eager calls between the replays that rewrite the same workspace and outputs; every replay must
equal the eager result bit for bit. The library records no memset nodes (it clears and fills
through kernels) and keeps every per-call table in kernel arguments, which a graph captures by
value."""
import pytest
import torch

from tests.helpers import kv_source

pytestmark = pytest.mark.gpu


def replays_match(dev, call, outs, disturb, n=3, kept=()):
    """outs: cleared before each replay and compared after it; kept: compared only (state the
    replays rewrite with the same values, e.g. cache rows)."""
    call()
    torch.cuda.synchronize()
    want = [o.clone() for o in outs]
    want_kept = [o.clone() for o in kept]
    s = torch.cuda.Stream(dev)
    s.wait_stream(torch.cuda.current_stream(dev))
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            call()
    torch.cuda.current_stream(dev).wait_stream(s)
    for i in range(n):
        disturb()
        for o in outs:
            o.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for o, w in zip(list(outs) + list(kept), want + want_kept):
            assert torch.equal(o, w), f"replay {i} differs from the eager result"


def randn(seed, shape, dtype=torch.bfloat16, dev="cuda"):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g).to(dtype).to(dev)


@pytest.mark.parametrize("dtype,d,sq,sk", [(torch.bfloat16, 128, 200, 200),  # MFMA prefill
                                           (torch.float16, 64, 100, 900),    # tile kernel
                                           (torch.bfloat16, 128, 1, 3000),   # row kernel, splits
                                           (torch.float32, 64, 100, 900),    # f32, column mode
                                           (torch.float32, 128, 1, 3000)])   # f32 rows, splits
def test_flash_attn_capture(cq, dev, dtype, d, sq, sk):
    b, hq, hkv = 2, 8, 2
    q, k, v = (randn(i, s, dtype, dev) for i, s in
               ((1, (b, sq, hq, d)), (2, (b, sk, hkv, d)), (3, (b, sk, hkv, d))))
    q2 = randn(4, (b, sq, hq, d), dtype, dev)
    n = cq.flash_attn_workspace_bytes(dtype, b, sq, sk, hq, hkv, d)
    ws = torch.zeros(max(n, 256), dtype=torch.uint8, device=dev)
    out, out2 = torch.empty_like(q), torch.empty_like(q)
    replays_match(dev, lambda: cq.flash_attn(q, k, v, d ** -0.5, True, out=out, workspace=ws),
                  [out], lambda: cq.flash_attn(q2, k, v, d ** -0.5, True, out=out2, workspace=ws))


def test_flash_attn_blocks_capture(cq, dev):
    b, hkv, d, hq = 2, 2, 128, 8
    blocks = []
    for i, (rows, cap) in enumerate(((300, 320), (150, 160), (70, 96))):
        blocks.append((randn(10 + i, (b, hkv, cap, d), dev=dev),
                       randn(20 + i, (b, hkv, cap, d), dev=dev), rows))
    q = randn(5, (b, hq, 1, d), dev=dev)
    q2 = randn(6, (b, hq, 1, d), dev=dev)
    ws = torch.zeros(16 << 20, dtype=torch.uint8, device=dev)
    out, out2 = torch.empty_like(q), torch.empty_like(q)
    replays_match(dev, lambda: cq.flash_attn_blocks(q, blocks, 0.1, out=out, workspace=ws),
                  [out], lambda: cq.flash_attn_blocks(q2, blocks[:2], 0.1, out=out2, workspace=ws))


def test_decode_and_append_capture(cq, dev):
    """A decode step as a serving loop captures it: the new token's K / V appended (TurboQuant-4
    keys, MXFP4 values), then the split-K decode over the cache (rotated values: the combine
    runs)."""
    b, hq, hkv, d, ctx = 4, 16, 4, 128, 2000
    cache = cq.TurboKvCache(cq.TURBO4, cq.MXFP4, b, hkv, d, ctx + 32, device=dev)
    cache.append(kv_source(1, (b, hkv, ctx, d)).to(dev), kv_source(2, (b, hkv, ctx, d)).to(dev))
    kn, vn = kv_source(3, (b, hkv, 1, d)).to(dev), kv_source(4, (b, hkv, 1, d)).to(dev)
    q = kv_source(5, (b, hq, 1, d)).to(dev)
    splits = cq.decode_splits(b, hkv, ctx + 1, cq.TURBO4, v_fmt=cq.MXFP4)
    ws = torch.zeros(cq.decode_workspace_bytes(b, hq, 1, d, max(splits, 1)), dtype=torch.uint8,
                     device=dev)
    out = torch.empty_like(q)
    q2, out2 = kv_source(6, (b, hq, 1, d)).to(dev), torch.empty_like(q)

    def step():
        cq.quant_append(cache.k, kn, ctx)
        cq.quant_append(cache.v, vn, ctx)
        cq.decode_attention(q, cache.k, cache.v, ctx + 1, 0.1, out=out, workspace=ws)
    replays_match(dev, step, [out],
                  lambda: cq.decode_attention(q2, cache.k, cache.v, ctx + 1, 0.1, out=out2,
                                              workspace=ws),
                  kept=[cache.k.codes, cache.k.scales, cache.v.codes, cache.v.scales])


def test_flash_attn_fp8_capture(cq, dev):
    from oracle import oracle as O
    b, sq, sk, hq, hkv, d = 2, 64, 500, 8, 2, 128
    q = randn(7, (b, sq, hq, d), dev=dev)
    q2 = randn(8, (b, sq, hq, d), dev=dev)
    k8 = torch.from_numpy(O.e4m3_encode(randn(9, (b, sk, hkv, d), dev="cpu").float().numpy()
                                        * 30)).to(dev)
    v8 = torch.from_numpy(O.e4m3_encode(randn(10, (b, sk, hkv, d), dev="cpu").float().numpy()
                                        * 30)).to(dev)
    ws = torch.zeros(cq.flash_attn_fp8_workspace_bytes(torch.bfloat16, b, sq, sk, hq, hkv, d),
                     dtype=torch.uint8, device=dev)
    out, out2 = torch.empty_like(q), torch.empty_like(q)
    call = lambda qq, oo: cq.flash_attn_fp8_codes(qq, k8, v8, d ** -0.5, True, 1 / 30, 1 / 30,
                                                  out=oo, workspace=ws)
    replays_match(dev, lambda: call(q, out), [out], lambda: call(q2, out2))
