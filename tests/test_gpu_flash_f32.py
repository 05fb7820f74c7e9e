"""GPU parity of the f32-query flash attention (csrc/flash_f32.h): f32 q / out over f32, f16,
bf16 and E4M3 K / V, the dtype pairs of the reference's kv_dtype_supported
(candle-core/src/accel/attention.rs:569-576) and kernels fa_row_f32_* / fa{2,3}_d*_f32_*
(candle-core/kernels/flash_attn_impl.h:49-443).

The bars are the reference's own for f32 queries (candle-nn/tests/accel_rocm.rs:667-840):
  * against the CPU path on the same K / V (the oracle's restatement of flash_attn.rs:930-1000
    in f32), rel = max |err| / max |ref| <= 1e-5, and the same against float64 attention;
  * f16 / bf16 K / V give exactly the bits of the f32 kernel on the widened K / V, and differ
    from f32 attention of the unrounded K / V by the storage rounding only: <= 1e-3 (f16),
    <= 1e-2 (bf16);
  * another key split of the same call (the paged form against the dense one): <= 4e-6."""
import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu

KV = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}
E4M3 = np.array([O.e4m3_to_f32(c) for c in range(256)], dtype=np.float32)


def randn(seed, shape, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g) * scale


def rel(got, ref):
    return float(np.abs(np.asarray(got, np.float64) - ref).max() / np.abs(ref).max())


def exact(q, k, v, scale, wl=-1, wr=-1, softcap=0.0, slopes=None):
    """float64 attention, q (b, hq, lq, d), k / v (b, hkv, lk, d) -> (b, hq, lq, d)."""
    q, k, v = (np.asarray(t, np.float64) for t in (q, k, v))
    b, hq, lq, d = q.shape
    hkv, lk = k.shape[1], k.shape[2]
    g = hq // hkv
    out = np.zeros(q.shape)
    for h in range(hq):
        s = np.einsum("bqd,bkd->bqk", q[:, h], k[:, h // g]) * scale
        if softcap > 0:
            s = softcap * np.tanh(s / softcap)
        for i in range(lq):
            lo, hi = O.key_range(i, lq, lk, wl, wr)
            if slopes is not None:
                pos = i + lk - lq
                s[:, i] -= np.asarray(slopes, np.float64)[..., h].reshape(-1, 1) * \
                    np.abs(pos - np.arange(lk))
            s[:, i, :lo] = -np.inf
            s[:, i, hi:] = -np.inf
        m = s.max(-1, keepdims=True)
        p = np.where(np.isfinite(s), np.exp(s - np.where(np.isfinite(m), m, 0)), 0.0)
        den = p.sum(-1, keepdims=True)
        out[:, h] = np.einsum("bqk,bkd->bqd", p, v[:, h // g]) / np.where(den > 0, den, 1)
    return out


def bhsd(t):
    return t.permute(0, 2, 1, 3).contiguous()


def run_dense(cq, dev, q, k, v, scale, **kw):
    """q (b, hq, lq, d) f32, k / v (b, hkv, lk, d) of any dtype -> out (b, hq, lq, d) f32."""
    out = cq.flash_attn(bhsd(q).to(dev), bhsd(k).to(dev), bhsd(v).to(dev), scale, **kw)
    torch.cuda.synchronize()
    assert out.dtype == torch.float32
    return bhsd(out).cpu().numpy()


@pytest.mark.parametrize("kvd", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("hq,hkv,d,lk", [(16, 4, 256, 1500), (16, 8, 128, 700), (32, 2, 64, 300),
                                         (12, 4, 128, 200)])
@pytest.mark.parametrize("lq", [1, 3, 37])
def test_f32_queries_vs_cpu(cq, dev, kvd, hq, hkv, d, lk, lq):
    """The reference's GQA cases (accel_rocm.rs:679-693): decode (row kernel, split-K) and 37
    queries (column kernel), non-causal, against the CPU path on the same K / V."""
    seed = 7 * d + lk + lq
    q = randn(seed, (1, hq, lq, d))
    k = randn(seed + 1, (1, hkv, lk, d)).to(KV[kvd])
    v = randn(seed + 2, (1, hkv, lk, d)).to(KV[kvd])
    scale = 1.0 / d ** 0.5
    got = run_dense(cq, dev, q, k, v, scale, causal=False)
    kf, vf = k.float().numpy(), v.float().numpy()
    want = O.attention_unfused(q.numpy(), kf, vf, scale, threads=16)
    assert rel(got, want) <= 1e-5
    assert rel(got, exact(q.numpy(), kf, vf, scale)) <= 1e-5


@pytest.mark.parametrize("hq,hkv,d,lk", [(16, 4, 256, 1100), (16, 8, 128, 900), (8, 2, 64, 700),
                                         (8, 2, 80, 500)])
@pytest.mark.parametrize("lq", [1, 4, 37])
def test_half_kv_equals_widened(cq, dev, hq, hkv, d, lk, lq):
    """half_kv_with_f32_queries (accel_rocm.rs:780-841): f16 / bf16 K / V have the bits of the
    f32 kernel on the widened K / V, and stay within the storage rounding of f32 attention on
    the unrounded K / V."""
    seed = 2000 + d + lk
    k, v = randn(seed, (1, hkv, lk, d)), randn(seed + 1, (1, hkv, lk, d))
    q = randn(seed + 10 + lq, (1, hq, lq, d))
    scale = 1.0 / d ** 0.5
    full = exact(q.numpy(), k.numpy(), v.numpy(), scale, wr=0)
    for kvd, tol in (("f16", 1e-3), ("bf16", 1e-2)):
        kh, vh = k.to(KV[kvd]), v.to(KV[kvd])
        got = run_dense(cq, dev, q, kh, vh, scale, causal=True)
        widened = run_dense(cq, dev, q, kh.float(), vh.float(), scale, causal=True)
        np.testing.assert_array_equal(got, widened)
        same = O.attention_unfused(q.numpy(), kh.float().numpy(), vh.float().numpy(), scale,
                                   wr=0, threads=16)
        assert rel(got, same) <= 1e-5
        assert rel(got, full) <= tol


@pytest.mark.parametrize("kvd", ["f32", "bf16"])
@pytest.mark.parametrize("sq,sk,wl,wr", [(200, 200, -1, 0), (64, 900, 100, 0), (1, 3000, -1, 0),
                                         (5, 40, -1, 0), (40, 300, 20, 3)])
def test_f32_masks(cq, dev, kvd, sq, sk, wl, wr):
    """Causal prefill (column kernel), sliding windows, fewer keys than queries (rows that see
    no key are zero), bottom-right aligned as in the reference."""
    b, hq, hkv, d = 2, 8, 2, 128
    q = randn(31 + sq, (b, hq, sq, d))
    k = randn(32 + sk, (b, hkv, sk, d)).to(KV[kvd])
    v = randn(33 + sk, (b, hkv, sk, d)).to(KV[kvd])
    scale = 1.0 / d ** 0.5
    got = run_dense(cq, dev, q, k, v, scale, causal=False, window_left=wl, window_right=wr)
    want = exact(q.numpy(), k.float().numpy(), v.float().numpy(), scale, wl=wl, wr=wr)
    assert rel(got, want) <= 1e-5
    if sq > sk and wr == 0:
        assert (got[:, :, :sq - sk] == 0).all()


@pytest.mark.parametrize("per_batch", [False, True])
def test_f32_softcap_alibi(cq, dev, per_batch):
    b, hq, hkv, d, sq, sk = 2, 8, 4, 64, 50, 400
    q = randn(41, (b, hq, sq, d), 2.0)
    k, v = randn(42, (b, hkv, sk, d)), randn(43, (b, hkv, sk, d))
    slopes = torch.rand(b, hq) if per_batch else torch.rand(hq)
    scale = 1.0 / d ** 0.5
    got = run_dense(cq, dev, q, k, v, scale, causal=True, softcap=5.0,
                    alibi_slopes=slopes.to(dev))
    al = slopes.numpy()[:, None, :] if per_batch else slopes.numpy()
    want = exact(q.numpy(), k.numpy(), v.numpy(), scale, wr=0, softcap=5.0,
                 slopes=al.reshape(b, hq) if per_batch else al)
    assert rel(got, want) <= 1e-5


def test_f32_varlen(cq, dev):
    hq, hkv, d = 8, 2, 128
    lens_q, lens_k = [3, 70, 1, 20], [100, 70, 500, 20]
    qs = [randn(50 + i, (n, hq, d)) for i, n in enumerate(lens_q)]
    ks = [randn(60 + i, (n, hkv, d)).half() for i, n in enumerate(lens_k)]
    vs = [randn(70 + i, (n, hkv, d)).half() for i, n in enumerate(lens_k)]
    cu = lambda ls: torch.tensor(np.concatenate([[0], np.cumsum(ls)]), dtype=torch.int32).to(dev)
    scale = 0.1
    got = cq.flash_attn_varlen(torch.cat(qs).to(dev), torch.cat(ks).to(dev), torch.cat(vs).to(dev),
                               cu(lens_q), cu(lens_k), max(lens_q), max(lens_k), scale, True)
    torch.cuda.synchronize()
    got = got.cpu().numpy()
    off = 0
    for qq, kk, vv in zip(qs, ks, vs):
        n = qq.shape[0]
        want = exact(bhsd(qq[None]).numpy(), bhsd(kk[None].float()).numpy(),
                     bhsd(vv[None].float()).numpy(), scale, wr=0)
        assert rel(bhsd(torch.from_numpy(got[None, off:off + n])).numpy(), want) <= 1e-5
        off += n


@pytest.mark.parametrize("kvd", ["f32", "f16"])
@pytest.mark.parametrize("lq", [1, 20])
def test_f32_blocks_equal_dense(cq, dev, kvd, lq):
    """The paged form over blocks (another key split than the dense call) within 4e-6, and the
    CPU path over the concatenated rows within 1e-5."""
    b, hq, hkv, d = 2, 16, 4, 128
    rows, caps = (300, 150, 70, 0, 513), (320, 160, 96, 32, 544)
    blocks, kk, vv = [], [], []
    for i, (n, c) in enumerate(zip(rows, caps)):
        k = randn(80 + i, (b, hkv, c, d)).to(KV[kvd])
        v = randn(90 + i, (b, hkv, c, d)).to(KV[kvd])
        blocks.append((k.to(dev), v.to(dev), n))
        kk.append(k[:, :, :n])
        vv.append(v[:, :, :n])
    q = randn(99, (b, hq, lq, d))
    scale = 1.0 / d ** 0.5
    got = cq.flash_attn_blocks(q.to(dev), blocks, scale, window_right=0)
    torch.cuda.synchronize()
    got = got.cpu().numpy()
    k, v = torch.cat(kk, 2), torch.cat(vv, 2)
    dense = run_dense(cq, dev, q, k, v, scale, causal=True)
    assert rel(got, dense) <= 4e-6
    want = exact(q.numpy(), k.float().numpy(), v.float().numpy(), scale, wr=0)
    assert rel(got, want) <= 1e-5


@pytest.mark.parametrize("lq,d", [(1, 128), (3, 256), (64, 128), (40, 80)])
def test_f32_queries_fp8_kv(cq, dev, lq, d):
    """E4M3 K / V with f32 queries (fa_row_f32_fp8): the codes widened exactly, times the
    descales (host factors and device scales), f32 math."""
    b, hq, hkv, lk = 2, 8, 2, 700
    q = randn(101, (b, hq, lq, d))
    k8 = torch.from_numpy(O.e4m3_encode(randn(102, (b, hkv, lk, d)).numpy() * 30))
    v8 = torch.from_numpy(O.e4m3_encode(randn(103, (b, hkv, lk, d)).numpy() * 30))
    kd, vd = 1.0 / 30, 1.0 / 25
    ks = torch.tensor([0.5, 0.0], device=dev)
    vs = torch.tensor([2.0, 0.0], device=dev)
    scale = 1.0 / d ** 0.5
    got = cq.flash_attn_fp8_codes(bhsd(q).to(dev), bhsd(k8).to(dev), bhsd(v8).to(dev), scale, True,
                                  kd, vd, k_scale=ks, v_scale=vs)
    torch.cuda.synchronize()
    assert got.dtype == torch.float32
    got = bhsd(got).cpu().numpy()
    kf = E4M3[k8.numpy()].astype(np.float64) * (np.float32(kd) * 0.5)
    vf = E4M3[v8.numpy()].astype(np.float64) * (np.float32(vd) * 2.0)
    assert rel(got, exact(q.numpy(), kf, vf, scale, wr=0)) <= 1e-5
    # a caller workspace of the query's size gives the same bits (no staging with f32 queries)
    n = cq.flash_attn_fp8_workspace_bytes(torch.float32, b, lq, lk, hq, hkv, d)
    ws = torch.zeros(max(n, 256), dtype=torch.uint8, device=dev)
    again = cq.flash_attn_fp8_codes(bhsd(q).to(dev), bhsd(k8).to(dev), bhsd(v8).to(dev), scale,
                                    True, kd, vd, k_scale=ks, v_scale=vs, workspace=ws)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bhsd(again).cpu().numpy(), got)


def test_f32_queries_with_cache_append(cq, dev):
    """f32 queries over f16 K / V that are also appended to an FP8 / MXFP4 cache in the same call:
    the cache rows equal a plain append of the same f16 rows."""
    b, hq, hkv, d, s = 2, 8, 2, 128, 96
    q = randn(111, (b, s, hq, d)).to(dev)
    k, v = randn(112, (b, s, hkv, d)).half().to(dev), randn(113, (b, s, hkv, d)).half().to(dev)
    kc = cq.CacheSide.empty(cq.FP8, False, b, hkv, d, 128, dev)
    vc = cq.CacheSide.empty(cq.MXFP4, True, b, hkv, d, 128, dev)
    out = cq.flash_attn(q, k, v, 0.1, True, k_cache=kc, v_cache=vc, position=8)
    kr = cq.CacheSide.empty(cq.FP8, False, b, hkv, d, 128, dev)
    vr = cq.CacheSide.empty(cq.MXFP4, True, b, hkv, d, 128, dev)
    cq.quant_append(kr, k.permute(0, 2, 1, 3), 8)
    cq.quant_append(vr, v.permute(0, 2, 1, 3), 8)
    torch.cuda.synchronize()
    for a, r in ((kc, kr), (vc, vr)):
        assert torch.equal(a.codes, r.codes) and torch.equal(a.scales, r.scales)
    want = cq.flash_attn(q, k.float(), v.float(), 0.1, True)
    torch.cuda.synchronize()
    assert torch.equal(out, want)


def test_f32_refusals(cq, dev):
    q = torch.zeros(1, 4, 8, 64, device=dev)
    kh = torch.zeros(1, 4, 2, 64, dtype=torch.float16, device=dev)
    with pytest.raises(cq.CqkvError):  # f16 queries over f32 K / V
        cq.flash_attn(q.half(), kh.float(), kh.float(), 0.1, True)
    with pytest.raises(cq.CqkvError):  # K and V of different dtypes
        cq.flash_attn(q, kh, kh.bfloat16(), 0.1, True)
    with pytest.raises(cq.CqkvError):  # bf16 queries over f16 K / V
        cq.flash_attn(q.bfloat16(), kh, kh, 0.1, True)
