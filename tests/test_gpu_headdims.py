"""GPU parity of quantized caches at every head dim the reference's fused path takes (d <= 256,
FA_MAX_HEAD_DIM: candle-nn/src/turbo_quant.rs:1158, candle-core/src/accel/attention.rs:23), the
Dense rotation that RotationKind::Auto / Hadamard resolve to at head dims that are not powers of
two (candle-core/src/accel/config.rs:131-138, turbo.rs:204-230), the score terms of the fused
decode (soft-capping, ALiBi: tq_logit, candle-core/kernels/turbo_quant_impl.h:37-41) and the
dequantization entry (TqDequant / dequantize_rows / keys_values, candle-nn/src/turbo_quant.rs:
250-300, 612-689, 948-966).

Rows: bit for bit against the oracle's encoder of the (rotated) source rows, rotated sides by the
reference's flip criterion (its rotation is an f32 matmul of unpinned summation order).
Attention: against the oracle's restatement of the reference CPU path (dequantize, unrotate,
bf16, unfused f32 attention) on the codes the GPU wrote, by the criterion of rotated caches.
Dequantization: bit for bit (the rotated-domain values are rsc0 * element in f32, the TurboProd
correction and the unrotation sum in index order as the oracle does)."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import (assert_decode_parity, assert_rotated_rows_close, exact_decode,
                           exact_scores, kv_source, obits, oracle_decode, oracle_rows, rotates,
                           side_pi)

pytestmark = pytest.mark.gpu

FMTS = {"fp8": 5, "mxfp4": 2, "turbo4": 0, "nvfp4": 3, "mxfp8": 4, "turboprod": 1}
ROT_DEFAULT, ROT_NONE, ROT_HADAMARD, ROT_DENSE, ROT_AUTO = 0, 1, 2, 3, 4


def valid(fmt: int, d: int) -> bool:
    """QuantFormat::validate (candle-core/src/accel/formats.rs:166-187): whole blocks."""
    return not ((fmt in (2, 4) and d % 32) or (fmt == 3 and d % 16))


def export_np(cq, side, tokens, position=0):
    return cq.rows_export(side, tokens, position).cpu().numpy().view(np.uint32)


def check_rows(f, got, src, seed, rotation, d):
    want = oracle_rows(f, src, seed, rotation)
    if f == 1:
        from tests.helpers import assert_prod_rows_close
        assert_prod_rows_close(got, want, d, 4)
    elif rotates(f, rotation, d) or f == 0:
        assert_rotated_rows_close(f, got, want, d)
    else:
        np.testing.assert_array_equal(got, want)


CASES = [(f, d, rot) for f in ("fp8", "mxfp4", "mxfp8", "nvfp4", "turbo4", "turboprod")
         for d, rot in ((256, ROT_DEFAULT), (96, ROT_DEFAULT), (80, ROT_DEFAULT), (48, ROT_DEFAULT),
                        (96, ROT_DENSE), (128, ROT_DENSE), (256, ROT_HADAMARD))
         if valid(FMTS[f], d)]


@pytest.mark.parametrize("fmt,d,rotation", CASES)
@pytest.mark.parametrize("is_value", [False, True])
def test_append_rows_head_dims(cq, dev, fmt, d, rotation, is_value):
    f = FMTS[fmt]
    if is_value and f == 1:
        pytest.skip("TurboProd is a key format")
    b, h, t, pos = 2, 3, 37, 5
    x = kv_source(100 + d, (b, h, t, d), outliers=True)
    x[0, 0, 0, :] = 0.0
    seed = 44 if is_value else 42
    side = cq.CacheSide.empty(f, is_value, b, h, d, 64, dev, seed=seed, rotation=rotation)
    cq.quant_append(side, x.to(dev), pos)
    torch.cuda.synchronize()
    check_rows(f, export_np(cq, side, t, pos), x, seed, rotation, d)


def run_decode(cq, dev, kf, vf, d, rotation=ROT_DEFAULT, b=2, hq=8, hkv=2, ctx=300, lq=1,
               splits=0, wl=-1, wr=-1, softcap=0.0, alibi=None, seed=0, outliers=True):
    k_fmt, v_fmt = FMTS[kf], FMTS[vf]
    q = kv_source(seed + 1, (b, hq, lq, d))
    k = kv_source(seed + 2, (b, hkv, ctx, d), outliers=outliers)
    v = kv_source(seed + 3, (b, hkv, ctx, d), outliers=outliers)
    cache = cq.TurboKvCache(k_fmt, v_fmt, b, hkv, d, ctx, device=dev, rotation=rotation)
    cache.append(k.to(dev), v.to(dev))
    scale = 1.0 / d ** 0.5
    al = None if alibi is None else torch.tensor(alibi, dtype=torch.float32, device=dev)
    got = cq.decode_attention(q.to(dev), cache.k, cache.v, ctx, scale, window_left=wl,
                              window_right=wr, splits=splits, softcap=softcap, alibi_slopes=al)
    torch.cuda.synchronize()
    kr, vr = export_np(cq, cache.k, ctx), export_np(cq, cache.v, ctx)
    check_rows(k_fmt, kr, k, 42, rotation, d)
    check_rows(v_fmt, vr, v, 44, rotation, d)
    kw = dict(wl=wl, wr=wr, v_fmt=v_fmt, rotation=rotation, softcap=softcap,
              alibi=None if alibi is None else np.array(alibi, np.float32))
    want = oracle_decode(k_fmt, q, kr, vr, ctx, scale, **kw)
    exact = exact_decode(k_fmt, q, kr, vr, ctx, scale, **kw)
    rotated = rotates(k_fmt, rotation, d) or rotates(v_fmt, rotation, d) or exact_scores(k_fmt)
    assert_decode_parity(k_fmt, got.float().cpu().numpy(), want, exact, rotated=rotated,
                         value_bf16=v_fmt != 0)
    return got, cache, q


@pytest.mark.parametrize("fmt", ["fp8", "mxfp4", "mxfp8", "nvfp4", "turbo4"])
@pytest.mark.parametrize("splits", [1, 0])
def test_decode_d256(cq, dev, fmt, splits):
    """Plane rows of 256 (one wavefront per SIMD); TurboQuant with the in-register Hadamard
    transform at 256."""
    run_decode(cq, dev, fmt, fmt, 256, splits=splits, ctx=400)


@pytest.mark.parametrize("kf,vf", [("fp8", "fp8"), ("turbo4", "turbo4"), ("nvfp4", "nvfp4"),
                                   ("mxfp4", "mxfp8"), ("turboprod", "turbo4"),
                                   ("fp8", "turbo4")])
@pytest.mark.parametrize("d", [96, 80])
def test_decode_padded_head_dims(cq, dev, kf, vf, d):
    """Head dims below a plane row length: padded rows of zeros, queries padded, outputs cut;
    TurboQuant sides at these dims take the Dense rotation (Auto), through the matrix path."""
    if not (valid(FMTS[kf], d) and valid(FMTS[vf], d)):
        pytest.skip("the format needs whole blocks")
    run_decode(cq, dev, kf, vf, d, lq=2, wl=100, wr=0)


@pytest.mark.parametrize("fmt", ["fp8", "mxfp4", "nvfp4", "turbo4"])
@pytest.mark.parametrize("d", [128, 96])
def test_decode_dense_rotation(cq, dev, fmt, d):
    """RotationKind::Dense on both sides of any format: q Pi_k^T before the decode, the combined
    rows times Pi_v after it."""
    run_decode(cq, dev, fmt, fmt, d, rotation=ROT_DENSE, splits=3)


def test_decode_d256_turboprod_and_windows(cq, dev):
    run_decode(cq, dev, "turboprod", "turbo4", 256, lq=3, wl=64, wr=0, ctx=257)


@pytest.mark.parametrize("kf,vf", [("fp8", "fp8"), ("turbo4", "turbo4"), ("mxfp4", "mxfp4"),
                                   ("turboprod", "turbo4")])
@pytest.mark.parametrize("terms", ["softcap", "alibi", "both"])
def test_decode_score_terms(cq, dev, kf, vf, terms):
    """Soft-capping and ALiBi of the reference's fused decode (tq_logit: cap tanh(s / cap), then
    - slope |pos - key|) against its CPU path with the same terms. Unit-scale values: ALiBi
    concentrates the weights on the nearest keys, so outlier channels (x8) would put outputs
    above 4, where one bf16 step (0.031) exceeds the 2e-2 bar."""
    hq = 8
    softcap = 2.5 if terms in ("softcap", "both") else 0.0
    alibi = ([0.05 * (i + 1) for i in range(hq)] if terms in ("alibi", "both") else None)
    run_decode(cq, dev, kf, vf, 128, hq=hq, lq=2, softcap=softcap, alibi=alibi, splits=0,
               outliers=False)


def test_decode_alibi_per_batch_slopes(cq, dev):
    """ALiBi slopes per (batch, head): each batch entry against the CPU path with its row."""
    b, hq, hkv, d, ctx = 2, 4, 2, 128, 200
    q = kv_source(11, (b, hq, 1, d))
    k = kv_source(12, (b, hkv, ctx, d))
    v = kv_source(13, (b, hkv, ctx, d))
    cache = cq.TurboKvCache(5, 5, b, hkv, d, ctx, device=dev)
    cache.append(k.to(dev), v.to(dev))
    slopes = np.array([[0.1, 0.2, 0.3, 0.4], [0.05, 0.0, 0.5, 0.25]], np.float32)
    got = cq.decode_attention(q.to(dev), cache.k, cache.v, ctx, 0.1,
                              alibi_slopes=torch.tensor(slopes, device=dev)).float().cpu().numpy()
    kr, vr = export_np(cq, cache.k, ctx), export_np(cq, cache.v, ctx)
    for bi in range(b):
        want = oracle_decode(5, q[bi:bi + 1], kr[bi:bi + 1], vr[bi:bi + 1], ctx, 0.1,
                             alibi=slopes[bi])
        err = np.abs(got[bi:bi + 1] - want)
        assert err.max() <= 2e-2 and err.mean() <= 2e-3, (bi, err.max())


@pytest.mark.parametrize("fmt", ["fp8", "turbo4"])
@pytest.mark.parametrize("d", [256, 96])
def test_paged_equals_dense_head_dims(cq, dev, fmt, d):
    f = FMTS[fmt]
    b, hq, hkv, ctx = 2, 4, 2, 230
    q = kv_source(5, (b, hq, 1, d)).to(dev)
    k = kv_source(6, (b, hkv, ctx, d)).to(dev)
    v = kv_source(7, (b, hkv, ctx, d)).to(dev)
    dense = cq.TurboKvCache(f, f, b, hkv, d, ctx, device=dev)
    dense.append(k, v)
    blocks = []
    for lo, hi in ((0, 100), (100, 101), (101, 230)):
        c = cq.TurboKvCache(f, f, b, hkv, d, 128, device=dev)
        c.append(k[:, :, lo:hi], v[:, :, lo:hi])
        blocks.append((c.k, c.v, hi - lo))
    # f32 outputs: the kernels' difference, not a bf16 rounding of the output
    o1 = torch.empty((b, hq, 1, d), dtype=torch.float32, device=dev)
    o2 = torch.empty_like(o1)
    want = cq.decode_attention(q, dense.k, dense.v, ctx, 0.1, splits=1, out=o1)
    got = cq.decode_attention_paged(q, blocks, 0.1, out=o2)
    torch.cuda.synchronize()
    tol = 1e-5 if f != 0 else 2e-3  # TurboQuant: one f16 rounding of P per split point
    assert (got - want).abs().max().item() <= tol


# ---------------------------------------------------------------------------------------------
# dequantization
# ---------------------------------------------------------------------------------------------
DQ = [(f, d) for f in ("fp8", "mxfp4", "mxfp8", "nvfp4", "turbo4", "turboprod")
      for d in (128, 64, 256, 96, 80) if valid(FMTS[f], d)]


@pytest.mark.parametrize("fmt,d", DQ)
@pytest.mark.parametrize("is_value", [False, True])
def test_dequantize_bit_exact(cq, dev, fmt, d, is_value):
    """cqkv_dequantize_rows against the oracle's dequantize_row (RowCodec::dequantize_row,
    candle-core/src/accel/turbo.rs:398-424) of the exported rows, bit for bit: rotated-domain
    values (unrotate off), then y Pi (unrotate on), then the bf16 cast of keys_values."""
    f = FMTS[fmt]
    if is_value and f == 1:
        pytest.skip("TurboProd is a key format")
    b, h, t, pos = 2, 3, 45, 3
    seed = 44 if is_value else 42
    x = kv_source(200 + d, (b, h, t + pos, d), outliers=True)
    side = cq.CacheSide.empty(f, is_value, b, h, d, 64, dev, seed=seed)
    cq.quant_append(side, x.to(dev), 0)
    rows = export_np(cq, side, t, pos)
    got = cq.dequantize(side, t, pos, unrotate=False).cpu().numpy()
    if f == 1:
        want = O.dequantize_rows_qjl(obits(1), d, rows, O.qjl_matrix(d, seed))
    else:
        want = O.dequantize_rows(f, obits(f), d, rows)
    np.testing.assert_array_equal(got, want)
    pi = side_pi(f, ROT_DEFAULT, d, seed)
    got_u = cq.dequantize(side, t, pos, unrotate=True).cpu().numpy()
    want_u = want if pi is None else O.unrotate_rows(pi, want.reshape(-1, d)).reshape(want.shape)
    np.testing.assert_array_equal(got_u, want_u)
    got_b = cq.dequantize(side, t, pos, dtype=torch.bfloat16).float().cpu().numpy()
    np.testing.assert_array_equal(got_b, O.round_bf16(want_u))


def test_keys_values_matches_decode_inputs(cq, dev):
    """TurboKvCache::keys_values: the dequantized, unrotated cache; attention over it (the
    reference's non-fused path) agrees with the fused decode."""
    b, hq, hkv, d, ctx = 1, 8, 2, 96, 150
    k = kv_source(31, (b, hkv, ctx, d)).to(dev)
    v = kv_source(32, (b, hkv, ctx, d)).to(dev)
    q = kv_source(33, (b, hq, 1, d)).to(dev)
    cache = cq.TurboKvCache(0, 0, b, hkv, d, ctx, device=dev)  # TurboQuant-4, Dense (Auto)
    cache.append(k, v)
    kv = cache.keys_values(torch.bfloat16)
    assert kv[0].shape == (b, hkv, ctx, d) and kv[0].dtype == torch.bfloat16
    kf, vf = kv[0].float().repeat_interleave(hq // hkv, 1), kv[1].float().repeat_interleave(hq // hkv, 1)
    s = (q.float() @ kf.transpose(-1, -2)) / d ** 0.5
    want = torch.softmax(s, -1) @ vf
    got = cache.attention(q, 1.0 / d ** 0.5).float()
    assert (got - want).abs().max().item() <= 3e-2


@pytest.mark.parametrize("fmt,d", [("fp8", 96), ("nvfp4", 80), ("turbo4", 80), ("mxfp4", 256),
                                   ("turboprod", 96), ("turbo4", 256)])
def test_import_export_round_trip_head_dims(cq, dev, fmt, d):
    """Reference rows of d elements to padded plane rows and back, bit for bit; the imported
    cache decodes like the one appended directly."""
    f = FMTS[fmt]
    b, h, t = 2, 2, 40
    src = cq.CacheSide.empty(f, False, b, h, d, 64, dev, seed=42)
    cq.quant_append(src, kv_source(9, (b, h, t, d)).to(dev), 0)
    rows = cq.rows_export(src, t)
    dst = cq.CacheSide.empty(f, False, b, h, d, 64, dev, seed=42)
    cq.rows_import(dst, rows)
    np.testing.assert_array_equal(export_np(cq, dst, t), rows.cpu().numpy().view(np.uint32))
    assert torch.equal(dst.codes, src.codes) and torch.equal(dst.scales, src.scales)


@pytest.mark.parametrize("d,kind", [(256, 1), (96, 1), (96, 2)])
def test_rope_append_head_dims(cq, dev, d, kind):
    """The fused RoPE + append at plane rows of 256 and padded head dims (separate launches):
    rotated queries against the oracle's rope, cache rows against the plain append of the
    oracle's rotated keys."""
    b, hq, hkv, t, pos = 2, 4, 2, 20, 3
    q = kv_source(41, (b, hq, t, d))
    k = kv_source(42, (b, hkv, t, d))
    v = kv_source(43, (b, hkv, t, d))
    ang = torch.arange(64)[:, None].float() * (1.0 / 10000 ** (torch.arange(d // 2).float() / (d // 2)))
    cos, sin = torch.cos(ang).to(torch.bfloat16), torch.sin(ang).to(torch.bfloat16)
    cache = cq.TurboKvCache(0, 5, b, hkv, d, 64, device=dev)
    cache._len = pos
    qo = cache.rope_append(q.to(dev), k.to(dev), v.to(dev), cos.to(dev), sin.to(dev), kind)
    torch.cuda.synchronize()
    qr = O.rope(q.float().numpy(), cos.float().numpy(), sin.float().numpy(), kind, pos)
    np.testing.assert_array_equal(qo.float().cpu().numpy(), O.round_bf16(qr))
    kr = torch.tensor(O.round_bf16(O.rope(k.float().numpy(), cos.float().numpy(),
                                          sin.float().numpy(), kind, pos))).to(torch.bfloat16)
    ref = cq.TurboKvCache(0, 5, b, hkv, d, 64, device=dev)
    ref._len = pos
    ref.append(kr.to(dev), v.to(dev))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(export_np(cq, cache.k, t, pos), export_np(cq, ref.k, t, pos))
    np.testing.assert_array_equal(export_np(cq, cache.v, t, pos), export_np(cq, ref.v, t, pos))
