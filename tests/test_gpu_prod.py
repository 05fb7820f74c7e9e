"""GPU parity of TurboProd (QJL) keys, QuantFormat::TurboProd{bits: 4} (3-bit MSE codes of the
rotated unit row, the sign bits of S r and |r|; candle-core/src/accel/turbo.rs:236-239, 299-323,
401-424), and of the fused decode over them (turbo_quant_impl.h:259-279: score =
r0 (q . c + r1 sqrt(pi / 2) / D (S q) . z)).

Rows: against the oracle's RowCodec restatement (itself pinned to the reference's tq_quant /
tq_signs kernels, tests/test_oracle.py) by helpers.assert_prod_rows_close. Decode: against the
reference's fused kernel fixture (tests/golden/ref_prod4.npz) and against the reference CPU path
on the codes the GPU wrote, by the criterion of rotated caches."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import (assert_close_bf16, assert_decode_parity, assert_prod_rows_close,
                           exact_decode, kv_source, oracle_decode, oracle_rows)
from tests.test_oracle import prod_inputs

pytestmark = pytest.mark.gpu

PROD, TURBO4, FP8, MXFP4, NVFP4, MXFP8 = 1, 0, 5, 2, 3, 4


def export_np(cq, side, tokens, position=0):
    return cq.rows_export(side, tokens, position).cpu().numpy().view(np.uint32)


def test_qjl_matrix_matches_oracle(cq):
    """The library's host S (cqkv_qjl_matrix) is the oracle's qjl_matrix bit for bit."""
    for d, seed in ((64, 42), (128, 42), (128, 7)):
        np.testing.assert_array_equal(cq.qjl_matrix(d, seed).numpy(), O.qjl_matrix(d, seed))


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_prod_append_rows(cq, dev, d, dtype):
    b, h, t, pos = 2, 3, 77, 5
    x = kv_source(11 + d, (b, h, t, d), outliers=True)
    x[0, 0, 0, :] = 0.0  # an all-zero row: norm 0, codes of u = 0
    side = cq.CacheSide.empty(PROD, False, b, h, d, 96, dev, seed=42)
    cq.quant_append(side, x.to(dtype).to(dev), pos)
    torch.cuda.synchronize()
    got = export_np(cq, side, t, pos)
    assert_prod_rows_close(got, oracle_rows(PROD, x, 42), d)


def test_prod_rows_import_export_roundtrip(cq, dev):
    rows = oracle_rows(PROD, kv_source(3, (2, 2, 45, 128)), 42)
    side = cq.CacheSide.empty(PROD, False, 2, 2, 128, 64, dev, seed=42)
    cq.rows_import(side, torch.from_numpy(rows.view(np.int32)).to(dev), 9)
    np.testing.assert_array_equal(export_np(cq, side, 45, 9), rows)


def test_prod_refused_as_values(cq, dev):
    with pytest.raises(cq.CqkvError):
        cq.TurboKvCache(FP8, PROD, 1, 1, 128, 32, device=dev)
    side = cq.CacheSide.empty(PROD, True, 1, 1, 128, 32, dev, seed=44)
    with pytest.raises(cq.CqkvError):
        cq.quant_append(side, torch.zeros(1, 1, 4, 128, dtype=torch.bfloat16, device=dev))


@pytest.mark.parametrize("splits", [1, 3])
def test_prod_decode_vs_reference_fused_kernel(cq, dev, splits):
    """The reference's rows (imported) decoded by the HIP kernel: within the tolerance of the
    reference's fused kernel output, which equals float64 attention over the same codes to
    1.6e-6."""
    g = np.load(__import__("os").path.join(__import__("os").path.dirname(__file__), "golden",
                                           "ref_prod4.npz"))
    q, _, _ = prod_inputs()
    b, hq, lq, d = q.shape
    hkv, lk = g["kd"].shape[1], g["kd"].shape[2]
    ks = cq.CacheSide.empty(PROD, False, b, hkv, d, 320, dev, seed=42)
    vs = cq.CacheSide.empty(TURBO4, True, b, hkv, d, 320, dev, seed=44)
    cq.rows_import(ks, torch.from_numpy(g["kd"].view(np.int32)).to(dev))
    cq.rows_import(vs, torch.from_numpy(g["vd"].view(np.int32)).to(dev))
    out = torch.empty((b, hq, lq, d), dtype=torch.float32, device=dev)
    got = cq.decode_attention(torch.from_numpy(q).to(torch.bfloat16).to(dev), ks, vs, lk,
                              float(g["scale"]), splits=splits, out=out).cpu().numpy()
    err = np.abs(got - g["out"])
    assert err.max() <= 2e-2 and err.mean() <= 2e-3, (err.max(), err.mean())
    assert err.max() <= 5e-3, err.max()  # the f16 operands' rounding, well inside


@pytest.mark.parametrize("vf", [TURBO4, FP8, MXFP4, NVFP4, MXFP8])
@pytest.mark.parametrize("d", [64, 128])
def test_prod_decode_mixed_values(cq, dev, vf, d):
    """TurboProd keys with values of every format (TurboKvCache::with_formats(TurboProd{4},
    value, ..)), appended and decoded on the GPU, against the reference CPU path on the GPU's
    codes and the exact value."""
    b, hq, hkv, ctx, lq = 2, 8, 2, 600, 2
    q = kv_source(21, (b, hq, lq, d))
    k = kv_source(22, (b, hkv, ctx, d), outliers=True)
    v = kv_source(23, (b, hkv, ctx, d), outliers=True)
    cache = cq.TurboKvCache(PROD, vf, b, hkv, d, ctx, device=dev)
    cache.append(k.to(dev), v.to(dev))
    scale = 1.0 / d ** 0.5
    out = torch.empty((b, hq, lq, d), dtype=torch.float32, device=dev)
    got = cq.decode_attention(q.to(dev), cache.k, cache.v, ctx, scale, window_right=0,
                              out=out).cpu().numpy()
    kr, vr = export_np(cq, cache.k, ctx), export_np(cq, cache.v, ctx)
    assert_prod_rows_close(kr, oracle_rows(PROD, k, 42), d)
    kw = dict(wr=0, v_fmt=vf)
    want = oracle_decode(PROD, q, kr, vr, ctx, scale, **kw)
    exact = exact_decode(PROD, q, kr, vr, ctx, scale, **kw)
    assert_decode_parity(PROD, got, want, exact, rotated=True, value_bf16=vf != TURBO4)


def test_prod_decode_ragged_windows_columns(cq, dev):
    """Ragged lengths, a window and 40 (query, head) columns per kv head (three column blocks)."""
    b, hq, hkv, d, ctx, lq = 3, 8, 2, 128, 700, 10
    q = kv_source(31, (b, hq, lq, d))
    k = kv_source(32, (b, hkv, ctx, d))
    v = kv_source(33, (b, hkv, ctx, d))
    cache = cq.TurboKvCache(PROD, FP8, b, hkv, d, 704, device=dev)
    cache.append(k.to(dev), v.to(dev))
    lens = [700, 33, 1]
    lens_t = torch.tensor(lens, dtype=torch.int32, device=dev)
    out = torch.empty((b, hq, lq, d), dtype=torch.float32, device=dev)
    got = cq.decode_attention(q.to(dev), cache.k, cache.v, ctx, 0.1, kv_lens=lens_t,
                              window_left=200, window_right=0, out=out).cpu().numpy()
    kr, vr = export_np(cq, cache.k, ctx), export_np(cq, cache.v, ctx)
    kw = dict(kv_lens=np.array(lens, np.int32), wl=200, wr=0, v_fmt=FP8)
    want = oracle_decode(PROD, q, kr, vr, ctx, 0.1, **kw)
    exact = exact_decode(PROD, q, kr, vr, ctx, 0.1, **kw)
    assert_decode_parity(PROD, got, want, exact, rotated=True, value_bf16=True)


def test_prod_paged_equals_dense(cq, dev):
    """FP8 values (their P goes in as a hi + lo pair: a split changes only the summation order,
    within 1e-5)."""
    b, hq, hkv, d, n1, n2 = 2, 8, 2, 128, 300, 170
    q = kv_source(41, (b, hq, 1, d)).to(dev)
    k, v = kv_source(42, (b, hkv, n1 + n2, d)), kv_source(43, (b, hkv, n1 + n2, d))
    dense = cq.TurboKvCache(PROD, FP8, b, hkv, d, n1 + n2, device=dev)
    dense.append(k.to(dev), v.to(dev))
    f32 = torch.float32
    want = cq.decode_attention(q, dense.k, dense.v, n1 + n2, 0.1, splits=1,
                               out=torch.empty(q.shape, dtype=f32, device=dev))
    blocks = []
    for off, n in ((0, n1), (n1, n2)):
        kc = cq.CacheSide.empty(PROD, False, b, hkv, d, 320, dev, seed=42)
        kc.qjl = dense.k.qjl  # blocks of one cache share its S
        vc = cq.CacheSide.empty(FP8, True, b, hkv, d, 320, dev, seed=44)
        cq.quant_append(kc, k[:, :, off:off + n].to(dev), 0)
        cq.quant_append(vc, v[:, :, off:off + n].to(dev), 0)
        blocks.append((kc, vc, n))
    got = cq.decode_attention_paged(q, blocks, 0.1, out=torch.empty(q.shape, dtype=f32,
                                                                     device=dev))
    torch.cuda.synchronize()
    np.testing.assert_allclose(got.cpu().numpy(), want.cpu().numpy(), atol=1e-5, rtol=1e-4)
    # blocks whose QJL matrices differ are refused
    kx = cq.CacheSide.empty(PROD, False, b, hkv, d, 320, dev, seed=42)
    with pytest.raises(cq.CqkvError):
        cq.decode_attention_paged(q, [blocks[0], (kx, blocks[1][1], n2)], 0.1)


def test_prod_rope_append_and_growth(cq, dev):
    """The fused RoPE + append with TurboProd keys (values of another format by their own
    launch) equals rope then two plain appends: the values bit for bit, the keys by the TurboProd
    criterion (the fused kernel keeps the row-parallel encoder, the plain append of bf16 rows
    takes the MFMA one; both hold the reference's criterion, with their own f32 rounding of the
    rotation); a cache that grows past its capacity holds the rows of one large cache."""
    b, hq, hkv, t, d, pos, cap = 2, 8, 2, 19, 128, 5, 64
    qkv = kv_source(51, (b, t, 1, (hq + 2 * hkv) * d))[:, :, 0].to(dev)
    q, k, v = cq.split_qkv(qkv, hq, hkv)
    inv = 1.0 / 10000.0 ** (np.arange(0, d, 2, dtype=np.float64) / d)
    ang = np.arange(pos + t + 3, dtype=np.float64)[:, None] * inv[None, :]
    cos = torch.from_numpy(np.cos(ang).astype(np.float32)).to(torch.bfloat16)
    sin = torch.from_numpy(np.sin(ang).astype(np.float32)).to(torch.bfloat16)

    def sides():
        return (cq.CacheSide.empty(PROD, False, b, hkv, d, cap, dev, seed=42),
                cq.CacheSide.empty(TURBO4, True, b, hkv, d, cap, dev, seed=44))
    ks, vs = sides()
    cq.rope_quant_append(ks, vs, q, k, v, cos.to(dev), sin.to(dev), cq.ROPE_HALVES, pos)
    k_rot = O.round_to(O.rope(k.float().cpu().numpy(), cos.float().numpy(), sin.float().numpy(),
                              cq.ROPE_HALVES, pos), "bf16")
    ks2, vs2 = sides()
    cq.quant_append(ks2, torch.from_numpy(k_rot).to(torch.bfloat16).to(dev), pos)
    cq.quant_append(vs2, v, pos)
    torch.cuda.synchronize()
    assert_prod_rows_close(export_np(cq, ks, cap), export_np(cq, ks2, cap), d)
    np.testing.assert_array_equal(export_np(cq, vs, cap), export_np(cq, vs2, cap))

    kk, vv = kv_source(61, (2, 2, 150, 128)), kv_source(62, (2, 2, 150, 128))
    grown = cq.TurboKvCache(PROD, FP8, 2, 2, 128, 32, device=dev, grow_by=16)
    big = cq.TurboKvCache(PROD, FP8, 2, 2, 128, 256, device=dev)
    for off, n in ((0, 40), (40, 60), (100, 50)):
        grown.append(kk[:, :, off:off + n].to(dev), vv[:, :, off:off + n].to(dev))
        big.append(kk[:, :, off:off + n].to(dev), vv[:, :, off:off + n].to(dev))
    np.testing.assert_array_equal(export_np(cq, grown.k, 150), export_np(cq, big.k, 150))
    qd = kv_source(63, (2, 8, 1, 128)).to(dev)
    np.testing.assert_array_equal(grown.attention(qd, 0.1).float().cpu().numpy(),
                                  big.attention(qd, 0.1).float().cpu().numpy())
