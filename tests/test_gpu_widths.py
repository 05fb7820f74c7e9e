"""GPU parity of the TurboQuant widths other than 4: QuantFormat::TurboMse{1, 2, 3} on keys and
values and TurboProd{2, 3, 5} on keys (candle-core/src/accel/formats.rs:22-29, code widths of
formats.rs:138-160; Lloyd-Max codebooks of turbo.rs:58-146 at those widths), cqkv_side.bits.

The cache keeps the codes as nibbles at every width; rows are compared in the reference layout
(b-bit codes packed LSB first) against the oracle's RowCodec restatement, itself pinned to the
reference kernels' rows at these widths (tests/test_oracle.py, tests/golden/ref_quant_turbo{1,2,3}
and ref_prod_widths). Decode: against the reference's fused kernel over its own rows
(tests/golden/ref_decode_widths.npz: TurboMse{4} keys + TurboMse{3} values, the pairing of the
reference's turbo_kv_cache_fused_matches_unfused test, and TurboProd{3} keys + TurboMse{2}
values), and against the reference CPU path on the codes the GPU wrote by the criterion of
rotated caches (assert_decode_parity)."""
import os

import numpy as np
import pytest
import torch

from tests.helpers import (assert_decode_parity, assert_rows_match_source, exact_decode,
                           kv_source, oracle_decode)
from tests.test_oracle import widths_inputs

pytestmark = pytest.mark.gpu

TURBO, PROD, MXFP4, NVFP4, MXFP8, FP8 = 0, 1, 2, 3, 4, 5
GOLD = os.path.join(os.path.dirname(__file__), "golden")


def export_np(cq, side, tokens, position=0):
    return cq.rows_export(side, tokens, position).cpu().numpy().view(np.uint32)


@pytest.mark.parametrize("fmt,bits,is_value", [(TURBO, 3, False), (TURBO, 3, True),
                                               (TURBO, 2, False), (TURBO, 2, True),
                                               (TURBO, 1, False), (TURBO, 1, True),
                                               (PROD, 3, False), (PROD, 2, False),
                                               (PROD, 5, False)])
@pytest.mark.parametrize("d", [64, 128])
def test_width_append_rows(cq, dev, fmt, bits, is_value, d):
    b, h, t, pos = 2, 3, 77, 5
    x = kv_source(40 + bits + d, (b, h, t, d), outliers=True)
    x[0, 0, 0, :] = 0.0  # an all-zero row
    seed = 44 if is_value else 42
    side = cq.CacheSide.empty(fmt, is_value, b, h, d, 96, dev, seed=seed, bits=bits)
    cq.quant_append(side, x.to(dev), pos)
    torch.cuda.synchronize()
    assert_rows_match_source(fmt, export_np(cq, side, t, pos), x, seed, bits=bits)


@pytest.mark.parametrize("name,bits,d", [("turbo3_d128", 3, 128), ("turbo2_d64", 2, 64),
                                         ("turbo1_d64", 1, 64)])
@pytest.mark.parametrize("is_value", [False, True])
def test_width_rows_import_export_roundtrip(cq, dev, name, bits, d, is_value):
    """The reference kernel's packed rows in, the same rows out, bit for bit (keys row-major,
    values through the 8-token tiles)."""
    rows = np.load(os.path.join(GOLD, f"ref_quant_{name}.npz"))["rows"]
    n = rows.shape[0]
    side = cq.CacheSide.empty(TURBO, is_value, 1, 1, d, 64, dev, seed=42, bits=bits)
    cq.rows_import(side, torch.from_numpy(rows.view(np.int32)).reshape(1, 1, n, -1).to(dev), 3)
    np.testing.assert_array_equal(export_np(cq, side, n, 3).reshape(n, -1), rows)


@pytest.mark.parametrize("name,kfmt,kbits,vbits", [("mse4_mse3", TURBO, 4, 3),
                                                   ("prod3_mse2", PROD, 3, 2)])
@pytest.mark.parametrize("splits", [1, 3, 0])
def test_width_decode_vs_reference_fused_kernel(cq, dev, name, kfmt, kbits, vbits, splits):
    """The reference's rows (imported) decoded by the HIP kernel, against the reference's fused
    kernel output over them (which is float64 attention of the codes to 1e-5)."""
    g = np.load(os.path.join(GOLD, "ref_decode_widths.npz"))
    q, _, _ = widths_inputs()
    b, hq, lq, d = q.shape
    kd, vd = g[f"kd_{name}"], g[f"vd_{name}"]
    hkv, lk = kd.shape[1], kd.shape[2]
    ks = cq.CacheSide.empty(kfmt, False, b, hkv, d, 320, dev, seed=42, bits=kbits)
    vs = cq.CacheSide.empty(TURBO, True, b, hkv, d, 320, dev, seed=44, bits=vbits)
    cq.rows_import(ks, torch.from_numpy(kd.view(np.int32)).to(dev))
    cq.rows_import(vs, torch.from_numpy(vd.view(np.int32)).to(dev))
    out = torch.empty((b, hq, lq, d), dtype=torch.float32, device=dev)
    got = cq.decode_attention(torch.from_numpy(q).to(torch.bfloat16).to(dev), ks, vs, lk,
                              float(g["scale"]), splits=splits, out=out).cpu().numpy()
    err = np.abs(got - g[f"out_{name}"])
    assert err.max() <= 2e-2 and err.mean() <= 2e-3, (err.max(), err.mean())
    assert err.max() <= 5e-3, err.max()  # the f16 operands' rounding, well inside


# (key format, key bits, value format, value bits): equal and different TurboMse widths (the
# narrower side on its compact table), TurboMse with the other formats, TurboProd widths
# (TurboProd{5}: 4-bit MSE codes on the 64 KB table, values sharing it or on their own)
PAIRS = [(TURBO, 4, TURBO, 3), (TURBO, 2, TURBO, 4), (TURBO, 3, TURBO, 3), (TURBO, 1, FP8, 0),
         (FP8, 0, TURBO, 2), (MXFP4, 0, TURBO, 1), (PROD, 3, TURBO, 2), (PROD, 2, MXFP4, 0),
         (PROD, 3, TURBO, 4), (PROD, 5, TURBO, 4), (PROD, 5, TURBO, 2), (PROD, 5, FP8, 0),
         (PROD, 5, MXFP4, 0), (PROD, 5, NVFP4, 0)]


@pytest.mark.parametrize("kf,kb,vf,vb", PAIRS)
@pytest.mark.parametrize("d", [64, 128])
def test_width_decode_pairs(cq, dev, kf, kb, vf, vb, d):
    b, hq, hkv, ctx, lq = 2, 8, 2, 500, 2
    q = kv_source(51, (b, hq, lq, d))
    k = kv_source(52, (b, hkv, ctx, d), outliers=True)
    v = kv_source(53, (b, hkv, ctx, d), outliers=True)
    cache = cq.TurboKvCache(kf, vf, b, hkv, d, ctx, device=dev, key_bits=kb, value_bits=vb)
    cache.append(k.to(dev), v.to(dev))
    scale = 1.0 / d ** 0.5
    out = torch.empty((b, hq, lq, d), dtype=torch.float32, device=dev)
    got = cq.decode_attention(q.to(dev), cache.k, cache.v, ctx, scale, window_right=0,
                              out=out).cpu().numpy()
    kr, vr = export_np(cq, cache.k, ctx), export_np(cq, cache.v, ctx)
    assert_rows_match_source(kf, kr, k, 42, bits=kb)
    assert_rows_match_source(vf, vr, v, 44, bits=vb)
    kw = dict(wr=0, v_fmt=vf, k_bits=kb, v_bits=vb)
    want = oracle_decode(kf, q, kr, vr, ctx, scale, **kw)
    exact = exact_decode(kf, q, kr, vr, ctx, scale, **kw)
    turbo_v = vf == TURBO
    assert_decode_parity(kf, got, want, exact, rotated=True, value_bf16=not turbo_v)


def test_width_paged_equals_dense_and_growth(cq, dev):
    """TurboMse{4} keys + TurboMse{3} values: the paged call over two blocks equals the dense
    call within the one-operand P bound of TurboQuant values (2e-3), and a cache grown step by
    step (cqkv_side_copy at the reference's growth rule) holds the same rows as one large
    cache."""
    b, hq, hkv, d, n1, n2 = 2, 8, 2, 128, 300, 170
    q = kv_source(61, (b, hq, 1, d)).to(dev)
    k, v = kv_source(62, (b, hkv, n1 + n2, d)), kv_source(63, (b, hkv, n1 + n2, d))
    dense = cq.TurboKvCache(TURBO, TURBO, b, hkv, d, n1 + n2, device=dev, key_bits=4,
                            value_bits=3)
    dense.append(k.to(dev), v.to(dev))
    f32 = torch.float32
    want = cq.decode_attention(q, dense.k, dense.v, n1 + n2, 0.1, splits=1,
                               out=torch.empty(q.shape, dtype=f32, device=dev))
    blocks = []
    for off, n in ((0, n1), (n1, n2)):
        kc = cq.CacheSide.empty(TURBO, False, b, hkv, d, 320, dev, seed=42, bits=4)
        vc = cq.CacheSide.empty(TURBO, True, b, hkv, d, 320, dev, seed=44, bits=3)
        cq.quant_append(kc, k[:, :, off:off + n].to(dev), 0)
        cq.quant_append(vc, v[:, :, off:off + n].to(dev), 0)
        blocks.append((kc, vc, n))
    got = cq.decode_attention_paged(q, blocks, 0.1, out=torch.empty(q.shape, dtype=f32,
                                                                     device=dev))
    torch.cuda.synchronize()
    np.testing.assert_allclose(got.cpu().numpy(), want.cpu().numpy(), atol=2e-3, rtol=4e-3)
    # blocks whose value widths differ are refused
    vx = cq.CacheSide.empty(TURBO, True, b, hkv, d, 320, dev, seed=44, bits=2)
    with pytest.raises(cq.CqkvError):
        cq.decode_attention_paged(q, [blocks[0], (blocks[1][0], vx, n2)], 0.1)
    grown = cq.TurboKvCache(TURBO, TURBO, b, hkv, d, 64, device=dev, key_bits=4, value_bits=3,
                            grow_by=64)
    for off in range(0, n1 + n2, 97):
        t = min(97, n1 + n2 - off)
        grown.append(k[:, :, off:off + t].to(dev), v[:, :, off:off + t].to(dev))
    for gs, ds in ((grown.k, dense.k), (grown.v, dense.v)):
        np.testing.assert_array_equal(export_np(cq, gs, n1 + n2), export_np(cq, ds, n1 + n2))


@pytest.mark.parametrize("d", [128, 64])
def test_prod5_rows_import_export_roundtrip(cq, dev, d):
    """TurboProd{5} rows of the reference kernels in, the same rows out, bit for bit."""
    rows = np.load(os.path.join(GOLD, "ref_prod5.npz"))[f"rows_d{d}"]
    n = rows.shape[0]
    side = cq.CacheSide.empty(PROD, False, 1, 1, d, 64, dev, seed=42, bits=5)
    cq.rows_import(side, torch.from_numpy(rows.view(np.int32)).reshape(1, 1, n, -1).to(dev), 3)
    np.testing.assert_array_equal(export_np(cq, side, n, 3).reshape(n, -1), rows)


@pytest.mark.parametrize("vbits", [4, 3])
@pytest.mark.parametrize("splits", [1, 3, 0])
def test_prod5_decode_vs_reference_fused_kernel(cq, dev, vbits, splits):
    """The reference's TurboProd{5} rows (imported) with TurboMse{4} values (sharing the 64 KB
    code table) or TurboMse{3} values (on their compact table), decoded by the HIP kernel,
    against the reference's fused kernel over them."""
    g = np.load(os.path.join(GOLD, "ref_prod5.npz"))
    q, _, _ = widths_inputs()
    b, hq, lq, d = q.shape
    kd, vd = g["kd"], g[f"vd_mse{vbits}"]
    hkv, lk = kd.shape[1], kd.shape[2]
    ks = cq.CacheSide.empty(PROD, False, b, hkv, d, 320, dev, seed=42, bits=5)
    vs = cq.CacheSide.empty(TURBO, True, b, hkv, d, 320, dev, seed=44, bits=vbits)
    cq.rows_import(ks, torch.from_numpy(kd.view(np.int32)).to(dev))
    cq.rows_import(vs, torch.from_numpy(vd.view(np.int32)).to(dev))
    out = torch.empty((b, hq, lq, d), dtype=torch.float32, device=dev)
    got = cq.decode_attention(torch.from_numpy(q).to(torch.bfloat16).to(dev), ks, vs, lk,
                              float(g["scale"]), splits=splits, out=out).cpu().numpy()
    err = np.abs(got - g[f"out_mse{vbits}"])
    assert err.max() <= 5e-3 and err.mean() <= 2e-3, (err.max(), err.mean())


def test_width_arguments_refused(cq, dev):
    with pytest.raises(cq.CqkvError):  # TurboMse 5 bits
        side = cq.CacheSide.empty(TURBO, False, 1, 1, 128, 32, dev, bits=5)
        cq.quant_append(side, torch.zeros(1, 1, 4, 128, dtype=torch.bfloat16, device=dev))
    with pytest.raises(cq.CqkvError):  # TurboProd 1 bit
        side = cq.CacheSide.empty(PROD, False, 1, 1, 128, 32, dev, seed=42, bits=1)
        cq.quant_append(side, torch.zeros(1, 1, 4, 128, dtype=torch.bfloat16, device=dev))
    with pytest.raises(cq.CqkvError):  # TurboProd 6 bits
        side = cq.CacheSide.empty(PROD, False, 1, 1, 128, 32, dev, seed=42, bits=6)
        cq.quant_append(side, torch.zeros(1, 1, 4, 128, dtype=torch.bfloat16, device=dev))
    with pytest.raises(cq.CqkvError):  # a width for a format without one
        side = cq.CacheSide.empty(FP8, False, 1, 1, 128, 32, dev, bits=4)
        cq.quant_append(side, torch.zeros(1, 1, 4, 128, dtype=torch.bfloat16, device=dev))
    a = cq.CacheSide.empty(TURBO, True, 1, 1, 128, 32, dev, seed=44, bits=3)
    c = cq.CacheSide.empty(TURBO, True, 1, 1, 128, 64, dev, seed=44, bits=4)
    with pytest.raises(cq.CqkvError):  # growth between different widths
        cq.side_copy(c, a, 8)
