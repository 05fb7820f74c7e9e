"""GPU parity of the TurboProd key append on MFMA (csrc/append_turbo.hip, prod_mfma_kernel), the
form that 16-byte aligned bf16 / f16 rows of a Hadamard-rotated TurboProd side take at D = 64 and
128 (RowCodec::quantize_row, candle-core/src/accel/turbo.rs:299-323, after TurboQuantizer::rotate,
candle-nn/src/turbo_quant.rs:182-189).

Rows are held to the TurboProd criterion of tests/helpers.py:assert_prod_rows_close (the MSE codes
and norms by the reference's TurboQuant criterion, candle-core/tests/accel_kernels_host.rs:998-1027;
|r| and the QJL sign bits in rows without a code flip) against the oracle's encoder of the source
rows, and against this library's row-parallel encoder (the f32 form of the same rows takes it).
Rows whose norm is zero or not finite have their codes fixed by the reference's rule (inv = 0
unless norm > 0, then u = y * inv): those codes are compared bit for bit."""
import numpy as np
import pytest
import torch

from tests.helpers import (assert_prod_rows_close, assert_rows_match_source, kv_source,
                           obits, oracle_rows, packed_codes)

pytestmark = pytest.mark.gpu

PROD = 1
DT = {"bf16": torch.bfloat16, "f16": torch.float16}


def export_np(cq, side, tokens, position=0):
    return cq.rows_export(side, tokens, position).cpu().numpy().view(np.uint32)


@pytest.mark.parametrize("bits", [4, 3, 2, 5])
@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_prod_mfma_append_vs_reference(cq, dev, bits, d, dtype):
    """An unaligned start, a length that is not a multiple of the 32-token wavefront groups,
    several chunks per plane; rows already in the cache stay."""
    b, h, t, pos, cap = 2, 3, 600, 5, 640
    x = kv_source(170 + bits + d, (b, h, t, d), outliers=True).to(DT[dtype])
    side = cq.CacheSide.empty(PROD, False, b, h, d, cap, dev, seed=42, bits=bits)
    pre = oracle_rows(PROD, kv_source(171, (b, h, cap, d)), 42, bits=bits)
    cq.rows_import(side, torch.from_numpy(pre.view(np.int32)).to(dev), 0)
    cq.quant_append(side, x.to(dev), pos)
    torch.cuda.synchronize()
    got = export_np(cq, side, cap)
    assert_rows_match_source(PROD, got[:, :, pos:pos + t], x, 42, bits=bits)
    outside = np.ones(cap, bool)
    outside[pos:pos + t] = False
    np.testing.assert_array_equal(got[:, :, outside], pre[:, :, outside])
    # the row-parallel encoder (f32 rows of the same values) within the same criterion
    side2 = cq.CacheSide.empty(PROD, False, b, h, d, cap, dev, seed=42, bits=bits)
    cq.quant_append(side2, x.float().to(dev), pos)
    torch.cuda.synchronize()
    assert_prod_rows_close(got[:, :, pos:pos + t], export_np(cq, side2, cap)[:, :, pos:pos + t],
                           d, obits(PROD, bits))


@pytest.mark.parametrize("bits,d,dtype", [(4, 128, "bf16"), (3, 64, "f16"), (5, 128, "f16")])
def test_prod_mfma_append_per_batch_positions(cq, dev, bits, d, dtype):
    """Per-sequence positions: every chunk starts up to 7 tokens early; a position that is not a
    multiple of 8, and one whose append is cut off at the capacity (positions past it are
    skipped)."""
    b, h, t, cap = 4, 2, 37, 96
    x = kv_source(181 + bits + d, (b, h, t, d)).to(DT[dtype])
    pos = [3, 0, 13, 70]  # 70 + 37 > 96: the last 11 tokens fall past the capacity
    side = cq.CacheSide.empty(PROD, False, b, h, d, cap, dev, seed=42, bits=bits)
    cq.quant_append(side, x.to(dev), 0,
                    positions=torch.tensor(pos, dtype=torch.int32, device=dev))
    torch.cuda.synchronize()
    got = export_np(cq, side, cap)
    for i, p in enumerate(pos):
        n = min(t, cap - p)
        assert_rows_match_source(PROD, got[i:i + 1, :, p:p + n], x[i:i + 1, :, :n], 42, bits=bits)
        assert (got[i, :, :p] == 0).all() and (got[i, :, p + n:] == 0).all()


@pytest.mark.parametrize("d", [64, 128])
def test_prod_mfma_append_special_rows(cq, dev, d):
    """A zero row, a row with a NaN, a row with an infinity, a huge row (its squares overflow), a
    row of bf16 subnormals (its squares underflow), a tiny normal row and ordinary rows: the codes
    of the first five equal the oracle's bit for bit (they follow from inv = 0 or a NaN u), and
    every row holds the TurboProd criterion against the oracle (NaN norms and |r| included)."""
    x = kv_source(190, (1, 1, 40, d))
    x[0, 0, 0] = 0.0
    x[0, 0, 1, 7] = float("nan")
    x[0, 0, 2, 9] = float("inf")
    x[0, 0, 3] = x[0, 0, 3] * 1e30
    x[0, 0, 4] = torch.full((d,), 5e-39).to(torch.bfloat16) * torch.sign(x[0, 0, 4])
    x[0, 0, 5] = (x[0, 0, 5].float() * 1e-18).to(torch.bfloat16)
    x = x.to(torch.bfloat16)
    side = cq.CacheSide.empty(PROD, False, 1, 1, d, 64, dev, seed=42)
    cq.quant_append(side, x.to(dev), 0)
    torch.cuda.synchronize()
    got = export_np(cq, side, 40)
    want = oracle_rows(PROD, x, 42)
    np.testing.assert_array_equal(packed_codes(got, 3, d)[0, 0, :5], packed_codes(want, 3, d)[0, 0, :5])
    assert_prod_rows_close(got, want, d)


def test_prod_mfma_append_config2_shape_sampled_planes(cq, dev):
    """The bench's append workload (B=32, 8 kv heads, 2048 tokens, D=128, bf16 with outlier
    channels): 2,304 chunks over the 256 workgroups; the first and the last plane against the
    oracle."""
    b, h, t, d = 32, 8, 2048, 128
    x = kv_source(201, (b, h, t, d), outliers=True).to(dev)
    side = cq.CacheSide.empty(PROD, False, b, h, d, t, dev, seed=42)
    cq.quant_append(side, x, 0)
    torch.cuda.synchronize()
    got = export_np(cq, side, t)
    for bi, hi in ((0, 0), (b - 1, h - 1)):
        assert_prod_rows_close(got[bi:bi + 1, hi:hi + 1],
                               oracle_rows(PROD, x[bi:bi + 1, hi:hi + 1].cpu(), 42), d)
