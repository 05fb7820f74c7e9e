"""GPU parity of the TurboMse append with the rotation on MFMA (csrc/append_turbo.hip), the form
that 16-byte aligned bf16 / f16 rows of a Hadamard-rotated TurboQuant side take
(RowCodec::quantize_row, candle-core/src/accel/turbo.rs:299-323, after TurboQuantizer::rotate,
candle-nn/src/turbo_quant.rs:182-189).

Rows are held to the reference's own TurboQuant criterion (candle-core/tests/
accel_kernels_host.rs:998-1027: norms within rtol 1e-5, at most 0.1 % of the codes flipped, each
to a neighbour) against the oracle's encoder of the source rows, and against the row-parallel
encoder of this library (the f32 form of the same rows takes it). Rows whose norm is zero or not
finite have codes fixed by the reference's rule (inv = 0 unless norm > 0, then u = y * inv):
those are compared bit for bit."""
import numpy as np
import pytest
import torch

from tests.helpers import (assert_rows_match_source, assert_turbo_rows_close, kv_source,
                           oracle_rows, packed_codes)

pytestmark = pytest.mark.gpu

TURBO = 0
DT = {"bf16": torch.bfloat16, "f16": torch.float16}


def export_np(cq, side, tokens, position=0):
    return cq.rows_export(side, tokens, position).cpu().numpy().view(np.uint32)


@pytest.mark.parametrize("bits", [4, 3, 2, 1])
@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("is_value", [False, True])
@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_mfma_append_vs_reference(cq, dev, bits, d, is_value, dtype):
    """An unaligned start, a length that is not a multiple of the 8-token tiles or the 16-row
    groups, several chunks per plane; rows already in the cache stay."""
    b, h, t, pos, cap = 2, 3, 333, 5, 352
    seed = 44 if is_value else 42
    x = kv_source(70 + bits + d, (b, h, t, d), outliers=True).to(DT[dtype])
    side = cq.CacheSide.empty(TURBO, is_value, b, h, d, cap, dev, seed=seed, bits=bits)
    pre = oracle_rows(TURBO, kv_source(71, (b, h, cap, d)), seed, bits=bits)
    cq.rows_import(side, torch.from_numpy(pre.view(np.int32)).to(dev), 0)
    cq.quant_append(side, x.to(dev), pos)
    torch.cuda.synchronize()
    got = export_np(cq, side, cap)
    assert_rows_match_source(TURBO, got[:, :, pos:pos + t], x, seed, bits=bits)
    outside = np.ones(cap, bool)
    outside[pos:pos + t] = False
    np.testing.assert_array_equal(got[:, :, outside], pre[:, :, outside])
    # the row-parallel encoder (f32 rows of the same values) within the same criterion
    side2 = cq.CacheSide.empty(TURBO, is_value, b, h, d, cap, dev, seed=seed, bits=bits)
    cq.quant_append(side2, x.float().to(dev), pos)
    torch.cuda.synchronize()
    assert_turbo_rows_close(got[:, :, pos:pos + t], export_np(cq, side2, cap)[:, :, pos:pos + t],
                            d, bits)


@pytest.mark.parametrize("is_value", [False, True])
@pytest.mark.parametrize("bits,d,dtype", [(4, 128, "bf16"), (3, 64, "f16"), (2, 128, "f16"),
                                          (1, 64, "bf16"), (4, 64, "f16")])
def test_mfma_append_per_batch_positions(cq, dev, is_value, bits, d, dtype):
    """Per-sequence positions: every chunk starts up to 7 tokens early (the first value tile of
    any position); a position that is not a multiple of 8, and one whose append is cut off at the
    capacity (positions past it are skipped)."""
    b, h, t, cap = 4, 2, 37, 96
    seed = 44 if is_value else 42
    x = kv_source(81 + bits + d, (b, h, t, d)).to(DT[dtype])
    pos = [3, 0, 13, 70]  # 70 + 37 > 96: the last 11 tokens fall past the capacity
    side = cq.CacheSide.empty(TURBO, is_value, b, h, d, cap, dev, seed=seed, bits=bits)
    cq.quant_append(side, x.to(dev), 0,
                    positions=torch.tensor(pos, dtype=torch.int32, device=dev))
    torch.cuda.synchronize()
    got = export_np(cq, side, cap)
    for i, p in enumerate(pos):
        n = min(t, cap - p)
        assert_rows_match_source(TURBO, got[i:i + 1, :, p:p + n], x[i:i + 1, :, :n], seed,
                                 bits=bits)
        assert (got[i, :, :p] == 0).all() and (got[i, :, p + n:] == 0).all()


@pytest.mark.parametrize("is_value", [False, True])
def test_mfma_append_special_rows(cq, dev, is_value):
    """A zero row (every code 8), a row with a NaN (NaN norm: inv = 0, so every finite element
    codes 8 and the NaN one 0 after the rotation spreads it: all 0), a row with an infinity (norm
    inf, u = inf * 0 = NaN: all 0), a huge row (its squares overflow: norm inf, u = y * 0 = 0: all
    8), a row of bf16 subnormals (its squares underflow: norm 0, all 8), a tiny normal row and an
    ordinary row (by the criterion)."""
    d, seed = 128, 44 if is_value else 42
    x = kv_source(90, (1, 1, 16, d))
    x[0, 0, 0] = 0.0
    x[0, 0, 1, 7] = float("nan")
    x[0, 0, 2, 9] = float("inf")
    x[0, 0, 3] = x[0, 0, 3] * 1e30
    x[0, 0, 4] = torch.full((d,), 5e-39).to(torch.bfloat16) * torch.sign(x[0, 0, 4])
    x[0, 0, 5] = (x[0, 0, 5].float() * 1e-18).to(torch.bfloat16)
    side = cq.CacheSide.empty(TURBO, is_value, 1, 1, d, 32, dev, seed=seed)
    cq.quant_append(side, x.to(dev), 0)
    torch.cuda.synchronize()
    got = export_np(cq, side, 16)
    codes = packed_codes(got, 4, d)[0, 0]
    norms = got[0, 0, :, d // 8].view(np.float32)
    assert (codes[0] == 8).all() and norms[0] == 0.0
    assert (codes[1] == 0).all() and np.isnan(norms[1])
    assert (codes[2] == 0).all() and norms[2] == np.inf
    assert (codes[3] == 8).all() and norms[3] == np.inf
    assert (codes[4] == 8).all() and norms[4] == 0.0
    assert_rows_match_source(TURBO, got[:, :, 5:], x[:, :, 5:], seed)
