"""Shared input generators and oracle wrappers of the GPU parity tests."""
from __future__ import annotations

import numpy as np
import torch

from oracle import oracle as O

BITS = {5: 0, 2: 0, 0: 4, 3: 0, 4: 0}  # oracle (mode, bits): FP8, MXFP4, TURBO4, NVFP4, MXFP8


def kv_source(seed: int, shape, outliers: bool = False) -> torch.Tensor:
    """bf16 N(0, 1) values (b, h, t, d); with `outliers`, 1 % of the (head, dim) channels -
    drawn once per tensor by a seeded Bernoulli(0.01) and held across batch and tokens - are
    scaled by 8 before the bf16 rounding."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(*shape, generator=g)
    if outliers:
        mask = torch.rand(shape[1], shape[3], generator=g) < 0.01
        x = torch.where(mask[None, :, None, :], x * 8.0, x)
    return x.to(torch.bfloat16)


def oracle_rows(fmt: int, x: torch.Tensor, seed: int = 0) -> np.ndarray:
    """Reference rows of x (.., d) bf16 (TURBO4: rotated by the seed's Hadamard first)."""
    xf = x.float().numpy()
    if fmt == 0:
        pi = O.rotation_matrix(x.shape[-1], O.ROT_HADAMARD, seed)
        xf = O.rotate_rows(pi, xf.reshape(-1, x.shape[-1])).reshape(xf.shape)
    return O.quantize_rows(fmt, BITS[fmt], xf)


def oracle_decode(fmt: int, q: torch.Tensor, k_rows: np.ndarray, v_rows: np.ndarray, lk: int,
                  scale: float, kv_lens=None, wl=-1, wr=-1, k_seed=42, v_seed=44) -> np.ndarray:
    """The reference CPU decode path (dequantize, unrotate, bf16, unfused f32 attention),
    rounded to bf16 like the reference's output."""
    d = q.shape[-1]
    pk = pv = None
    if fmt == 0:
        pk = O.rotation_matrix(d, O.ROT_HADAMARD, k_seed)
        pv = O.rotation_matrix(d, O.ROT_HADAMARD, v_seed)
    qb = O.f32_to_bf16_bits(q.float().numpy())
    out = O.cache_attention(qb, k_rows, v_rows, (fmt, BITS[fmt]), (fmt, BITS[fmt]), pk, pv, lk,
                            scale, kv_lens=kv_lens, wl=wl, wr=wr, threads=16)
    return O.round_bf16(out)


def assert_close_bf16(got: np.ndarray, want: np.ndarray, max_abs=2e-2, mean_abs=2e-3):
    """The BASELINE tolerance of bf16 attention outputs."""
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    assert np.isfinite(got).all(), "non-finite output"
    assert err.max() <= max_abs and err.mean() <= mean_abs, (err.max(), err.mean())
    return err.max(), err.mean()


def exact_decode(fmt: int, q: torch.Tensor, k_rows: np.ndarray, v_rows: np.ndarray, lk: int,
                 scale: float, kv_lens=None, wl=-1, wr=-1, k_seed=42, v_seed=44) -> np.ndarray:
    """float64 attention over the dequantized (and unrotated) codes, without the reference
    path's bf16 rounding of the cache: the mathematical value both paths approximate."""
    b, hq, lq, d = q.shape
    hkv = k_rows.shape[1]
    kd = O.dequantize_rows(fmt, BITS[fmt], d, k_rows[:, :, :lk]).astype(np.float64)
    vd = O.dequantize_rows(fmt, BITS[fmt], d, v_rows[:, :, :lk]).astype(np.float64)
    if fmt == 0:
        kd = kd @ O.rotation_matrix(d, O.ROT_HADAMARD, k_seed).astype(np.float64)
        vd = vd @ O.rotation_matrix(d, O.ROT_HADAMARD, v_seed).astype(np.float64)
    qq = q.float().numpy().astype(np.float64)
    out = np.zeros((b, hq, lq, d))
    g = hq // hkv
    for bi in range(b):
        n = lk if kv_lens is None else int(kv_lens[bi])
        for h in range(hq):
            for i in range(lq):
                lo, hi = O.key_range(i, lq, n, wl, wr)
                if lo >= hi:
                    continue
                s = kd[bi, h // g, lo:hi] @ qq[bi, h, i] * scale
                p = np.exp(s - s.max())
                out[bi, h, i] = p @ vd[bi, h // g, lo:hi] / p.sum()
    return out


def assert_decode_parity(fmt: int, got: np.ndarray, ref: np.ndarray, exact: np.ndarray | None):
    """FP8 / MX / NVFP4: the BASELINE tolerance against the reference path. TurboQuant: the same
    tolerance against the exact value of the same codes, and against the reference path within
    that path's own deviation from the exact value (its bf16 rounding of the unrotated cache
    alone moves outputs by up to ~4e-2 on outlier-heavy inputs) plus the tolerance. The exact
    value is what the reference's own fused kernel computes: on the committed fixture
    tests/golden/ref_decode_turbo4.npz it agrees with the exact value to 4e-6, and the
    reference's CPU path differs from it by 3.0e-2."""
    if fmt != 0 or exact is None:
        return assert_close_bf16(got, ref)
    assert_close_bf16(got, exact)
    own = np.abs(ref - exact).max()
    err = np.abs(got.astype(np.float64) - ref)
    assert err.max() <= own + 2e-2 and err.mean() <= 2e-3, (err.max(), own, err.mean())


def assert_turbo_rows_close(got: np.ndarray, want: np.ndarray, d: int):
    """TurboQuant-4 rows against the reference encoder's rows under the reference's own
    end-to-end criterion (candle-core/tests/accel_kernels_host.rs:998-1027): norms within rtol
    1e-5, at most 0.1 % of the codes flipped, each flip to a neighbouring code."""
    cw = d // 8
    np.testing.assert_allclose(got[..., cw].view(np.float32), want[..., cw].view(np.float32),
                               rtol=1e-5)
    assert (got[..., cw + 1] == 0).all()
    gc = np.stack([(got[..., :cw] >> (4 * i)) & 15 for i in range(8)])
    wc = np.stack([(want[..., :cw] >> (4 * i)) & 15 for i in range(8)])
    flips = (gc != wc).sum()
    assert flips <= gc.size // 1000, flips
    assert (np.abs(gc.astype(int) - wc.astype(int)) <= 1).all()


def assert_rows_match_source(fmt: int, got: np.ndarray, src: torch.Tensor, seed: int):
    """Cache rows (exported in the reference layout) against the reference encoder applied to
    the source rows: bit for bit, TurboQuant-4 by the reference's flip criterion."""
    want = oracle_rows(fmt, src, seed)
    if fmt == 0:
        assert_turbo_rows_close(got, want, src.shape[-1])
    else:
        np.testing.assert_array_equal(got, want)


E4M3_SWEEP_END = 0x43E08001  # f32 patterns [0, 449.0]: every |q| the FP8 encoders convert


def e4m3_thresholds() -> np.ndarray:
    """thr[c - 1] = the first non-negative f32 bit pattern whose reference E4M3 code (the
    oracle's restatement of f32_to_e4m3, candle-core/src/accel/formats.rs:288-308) is at least c,
    c = 1 .. 126, by bisection: round-to-nearest onto a monotone grid with saturation makes the
    code of a non-negative input non-decreasing in its bit pattern, so these 126 patterns give the
    code of every input in [0, 449]."""
    thr = []
    for c in range(1, 127):
        lo, hi = 0, E4M3_SWEEP_END
        while lo < hi:
            mid = (lo + hi) // 2
            if O.f32_to_e4m3(float(np.uint32(mid).view(np.float32))) >= c:
                hi = mid
            else:
                lo = mid + 1
        thr.append(lo)
    return np.array(thr, dtype=np.uint32)


FP4_SWEEP_END = 0x41000000  # f32 patterns [0, 8): every |q| the MXFP4 / NVFP4 encoders convert


def fp4_thresholds() -> np.ndarray:
    """thr[c - 1] = the first non-negative f32 bit pattern whose reference E2M1 code (the oracle's
    f32_to_fp4, candle-core/src/accel/formats.rs:329-350) is at least c, c = 1 .. 7."""
    thr = []
    for c in range(1, 8):
        lo, hi = 0, FP4_SWEEP_END
        while lo < hi:
            mid = (lo + hi) // 2
            if O.f32_to_fp4(float(np.uint32(mid).view(np.float32))) >= c:
                hi = mid
            else:
                lo = mid + 1
        thr.append(lo)
    return np.array(thr, dtype=np.uint32)
