"""Shared input generators and oracle wrappers of the GPU parity tests."""
from __future__ import annotations

import numpy as np
import torch

from oracle import oracle as O

BITS = {5: 0, 2: 0, 0: 4, 3: 0, 4: 0, 1: 4}  # oracle (mode, bits): FP8, MXFP4, TURBO4, NVFP4,
# MXFP8, TURBOPROD


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


def rot_kind(fmt: int, rotation: int = 0, d: int = 128):
    """The oracle rotation kind (O.ROT_HADAMARD / O.ROT_DENSE) a cache side of `fmt` uses at
    head dim d under cqkv rotation `rotation` (0 default: AUTO for the TurboQuant formats, none
    for the others; 1 none; 2 Hadamard; 3 dense; 4 auto), or None without rotation:
    RotationKind::resolve (candle-core/src/accel/config.rs:131-138) - Hadamard at power-of-two
    head dims, dense otherwise."""
    if rotation == 1 or (rotation == 0 and fmt not in (0, 1)):
        return None
    if rotation == 3:
        return O.ROT_DENSE
    return O.ROT_HADAMARD if d & (d - 1) == 0 else O.ROT_DENSE


def rotates(fmt: int, rotation: int = 0, d: int = 128) -> bool:
    """Whether a cache side of `fmt` stores rotated rows under cqkv rotation `rotation`."""
    return rot_kind(fmt, rotation, d) is not None


def side_pi(fmt: int, rotation: int, d: int, seed: int):
    """The oracle's rotation matrix of a cache side (None without rotation)."""
    k = rot_kind(fmt, rotation, d)
    return None if k is None else O.rotation_matrix(d, k, seed)


def obits(fmt: int, bits: int = 0) -> int:
    """The oracle's (mode, bits) width of a cache side of cqkv width `bits` (0: 4)."""
    return (bits or 4) if fmt in (0, 1) else BITS[fmt]


def oracle_rows(fmt: int, x: torch.Tensor, seed: int = 0, rotation: int = 0,
                bits: int = 0) -> np.ndarray:
    """Reference rows of x (.., d) bf16, rotated by the seed's Hadamard first when the side
    rotates (TurboQuantizer::quantize_rows, candle-nn/src/turbo_quant.rs:180-215); `bits` the
    TurboQuant width (0: 4)."""
    xf = x.float().numpy()
    pi = side_pi(fmt, rotation, x.shape[-1], seed)
    if pi is not None:
        xf = O.rotate_rows(pi, xf.reshape(-1, x.shape[-1])).reshape(xf.shape)
    if fmt == 1:
        return O.quantize_rows_qjl(obits(1, bits), xf, O.qjl_matrix(x.shape[-1], seed))
    return O.quantize_rows(fmt, obits(fmt, bits), xf)


def oracle_decode(fmt: int, q: torch.Tensor, k_rows: np.ndarray, v_rows: np.ndarray, lk: int,
                  scale: float, kv_lens=None, wl=-1, wr=-1, k_seed=42, v_seed=44,
                  v_fmt: int | None = None, rotation: int = 0, k_bits: int = 0,
                  v_bits: int = 0, softcap: float = 0.0, alibi=None) -> np.ndarray:
    """The reference CPU decode path (dequantize, unrotate, bf16, unfused f32 attention),
    rounded to bf16 like the reference's output; keys in `fmt`, values in `v_fmt`; softcap and
    per-head ALiBi slopes as FlashAttnConfig's."""
    d = q.shape[-1]
    v_fmt = fmt if v_fmt is None else v_fmt
    pk = side_pi(fmt, rotation, d, k_seed)
    pv = side_pi(v_fmt, rotation, d, v_seed)
    qb = O.f32_to_bf16_bits(q.float().numpy())
    sk = O.qjl_matrix(d, k_seed) if fmt == 1 else None
    out = O.cache_attention(qb, k_rows, v_rows, (fmt, obits(fmt, k_bits)),
                            (v_fmt, obits(v_fmt, v_bits)), pk, pv,
                            lk, scale, kv_lens=kv_lens, wl=wl, wr=wr, threads=16, qjl_k=sk,
                            softcap=softcap, alibi=alibi)
    return O.round_bf16(out)


def assert_close_bf16(got: np.ndarray, want: np.ndarray, max_abs=2e-2, mean_abs=2e-3):
    """The BASELINE tolerance of bf16 attention outputs."""
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    assert np.isfinite(got).all(), "non-finite output"
    assert err.max() <= max_abs and err.mean() <= mean_abs, (err.max(), err.mean())
    return err.max(), err.mean()


def exact_decode(fmt: int, q: torch.Tensor, k_rows: np.ndarray, v_rows: np.ndarray, lk: int,
                 scale: float, kv_lens=None, wl=-1, wr=-1, k_seed=42, v_seed=44,
                 v_fmt: int | None = None, rotation: int = 0, k_bits: int = 0,
                 v_bits: int = 0, softcap: float = 0.0, alibi=None) -> np.ndarray:
    """float64 attention over the dequantized (and unrotated) codes, without the reference
    path's bf16 rounding of the cache: the mathematical value both paths approximate (softcap
    and per-head ALiBi slopes as the reference's score terms)."""
    b, hq, lq, d = q.shape
    v_fmt = fmt if v_fmt is None else v_fmt
    hkv = k_rows.shape[1]
    if fmt == 1:
        kd = O.dequantize_rows_qjl(obits(1, k_bits), d, k_rows[:, :, :lk],
                                   O.qjl_matrix(d, k_seed))
        kd = kd.astype(np.float64)
    else:
        kd = O.dequantize_rows(fmt, obits(fmt, k_bits), d, k_rows[:, :, :lk]).astype(np.float64)
    vd = O.dequantize_rows(v_fmt, obits(v_fmt, v_bits), d, v_rows[:, :, :lk]).astype(np.float64)
    pk, pv = side_pi(fmt, rotation, d, k_seed), side_pi(v_fmt, rotation, d, v_seed)
    if pk is not None:
        kd = kd @ pk.astype(np.float64)
    if pv is not None:
        vd = vd @ pv.astype(np.float64)
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
                if softcap > 0:
                    s = softcap * np.tanh(s / softcap)
                if alibi is not None:
                    s = s - float(alibi[h]) * np.abs(i + n - lq - np.arange(lo, hi))
                p = np.exp(s - s.max())
                out[bi, h, i] = p @ vd[bi, h // g, lo:hi] / p.sum()
    return out


def exact_scores(fmt: int) -> bool:
    """Key formats whose decode scores are the exact value of the codes, as in the reference's
    fused kernel: TurboQuant (f16 codebook values times the f32 norm) and NVFP4 (E2M1 code times
    E4M3 block scale, exact in f16, times the f32 token scale). Their outputs are held to
    assert_decode_parity's exact-value criterion."""
    return fmt in (0, 3)


def assert_decode_parity(fmt: int, got: np.ndarray, ref: np.ndarray, exact: np.ndarray | None,
                         rotated: bool | None = None, value_bf16: bool = False):
    """FP8 / MX / NVFP4: the BASELINE tolerance against the reference path. TurboQuant: the same
    tolerance against the exact value of the same codes, and against the reference path within
    that path's own deviation from the exact value (its bf16 rounding of the unrotated cache
    alone moves outputs by up to ~4e-2 on outlier-heavy inputs) plus the tolerance. The exact
    value is what the reference's own fused kernel computes: on the committed fixture
    tests/golden/ref_decode_turbo4.npz it agrees with the exact value to 4e-6, and the
    reference's CPU path differs from it by 3.0e-2. NVFP4 keys take the same criterion: their
    scores are exact too (E2M1 code times E4M3 block scale is exact in f16, the f32 token scale
    multiplies the score), where the reference path rounds the dequantized keys to bf16 first,
    so outputs of |x| >= 4 can sit one bf16 step (0.031) from it. `rotated` (default: fmt is
    TurboQuant or NVFP4) selects the second criterion for any cache whose key or value side
    rotates: the reference path then unrotates in f32 and rounds to bf16 as for TurboQuant. `value_bf16`: the kernel
    rounds the dequantized (rotated) values to bf16 as the reference path rounds the unrotated
    ones, each a bf16 rounding at the value's magnitude (outlier channels reach |v| ~ 25, where
    one rounding is up to 6e-2): the exact value is then met within the tolerance plus 2^-8 of
    its magnitude, elementwise."""
    rotated = exact_scores(fmt) if rotated is None else rotated
    if not rotated or exact is None:
        return assert_close_bf16(got, ref)
    tol = 2e-2 + (2.0 ** -8 * np.abs(exact) if value_bf16 else 0.0)
    ex = np.abs(got.astype(np.float64) - exact)
    assert np.isfinite(got).all(), "non-finite output"
    assert (ex <= tol).all() and ex.mean() <= 2e-3, (ex.max(), (ex > tol).sum(), ex.mean())
    # against the reference path: its own deviation from the exact value plus the same allowance
    own = np.abs(ref - exact)
    err = np.abs(got.astype(np.float64) - ref)
    assert (err <= own.max() + tol).all() and err.mean() <= 2e-3, (err.max(), own.max(),
                                                                    err.mean())


def packed_codes(rows: np.ndarray, bits: int, d: int) -> np.ndarray:
    """The `bits`-bit codes of reference rows (LSB first across the code words)."""
    out = np.zeros(rows.shape[:-1] + (d,), dtype=np.int64)
    for j in range(d):
        for bit in range(bits):
            pos = bits * j + bit
            out[..., j] |= ((rows[..., pos // 32] >> (pos % 32)) & 1).astype(np.int64) << bit
    return out


def assert_turbo_rows_close(got: np.ndarray, want: np.ndarray, d: int, bits: int = 4):
    """TurboQuant (TurboMse{bits}) rows against the reference encoder's rows under the
    reference's own end-to-end criterion (candle-core/tests/accel_kernels_host.rs:998-1027):
    norms within rtol 1e-5, at most 0.1 % of the codes flipped, each flip to a neighbouring
    code."""
    cw = (d * bits + 31) // 32
    np.testing.assert_allclose(got[..., cw].view(np.float32), want[..., cw].view(np.float32),
                               rtol=1e-5)
    assert (got[..., cw + 1] == 0).all()
    gc, wc = packed_codes(got, bits, d), packed_codes(want, bits, d)
    flips = (gc != wc).sum()
    assert flips <= gc.size // 1000, flips
    assert (np.abs(gc - wc) <= 1).all()


def assert_rotated_rows_close(fmt: int, got: np.ndarray, want: np.ndarray, d: int):
    """Rows of a Hadamard-rotated FP8 / MX / NVFP4 side against the reference encoder's rows of
    the same source, by the reference's TurboQuant criterion carried over (its rotation is an f32
    matmul whose summation order it does not pin, so a code may move where the rotated value sits
    within rounding of a boundary): f32 vector scales within rtol 1e-5, block scale bytes equal
    but for <= 0.1 % of the blocks (each one step away), and in blocks of equal scale at most
    0.1 % of the element codes changed, each to a neighbouring code of the same sign-magnitude
    order."""
    if fmt == 0:
        return assert_turbo_rows_close(got, want, d)
    lay = O.row_layout(fmt, BITS[fmt], d)
    cw, aw = lay.code_words, lay.aux_words
    # rsc0: the FP8 / NVFP4 vector scale (1 for MX)
    np.testing.assert_allclose(got[..., cw + aw].view(np.float32),
                               want[..., cw + aw].view(np.float32), rtol=1e-5)
    bits = 8 if fmt in (4, 5) else 4
    per = 32 // bits

    def codes(rows):
        c = np.stack([(rows[..., :cw] >> (bits * i)) & ((1 << bits) - 1) for i in range(per)], -1)
        c = c.reshape(*rows.shape[:-1], d).astype(np.int64)
        mag, neg = c & ((1 << (bits - 1)) - 1), c >> (bits - 1)
        return np.where(neg == 1, -mag, mag)

    gc, wc = codes(got), codes(want)
    blk = {2: 32, 4: 32, 3: 16}.get(fmt, d)
    if aw:
        gs = got[..., cw:cw + aw].copy().view(np.uint8)[..., :d // blk].astype(np.int64)
        ws = want[..., cw:cw + aw].copy().view(np.uint8)[..., :d // blk].astype(np.int64)
        moved = gs != ws
        assert moved.sum() <= moved.size // 1000, moved.sum()
        assert (np.abs(gs - ws) <= 1).all()
        same = np.repeat(~moved, blk, axis=-1)
    else:
        same = np.ones(gc.shape, bool)
    flips = (gc != wc) & same
    assert flips.sum() <= gc.size // 1000, flips.sum()
    assert (np.abs(gc - wc)[same] <= 1).all()


def assert_prod_rows_close(got: np.ndarray, want: np.ndarray, d: int, bits: int = 4):
    """TurboProd{bits} rows against the reference encoder's: the (bits - 1)-bit codes and the norm by the
    TurboQuant criterion (<= 0.1 % code flips to a neighbour, norms rtol 1e-5); in rows without a
    code flip |r| within rtol 1e-4 and the QJL sign bits equal but for <= 0.1 % (a projection of
    the residual within rounding of zero; the reference leaves the matmul's summation order
    open)."""
    lay = O.row_layout(1, bits, d)
    cw, aw = lay.code_words, lay.aux_words
    gc, wc = packed_codes(got, bits - 1, d), packed_codes(want, bits - 1, d)
    flips = gc != wc
    assert flips.sum() <= gc.size // 1000, flips.sum()
    assert (np.abs(gc - wc) <= 1).all()
    np.testing.assert_allclose(got[..., cw + aw].view(np.float32),
                               want[..., cw + aw].view(np.float32), rtol=1e-5)
    clean = ~flips.any(-1)
    np.testing.assert_allclose(got[..., cw + aw + 1].view(np.float32)[clean],
                               want[..., cw + aw + 1].view(np.float32)[clean], rtol=1e-4)
    gs = np.unpackbits(got[..., cw:cw + aw].copy().view(np.uint8), axis=-1)[clean]
    ws = np.unpackbits(want[..., cw:cw + aw].copy().view(np.uint8), axis=-1)[clean]
    assert (gs != ws).sum() <= gs.size // 1000, (gs != ws).sum()


def assert_rows_match_source(fmt: int, got: np.ndarray, src: torch.Tensor, seed: int,
                             rotation: int = 0, bits: int = 0):
    """Cache rows (exported in the reference layout) against the reference encoder applied to
    the source rows: bit for bit, TurboQuant by the reference's flip criterion."""
    want = oracle_rows(fmt, src, seed, rotation, bits)
    if fmt == 1:
        assert_prod_rows_close(got, want, src.shape[-1], obits(1, bits))
    elif fmt == 0 and rotates(fmt, rotation, src.shape[-1]):
        assert_turbo_rows_close(got, want, src.shape[-1], obits(0, bits))
    elif rotates(fmt, rotation, src.shape[-1]):
        assert_rotated_rows_close(fmt, got, want, src.shape[-1])
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


# README.md:301-311 of the reference, produced by turbo_quant::accuracy::attention_error_by_format
# (candle-nn/src/turbo_quant.rs:1644-1719): (key format, value format) -> relative RMS error of
# the attention output, mean over seeds 0-5. Oracle (mode, bits).
PUBLISHED_ERRORS = [((O.FP8, 0), (O.FP8, 0), 0.036), ((O.NVFP4, 0), (O.NVFP4, 0), 0.133),
                    ((O.TURBO_MSE, 4), (O.TURBO_MSE, 4), 0.137),
                    ((O.MXFP4, 0), (O.MXFP4, 0), 0.162),
                    ((O.TURBO_PROD, 4), (O.TURBO_MSE, 4), 0.247),
                    ((O.TURBO_MSE, 3), (O.TURBO_MSE, 3), 0.253)]


def accuracy_inputs(seed: int, d: int = 128):
    """The reference test's inputs: one SplitMix64(seed * 77 + d) normal stream, as f32, filling
    k (1, 2, 256, d), then v (1, 2, 256, d), then q (1, 8, 1, d) (turbo_quant.rs:1673-1679)."""
    n = 2 * 256 * d
    x = O.normal(seed * 77 + d, (2 * n + 8 * d,))
    return (x[:n].reshape(1, 2, 256, d), x[n:2 * n].reshape(1, 2, 256, d),
            x[2 * n:].reshape(1, 8, 1, d))


def gqa_attention_f64(q, k, v, scale):
    """softmax(scale q k^T) v in float64, q (1, hq, 1, d), k / v (1, hkv, lk, d)."""
    q, k, v = (np.asarray(a, np.float64) for a in (q, k, v))
    g = q.shape[1] // k.shape[1]
    out = np.zeros_like(q)
    for h in range(q.shape[1]):
        s = k[0, h // g] @ q[0, h, 0] * scale
        p = np.exp(s - s.max())
        out[0, h, 0] = p @ v[0, h // g] / p.sum()
    return out


def relative_rms(got, exact) -> float:
    return float(np.sqrt(((got - exact) ** 2).sum() / (exact ** 2).sum()))
