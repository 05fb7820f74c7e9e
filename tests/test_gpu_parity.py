"""GPU parity of the HIP path against the CPU oracle, through the C ABI.

Cache codes and scales: bit-exact with the reference encoders (RowCodec::quantize_row,
candle-core/src/accel/turbo.rs:293-381) for FP8 and MXFP4; TurboQuant within the reference's
own end-to-end criterion (<= 0.1 % code flips, norm rtol 1e-5;
candle-core/tests/accel_kernels_host.rs:998-1027), since its rotation is a matmul whose f32
summation order the reference does not pin. Attention outputs: within max-abs 2e-2 / mean-abs
2e-3 of the reference CPU path (dequantize -> bf16 -> f32 softmax attention)."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import (assert_close_bf16, assert_decode_parity, assert_rows_match_source,
                           assert_turbo_rows_close, exact_decode, exact_scores, kv_source,
                           oracle_decode, oracle_rows)

pytestmark = pytest.mark.gpu

FMTS = {"fp8": 5, "mxfp4": 2, "turbo4": 0, "nvfp4": 3, "mxfp8": 4}


def export_np(cq, side, tokens, position=0):
    return cq.rows_export(side, tokens, position).cpu().numpy().view(np.uint32)


# ---------------------------------------------------------------------------------------------
# quantize-and-append
# ---------------------------------------------------------------------------------------------
@pytest.mark.parametrize("fmt", ["fp8", "mxfp4", "mxfp8", "nvfp4"])
@pytest.mark.parametrize("is_value", [False, True])
@pytest.mark.parametrize("d", [64, 128])
def test_append_codes_bit_exact(cq, dev, fmt, is_value, d):
    f = FMTS[fmt]
    b, h, t, pos = 2, 3, 37, 5
    x = kv_source(11 + d, (b, h, t, d), outliers=True)
    x[0, 0, 0, :] = 0.0                      # an all-zero row
    x[1, 2, 3, 7] = 3.0e4                    # a large outlier
    x[0, 1, 4, :32] = 1e-30                  # a subnormal-range block
    side = cq.CacheSide.empty(f, is_value, b, h, d, 64, dev)
    # rows already in the cache around the appended range must survive untouched
    pre = oracle_rows(f, kv_source(99, (b, h, 64, d)))
    cq.rows_import(side, torch.from_numpy(pre.view(np.int32)).to(dev), 0)
    cq.quant_append(side, x.to(dev), pos)
    got = export_np(cq, side, 64)
    want = pre.copy()
    want[:, :, pos:pos + t] = oracle_rows(f, x)
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("fmt", ["fp8", "mxfp4", "mxfp8", "nvfp4"])
@pytest.mark.parametrize("layout", ["f32", "f16", "bf16_odd_stride"])
def test_append_input_dtypes_and_strides(cq, dev, fmt, layout):
    """f32 / f16 rows (paired loads of one 8- / 4-byte word) and bf16 rows whose element pairs
    are not word-aligned (token stride 129: single-element loads) encode bit-exactly."""
    f = FMTS[fmt]
    b, h, t, d = 2, 2, 21, 128
    x = kv_source(23, (b, h, t, d), outliers=True)
    if layout == "f32":
        xin = x.float() * 1.001  # values off the bf16 grid
        xref = xin
    elif layout == "f16":
        xin = x.to(torch.float16)
        xref = xin.float()
    else:
        big = torch.zeros(b, h, t, d + 1, dtype=torch.bfloat16)
        big[..., :d] = x
        xin = big[..., :d]
        xref = x
    side = cq.CacheSide.empty(f, fmt == "fp8", b, h, d, 32, dev)
    cq.quant_append(side, xin.to(dev) if layout != "bf16_odd_stride" else big.to(dev)[..., :d])
    rows = O.quantize_rows(f, 0, xref.float().numpy())
    np.testing.assert_array_equal(export_np(cq, side, t), rows)


@pytest.mark.parametrize("is_value", [False, True])
def test_append_per_batch_positions(cq, dev, is_value):
    b, h, d = 4, 2, 128
    x = kv_source(5, (b, h, 3, d))
    pos = torch.tensor([0, 7, 30, 61], dtype=torch.int32, device=dev)
    side = cq.CacheSide.empty(5, is_value, b, h, d, 64, dev)
    cq.quant_append(side, x.to(dev), positions=pos)
    got = export_np(cq, side, 64)
    rows = oracle_rows(5, x)
    for bi, p in enumerate(pos.tolist()):
        n = min(3, 64 - p)  # positions past the capacity are skipped
        np.testing.assert_array_equal(got[bi, :, p:p + n], rows[bi, :, :n])
        mask = np.ones(64, bool)
        mask[p:p + n] = False
        assert (got[bi, :, mask] == 0).all()


@pytest.mark.parametrize("is_value", [False, True])
@pytest.mark.parametrize("d", [64, 128])
def test_append_turbo4_vs_reference_criterion(cq, dev, is_value, d):
    b, h, t = 2, 2, 200
    x = kv_source(21, (b, h, t, d), outliers=True)
    seed = 44 if is_value else 42
    side = cq.CacheSide.empty(0, is_value, b, h, d, t, dev, seed=seed)
    cq.quant_append(side, x.to(dev), 0)
    assert_turbo_rows_close(export_np(cq, side, t), oracle_rows(0, x, seed), d)


@pytest.mark.parametrize("d", [64, 128])
def test_rows_import_export_roundtrip(cq, dev, d):
    for f in FMTS.values():
        for is_value in (False, True):
            rows = oracle_rows(f, kv_source(3, (2, 2, 45, d)), 42)
            side = cq.CacheSide.empty(f, is_value, 2, 2, d, 64, dev, seed=42)
            cq.rows_import(side, torch.from_numpy(rows.view(np.int32)).to(dev), 9)
            np.testing.assert_array_equal(export_np(cq, side, 45, 9), rows)


# ---------------------------------------------------------------------------------------------
# decode attention
# ---------------------------------------------------------------------------------------------
def run_decode(cq, dev, fmt, b, hq, hkv, d, ctx, lq=1, splits=0, kv_lens=None, wl=-1, wr=-1,
               outliers=False, cap=None, seed=0, out_dtype=None):
    f = FMTS[fmt]
    cap = cap or ctx
    q = kv_source(seed + 1, (b, hq, lq, d))
    k = kv_source(seed + 2, (b, hkv, ctx, d), outliers)
    v = kv_source(seed + 3, (b, hkv, ctx, d), outliers)
    cache = cq.TurboKvCache(f, f, b, hkv, d, cap, device=dev)
    cache.append(k.to(dev), v.to(dev))
    scale = 1.0 / d ** 0.5
    lens_t = None if kv_lens is None else torch.tensor(kv_lens, dtype=torch.int32, device=dev)
    out = None if out_dtype is None else torch.empty((b, hq, lq, d), dtype=out_dtype, device=dev)
    got = cq.decode_attention(q.to(dev), cache.k, cache.v, ctx, scale, kv_lens=lens_t,
                              window_left=wl, window_right=wr, splits=splits, out=out)
    torch.cuda.synchronize()
    kr, vr = oracle_rows(f, k, 42), oracle_rows(f, v, 44)
    if f == 0:
        # TurboQuant codes may flip at codebook boundaries (<= 0.1 %, checked by the append
        # tests): check the decode on the codes the GPU wrote, as the reference separates
        # its encoder and attention checks (candle-core/tests/accel_kernels_host.rs:998-1027)
        kr, vr = export_np(cq, cache.k, ctx), export_np(cq, cache.v, ctx)
    lens_np = None if kv_lens is None else np.array(kv_lens, np.int32)
    want = oracle_decode(f, q, kr, vr, ctx, scale, kv_lens=lens_np, wl=wl, wr=wr)
    got = got.float().cpu().numpy()
    if exact_scores(f):
        exact = exact_decode(f, q, kr, vr, ctx, scale, kv_lens=lens_np, wl=wl, wr=wr)
        assert_decode_parity(f, got, want, exact)
        want = exact
    return got, want


def test_decode_fp8_config1(cq, dev):
    # batch 1, 8 / 8 heads, head_dim 64, context 512, no mask
    got, want = run_decode(cq, dev, "fp8", 1, 8, 8, 64, 512)
    assert_close_bf16(got, want)


@pytest.mark.parametrize("fmt", ["mxfp4", "turbo4", "nvfp4", "mxfp8"])
@pytest.mark.parametrize("d", [64, 128])
def test_decode_block_formats_small(cq, dev, fmt, d):
    got, want = run_decode(cq, dev, fmt, 1, 8, 8, d, 512, outliers=True)
    assert_close_bf16(got, want)


@pytest.mark.parametrize("fmt", ["fp8", "mxfp4", "turbo4", "nvfp4", "mxfp8"])
@pytest.mark.parametrize("splits", [1, 3, 0])
def test_decode_gqa_splits(cq, dev, fmt, splits):
    got, want = run_decode(cq, dev, fmt, 2, 16, 4, 128, 1000, splits=splits, outliers=True)
    assert_close_bf16(got, want)


@pytest.mark.parametrize("fmt", ["fp8", "mxfp4", "turbo4", "nvfp4", "mxfp8"])
def test_decode_split_invariance(cq, dev, fmt):
    """Changing the split count changes only the f32 summation order (the reference checks its
    dense split kernels against unsplit ones within 4e-6, candle-nn/tests/accel_rocm.rs:749-752).
    FP8 and MXFP8 carry P into the MFMA as a hi + lo pair and meet that bar; MXFP4 carries the
    block-scaled P as one bf16 operand, TurboQuant-4 the norm-scaled P and NVFP4 the token-scaled
    P as one f16 operand, so a split moves each weight by up to one bf16 (2^-9) or f16 (2^-12)
    rounding of P measured against another running maximum (outputs here are below 0.1: the f16
    rounding moves them by at most a few 1e-5)."""
    outs = [run_decode(cq, dev, fmt, 2, 8, 2, 128, 2048, splits=s, out_dtype=torch.float32)[0]
            for s in (1, 2, 7, 64)]
    atol, rtol = {"mxfp4": (2e-3, 4e-3), "turbo4": (2e-3, 4e-3), "nvfp4": (1e-4, 1e-3)}.get(fmt, (1e-5, 1e-4))
    for o in outs[1:]:
        np.testing.assert_allclose(o, outs[0], atol=atol, rtol=rtol)


@pytest.mark.parametrize("fmt", ["fp8", "mxfp4", "turbo4", "nvfp4", "mxfp8"])
def test_decode_ragged_lengths(cq, dev, fmt):
    lens = [1000, 1, 0, 33, 517]
    got, want = run_decode(cq, dev, fmt, 5, 8, 2, 128, 1000, kv_lens=lens, cap=1024)
    assert_close_bf16(got, want)
    assert (got[2] == 0).all()  # a sequence without keys gives zeros


@pytest.mark.parametrize("fmt", ["fp8", "mxfp4", "turbo4", "nvfp4", "mxfp8"])
@pytest.mark.parametrize("wl,wr", [(-1, 0), (5, 0), (40, 2), (-1, -1)])
def test_decode_multi_query_windows(cq, dev, fmt, wl, wr):
    got, want = run_decode(cq, dev, fmt, 2, 8, 2, 64, 300, lq=3, wl=wl, wr=wr)
    assert_close_bf16(got, want)


@pytest.mark.parametrize("splits", [1, 0])
def test_decode_mxfp4_masked_keys_with_huge_value_scales(cq, dev, splits):
    """Keys a window masks contribute nothing, whatever their value block scales. MXFP4 values
    enter P by adding their E8M0 codes to P's exponent fields; keys 250-258 carry values of
    magnitude 2^100 (codes near 227) and every other key 2^-20, and a causal window of 40 keys
    leaves keys 257 and 258 visible to the first query, 258 to the second and neither to the
    third. A masked key's operand has to be exactly zero here: any remnant of 2^100 weighed
    against 2^-20 values would dominate the third query's output. Checked against the oracle
    per output row, relative to the row's largest value."""
    b, hq, hkv, d, ctx, lq = 1, 8, 2, 128, 300, 3
    q = kv_source(11, (b, hq, lq, d))
    k = kv_source(12, (b, hkv, ctx, d))
    vf = kv_source(13, (b, hkv, ctx, d)).float() * 2.0 ** -20
    vf[:, :, 250:259] *= 2.0 ** 120
    v = vf.to(torch.bfloat16)
    cache = cq.TurboKvCache(2, 2, b, hkv, d, ctx, device=dev)
    cache.append(k.to(dev), v.to(dev))
    scale = 1.0 / d ** 0.5
    got = cq.decode_attention(q.to(dev), cache.k, cache.v, ctx, scale, window_left=40,
                              window_right=0, splits=splits,
                              out=torch.empty((b, hq, lq, d), dtype=torch.float32, device=dev))
    torch.cuda.synchronize()
    got = got.cpu().numpy()
    want = oracle_decode(2, q, oracle_rows(2, k, 42), oracle_rows(2, v, 44), ctx, scale, wl=40, wr=0)
    peak = np.abs(want).max(axis=-1, keepdims=True)
    assert (peak[..., 2, :] < 1e-3).all() and (peak[..., 0, :] > 1e20).all()
    ratio = (np.abs(got - want) / peak).max(axis=(0, 1, 3))  # per query
    assert (ratio < 2e-2).all(), ratio


def test_decode_f32_queries(cq, dev):
    """f32 queries (not bf16-representable) take the hi + lo query operands."""
    b, hq, hkv, d, ctx = 2, 8, 2, 128, 700
    q = torch.randn(b, hq, 1, d, generator=torch.Generator().manual_seed(3))
    k, v = kv_source(4, (b, hkv, ctx, d)), kv_source(5, (b, hkv, ctx, d))
    cache = cq.TurboKvCache(5, 5, b, hkv, d, ctx, device=dev)
    cache.append(k.to(dev), v.to(dev))
    got = cache.attention(q.to(dev), 0.1).cpu().numpy()
    kr, vr = oracle_rows(5, k), oracle_rows(5, v)
    qf = q.numpy()
    # the FP8 operands are the reference's bf16 cache values exactly (bf16(scale * e4m3)), so
    # only the query's f32 precision (hi + lo operands) and the summation order are under test
    kd = O.round_bf16(O.dequantize_rows(5, 0, d, kr))
    vd = O.round_bf16(O.dequantize_rows(5, 0, d, vr))
    want = O.attention_unfused(qf, kd, vd, 0.1)
    np.testing.assert_allclose(got, want, atol=2e-5, rtol=1e-4)


def test_decode_imported_reference_rows(cq, dev):
    """Rows in the reference layout (e.g. written by the reference's own encoder) are consumed
    after cqkv_rows_import."""
    b, hq, hkv, d, ctx = 2, 8, 2, 128, 300
    q = kv_source(7, (b, hq, 1, d))
    kr = oracle_rows(5, kv_source(8, (b, hkv, ctx, d)))
    vr = oracle_rows(5, kv_source(9, (b, hkv, ctx, d)))
    ks = cq.CacheSide.empty(5, False, b, hkv, d, 320, dev)
    vs = cq.CacheSide.empty(5, True, b, hkv, d, 320, dev)
    cq.rows_import(ks, torch.from_numpy(kr.view(np.int32)).to(dev))
    cq.rows_import(vs, torch.from_numpy(vr.view(np.int32)).to(dev))
    got = cq.decode_attention(q.to(dev), ks, vs, ctx, 0.1).float().cpu().numpy()
    assert_close_bf16(got, oracle_decode(5, q, kr, vr, ctx, 0.1))


def test_decode_every_e4m3_value_code(cq, dev):
    """All 254 non-NaN E4M3 codes through the value load path (candle-nn/tests/accel_rocm.rs
    checks every code through the reference's FP8 loaders): with a window of width one, query i
    sees exactly one key, so its output is that key's value row, code * scale, exactly."""
    d, ctx = 128, 256
    codes = np.arange(256, dtype=np.uint8)
    codes[0x7F] = codes[0xFF] = 0  # the NaN codes never come out of the encoder
    kr = np.zeros((1, 1, ctx, 34), np.uint32)
    vr = np.zeros((1, 1, ctx, 34), np.uint32)
    kr[0, 0, :, 32] = np.float32(1.0).view(np.uint32)
    vr[0, 0, :, :32] = (codes.astype(np.uint32) * 0x01010101)[:, None]
    vr[0, 0, :, 32] = np.float32(1.0).view(np.uint32)
    ks = cq.CacheSide.empty(5, False, 1, 1, d, ctx, dev)
    vs = cq.CacheSide.empty(5, True, 1, 1, d, ctx, dev)
    cq.rows_import(ks, torch.from_numpy(kr.view(np.int32)).to(dev))
    cq.rows_import(vs, torch.from_numpy(vr.view(np.int32)).to(dev))
    table = np.array([O.e4m3_to_f32(int(c)) for c in codes], np.float32)
    q = torch.ones(1, 1, 16, d, dtype=torch.bfloat16, device=dev)
    for c in range(16):  # 16 queries over the first 16 (c + 1) keys: query i sees key 16 c + i
        out = cq.decode_attention(q, ks, vs, 16 * (c + 1), 1.0, window_left=0, window_right=0,
                                  out=torch.empty(1, 1, 16, d, device=dev), splits=1)
        got = out.cpu().numpy()[0, 0]
        np.testing.assert_array_equal(got, np.repeat(table[16 * c:16 * c + 16, None], d, 1))


def full_size_case(cq, dev, fmt, b, hq, hkv, d, ctx, lens=None, check=(0,), splits=0):
    """Fills a cache of the full BASELINE shape on the GPU (torch N(0,1) bf16, 1 % x8
    outlier channels), decodes all sequences, and checks the sequences in `check` against the
    oracle's CPU path over the very codes the GPU wrote (exported as reference rows). The codes
    themselves are checked against the reference encoder applied to the source K / V for the
    first and the last sequence (the last plane of the cache) over the first and the last
    append chunk, so an indexing error at large plane offsets cannot hide behind the decode
    check."""
    f = FMTS[fmt]
    cache = cq.TurboKvCache(f, f, b, hkv, d, ctx, device=dev)
    g = torch.Generator(device=dev).manual_seed(1234)
    mask = torch.rand(hkv, d, generator=g, device=dev) < 0.01
    chunk = 4096
    last0 = (ctx - 1) // chunk * chunk
    src = {}  # (t0) -> K, V source rows of sequences 0 and b - 1
    for t0 in range(0, ctx, chunk):
        t = min(chunk, ctx - t0)
        kv = [torch.randn(b, hkv, t, d, generator=g, device=dev) for _ in range(2)]
        kv = [torch.where(mask[None, :, None, :], x * 8, x).to(torch.bfloat16) for x in kv]
        if t0 in (0, last0):
            src[t0] = [x[[0, b - 1]].cpu() for x in kv]
        cache.append(*kv)
    q = torch.randn(b, hq, 1, d, generator=g, device=dev).to(torch.bfloat16)
    lens_t = None if lens is None else torch.tensor(lens, dtype=torch.int32, device=dev)
    out = cq.decode_attention(q, cache.k, cache.v, ctx, 1.0 / d ** 0.5, kv_lens=lens_t,
                              splits=splits)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    kr = cache_rows(cq, cache.k, ctx)
    vr = cache_rows(cq, cache.v, ctx)
    for t0, (ks, vs) in src.items():
        t = ks.shape[2]
        assert_rows_match_source(f, kr[[0, b - 1], :, t0:t0 + t], ks, 42)
        assert_rows_match_source(f, vr[[0, b - 1], :, t0:t0 + t], vs, 44)
    for bi in check:
        n = ctx if lens is None else lens[bi]
        qb, kb, vb = q[bi:bi + 1].cpu(), kr[bi:bi + 1, :, :n], vr[bi:bi + 1, :, :n]
        want = oracle_decode(f, qb, kb, vb, n, 1.0 / d ** 0.5)
        # TurboQuant-4: the exact value of the codes (what the reference's fused kernel computes)
        # at the tolerance, the reference CPU path within its own deviation from it plus the
        # tolerance (assert_decode_parity); one sequence at a time to bound host memory
        exact = exact_decode(f, qb, kb, vb, n, 1.0 / d ** 0.5) if exact_scores(f) else None
        if exact is not None:
            print(f"seq {bi}: max|o| {np.abs(exact).max():.3f}, gpu-exact "
                  f"{np.abs(got[bi:bi + 1] - exact).max():.3e}, cpu path-exact "
                  f"{np.abs(want - exact).max():.3e}, gpu-cpu path "
                  f"{np.abs(got[bi:bi + 1] - want).max():.3e}")
        assert_decode_parity(f, got[bi:bi + 1], want, exact)
    assert np.isfinite(got).all()
    return got


def cache_rows(cq, side, ctx):
    return cq.rows_export(side, ctx).cpu().numpy().view(np.uint32)


def test_decode_fp8_config2_full_size(cq, dev):
    """BASELINE config 2 at its full size: B=32, 32 / 8 heads, D=128, ctx 8192, outliers;
    every sequence checked."""
    full_size_case(cq, dev, "fp8", 32, 32, 8, 128, 8192, check=range(32))


def test_decode_mxfp4_config3_full_size(cq, dev):
    """B=64, 32 / 8 heads, D=128, MXFP4, ragged lengths U[1024, 32768]."""
    rng = np.random.default_rng(3)
    lens = rng.integers(1024, 32768, size=64, endpoint=True).tolist()
    full_size_case(cq, dev, "mxfp4", 64, 32, 8, 128, 32768, lens=lens, check=(0, 1, 17, 63))


def test_decode_turbo4_config5_full_size(cq, dev):
    """B=8, 64 / 8 heads, D=128, TurboQuant-4, context 131072."""
    full_size_case(cq, dev, "turbo4", 8, 64, 8, 128, 131072, check=range(8))


@pytest.mark.parametrize("fmt", ["mxfp8", "nvfp4"])
def test_decode_block_formats_config2_shape_full_size(cq, dev, fmt):
    """MXFP8 / NVFP4 caches at the config-2 shape (32 sequences x 8192 keys, 32 / 8 heads)."""
    full_size_case(cq, dev, fmt, 32, 32, 8, 128, 8192, check=(0, 31))


GOLD = __import__("os").path.join(__import__("os").path.dirname(__file__), "golden")


@pytest.mark.parametrize("name", ["turbo4", "mxfp4", "nvfp4", "mxfp8"])
@pytest.mark.parametrize("splits", [0, 1, 3])
def test_decode_vs_reference_fused_kernel_fixture(cq, dev, name, splits):
    """The reference's own fused decode (tq_attng4 + tq_combine on its host emulator, then the
    value unrotation; tests/golden/make_vectors.py attn_format_case) over rows the reference
    kernel encoded, with outlier channels, two queries per head: the GPU decode of the same rows
    is held to max-abs 2e-2 / mean-abs 2e-3 of it. Against the reference's CPU path (bf16-rounded
    cache) the bar adds that path's own deviation from the fused kernel, which the fixture shows
    (about 3e-2 for TurboQuant-4, below 2e-2 for the block formats)."""
    g = np.load(f"{GOLD}/ref_decode_{name}.npz")
    mode, scale = int(g["mode"]), float(g["scale"])
    kd, vd = g["kd"], g["vd"]
    b, hkv, lk, _ = kd.shape
    d = g["q"].shape[-1]
    q = torch.from_numpy(g["q"]).to(torch.bfloat16)  # the fixture's queries are bf16 values
    ks = cq.CacheSide.empty(mode, False, b, hkv, d, lk, dev, seed=42)
    vs = cq.CacheSide.empty(mode, True, b, hkv, d, lk, dev, seed=44)
    cq.rows_import(ks, torch.from_numpy(kd.view(np.int32)).to(dev))
    cq.rows_import(vs, torch.from_numpy(vd.view(np.int32)).to(dev))
    out = torch.empty(q.shape, dtype=torch.float32, device=dev)
    got = cq.decode_attention(q.to(dev), ks, vs, lk, scale, out=out, splits=splits).cpu().numpy()
    assert_close_bf16(got, g["out"])
    cpu = oracle_decode(mode, q, kd, vd, lk, scale)
    own = np.abs(cpu - g["out"]).max()
    err = np.abs(got - cpu)
    assert err.max() <= own + 2e-2 and err.mean() <= 2e-3, (err.max(), own, err.mean())


@pytest.mark.parametrize("fmt", ["fp8", "mxfp4", "turbo4", "nvfp4", "mxfp8"])
@pytest.mark.parametrize("lq,hq,hkv,wl,wr", [(10, 8, 2, -1, 0), (33, 4, 4, 20, 0), (7, 32, 8, -1, -1)])
def test_decode_more_than_16_query_columns(cq, dev, fmt, lq, hq, hkv, wl, wr):
    """q_len x group above 16 (chunked prefill / speculative decode over the cache: 40, 33 and
    28 (query, head) columns per kv head), causal and windowed, against the oracle."""
    got, want = run_decode(cq, dev, fmt, 2, hq, hkv, 128, 300, lq=lq, wl=wl, wr=wr)
    assert_close_bf16(got, want)


@pytest.mark.parametrize("splits", [1, 4])
def test_decode_many_columns_split_and_paged(cq, dev, splits):
    """64 columns (q_len 16 x group 4) with explicit splits, and the same through the paged
    entry point over two blocks: the column blocks and the splits combine as the dense call."""
    b, hq, hkv, d, n1, n2 = 1, 8, 2, 128, 200, 150
    q = kv_source(61, (b, hq, 16, d)).to(dev)
    k, v = kv_source(62, (b, hkv, n1 + n2, d)), kv_source(63, (b, hkv, n1 + n2, d))
    dense = cq.TurboKvCache(5, 5, b, hkv, d, n1 + n2, device=dev)
    dense.append(k.to(dev), v.to(dev))
    want = cq.decode_attention(q, dense.k, dense.v, n1 + n2, 0.1, window_right=0, splits=splits,
                               out=torch.empty(q.shape, dtype=torch.float32, device=dev))
    blocks = []
    for off, n in ((0, n1), (n1, n2)):
        kc = cq.CacheSide.empty(5, False, b, hkv, d, 224, dev)
        vc = cq.CacheSide.empty(5, True, b, hkv, d, 224, dev)
        cq.quant_append(kc, k[:, :, off:off + n].to(dev), 0)
        cq.quant_append(vc, v[:, :, off:off + n].to(dev), 0)
        blocks.append((kc, vc, n))
    got = cq.decode_attention_paged(q, blocks, 0.1, window_right=0,
                                    out=torch.empty(q.shape, dtype=torch.float32, device=dev))
    torch.cuda.synchronize()
    np.testing.assert_allclose(got.cpu().numpy(), want.cpu().numpy(), atol=1e-5, rtol=1e-4)
    ref = oracle_decode(5, q.cpu(), oracle_rows(5, k), oracle_rows(5, v), n1 + n2, 0.1, wr=0)
    assert_close_bf16(want.cpu().numpy(), ref)
