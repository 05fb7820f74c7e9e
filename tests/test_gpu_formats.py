"""GPU parity of cache configurations beyond one format per cache: a Hadamard rotation on sides of
every format, key and value sides in different formats, and a cache that grows.

The reference builds them through TurboKvCache::with_formats(key, value, dim, rotation, seed, ..)
(candle-nn/src/turbo_quant.rs:858-879): TurboQuantizer::new per side with the same RotationKind
(Auto: Hadamard at power-of-two head dims), seeds `seed` and `seed + 2`; its fused decode rotates
the queries with the key rotation and unrotates the output with the value rotation
(turbo_quant.rs:1143-1264). Cache::append grows by max(grow_by, capacity / 2) and copies the
rows so far (candle-nn/src/kv_cache.rs:56-99).

Rows of rotated sides: the reference's encoder applied to the source rotated by the oracle,
within the reference's TurboQuant flip criterion (its rotation is an f32 matmul whose summation
order it leaves open). Attention: against the reference CPU path on the codes the GPU wrote,
by the criterion of rotated caches (helpers.assert_decode_parity)."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import (assert_close_bf16, assert_decode_parity, assert_rotated_rows_close,
                           assert_turbo_rows_close, exact_decode, exact_scores, kv_source,
                           oracle_decode, oracle_rows, rotates)

pytestmark = pytest.mark.gpu

FMTS = {"fp8": 5, "mxfp4": 2, "turbo4": 0, "nvfp4": 3, "mxfp8": 4}
ROT_DEFAULT, ROT_NONE, ROT_HADAMARD = 0, 1, 2


def export_np(cq, side, tokens, position=0):
    return cq.rows_export(side, tokens, position).cpu().numpy().view(np.uint32)


# ---------------------------------------------------------------------------------------------
# appends into rotated sides
# ---------------------------------------------------------------------------------------------
@pytest.mark.parametrize("fmt", ["fp8", "mxfp4", "mxfp8", "nvfp4"])
@pytest.mark.parametrize("is_value", [False, True])
@pytest.mark.parametrize("d", [64, 128])
def test_append_rotated_rows(cq, dev, fmt, is_value, d):
    f = FMTS[fmt]
    b, h, t, pos = 2, 3, 37, 5
    x = kv_source(21 + d, (b, h, t, d), outliers=True)
    x[0, 0, 0, :] = 0.0  # an all-zero row stays zero after the rotation
    seed = 44 if is_value else 42
    side = cq.CacheSide.empty(f, is_value, b, h, d, 64, dev, seed=seed, rotation=ROT_HADAMARD)
    cq.quant_append(side, x.to(dev), pos)
    torch.cuda.synchronize()
    got = export_np(cq, side, t, pos)
    assert_rotated_rows_close(f, got, oracle_rows(f, x, seed, ROT_HADAMARD), d)
    # the seed selects the rotation: the rows of another seed fail the same criterion
    with pytest.raises(AssertionError):
        assert_rotated_rows_close(f, got, oracle_rows(f, x, seed + 1, ROT_HADAMARD), d)


@pytest.mark.parametrize("is_value", [False, True])
def test_append_unrotated_turbo4(cq, dev, is_value):
    """TurboMse with RotationKind::None: the codebook applied to the rows as they are."""
    b, h, t, d = 2, 2, 33, 128
    x = kv_source(31, (b, h, t, d))
    side = cq.CacheSide.empty(0, is_value, b, h, d, 64, dev, seed=42, rotation=ROT_NONE)
    cq.quant_append(side, x.to(dev), 0)
    assert_turbo_rows_close(export_np(cq, side, t), oracle_rows(0, x, 42, ROT_NONE), d)


# ---------------------------------------------------------------------------------------------
# decode over rotated and mixed-format caches
# ---------------------------------------------------------------------------------------------
def run_cache_decode(cq, dev, kf, vf, rotation, b=2, hq=8, hkv=2, d=128, ctx=700, lq=1,
                     splits=0, kv_lens=None, wl=-1, wr=-1, seed=0, cap=None,
                     out_dtype=torch.bfloat16):
    k_fmt, v_fmt = FMTS[kf], FMTS[vf]
    q = kv_source(seed + 1, (b, hq, lq, d))
    k = kv_source(seed + 2, (b, hkv, ctx, d), outliers=True)
    v = kv_source(seed + 3, (b, hkv, ctx, d), outliers=True)
    cache = cq.TurboKvCache(k_fmt, v_fmt, b, hkv, d, cap or ctx, device=dev, rotation=rotation)
    cache.append(k.to(dev), v.to(dev))
    scale = 1.0 / d ** 0.5
    lens_t = None if kv_lens is None else torch.tensor(kv_lens, dtype=torch.int32, device=dev)
    out = torch.empty((b, hq, lq, d), dtype=out_dtype, device=dev)
    got = cq.decode_attention(q.to(dev), cache.k, cache.v, ctx, scale, kv_lens=lens_t,
                              window_left=wl, window_right=wr, splits=splits, out=out)
    torch.cuda.synchronize()
    # the codes the GPU wrote (rotated codes may sit one step from the oracle's, as the append
    # tests allow), checked against the source rows here as well
    kr, vr = export_np(cq, cache.k, ctx), export_np(cq, cache.v, ctx)
    for f, rows, src, s in ((k_fmt, kr, k, 42), (v_fmt, vr, v, 44)):
        want_rows = oracle_rows(f, src, s, rotation)
        if rotates(f, rotation) or f == 0:  # TurboQuant: the flip criterion in any case
            assert_rotated_rows_close(f, rows, want_rows, d)
        else:
            np.testing.assert_array_equal(rows, want_rows)
    lens = None if kv_lens is None else np.array(kv_lens, np.int32)
    kw = dict(kv_lens=lens, wl=wl, wr=wr, v_fmt=v_fmt, rotation=rotation)
    want = oracle_decode(k_fmt, q, kr, vr, ctx, scale, **kw)
    exact = exact_decode(k_fmt, q, kr, vr, ctx, scale, **kw)
    got = got.float().cpu().numpy()
    rotated = rotates(k_fmt, rotation) or rotates(v_fmt, rotation) or exact_scores(k_fmt)
    assert_decode_parity(k_fmt, got, want, exact, rotated=rotated, value_bf16=v_fmt != 0)
    return got


@pytest.mark.parametrize("fmt", ["fp8", "mxfp4", "mxfp8", "nvfp4", "turbo4"])
@pytest.mark.parametrize("splits", [1, 0])
def test_decode_hadamard_every_format(cq, dev, fmt, splits):
    """RotationKind::Hadamard on both sides (the reference's Auto at D = 128): queries rotated
    with the key rotation in the kernel, outputs unrotated with the value rotation, in the
    single-split epilogue or in the combine."""
    run_cache_decode(cq, dev, fmt, fmt, ROT_HADAMARD, splits=splits)


@pytest.mark.parametrize("fmt", ["fp8", "mxfp4"])
def test_decode_hadamard_d64_windows(cq, dev, fmt):
    run_cache_decode(cq, dev, fmt, fmt, ROT_HADAMARD, d=64, ctx=300, lq=3, wl=40, wr=0)


def test_decode_unrotated_turbo4(cq, dev):
    run_cache_decode(cq, dev, "turbo4", "turbo4", ROT_NONE)


MIXED = [("fp8", "mxfp4"), ("mxfp4", "fp8"), ("turbo4", "fp8"), ("fp8", "turbo4"),
         ("nvfp4", "mxfp8"), ("mxfp8", "turbo4"), ("turbo4", "mxfp4"), ("mxfp4", "nvfp4")]


@pytest.mark.parametrize("kf,vf", MIXED)
def test_decode_mixed_formats(cq, dev, kf, vf):
    """Keys and values in different formats (TurboKvCache::with_formats(key, value, ..)), the
    TurboQuant side rotated by default."""
    run_cache_decode(cq, dev, kf, vf, ROT_DEFAULT)


@pytest.mark.parametrize("kf,vf", [("fp8", "mxfp4"), ("turbo4", "nvfp4")])
def test_decode_mixed_formats_ragged_windows(cq, dev, kf, vf):
    """f32 outputs: the one-key sequence returns its value row (outlier channels up to ~25, where
    a bf16 output alone rounds by up to 6e-2)."""
    run_cache_decode(cq, dev, kf, vf, ROT_HADAMARD, b=4, lq=2, ctx=600, kv_lens=[600, 1, 0, 257],
                     cap=640, wl=100, wr=0, out_dtype=torch.float32)


@pytest.mark.parametrize("kf,vf", [("mxfp4", "fp8"), ("fp8", "fp8")])
def test_decode_paged_mixed_rotated(cq, dev, kf, vf):
    """The paged entry point over blocks of mixed-format, Hadamard-rotated sides equals the dense
    call over the same rows."""
    k_fmt, v_fmt = FMTS[kf], FMTS[vf]
    b, hq, hkv, d, n1, n2 = 2, 8, 2, 128, 300, 170
    q = kv_source(71, (b, hq, 1, d)).to(dev)
    k, v = kv_source(72, (b, hkv, n1 + n2, d)), kv_source(73, (b, hkv, n1 + n2, d))
    dense = cq.TurboKvCache(k_fmt, v_fmt, b, hkv, d, n1 + n2, device=dev,
                            rotation=ROT_HADAMARD)
    dense.append(k.to(dev), v.to(dev))
    f32 = torch.float32
    want = cq.decode_attention(q, dense.k, dense.v, n1 + n2, 0.1, splits=1,
                               out=torch.empty(q.shape, dtype=f32, device=dev))
    blocks = []
    for off, n in ((0, n1), (n1, n2)):
        kc = cq.CacheSide.empty(k_fmt, False, b, hkv, d, 320, dev, seed=42,
                                rotation=ROT_HADAMARD)
        vc = cq.CacheSide.empty(v_fmt, True, b, hkv, d, 320, dev, seed=44,
                                rotation=ROT_HADAMARD)
        cq.quant_append(kc, k[:, :, off:off + n].to(dev), 0)
        cq.quant_append(vc, v[:, :, off:off + n].to(dev), 0)
        blocks.append((kc, vc, n))
    got = cq.decode_attention_paged(q, blocks, 0.1, out=torch.empty(q.shape, dtype=f32,
                                                                     device=dev))
    torch.cuda.synchronize()
    np.testing.assert_allclose(got.cpu().numpy(), want.cpu().numpy(), atol=1e-5, rtol=1e-4)
    # blocks whose rotations differ are refused
    kx = cq.CacheSide.empty(k_fmt, False, b, hkv, d, 320, dev, seed=42, rotation=ROT_NONE)
    with pytest.raises(cq.CqkvError):
        cq.decode_attention_paged(q, [blocks[0], (kx, blocks[1][1], n2)], 0.1)


# ---------------------------------------------------------------------------------------------
# fused RoPE + append and the prefill's append into rotated / mixed sides
# ---------------------------------------------------------------------------------------------
@pytest.mark.parametrize("kf,vf,rotation", [("fp8", "mxfp4", ROT_DEFAULT),
                                            ("mxfp8", "mxfp8", ROT_HADAMARD),
                                            ("nvfp4", "turbo4", ROT_HADAMARD)])
def test_rope_append_rotated_and_mixed(cq, dev, kf, vf, rotation):
    """One fused launch (values of another format: a second launch for them) equals rope in the
    dtype followed by two plain appends, bit for bit, on the same rotated inputs."""
    k_fmt, v_fmt = FMTS[kf], FMTS[vf]
    b, hq, hkv, t, d, pos, cap = 2, 8, 2, 19, 128, 5, 64
    qkv = kv_source(81, (b, t, 1, (hq + 2 * hkv) * d))[:, :, 0].to(dev)
    q, k, v = cq.split_qkv(qkv, hq, hkv)
    inv = 1.0 / 10000.0 ** (np.arange(0, d, 2, dtype=np.float64) / d)
    ang = np.arange(pos + t + 3, dtype=np.float64)[:, None] * inv[None, :]
    cos = torch.from_numpy(np.cos(ang).astype(np.float32)).to(torch.bfloat16)
    sin = torch.from_numpy(np.sin(ang).astype(np.float32)).to(torch.bfloat16)

    def sides():
        return (cq.CacheSide.empty(k_fmt, False, b, hkv, d, cap, dev, seed=42, rotation=rotation),
                cq.CacheSide.empty(v_fmt, True, b, hkv, d, cap, dev, seed=44, rotation=rotation))
    ks, vs = sides()
    q_out = cq.rope_quant_append(ks, vs, q, k, v, cos.to(dev), sin.to(dev), cq.ROPE_HALVES, pos)
    k_rot = O.round_to(O.rope(k.float().cpu().numpy(), cos.float().numpy(), sin.float().numpy(),
                              cq.ROPE_HALVES, pos), "bf16")
    ks2, vs2 = sides()
    cq.quant_append(ks2, torch.from_numpy(k_rot).to(torch.bfloat16).to(dev), pos)
    cq.quant_append(vs2, v, pos)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(export_np(cq, ks, cap), export_np(cq, ks2, cap))
    np.testing.assert_array_equal(export_np(cq, vs, cap), export_np(cq, vs2, cap))
    want_q = O.round_to(O.rope(q.float().cpu().numpy(), cos.float().numpy(), sin.float().numpy(),
                               cq.ROPE_HALVES, pos), "bf16")
    np.testing.assert_array_equal(q_out.float().cpu().numpy(), want_q)


@pytest.mark.parametrize("kf,vf,rotation", [("fp8", "fp8", ROT_HADAMARD),
                                            ("mxfp4", "fp8", ROT_DEFAULT)])
def test_prefill_append_rotated_and_mixed(cq, dev, kf, vf, rotation):
    """flash_attn with cache sides that the pre-pass does not encode (rotated, or not FP8):
    the attention is unchanged and the sides hold what cqkv_quant_append writes."""
    k_fmt, v_fmt = FMTS[kf], FMTS[vf]
    b, s, hq, hkv, d, pos, cap = 2, 150, 8, 2, 128, 16, 192
    q = kv_source(91, (b, s, hq, d)).to(dev)
    k = kv_source(92, (b, s, hkv, d)).to(dev)
    v = kv_source(93, (b, s, hkv, d)).to(dev)

    def sides():
        return (cq.CacheSide.empty(k_fmt, False, b, hkv, d, cap, dev, seed=42, rotation=rotation),
                cq.CacheSide.empty(v_fmt, True, b, hkv, d, cap, dev, seed=44, rotation=rotation))
    kc, vc = sides()
    got = cq.flash_attn(q, k, v, 0.1, True, k_cache=kc, v_cache=vc, position=pos)
    plain = cq.flash_attn(q, k, v, 0.1, True)
    kc2, vc2 = sides()
    cq.quant_append(kc2, k.transpose(1, 2), pos)
    cq.quant_append(vc2, v.transpose(1, 2), pos)
    torch.cuda.synchronize()
    assert torch.equal(got, plain)
    np.testing.assert_array_equal(export_np(cq, kc, s, pos), export_np(cq, kc2, s, pos))
    np.testing.assert_array_equal(export_np(cq, vc, s, pos), export_np(cq, vc2, s, pos))


# ---------------------------------------------------------------------------------------------
# cache growth
# ---------------------------------------------------------------------------------------------
@pytest.mark.parametrize("kf,vf,rotation", [("fp8", "fp8", ROT_DEFAULT),
                                            ("nvfp4", "turbo4", ROT_DEFAULT),
                                            ("mxfp4", "mxfp8", ROT_HADAMARD)])
def test_cache_growth_matches_one_large_cache(cq, dev, kf, vf, rotation):
    """Appends past the capacity regrow the sides as Cache::append does (capacity 32, grow_by 16:
    32 -> 64 -> 96 -> 160) and leave every row and every attention output as one cache of the
    final size holds them, bit for bit."""
    k_fmt, v_fmt = FMTS[kf], FMTS[vf]
    b, hkv, hq, d = 2, 2, 8, 128
    chunks = [20, 27, 33, 57]
    n = sum(chunks)
    k, v = kv_source(101, (b, hkv, n, d)), kv_source(102, (b, hkv, n, d))
    q = kv_source(103, (b, hq, 1, d)).to(dev)
    grown = cq.TurboKvCache(k_fmt, v_fmt, b, hkv, d, 32, device=dev, grow_by=16,
                            rotation=rotation)
    big = cq.TurboKvCache(k_fmt, v_fmt, b, hkv, d, 256, device=dev, rotation=rotation)
    caps, off = [], 0
    for c in chunks:
        grown.append(k[:, :, off:off + c].to(dev), v[:, :, off:off + c].to(dev))
        big.append(k[:, :, off:off + c].to(dev), v[:, :, off:off + c].to(dev))
        off += c
        caps.append(grown.k.capacity)
        np.testing.assert_array_equal(
            grown.attention(q, 0.1).float().cpu().numpy(),
            big.attention(q, 0.1).float().cpu().numpy())
    assert caps == [32, 64, 96, 160], caps
    assert grown.seq_len() == n
    np.testing.assert_array_equal(export_np(cq, grown.k, n), export_np(cq, big.k, n))
    np.testing.assert_array_equal(export_np(cq, grown.v, n), export_np(cq, big.v, n))
