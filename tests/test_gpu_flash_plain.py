"""GPU parity of the plain-dtype flash attention (csrc/flash_plain.h): f16 inputs, head dims
other than 128 (any multiple of 8 up to the reference's FA_MAX_HEAD_DIM = 256), decode-shaped
calls (the reference's row kernels fa_row_* / fa_rowg_* with split-K and combine,
candle-core/kernels/flash_attn_impl.h:49-328) and the paged form over blocks of plain K / V
(flash_attn_blocks, candle-nn/src/flash_attn.rs:719-765; fa_rowp_*).

The oracle is the reference CPU path restated (candle-nn/src/flash_attn.rs:930-1000: inputs to
f32, q k^T, scale, mask, softmax, p v, output rounded to the input dtype). Tolerance: max-abs
2e-2 / mean-abs 2e-3 on the outputs (the BASELINE bar for bf16; f16 outputs are held to the
same)."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import assert_close_bf16

pytestmark = pytest.mark.gpu

DT = {"bf16": torch.bfloat16, "f16": torch.float16}


def randn(seed, shape, dtype, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(DT[dtype])


def oracle_bshd(q, k, v, scale, wl=-1, wr=-1, softcap=0.0, slopes=None, dtype="bf16"):
    """q (b, sq, hq, d), k / v (b, sk, hkv, d) -> the reference path's output in the dtype."""
    out = []
    for bi in range(q.shape[0]):
        qf = q[bi:bi + 1].float().permute(0, 2, 1, 3).contiguous().numpy()
        kf = k[bi:bi + 1].float().permute(0, 2, 1, 3).contiguous().numpy()
        vf = v[bi:bi + 1].float().permute(0, 2, 1, 3).contiguous().numpy()
        al = None
        if slopes is not None:
            al = slopes.numpy() if slopes.dim() == 1 else slopes[bi].numpy()
        o = O.attention_unfused(qf, kf, vf, scale, softcap=softcap, wl=wl, wr=wr, alibi=al,
                                threads=16)
        out.append(O.round_to(o, dtype).transpose(0, 2, 1, 3))
    return np.concatenate(out, axis=0)


def run(cq, dev, dtype, b, sq, sk, hq, hkv, d, causal=True, wl=-1, wr=-1, softcap=0.0,
        slopes=None, seed=0, qscale=1.0):
    q = randn(seed + 1, (b, sq, hq, d), dtype, qscale)
    k = randn(seed + 2, (b, sk, hkv, d), dtype)
    v = randn(seed + 3, (b, sk, hkv, d), dtype)
    scale = 1.0 / d ** 0.5
    got = cq.flash_attn(q.to(dev), k.to(dev), v.to(dev), scale, causal, window_left=wl,
                        window_right=wr, softcap=softcap,
                        alibi_slopes=None if slopes is None else slopes.to(dev))
    torch.cuda.synchronize()
    want = oracle_bshd(q, k, v, scale, wl, 0 if causal else wr, softcap, slopes, dtype)
    return got.float().cpu().numpy(), want


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("d", [64, 80, 128, 256])
def test_prefill_head_dims_and_f16(cq, dev, dtype, d):
    got, want = run(cq, dev, dtype, 2, 150, 150, 8, 2, d)
    assert_close_bf16(got, want)


@pytest.mark.parametrize("hq,hkv", [(12, 2), (8, 8), (28, 4)])
@pytest.mark.parametrize("d", [128, 256])
def test_f16_gqa_groups(cq, dev, hq, hkv, d):
    """Groups that are not a multiple of the workgroup's heads (4 at D = 128, 2 at D = 256) leave
    spare wavefronts that only copy and wait."""
    got, want = run(cq, dev, "f16", 1, 77, 200, hq, hkv, d, causal=True)
    assert_close_bf16(got, want)


@pytest.mark.parametrize("sq,sk,causal,wl,wr", [(1, 333, True, -1, -1), (3, 1000, True, 100, -1),
                                                (16, 4100, True, -1, -1), (2, 64, False, -1, -1),
                                                (70, 50, True, -1, -1), (40, 300, False, 20, 3)])
@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_decode_shapes_and_masks(cq, dev, sq, sk, causal, wl, wr, dtype):
    """q_len <= 16 always takes the split-K row kernel (bf16 at head dim 128 included)."""
    got, want = run(cq, dev, dtype, 2, sq, sk, 8, 2, 128, causal=causal, wl=wl, wr=wr)
    assert_close_bf16(got, want)
    if causal and sq > sk:  # more queries than keys: the first sq - sk see no key
        assert (got[:, :sq - sk] == 0).all()


def test_decode_long_context_many_splits(cq, dev):
    """ctx 20000, one query, group 8: the keys split across many workgroups and merge in the
    combine."""
    got, want = run(cq, dev, "bf16", 1, 1, 20000, 32, 4, 128, causal=True, seed=5)
    assert_close_bf16(got, want)


@pytest.mark.parametrize("softcap,per_batch", [(4.0, False), (0.0, True), (2.5, True)])
def test_softcap_alibi_plain(cq, dev, softcap, per_batch):
    b, hq = 2, 8
    slopes = (0.03 * (1 + torch.arange(b * hq, dtype=torch.float32))).reshape(b, hq)
    if not per_batch:
        slopes = slopes[0].contiguous()
    got, want = run(cq, dev, "f16", b, 60, 180, hq, 2, 64, causal=False, wl=50, wr=10,
                    softcap=softcap, slopes=slopes, qscale=3.0)
    assert_close_bf16(got, want)


def test_varlen_f16_d64(cq, dev):
    """Variable-length batches on the plain kernel: per sequence against the oracle and against
    the dense call, bit for bit."""
    lens_q, lens_k = [50, 0, 1, 90], [60, 30, 1, 200]
    hq, hkv, d = 8, 2, 64
    cu_q = np.concatenate([[0], np.cumsum(lens_q)]).astype(np.int32)
    cu_k = np.concatenate([[0], np.cumsum(lens_k)]).astype(np.int32)
    q = randn(61, (int(cu_q[-1]), hq, d), "f16")
    k = randn(62, (int(cu_k[-1]), hkv, d), "f16")
    v = randn(63, (int(cu_k[-1]), hkv, d), "f16")
    got = cq.flash_attn_varlen(q.to(dev), k.to(dev), v.to(dev),
                               torch.from_numpy(cu_q).to(dev), torch.from_numpy(cu_k).to(dev),
                               max(lens_q), max(lens_k), 0.125, True).float().cpu().numpy()
    for i, (lq, lk) in enumerate(zip(lens_q, lens_k)):
        if lq == 0:
            continue
        qs, ks = slice(cu_q[i], cu_q[i + 1]), slice(cu_k[i], cu_k[i + 1])
        want = oracle_bshd(q[qs][None], k[ks][None], v[ks][None], 0.125, -1, 0, dtype="f16")[0]
        assert_close_bf16(got[qs], want)
        dense = cq.flash_attn(q[qs][None].to(dev), k[ks][None].to(dev), v[ks][None].to(dev),
                              0.125, True)
        np.testing.assert_array_equal(got[qs], dense[0].float().cpu().numpy())


def test_unaligned_q_takes_plain_kernel(cq, dev):
    """A q view whose rows are not 16-byte aligned (bf16, head dim 128, a prefill shape) runs the
    plain kernel instead of the MFMA prefill, with the same results."""
    b, s, hq, hkv, d = 1, 100, 4, 2, 128
    base = randn(71, (b * s * hq * d + 1,), "bf16")
    q = base[1:].view(b, s, hq, d)
    k = randn(72, (b, s, hkv, d), "bf16")
    v = randn(73, (b, s, hkv, d), "bf16")
    got = cq.flash_attn(q.to(dev), k.to(dev), v.to(dev), 0.1, True)
    assert got.data_ptr() % 16 == 0
    want = oracle_bshd(q, k, v, 0.1, -1, 0)
    assert_close_bf16(got.float().cpu().numpy(), want)


def test_explicit_workspace_matches_allocated(cq, dev):
    b, sq, sk, hq, hkv, d = 2, 4, 3000, 8, 2, 128
    q = randn(81, (b, sq, hq, d), "f16").to(dev)
    k = randn(82, (b, sk, hkv, d), "f16").to(dev)
    v = randn(83, (b, sk, hkv, d), "f16").to(dev)
    n = cq.flash_attn_workspace_bytes(torch.float16, b, sq, sk, hq, hkv, d)
    assert n > 0
    ws = torch.empty(n, dtype=torch.uint8, device=dev)
    a = cq.flash_attn(q, k, v, 0.1, True, workspace=ws)
    bb = cq.flash_attn(q, k, v, 0.1, True)
    assert torch.equal(a, bb)
    with pytest.raises(cq.CqkvError):
        cq.flash_attn(q, k, v, 0.1, True, workspace=ws[:n // 2])


def test_refused_inputs(cq, dev):
    q = randn(91, (1, 8, 4, 128), "bf16").to(dev)
    with pytest.raises(cq.CqkvError):  # f32 K / V under bf16 queries (f32 queries take them)
        cq.flash_attn(q, q.float(), q.float(), 0.1, True)
    with pytest.raises(cq.CqkvError):  # mixed dtypes
        cq.flash_attn(q, q.half(), q, 0.1, True)
    with pytest.raises(cq.CqkvError):  # head dim not contiguous
        t = torch.zeros(1, 128, 4, 8, dtype=torch.bfloat16, device=dev).transpose(1, 3)
        cq.flash_attn(t, q, q, 0.1, True)
    with pytest.raises(cq.CqkvError):  # a head dim the kernels do not take
        x = torch.zeros(1, 8, 4, 100, dtype=torch.bfloat16, device=dev)
        cq.flash_attn(x, x, x, 0.1, True)


def test_f16_prefill_with_cache_append(cq, dev):
    """f16 inputs with cache sides: the plain kernel's attention, then the sides hold what
    cqkv_quant_append writes from the same f16 K / V."""
    b, s, hq, hkv, d = 1, 90, 8, 2, 128
    q, k, v = (randn(100 + i, (b, s, h, d), "f16").to(dev) for i, h in enumerate((hq, hkv, hkv)))
    kc = cq.CacheSide.empty(cq.FP8, False, b, hkv, d, 128, dev)
    vc = cq.CacheSide.empty(cq.MXFP4, True, b, hkv, d, 128, dev)
    got = cq.flash_attn(q, k, v, 0.1, True, k_cache=kc, v_cache=vc, position=8)
    kc2 = cq.CacheSide.empty(cq.FP8, False, b, hkv, d, 128, dev)
    vc2 = cq.CacheSide.empty(cq.MXFP4, True, b, hkv, d, 128, dev)
    cq.quant_append(kc2, k.transpose(1, 2), 8)
    cq.quant_append(vc2, v.transpose(1, 2), 8)
    torch.cuda.synchronize()
    assert torch.equal(got, cq.flash_attn(q, k, v, 0.1, True))
    for a_, b_ in ((kc, kc2), (vc, vc2)):
        assert torch.equal(cq.rows_export(a_, s, 8), cq.rows_export(b_, s, 8))


# ---------------------------------------------------------------------------------------------
# paged blocks of plain K / V
# ---------------------------------------------------------------------------------------------
def blocks_case(dev, dtype, d, rows, b=2, hkv=2, caps=None, seed=0):
    caps = caps or [r + 16 for r in rows]
    ks, vs, bl = [], [], []
    for i, (r, c) in enumerate(zip(rows, caps)):
        k = randn(seed + 10 * i + 1, (b, hkv, c, d), dtype).to(dev)
        v = randn(seed + 10 * i + 2, (b, hkv, c, d), dtype).to(dev)
        ks.append(k[:, :, :r])
        vs.append(v[:, :, :r])
        bl.append((k, v, r))
    return bl, torch.cat(ks, 2), torch.cat(vs, 2)


@pytest.mark.parametrize("dtype,d,lq", [("bf16", 128, 1), ("f16", 128, 3), ("bf16", 64, 4),
                                        ("f16", 256, 2)])
def test_blocks_vs_concatenated_oracle(cq, dev, dtype, d, lq):
    rows = [100, 0, 37, 256, 5]
    bl, kcat, vcat = blocks_case(dev, dtype, d, rows)
    b, hq, hkv = 2, 8, 2
    q = randn(7, (b, hq, lq, d), dtype).to(dev)
    got = cq.flash_attn_blocks(q, bl, 0.1, window_right=0).float().cpu().numpy()
    want = O.round_to(O.attention_unfused(q.float().cpu().numpy(), kcat.float().cpu().numpy(),
                                          vcat.float().cpu().numpy(), 0.1, wr=0, threads=16),
                      dtype)
    assert_close_bf16(got, want)


def test_blocks_equal_dense_call(cq, dev):
    """The paged call over blocks and the dense call over their concatenation: the same
    attention up to the summation order."""
    rows = [300, 200, 500]
    bl, kcat, vcat = blocks_case(dev, "bf16", 128, rows, seed=20)
    q = randn(27, (2, 8, 2, 128), "bf16").to(dev)
    got = cq.flash_attn_blocks(q, bl, 0.1, window_left=400, window_right=0, softcap=3.0)
    dense = cq.flash_attn(q.transpose(1, 2), kcat.transpose(1, 2), vcat.transpose(1, 2), 0.1,
                          True, window_left=400, softcap=3.0)
    torch.cuda.synchronize()
    np.testing.assert_allclose(got.float().cpu().numpy(),
                               dense.transpose(1, 2).float().cpu().numpy(), atol=8e-3, rtol=0)


def test_blocks_many_segments_and_workspace(cq, dev):
    rows = [33] * 40  # 40 blocks: more than one launch of the segment table writer
    bl, kcat, vcat = blocks_case(dev, "f16", 64, rows, b=1, seed=30)
    q = randn(37, (1, 8, 1, 64), "f16").to(dev)
    got = cq.flash_attn_blocks(q, bl, 0.125).float().cpu().numpy()
    want = O.round_to(O.attention_unfused(q.float().cpu().numpy(), kcat.float().cpu().numpy(),
                                          vcat.float().cpu().numpy(), 0.125, threads=16), "f16")
    assert_close_bf16(got, want)
