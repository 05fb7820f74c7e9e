"""GPU parity of the bf16 MFMA prefill (cqkv_flash_attn, the candle_flash_attn::flash_attn
entry point, candle-flash-attn/src/lib.rs:149-157) against the oracle's restatement of the
reference CPU path (candle-nn/src/flash_attn.rs:930-1000: bf16 inputs to f32, q k^T, scale,
-1e30 mask, softmax_last_dim, p v, bf16 output), and of its fused FP8 quantize-and-append
against the reference encoder (bit-exact codes and scales)."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import assert_close_bf16, oracle_rows

pytestmark = pytest.mark.gpu


def bf16_randn(seed, shape, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(torch.bfloat16)


def oracle_flash(q, k, v, scale, wl=-1, wr=-1):
    """q (b, sq, hq, d), k / v (b, sk, hkv, d) bf16 -> reference CPU output rounded to bf16."""
    qf = q.float().permute(0, 2, 1, 3).contiguous().numpy()
    kf = k.float().permute(0, 2, 1, 3).contiguous().numpy()
    vf = v.float().permute(0, 2, 1, 3).contiguous().numpy()
    out = O.attention_unfused(qf, kf, vf, scale, wl=wl, wr=wr, threads=16)
    return O.round_bf16(out).transpose(0, 2, 1, 3)


def run_flash(cq, dev, b, sq, sk, hq, hkv, d=128, causal=True, wl=-1, wr=-1, seed=0):
    q = bf16_randn(seed + 1, (b, sq, hq, d))
    k = bf16_randn(seed + 2, (b, sk, hkv, d))
    v = bf16_randn(seed + 3, (b, sk, hkv, d))
    scale = 1.0 / d ** 0.5
    got = cq.flash_attn(q.to(dev), k.to(dev), v.to(dev), scale, causal, window_left=wl,
                        window_right=wr)
    torch.cuda.synchronize()
    want = oracle_flash(q, k, v, scale, wl, 0 if causal else wr)
    return got.float().cpu().numpy(), want


@pytest.mark.parametrize("hq,hkv", [(8, 2), (4, 4), (8, 4), (16, 2), (28, 4), (20, 4), (12, 2)])
def test_prefill_causal_gqa(cq, dev, hq, hkv):
    got, want = run_flash(cq, dev, 2, 200, 200, hq, hkv)
    assert_close_bf16(got, want)


@pytest.mark.parametrize("sq,sk,causal,wl,wr", [(70, 300, True, -1, -1), (64, 64, False, -1, -1),
                                                (130, 130, True, 50, -1), (100, 257, False, 20, 3),
                                                (1, 333, True, -1, -1)])
def test_prefill_masks_and_lengths(cq, dev, sq, sk, causal, wl, wr):
    got, want = run_flash(cq, dev, 1, sq, sk, 8, 2, causal=causal, wl=wl, wr=wr)
    assert_close_bf16(got, want)


def test_prefill_rows_without_keys_are_zero(cq, dev):
    # q_len > kv_len, causal: the first q_len - kv_len queries see no key
    got, want = run_flash(cq, dev, 1, 100, 40, 4, 1)
    assert (got[0, :60] == 0).all()
    assert_close_bf16(got, want)


@pytest.mark.parametrize("pos", [37, 40, 0])
def test_prefill_fused_fp8_append(cq, dev, pos):
    """Positions that are multiples of 8 take the in-pre-pass append (150 tokens: a partial last
    8-token group keeps the cache bytes past it), others the separate append launches."""
    b, s, hq, hkv, d = 2, 150, 8, 2, 128
    q = bf16_randn(11, (b, s, hq, d))
    k = bf16_randn(12, (b, s, hkv, d))
    v = bf16_randn(13, (b, s, hkv, d))
    kc = cq.CacheSide.empty(cq.FP8, False, b, hkv, d, 256, dev)
    vc = cq.CacheSide.empty(cq.FP8, True, b, hkv, d, 256, dev)
    got = cq.flash_attn(q.to(dev), k.to(dev), v.to(dev), 0.1, True, k_cache=kc, v_cache=vc,
                        position=pos)
    torch.cuda.synchronize()
    assert_close_bf16(got.float().cpu().numpy(), oracle_flash(q, k, v, 0.1, -1, 0))
    for side, x in ((kc, k), (vc, v)):
        rows = cq.rows_export(side, s, pos).cpu().numpy().view(np.uint32)
        np.testing.assert_array_equal(rows, oracle_rows(cq.FP8, x.permute(0, 2, 1, 3)))


def test_prefill_config4_full_size_sampled_rows(cq, dev):
    """B=4, S=4096, 32 / 8 heads, D=128, causal; 96 sampled (batch, head,
    query) rows checked in float64 against softmax(q k^T / sqrt(128)) v over the bf16 inputs,
    and the fused FP8 append of all 4 x 4096 x 8 K / V rows checked bit for bit (codes and
    scales) against the reference encoder."""
    b, s, hq, hkv, d = 4, 4096, 32, 8, 128
    g = torch.Generator(device=dev).manual_seed(7)
    q = torch.randn(b, s, hq, d, generator=g, device=dev).to(torch.bfloat16)
    k = torch.randn(b, s, hkv, d, generator=g, device=dev).to(torch.bfloat16)
    v = torch.randn(b, s, hkv, d, generator=g, device=dev).to(torch.bfloat16)
    kc = cq.CacheSide.empty(cq.FP8, False, b, hkv, d, s, dev)
    vc = cq.CacheSide.empty(cq.FP8, True, b, hkv, d, s, dev)
    out = cq.flash_attn(q, k, v, 1.0 / d ** 0.5, True, k_cache=kc, v_cache=vc)
    torch.cuda.synchronize()
    rng = np.random.default_rng(0)
    picks = [(int(rng.integers(b)), int(rng.integers(hq)), int(x)) for x in
             np.concatenate([[0, 1, 63, 64, 4095], rng.integers(0, s, 91)])]
    qn, kn, vn, on = (t.float().cpu().numpy() for t in (q, k, v, out))
    got, want = [], []
    for bi, h, i in picks:
        kk = kn[bi, :i + 1, h // 4].astype(np.float64)
        vv = vn[bi, :i + 1, h // 4].astype(np.float64)
        sc = kk @ qn[bi, i, h].astype(np.float64) / np.sqrt(d)
        p = np.exp(sc - sc.max())
        want.append(O.round_bf16((p @ vv / p.sum()).astype(np.float32)))
        got.append(on[bi, i, h])
    assert_close_bf16(np.array(got), np.array(want))
    # fused append: per-row FP8 scales equal absmax / 448 of the bf16 rows, and every code of
    # every (batch, head, token) row equals the reference encoder's
    ks = kc.scales.view(torch.float32).view(b, hkv, s).cpu().numpy()
    np.testing.assert_array_equal(ks, (np.abs(kn).max(-1).transpose(0, 2, 1) / np.float32(448)))
    vs = vc.scales.view(torch.float32).view(b, hkv, s).cpu().numpy()
    np.testing.assert_array_equal(vs, (np.abs(vn).max(-1).transpose(0, 2, 1) / np.float32(448)))
    for side, x in ((kc, k), (vc, v)):
        rows = cq.rows_export(side, s).cpu().numpy().view(np.uint32)
        np.testing.assert_array_equal(rows, oracle_rows(cq.FP8, x.permute(0, 2, 1, 3).cpu()))
