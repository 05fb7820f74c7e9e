"""Empty inputs on the GPU, as the reference's accelerated attention treats them
(candle-core/src/rocm_backend/accel.rs:87, 197, 481: no output rows return an empty output
before any launch) and as its CPU flash path writes them (candle-nn/src/attention/cpu_flash/
varlen.rs:216-219: a query with no keys is a zero row).

  * no keys (kv_len 0) with queries: every output row is zero, for each dtype pair, the decode
    shape (q_len 1) and the prefill shape, and for E4M3 K / V;
  * no queries (q_len 0) with K / V and a cache: nothing is written to `out`, and the cache
    append still runs, bit for bit as the plain append of the same rows;
  * batch 0 and q_len 0 decodes return at once, leaving `out` as it was."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

DT = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}
PAIRS = [("bf16", "bf16"), ("f16", "f16"), ("f32", "f32"), ("f32", "bf16"), ("f32", "f16")]


@pytest.mark.parametrize("q_dt,kv_dt", PAIRS)
@pytest.mark.parametrize("lq,d", [(1, 128), (40, 128), (300, 64), (17, 256)])
def test_no_keys_give_zero_rows(cq, dev, q_dt, kv_dt, lq, d):
    b, hq, hkv = 2, 8, 2
    q = torch.randn(b, lq, hq, d, device=dev).to(DT[q_dt])
    k = torch.empty(b, 0, hkv, d, device=dev, dtype=DT[kv_dt])
    out = torch.full_like(q, 7.0)
    cq.flash_attn(q, k, k, d ** -0.5, True, out=out)
    torch.cuda.synchronize()
    assert (out == 0).all()


@pytest.mark.parametrize("q_dt", ["bf16", "f16", "f32"])
def test_no_fp8_keys_give_zero_rows(cq, dev, q_dt):
    b, lq, hq, hkv, d = 1, 33, 4, 4, 128
    q = torch.randn(b, lq, hq, d, device=dev).to(DT[q_dt])
    k8 = torch.empty(b, 0, hkv, d, device=dev, dtype=torch.uint8)
    out = torch.full_like(q, 7.0)
    cq.flash_attn_fp8_codes(q, k8, k8, d ** -0.5, False, 2.0, 3.0, out=out)
    torch.cuda.synchronize()
    assert (out == 0).all()


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_no_queries_still_append_the_cache(cq, dev, dtype):
    b, lk, hkv, d, cap, pos = 2, 45, 2, 128, 64, 3
    k = torch.randn(b, lk, hkv, d, device=dev).to(DT[dtype])
    v = torch.randn(b, lk, hkv, d, device=dev).to(DT[dtype])
    q = torch.empty(b, 0, 8, d, device=dev, dtype=DT[dtype])
    sides = [cq.CacheSide.empty(cq.FP8, iv, b, hkv, d, cap, dev) for iv in (False, True)]
    out = cq.flash_attn(q, k, v, d ** -0.5, True, k_cache=sides[0], v_cache=sides[1],
                        position=pos)
    assert out.shape == q.shape
    want = [cq.CacheSide.empty(cq.FP8, iv, b, hkv, d, cap, dev) for iv in (False, True)]
    cq.quant_append(want[0], k.transpose(1, 2), pos)
    cq.quant_append(want[1], v.transpose(1, 2), pos)
    torch.cuda.synchronize()
    for got, ref in zip(sides, want):
        np.testing.assert_array_equal(cq.rows_export(got, cap).cpu().numpy(),
                                      cq.rows_export(ref, cap).cpu().numpy())


def test_empty_decodes_return_at_once(cq, dev):
    b, hkv, d, cap = 2, 2, 128, 64
    k = cq.CacheSide.empty(cq.FP8, False, b, hkv, d, cap, dev)
    v = cq.CacheSide.empty(cq.FP8, True, b, hkv, d, cap, dev)
    q = torch.empty(b, 8, 0, d, device=dev, dtype=torch.bfloat16)
    assert cq.decode_attention(q, k, v, 10, 0.1).shape == q.shape
    kb = torch.empty(2, hkv, 16, d, device=dev, dtype=torch.bfloat16)
    out = cq.flash_attn_blocks(q, [(kb, kb, 16)], 0.1)
    assert out.shape == q.shape
    q0 = torch.empty(0, 0, 8, d, device=dev, dtype=torch.bfloat16)  # (batch, q_len, heads, D)
    k0 = torch.empty(0, 0, hkv, d, device=dev, dtype=torch.bfloat16)
    assert cq.flash_attn(q0, k0, k0, 0.1, True).shape == q0.shape
    torch.cuda.synchronize()
