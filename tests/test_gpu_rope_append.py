"""GPU parity of the fused RoPE + quantize-append (cqkv_rope_quant_append).

The reference runs the model step as separate ops: rope(q), rope(k) in the tensor dtype
(candle-nn/src/rotary_emb.rs:585-611 / 275-303, ROCm kernels candle-core/kernels/nn.hip:107-148)
then TurboKvCache::append(k, v) (candle-nn/src/turbo_quant.rs:916-945). Here that sequence is
one launch; the checks: rotated queries bit-exact with the oracle's rope rounded to the dtype;
key and value rows bit-exact with the oracle's encoders applied to those rotated keys (FP8,
MXFP4) or, for TurboQuant (whose rotation the reference leaves unpinned at the last bit), with
this library's unfused append of the same rotated keys."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import assert_turbo_rows_close, kv_source, oracle_rows

pytestmark = pytest.mark.gpu

FMTS = {"fp8": 5, "mxfp4": 2, "turbo4": 0}
TORCH = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}


def tables(rows, d, dtype):
    inv = 1.0 / 10000.0 ** (np.arange(0, d, 2, dtype=np.float64) / d)
    ang = np.arange(rows, dtype=np.float64)[:, None] * inv[None, :]
    cos = torch.from_numpy(np.cos(ang).astype(np.float32)).to(TORCH[dtype])
    sin = torch.from_numpy(np.sin(ang).astype(np.float32)).to(TORCH[dtype])
    return cos, sin


def export_np(cq, side, tokens):
    return cq.rows_export(side, tokens, 0).cpu().numpy().view(np.uint32)


def expected_rope(x, cos, sin, kind, pos, dtype):
    return O.round_to(O.rope(x.float().numpy(), cos.float().numpy(), sin.float().numpy(), kind,
                             pos), dtype)


def run_case(cq, dev, fmt, kind, d, dtype, b=2, hq=8, hkv=2, t=19, pos=5, cap=64,
             padded_out=False):
    f = FMTS[fmt]
    qkv = kv_source(7 + d + kind, (b, t, 1, (hq + 2 * hkv) * d), outliers=True)[:, :, 0]
    qkv = qkv.to(TORCH[dtype]).to(dev)
    q, k, v = cq.split_qkv(qkv, hq, hkv)  # strided views, as the models produce them
    cos, sin = tables(pos + t + 3, d, dtype)
    seed = 42
    ks = cq.CacheSide.empty(f, False, b, hkv, d, cap, dev, seed=seed)
    vs = cq.CacheSide.empty(f, True, b, hkv, d, cap, dev, seed=seed + 2)
    # rows already in the cache must survive
    pre_k = oracle_rows(f, kv_source(91, (b, hkv, cap, d)), seed)
    pre_v = oracle_rows(f, kv_source(92, (b, hkv, cap, d)), seed + 2)
    cq.rows_import(ks, torch.from_numpy(pre_k.view(np.int32)).to(dev), 0)
    cq.rows_import(vs, torch.from_numpy(pre_v.view(np.int32)).to(dev), 0)
    q_out = None
    if padded_out:  # odd row stride: the element-pair path instead of 16-byte lanes
        q_out = torch.zeros(b, hq, t, d + 1, dtype=TORCH[dtype], device=dev)[..., :d]
    q_out = cq.rope_quant_append(ks, vs, q, k, v, cos.to(dev), sin.to(dev), kind, pos,
                                 q_out=q_out)
    torch.cuda.synchronize()

    want_q = expected_rope(q.cpu(), cos, sin, kind, pos, dtype)
    np.testing.assert_array_equal(q_out.float().cpu().numpy(), want_q)
    k_rot = expected_rope(k.cpu(), cos, sin, kind, pos, dtype)
    got_k, got_v = export_np(cq, ks, cap), export_np(cq, vs, cap)
    if f != 0:
        want_k, want_v = pre_k.copy(), pre_v.copy()
        want_k[:, :, pos:pos + t] = O.quantize_rows(f, 0, k_rot)
        want_v[:, :, pos:pos + t] = O.quantize_rows(f, 0, v.float().cpu().numpy())
        np.testing.assert_array_equal(got_k, want_k)
        np.testing.assert_array_equal(got_v, want_v)
    else:  # fused == unfused append of the same rotated keys, bit for bit
        ks2 = cq.CacheSide.empty(f, False, b, hkv, d, cap, dev, seed=seed)
        vs2 = cq.CacheSide.empty(f, True, b, hkv, d, cap, dev, seed=seed + 2)
        cq.rows_import(ks2, torch.from_numpy(pre_k.view(np.int32)).to(dev), 0)
        cq.rows_import(vs2, torch.from_numpy(pre_v.view(np.int32)).to(dev), 0)
        cq.quant_append(ks2, torch.from_numpy(k_rot).to(dev), pos)
        cq.quant_append(vs2, v.float(), pos)
        np.testing.assert_array_equal(got_k, export_np(cq, ks2, cap))
        np.testing.assert_array_equal(got_v, export_np(cq, vs2, cap))
        outside = np.ones(cap, bool)
        outside[pos:pos + t] = False
        np.testing.assert_array_equal(got_k[:, :, outside], pre_k[:, :, outside])


@pytest.mark.parametrize("fmt", ["fp8", "mxfp4", "turbo4"])
@pytest.mark.parametrize("kind", [1, 2])
@pytest.mark.parametrize("d", [64, 128])
def test_rope_append_bf16(cq, dev, fmt, kind, d):
    run_case(cq, dev, fmt, kind, d, "bf16")


@pytest.mark.parametrize("dtype", ["f16", "f32"])
@pytest.mark.parametrize("kind", [1, 2])
def test_rope_append_dtypes(cq, dev, dtype, kind):
    run_case(cq, dev, "fp8", kind, 128, dtype)


@pytest.mark.parametrize("kind", [1, 2])
@pytest.mark.parametrize("d,hq,hkv", [(128, 6, 2), (64, 12, 4), (64, 4, 4)])
def test_rope_append_partial_head_groups(cq, dev, kind, d, hq, hkv):
    """Query head counts that do not fill the last 4- (D=128) or 8-head (D=64) lane group."""
    run_case(cq, dev, "fp8", kind, d, "bf16", hq=hq, hkv=hkv)


@pytest.mark.parametrize("kind", [1, 2])
def test_rope_append_padded_query_output(cq, dev, kind):
    run_case(cq, dev, "mxfp4", kind, 128, "bf16", padded_out=True)


def test_rope_append_single_token_decode_step(cq, dev):
    """The decode step: one token at position 63 (the last row of the cache)."""
    run_case(cq, dev, "fp8", 1, 128, "bf16", b=4, hq=32, hkv=8, t=1, pos=63)


def test_rope_append_per_batch_positions(cq, dev):
    """positions[b] per sequence; tokens past the capacity or the table are skipped (their
    query rows left as they were)."""
    b, hq, hkv, d, t, cap = 3, 4, 2, 128, 4, 32
    qkv = kv_source(3, (b, t, 1, (hq + 2 * hkv) * d))[:, :, 0].to(dev)
    q, k, v = cq.split_qkv(qkv, hq, hkv)
    cos, sin = tables(34, d, "bf16")  # rows 0..33
    pos = torch.tensor([0, 29, 31], dtype=torch.int32, device=dev)
    ks = cq.CacheSide.empty(5, False, b, hkv, d, cap, dev)
    vs = cq.CacheSide.empty(5, True, b, hkv, d, cap, dev)
    q_out = torch.full((b, hq, t, d), 7.0, dtype=torch.bfloat16, device=dev)
    cq.rope_quant_append(ks, vs, q, k, v, cos.to(dev), sin.to(dev), 1, positions=pos, q_out=q_out)
    torch.cuda.synchronize()
    got_k = export_np(cq, ks, cap)
    got_q = q_out.float().cpu().numpy()
    for bi, p in enumerate(pos.tolist()):
        nk = min(t, cap - p)   # keys / values: up to the capacity
        nq = min(t, 34 - p)    # queries: up to the table
        k_rot = expected_rope(k[bi:bi + 1, :, :nk].cpu(), cos, sin, 1, p, "bf16")
        np.testing.assert_array_equal(got_k[bi:bi + 1, :, p:p + nk], O.quantize_rows(5, 0, k_rot))
        q_rot = expected_rope(q[bi:bi + 1, :, :nq].cpu(), cos, sin, 1, p, "bf16")
        np.testing.assert_array_equal(got_q[bi:bi + 1, :, :nq], q_rot)
        assert (got_q[bi, :, nq:] == 7.0).all()


def test_turbo_kv_cache_rope_append_then_decode(cq, dev):
    """TurboKvCache.rope_append over two steps, then attention with the returned queries: equal
    to rope by the oracle + append + attention."""
    b, hq, hkv, d = 2, 8, 2, 128
    cache = cq.TurboKvCache(cq.FP8, cq.FP8, b, hkv, d, 64, dev)
    ref = cq.TurboKvCache(cq.FP8, cq.FP8, b, hkv, d, 64, dev)
    cos, sin = tables(64, d, "bf16")
    cd, sd = cos.to(dev), sin.to(dev)
    for step, t in enumerate((9, 1)):
        qkv = kv_source(50 + step, (b, t, 1, (hq + 2 * hkv) * d))[:, :, 0].to(dev)
        q, k, v = cq.split_qkv(qkv, hq, hkv)
        p = cache.seq_len()
        qr = cache.rope_append(q, k, v, cd, sd)
        qr_ref = torch.from_numpy(expected_rope(q.cpu(), cos, sin, 1, p, "bf16")).to(torch.bfloat16)
        kr_ref = torch.from_numpy(expected_rope(k.cpu(), cos, sin, 1, p, "bf16")).to(torch.bfloat16)
        ref.append(kr_ref.to(dev), v.contiguous())
        assert torch.equal(qr.cpu(), qr_ref)
    out = cache.attention(qr, 1.0 / d ** 0.5)
    want = ref.attention(qr_ref.to(dev), 1.0 / d ** 0.5)
    assert torch.equal(out, want)


def test_rope_append_config4_full_size(cq, dev):
    """At the BASELINE config-4 shape (B=4, 4096 tokens, 32 / 8 heads, D=128, FP8 cache): the
    fused launch equals, bit for bit, torch's rope in f32 (separate elementwise kernels: products
    rounded before the sum, as the reference's kernels) rounded to bf16, followed by this
    library's plain quantize-append of the rotated keys and of the values."""
    b, t, hq, hkv, d = 4, 4096, 32, 8, 128
    g = torch.Generator(device=dev).manual_seed(4)
    qkv = torch.randn(b, t, (hq + 2 * hkv) * d, generator=g, device=dev).to(torch.bfloat16)
    q, k, v = cq.split_qkv(qkv, hq, hkv)
    ang = torch.arange(t, dtype=torch.float64, device=dev)[:, None] / \
        10000.0 ** (torch.arange(0, d, 2, dtype=torch.float64, device=dev) / d)
    cos, sin = ang.cos().to(torch.bfloat16), ang.sin().to(torch.bfloat16)
    ks = cq.CacheSide.empty(5, False, b, hkv, d, t, dev)
    vs = cq.CacheSide.empty(5, True, b, hkv, d, t, dev)
    q_out = cq.rope_quant_append(ks, vs, q, k, v, cos, sin, cq.ROPE_HALVES, 0)

    def rope_ref(x):  # (b, h, t, d) bf16 -> bf16
        xf, c, s = x.float(), cos.float()[None, None], sin.float()[None, None]
        x1, x2 = xf[..., :d // 2], xf[..., d // 2:]
        return torch.cat([x1 * c - x2 * s, x1 * s + x2 * c], -1).to(torch.bfloat16)
    assert torch.equal(q_out, rope_ref(q))
    ks2 = cq.CacheSide.empty(5, False, b, hkv, d, t, dev)
    vs2 = cq.CacheSide.empty(5, True, b, hkv, d, t, dev)
    cq.quant_append(ks2, rope_ref(k), 0)
    cq.quant_append(vs2, v, 0)
    torch.cuda.synchronize()
    assert torch.equal(ks.codes, ks2.codes) and torch.equal(ks.scales, ks2.scales)
    assert torch.equal(vs.codes, vs2.codes) and torch.equal(vs.scales, vs2.scales)


@pytest.mark.parametrize("kf,vf", [(5, 5), (5, 0), (2, 5)])
def test_rope_append_positions_past_table_skip_keys_and_values(cq, dev, kf, vf):
    """Cos / sin tables shorter than the cache: a position past the table is skipped on both
    sides, so no value row is written without its key row (and rows already there survive).
    Values of another format than the keys (FP8 keys with TurboQuant-4 values through the MFMA
    append, MXFP4 keys with FP8 values) take their own launch, clipped at the table's end too."""
    b, hq, hkv, d, t, cap, rows = 3, 4, 2, 128, 4, 64, 40
    qkv = kv_source(5, (b, t, 1, (hq + 2 * hkv) * d))[:, :, 0].to(dev)
    q, k, v = cq.split_qkv(qkv, hq, hkv)
    cos, sin = tables(rows, d, "bf16")
    pos = torch.tensor([0, 37, 50], dtype=torch.int32, device=dev)
    ks = cq.CacheSide.empty(kf, False, b, hkv, d, cap, dev, seed=42)
    vs = cq.CacheSide.empty(vf, True, b, hkv, d, cap, dev, seed=44)
    pre_k = oracle_rows(kf, kv_source(93, (b, hkv, cap, d)), 42)
    pre_v = oracle_rows(vf, kv_source(94, (b, hkv, cap, d)), 44)
    cq.rows_import(ks, torch.from_numpy(pre_k.view(np.int32)).to(dev), 0)
    cq.rows_import(vs, torch.from_numpy(pre_v.view(np.int32)).to(dev), 0)
    cq.rope_quant_append(ks, vs, q, k, v, cos.to(dev), sin.to(dev), 1, positions=pos)
    torch.cuda.synchronize()
    got_k, got_v = export_np(cq, ks, cap), export_np(cq, vs, cap)
    want_k, want_v = pre_k.copy(), pre_v.copy()
    for bi, p in enumerate(pos.tolist()):
        n = max(0, min(t, rows - p))  # positions below the table's rows only
        if n == 0:
            continue
        k_rot = expected_rope(k[bi:bi + 1, :, :n].cpu(), cos, sin, 1, p, "bf16")
        want_k[bi:bi + 1, :, p:p + n] = oracle_rows(kf, torch.from_numpy(k_rot), 42)
        want_v[bi:bi + 1, :, p:p + n] = oracle_rows(vf, v[bi:bi + 1, :, :n].cpu(), 44)
    np.testing.assert_array_equal(got_k, want_k)
    if vf == 0:  # TurboQuant values: the flip criterion on the written rows, the rest untouched
        written = np.zeros(cap, bool)
        for p in pos.tolist():
            written[p:min(p + t, rows)] = True
        np.testing.assert_array_equal(got_v[:, :, ~written], want_v[:, :, ~written])
        assert_turbo_rows_close(got_v[:, :, written], want_v[:, :, written], d)
    else:
        np.testing.assert_array_equal(got_v, want_v)
