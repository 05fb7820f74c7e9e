"""GPU parity of the FP8 K / V attention path (flash_attn_fp8 and flash_attn_with_config on
F8E4M3 tensors with descale factors; candle-nn/src/flash_attn.rs:113-117, 862-892).

The per-tensor quantization is bit-exact with the oracle's restatement (codes and scale); the
attention is held to the BASELINE tolerance (max-abs 2e-2, mean-abs 2e-3) against the oracle's
unfused f32 attention over e4m3(code) * descale, the reference's own math (scores dot * k_descale,
outputs times v_descale / l: candle-core/kernels/flash_attn_impl.h:52-63, 381, 434)."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import assert_close_bf16

pytestmark = pytest.mark.gpu

E4M3 = None


def e4m3_values():
    global E4M3
    if E4M3 is None:
        E4M3 = np.array([O.e4m3_to_f32(c) for c in range(256)], np.float32)
    return E4M3


def oracle_fp8_attention(q, k8, v8, kd, vd, scale, wl, wr):
    """q (b, s_q, h_q, d) torch bf16, k8 / v8 (b, s_kv, h_kv, d) uint8 codes -> f32 output."""
    vals = e4m3_values()
    kf = vals[k8.cpu().numpy()] * np.float32(kd)
    vf = vals[v8.cpu().numpy()] * np.float32(vd)
    qf = q.float().cpu().numpy()
    out = O.attention_unfused(qf.transpose(0, 2, 1, 3), kf.transpose(0, 2, 1, 3),
                              vf.transpose(0, 2, 1, 3), scale, wl=wl, wr=wr, threads=16)
    return out.transpose(0, 2, 1, 3)


def inputs(seed, b, sq, sk, hq, hkv, d=128, kmag=1.0):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(b, sq, hq, d, generator=g).to(torch.bfloat16)
    k = (torch.randn(b, sk, hkv, d, generator=g) * kmag).to(torch.bfloat16)
    v = torch.randn(b, sk, hkv, d, generator=g).to(torch.bfloat16)
    return q, k, v


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_fp8_quantize_tensor_bit_exact(cq, dev, dtype):
    g = torch.Generator().manual_seed(3)
    x = torch.randn(3, 257, 5, 128, generator=g) * 7.0
    x[0, 0, 0, :5] = torch.tensor([0.0, -0.0, 1e-30, -1e-30, 3.0e4])
    x = x.to(dtype)
    codes, scale = cq.fp8_quantize_tensor(x.to(dev))
    want, ws = O.fp8_quantize_tensor(x.float().numpy())
    assert scale[0].item() == float(ws)
    np.testing.assert_array_equal(codes.cpu().numpy(), want)
    z, zs = cq.fp8_quantize_tensor(torch.zeros(1000, device=dev))
    assert zs[0].item() == 1.0 and int(z.sum()) == 0


@pytest.mark.parametrize("wl,wr", [(-1, 0), (100, 0), (-1, -1), (30, 5)])
def test_flash_attn_fp8_codes_host_descales(cq, dev, wl, wr):
    b, sq, sk, hq, hkv = 2, 200, 333, 8, 2
    q, k, v = inputs(1, b, sq, sk, hq, hkv)
    k8 = torch.from_numpy(O.e4m3_encode(k.float().numpy() * 50.0))
    v8 = torch.from_numpy(O.e4m3_encode(v.float().numpy() * 80.0))
    kd, vd, scale = 1 / 50.0, 1 / 80.0, 1 / 128 ** 0.5
    out = cq.flash_attn_fp8_codes(q.to(dev), k8.to(dev), v8.to(dev), scale, False, kd, vd, wl, wr)
    torch.cuda.synchronize()
    want = oracle_fp8_attention(q, k8, v8, kd, vd, scale, wl, wr)
    assert_close_bf16(out.float().cpu().numpy(), want)


def test_flash_attn_fp8_end_to_end(cq, dev):
    """flash_attn_fp8: the device scales equal the oracle's, the codes are the oracle's, and the
    output equals flash_attn_fp8_codes with those scales given as host descales, bit for bit.
    Unit-scale inputs, as in the reference's own FP8 attention tests (flash_attn.rs:1073-1095):
    the queries enter the MFMA in bf16, whose rounding grows with the score magnitudes."""
    b, sq, sk, hq, hkv = 2, 130, 130, 8, 2
    q, k, v = inputs(2, b, sq, sk, hq, hkv)
    scale = 1 / 128 ** 0.5
    out = cq.flash_attn_fp8(q.to(dev), k.to(dev), v.to(dev), scale, True)
    k8, ks = O.fp8_quantize_tensor(k.float().numpy())
    v8, vs = O.fp8_quantize_tensor(v.float().numpy())
    ref = cq.flash_attn_fp8_codes(q.to(dev), torch.from_numpy(k8).to(dev),
                                  torch.from_numpy(v8).to(dev), scale, True, float(ks), float(vs))
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    want = oracle_fp8_attention(q, torch.from_numpy(k8), torch.from_numpy(v8), ks, vs, scale, -1, 0)
    assert_close_bf16(out.float().cpu().numpy(), want)
    # and close to the bf16 attention it approximates (FP8 rounding of K / V only)
    full = cq.flash_attn(q.to(dev), k.to(dev), v.to(dev), scale, True).float().cpu().numpy()
    assert np.abs(full - out.float().cpu().numpy()).mean() < 2e-2


def test_flash_attn_fp8_decode_shape_and_float8_dtype(cq, dev):
    """One query row per sequence (the reference's fa_row decode case) and torch.float8_e4m3fn
    code tensors."""
    if getattr(torch, "float8_e4m3fn", None) is None:
        pytest.skip("torch without float8_e4m3fn")
    b, sq, sk, hq, hkv = 4, 1, 777, 32, 8
    q, k, v = inputs(3, b, sq, sk, hq, hkv)
    k8 = torch.from_numpy(O.e4m3_encode(k.float().numpy() * 100.0))
    v8 = torch.from_numpy(O.e4m3_encode(v.float().numpy() * 100.0))
    out = cq.flash_attn_fp8_codes(q.to(dev), k8.to(dev).view(torch.float8_e4m3fn),
                                  v8.to(dev).view(torch.float8_e4m3fn), 0.09, True, 0.01, 0.01)
    torch.cuda.synchronize()
    want = oracle_fp8_attention(q, k8, v8, 0.01, 0.01, 0.09, -1, 0)
    assert_close_bf16(out.float().cpu().numpy(), want)


@pytest.mark.parametrize("d,dtype,sq", [(64, torch.bfloat16, 150), (256, torch.float16, 77),
                                         (96, torch.float16, 3), (128, torch.float16, 200)])
def test_flash_attn_fp8_head_dims_f16_and_workspace(cq, dev, d, dtype, sq):
    """The reference's FP8 K / V path takes every head dim of its tile kernels and f16 queries
    (flash_attn.rs:862-892; kernels fa_*_f16_f8 of flash_attn_impl.h): head dims 64 / 96 / 256,
    f16 queries and outputs, prefill and decode shapes; a caller workspace of
    flash_attn_fp8_workspace_bytes gives the same output as the allocating call, and a smaller
    one is refused."""
    b, sk, hq, hkv = 2, 301, 8, 2
    q, k, v = inputs(7 + d, b, sq, sk, hq, hkv, d)
    q = q.to(dtype)
    k8 = torch.from_numpy(O.e4m3_encode(k.float().numpy() * 40.0))
    v8 = torch.from_numpy(O.e4m3_encode(v.float().numpy() * 60.0))
    kd, vd, scale = 1 / 40.0, 1 / 60.0, 1 / d ** 0.5
    qd, k8d, v8d = q.to(dev), k8.to(dev), v8.to(dev)
    out = cq.flash_attn_fp8_codes(qd, k8d, v8d, scale, True, kd, vd)
    n = cq.flash_attn_fp8_workspace_bytes(dtype, b, sq, sk, hq, hkv, d)
    assert n > 0
    ws = torch.empty(n, dtype=torch.uint8, device=dev)
    out2 = cq.flash_attn_fp8_codes(qd, k8d, v8d, scale, True, kd, vd, workspace=ws)
    torch.cuda.synchronize()
    assert out.dtype == dtype and torch.equal(out, out2)
    want = oracle_fp8_attention(q, k8, v8, kd, vd, scale, -1, 0)
    assert_close_bf16(out.float().cpu().numpy(), want)
    with pytest.raises(cq.CqkvError):
        cq.flash_attn_fp8_codes(qd, k8d, v8d, scale, True, kd, vd, workspace=ws[:n - 256])


@pytest.mark.parametrize("d", [2, 8, 32, 64, 128, 256])
def test_hadamard_rows_vs_oracle_rotation(cq, dev, d):
    """The rotation of flash_attn_fp8's switch: rotation_matrix(d, Hadamard, 0x46413346) in f32.
    The reference multiplies by the dense matrix (its f32 summation order is not pinned, as for
    TurboQuant's rotation): within 2e-6 relative in f32 before the bf16 rounding, and at most
    one bf16 ulp after it."""
    g = torch.Generator().manual_seed(9)
    x = torch.randn(3, 41, 4, d, generator=g)
    pi = O.rotation_matrix(d, O.ROT_HADAMARD, cq.FP8_HADAMARD_SEED)
    want = O.rotate_rows(pi, x.numpy().reshape(-1, d)).reshape(x.shape)
    got = cq.hadamard_rows(x.to(dev)).cpu().numpy()
    np.testing.assert_allclose(got, want, rtol=2e-6, atol=2e-6)
    xb = x.to(torch.bfloat16)
    gb = cq.hadamard_rows(xb.to(dev)).float().cpu().numpy()
    wb = O.round_bf16(O.rotate_rows(pi, xb.float().numpy().reshape(-1, d)).reshape(x.shape))
    # one bf16 step of the larger of the two, plus the f32 allowance above for sums that cancel
    # to (nearly) zero, where the two summation orders differ in the last bits
    ulp = np.maximum(np.abs(wb), np.abs(gb)) * 2.0 ** -7 + 2e-6
    assert (np.abs(gb - wb) <= ulp).all()
    assert (gb == wb).mean() > 0.99


def test_hadamard_rows_refuses_other_head_dims(cq, dev):
    """The reference rotates power-of-two head dims only (flash_attn.rs:869)."""
    x = torch.zeros(4, 96, device=dev)
    with pytest.raises(cq.CqkvError):
        cq.hadamard_rows(x)


def test_flash_attn_fp8_hadamard(cq, dev):
    """With the switch: equal to the oracle pipeline (rotate q and k, round to bf16, per-tensor
    FP8 of the rotated k, attention) to the tolerance, and to the unrotated bf16 attention to
    the FP8 error (the rotation leaves Q K^T unchanged)."""
    b, sq, sk, hq, hkv = 2, 96, 96, 8, 2
    q, k, v = inputs(5, b, sq, sk, hq, hkv)
    scale = 1 / 128 ** 0.5
    out = cq.flash_attn_fp8(q.to(dev), k.to(dev), v.to(dev), scale, True, hadamard=True)
    torch.cuda.synchronize()
    pi = O.rotation_matrix(128, O.ROT_HADAMARD, cq.FP8_HADAMARD_SEED)
    qr = O.round_bf16(O.rotate_rows(pi, q.float().numpy().reshape(-1, 128)).reshape(q.shape))
    kr = O.round_bf16(O.rotate_rows(pi, k.float().numpy().reshape(-1, 128)).reshape(k.shape))
    k8, ks = O.fp8_quantize_tensor(kr)
    v8, vs = O.fp8_quantize_tensor(v.float().numpy())
    want = oracle_fp8_attention(torch.from_numpy(qr), torch.from_numpy(k8), torch.from_numpy(v8),
                                ks, vs, scale, -1, 0)
    assert_close_bf16(out.float().cpu().numpy(), want)
    full = cq.flash_attn(q.to(dev), k.to(dev), v.to(dev), scale, True).float().cpu().numpy()
    assert np.abs(full - out.float().cpu().numpy()).mean() < 2e-2


def test_flash_attn_fp8_config4_full_size_matches_bf16_path(cq, dev):
    """At the config-4 shape with unit descales, the FP8 path is the bf16 prefill on the exact
    bf16 values of the codes: its staging pass (E4M3 -> bf16, strided K / V) must give the same
    output bit for bit as flash_attn on those values."""
    b, s, hq, hkv, d = 4, 4096, 32, 8, 128
    g = torch.Generator(device=dev).manual_seed(8)
    q = torch.randn(b, s, hq, d, generator=g, device=dev).to(torch.bfloat16)
    k8, _ = cq.fp8_quantize_tensor(torch.randn(b, s, hkv, d, generator=g, device=dev))
    v8, _ = cq.fp8_quantize_tensor(torch.randn(b, s, hkv, d, generator=g, device=dev))
    out = cq.flash_attn_fp8_codes(q, k8, v8, 1 / d ** 0.5, True)
    vals = torch.from_numpy(e4m3_values()).to(dev)
    kb = vals[k8.long()].to(torch.bfloat16)
    vb = vals[v8.long()].to(torch.bfloat16)
    ref = cq.flash_attn(q, kb, vb, 1 / d ** 0.5, True)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
