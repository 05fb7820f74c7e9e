"""GPU parity of the prefill's optional score terms and variable-length batches
(cqkv_flash_attn_ext; candle_flash_attn::flash_attn_alibi_windowed_softcap and
flash_attn_varlen, candle-flash-attn/src/lib.rs:41-511) against the oracle, whose soft-capping,
ALiBi and per-sequence semantics are pinned to the reference's fa_tile_impl in test_oracle.py.
Variable-length results must also equal the dense call on each sequence bit for bit (the
reference's own varlen invariant, candle-flash-attn/tests/api.rs:86-140)."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import assert_close_bf16
from tests.test_gpu_prefill import bf16_randn

pytestmark = pytest.mark.gpu


def oracle_terms(q, k, v, scale, wl, wr, softcap=0.0, slopes=None):
    """q (b, sq, hq, d), k / v (b, sk, hkv, d) bf16; slopes (hq,) or (b, hq) -> bf16-rounded
    oracle output (b, sq, hq, d)."""
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
        out.append(O.round_bf16(o).transpose(0, 2, 1, 3))
    return np.concatenate(out, axis=0)


@pytest.mark.parametrize("softcap,per_batch,wl,wr", [(5.0, False, -1, 0), (0.0, False, -1, 0),
                                                     (2.0, True, 30, 0), (3.0, False, 40, 5),
                                                     (0.0, True, -1, -1)])
@pytest.mark.parametrize("d", [128, 256])
def test_prefill_softcap_alibi(cq, dev, softcap, per_batch, wl, wr, d):
    """D = 256 runs the MFMA prefill's 32-key-tile, four-wavefront form."""
    b, sq, sk, hq, hkv = 2, 150, 190, 8, 2
    q = bf16_randn(31, (b, sq, hq, d), 3.0)  # large enough scores for tanh to bite
    k = bf16_randn(32, (b, sk, hkv, d))
    v = bf16_randn(33, (b, sk, hkv, d))
    slopes = (0.02 * (1 + torch.arange(b * hq, dtype=torch.float32))).reshape(b, hq)
    if not per_batch:
        slopes = slopes[0].contiguous()
    scale = 1.0 / d ** 0.5
    got = cq.flash_attn(q.to(dev), k.to(dev), v.to(dev), scale, False, window_left=wl,
                        window_right=wr, softcap=softcap, alibi_slopes=slopes.to(dev))
    torch.cuda.synchronize()
    want = oracle_terms(q, k, v, scale, wl, wr, softcap, slopes)
    assert_close_bf16(got.float().cpu().numpy(), want)


def test_prefill_softcap_only(cq, dev):
    b, s, hq, hkv, d = 1, 200, 4, 1, 128
    q = bf16_randn(41, (b, s, hq, d), 4.0)
    k = bf16_randn(42, (b, s, hkv, d))
    v = bf16_randn(43, (b, s, hkv, d))
    got = cq.flash_attn(q.to(dev), k.to(dev), v.to(dev), 0.09, True, softcap=1.5)
    torch.cuda.synchronize()
    assert_close_bf16(got.float().cpu().numpy(), oracle_terms(q, k, v, 0.09, -1, 0, 1.5))


def varlen_inputs(seed, lens_q, lens_k, hq, hkv, d=128):
    cu_q = np.concatenate([[0], np.cumsum(lens_q)]).astype(np.int32)
    cu_k = np.concatenate([[0], np.cumsum(lens_k)]).astype(np.int32)
    q = bf16_randn(seed, (int(cu_q[-1]), hq, d))
    k = bf16_randn(seed + 1, (int(cu_k[-1]), hkv, d))
    v = bf16_randn(seed + 2, (int(cu_k[-1]), hkv, d))
    return q, k, v, cu_q, cu_k


@pytest.mark.parametrize("causal,wl,softcap,alibi", [(True, -1, 0.0, False), (False, -1, 0.0, False),
                                                     (True, 70, 0.0, False), (True, -1, 3.0, True)])
@pytest.mark.parametrize("d", [128, 256])
def test_prefill_varlen(cq, dev, causal, wl, softcap, alibi, d):
    """Ragged sequences (an empty one, single-token ones, more queries than keys) against the
    oracle per sequence and against the dense call on each sequence."""
    lens_q = [100, 0, 1, 257, 64, 30]
    lens_k = [130, 60, 1, 257, 200, 20]
    hq, hkv = 8, 2
    q, k, v, cu_q, cu_k = varlen_inputs(51, lens_q, lens_k, hq, hkv, d)
    slopes = (0.03 * (1 + torch.arange(hq, dtype=torch.float32))) if alibi else None
    scale = 1.0 / d ** 0.5
    wr = 0 if causal else -1
    cuq, cuk = torch.from_numpy(cu_q).to(dev), torch.from_numpy(cu_k).to(dev)
    sl = None if slopes is None else slopes.to(dev)
    got = cq.flash_attn_varlen(q.to(dev), k.to(dev), v.to(dev), cuq, cuk, max(lens_q),
                               max(lens_k), scale, causal, window_left=wl, softcap=softcap,
                               alibi_slopes=sl)
    torch.cuda.synchronize()
    got = got.float().cpu()
    for bi in range(len(lens_q)):
        qs, qe, ks, ke = cu_q[bi], cu_q[bi + 1], cu_k[bi], cu_k[bi + 1]
        if qe == qs:
            continue
        qb, kb, vb = q[None, qs:qe], k[None, ks:ke], v[None, ks:ke]
        want = oracle_terms(qb, kb, vb, scale, wl, wr, softcap, slopes)
        assert_close_bf16(got[qs:qe].numpy()[None], want)
        dense = cq.flash_attn(qb.to(dev), kb.to(dev), vb.to(dev), scale, causal, window_left=wl,
                              softcap=softcap, alibi_slopes=sl)
        torch.cuda.synchronize()
        assert torch.equal(got[qs:qe], dense[0].float().cpu()), f"sequence {bi}"


def test_prefill_varlen_rows_outside_sequences_untouched(cq, dev):
    """Rows past the last sequence (total_q larger than cu_q[-1]) are not written."""
    q, k, v, cu_q, cu_k = varlen_inputs(61, [40, 70], [40, 90], 4, 4)
    qx = torch.cat([q, bf16_randn(64, (5, 4, 128))])
    out = torch.full(qx.shape, 7.0, dtype=torch.bfloat16, device=dev)
    cq.flash_attn_varlen(qx.to(dev), k.to(dev), v.to(dev), torch.from_numpy(cu_q).to(dev),
                         torch.from_numpy(cu_k).to(dev), 70, 90, 0.1, True, out=out)
    torch.cuda.synchronize()
    assert (out[110:].float() == 7.0).all()
