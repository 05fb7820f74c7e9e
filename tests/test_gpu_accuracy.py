"""The reference's published attention error per cache format (README.md:301-311 of the
reference), reproduced on the HIP decode.

The reference's test (turbo_quant::accuracy::attention_error_by_format, candle-nn/src/
turbo_quant.rs:1644-1719): one SplitMix64(seed * 77 + d) normal stream as f32 gives k, v
(1, 2, 256, 128) and q (1, 8, 1, 128); TurboKvCache::with_formats(kf, vf, d, Auto, seed, ..)
(keys seed s, values s + 2; Auto is Hadamard at d = 128, for every format); the attention over the
cache against the exact f32 attention of the inputs; relative RMS error of the output, mean over
seeds 0-5. Here the cache is written and attended by the library (f32 rows appended, f32 queries
and output) and each mean must lie within 0.003 of the published value. The oracle reproduces the
table to its three decimals on the CPU (tests/test_oracle.py)."""
import numpy as np
import pytest
import torch

from tests.helpers import PUBLISHED_ERRORS, accuracy_inputs, gqa_attention_f64, relative_rms

pytestmark = pytest.mark.gpu

ROT_AUTO = 4


@pytest.mark.parametrize("kf,vf,want", PUBLISHED_ERRORS)
def test_published_attention_error_on_the_gpu_decode(cq, dev, kf, vf, want):
    d = 128
    errs = []
    for seed in range(6):
        k, v, q = accuracy_inputs(seed, d)
        cache = cq.TurboKvCache(kf[0], vf[0], 1, 2, d, 256, device=dev, seed=seed,
                                rotation=ROT_AUTO, key_bits=kf[1], value_bits=vf[1])
        cache.append(torch.from_numpy(k).to(dev), torch.from_numpy(v).to(dev))
        got = cache.attention(torch.from_numpy(q).to(dev), d ** -0.5)
        torch.cuda.synchronize()
        assert got.dtype == torch.float32
        errs.append(relative_rms(got.cpu().numpy().astype(np.float64),
                                 gqa_attention_f64(q, k, v, d ** -0.5)))
    assert abs(np.mean(errs) - want) <= 3e-3, (np.mean(errs), want)
