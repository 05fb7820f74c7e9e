"""Exhaustive GPU check of the E4M3 conversions inside the FP8 encoders (cqkv_device.h), run by
the test-only kernels of tests/native/libcqkv_probe.so.

The FP8 row encoders (cache append, prefill's fused append, fused RoPE + append) turn each
quotient x / s into its code with the gfx950 conversion v_cvt_pk_fp8_f32 instead of the
reference's integer encoder (candle-core/src/accel/formats.rs:288-308), and form x / s as
x * (1 / s) plus one FMA correction instead of an IEEE division. Both shortcuts are held here to
the reference's codes:
  * every f32 value with |q| <= 449 (2.28e9 inputs, both signs) through the hardware conversion
    and through the device software encoder, against the oracle encoder's code thresholds;
  * 2^32 random rows (x, y) of finite bf16 values over the whole exponent range, the codes of
    the encoders' per-row choice (the division-free path for rows of absmax >= 2^-77) against the
    IEEE quotient's;
  * 2^32 random NVFP4 elements (finite bf16 x, row and block maxima over the whole exponent
    range), the codes of the encoders' per-block choice (FMA-corrected quotient and hardware E2M1
    conversion for blocks of maximum >= 2^-60) against E2M1 of the IEEE quotient;
  * every non-NaN f32 value (both signs, infinities included) through the gfx950 E2M1
    conversion at scale 1 (v_cvt_scalef32_pk_fp4_f32, used by the MXFP4 / NVFP4 encoders) and
    through the device software encoder, against the oracle's E2M1 code thresholds
    (candle-core/src/accel/formats.rs:329-350)."""
import ctypes
import os

import numpy as np
import pytest

from tests.helpers import E4M3_SWEEP_END, FP4_SWEEP_END, e4m3_thresholds, fp4_thresholds

pytestmark = pytest.mark.gpu

PROBE = os.path.join(os.path.dirname(__file__), "native", "libcqkv_probe.so")


@pytest.fixture(scope="module")
def probe(dev):
    if not os.path.exists(PROBE):
        raise RuntimeError(f"{PROBE} is missing: build it with `make -C tests/native`")
    L = ctypes.CDLL(PROBE)
    L.probe_e4m3_sweep.argtypes = [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_void_p,
                                   ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    L.probe_fp8_quotient.argtypes = [ctypes.c_uint64, ctypes.c_uint64, ctypes.c_void_p,
                                     ctypes.c_void_p]
    L.probe_fp4_sweep.argtypes = L.probe_e4m3_sweep.argtypes
    L.probe_nvfp4_quotient.argtypes = L.probe_fp8_quotient.argtypes
    return L


def test_e4m3_conversions_on_every_input_up_to_449(probe):
    thr = e4m3_thresholds()
    bad = np.zeros(2, np.uint64)
    first = np.zeros(1, np.uint32)
    assert probe.probe_e4m3_sweep(0, E4M3_SWEEP_END, thr.ctypes.data, len(thr),
                                  bad.ctypes.data, first.ctypes.data) == 0
    assert bad.tolist() == [0, 0], (bad, hex(int(first[0])))


def test_fp8_fast_quotient_codes_equal_ieee_division(probe):
    bad = np.zeros(1, np.uint64)
    first = np.zeros(1, np.uint64)
    assert probe.probe_fp8_quotient(1 << 32, 0x5eed, bad.ctypes.data, first.ctypes.data) == 0
    assert int(bad[0]) == 0, (bad, first)


def test_fp4_conversions_on_every_non_nan_input(probe):
    thr = fp4_thresholds()
    for lo, hi in ((0, FP4_SWEEP_END), (FP4_SWEEP_END, 0x7F800001)):
        bad = np.zeros(2, np.uint64)
        first = np.zeros(1, np.uint32)
        assert probe.probe_fp4_sweep(lo, hi, thr.ctypes.data, len(thr), bad.ctypes.data,
                                     first.ctypes.data) == 0
        assert bad.tolist() == [0, 0], (hex(lo), bad, hex(int(first[0])))


def test_nvfp4_fast_quotient_codes_equal_ieee_division(probe):
    bad = np.zeros(1, np.uint64)
    first = np.zeros(1, np.uint64)
    assert probe.probe_nvfp4_quotient(1 << 32, 0xa11ce, bad.ctypes.data, first.ctypes.data) == 0
    assert int(bad[0]) == 0, (bad, first)
