// Device-side building blocks of the cqkv kernels (gfx950 only): vector types, bounds-checked
// buffer loads, the cache element codecs, and wavefront reductions.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cqkv {

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

constexpr int kWave = 64;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// ---------------------------------------------------------------------------------------------
// Buffer resources: a base pointer plus a byte range. Loads past the range return zeros, so a
// plane read never leaves its plane whatever the lengths say.
// ---------------------------------------------------------------------------------------------
typedef __amdgpu_buffer_rsrc_t rsrc_t;

__device__ inline rsrc_t make_rsrc(const void *base, uint32_t bytes) {
    // word 3 = 0x00020000: 32-bit data format, raw (untyped) access
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes,
                                             0x00020000);
}
__device__ inline u32x4 ld128(rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
}
__device__ inline u32x2 ld64(rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0);
}
__device__ inline uint32_t ld32(rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
}
// Streaming loads for data read once per call (cache codes): cache policy 2 = nontemporal (NT),
// so the lines do not displace reusable data in L2 / MALL. Measured on MI355X: FP8 decode at
// BASELINE config 2 goes from 5.4 to 6.3 TB/s with these on the code loads.
__device__ inline u32x4 ld128_stream(rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 2);
}
__device__ inline u32x2 ld64_stream(rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 2);
}

// ---------------------------------------------------------------------------------------------
// 16-bit floats
// ---------------------------------------------------------------------------------------------
__device__ inline float bf16_bits_to_f32(uint32_t b) { return __uint_as_float(b << 16); }
__device__ inline float f16_bits_to_f32(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}
// f32 -> bf16 bits, round to nearest even (v_cvt_pk_bf16_f32)
__device__ inline uint32_t f32_to_bf16_bits(float f) {
    return (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)f);
}
__device__ inline uint32_t pack_bf16x2(float lo, float hi) {
    bf16x2 v;
    v.x = (__bf16)lo;
    v.y = (__bf16)hi;
    return __builtin_bit_cast(uint32_t, v);
}
// f32 pair -> f16 pair, round to nearest even (one v_cvt_pk_f16_f32)
__device__ inline uint32_t pack_f16x2(float lo, float hi) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    const h2 v = {(_Float16)lo, (_Float16)hi};
    return __builtin_bit_cast(uint32_t, v);
}

// Element dtype of q / k / v / out: 0 bf16, 1 f16, 2 f32 (the CQKV_* ids of cqkv.h).
__device__ inline float load_elem(const void *p, int64_t idx, int dtype) {
    if (dtype == 0) return bf16_bits_to_f32(((const uint16_t *)p)[idx]);
    if (dtype == 1) return f16_bits_to_f32(((const uint16_t *)p)[idx]);
    return ((const float *)p)[idx];
}
__device__ inline void store_elem(void *p, int64_t idx, int dtype, float v) {
    if (dtype == 0) ((uint16_t *)p)[idx] = (uint16_t)f32_to_bf16_bits(v);
    else if (dtype == 1) ((uint16_t *)p)[idx] = __builtin_bit_cast(uint16_t, (_Float16)v);
    else ((float *)p)[idx] = v;
}

// ---------------------------------------------------------------------------------------------
// E4M3 (OCP E4M3FN) and E2M1 / E8M0 codecs. The encoders are the reference's integer
// algorithms (candle-core/src/accel/formats.rs:288-308, 329-350, 354-372): codes must be bit
// for bit those of RowCodec::quantize_row.
// ---------------------------------------------------------------------------------------------
__device__ inline uint32_t e4m3_encode(float f) {
    const uint32_t x = __float_as_uint(f);
    const uint32_t s = (x >> 24) & 0x80u;
    const uint32_t ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) return s | 0x7fu;              // NaN
    const float a = __uint_as_float(ax);
    if (a >= 448.0f) return s | 0x7eu;                    // saturate (incl. inf)
    if (a < 0.015625f) return s | (uint32_t)__builtin_rintf(a * 512.0f);  // subnormals, RNE
    const uint32_t r = ax + 0x7ffffu + ((ax >> 20) & 1u);  // RNE at 3 mantissa bits
    uint32_t code = (((r >> 23) - 120u) << 3) | ((r >> 20) & 7u);
    return s | (code > 0x7eu ? 0x7eu : code);
}

// The quotient x / s of the FP8 row encoder, correctly rounded, from r = 1 / s (correctly
// rounded, computed once per row): q0 = x r, then one FMA correction q0 + r (x - q0 s) - the
// correctly rounded quotient when the residual does not underflow (Markstein's theorem on
// FMA-based division, P. Markstein, "IA-64 and Elementary Functions", 2000). Below |x| = 2^-96
// the residual may underflow and the IEEE division is used. Where the quotient itself
// underflows it can differ from x / s in its last bits, but every such quotient encodes to the
// same E4M3 code (signed zero).
__device__ inline float fp8_row_quotient(float x, float s, float r) {
    const float q0 = x * r;
    const float q = __builtin_fmaf(__builtin_fmaf(-q0, s, x), r, q0);
    return __builtin_fabsf(x) < 0x1p-96f ? x / s : q;
}

// E4M3 codes of two quotients (|q| <= 448 * (1 + 2^-23)): the gfx950 conversion rounds to
// nearest-even with the same subnormal and signed-zero results as e4m3_encode on that range
// (all 2^31 - 2^23 f32 values with |q| <= 449 compared).
__device__ inline uint32_t e4m3_encode2(float q0, float q1) {
    return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(q0, q1, 0, false) & 0xffffu;
}

// Codes of x0 / s and x1 / s (low byte: x0) for the FP8 row encoder, r = 1 / s. Non-finite
// inputs or scales take the division and the software encoder (the reference's NaN / infinity
// results); finite ones the fast path above.
__device__ inline uint32_t fp8_row_codes(float x0, float x1, float s, float r) {
    if (__builtin_isfinite(x0) && __builtin_isfinite(x1) && __builtin_isfinite(s))
        return e4m3_encode2(fp8_row_quotient(x0, s, r), fp8_row_quotient(x1, s, r));
    return e4m3_encode(x0 / s) | (e4m3_encode(x1 / s) << 8);
}

// The FMA-corrected quotient x / s from r = 1 / s with the sign of x: for x = -0 the correction
// gives (+0) r + (-0) = +0, while x / s is -0 (for x != 0 the sign is already that of x).
__device__ inline float signed_quotient(float x, float s, float r) {
    const float q0 = x * r;
    return __builtin_copysignf(__builtin_fmaf(__builtin_fmaf(-q0, s, x), r, q0), x);
}

// fp8_row_codes for a row known to be ordinary: finite scale s = amax / 448 with amax finite and
// at least 2^-77, finite elements. Every element then takes the FMA-corrected quotient, also
// below 2^-96: there |x / s| = 448 |x| / amax < 2^-10, both quotients encode to the signed zero
// of x, and the division is never computed (checked against the IEEE quotient on 2^32 random
// rows of finite bf16 values over the whole exponent range, signed zeros included).
constexpr float kFp8FastRowMin = 0x1p-77f;
__device__ inline uint32_t fp8_row_codes_fast(float x0, float x1, float s, float r) {
    return e4m3_encode2(signed_quotient(x0, s, r), signed_quotient(x1, s, r));
}

__device__ inline uint32_t fp4_encode(float f) {
    const uint32_t s = (__float_as_uint(f) >> 28) & 8u;
    const float a = __builtin_fabsf(f);
    uint32_t c;
    if (!(a > 0.25f)) c = 0;  // also NaN
    else if (a < 0.75f) c = 1;
    else if (a <= 1.25f) c = 2;
    else if (a < 1.75f) c = 3;
    else if (a <= 2.5f) c = 4;
    else if (a < 3.5f) c = 5;
    else if (a <= 5.0f) c = 6;
    else c = 7;
    return s | c;
}

// E2M1 codes of two quotients (low nibble: q0) by the gfx950 conversion at scale 1 (its scale
// operand divides, by the power of two of its exponent). It rounds to nearest-even, saturates to
// +-6 and keeps signed zeros exactly as fp4_encode does on every f32 input but NaN (all 2^32 - 2^24
// non-NaN patterns compared); a NaN gives code 7 here and 0 in fp4_encode, so NaN inputs need
// fp4_encode.
__device__ inline uint32_t fp4_encode_hw(float q0, float q1) {
    return __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(0u, q0, q1, 1.0f, 0) & 0xffu;
}

// NVFP4 element codes of x0 / eff and x1 / eff (low nibble: x0), eff > 0 the block's effective
// scale, r = 1 / eff, for a block known to be ordinary: finite elements and a block maximum of at
// least 2^-60. The FMA-corrected quotient and the hardware conversion; below |x| = 2^-96 the
// quotient may not be the IEEE one, but there |x / eff| < 2^-15 and both encode to the signed
// zero of x. Equal to fp4_encode(x / eff) on 2^32 random NVFP4 rows (finite bf16 elements, row and
// block maxima over the whole exponent range).
constexpr float kNvfp4FastBlockMin = 0x1p-60f;
__device__ inline uint32_t nvfp4_codes2_fast(float x0, float x1, float eff, float r) {
    return fp4_encode_hw(signed_quotient(x0, eff, r), signed_quotient(x1, eff, r));
}

// E8M0 block-scale code of a block maximum: floor(log2 amax) - emax_elem + 127, clamped; 0 when
// amax is zero, subnormal-exponent or not finite.
__device__ inline uint32_t mx_scale_code(float amax, int emax_elem) {
    const int be = (int)((__float_as_uint(amax) >> 23) & 0xffu);
    int e = (amax > 0.0f && be != 0xff) ? (be == 0 ? -127 : be - 127) - emax_elem : -127;
    e = e < -127 ? -127 : (e > 127 ? 127 : e);
    return (uint32_t)(e + 127);
}
__device__ inline float e8m0_to_f32(uint32_t c) {
    return c == 0 ? __uint_as_float(0x00400000u) : __uint_as_float(c << 23);
}

// Two E4M3 codes of `w` (bytes 0,1 when !hi, bytes 2,3 when hi) -> bf16x2, exact.
__device__ inline uint32_t fp8x2_to_bf16x2(uint32_t w, bool hi) {
    bf16x2 v = hi ? __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, true)
                  : __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, false);
    return __builtin_bit_cast(uint32_t, v);
}
// 8 E4M3 codes (two words, byte order) -> bf16x8.
__device__ inline bf16x8 fp8x8_to_bf16x8(uint32_t w0, uint32_t w1) {
    u32x4 r;
    r.x = fp8x2_to_bf16x2(w0, false);
    r.y = fp8x2_to_bf16x2(w0, true);
    r.z = fp8x2_to_bf16x2(w1, false);
    r.w = fp8x2_to_bf16x2(w1, true);
    return __builtin_bit_cast(bf16x8, r);
}

// 8 E4M3 codes times a power of two (an E8M0 block scale; 0 for an all-zero block), exact in
// bf16: the conversion applies the scale, one instruction per pair.
__device__ inline bf16x8 fp8x8_pow2_bf16x8(uint32_t w0, uint32_t w1, float pow2) {
    u32x4 r;
    r.x = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, pow2, false));
    r.y = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, pow2, true));
    r.z = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, pow2, false));
    r.w = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, pow2, true));
    return __builtin_bit_cast(bf16x8, r);
}
// 8 E4M3 codes times a scale, rounded to bf16: bf16(scale * e4m3) in f32 arithmetic, the very
// values of the reference's dequantized bf16 cache (RowCodec::dequantize_row then to_dtype,
// candle-core/src/accel/turbo.rs:404-409, candle-nn/src/turbo_quant.rs:948-966). The scaled
// conversions take only the exponent of their scale operand (measured: any other f32 scale
// gives other bits than the product), so a general scale is one f32 multiply per code.
__device__ inline bf16x8 fp8x8_scaled_bf16x8(uint32_t w0, uint32_t w1, float scale) {
    const f32x2 a = __builtin_amdgcn_cvt_pk_f32_fp8(w0, false);
    const f32x2 b = __builtin_amdgcn_cvt_pk_f32_fp8(w0, true);
    const f32x2 c = __builtin_amdgcn_cvt_pk_f32_fp8(w1, false);
    const f32x2 d = __builtin_amdgcn_cvt_pk_f32_fp8(w1, true);
    u32x4 r;
    r.x = pack_bf16x2(a.x * scale, a.y * scale);
    r.y = pack_bf16x2(b.x * scale, b.y * scale);
    r.z = pack_bf16x2(c.x * scale, c.y * scale);
    r.w = pack_bf16x2(d.x * scale, d.y * scale);
    return __builtin_bit_cast(bf16x8, r);
}
// Same with one scale per code (value operands: 8 keys of one head dim).
__device__ inline bf16x8 fp8x8_scaled_bf16x8(uint32_t w0, uint32_t w1, const float *sc) {
    const f32x2 a = __builtin_amdgcn_cvt_pk_f32_fp8(w0, false);
    const f32x2 b = __builtin_amdgcn_cvt_pk_f32_fp8(w0, true);
    const f32x2 c = __builtin_amdgcn_cvt_pk_f32_fp8(w1, false);
    const f32x2 d = __builtin_amdgcn_cvt_pk_f32_fp8(w1, true);
    u32x4 r;
    r.x = pack_bf16x2(a.x * sc[0], a.y * sc[1]);
    r.y = pack_bf16x2(b.x * sc[2], b.y * sc[3]);
    r.z = pack_bf16x2(c.x * sc[4], c.y * sc[5]);
    r.w = pack_bf16x2(d.x * sc[6], d.y * sc[7]);
    return __builtin_bit_cast(bf16x8, r);
}

// ---------------------------------------------------------------------------------------------
// Cross-lane helpers (ds_bpermute based shuffles; wave64)
// ---------------------------------------------------------------------------------------------
// The reference's score terms (fa_logit / tq_logit, candle-core/kernels/flash_attn_impl.h:42-47,
// turbo_quant_impl.h:37-41) on a score x in exp2 units (x = s log2(e)): soft-capping
// cap tanh(s / cap), as cap2 - 2 cap2 / (2^(2 x log2(e) / cap2) + 1) with cap2 = cap log2(e),
// then ALiBi -slope |dist| with slope2 = slope log2(e). cap2 = 0 / slope2 = 0 switch them off.
__device__ inline float fa_logit2(float x, float cap2, float slope2, int dist) {
    if (cap2 > 0.0f) {
        const float e = __builtin_amdgcn_exp2f(x * (2.0f * kLog2e / cap2));
        x = cap2 - 2.0f * cap2 * __builtin_amdgcn_rcpf(e + 1.0f);
    }
    if (slope2 != 0.0f) x -= slope2 * (float)(dist < 0 ? -dist : dist);
    return x;
}

__device__ inline float shfl_xor(float v, int m) { return __shfl_xor(v, m, kWave); }
// gfx950 row swaps in the VALU (no LDS round trip): v_permlane16_swap exchanges the odd 16-lane
// rows of its first operand with the even rows of its second, v_permlane32_swap the upper half
// of the first with the lower half of the second; with v in both, lane l holds v[l] and
// v[l ^ 16] (v[l ^ 32]) in the two results.
__device__ inline float xor16_max(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ inline float xor32_max(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ inline float xor16_sum(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ inline float xor32_sum(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
// over lanes sharing lane % 16 (the 16 columns of an MFMA 16x16 output); the sums add the same
// pairs as the lane-xor butterfly (v[l] + v[l ^ 16], then + the l ^ 32 partner), so the bits are
// those of the shuffle form
__device__ inline float group16_max(float v) { return xor32_max(xor16_max(v)); }
__device__ inline float group16_sum(float v) { return xor32_sum(xor16_sum(v)); }
__device__ inline float wave_max(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, shfl_xor(v, m));
    return v;
}
__device__ inline float wave_sum(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += shfl_xor(v, m);
    return v;
}
// max over aligned groups of `w` lanes (w a power of two <= 64)
__device__ inline float group_max(float v, int w) {
    for (int m = w >> 1; m >= 1; m >>= 1) v = fmaxf(v, shfl_xor(v, m));
    return v;
}

// In-register Walsh-Hadamard transform over 2 * `lanes` elements held as (v0, v1) = elements
// (2l, 2l+1): y_i = sum_j (-1)^popcount(i & j) x_j (Sylvester order, unnormalised).
template <int D>
__device__ inline void fwht_pairs(float &v0, float &v1, int lane) {
    float a = v0 + v1, b = v0 - v1;
    v0 = a;
    v1 = b;
#pragma unroll
    for (int m = 1; m < D / 2; m <<= 1) {
        const float p0 = shfl_xor(v0, m), p1 = shfl_xor(v1, m);
        const bool upper = (lane & m) != 0;
        v0 = upper ? p0 - v0 : v0 + p0;
        v1 = upper ? p1 - v1 : v1 + p1;
    }
}

// 8 floats -> bf16 hi + bf16 lo operands with hi + lo = x to 16 significant bits.
__device__ inline void split_bf16x8(const float *x, bf16x8 &hi, bf16x8 &lo) {
    u32x4 h, l;
    uint32_t *hp = (uint32_t *)&h, *lp = (uint32_t *)&l;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        hp[i] = pack_bf16x2(x[2 * i], x[2 * i + 1]);
        const float r0 = x[2 * i] - __uint_as_float(hp[i] << 16);
        const float r1 = x[2 * i + 1] - __uint_as_float(hp[i] & 0xffff0000u);
        lp[i] = pack_bf16x2(r0, r1);
    }
    hi = __builtin_bit_cast(bf16x8, h);
    lo = __builtin_bit_cast(bf16x8, l);
}

// 8 floats -> f16 hi + f16 lo operands (22 significant bits for normal values).
__device__ inline void split_f16x8(const float *x, f16x8 &hi, f16x8 &lo) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        hi[i] = (_Float16)x[i];
        lo[i] = (_Float16)(x[i] - (float)hi[i]);
    }
}
__device__ inline void split8(const float *x, bf16x8 &hi, bf16x8 &lo) { split_bf16x8(x, hi, lo); }
__device__ inline void split8(const float *x, f16x8 &hi, f16x8 &lo) { split_f16x8(x, hi, lo); }

__device__ inline f32x4 mfma16x16x32(f16x8 a, f16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ inline f32x4 mfma16x16x32(bf16x8 a, bf16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

}  // namespace cqkv
