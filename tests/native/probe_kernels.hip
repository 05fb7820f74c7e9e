// Test-only kernels (built into tests/native/libcqkv_probe.so, not part of libcqkv.so): exhaustive
// and randomized checks of the device E4M3 conversions that the cache encoders use, run over far
// more inputs than a row-level test can carry. They call the very functions of cqkv_device.h that
// the encoders call.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../candle-rocm-vulkan_amd/csrc/cqkv_device.h"

using namespace cqkv;

namespace {

// Code of the non-negative f32 pattern u expected from the reference encoder: the number of
// thresholds at or below u, thr[c - 1] being the first pattern whose code is at least c (the
// encoder is monotone in the pattern of a non-negative input).
__device__ inline uint32_t code_of(const uint32_t *thr, int nthr, uint32_t u) {
    int lo = 0, hi = nthr;  // first index with thr[i] > u
    while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (thr[mid] <= u) lo = mid + 1;
        else hi = mid;
    }
    return (uint32_t)lo;
}

struct SweepArgs {
    uint32_t lo, hi;  // non-negative patterns [lo, hi); each is checked with both signs
    const uint32_t *thr;
    int32_t nthr;
    unsigned long long *bad;  // [0] hardware conversion, [1] software encoder
    uint32_t *first_bad;      // smallest pattern with a mismatch (either path)
};

__global__ __launch_bounds__(256) void e4m3_sweep_kernel(SweepArgs a) {
    __shared__ uint32_t thr[128];
    for (int i = threadIdx.x; i < a.nthr; i += blockDim.x) thr[i] = a.thr[i];
    __syncthreads();
    unsigned long long bad_hw = 0, bad_sw = 0;
    uint32_t first = 0xffffffffu;
    const uint64_t step = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t u = a.lo + (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; u < a.hi; u += step) {
        const uint32_t c = code_of(thr, a.nthr, (uint32_t)u);
        const uint32_t want = c | ((0x80u | c) << 8);  // x, then -x (signed zero included)
        const float x = __uint_as_float((uint32_t)u);
        const uint32_t hw = e4m3_encode2(x, -x);
        const uint32_t sw = e4m3_encode(x) | (e4m3_encode(-x) << 8);
        if (hw != want) {
            ++bad_hw;
            first = min(first, (uint32_t)u);
        }
        if (sw != want) {
            ++bad_sw;
            first = min(first, (uint32_t)u);
        }
    }
    if (bad_hw) atomicAdd(a.bad, bad_hw);
    if (bad_sw) atomicAdd(a.bad + 1, bad_sw);
    if (first != 0xffffffffu) atomicMin(a.first_bad, first);
}

__device__ inline uint64_t splitmix64(uint64_t z) {
    z += 0x9e3779b97f4a7c15ull;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

// a finite bf16 value from 16 random bits (exponent 0xff folded onto 0xfe)
__device__ inline float finite_bf16(uint32_t bits) {
    if (((bits >> 7) & 0xffu) == 0xffu) bits &= ~0x0080u;
    return __uint_as_float(bits << 16);
}

struct QuotientArgs {
    uint64_t n, seed;
    unsigned long long *bad;
    uint64_t *first_bad;  // smallest sample index with a mismatch
};

// The FP8 row encoder's codes of (x, y) in a row whose absmax is max(|x|, |y|): the fast path
// (fp8_row_codes: one reciprocal per row, FMA-corrected quotients, hardware conversion) against
// the IEEE quotient x / s through the software encoder. x and y are random finite bf16 values
// over the whole exponent range (the encoders' inputs are bf16 / f16 / f32 rows).
__global__ __launch_bounds__(256) void fp8_quotient_kernel(QuotientArgs a) {
    unsigned long long bad = 0;
    uint64_t first = ~0ull;
    const uint64_t step = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < a.n; i += step) {
        const uint64_t h = splitmix64(a.seed + i);
        const float x = finite_bf16((uint32_t)h & 0xffffu);
        const float y = finite_bf16((uint32_t)(h >> 16) & 0xffffu);
        const float amax = fmaxf(__builtin_fabsf(x), __builtin_fabsf(y));
        const float s = amax > 0.0f ? amax / 448.0f : 1.0f;
        const float r = 1.0f / s;
        // the per-row choice of the encoders: the division-free path for ordinary rows
        const uint32_t fast = amax >= kFp8FastRowMin ? fp8_row_codes_fast(x, y, s, r)
                                                     : fp8_row_codes(x, y, s, r);
        const uint32_t ref = e4m3_encode(x / s) | (e4m3_encode(y / s) << 8);
        if (fast != ref) {
            ++bad;
            first = first < i ? first : i;
        }
    }
    if (bad) {
        atomicAdd(a.bad, bad);
        atomicMin((unsigned long long *)a.first_bad, (unsigned long long)first);
    }
}

// E2M1 (FP4) codes of the non-negative f32 patterns [lo, hi), both signs, from the gfx950
// conversion at scale 1 (fp4_encode_hw) and from the device software encoder (fp4_encode),
// against the reference encoder's 7 code thresholds.
__global__ __launch_bounds__(256) void fp4_sweep_kernel(SweepArgs a) {
    __shared__ uint32_t thr[8];
    if (threadIdx.x < (unsigned)a.nthr) thr[threadIdx.x] = a.thr[threadIdx.x];
    __syncthreads();
    unsigned long long bad_hw = 0, bad_sw = 0;
    uint32_t first = 0xffffffffu;
    const uint64_t step = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t u = a.lo + (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; u < a.hi; u += step) {
        const uint32_t c = code_of(thr, a.nthr, (uint32_t)u);
        const uint32_t want = c | ((8u | c) << 4);  // x, then -x (signed zero included)
        const float x = __uint_as_float((uint32_t)u);
        const uint32_t hw = fp4_encode_hw(x, -x);
        const uint32_t sw = fp4_encode(x) | (fp4_encode(-x) << 4);
        if (hw != want) {
            ++bad_hw;
            first = min(first, (uint32_t)u);
        }
        if (sw != want) {
            ++bad_sw;
            first = min(first, (uint32_t)u);
        }
    }
    if (bad_hw) atomicAdd(a.bad, bad_hw);
    if (bad_sw) atomicAdd(a.bad + 1, bad_sw);
    if (first != 0xffffffffu) atomicMin(a.first_bad, first);
}

// The NVFP4 encoder's element codes: E2M1 of x / eff, eff = e4m3(cs) * g with g = amax / 2688
// and cs = E4M3(bmax / 6 / g) (turbo.rs:348-365), by the encoder's per-block choice (the
// FMA-corrected quotient from r = 1 / eff and the hardware conversion for blocks of maximum at
// least 2^-60), against the IEEE quotient through the software encoder. Random finite bf16 x,
// and a row max amax and block max bmax with |x| <= bmax <= amax, all over the whole exponent
// range.
__global__ __launch_bounds__(256) void nvfp4_quotient_kernel(QuotientArgs a) {
    unsigned long long bad = 0;
    uint64_t first = ~0ull;
    const uint64_t step = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < a.n; i += step) {
        const uint64_t h = splitmix64(a.seed + i);
        const float x = finite_bf16((uint32_t)h & 0xffffu);
        const float u = __builtin_fabsf(finite_bf16((uint32_t)(h >> 16) & 0xffffu));
        const float w = __builtin_fabsf(finite_bf16((uint32_t)(h >> 32) & 0xffffu));
        const float bmax = fmaxf(__builtin_fabsf(x), fminf(u, w));
        const float amax = fmaxf(bmax, fmaxf(u, w));
        const float gs = amax > 0.0f ? amax / 2688.0f : 1.0f;
        const uint32_t cs = e4m3_encode(bmax / 6.0f / gs);
        const float eff = __builtin_amdgcn_cvt_f32_fp8(cs, 0) * gs;
        if (!(eff > 0.0f)) continue;
        const float y = finite_bf16((uint32_t)(h >> 48) & 0xffffu);
        const float y2 = __builtin_fabsf(y) <= bmax ? y : -x;
        // the per-block choice of the encoder: the division-free path for ordinary blocks
        const uint32_t fast = bmax >= kNvfp4FastBlockMin
                                  ? nvfp4_codes2_fast(x, y2, eff, 1.0f / eff)
                                  : fp4_encode(x / eff) | (fp4_encode(y2 / eff) << 4);
        const uint32_t ref = fp4_encode(x / eff) | (fp4_encode(y2 / eff) << 4);
        if (fast != ref) {
            ++bad;
            first = first < i ? first : i;
        }
    }
    if (bad) {
        atomicAdd(a.bad, bad);
        atomicMin((unsigned long long *)a.first_bad, (unsigned long long)first);
    }
}

}  // namespace

#define PROBE_CHECK(x)                              \
    do {                                            \
        if ((x) != hipSuccess) return -2;           \
    } while (0)

extern "C" int probe_e4m3_sweep(uint32_t lo, uint32_t hi, const uint32_t *thresholds, int nthr,
                                uint64_t *bad_out, uint32_t *first_bad_out) {
    if (nthr <= 0 || nthr > 128 || lo > hi) return -1;
    uint32_t *d_thr = nullptr, *d_first = nullptr;
    unsigned long long *d_bad = nullptr;
    PROBE_CHECK(hipMalloc(&d_thr, 128 * 4));
    PROBE_CHECK(hipMalloc(&d_bad, 16));
    PROBE_CHECK(hipMalloc(&d_first, 4));
    PROBE_CHECK(hipMemcpy(d_thr, thresholds, (size_t)nthr * 4, hipMemcpyHostToDevice));
    PROBE_CHECK(hipMemset(d_bad, 0, 16));
    PROBE_CHECK(hipMemset(d_first, 0xff, 4));
    SweepArgs a = {lo, hi, d_thr, nthr, d_bad, d_first};
    hipLaunchKernelGGL(e4m3_sweep_kernel, dim3(8192), dim3(256), 0, 0, a);
    PROBE_CHECK(hipGetLastError());
    PROBE_CHECK(hipDeviceSynchronize());
    PROBE_CHECK(hipMemcpy(bad_out, d_bad, 16, hipMemcpyDeviceToHost));
    PROBE_CHECK(hipMemcpy(first_bad_out, d_first, 4, hipMemcpyDeviceToHost));
    PROBE_CHECK(hipFree(d_thr));
    PROBE_CHECK(hipFree(d_bad));
    PROBE_CHECK(hipFree(d_first));
    return 0;
}

extern "C" int probe_fp8_quotient(uint64_t n, uint64_t seed, uint64_t *bad_out,
                                  uint64_t *first_bad_out) {
    unsigned long long *d_bad = nullptr;
    uint64_t *d_first = nullptr;
    PROBE_CHECK(hipMalloc(&d_bad, 8));
    PROBE_CHECK(hipMalloc(&d_first, 8));
    PROBE_CHECK(hipMemset(d_bad, 0, 8));
    PROBE_CHECK(hipMemset(d_first, 0xff, 8));
    QuotientArgs a = {n, seed, d_bad, d_first};
    hipLaunchKernelGGL(fp8_quotient_kernel, dim3(8192), dim3(256), 0, 0, a);
    PROBE_CHECK(hipGetLastError());
    PROBE_CHECK(hipDeviceSynchronize());
    PROBE_CHECK(hipMemcpy(bad_out, d_bad, 8, hipMemcpyDeviceToHost));
    PROBE_CHECK(hipMemcpy(first_bad_out, d_first, 8, hipMemcpyDeviceToHost));
    PROBE_CHECK(hipFree(d_bad));
    PROBE_CHECK(hipFree(d_first));
    return 0;
}

extern "C" int probe_fp4_sweep(uint32_t lo, uint32_t hi, const uint32_t *thresholds, int nthr,
                               uint64_t *bad_out, uint32_t *first_bad_out) {
    if (nthr <= 0 || nthr > 8 || lo > hi) return -1;
    uint32_t *d_thr = nullptr, *d_first = nullptr;
    unsigned long long *d_bad = nullptr;
    PROBE_CHECK(hipMalloc(&d_thr, 8 * 4));
    PROBE_CHECK(hipMalloc(&d_bad, 16));
    PROBE_CHECK(hipMalloc(&d_first, 4));
    PROBE_CHECK(hipMemcpy(d_thr, thresholds, (size_t)nthr * 4, hipMemcpyHostToDevice));
    PROBE_CHECK(hipMemset(d_bad, 0, 16));
    PROBE_CHECK(hipMemset(d_first, 0xff, 4));
    SweepArgs a = {lo, hi, d_thr, nthr, d_bad, d_first};
    hipLaunchKernelGGL(fp4_sweep_kernel, dim3(8192), dim3(256), 0, 0, a);
    PROBE_CHECK(hipGetLastError());
    PROBE_CHECK(hipDeviceSynchronize());
    PROBE_CHECK(hipMemcpy(bad_out, d_bad, 16, hipMemcpyDeviceToHost));
    PROBE_CHECK(hipMemcpy(first_bad_out, d_first, 4, hipMemcpyDeviceToHost));
    PROBE_CHECK(hipFree(d_thr));
    PROBE_CHECK(hipFree(d_bad));
    PROBE_CHECK(hipFree(d_first));
    return 0;
}

// Codes of a few single values through the FP4 conversion at a given scale operand (to read off
// whether the operand divides or multiplies): out[i] = byte of cvt(x[i], 0, scale).
__global__ void fp4_scale_kernel(const float *x, float scale, uint32_t *out, int n) {
    const int i = threadIdx.x;
    if (i < n) out[i] = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(0u, x[i], 0.0f, scale, 0) & 0xffu;
}

extern "C" int probe_fp4_scale(const float *x, int n, float scale, uint32_t *out) {
    if (n <= 0 || n > 256) return -1;
    float *dx = nullptr;
    uint32_t *dout = nullptr;
    PROBE_CHECK(hipMalloc(&dx, n * 4));
    PROBE_CHECK(hipMalloc(&dout, n * 4));
    PROBE_CHECK(hipMemcpy(dx, x, n * 4, hipMemcpyHostToDevice));
    hipLaunchKernelGGL(fp4_scale_kernel, dim3(1), dim3(256), 0, 0, dx, scale, dout, n);
    PROBE_CHECK(hipGetLastError());
    PROBE_CHECK(hipMemcpy(out, dout, n * 4, hipMemcpyDeviceToHost));
    PROBE_CHECK(hipFree(dx));
    PROBE_CHECK(hipFree(dout));
    return 0;
}

extern "C" int probe_nvfp4_quotient(uint64_t n, uint64_t seed, uint64_t *bad_out,
                                   uint64_t *first_bad_out) {
    unsigned long long *d_bad = nullptr;
    uint64_t *d_first = nullptr;
    PROBE_CHECK(hipMalloc(&d_bad, 8));
    PROBE_CHECK(hipMalloc(&d_first, 8));
    PROBE_CHECK(hipMemset(d_bad, 0, 8));
    PROBE_CHECK(hipMemset(d_first, 0xff, 8));
    QuotientArgs a = {n, seed, d_bad, d_first};
    hipLaunchKernelGGL(nvfp4_quotient_kernel, dim3(8192), dim3(256), 0, 0, a);
    PROBE_CHECK(hipGetLastError());
    PROBE_CHECK(hipDeviceSynchronize());
    PROBE_CHECK(hipMemcpy(bad_out, d_bad, 8, hipMemcpyDeviceToHost));
    PROBE_CHECK(hipMemcpy(first_bad_out, d_first, 8, hipMemcpyDeviceToHost));
    PROBE_CHECK(hipFree(d_bad));
    PROBE_CHECK(hipFree(d_first));
    return 0;
}
