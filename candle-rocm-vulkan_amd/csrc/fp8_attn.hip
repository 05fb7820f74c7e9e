// FP8 (E4M3) K / V with per-tensor descale factors: candle_nn::flash_attn::flash_attn_fp8 and the
// F8E4M3 K / V branch of flash_attn_with_config (paths relative to the reference repository
// root: candle-nn/src/flash_attn.rs:862-892 and FlashAttnConfig::descale :113-117; kernels
// candle-core/kernels/flash_attn_impl.h:52-63, 153, 381, 434: scores dot * k_descale, outputs
// times v_descale / l).
//
//  * cqkv_fp8_quantize_tensor: the per-tensor quantization of flash_attn_fp8 (:882-887):
//    amax = max |x|, scale = amax > 0 ? amax / 448 : 1, codes E4M3(x * f32(1 / f64(scale)) + 0)
//    (candle's `x / scale` is affine(1 / scale, 0), candle-core/src/tensor.rs:3124 and
//    cpu_backend/mod.rs:313-315). The scale is written to device memory, so nothing waits on the
//    host. Three launches: clear the maximum, the maximum (at most 512 workgroups, one atomic
//    each on the float bits), the codes.
//  * cqkv_flash_attn_fp8: K and V are E4M3 tensors (E4M3 is exact in bf16 and f16). Calls the
//    MFMA prefill takes (bf16 / f16 queries, D = 128, more than 16 queries) widen the codes in
//    its V^T pre-pass, K into the workspace and V straight into V^T, one pass over the codes;
//    other calls first write K and V in the query dtype into the workspace (fp8_stage_kernel)
//    and run the plain-dtype kernels on that. k_descale is folded into the query pre-scale and
//    v_descale into the output normalisation. f32 queries read the codes directly.
#include "cqkv_device.h"
#include "cqkv_host.h"

namespace cqkv {

struct Fp8QuantArgs {
    const void *x;
    int64_t n;
    int32_t dtype;
    uint8_t *codes;
    float *scale;  // [0] the scale, [1] the maximum |x| as float bits (scratch)
};

__global__ __launch_bounds__(64) void fp8_clear_kernel(float *scale) {
    if (threadIdx.x == 0) ((uint32_t *)scale)[1] = 0u;
}

__global__ __launch_bounds__(256) void fp8_amax_kernel(Fp8QuantArgs a) {
    float m = 0.0f;
    const int64_t t0 = (int64_t)blockIdx.x * 256 + threadIdx.x, step = (int64_t)gridDim.x * 256;
    int64_t tail = 0;
    if (a.dtype != CQKV_F32 && ((uintptr_t)a.x & 15) == 0) {
        // 16-bit elements, 16-byte aligned: 8 per load
        const int64_t n8 = a.n / 8;
        const bool bf = a.dtype == CQKV_BF16;
        auto fold = [&](const u32x4 &w) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float lo = bf ? bf16_bits_to_f32(w[e] & 0xffffu) : f16_bits_to_f32(w[e] & 0xffffu);
                const float hi = bf ? bf16_bits_to_f32(w[e] >> 16) : f16_bits_to_f32(w[e] >> 16);
                m = fmaxf(m, fmaxf(__builtin_fabsf(lo), __builtin_fabsf(hi)));
            }
        };
        int64_t i = t0;
        for (; i + 3 * step < n8; i += 4 * step) {  // four loads in flight
            const u32x4 w0 = ((const u32x4 *)a.x)[i], w1 = ((const u32x4 *)a.x)[i + step];
            const u32x4 w2 = ((const u32x4 *)a.x)[i + 2 * step], w3 = ((const u32x4 *)a.x)[i + 3 * step];
            fold(w0);
            fold(w1);
            fold(w2);
            fold(w3);
        }
        for (; i < n8; i += step) fold(((const u32x4 *)a.x)[i]);
        tail = n8 * 8;
    }
    for (int64_t i = tail + t0; i < a.n; i += step)
        m = fmaxf(m, __builtin_fabsf(load_elem(a.x, i, a.dtype)));
    m = wave_max(m);
    __shared__ float part[4];
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = m;
    __syncthreads();
    if (threadIdx.x == 0) {
        const float b = fmaxf(fmaxf(part[0], part[1]), fmaxf(part[2], part[3]));
        // non-negative floats order as their bit patterns; fmaxf skips NaN inputs, as Rust's
        // f32::max in candle's max_all does
        atomicMax((uint32_t *)a.scale + 1, __float_as_uint(b));
    }
}

__global__ __launch_bounds__(256) void fp8_quant_kernel(Fp8QuantArgs a) {
    const float amax = __uint_as_float(((const uint32_t *)a.scale)[1]);
    const float s = amax > 0.0f ? amax / 448.0f : 1.0f;
    const float mul = (float)(1.0 / (double)s);
    if (blockIdx.x == 0 && threadIdx.x == 0) a.scale[0] = s;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < a.n; i += (int64_t)gridDim.x * 256) {
        const float q = load_elem(a.x, i, a.dtype) * mul + 0.0f;  // affine(mul, 0): -0 -> +0
        a.codes[i] = (uint8_t)e4m3_encode(q);
    }
}

struct Fp8StageArgs {
    const uint8_t *k, *v;
    int64_t k_sb, k_st, k_sh, v_sb, v_st, v_sh;  // element strides: batch, token, head
    uint16_t *kb, *vb;                           // (batch, kv_heads, kv_len, D) of the dtype
    int32_t kv_len, kv_heads, head_dim, f16;
};

// One thread per 8 head dims of one token: 8 code bytes in, their 8 bf16 / f16 values out (exact
// in either: E4M3 has 4 significant bits and its range inside both), K and V.
__global__ __launch_bounds__(256) void fp8_stage_kernel(Fp8StageArgs a) {
    const int h = blockIdx.y, b = blockIdx.z;
    const int cpt = a.head_dim / 8, tpb = 256 / cpt;  // chunks per token, tokens per block
    const int t = blockIdx.x * tpb + (int)threadIdx.x / cpt, c = (int)threadIdx.x % cpt;
    if ((int)threadIdx.x >= tpb * cpt || t >= a.kv_len) return;
    const int64_t dst = (((int64_t)b * a.kv_heads + h) * a.kv_len + t) * a.head_dim + 8 * c;
    const uint8_t *kp = a.k + (int64_t)b * a.k_sb + (int64_t)t * a.k_st + (int64_t)h * a.k_sh + 8 * c;
    const uint8_t *vp = a.v + (int64_t)b * a.v_sb + (int64_t)t * a.v_st + (int64_t)h * a.v_sh + 8 * c;
    const u32x2 kw = *(const u32x2 *)kp, vw = *(const u32x2 *)vp;
    f32x2 kf[4], vf[4];  // code pairs (0,1) (2,3) of each word: the selector is an immediate
    kf[0] = __builtin_amdgcn_cvt_pk_f32_fp8(kw.x, false);
    kf[1] = __builtin_amdgcn_cvt_pk_f32_fp8(kw.x, true);
    kf[2] = __builtin_amdgcn_cvt_pk_f32_fp8(kw.y, false);
    kf[3] = __builtin_amdgcn_cvt_pk_f32_fp8(kw.y, true);
    vf[0] = __builtin_amdgcn_cvt_pk_f32_fp8(vw.x, false);
    vf[1] = __builtin_amdgcn_cvt_pk_f32_fp8(vw.x, true);
    vf[2] = __builtin_amdgcn_cvt_pk_f32_fp8(vw.y, false);
    vf[3] = __builtin_amdgcn_cvt_pk_f32_fp8(vw.y, true);
    u32x4 ko, vo;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        ko[i] = a.f16 ? pack_f16x2(kf[i].x, kf[i].y) : pack_bf16x2(kf[i].x, kf[i].y);
        vo[i] = a.f16 ? pack_f16x2(vf[i].x, vf[i].y) : pack_bf16x2(vf[i].x, vf[i].y);
    }
    *(u32x4 *)(a.kb + dst) = ko;
    *(u32x4 *)(a.vb + dst) = vo;
}

}  // namespace cqkv

using namespace cqkv;

extern "C" int cqkv_fp8_quantize_tensor(const void *x, int32_t x_dtype, int64_t n, uint8_t *codes,
                                        float *scale, cqkv_stream_t stream) {
    clear_error();
    if (!x || !codes || !scale) return fail(CQKV_ERR_ARG, "cqkv_fp8_quantize_tensor: null pointer");
    if (x_dtype < CQKV_BF16 || x_dtype > CQKV_F32)
        return fail(CQKV_ERR_ARG, "cqkv_fp8_quantize_tensor: dtype %d", x_dtype);
    if (n < 0) return fail(CQKV_ERR_ARG, "cqkv_fp8_quantize_tensor: n %lld", (long long)n);
    const hipStream_t st = (hipStream_t)stream;
    Fp8QuantArgs a = {x, n, x_dtype, codes, scale};
    const int64_t want = (n + 255) / 256;
    const unsigned blocks = (unsigned)(want < 1 ? 1 : (want > 4096 ? 4096 : want));
    // the maximum: few workgroups, since each ends with an atomic on the one address
    const unsigned mblocks = blocks > 512 ? 512 : blocks;
    hipLaunchKernelGGL(fp8_clear_kernel, dim3(1), dim3(64), 0, st, scale);
    hipLaunchKernelGGL(fp8_amax_kernel, dim3(mblocks), dim3(256), 0, st, a);
    hipLaunchKernelGGL(fp8_quant_kernel, dim3(blocks), dim3(256), 0, st, a);
    CQKV_HIP_CHECK(hipGetLastError());
    return CQKV_OK;
}

// Workspace of cqkv_flash_attn_fp8: the staged K / V (dtype copies of the codes), 256-aligned,
// then the attention's own (flash_attn_workspace); 0 for invalid sizes. It also covers the MFMA
// prefill's E4M3 path (V^T and the widened K, prefill_e4m3_workspace), which needs less.
static size_t fp8_stage_bytes(int32_t batch, int32_t kv_len, int32_t kv_heads, int32_t head_dim) {
    return ((size_t)batch * kv_heads * kv_len * head_dim * 2 * 2 + 255) / 256 * 256;
}

extern "C" size_t cqkv_flash_attn_fp8_workspace_bytes(int32_t dtype, int32_t batch, int32_t q_len,
                                                      int32_t kv_len, int32_t q_heads,
                                                      int32_t kv_heads, int32_t head_dim) {
    // (no query rows or no keys need nothing: see cqkv_flash_attn_fp8)
    if ((dtype != CQKV_BF16 && dtype != CQKV_F16 && dtype != CQKV_F32) || batch <= 0 ||
        q_len <= 0 || kv_len <= 0 || q_heads <= 0 || kv_heads <= 0 || q_heads % kv_heads != 0 ||
        head_dim <= 0 || head_dim > 256 || head_dim % 8 != 0)
        return 0;
    // f32 queries read the codes directly (no staged copy)
    const size_t stage = dtype == CQKV_F32 ? 0 : fp8_stage_bytes(batch, kv_len, kv_heads, head_dim);
    return stage +
           flash_attn_workspace(dtype, batch, q_len, kv_len, q_heads, kv_heads, head_dim, false);
}

extern "C" int cqkv_flash_attn_fp8(const void *q, const int64_t q_strides[3], const void *k8,
                                   const int64_t k_strides[3], const void *v8,
                                   const int64_t v_strides[3], void *out,
                                   const int64_t out_strides[3], int32_t dtype, int32_t batch,
                                   int32_t q_len, int32_t kv_len, int32_t q_heads,
                                   int32_t kv_heads, int32_t head_dim, float softmax_scale,
                                   int32_t window_left, int32_t window_right, float k_descale,
                                   float v_descale, const float *k_scale, const float *v_scale,
                                   void *workspace, size_t workspace_bytes, cqkv_stream_t stream) {
    clear_error();
    static const char *who = "cqkv_flash_attn_fp8";
    if (!q_strides || !k_strides || !v_strides || !out_strides)
        return fail(CQKV_ERR_ARG, "%s: null strides", who);
    if (dtype != CQKV_BF16 && dtype != CQKV_F16 && dtype != CQKV_F32)
        return fail(CQKV_ERR_ARG, "%s: dtype %d (bf16, f16 or f32 q / out)", who, dtype);
    if (head_dim <= 0 || head_dim > 256 || head_dim % 8 != 0)
        return fail(CQKV_ERR_ARG, "%s: head_dim %d (a multiple of 8 up to 256)", who, head_dim);
    // the attention's own limits, checked before the staging pass is launched
    if (batch < 0 || q_len < 0 || kv_len < 0 || kv_heads <= 0 || q_heads <= 0 ||
        q_heads % kv_heads != 0 || kv_len > (1 << 23))
        return fail(CQKV_ERR_ARG, "%s: batch %d q_len %d kv_len %d heads %d / %d", who, batch,
                    q_len, kv_len, q_heads, kv_heads);
    // empty inputs as the reference's: no query rows give an empty output, no keys zero rows;
    // empty tensors may have null data
    const bool no_rows = batch == 0 || q_len == 0;
    if (no_rows) return CQKV_OK;
    if (!q || !out || (kv_len > 0 && (!k8 || !v8)))
        return fail(CQKV_ERR_ARG, "%s: null tensor", who);
    if (!(k_descale == k_descale) || !(v_descale == v_descale))
        return fail(CQKV_ERR_ARG, "%s: NaN descale", who);
    for (int i = 0; i < 3; ++i)
        if (k_strides[i] % 8 != 0 || v_strides[i] % 8 != 0)
            return fail(CQKV_ERR_ARG, "%s: K / V strides must be multiples of 8 bytes", who);
    if ((uintptr_t)k8 % 8 != 0 || (uintptr_t)v8 % 8 != 0)
        return fail(CQKV_ERR_ARG, "%s: K / V must be 8-byte aligned", who);
    if (kv_len == 0) {
        // zero rows from the plain kernel of the query dtype (no K / V is read)
        const int64_t ss[3] = {0, head_dim, 0};
        return flash_attn_impl(q, q_strides, nullptr, ss, nullptr, ss, out, out_strides, dtype,
                               dtype, batch, q_len, 0, q_heads, kv_heads, head_dim, softmax_scale,
                               window_left, window_right, 0.0f, nullptr, 0, nullptr, nullptr, 0, 0,
                               nullptr, nullptr, 0, nullptr, 0, stream, 1.0f, nullptr, 1.0f,
                               nullptr);
    }
    if (dtype == CQKV_F32) {
        // the f32-query kernel reads the E4M3 codes and widens them exactly, with k_descale in the
        // scores' scale and v_descale in the output, as the reference's fa_row_f32_fp8 does
        return flash_attn_impl(q, q_strides, k8, k_strides, v8, v_strides, out, out_strides, dtype,
                               kKvE4M3, batch, q_len, kv_len, q_heads, kv_heads, head_dim,
                               softmax_scale, window_left, window_right, 0.0f, nullptr, 0, nullptr,
                               nullptr, 0, 0, nullptr, nullptr, 0, workspace, workspace_bytes,
                               stream, k_descale, k_scale, v_descale, v_scale);
    }
    if (prefill_takes(dtype, head_dim, q_len, q, q_strides, out, out_strides)) {
        // the MFMA prefill's pre-pass widens the codes itself (K into the workspace, V into its
        // V^T), so no separate staging pass runs; a caller workspace is still held to the size
        // cqkv_flash_attn_fp8_workspace_bytes gives, whichever path the call takes
        const size_t need = cqkv_flash_attn_fp8_workspace_bytes(dtype, batch, q_len, kv_len,
                                                                q_heads, kv_heads, head_dim);
        if (workspace && workspace_bytes < need)
            return fail(CQKV_ERR_WORKSPACE, "%s: workspace %zu bytes, need %zu", who,
                        workspace_bytes, need);
        return flash_attn_impl(q, q_strides, k8, k_strides, v8, v_strides, out, out_strides, dtype,
                               kKvE4M3, batch, q_len, kv_len, q_heads, kv_heads, head_dim,
                               softmax_scale, window_left, window_right, 0.0f, nullptr, 0, nullptr,
                               nullptr, 0, 0, nullptr, nullptr, 0, workspace, workspace_bytes,
                               stream, k_descale, k_scale, v_descale, v_scale);
    }
    const hipStream_t st = (hipStream_t)stream;
    const size_t stage = fp8_stage_bytes(batch, kv_len, kv_heads, head_dim);
    const size_t need = cqkv_flash_attn_fp8_workspace_bytes(dtype, batch, q_len, kv_len, q_heads,
                                                            kv_heads, head_dim);
    void *ws = workspace;
    if (ws) {
        if (workspace_bytes < need)
            return fail(CQKV_ERR_WORKSPACE, "%s: workspace %zu bytes, need %zu", who,
                        workspace_bytes, need);
    } else {
        CQKV_HIP_CHECK(hipMallocAsync(&ws, need, st));
    }
    const size_t plane = (size_t)batch * kv_heads * kv_len * head_dim;
    Fp8StageArgs s = {};
    s.k = (const uint8_t *)k8;
    s.v = (const uint8_t *)v8;
    s.k_sb = k_strides[0];
    s.k_st = k_strides[1];
    s.k_sh = k_strides[2];
    s.v_sb = v_strides[0];
    s.v_st = v_strides[1];
    s.v_sh = v_strides[2];
    s.kb = (uint16_t *)ws;
    s.vb = (uint16_t *)ws + plane;
    s.kv_len = kv_len;
    s.kv_heads = kv_heads;
    s.head_dim = head_dim;
    s.f16 = dtype == CQKV_F16 ? 1 : 0;
    const int tpb = 256 / (head_dim / 8);
    hipLaunchKernelGGL(fp8_stage_kernel, dim3((kv_len + tpb - 1) / tpb, kv_heads, batch),
                       dim3(256), 0, st, s);
    int rc = CQKV_OK;
    if (hipGetLastError() != hipSuccess) {
        rc = fail(CQKV_ERR_HIP, "%s: staging launch failed", who);
    } else {
        // the staged K / V are (batch, kv_heads, kv_len, D): (batch, token, head) strides
        const int64_t ss[3] = {(int64_t)kv_heads * kv_len * head_dim, head_dim,
                               (int64_t)kv_len * head_dim};
        rc = flash_attn_impl(q, q_strides, s.kb, ss, s.vb, ss, out, out_strides, dtype, dtype, batch,
                             q_len, kv_len, q_heads, kv_heads, head_dim, softmax_scale,
                             window_left, window_right, 0.0f, nullptr, 0, nullptr, nullptr, 0, 0,
                             nullptr, nullptr, 0, (uint8_t *)ws + stage, need - stage, stream,
                             k_descale, k_scale, v_descale, v_scale);
    }
    if (!workspace) {
        const hipError_t fe = hipFreeAsync(ws, st);
        if (rc != CQKV_OK) return rc;
        CQKV_HIP_CHECK(fe);
    }
    return rc;
}

// ---------------------------------------------------------------------------------------------
// Hadamard rotation of rows (the incoherent processing of flash_attn_fp8, flash_attn.rs:868-880:
// q and k times rotation_matrix(d, Hadamard, seed)^T in f32, cast back to their dtype; the
// matrix is the sign-flipped Sylvester Hadamard / sqrt(d) of candle-core/src/accel/turbo.rs:
// 180-203, signs from SplitMix64(seed ^ "HADAMARD")). One wavefront per row: sign flip, the
// in-register transform, 1 / sqrt(d), the rounding to the dtype.
// ---------------------------------------------------------------------------------------------
namespace cqkv {

struct HadamardArgs {
    const void *x;
    void *out;
    int64_t rows, x_row, out_row;  // element strides between rows
    int32_t dtype;
    uint32_t sign_bits[8];
    float scale;
};

// D a power of two up to 128: lane l holds elements 2l, 2l+1 (lanes past D / 2 idle); D = 256:
// also 128 + 2l, 129 + 2l, the stride-128 stage in the lane (H_256 = H_2 x H_128).
template <int D>
__global__ __launch_bounds__(256) void hadamard_rows_kernel(HadamardArgs a) {
    constexpr int NP = D == 256 ? 2 : 1;  // element pairs per lane
    constexpr int DH = D == 256 ? 128 : D;
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= a.rows) return;
    const bool act = lane < DH / 2;
    float v[2 * NP] = {};
#pragma unroll
    for (int p = 0; p < NP; ++p)
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const int j = 128 * p + 2 * lane + e;
            if (act) {
                v[2 * p + e] = load_elem(a.x, row * a.x_row + j, a.dtype);
                if ((a.sign_bits[j >> 5] >> (j & 31)) & 1u) v[2 * p + e] = -v[2 * p + e];
            }
        }
#pragma unroll
    for (int p = 0; p < NP; ++p) fwht_pairs<DH>(v[2 * p], v[2 * p + 1], lane);
    if constexpr (NP == 2) {
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const float s0 = v[e] + v[2 + e], s1 = v[e] - v[2 + e];
            v[e] = s0;
            v[2 + e] = s1;
        }
    }
    if (!act) return;
#pragma unroll
    for (int p = 0; p < NP; ++p)
#pragma unroll
        for (int e = 0; e < 2; ++e)
            store_elem(a.out, row * a.out_row + 128 * p + 2 * lane + e, a.dtype, v[2 * p + e] * a.scale);
}

}  // namespace cqkv

extern "C" int cqkv_hadamard_rows(const void *x, int32_t dtype, int64_t rows, int64_t x_row_stride,
                                  int32_t head_dim, uint64_t seed, void *out,
                                  int64_t out_row_stride, cqkv_stream_t stream) {
    clear_error();
    if (!x || !out) return fail(CQKV_ERR_ARG, "cqkv_hadamard_rows: null pointer");
    if (dtype < CQKV_BF16 || dtype > CQKV_F32)
        return fail(CQKV_ERR_ARG, "cqkv_hadamard_rows: dtype %d", dtype);
    if (head_dim < 2 || head_dim > 256 || (head_dim & (head_dim - 1)) != 0)
        return fail(CQKV_ERR_ARG, "cqkv_hadamard_rows: head_dim %d (a power of two, 2-256)",
                    head_dim);
    // four rows per 256-thread workgroup along x: rows * 64 threads within one launch
    if (rows < 0 || rows > (int64_t)(UINT32_MAX / 64) || x_row_stride < head_dim ||
        out_row_stride < head_dim)
        return fail(CQKV_ERR_ARG, "cqkv_hadamard_rows: rows %lld / row strides", (long long)rows);
    if (rows == 0) return CQKV_OK;
    HadamardArgs a = {};
    a.x = x;
    a.out = out;
    a.rows = rows;
    a.x_row = x_row_stride;
    a.out_row = out_row_stride;
    a.dtype = dtype;
    float signs[256];
    turbo_signs(head_dim, seed, signs);
    for (int j = 0; j < head_dim; ++j)
        if (signs[j] < 0.0f) a.sign_bits[j >> 5] |= 1u << (j & 31);
    a.scale = 1.0f / sqrtf((float)head_dim);
    const dim3 grid((unsigned)((rows + 3) / 4));
    const hipStream_t st = (hipStream_t)stream;
    switch (head_dim) {
    case 2: hipLaunchKernelGGL(hadamard_rows_kernel<2>, grid, dim3(256), 0, st, a); break;
    case 4: hipLaunchKernelGGL(hadamard_rows_kernel<4>, grid, dim3(256), 0, st, a); break;
    case 8: hipLaunchKernelGGL(hadamard_rows_kernel<8>, grid, dim3(256), 0, st, a); break;
    case 16: hipLaunchKernelGGL(hadamard_rows_kernel<16>, grid, dim3(256), 0, st, a); break;
    case 32: hipLaunchKernelGGL(hadamard_rows_kernel<32>, grid, dim3(256), 0, st, a); break;
    case 64: hipLaunchKernelGGL(hadamard_rows_kernel<64>, grid, dim3(256), 0, st, a); break;
    case 128: hipLaunchKernelGGL(hadamard_rows_kernel<128>, grid, dim3(256), 0, st, a); break;
    default: hipLaunchKernelGGL(hadamard_rows_kernel<256>, grid, dim3(256), 0, st, a); break;
    }
    CQKV_HIP_CHECK(hipGetLastError());
    return CQKV_OK;
}
