// Dense bf16 flash attention (causal prefill) on MFMA for gfx950, with the FP8 quantize-and-append
// of K / V into the decode cache in the same call.
//
// Reference behaviour (paths relative to the reference repository root): FlashAttnOp /
// RocmStorage::flash_attn (candle-nn/src/flash_attn.rs:221-273, 339-350;
// candle-core/src/rocm_backend/accel.rs:54-158; tile kernel fa_tile_impl in
// candle-core/kernels/flash_attn_impl.h:330-443) behind candle_flash_attn::flash_attn
// (candle-flash-attn/src/lib.rs:149-157): softmax(scale q k^T) v with bottom-right aligned
// windows (causal = (-1, 0), candle-core/src/accel/attention.rs:80-92), bf16 in / out, f32
// accumulation; rows with no visible key give zeros.
//
// Kernel shape (one workgroup = 4 wavefronts = 64 queries of 4 query heads sharing a kv head):
//  * Both products run on v_mfma_f32_32x32x16_bf16. S^T = K Q^T: K (32 keys x 16 dims) comes
//    from LDS with ds_read_b128, Q^T stays in registers for the whole key loop. The S^T
//    accumulator of a lane holds one query column, so the row-wise online softmax needs one
//    cross-lane step, and its registers 4i0..4i0+7 are directly the P^T operand of a 16-key
//    step of O^T = V^T P^T (the k order inside a step is permuted to match).
//  * V^T operands come from the row-major V tile in LDS through ds_read_b64_tr_b16: in each
//    16-lane group, source lane 4p+q points at V[key0 + p][d0 + 4q .. +3], and lane i receives
//    V[key0 .. key0 + 3][d0 + i] - four keys of one head dim, the k-slots the MFMA needs.
//  * K / V tiles of 64 keys are double-buffered in LDS (rows padded to 288 B so the row reads of
//    ds_read_b128 and the 4-row groups of the transposing reads hit distinct banks); the next
//    tile's global loads are in flight while the current one is computed, one barrier per tile.
//  * Causal work is uneven: the workgroups with the most key tiles are dispatched first.
#include "cqkv_device.h"
#include "cqkv_host.h"

namespace cqkv {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

constexpr int kPfD = 128;          // head dim
constexpr int kPfBQ = 64;          // queries per wavefront (and per workgroup)
constexpr int kPfBK = 64;          // keys per tile
constexpr int kPfPitch = 288;      // LDS bytes per key row (256 + 32 padding)
constexpr int kPfTile = kPfBK * kPfPitch;  // one K or V tile in LDS

struct PrefillArgs {
    const uint16_t *q, *k, *v;
    uint16_t *out;
    int64_t q_sb, q_st, q_sh;  // element strides: batch, token, head
    int64_t k_sb, k_st, k_sh;
    int64_t v_sb, v_st, v_sh;
    int64_t o_sb, o_st, o_sh;
    int32_t q_len, kv_len, q_heads, kv_heads, group, heads_per_wg, q_blocks;
    int32_t wl, wr;
    float scale_log2;
};

__device__ inline f32x16 mfma32x32x16(bf16x8 a, bf16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__device__ inline u32x4 ldg128(const uint16_t *p) { return *(const u32x4 *)p; }

// visible keys [lo, hi) of query position i (bottom-right aligned)
__device__ inline void pf_key_range(int i, int lq, int lk, int wl, int wr, int &lo, int &hi) {
    const int pos = i + lk - lq;
    lo = wl >= 0 ? max(pos - wl, 0) : 0;
    hi = wr >= 0 ? min(pos + wr + 1, lk) : lk;
    lo = min(lo, lk);
    hi = max(hi, lo);
}

__global__ __launch_bounds__(256, 1) void prefill_kernel(PrefillArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];  // 2 stages x (K, V)
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int qr = lane & 31, h = lane >> 5;  // MFMA column / half

    // heaviest query blocks first
    const int qb = a.q_blocks - 1 - (int)blockIdx.x;
    const int hk = blockIdx.y % a.kv_heads;
    const int hgrp = blockIdx.y / a.kv_heads;
    const int b = blockIdx.z;
    const int head = hk * a.group + hgrp * a.heads_per_wg + wave;
    const bool wave_live = wave < a.heads_per_wg;
    const int q0 = qb * kPfBQ;

    // key tiles this workgroup visits
    int lo_first, hi_first, lo_last, hi_last;
    pf_key_range(q0, a.q_len, a.kv_len, a.wl, a.wr, lo_first, hi_first);
    pf_key_range(min(q0 + kPfBQ, a.q_len) - 1, a.q_len, a.kv_len, a.wl, a.wr, lo_last, hi_last);
    const int kt_begin = lo_first / kPfBK;
    const int kt_end = (hi_last + kPfBK - 1) / kPfBK;

    // ---- Q^T operands (B of S^T = K Q^T): lane (qr, h), N-block nb, k-step ks -> 8 dims ----
    bf16x8 qop[2][8];
    const uint16_t *qbase = a.q + (int64_t)b * a.q_sb + (int64_t)min(head, a.q_heads - 1) * a.q_sh;
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
        const int qi = q0 + 32 * nb + qr;
        const bool ok = wave_live && qi < a.q_len;
        const uint16_t *row = qbase + (int64_t)min(qi, a.q_len - 1) * a.q_st;
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) {
            u32x4 w = ok ? ldg128(row + 16 * ks + 8 * h) : u32x4{0u, 0u, 0u, 0u};
            qop[nb][ks] = __builtin_bit_cast(bf16x8, w);
        }
    }

    // per-lane query rows of the two N-blocks and their visible key ranges
    int qlo[2], qhi[2];
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
        const int qi = q0 + 32 * nb + qr;
        if (qi < a.q_len) pf_key_range(qi, a.q_len, a.kv_len, a.wl, a.wr, qlo[nb], qhi[nb]);
        else qlo[nb] = qhi[nb] = 0;
    }

    f32x16 acc[4][2];  // O^T: d-block md (32 dims), query block nb
#pragma unroll
    for (int md = 0; md < 4; ++md)
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) acc[md][nb] = f32x16{};
    float m_run[2] = {-__builtin_inff(), -__builtin_inff()}, l_run[2] = {0.f, 0.f};

    // ---- K / V staging: thread t copies key t / 4, dims 32 (t % 4) .. +31 of both tiles ----
    const int skey = threadIdx.x >> 2, spart = threadIdx.x & 3;
    const uint16_t *kbase = a.k + (int64_t)b * a.k_sb + (int64_t)hk * a.k_sh + 32 * spart;
    const uint16_t *vbase = a.v + (int64_t)b * a.v_sb + (int64_t)hk * a.v_sh + 32 * spart;
    u32x4 stk[4], stv[4];
    auto fetch = [&](int kt) {
        const int key = kt * kPfBK + skey;
        const bool ok = key < a.kv_len;
        const uint16_t *kr = kbase + (int64_t)min(key, a.kv_len - 1) * a.k_st;
        const uint16_t *vr = vbase + (int64_t)min(key, a.kv_len - 1) * a.v_st;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            stk[i] = ok ? ldg128(kr + 8 * i) : u32x4{0u, 0u, 0u, 0u};
            stv[i] = ok ? ldg128(vr + 8 * i) : u32x4{0u, 0u, 0u, 0u};
        }
    };
    auto stash = [&](int stage) {
        uint8_t *kt_lds = smem + stage * 2 * kPfTile;
        uint8_t *vt_lds = kt_lds + kPfTile;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            *(u32x4 *)(kt_lds + skey * kPfPitch + (32 * spart + 8 * i) * 2) = stk[i];
            *(u32x4 *)(vt_lds + skey * kPfPitch + (32 * spart + 8 * i) * 2) = stv[i];
        }
    };

    if (kt_begin < kt_end) fetch(kt_begin);
    for (int kt = kt_begin; kt < kt_end; ++kt) {
        const int stage = (kt - kt_begin) & 1;
        stash(stage);
        __syncthreads();
        if (kt + 1 < kt_end) fetch(kt + 1);
        if (!wave_live) continue;
        const uint8_t *k_lds = smem + stage * 2 * kPfTile;
        const uint8_t *v_lds = k_lds + kPfTile;
        const int k0 = kt * kPfBK;

        // S^T = K Q^T: key block mb (32 keys), query block nb
        f32x16 s[2][2];
#pragma unroll
        for (int mb = 0; mb < 2; ++mb) {
            s[mb][0] = f32x16{};
            s[mb][1] = f32x16{};
#pragma unroll
            for (int ks = 0; ks < 8; ++ks) {
                const bf16x8 kop = __builtin_bit_cast(
                    bf16x8, *(const u32x4 *)(k_lds + (32 * mb + qr) * kPfPitch + (16 * ks + 8 * h) * 2));
                s[mb][0] = mfma32x32x16(kop, qop[0][ks], s[mb][0]);
                s[mb][1] = mfma32x32x16(kop, qop[1][ks], s[mb][1]);
            }
        }
        // masks: only tiles that cross some query's visible range
        const bool full = k0 >= lo_last && k0 + kPfBK <= hi_first;
        if (!full) {
#pragma unroll
            for (int nb = 0; nb < 2; ++nb)
#pragma unroll
                for (int mb = 0; mb < 2; ++mb)
#pragma unroll
                    for (int j = 0; j < 16; ++j) {
                        const int key = k0 + 32 * mb + 8 * (j >> 2) + 4 * h + (j & 3);
                        if (!(key >= qlo[nb] && key < qhi[nb])) s[mb][nb][j] = -__builtin_inff();
                    }
        }
        // online softmax per query column (exp2 domain)
        bf16x8 pop[2][4];  // P^T operands: query block nb, 16-key step kk
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) {
            float mx = -__builtin_inff();
#pragma unroll
            for (int mb = 0; mb < 2; ++mb)
#pragma unroll
                for (int j = 0; j < 16; ++j) mx = fmaxf(mx, s[mb][nb][j]);
            mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
            const float m_new = fmaxf(m_run[nb], mx * a.scale_log2);
            const bool none = m_new == -__builtin_inff();
            const float alpha = none ? 1.0f : __builtin_amdgcn_exp2f(m_run[nb] - m_new);
            const float mneg = none ? 0.0f : m_new;
            float psum = 0.0f;
#pragma unroll
            for (int mb = 0; mb < 2; ++mb) {
                float p[16];
#pragma unroll
                for (int j = 0; j < 16; ++j) {
                    p[j] = __builtin_amdgcn_exp2f(s[mb][nb][j] * a.scale_log2 - mneg);
                    psum += p[j];
                }
#pragma unroll
                for (int half = 0; half < 2; ++half) {
                    u32x4 w;
                    w.x = pack_bf16x2(p[8 * half + 0], p[8 * half + 1]);
                    w.y = pack_bf16x2(p[8 * half + 2], p[8 * half + 3]);
                    w.z = pack_bf16x2(p[8 * half + 4], p[8 * half + 5]);
                    w.w = pack_bf16x2(p[8 * half + 6], p[8 * half + 7]);
                    pop[nb][2 * mb + half] = __builtin_bit_cast(bf16x8, w);
                }
            }
            l_run[nb] = l_run[nb] * alpha + psum;
            m_run[nb] = m_new;
            if (__any(alpha != 1.0f)) {
#pragma unroll
                for (int md = 0; md < 4; ++md) acc[md][nb] *= alpha;
            }
        }
        // O^T += V^T P^T: 16-key step kk = keys 32 mb + 16 i + [0, 16), mb = kk / 2, i = kk % 2
        const int g16 = lane >> 4, idx = lane & 15, sp = idx >> 2, sq = idx & 3;
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
            const int key0 = 32 * (kk >> 1) + 16 * (kk & 1) + 4 * h + sp;
#pragma unroll
            for (int md = 0; md < 4; ++md) {
                const int d0 = 32 * md + 16 * (g16 & 1) + 4 * sq;
                const uint8_t *src = v_lds + key0 * kPfPitch + d0 * 2;
                const s16x4 lo4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4 *)src);
                const s16x4 hi4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4 *)(src + 8 * kPfPitch));
                const u32x2 l2 = __builtin_bit_cast(u32x2, lo4), h2 = __builtin_bit_cast(u32x2, hi4);
                const bf16x8 vt = __builtin_bit_cast(bf16x8, u32x4{l2.x, l2.y, h2.x, h2.y});
                acc[md][0] = mfma32x32x16(vt, pop[0][kk], acc[md][0]);
                acc[md][1] = mfma32x32x16(vt, pop[1][kk], acc[md][1]);
            }
        }
    }
    if (!wave_live) return;

    // ---- normalise and write O (bf16): lane (qr, h), d = 32 md + 8 (j / 4) + 4 h + j % 4 ----
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
        const float l = l_run[nb] + __shfl_xor(l_run[nb], 32, 64);
        const float inv = l > 0.0f ? 1.0f / l : 0.0f;
        const int qi = q0 + 32 * nb + qr;
        if (qi >= a.q_len) continue;
        uint16_t *orow = a.out + (int64_t)b * a.o_sb + (int64_t)qi * a.o_st + (int64_t)head * a.o_sh;
#pragma unroll
        for (int md = 0; md < 4; ++md)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                u32x2 w;
                w.x = pack_bf16x2(acc[md][nb][4 * i + 0] * inv, acc[md][nb][4 * i + 1] * inv);
                w.y = pack_bf16x2(acc[md][nb][4 * i + 2] * inv, acc[md][nb][4 * i + 3] * inv);
                *(u32x2 *)(orow + 32 * md + 8 * i + 4 * h) = w;
            }
    }
}

int quant_append_launch(const cqkv_side *side, const void *x, int32_t x_dtype,
                        const int64_t xs[3], int32_t batch, int32_t tokens,
                        const int32_t *positions, int32_t position, hipStream_t stream);

}  // namespace cqkv

using namespace cqkv;

extern "C" int cqkv_flash_attn(const void *q, const int64_t q_strides[3], const void *k,
                               const int64_t k_strides[3], const void *v,
                               const int64_t v_strides[3], void *out,
                               const int64_t out_strides[3], int32_t batch, int32_t q_len,
                               int32_t kv_len, int32_t q_heads, int32_t kv_heads,
                               int32_t head_dim, float softmax_scale, int32_t window_left,
                               int32_t window_right, const cqkv_side *k_cache,
                               const cqkv_side *v_cache, int32_t position, cqkv_stream_t stream) {
    clear_error();
    if (!q || !k || !v || !out || !q_strides || !k_strides || !v_strides || !out_strides)
        return fail(CQKV_ERR_ARG, "cqkv_flash_attn: null tensor or strides");
    if (head_dim != kPfD)
        return fail(CQKV_ERR_ARG, "cqkv_flash_attn: head_dim %d not supported (128)", head_dim);
    if (batch <= 0 || q_len <= 0 || kv_len <= 0 || q_heads <= 0 || kv_heads <= 0 ||
        q_heads % kv_heads != 0)
        return fail(CQKV_ERR_ARG, "cqkv_flash_attn: batch %d q_len %d kv_len %d heads %d / %d",
                    batch, q_len, kv_len, q_heads, kv_heads);
    if ((k_cache == nullptr) != (v_cache == nullptr))
        return fail(CQKV_ERR_ARG, "cqkv_flash_attn: give both cache sides or neither");
    hipStream_t st = (hipStream_t)stream;
    if (k_cache) {
        if (int rc = check_side(k_cache, "cqkv_flash_attn (key cache)")) return rc;
        if (int rc = check_side(v_cache, "cqkv_flash_attn (value cache)")) return rc;
        if (k_cache->format != CQKV_FMT_FP8 || v_cache->format != CQKV_FMT_FP8 ||
            k_cache->is_value != 0 || v_cache->is_value != 1 || k_cache->head_dim != head_dim ||
            v_cache->head_dim != head_dim || k_cache->kv_heads != kv_heads ||
            v_cache->kv_heads != kv_heads)
            return fail(CQKV_ERR_ARG, "cqkv_flash_attn: the fused append takes FP8 key / value sides of the same shape");
        if (position < 0 || (int64_t)position + kv_len > k_cache->capacity ||
            (int64_t)position + kv_len > v_cache->capacity)
            return fail(CQKV_ERR_ARG, "cqkv_flash_attn: append [%d, %d) exceeds the cache capacity",
                        position, position + kv_len);
    }
    PrefillArgs a = {};
    a.q = (const uint16_t *)q;
    a.k = (const uint16_t *)k;
    a.v = (const uint16_t *)v;
    a.out = (uint16_t *)out;
    a.q_sb = q_strides[0];
    a.q_st = q_strides[1];
    a.q_sh = q_strides[2];
    a.k_sb = k_strides[0];
    a.k_st = k_strides[1];
    a.k_sh = k_strides[2];
    a.v_sb = v_strides[0];
    a.v_st = v_strides[1];
    a.v_sh = v_strides[2];
    a.o_sb = out_strides[0];
    a.o_st = out_strides[1];
    a.o_sh = out_strides[2];
    a.q_len = q_len;
    a.kv_len = kv_len;
    a.q_heads = q_heads;
    a.kv_heads = kv_heads;
    a.group = q_heads / kv_heads;
    a.heads_per_wg = a.group < 4 ? a.group : 4;
    if (a.group % a.heads_per_wg != 0)
        return fail(CQKV_ERR_ARG, "cqkv_flash_attn: q_heads / kv_heads = %d not a multiple of 4 or below 4",
                    a.group);
    a.q_blocks = (q_len + kPfBQ - 1) / kPfBQ;
    a.wl = window_left;
    a.wr = window_right;
    a.scale_log2 = softmax_scale * kLog2e;
    const dim3 grid(a.q_blocks, kv_heads * (a.group / a.heads_per_wg), batch);
    const size_t lds = 4 * (size_t)kPfTile;
    static bool lds_set = false;
    if (!lds_set) {
        CQKV_HIP_CHECK(hipFuncSetAttribute((const void *)prefill_kernel,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
        lds_set = true;
    }
    hipLaunchKernelGGL(prefill_kernel, grid, dim3(256), lds, st, a);
    CQKV_HIP_CHECK(hipGetLastError());
    if (k_cache) {
        // K / V are (batch, kv_len, kv_heads, D): the append kernel's (batch, head, token)
        const int64_t ks[3] = {k_strides[0], k_strides[2], k_strides[1]};
        const int64_t vs[3] = {v_strides[0], v_strides[2], v_strides[1]};
        if (int rc = quant_append_launch(k_cache, k, CQKV_BF16, ks, batch, kv_len, nullptr, position, st))
            return rc;
        if (int rc = quant_append_launch(v_cache, v, CQKV_BF16, vs, batch, kv_len, nullptr, position, st))
            return rc;
    }
    return CQKV_OK;
}
