// Flash attention with f32 queries and f32 math (the reference's fa_row_f32_* / fa{2,3}_d*_f32_*
// kernels, candle-core/kernels/flash_attn_impl.h:49-443, dtype pairs of kv_dtype_supported,
// candle-core/src/accel/attention.rs:569-576): K / V in f32, f16, bf16 or E4M3 (per-tensor
// descale), every element widened exactly to f32, both products on v_mfma_f32_16x16x4f32, the
// online softmax in f32, f32 output.
//
// A wavefront owns 16 columns (a column is a (query, q head) pair of one kv head) and walks the
// keys in 16-key tiles. K and V go straight from memory into MFMA operand registers, with no LDS
// staging: the k-slot order of each product is chosen so that every lane reads 4 consecutive
// elements of one row.
//  * S^T = K Q^T, step (i, e) of D / 4: lane (m, g) = (lane % 16, lane / 16) gives
//    K[key m][16 i + 4 g + e] and Q[col m][16 i + 4 g + e]; lane (n, g) then holds the scores
//    of keys 4 g .. 4 g + 3 for column n.
//  * O^T += V^T P^T, step (j, blk, e): k-slot g is key 4 g + j, which is exactly the P this lane
//    holds for key 4 g + j; lane (m, g) gives V[key 4 g + j][64 blk + 4 m + e], so output row m
//    of step (blk, e) is head dim 64 blk + 4 m + e, and lane (n, g) ends with the four
//    consecutive head dims 64 blk + 16 g + 4 r .. + 3 of column n in acc[blk][0..3][r].
// Row mode (at most 16 columns per kv head: decode): the four wavefronts take alternating tiles
// of the workgroup's key split and merge (m, l, O) in LDS. Column mode (more columns): wavefront
// w takes columns 64 cb + 16 w .. + 15 over the whole split, with no merge; the four read the
// same tiles close together in time, so the re-reads hit the CU's cache.
#pragma once

#include "flash_plain.h"

namespace cqkv {

// K / V element types of the f32 kernel
enum { kFa32F32 = 0, kFa32F16 = 1, kFa32BF16 = 2, kFa32E4M3 = 3 };

template <int KV>
constexpr int fa32_esz() {
    return KV == kFa32F32 ? 4 : KV == kFa32E4M3 ? 1 : 2;
}

// Raw words of 4 consecutive elements of one row.
template <int KV>
struct Fa32Raw {
    using t = typename std::conditional<
        KV == kFa32F32, u32x4, typename std::conditional<KV == kFa32E4M3, uint32_t, u32x2>::type>::type;
};

template <int KV>
__device__ inline typename Fa32Raw<KV>::t fa32_load(rsrc_t r, uint32_t off) {
    if constexpr (KV == kFa32F32) return ld128(r, off);
    else if constexpr (KV == kFa32E4M3) return ld32(r, off);
    else return ld64(r, off);
}

// The 4 elements as f32, exactly.
template <int KV>
__device__ inline f32x4 fa32_widen(typename Fa32Raw<KV>::t w) {
    if constexpr (KV == kFa32F32) {
        return __builtin_bit_cast(f32x4, w);
    } else if constexpr (KV == kFa32F16) {
        return f32x4{f16_bits_to_f32(w.x & 0xffffu), f16_bits_to_f32(w.x >> 16),
                     f16_bits_to_f32(w.y & 0xffffu), f16_bits_to_f32(w.y >> 16)};
    } else if constexpr (KV == kFa32BF16) {
        return f32x4{__uint_as_float(w.x << 16), __uint_as_float(w.x & 0xffff0000u),
                     __uint_as_float(w.y << 16), __uint_as_float(w.y & 0xffff0000u)};
    } else {
        const f32x2 lo = __builtin_amdgcn_cvt_pk_f32_fp8(w, false);
        const f32x2 hi = __builtin_amdgcn_cvt_pk_f32_fp8(w, true);
        return f32x4{lo.x, lo.y, hi.x, hi.y};
    }
}

__device__ inline f32x4 mfma16x16x4f32(float a, float b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// One 16-key tile's operand registers: K (D / 16 loads) and V (4 keys x D / 64 loads).
template <int KV, int D>
struct Fa32Tile {
    typename Fa32Raw<KV>::t k[D / 16];
    typename Fa32Raw<KV>::t v[4][D / 64];
};

// Issues the loads of 16-key tile t (rows 16 t .. of the plane); rows past `rows` and head dims
// past head_dim read zeros (the resource ends at the last valid element; koff / voff point past
// it for head dims beyond head_dim). A tile past the end (valid false) reads zeros only.
template <int KV, int D>
__device__ inline void fa32_issue(Fa32Tile<KV, D> &tl, const uint8_t *kplane, const uint8_t *vplane,
                                  int64_t k_rb, int64_t v_rb, int rows, int head_dim, int t,
                                  bool valid, const uint32_t *koff, const uint32_t *voff) {
    constexpr int ESZ = fa32_esz<KV>();
    const int row0 = valid ? 16 * t : 0;
    const int nvalid = valid ? min(16, rows - row0) : 0;
    const uint32_t kb =
        nvalid > 0 ? (uint32_t)((int64_t)(nvalid - 1) * k_rb + ESZ * head_dim) : 0u;
    const uint32_t vb =
        nvalid > 0 ? (uint32_t)((int64_t)(nvalid - 1) * v_rb + ESZ * head_dim) : 0u;
    const rsrc_t rk = make_rsrc(kplane + (int64_t)row0 * k_rb, __builtin_amdgcn_readfirstlane(kb));
    const rsrc_t rv = make_rsrc(vplane + (int64_t)row0 * v_rb, __builtin_amdgcn_readfirstlane(vb));
#pragma unroll
    for (int i = 0; i < D / 16; ++i) tl.k[i] = fa32_load<KV>(rk, koff[i]);
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int blk = 0; blk < D / 64; ++blk) tl.v[j][blk] = fa32_load<KV>(rv, voff[j * (D / 64) + blk]);
}

// Scores, online softmax and O^T += V^T P^T for one 16-key tile of a wavefront.
template <int KV, int D>
__device__ inline void fa32_tile(const Fa32Tile<KV, D> &tl, const f32x4 *qop, int t, int g,
                                 int lo, int hi, int lo_max, int hi_min, int L, int koff,
                                 float scale_log2, float cap2, float slope2, int pos,
                                 float &m_run, float &l_run, f32x4 (*acc)[4]) {
    constexpr int NB = D / 64;
    f32x4 s[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) s[e] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < D / 16; ++i) {
        const f32x4 kv = fa32_widen<KV>(tl.k[i]);
#pragma unroll
        for (int e = 0; e < 4; ++e) s[e] = mfma16x16x4f32(kv[e], qop[i][e], s[e]);
    }
    // x[r]: key 16 t + 4 g + r of the tile, this lane's column
    float x[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) x[r] = ((s[0][r] + s[1][r]) + (s[2][r] + s[3][r])) * scale_log2;
    const int t0 = 16 * t;
    if (cap2 > 0.0f || slope2 != 0.0f) {
#pragma unroll
        for (int r = 0; r < 4; ++r) x[r] = fa_logit2(x[r], cap2, slope2, pos - (koff + t0 + 4 * g + r));
    }
    const bool full = koff + t0 >= lo_max && koff + t0 + 16 <= hi_min && t0 + 16 <= L;
    if (!full) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row = t0 + 4 * g + r, key = koff + row;
            if (!(key >= lo && key < hi && row < L)) x[r] = -__builtin_inff();
        }
    }
    float mx = fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3]));
    mx = group16_max(mx);
    const float m_new = fmaxf(m_run, mx);
    const bool none = m_new == -__builtin_inff();
    const float alpha = none ? 1.0f : __builtin_amdgcn_exp2f(m_run - m_new);
    float p[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) p[r] = none ? 0.0f : __builtin_amdgcn_exp2f(x[r] - m_new);
    m_run = m_new;
    l_run = l_run * alpha + ((p[0] + p[1]) + (p[2] + p[3]));
    if (__any(alpha != 1.0f)) {
#pragma unroll
        for (int blk = 0; blk < NB; ++blk)
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[blk][e] *= alpha;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int blk = 0; blk < NB; ++blk) {
            const f32x4 vv = fa32_widen<KV>(tl.v[j][blk]);
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[blk][e] = mfma16x16x4f32(vv[e], p[j], acc[blk][e]);
        }
}

template <int KV, int D, bool COLS>
__global__ __launch_bounds__(256) void fa32_kernel(FaArgs a) {
    constexpr int W = 4, NB = D / 64, ESZ = fa32_esz<KV>();
    __shared__ float sm_o[COLS ? 1 : W][COLS ? 1 : 16][COLS ? 1 : D];
    __shared__ float sm_m[W][16], sm_l[W][16];

    const int planes = a.batch * a.kv_heads;
    const int rest = (int)blockIdx.x / planes, plane_id = (int)blockIdx.x % planes;
    const int split = rest / a.col_blocks, cb = rest % a.col_blocks;
    const int b = plane_id / a.kv_heads, hk = plane_id % a.kv_heads;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n = lane & 15, g = lane >> 4;
    const FaSeq sq = fa_sequence(a, b);
    const int ncols = sq.lq * a.group;
    // this wavefront's 16 columns
    const int c0 = COLS ? 64 * cb + 16 * wave : 16 * cb;
    if (COLS ? 64 * cb >= ncols : c0 >= ncols) return;  // the whole workgroup
    const int ncb = max(0, min(16, ncols - c0));
    if (COLS && ncb == 0) return;  // this wavefront only: column mode has no barrier
    const bool col_ok = n < ncb;
    const int col = c0 + (col_ok ? n : 0);
    const int qi = col / a.group, head = hk * a.group + col % a.group;
    int lo, hi, lo_min, hi_min, lo_max, hi_max;
    fa_key_range(qi, sq.lq, sq.lk, a.wl, a.wr, lo, hi);
    if (!col_ok) lo = hi = 0;
    fa_key_range(c0 / a.group, sq.lq, sq.lk, a.wl, a.wr, lo_min, hi_min);
    fa_key_range((c0 + max(ncb, 1) - 1) / a.group, sq.lq, sq.lk, a.wl, a.wr, lo_max, hi_max);

    // the split's keys (whole 32-key tiles of the planner) as 16-key tiles
    const uint8_t *kplane, *vplane;
    int koff = 0, Lb, tb, te;
    if (a.segs) {
        const FaSeg sg = a.segs[split];
        kplane = (const uint8_t *)sg.k + ((int64_t)b * sg.k_sb + (int64_t)hk * sg.k_sh) * ESZ;
        vplane = (const uint8_t *)sg.v + ((int64_t)b * sg.v_sb + (int64_t)hk * sg.v_sh) * ESZ;
        koff = sg.key_offset;
        Lb = sg.rows;
        tb = max(2 * sg.tile_begin, max(lo_min - koff, 0) / 16);
        te = min(2 * sg.tile_end, (max(hi_max - koff, 0) + 15) / 16);
    } else {
        kplane = (const uint8_t *)a.k + (sq.k0 + (int64_t)hk * a.k_sh) * ESZ;
        vplane = (const uint8_t *)a.v + (sq.v0 + (int64_t)hk * a.v_sh) * ESZ;
        Lb = sq.lk;
        tb = max(2 * split * a.tiles_per_split, lo_min / 16);
        te = min(2 * (split + 1) * a.tiles_per_split, (hi_max + 15) / 16);
    }

    // Q operands: qop[i][e] = q[col][16 i + 4 g + e], exact (scores are scaled in f32)
    float scale_log2 = a.scale_log2;
    if (a.q_mul_dev) scale_log2 *= *a.q_mul_dev;
    f32x4 qop[D / 16];
    {
        const float *qrow = (const float *)a.q + sq.q0 + (int64_t)qi * a.q_st + (int64_t)head * a.q_sh;
#pragma unroll
        for (int i = 0; i < D / 16; ++i) {
            const int d0 = 16 * i + 4 * g;
            f32x4 w = {0.f, 0.f, 0.f, 0.f};
            if (col_ok && d0 < a.head_dim) {
                if (a.q_vec) w = *(const f32x4 *)(qrow + d0);
                else w = f32x4{qrow[d0], qrow[d0 + 1], qrow[d0 + 2], qrow[d0 + 3]};
            }
            qop[i] = w;
        }
    }
    const float slope2 = a.alibi ? a.alibi[b * a.alibi_bs + head] * kLog2e : 0.0f;
    const int pos = qi + sq.lk - sq.lq;

    // per-lane byte offsets from a tile's row 0
    const int64_t k_rb = a.k_st * ESZ, v_rb = a.v_st * ESZ;
    uint32_t koffs[D / 16], voffs[4 * NB];
#pragma unroll
    for (int i = 0; i < D / 16; ++i) {
        const int d0 = 16 * i + 4 * g;
        koffs[i] = d0 < a.head_dim ? (uint32_t)(n * k_rb + ESZ * d0) : kFaOOB;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int blk = 0; blk < NB; ++blk) {
            const int d0 = 64 * blk + 4 * n;
            voffs[j * NB + blk] = d0 < a.head_dim ? (uint32_t)((4 * g + j) * v_rb + ESZ * d0) : kFaOOB;
        }

    f32x4 acc[NB][4];
#pragma unroll
    for (int blk = 0; blk < NB; ++blk)
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[blk][e] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m_run = -__builtin_inff(), l_run = 0.0f;

    const int step = COLS ? 1 : W;
    int t = tb + (COLS ? 0 : wave);
    Fa32Tile<KV, D> ta, tb2;
    fa32_issue<KV, D>(ta, kplane, vplane, k_rb, v_rb, Lb, a.head_dim, t, t < te, koffs, voffs);
    fa32_issue<KV, D>(tb2, kplane, vplane, k_rb, v_rb, Lb, a.head_dim, t + step, t + step < te,
                      koffs, voffs);
    for (; t < te; t += 2 * step) {
        fa32_tile<KV, D>(ta, qop, t, g, lo, hi, lo_max, hi_min, Lb, koff, scale_log2, a.softcap2,
                         slope2, pos, m_run, l_run, acc);
        fa32_issue<KV, D>(ta, kplane, vplane, k_rb, v_rb, Lb, a.head_dim, t + 2 * step,
                          t + 2 * step < te, koffs, voffs);
        if (t + step >= te) break;
        fa32_tile<KV, D>(tb2, qop, t + step, g, lo, hi, lo_max, hi_min, Lb, koff, scale_log2,
                         a.softcap2, slope2, pos, m_run, l_run, acc);
        fa32_issue<KV, D>(tb2, kplane, vplane, k_rb, v_rb, Lb, a.head_dim, t + 3 * step,
                          t + 3 * step < te, koffs, voffs);
    }

    const int rows = a.batch * a.q_heads * a.q_len;
    const bool single = a.splits == 1;
    float o_mul = a.o_mul;
    if (a.o_mul_dev) o_mul *= *a.o_mul_dev;
    const float l_col = group16_sum(l_run);
    if constexpr (COLS) {
        // each lane: head dims 64 blk + 16 g + 4 r .. + 3 of its column
        if (!col_ok) return;
        const bool any = m_run != -__builtin_inff();
        const float inv = any ? 1.0f / l_col : 0.0f;
        const float lse = any ? m_run + __builtin_log2f(l_col) : -__builtin_inff();
        const int64_t row = ((int64_t)b * a.q_heads + head) * a.q_len + qi;
        float *dst;
        if (single) dst = (float *)a.out + sq.o0 + (int64_t)qi * a.o_st + (int64_t)head * a.o_sh;
        else dst = a.part_o + ((int64_t)split * rows + row) * D;
        const bool vec = !single || a.o_vec;
#pragma unroll
        for (int blk = 0; blk < NB; ++blk)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int d0 = 64 * blk + 16 * g + 4 * r;
                if (d0 >= a.head_dim) continue;
                const float mul = single ? inv * o_mul : inv;
                const f32x4 o = {acc[blk][0][r] * mul, acc[blk][1][r] * mul, acc[blk][2][r] * mul,
                                 acc[blk][3][r] * mul};
                if (vec) {
                    *(f32x4 *)(dst + d0) = o;
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e) dst[d0 + e] = o[e];
                }
            }
        if (!single && g == 0) a.part_lse[(int64_t)split * rows + row] = lse;
    } else {
        // ---- merge the wavefronts ----
#pragma unroll
        for (int blk = 0; blk < NB; ++blk)
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int e = 0; e < 4; ++e) sm_o[wave][n][64 * blk + 16 * g + 4 * r + e] = acc[blk][e][r];
        if (g == 0) {
            sm_m[wave][n] = m_run;
            sm_l[wave][n] = l_col;
        }
        __syncthreads();
        for (int idx = threadIdx.x; idx < ncb * D; idx += W * 64) {
            const int c = idx / D, d = idx % D;
            if (d >= a.head_dim) continue;
            float M = -__builtin_inff();
#pragma unroll
            for (int w = 0; w < W; ++w) M = fmaxf(M, sm_m[w][c]);
            float o = 0.0f, lse = -__builtin_inff();
            if (M != -__builtin_inff()) {
                float wsum = 0.0f, osum = 0.0f;
#pragma unroll
                for (int w = 0; w < W; ++w) {
                    const float f = __builtin_amdgcn_exp2f(sm_m[w][c] - M);
                    wsum += sm_l[w][c] * f;
                    osum += sm_o[w][c][d] * f;
                }
                o = osum / wsum;
                lse = M + __builtin_log2f(wsum);
            }
            const int cc = c0 + c;
            const int qc = cc / a.group, hc = hk * a.group + cc % a.group;
            if (!single) {
                const int64_t row = ((int64_t)b * a.q_heads + hc) * a.q_len + qc;
                a.part_o[((int64_t)split * rows + row) * D + d] = o;
                if (d == 0) a.part_lse[(int64_t)split * rows + row] = lse;
            } else {
                ((float *)a.out)[sq.o0 + (int64_t)qc * a.o_st + (int64_t)hc * a.o_sh + d] = o * o_mul;
            }
        }
    }
}

}  // namespace cqkv
