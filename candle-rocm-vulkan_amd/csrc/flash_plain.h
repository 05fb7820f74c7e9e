// Flash attention over plain bf16 / f16 K / V (the reference's row kernels fa_row_* / fa_rowg_*
// and their paged form fa_rowp_*, candle-core/kernels/flash_attn_impl.h:49-328, and the tile
// kernels for every head dim <= 256, :330-443), on MFMA for gfx950.
//
// One workgroup = W wavefronts on the same 16 columns (a column is a (query, q head) pair of one
// kv head: the query heads of a GQA group share every K / V read) and one split of the keys;
// the wavefronts take alternating 32-key tiles and merge at the end; splits merge in
// fa_combine_kernel. Per wavefront, per tile:
//  * K and V tiles (32 rows x D) arrive by asynchronous buffer_load ... lds copies into a private
//    two-stage LDS ring, one tile ahead; rows past the valid keys and head dims past head_dim
//    read zeros. 16-byte chunks are XOR-swizzled by row.
//  * S^T = K Q^T on v_mfma_f32_16x16x32 (bf16 or f16): K from LDS (ds_read_b128), Q^T in
//    registers. The online softmax runs in the exp2 domain on the S^T accumulators.
//  * O^T += V^T P^T: the V^T operands come from the row-major V tile through ds_read_b64_tr_b16
//    (lane i of a 16-lane group receives four keys of head dim d0 + i), P^T as a hi + lo pair.
#pragma once

#include <type_traits>

#include "cqkv_device.h"
#include "cqkv_host.h"

namespace cqkv {

// A run of key rows: one block of a paged call, or (dense calls) unused.
struct FaSeg {
    const uint16_t *k, *v;          // element (batch 0, kv head 0, row 0) of the block
    int64_t k_sb, k_sh, v_sb, v_sh;  // element strides of batch and kv head (rows: FaArgs k_st)
    int32_t rows;                    // valid rows of the block
    int32_t key_offset;              // keys of the call before the block's row 0
    int32_t tile_begin, tile_end;    // this split's 32-row tiles of the block
};

struct FaArgs {
    const uint16_t *q;
    int64_t q_sb, q_st, q_sh;  // element strides: batch, query, head
    void *out;
    int64_t o_sb, o_st, o_sh;
    const uint16_t *k, *v;  // dense calls
    int64_t k_sb, k_st, k_sh, v_sb, v_st, v_sh;
    const int32_t *cu_q, *cu_k;  // variable-length batches (null: dense)
    int32_t total_q, total_k;
    const FaSeg *segs;  // paged calls: one segment per split (null: dense)
    float *part_o, *part_lse;
    int32_t batch, q_len, kv_len, q_heads, kv_heads, group, head_dim, dtype;
    int32_t kv_dtype;  // K / V element type: dtype, or with f32 queries f16 / bf16 / E4M3 (3)
    int32_t splits, tiles_per_split, col_blocks;
    int32_t wl, wr;
    int32_t q_vec;  // q rows 16-byte aligned with strides of whole 16-byte chunks
    int32_t o_vec;  // f32 out rows likewise (f32 kernel, column mode)
    float scale_log2;  // softmax scale * log2(e) (times the host query factor)
    float softcap2;    // softcap * log2(e), 0: off
    const float *alibi;
    int32_t alibi_bs;
    float o_mul;                         // output factor (FP8 V descale), 1 otherwise
    const float *q_mul_dev, *o_mul_dev;  // device factors of the same (null: 1)
};

// (first q / out / k / v element, lengths) of sequence b, as the MFMA prefill clamps them
struct FaSeq {
    int64_t q0, o0, k0, v0;
    int lq, lk;
};
__device__ inline FaSeq fa_sequence(const FaArgs &a, int b) {
    FaSeq r;
    if (a.cu_q) {
        const int qa = min(max(a.cu_q[b], 0), a.total_q), qe = min(max(a.cu_q[b + 1], qa), a.total_q);
        const int ka = min(max(a.cu_k[b], 0), a.total_k), ke = min(max(a.cu_k[b + 1], ka), a.total_k);
        r.lq = min(qe - qa, a.q_len);
        r.lk = min(ke - ka, a.kv_len);
        r.q0 = (int64_t)qa * a.q_st;
        r.o0 = (int64_t)qa * a.o_st;
        r.k0 = (int64_t)ka * a.k_st;
        r.v0 = (int64_t)ka * a.v_st;
    } else {
        r.lq = a.q_len;
        r.lk = a.kv_len;
        r.q0 = (int64_t)b * a.q_sb;
        r.o0 = (int64_t)b * a.o_sb;
        r.k0 = (int64_t)b * a.k_sb;
        r.v0 = (int64_t)b * a.v_sb;
    }
    return r;
}

__device__ inline void fa_key_range(int i, int lq, int lk, int wl, int wr, int &lo, int &hi) {
    const int pos = i + lk - lq;
    lo = wl >= 0 ? max(pos - wl, 0) : 0;
    hi = wr >= 0 ? min(pos + wr + 1, lk) : lk;
    lo = min(lo, lk);
    hi = max(hi, lo);
}

constexpr uint32_t kFaOOB = 0x80000000u;  // a copy offset past every resource range

typedef __attribute__((address_space(3))) void fa_lds_void;
typedef short fa_s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) fa_s16x4 fa_lds_s16x4;

// s_waitcnt vmcnt(n) (gfx9 encoding; expcnt and lgkmcnt left at their maxima)
#define FA_WAIT_VMCNT(n) __builtin_amdgcn_s_waitcnt((((n) & 15) | (((n) >> 4) << 14)) | 0x0f70)

template <int D>
struct FaTileGeom {
    static constexpr int RB = 2 * D;           // bytes per row
    static constexpr int TILE = 32 * RB;       // one K or V tile
    static constexpr int NCP = TILE / 1024;    // copies (1 KB each) per tile and side
    static constexpr int ROWS_PER_CP = 1024 / RB;
};

// Byte offset in LDS of 16-byte chunk c of tile row r (chunks XOR-swizzled by the row: by its
// low 3 bits for the 8-chunk rows of D = 64, 4 bits for longer rows, so that the 16 rows a
// 16-lane group reads hit 16 different 16-byte bank groups).
template <int D>
__device__ inline int fa_swz(int r) { return r & (D >= 128 ? 15 : 7); }
template <int D>
__device__ inline uint32_t fa_chunk_off(int r, int c) {
    return (uint32_t)(r * FaTileGeom<D>::RB + ((c ^ fa_swz<D>(r)) << 4));
}

// The source offsets (bytes from a tile's row 0) of this lane's part of each 1 KB copy: copy i
// fills LDS bytes [1024 i, 1024 i + 1024) of the tile, lane l the 16 bytes at 1024 i + 16 l,
// i.e. the swizzled chunk of a row; chunks past head_dim are pointed past the resource (zeros).
template <int D>
__device__ inline void fa_copy_offsets(uint32_t (&off)[FaTileGeom<D>::NCP], int64_t row_stride,
                                       int head_dim, int lane) {
    using G = FaTileGeom<D>;
#pragma unroll
    for (int i = 0; i < G::NCP; ++i) {
        const int o = 1024 * i + 16 * lane;
        const int r = o / G::RB, ph = (o % G::RB) >> 4;
        const int c = ph ^ fa_swz<D>(r);
        off[i] = 8 * c < head_dim ? (uint32_t)(r * row_stride * 2 + 16 * c) : kFaOOB;
    }
}

// Asynchronous copies of 32-row tile kt of a plane into the LDS tile at dst (wavefront-uniform);
// rows >= rows read zeros; a tile past the end (valid false) copies nothing (zero-size resource).
// The row kernel reads each K / V row once per call: the copies are nontemporal (config-2 shape
// bf16 186 -> 171 us, f16 193 -> 174 us same-box).
template <int D>
__device__ inline void fa_issue_tile(uint8_t *dst, const uint16_t *plane, int64_t row_stride,
                                     int rows, int head_dim, int kt, bool valid,
                                     const uint32_t *off) {
    using G = FaTileGeom<D>;
    const int row0 = valid ? kt * 32 : 0;
    const int nvalid = valid ? min(32, rows - row0) : 0;
    const uint64_t p = (uint64_t)(plane + (int64_t)row0 * row_stride);
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)p);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(p >> 32));
    const uint32_t bytes =
        nvalid > 0 ? (uint32_t)((int64_t)(nvalid - 1) * row_stride * 2 + 2 * head_dim) : 0u;
    const rsrc_t r = make_rsrc((const void *)(((uint64_t)hi << 32) | lo),
                               __builtin_amdgcn_readfirstlane(bytes));
#pragma unroll
    for (int i = 0; i < G::NCP; ++i)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (fa_lds_void *)(dst + 1024 * i), 16, off[i], 0,
                                                 0, 2);
}

template <bool F16>
using fa_op_t = typename std::conditional<F16, f16x8, bf16x8>::type;

// The score terms of fa_logit (candle-core/kernels/flash_attn_impl.h:42-47) in exp2 units:
// cap * tanh(s / cap) = cap - 2 cap / (e^(2 s / cap) + 1), then - slope * |pos - key|.
// Sum of the 8 elements of a bf16 / f16 operand (four dot2 with ones).
template <bool F16>
__device__ inline float fa_sum8(fa_op_t<F16> v) {
    const u32x4 w = __builtin_bit_cast(u32x4, v);
    float a = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t x = w[i];
        if constexpr (F16) {
            typedef _Float16 h2 __attribute__((ext_vector_type(2)));
            const h2 ones = {(_Float16)1.0f, (_Float16)1.0f};
            a = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, x), ones, a, false);
        } else {
            const bf16x2 ones = {(__bf16)1.0f, (__bf16)1.0f};
            a = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, x), ones, a, false);
        }
    }
    return a;
}

// One 32-key tile of a wavefront: S^T, online softmax, O^T += V^T P^T (PLO: P as a hi + lo
// pair and the scores scaled here; else, as the MFMA prefill does, one P operand of the dtype
// and queries pre-scaled by scale * log2(e) before they were rounded to the dtype).
template <bool F16, int D, bool PLO = true>
__device__ inline void fa_tile(const uint8_t *kst, const uint8_t *vst, const fa_op_t<F16> *qop,
                               int t, int lane, int lo, int hi, int lo_max, int hi_min, int L,
                               int koff, float scale_log2, float cap2, float slope2, int pos,
                               float &m_run, float &l_run, f32x4 *acc) {
    using op_t = fa_op_t<F16>;
    constexpr int NJ = D / 32, NU = D / 16;
    const int m = lane & 15, g = lane >> 4;
    f32x4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const op_t k0 = __builtin_bit_cast(op_t, *(const u32x4 *)(kst + fa_chunk_off<D>(m, 4 * j + g)));
        const op_t k1 =
            __builtin_bit_cast(op_t, *(const u32x4 *)(kst + fa_chunk_off<D>(16 + m, 4 * j + g)));
        s0 = mfma16x16x32(k0, qop[j], s0);
        s1 = mfma16x16x32(k1, qop[j], s1);
    }
    // x[e]: key 4 g + e (e < 4) or 16 + 4 g + e - 4 of the tile, for this lane's column
    float x[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
    const int t0 = t * 32;
    if constexpr (PLO) {
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] *= scale_log2;
    }
    if (cap2 > 0.0f || slope2 != 0.0f) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int key = koff + t0 + (e < 4 ? 4 * g + e : 16 + 4 * g + e - 4);
            x[e] = fa_logit2(x[e], cap2, slope2, pos - key);
        }
    }
    const bool full = koff + t0 >= lo_max && koff + t0 + 32 <= hi_min && t0 + 32 <= L;
    if (!full) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int r = t0 + (e < 4 ? 4 * g + e : 16 + 4 * g + e - 4);
            const int key = koff + r;
            if (!(key >= lo && key < hi && r < L)) x[e] = -__builtin_inff();
        }
    }
    float mx = x[0];
#pragma unroll
    for (int e = 1; e < 8; ++e) mx = fmaxf(mx, x[e]);
    mx = group16_max(mx);
    const float m_new = fmaxf(m_run, mx);
    const bool none = m_new == -__builtin_inff();
    const float alpha = none ? 1.0f : __builtin_amdgcn_exp2f(m_run - m_new);
    float p[8], psum = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        p[e] = none ? 0.0f : __builtin_amdgcn_exp2f(x[e] - m_new);
        if constexpr (PLO) psum += p[e];
    }
    m_run = m_new;
    if (__any(alpha != 1.0f)) {
#pragma unroll
        for (int u = 0; u < NU; ++u) acc[u] *= alpha;
    }
    op_t phi, plo;
    split8(p, phi, plo);
    // the row sum of the P the product uses (hi + lo: p itself)
    l_run = l_run * alpha + (PLO ? psum : fa_sum8<F16>(phi));
    // V^T operands: lane (16-lane group g, index 4 pp + qq) points at key row 4 g + pp (then
    // 16 + 4 g + pp), head dims 16 u + 4 qq .. +3; lane i of the group receives those four keys
    // of head dim 16 u + i: k-slots 8 g .. 8 g + 3 and 8 g + 4 .. 8 g + 7, the keys of p[].
    const int pp = m >> 2, qq = m & 3;
    const int r0 = 4 * g + pp, r1 = 16 + 4 * g + pp;
#pragma unroll
    for (int u = 0; u < NU; ++u) {
        const int c = 2 * u + (qq >> 1), sub = (qq & 1) * 8;
        const fa_s16x4 a0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (fa_lds_s16x4 *)(vst + fa_chunk_off<D>(r0, c) + sub));
        const fa_s16x4 a1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (fa_lds_s16x4 *)(vst + fa_chunk_off<D>(r1, c) + sub));
        const u32x2 w0 = __builtin_bit_cast(u32x2, a0), w1 = __builtin_bit_cast(u32x2, a1);
        const op_t va = __builtin_bit_cast(op_t, u32x4{w0.x, w0.y, w1.x, w1.y});
        acc[u] = mfma16x16x32(va, phi, acc[u]);
        if constexpr (PLO) acc[u] = mfma16x16x32(va, plo, acc[u]);
    }
}

template <int D>
constexpr int fa_waves() {
    return D == 256 ? 2 : 4;
}

template <bool F16, int D, int W>
__global__ __launch_bounds__(W * 64) void fa_row_kernel(FaArgs a) {
    using op_t = fa_op_t<F16>;
    using G = FaTileGeom<D>;
    constexpr int NJ = D / 32, NU = D / 16;
    // stage s of wavefront w: K tile at ring_s + 2 w TILE, V tile right after it
    __shared__ __attribute__((aligned(1024))) uint8_t ring0[W * 2 * G::TILE];
    __shared__ __attribute__((aligned(1024))) uint8_t ring1[W * 2 * G::TILE];
    __shared__ float sm_m[W][16], sm_l[W][16];
    static_assert(W * 16 * D * 4 <= W * 2 * G::TILE, "merge buffer inside stage 0");

    const int planes = a.batch * a.kv_heads;
    const int rest = (int)blockIdx.x / planes, plane_id = (int)blockIdx.x % planes;
    const int split = rest / a.col_blocks, cb = rest % a.col_blocks;
    const int b = plane_id / a.kv_heads, hk = plane_id % a.kv_heads;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n = lane & 15, g = lane >> 4;
    const FaSeq sq = fa_sequence(a, b);
    const int ncols = sq.lq * a.group, c0 = 16 * cb;
    if (c0 >= ncols) return;  // the whole workgroup: no columns of this sequence here
    const int ncb = min(16, ncols - c0);
    const bool col_ok = n < ncb;
    const int col = c0 + (col_ok ? n : 0);
    const int qi = col / a.group, head = hk * a.group + col % a.group;
    int lo, hi, lo_min, hi_min, lo_max, hi_max;
    fa_key_range(qi, sq.lq, sq.lk, a.wl, a.wr, lo, hi);
    if (!col_ok) lo = hi = 0;
    fa_key_range(c0 / a.group, sq.lq, sq.lk, a.wl, a.wr, lo_min, hi_min);
    fa_key_range((c0 + ncb - 1) / a.group, sq.lq, sq.lk, a.wl, a.wr, lo_max, hi_max);

    // the split's tiles and the planes they live in
    const uint16_t *kplane, *vplane;
    int koff = 0, Lb, tb, te;
    if (a.segs) {
        const FaSeg sg = a.segs[split];
        kplane = sg.k + (int64_t)b * sg.k_sb + (int64_t)hk * sg.k_sh;
        vplane = sg.v + (int64_t)b * sg.v_sb + (int64_t)hk * sg.v_sh;
        koff = sg.key_offset;
        Lb = sg.rows;
        tb = max(sg.tile_begin, max(lo_min - koff, 0) / 32);
        te = min(sg.tile_end, (max(hi_max - koff, 0) + 31) / 32);
    } else {
        kplane = a.k + sq.k0 + (int64_t)hk * a.k_sh;
        vplane = a.v + sq.v0 + (int64_t)hk * a.v_sh;
        Lb = sq.lk;
        tb = max(split * a.tiles_per_split, lo_min / 32);
        te = min((split + 1) * a.tiles_per_split, (hi_max + 31) / 32);
    }

    // Q^T operands: chunk j holds head dims 32 j + 8 g .. + 7 of this lane's column (exact; the
    // scores are scaled in f32)
    float scale_log2 = a.scale_log2;
    if (a.q_mul_dev) scale_log2 *= *a.q_mul_dev;
    op_t qop[NJ];
    {
        const uint16_t *qrow = a.q + sq.q0 + (int64_t)qi * a.q_st + (int64_t)head * a.q_sh;
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const int d0 = 32 * j + 8 * g;
            u32x4 w = {0u, 0u, 0u, 0u};
            if (col_ok && d0 < a.head_dim) {
                if (a.q_vec) {
                    w = *(const u32x4 *)(qrow + d0);
                } else {
                    uint32_t *wp = (uint32_t *)&w;
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        wp[e] = (uint32_t)qrow[d0 + 2 * e] | ((uint32_t)qrow[d0 + 2 * e + 1] << 16);
                }
            }
            qop[j] = __builtin_bit_cast(op_t, w);
        }
    }
    const float slope2 = a.alibi ? a.alibi[b * a.alibi_bs + head] * kLog2e : 0.0f;
    const int pos = qi + sq.lk - sq.lq;  // the column's query position in key coordinates

    uint32_t koffs[G::NCP], voffs[G::NCP];
    fa_copy_offsets<D>(koffs, a.k_st, a.head_dim, lane);
    fa_copy_offsets<D>(voffs, a.v_st, a.head_dim, lane);
    uint8_t *k0s = ring0 + 2 * wave * G::TILE, *v0s = k0s + G::TILE;
    uint8_t *k1s = ring1 + 2 * wave * G::TILE, *v1s = k1s + G::TILE;

    f32x4 acc[NU];
#pragma unroll
    for (int u = 0; u < NU; ++u) acc[u] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m_run = -__builtin_inff(), l_run = 0.0f;

    int t = tb + wave;
    fa_issue_tile<D>(k0s, kplane, a.k_st, Lb, a.head_dim, t, t < te, koffs);
    fa_issue_tile<D>(v0s, vplane, a.v_st, Lb, a.head_dim, t, t < te, voffs);
    fa_issue_tile<D>(k1s, kplane, a.k_st, Lb, a.head_dim, t + W, t + W < te, koffs);
    fa_issue_tile<D>(v1s, vplane, a.v_st, Lb, a.head_dim, t + W, t + W < te, voffs);
    for (; t < te; t += 2 * W) {
        FA_WAIT_VMCNT(2 * G::NCP);  // stage 0 (tile t) has landed; stage 1's copies may not
        fa_tile<F16, D>(k0s, v0s, qop, t, lane, lo, hi, lo_max, hi_min, Lb, koff, scale_log2,
                        a.softcap2, slope2, pos, m_run, l_run, acc);
        __builtin_amdgcn_sched_barrier(0);
        fa_issue_tile<D>(k0s, kplane, a.k_st, Lb, a.head_dim, t + 2 * W, t + 2 * W < te, koffs);
        fa_issue_tile<D>(v0s, vplane, a.v_st, Lb, a.head_dim, t + 2 * W, t + 2 * W < te, voffs);
        if (t + W >= te) break;
        FA_WAIT_VMCNT(2 * G::NCP);
        fa_tile<F16, D>(k1s, v1s, qop, t + W, lane, lo, hi, lo_max, hi_min, Lb, koff, scale_log2,
                        a.softcap2, slope2, pos, m_run, l_run, acc);
        __builtin_amdgcn_sched_barrier(0);
        fa_issue_tile<D>(k1s, kplane, a.k_st, Lb, a.head_dim, t + 3 * W, t + 3 * W < te, koffs);
        fa_issue_tile<D>(v1s, vplane, a.v_st, Lb, a.head_dim, t + 3 * W, t + 3 * W < te, voffs);
    }
    FA_WAIT_VMCNT(0);  // every copy of this wavefront has landed before stage 0 is reused

    // ---- merge the wavefronts (stage 0 holds the per-wavefront outputs) ----
    __syncthreads();
    float(*sm_o)[16][D] = (float(*)[16][D])ring0;
    const float l_col = group16_sum(l_run);
#pragma unroll
    for (int u = 0; u < NU; ++u)
#pragma unroll
        for (int i = 0; i < 4; ++i) sm_o[wave][n][16 * u + 4 * g + i] = acc[u][i];
    if (g == 0) {
        sm_m[wave][n] = m_run;
        sm_l[wave][n] = l_col;
    }
    __syncthreads();
    const int rows = a.batch * a.q_heads * a.q_len;
    const bool single = a.splits == 1;
    float o_mul = a.o_mul;
    if (a.o_mul_dev) o_mul *= *a.o_mul_dev;
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
            store_elem(a.out, sq.o0 + (int64_t)qc * a.o_st + (int64_t)hc * a.o_sh + d, a.dtype,
                       o * o_mul);
        }
    }
}

// This wavefront's share of the copies of tile t (K and V) into a stage of the shared ring:
// the 1 KB pieces wave, wave + 4, ... of each side; a tile past te copies nothing.
template <int D, int NCPW>
__device__ inline void fa_issue_shared(uint8_t *stage, int t, int te, const uint16_t *kplane,
                                       const uint16_t *vplane, int64_t k_st, int64_t v_st, int L,
                                       int head_dim, int wave, const uint32_t *koffs,
                                       const uint32_t *voffs) {
    using G = FaTileGeom<D>;
    const bool valid = t < te;
    const int row0 = valid ? t * 32 : 0;
    const int nvalid = valid ? min(32, L - row0) : 0;
#pragma unroll
    for (int side = 0; side < 2; ++side) {
        const uint16_t *plane = side ? vplane : kplane;
        const int64_t rs = side ? v_st : k_st;
        const uint64_t p = (uint64_t)(plane + (int64_t)row0 * rs);
        const uint32_t plo = __builtin_amdgcn_readfirstlane((uint32_t)p);
        const uint32_t phi = __builtin_amdgcn_readfirstlane((uint32_t)(p >> 32));
        const uint32_t bytes =
            nvalid > 0 ? (uint32_t)((int64_t)(nvalid - 1) * rs * 2 + 2 * head_dim) : 0u;
        const rsrc_t r = make_rsrc((const void *)(((uint64_t)phi << 32) | plo),
                                   __builtin_amdgcn_readfirstlane(bytes));
#pragma unroll
        for (int j = 0; j < NCPW; ++j)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                r, (fa_lds_void *)(stage + side * G::TILE + 1024 * (wave + 4 * j)), 16,
                side ? voffs[j] : koffs[j], 0, 0, 0);
    }
}

// Prefill-shaped calls: one workgroup = 4 wavefronts on 4 consecutive 16-column blocks (64
// columns of a kv head) over one split of the keys. The wavefronts share every K / V tile: each
// issues a quarter of a tile's copies into a three-stage LDS ring (two at D = 256, so that two
// workgroups share a CU), one barrier per tile, and computes its own columns; no merge across
// wavefronts.
template <bool F16, int D>
__global__ __launch_bounds__(256) void fa_tile_kernel(FaArgs a) {
    using op_t = fa_op_t<F16>;
    using G = FaTileGeom<D>;
    constexpr int NJ = D / 32, NU = D / 16, W = 4, NCPW = G::NCP / W;
    constexpr int NST = D == 256 ? 2 : 3;  // ring stages (96 KB of three at D = 256: one workgroup per CU)
    static_assert(G::NCP % W == 0, "copies per wavefront");
    __shared__ __attribute__((aligned(1024))) uint8_t st0[2 * G::TILE];
    __shared__ __attribute__((aligned(1024))) uint8_t st1[2 * G::TILE];
    __shared__ __attribute__((aligned(1024))) uint8_t st2[NST == 3 ? 2 * G::TILE : 1024];

    const int planes = a.batch * a.kv_heads;
    const int rest = (int)blockIdx.x / planes, plane_id = (int)blockIdx.x % planes;
    const int split = rest / a.col_blocks, cgrp = rest % a.col_blocks;
    const int b = plane_id / a.kv_heads, hk = plane_id % a.kv_heads;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n = lane & 15, g = lane >> 4;
    const FaSeq sq = fa_sequence(a, b);
    const int ncols = sq.lq * a.group, g0 = 64 * cgrp;
    if (g0 >= ncols) return;  // the whole workgroup
    const int c0 = g0 + 16 * wave;
    const bool wave_live = c0 < ncols;
    const int ncb = wave_live ? min(16, ncols - c0) : 0;
    const bool col_ok = n < ncb;
    const int col = col_ok ? c0 + n : g0;
    const int qi = col / a.group, head = hk * a.group + col % a.group;
    int lo, hi, lo_min, hi_min, lo_max, hi_max, wlo, whi;
    fa_key_range(qi, sq.lq, sq.lk, a.wl, a.wr, lo, hi);
    if (!col_ok) lo = hi = 0;
    // the workgroup's keys: its first and last columns; the `full` bounds: this wavefront's
    fa_key_range(g0 / a.group, sq.lq, sq.lk, a.wl, a.wr, lo_min, hi_min);
    fa_key_range((min(g0 + 64, ncols) - 1) / a.group, sq.lq, sq.lk, a.wl, a.wr, lo_max, hi_max);
    int wlo_max = 0, whi_min = 0;
    if (wave_live) {
        fa_key_range(c0 / a.group, sq.lq, sq.lk, a.wl, a.wr, wlo, whi_min);
        fa_key_range((c0 + ncb - 1) / a.group, sq.lq, sq.lk, a.wl, a.wr, wlo_max, whi);
    }
    const uint16_t *kplane = a.k + sq.k0 + (int64_t)hk * a.k_sh;
    const uint16_t *vplane = a.v + sq.v0 + (int64_t)hk * a.v_sh;
    const int Lb = sq.lk;
    const int tb = max(split * a.tiles_per_split, lo_min / 32);
    const int te = min((split + 1) * a.tiles_per_split, (hi_max + 31) / 32);

    float scale_log2 = a.scale_log2;
    if (a.q_mul_dev) scale_log2 *= *a.q_mul_dev;
    // queries pre-scaled by scale * log2(e) and rounded to the dtype (the MFMA prefill's order,
    // and the reference tile kernel's, which scales q first: flash_attn_impl.h:364)
    op_t qop[NJ];
    {
        const uint16_t *qrow = a.q + sq.q0 + (int64_t)qi * a.q_st + (int64_t)head * a.q_sh;
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const int d0 = 32 * j + 8 * g;
            u32x4 w = {0u, 0u, 0u, 0u};
            if (col_ok && d0 < a.head_dim) {
                if (a.q_vec) {
                    w = *(const u32x4 *)(qrow + d0);
                } else {
                    uint32_t *wp = (uint32_t *)&w;
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        wp[e] = (uint32_t)qrow[d0 + 2 * e] | ((uint32_t)qrow[d0 + 2 * e + 1] << 16);
                }
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                if constexpr (F16)
                    w[e] = pack_f16x2(f16_bits_to_f32(w[e] & 0xffffu) * scale_log2,
                                      f16_bits_to_f32(w[e] >> 16) * scale_log2);
                else
                    w[e] = pack_bf16x2(__uint_as_float(w[e] << 16) * scale_log2,
                                       __uint_as_float(w[e] & 0xffff0000u) * scale_log2);
            }
            qop[j] = __builtin_bit_cast(op_t, w);
        }
    }
    const float slope2 = a.alibi ? a.alibi[b * a.alibi_bs + head] * kLog2e : 0.0f;
    const int pos = qi + sq.lk - sq.lq;

    // this wavefront's copies of a tile: 1 KB pieces wave, wave + 4, ... of the K and the V tile
    uint32_t koffs[NCPW], voffs[NCPW];
    {
        uint32_t ka[G::NCP], va[G::NCP];
        fa_copy_offsets<D>(ka, a.k_st, a.head_dim, lane);
        fa_copy_offsets<D>(va, a.v_st, a.head_dim, lane);
#pragma unroll
        for (int j = 0; j < NCPW; ++j) {
            // wave is uniform: select with a switch-free expression on the unrolled copies
            uint32_t kk = ka[0], vv = va[0];
#pragma unroll
            for (int i = 0; i < G::NCP; ++i)
                if (i == wave + W * j) {
                    kk = ka[i];
                    vv = va[i];
                }
            koffs[j] = kk;
            voffs[j] = vv;
        }
    }
    f32x4 acc[NU];
#pragma unroll
    for (int u = 0; u < NU; ++u) acc[u] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m_run = -__builtin_inff(), l_run = 0.0f;

    fa_issue_shared<D, NCPW>(st0, tb, te, kplane, vplane, a.k_st, a.v_st, Lb, a.head_dim, wave,
                             koffs, voffs);
    if constexpr (NST == 3)
        fa_issue_shared<D, NCPW>(st1, tb + 1, te, kplane, vplane, a.k_st, a.v_st, Lb, a.head_dim,
                                 wave, koffs, voffs);
    // step t: stage t % NST holds tile t; after the barrier every copy of tile t has landed and
    // every wavefront is done with tile t - 1, whose stage takes tile t + NST - 1 (with two
    // stages the wait covers every copy in flight: the next tile's are issued after the barrier)
#define FA_TSTEP(CUR, NEXT)                                                                     \
    {                                                                                          \
        if (t >= te) break;                                                                    \
        FA_WAIT_VMCNT(NST == 3 ? 2 * NCPW : 0);                                                \
        __syncthreads();                                                                       \
        fa_issue_shared<D, NCPW>(NEXT, t + NST - 1, te, kplane, vplane, a.k_st, a.v_st, Lb,     \
                                 a.head_dim, wave, koffs, voffs);                              \
        if (wave_live)                                                                         \
            fa_tile<F16, D, false>(CUR, CUR + G::TILE, qop, t, lane, lo, hi, wlo_max, whi_min,  \
                                   Lb, 0, scale_log2, a.softcap2, slope2, pos, m_run, l_run,    \
                                   acc);                                                        \
        __builtin_amdgcn_sched_barrier(0);                                                     \
        ++t;                                                                                   \
    }
    if constexpr (NST == 3) {
        for (int t = tb;;) {
            FA_TSTEP(st0, st2)
            FA_TSTEP(st1, st0)
            FA_TSTEP(st2, st1)
        }
    } else {
        for (int t = tb;;) {
            FA_TSTEP(st0, st1)
            FA_TSTEP(st1, st0)
        }
    }
#undef FA_TSTEP
    FA_WAIT_VMCNT(0);
    if (!wave_live) return;

    // ---- outputs of this wavefront's columns, straight from the accumulators ----
    const float l_col = group16_sum(l_run);
    if (!col_ok) return;
    const int rows = a.batch * a.q_heads * a.q_len;
    float o_mul = a.o_mul;
    if (a.o_mul_dev) o_mul *= *a.o_mul_dev;
    const float inv = l_col > 0.0f ? 1.0f / l_col : 0.0f;
    if (a.splits == 1) {
        const int64_t base = sq.o0 + (int64_t)qi * a.o_st + (int64_t)head * a.o_sh;
#pragma unroll
        for (int u = 0; u < NU; ++u)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int d = 16 * u + 4 * g + i;
                if (d < a.head_dim) store_elem(a.out, base + d, a.dtype, acc[u][i] * inv * o_mul);
            }
    } else {
        const int64_t row = ((int64_t)b * a.q_heads + head) * a.q_len + qi;
        float *po = a.part_o + ((int64_t)split * rows + row) * D;
#pragma unroll
        for (int u = 0; u < NU; ++u)
#pragma unroll
            for (int i = 0; i < 4; ++i) po[16 * u + 4 * g + i] = acc[u][i] * inv;
        if (g == 0)
            a.part_lse[(int64_t)split * rows + row] =
                l_col > 0.0f ? m_run + __builtin_log2f(l_col) : -__builtin_inff();
    }
}

// Split combine: o = sum_s 2^(lse_s - M) o_s / sum_s 2^(lse_s - M) (tq_combine / fa_combine,
// candle-core/kernels/flash_attn_impl.h), times the output factor. One wavefront per output
// row (lane l: head dims l, l + 64, ...), four rows per workgroup.
template <int D>
__global__ __launch_bounds__(256) void fa_combine_kernel(FaArgs a) {
    const int lane = threadIdx.x & 63;
    const int rows = a.batch * a.q_heads * a.q_len;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const int qi = row % a.q_len, head = (row / a.q_len) % a.q_heads;
    const int b = row / (a.q_len * a.q_heads);
    const FaSeq sq = fa_sequence(a, b);
    if (qi >= sq.lq) return;
    const float *lse = a.part_lse + row;
    float M = -__builtin_inff();
    for (int s = 0; s < a.splits; ++s) M = fmaxf(M, lse[(int64_t)s * rows]);
    constexpr int PER = D / 64;
    float o[PER > 0 ? PER : 1];
#pragma unroll
    for (int k = 0; k < PER; ++k) o[k] = 0.0f;
    if (M != -__builtin_inff()) {
        float wsum = 0.0f;
        const float *po = a.part_o + (int64_t)row * D + lane;
        const int64_t step = (int64_t)rows * D;
        for (int s = 0; s < a.splits; ++s) {
            const float e = lse[(int64_t)s * rows];
            const float w = e == -__builtin_inff() ? 0.0f : __builtin_amdgcn_exp2f(e - M);
            wsum += w;
#pragma unroll
            for (int k = 0; k < PER; ++k) o[k] += w * po[s * step + 64 * k];
        }
#pragma unroll
        for (int k = 0; k < PER; ++k) o[k] /= wsum;
    }
    float o_mul = a.o_mul;
    if (a.o_mul_dev) o_mul *= *a.o_mul_dev;
    const int64_t base = sq.o0 + (int64_t)qi * a.o_st + (int64_t)head * a.o_sh;
#pragma unroll
    for (int k = 0; k < PER; ++k) {
        const int d = lane + 64 * k;
        if (d < a.head_dim) store_elem(a.out, base + d, a.dtype, o[k] * o_mul);
    }
}

}  // namespace cqkv
