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
// Kernel shape (head dim D = 128 or 64; one workgroup = 8 wavefronts = 64 queries x 4 query heads
// sharing a kv head, 32 queries per wavefront):
//  * Both products run on v_mfma_f32_32x32x16_bf16. S^T = K Q^T: K (32 keys x 16 dims) comes
//    from LDS with ds_read_b128, Q^T (pre-scaled by scale * log2(e), rounded to bf16) stays in
//    registers for the whole key loop. The S^T accumulator of a lane holds one query column, so
//    the row-wise online softmax needs one cross-lane step, and its registers 4i0..4i0+7 are
//    directly the P^T operand of a 16-key step of O^T = V^T P^T (the k order inside a step is
//    permuted to match).
//  * V^T operands come by ds_read_b128 from a V^T tile written by the pre-pass
//    (prefill_stage_kernel) with its keys already in that permuted order.
//  * K and V^T tiles of 64 keys stream through two 4-stage LDS rings, filled by asynchronous
//    buffer_load_dwordx4 ... lds copies issued three tiles ahead; one barrier per tile. Chunks
//    of a row are XOR-swizzled so the reads are free of bank conflicts.
//  * Software-pipelined tile loop: each wavefront computes S of the next tile on the MFMA pipe
//    while its VALU exponentiates this tile's scores, then runs P V of this tile on the MFMA
//    pipe while its VALU sums P and takes the next tile's row maxima. The MFMA and VALU work of
//    one wavefront are interleaved instruction by instruction (sched_group_barrier), and the two
//    wavefronts of each SIMD fill each other's stalls.
//  * Causal work is uneven: the workgroups with the most key tiles are dispatched first.
#include <algorithm>
#include <type_traits>

#include "cqkv_device.h"
#include "cqkv_host.h"
#include "flash_plain.h"

namespace cqkv {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

constexpr int kPfD = 128;          // head dim of the fused FP8 append and the E4M3 K / V path
constexpr int kPfBQ = 64;          // queries per workgroup (two wavefronts of 32 per head)
constexpr int kPfBK = 64;          // keys per tile of the pre-pass and of the attention at D <= 128

struct PrefillArgs {
    const uint16_t *q, *k, *v;
    uint16_t *out;
    int64_t q_sb, q_st, q_sh;  // element strides: batch, token, head
    int64_t k_sb, k_st, k_sh;
    int64_t v_sb, v_st, v_sh;
    int64_t o_sb, o_st, o_sh;
    const uint16_t *vt;  // V transposed: (batch, kv head, D, vt_len), keys in S^T register order
    int32_t vt_len;      // keys per row of vt: kv_len rounded up to the key tile
    // fused FP8 append (append != 0): codes / scales planes of the key and value cache sides
    uint8_t *kc, *ks, *vc, *vs;
    uint32_t kc_plane, ks_plane, vc_plane, vs_plane;
    int32_t append, position;
    int32_t q_len, kv_len, q_heads, kv_heads, group, heads_per_wg, q_blocks, batch;
    int32_t wl, wr;
    float scale_log2;
    // score terms (candle-core/kernels/flash_attn_impl.h:42-47, fa_logit), in the exp2 units of
    // the scores: softcap2 = softcap * log2(e) (0: off), slopes * log2(e) from alibi[b * alibi_bs
    // + head] (null: off)
    float softcap2;
    const float *alibi;
    int32_t alibi_bs;
    // variable-length batches (flash_attn.rs varlen, cu_seqlens): sequence b is rows cu_q[b] ..
    // cu_q[b + 1] - 1 of q / out and cu_k[b] .. of k / v (null: dense, batch strides); q_len /
    // kv_len are the maximum lengths, total_q / total_k the row counts of the tensors
    const int32_t *cu_q, *cu_k;
    int32_t total_q, total_k;
    // FP8 K / V descales (flash_attn_impl.h:63, 434: scores dot * k_descale, outputs times
    // v_descale / l): host factors times device factors (null: 1), folded into the query
    // pre-scale and the output normalisation
    float q_mul, o_mul;
    const float *q_mul_dev, *o_mul_dev;
    // E4M3 K / V (e4m3 != 0, dense batches): the pre-pass widens the codes of k8 / v8 (byte
    // strides) to the dtype (exact in bf16 and f16): K into kst (batch, kv head, kv_len, D),
    // which the attention kernel then reads as k, V straight into V^T
    const uint8_t *k8, *v8;
    int64_t k8_sb, k8_st, k8_sh, v8_sb, v8_st, v8_sh;
    uint16_t *kst;
    int32_t e4m3, f16;
};

// First rows and lengths of sequence b. Variable-length offsets are clamped into the tensors
// and the lengths to q_len / kv_len, so inconsistent prefix sums cannot address memory outside
// them (they give wrong rows, not faults).
struct PfSeq {
    int64_t q0, k0;  // element offsets of the sequence's first q / out row and k / v row
    int64_t o0, v0;
    int lq, lk;
};
__device__ inline PfSeq pf_sequence(const PrefillArgs &a, int b) {
    PfSeq r;
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

__device__ inline f32x16 mfma32x32x16(bf16x8 a, bf16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
__device__ inline f32x16 mfma32x32x16(f16x8 a, f16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}
// MFMA operands of the input dtype: q, K, V^T and P all in bf16, or all in f16
template <bool F16>
using pf_op_t = typename std::conditional<F16, f16x8, bf16x8>::type;

__device__ inline u32x4 ldg128(const uint16_t *p) { return *(const u32x4 *)p; }

// visible keys [lo, hi) of query position i (bottom-right aligned)
__device__ inline void pf_key_range(int i, int lq, int lk, int wl, int wr, int &lo, int &hi) {
    const int pos = i + lk - lq;
    lo = wl >= 0 ? max(pos - wl, 0) : 0;
    hi = wr >= 0 ? min(pos + wr + 1, lk) : lk;
    lo = min(lo, lk);
    hi = max(hi, lo);
}

// LDS K tile layout: 64 rows (keys) x 2 D bytes, no padding; the 16-byte chunk c of row r sits at
// chunk position c ^ swz(r). At D = 128 (16 chunks a row) swz takes 16 distinct values over any 16
// consecutive rows (the 16 rows of one ds_read_b128 pass); at D = 64 (8 chunks a row, two rows per
// 256 bytes of banks) (r % 2, c ^ swz(r)) takes 16 distinct values over them: either way the
// reads are conflict-free.
template <int D>
__device__ inline int swz(int r) {
    if constexpr (D >= 128) return ((r & 7) << 1) | ((r >> 3) & 1);  // rows of 16 or 32 chunks
    else return (r >> 1) & 7;
}
// V^T tile layout in LDS: D rows (head dims) x VTROW bytes (keys of the tile); the 16-byte chunk j
// (8 keys) of row d sits at position j ^ swz_vt(d). With 128-byte rows, over any 16 consecutive
// rows (d % 2, position) takes 16 distinct values; with 64-byte rows, (d % 4, position) does: a
// ds_read_b128 of one chunk across 16 rows is conflict-free either way.
template <int VTROW>
__device__ inline int swz_vt(int d) {
    if constexpr (VTROW == 128) return (d >> 1) & 7;
    else return (d >> 2) & 3;
}
// Per head dim:
//  * the workgroup: W wavefronts, W / 2 query heads x 2 halves of the 64 queries (8 at D <= 128,
//    two per SIMD; 4 at D = 256, one per SIMD with VGPRs and AGPRs, as the 32 x 256 accumulator,
//    the queries and the scores take more than 256 registers);
//  * key tiles of BK keys (64; 32 at D = 256, so that four ring stages of K and V^T fit in LDS):
//    MB 32-key blocks of S, KK 16-key steps of O^T += V^T P^T;
//  * 16-dim k-steps of S = K Q^T, 32-dim blocks of O^T, bytes of a K row and tile, of a V^T row
//    (BK keys) and tile, and each wavefront's 1 KB copies of a tile: K rows (BK / W) w .., V^T rows
//    (D / W) w .. in pieces of 1024 / VTROW rows.
//  * The V^T stages follow the four K stages in LDS: VBIAS shifts V^T read offsets so that
//    (stage - VBIAS) + block offset fits the 16-bit DS offset.
//  * VALU instructions per MFMA of the two blocks of a tile step (scores: exponentials and
//    conversions; then row sums, shift and row maximum).
template <int D>
struct PfGeom {
    static constexpr int W = D == 256 ? 4 : 8;
    static constexpr int BK = D == 256 ? 32 : 64, MB = BK / 32, KK = BK / 16, VTROW = 2 * BK;
    static constexpr int KS = D / 16, MD = D / 32;
    static constexpr int ROW = 2 * D, KTILE = BK * ROW, VTILE = D * VTROW;
    static constexpr int RPC = 1024 / ROW;  // K rows per copy
    static constexpr int KCP = KTILE / 1024 / W, VCP = VTILE / 1024 / W;
    static constexpr int CP = KCP + VCP;    // copies per wavefront and tile
    static constexpr uint32_t VBIAS = 4 * KTILE;
    static constexpr int NM = MB * KS;      // MFMAs per block (S(t + 1); O^T += V^T P^T)
    static constexpr int V1 = (24 * MB + NM - 1) / NM, V2 = (32 * MB + NM - 1) / NM;
    static constexpr int V2C = (16 * MB + NM - 1) / NM;  // block 2 when the MFMA adds -m_run
    // D = 256: the queries enter the MFMA as given and the scores are scaled in f32 (the shift
    // becomes one FMA); with sums over 256 dims the rounding of pre-scaled queries to the dtype
    // moved outputs by up to 3 bf16 ulps
    static constexpr bool QRAW = D == 256;
    static_assert(NM == MD * KK, "both blocks of a step have NM products");
};

typedef __attribute__((address_space(3))) void lds_void;

#define PF_INLINE __device__ __attribute__((always_inline)) inline

// A buffer resource from wavefront-uniform values, built in scalar registers (the compiler can
// otherwise move the address to vector registers and wrap each copy in a per-lane loop).
PF_INLINE rsrc_t pf_rsrc(const void *base, uint32_t bytes) {
    const uint64_t p = (uint64_t)base;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)p);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(p >> 32));
    return make_rsrc((const void *)(((uint64_t)hi << 32) | lo), __builtin_amdgcn_readfirstlane(bytes));
}
// Asynchronous global -> LDS copy of key tile kt into the stages kstage / vstage: K rows (keys)
// and V^T rows (head dims), one buffer_load_dwordx4 ... lds (1 KB) per 1024 / (2 D) K rows / 8
// V^T rows. Wavefront w copies K rows 8w .. 8w+7 and V^T rows (D / 8) w .. K: lane l writes
// chunk position l % (D / 8) of its row, so it loads logical chunk (l % (D / 8)) ^ swz(row); the
// buffer range ends at the last key, so rows past it read zeros. V^T: lane l writes chunk
// position l % 8 of row l / 8 (the pre-pass zero-fills keys past the end). Tiles past the last one
// (valid false) get a zero-size resource: no memory access, zeros into a stage nobody reads
// again. Buffer loads count on vmcnt only, so the LDS reads of other stages need no wait on
// these copies.
template <int D>
PF_INLINE void pf_issue_tile(uint8_t *kstage, uint8_t *vstage, const uint16_t *kplane,
                             const uint16_t *vtplane, int64_t k_st, int vt_len,
                             const uint32_t *koff, const uint32_t *voff, int kt, int kv_len,
                             int wave, bool valid) {
    using G = PfGeom<D>;
    const int row0 = valid ? kt * G::BK : 0;
    const int nvalid = min(G::BK, kv_len - row0);
    const rsrc_t kr = pf_rsrc(kplane + (int64_t)row0 * k_st,
                              valid ? (uint32_t)((int64_t)(nvalid - 1) * k_st * 2 + G::ROW) : 0u);
#pragma unroll
    for (int r = 0; r < G::KCP; ++r)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            kr, (lds_void *)(kstage + ((G::BK / G::W) * wave + G::RPC * r) * G::ROW), 16, koff[r], 0, 0, 0);
    const rsrc_t vr = pf_rsrc(vtplane + row0, valid ? (uint32_t)(((int64_t)D * vt_len - row0) * 2) : 0u);
#pragma unroll
    for (int r8 = 0; r8 < G::VCP; ++r8)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            vr, (lds_void *)(vstage + ((D / G::W) * wave + (1024 / G::VTROW) * r8) * G::VTROW), 16,
            voff[r8], 0, 0, 0);
}
// byte offsets of this lane's copy sources from a tile's first K row / first V^T key
template <int D>
PF_INLINE void pf_copy_offsets(uint32_t *koff, uint32_t *voff, int64_t k_st, int vt_len, int wave,
                               int lane) {
    using G = PfGeom<D>;
    constexpr int CPR = G::ROW / 16;  // 16-byte chunks per K row
#pragma unroll
    for (int r = 0; r < G::KCP; ++r) {
        const int row = (G::BK / G::W) * wave + G::RPC * r + lane / CPR;
        koff[r] = (uint32_t)(((int64_t)row * k_st + 8 * ((lane % CPR) ^ swz<D>(row))) * 2);
    }
    constexpr int VCPR = G::VTROW / 16;  // 16-byte chunks per V^T row
#pragma unroll
    for (int r8 = 0; r8 < G::VCP; ++r8) {
        const int d = (D / G::W) * wave + (1024 / G::VTROW) * r8 + lane / VCPR;
        voff[r8] = (uint32_t)(((int64_t)d * vt_len + 8 * ((lane % VCPR) ^ swz_vt<G::VTROW>(d))) * 2);
    }
}

// s_waitcnt vmcnt(n) (gfx9 encoding; expcnt and lgkmcnt left at their maxima)
#define PF_WAIT_VMCNT(n) __builtin_amdgcn_s_waitcnt((((n) & 15) | (((n) >> 4) << 14)) | 0x0f70)

template <int D>
struct PfState {
    u32x4 qop[D / 16];  // Q^T operands (16-dim steps ks) of this wavefront's 32 queries, raw bits
    f32x16 acc[D / 32]; // O^T: 32-dim block md
    float negm;      // -m_run (0 before the first key), added to the raw scores
    f32x16 negv;     // negm in every register: the initial value of the score products when
                     // the scores need no f32 scaling or terms before the shift
    float m_run, l_run;
    float c2;        // scores' factor when the queries enter unscaled (QRAW): scale * log2(e)
    float mraw;      // the mask value of unscaled scores: -inf times the sign of c2
    float thr;       // the row maximum moves when a tile's maximum exceeds thr: -inf before the
                     // row's first key, then 8 (p stays below 2^8)
    int qlo, qhi;    // visible keys of this lane's query
};

constexpr int kDsRead = 0x100, kMfma = 0x008, kValu = 0x402;  // sched_group_barrier classes (VALU + TRANS)

// Orders a block of NM MFMAs with its NM LDS operand reads, VALU VALU instructions per MFMA
// and the VMEM (tile copy) instructions: four reads first, then MFMA, read, copy, VALU x VALU,
// so each MFMA's operand was requested four MFMAs earlier and the VALU work fills the MFMA
// pipe's busy cycles.
template <int VALU, int VMEM = 0, int NM = 16>
PF_INLINE void pf_block_schedule() {
#pragma unroll
    for (int i = 0; i < 4; ++i) __builtin_amdgcn_sched_group_barrier(kDsRead, 1, 0);
#pragma unroll
    for (int i = 0; i < NM; ++i) {
        __builtin_amdgcn_sched_group_barrier(kMfma, 1, 0);
        if (i < NM - 4) __builtin_amdgcn_sched_group_barrier(kDsRead, 1, 0);
        if (i < VMEM) __builtin_amdgcn_sched_group_barrier(0x010, 1, 0);
        if (VALU > 0) __builtin_amdgcn_sched_group_barrier(kValu, VALU, 0);
    }
}

// Per-lane LDS read offsets from the first stage of each ring, kept in registers and made opaque
// at every step, so each read is one register plus a constant that fits the 16-bit DS offset
// field (stage, key block, head-dim block); left alone, the compiler keeps a register per
// (stage, offset) pair.
template <int D>
struct PfAddr {
    uint32_t k[D / 16];           // K row qr, chunk 2 ks + h (swizzled), of key block 0
    uint32_t v[PfGeom<D>::KK];    // VBIAS + V^T row qr, chunk 2 kk + h (swizzled), of head-dim block 0
};
// The V^T stages follow the four K stages; biasing the V^T offsets by their size (64 KB at
// D = 128) leaves (stage address - bias) + head-dim block offset, below 64 KB, as the constant
// part.
template <int D>
PF_INLINE void pf_addr_init(PfAddr<D> &ad, int lane) {
    const int qr = lane & 31, h = lane >> 5;
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks)
        ad.k[ks] = qr * PfGeom<D>::ROW + (((2 * ks + h) ^ swz<D>(qr)) << 4);
#pragma unroll
    for (int kk = 0; kk < PfGeom<D>::KK; ++kk)
        ad.v[kk] = PfGeom<D>::VBIAS + qr * PfGeom<D>::VTROW +
                   (((2 * kk + h) ^ swz_vt<PfGeom<D>::VTROW>(qr)) << 4);
}
template <int D>
PF_INLINE void pf_addr_opaque(PfAddr<D> &ad) {
#pragma unroll
    for (int i = 0; i < D / 16; ++i) asm volatile("" : "+v"(ad.k[i]));
#pragma unroll
    for (int i = 0; i < PfGeom<D>::KK; ++i) asm volatile("" : "+v"(ad.v[i]));
}

// S^T (BK keys x 32 queries) = K Q^T for the tile at k_lds: MB 32-key blocks.
template <bool F16, int D>
PF_INLINE void pf_qk(f32x16 *s, const PfState<D> &st, const uint8_t *k_lds, const PfAddr<D> &ad,
                     const f32x16 &c0) {
    using op_t = pf_op_t<F16>;
    constexpr int KS = D / 16, MB = PfGeom<D>::MB;
    op_t kop[MB * KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
            kop[KS * mb + ks] = __builtin_bit_cast(
                op_t, *(const u32x4 *)(k_lds + ad.k[ks] + 32 * mb * PfGeom<D>::ROW));
    // with two key blocks their chains alternate, so consecutive products are independent
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
        s[mb] = mfma32x32x16(kop[KS * mb], __builtin_bit_cast(op_t, st.qop[0]), c0);
#pragma unroll
    for (int ks = 1; ks < KS; ++ks)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
            s[mb] = mfma32x32x16(kop[KS * mb + ks], __builtin_bit_cast(op_t, st.qop[ks]), s[mb]);
}

// Soft-capping and ALiBi of the raw scores of a tile whose first key is k0 (exp2 units, in the
// reference's order: cap * tanh(s / cap), then - slope * |pos - key|; fa_logit,
// candle-core/kernels/flash_attn_impl.h:42-47). pos is the lane's query position in key
// coordinates.
struct PfLogit {
    float cap2;   // softcap * log2(e) (0: off)
    float e2;     // 2 log2(e) / cap2: exp2(s * e2) = e^(2 s / cap2)
    float slope2; // ALiBi slope * log2(e) of the wavefront's head (0: off)
    int pos;
};
// cap * tanh(x / cap) = cap - 2 cap / (e^(2x / cap) + 1): one exp2 and one reciprocal, exact
// limits at both ends (e -> inf: cap; e -> 0: -cap), absolute error ~1e-7 cap
template <int MB>
PF_INLINE void pf_logit(f32x16 *s, const PfLogit &lg, int k0, int lane) {
    if (lg.cap2 > 0.0f) {
        const float two_cap = 2.0f * lg.cap2;
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const float e = __builtin_amdgcn_exp2f(s[mb][j] * lg.e2);
                s[mb][j] = lg.cap2 - two_cap * __builtin_amdgcn_rcpf(e + 1.0f);
            }
    }
    if (lg.slope2 != 0.0f) {
        const int d0 = lg.pos - (k0 + 4 * (lane >> 5));  // pos - key of register 0
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const int dist = d0 - (32 * mb + 8 * (j >> 2) + (j & 3));
                s[mb][j] -= lg.slope2 * (float)(dist < 0 ? -dist : dist);
            }
    }
}

// masks scores of keys outside the lane's visible range (tiles that cross a range end only)
template <int D>
PF_INLINE void pf_mask(f32x16 *s, const PfState<D> &st, int k0, int lane,
                       float mval = -__builtin_inff()) {
    const int h = lane >> 5;
    // key - qlo of register 0, made opaque so the per-register offsets stay immediates
    int u = k0 + 4 * h - st.qlo;
    asm volatile("" : "+v"(u));
    const uint32_t w = (uint32_t)(st.qhi - st.qlo);
#pragma unroll
    for (int mb = 0; mb < PfGeom<D>::MB; ++mb)
#pragma unroll
        for (int j = 0; j < 16; ++j)
            if ((uint32_t)(u + 32 * mb + 8 * (j >> 2) + (j & 3)) >= w) s[mb][j] = mval;
}

PF_INLINE float pf_max_halves(float x) {  // max of lanes l and l ^ 32
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
PF_INLINE float pf_sum_halves(float x) {  // sum of lanes l and l ^ 32
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// scores relative to the running maximum
template <int MB>
PF_INLINE void pf_scale(f32x16 *s, float c) {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int j = 0; j < 16; ++j) s[mb][j] *= c;
}
// unscaled scores to the exponent: s * c - m_run, one FMA each
template <int MB>
PF_INLINE void pf_shift_scaled(f32x16 *s, float c, float negm) {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int j = 0; j < 16; ++j) s[mb][j] = __builtin_fmaf(s[mb][j], c, negm);
}
template <int MB>
PF_INLINE void pf_shift(f32x16 *s, float negm) {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int j = 0; j < 16; ++j) s[mb][j] += negm;
}

// this lane's maximum over the tile (two chains: the two key blocks, or the even and odd
// registers of one)
template <int MB>
PF_INLINE float pf_rowmax(const f32x16 *s) {
    if constexpr (MB == 2) {
        float m0 = s[0][0], m1 = s[1][0];
#pragma unroll
        for (int j = 1; j < 16; ++j) {
            m0 = fmaxf(m0, s[0][j]);
            m1 = fmaxf(m1, s[1][j]);
        }
        return fmaxf(m0, m1);
    } else {
        float m0 = s[0][0], m1 = s[0][1];
#pragma unroll
        for (int j = 2; j < 16; j += 2) {
            m0 = fmaxf(m0, s[0][j]);
            m1 = fmaxf(m1, s[0][j + 1]);
        }
        return fmaxf(m0, m1);
    }
}

// The row maximum moves (rare): s is shifted to the new maximum, O and the row sum rescaled.
// Q carries scale * log2(e) and pf_shift adds -m_run, so s is the exponent of p = exp2(s)
// relative to m_run.
template <int D>
PF_INLINE void pf_rescale(f32x16 *s, PfState<D> &st, float mx, bool need) {
    const bool fresh = st.m_run == -__builtin_inff();
    const float shift = need ? mx : 0.0f;
    const float m_new = need ? (fresh ? 0.0f : st.m_run) + mx : st.m_run;
    const float alpha = need ? __builtin_amdgcn_exp2f(st.m_run - m_new) : 1.0f;
#pragma unroll
    for (int mb = 0; mb < PfGeom<D>::MB; ++mb)
#pragma unroll
        for (int j = 0; j < 16; ++j) s[mb][j] -= shift;
#pragma unroll
    for (int md = 0; md < D / 32; ++md) st.acc[md] *= alpha;
    st.l_run *= alpha;
    st.m_run = m_new;
    st.thr = m_new == -__builtin_inff() ? -__builtin_inff() : 8.0f;
    st.negm -= shift;  // -m_new: 0 - mx for a row's first keys, -m_run - mx after
#pragma unroll
    for (int j = 0; j < 16; ++j) st.negv[j] = st.negm;
}

// p = exp2(s), packed to the P^T operands of the dtype (raw bits)
template <bool F16, int MB>
PF_INLINE void pf_exp(u32x4 *pop, const f32x16 *s) {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            uint32_t w[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float p0 = __builtin_amdgcn_exp2f(s[mb][8 * half + 2 * e]);
                const float p1 = __builtin_amdgcn_exp2f(s[mb][8 * half + 2 * e + 1]);
                if constexpr (F16) {
                    w[e] = pack_f16x2(p0, p1);
                } else {
                    const bf16x2 pp = {(__bf16)p0, (__bf16)p1};
                    w[e] = __builtin_bit_cast(uint32_t, pp);
                }
            }
            pop[2 * mb + half] = u32x4{w[0], w[1], w[2], w[3]};
        }
}

// the row sum adds the bf16 values the product uses, two per dot2 instruction, in two chains
// (each word goes through a scalar: clang's __builtin_bit_cast of a vector element reads
// element 0)
template <bool F16>
PF_INLINE float pf_dot2_ones(uint32_t w, float acc) {
    if constexpr (F16) {
        typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
        const f16x2_t ones = {(_Float16)1.0f, (_Float16)1.0f};
        return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, w), ones, acc, false);
    } else {
        const bf16x2 ones = {(__bf16)1.0f, (__bf16)1.0f};
        return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w), ones, acc, false);
    }
}
template <bool F16, int D>
PF_INLINE void pf_psum(PfState<D> &st, const u32x4 *pop) {
    float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
    for (int i = 0; i < 2 * PfGeom<D>::MB; ++i) {
        const u32x4 w = pop[i];
        const uint32_t w0 = w.x, w1 = w.y, w2 = w.z, w3 = w.w;
        a0 = pf_dot2_ones<F16>(w0, a0);
        a1 = pf_dot2_ones<F16>(w1, a1);
        a0 = pf_dot2_ones<F16>(w2, a0);
        a1 = pf_dot2_ones<F16>(w3, a1);
    }
    st.l_run += a0 + a1;
}

// O^T += V^T P^T over the V^T tile at v_lds. 16-key step kk = keys 16 kk + [0, 16): the P^T
// operand holds S^T registers 8 (kk % 2) .. +7 of key block kk / 2, i.e. lane half h holds keys
// 16 kk + 8 (e / 4) + 4 h + e % 4 in k-slot 8 h + e; the pre-pass stores V^T keys in that order
// (bits 2 and 3 of the key swapped), so the A operand of lane (d, h) is chunk 2 kk + h of row d.
template <bool F16, int D>
PF_INLINE void pf_pv(PfState<D> &st, const u32x4 *pop, const uint8_t *v_lds, const PfAddr<D> &ad) {
    using op_t = pf_op_t<F16>;
    constexpr int MD = D / 32, KK = PfGeom<D>::KK;
    op_t vt[KK * MD];
#pragma unroll
    for (int kk = 0; kk < KK; ++kk)
#pragma unroll
        for (int md = 0; md < MD; ++md)
            vt[MD * kk + md] = __builtin_bit_cast(
                op_t, *(const u32x4 *)(v_lds + (ad.v[kk] - PfGeom<D>::VBIAS) + md * 32 * PfGeom<D>::VTROW));
#pragma unroll
    for (int kk = 0; kk < KK; ++kk)
#pragma unroll
        for (int md = 0; md < MD; ++md)
            st.acc[md] = mfma32x32x16(vt[MD * kk + md], __builtin_bit_cast(op_t, pop[kk]), st.acc[md]);
}

// One key tile t of a wavefront (not the last), with S(t) in `cur`:
//  * block 1: S(t + 1) = K(t + 1) Q^T into `nxt` on the MFMA pipe while the VALU turns S(t)
//    into P(t) = exp2(S(t));
//  * on tiles that cross a range end, S(t + 1) is masked;
//  * block 2: O += V(t)^T P(t) on the MFMA pipe while the VALU adds up the row sum of P(t),
//    shifts S(t + 1) by -m_run and takes its row maximum; the copies of a later tile
//    (issue_copies) are issued among its first MFMAs;
//  * then, rarely, the row maximum moves (pf_rescale).
// At D = 64 each block has half the MFMAs of D = 128 for the same softmax work: twice the VALU
// instructions go between consecutive MFMAs.
template <bool LOGIT, bool F16, int D, typename IssueCopies>
PF_INLINE void pf_tile(f32x16 *cur, f32x16 *nxt, u32x4 *pop, PfState<D> &st,
                       const uint8_t *k_next, const uint8_t *v_cur, const PfAddr<D> &ad,
                       bool masked, int k1, int lane, const PfLogit &lg, IssueCopies &&issue_copies) {
    using G = PfGeom<D>;
    constexpr int NM = G::NM;  // MFMAs per block
    // scores that need no f32 scaling or terms start from -m_run in the MFMA: no shift
    constexpr bool CM = !G::QRAW && !LOGIT;
    if constexpr (CM) pf_qk<F16, D>(nxt, st, k_next, ad, st.negv);
    else pf_qk<F16, D>(nxt, st, k_next, ad, f32x16{});
    pf_exp<F16, G::MB>(pop, cur);
    pf_block_schedule<G::V1, 0, NM>();
    __builtin_amdgcn_sched_barrier(0);
    // P(t) is used only after the branch below: pin its computation to block 1
#pragma unroll
    for (int i = 0; i < 2 * G::MB; ++i) asm volatile("" ::"v"(pop[i]));
    if (LOGIT) {
        if constexpr (G::QRAW) pf_scale<G::MB>(nxt, st.c2);
        pf_logit<G::MB>(nxt, lg, k1, lane);
    }
    // (unscaled scores of the QRAW form take the mask value that their scaling turns into -inf)
    if (masked) pf_mask(nxt, st, k1, lane, G::QRAW && !LOGIT ? st.mraw : -__builtin_inff());
    issue_copies();
    pf_pv<F16, D>(st, pop, v_cur, ad);
    pf_psum<F16, D>(st, pop);
    if (G::QRAW && !LOGIT) pf_shift_scaled<G::MB>(nxt, st.c2, st.negm);
    else if (!CM) pf_shift<G::MB>(nxt, st.negm);
    float mx = pf_rowmax<G::MB>(nxt);
    pf_block_schedule<CM ? G::V2C : G::V2, G::CP, NM>();
    __builtin_amdgcn_sched_barrier(0);
    mx = pf_max_halves(mx);
    const bool need = mx > st.thr;
    if (__builtin_expect(__any(need), 0)) pf_rescale(nxt, st, mx, need);
}

// The last key tile: P(t) and O += V(t)^T P(t).
template <bool F16, int D>
PF_INLINE void pf_last_tile(const f32x16 *cur, u32x4 *pop, PfState<D> &st,
                            const uint8_t *v_cur, const PfAddr<D> &ad) {
    pf_exp<F16, PfGeom<D>::MB>(pop, cur);
    pf_pv<F16, D>(st, pop, v_cur, ad);
    pf_psum<F16, D>(st, pop);
    pf_block_schedule<(D == 256 ? PfGeom<D>::V1 : 128 / D), 0, PfGeom<D>::NM>();
}

// Two wavefronts per SIMD (8 per workgroup, ~240 registers each at D = 128).
// LOGIT: soft-capping and / or ALiBi (a separate instantiation keeps them off the plain path)
template <bool LOGIT, bool F16, int D>
__global__ __launch_bounds__(PfGeom<D>::W * 64, 1) void prefill_kernel(PrefillArgs a) {
    using G = PfGeom<D>;
    // the K and V^T rings: four stages each, as distinct arrays named statically below, so the
    // compiler can tell the asynchronous copy into one stage from the reads of another (a
    // dynamically selected stage makes it wait for every copy before every LDS read); K stages
    // first, so a K read address plus any stage offset fits the 16-bit LDS offset field
    __shared__ __attribute__((aligned(1024))) uint8_t ks0[G::KTILE];
    __shared__ __attribute__((aligned(1024))) uint8_t ks1[G::KTILE];
    __shared__ __attribute__((aligned(1024))) uint8_t ks2[G::KTILE];
    __shared__ __attribute__((aligned(1024))) uint8_t ks3[G::KTILE];
    __shared__ __attribute__((aligned(1024))) uint8_t vs0[G::VTILE];
    __shared__ __attribute__((aligned(1024))) uint8_t vs1[G::VTILE];
    __shared__ __attribute__((aligned(1024))) uint8_t vs2[G::VTILE];
    __shared__ __attribute__((aligned(1024))) uint8_t vs3[G::VTILE];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int qr = lane & 31, h = lane >> 5;

    // 1-D grid: consecutive workgroup ids walk the planes (batch, kv head, head group) first, so
    // the workgroups of one plane share an XCD (ids are dealt round-robin to the 8 XCDs) and its
    // L2; the query blocks with the most key tiles come first.
    // head groups of up to heads_per_wg heads; the last one of a group that is not a multiple
    // (e.g. 7 = 4 + 3 for 28 / 4 heads) leaves its spare wavefronts idle
    const int hgroups = (a.group + a.heads_per_wg - 1) / a.heads_per_wg;
    const int nplanes = a.kv_heads * hgroups * a.batch;
    const int plane = (int)blockIdx.x % nplanes;
    const int qb = a.q_blocks - 1 - (int)blockIdx.x / nplanes;
    const int b = plane / (a.kv_heads * hgroups);
    const int rem = plane % (a.kv_heads * hgroups);
    const int hk = rem % a.kv_heads, hgrp = rem / a.kv_heads;
    const int hslot = wave % (G::W / 2), qhalf = wave / (G::W / 2);
    const int head = hk * a.group + hgrp * a.heads_per_wg + hslot;
    const bool wave_live = hslot < a.heads_per_wg && hgrp * a.heads_per_wg + hslot < a.group;
    const int q0 = qb * kPfBQ;
    const PfSeq sq = pf_sequence(a, b);
    const int lq = sq.lq, lk = sq.lk;
    if (q0 >= lq) return;  // a shorter sequence of a variable-length batch: the whole workgroup

    int lo_first, hi_first, lo_last, hi_last;
    pf_key_range(q0, lq, lk, a.wl, a.wr, lo_first, hi_first);
    pf_key_range(min(q0 + kPfBQ, lq) - 1, lq, lk, a.wl, a.wr, lo_last, hi_last);
    const int kt_begin = lo_first / G::BK;
    const int ntiles = (hi_last + G::BK - 1) / G::BK - kt_begin;

    PfState<D> st;
    {
        const int qi = q0 + 32 * qhalf + qr;
        const bool ok = wave_live && qi < lq;
        const uint16_t *row = a.q + sq.q0 + (int64_t)min(head, a.q_heads - 1) * a.q_sh +
                              (int64_t)min(qi, lq - 1) * a.q_st;
        const float qs = a.scale_log2 * a.q_mul * (a.q_mul_dev ? a.q_mul_dev[0] : 1.0f);
        // (QRAW: a zero factor is made the smallest normal one, so masked scores stay -inf)
        st.c2 = qs == 0.0f ? 1.17549435e-38f : qs;
        st.mraw = st.c2 > 0.0f ? -__builtin_inff() : __builtin_inff();
#pragma unroll
        for (int ks = 0; ks < G::KS; ++ks) {
            u32x4 w = ok ? ldg128(row + 16 * ks + 8 * h) : u32x4{0u, 0u, 0u, 0u};
            // q * scale * log2(e) (* k_descale), rounded to the dtype
#pragma unroll
            for (int e = 0; e < 4 && !G::QRAW; ++e) {
                if constexpr (F16)
                    w[e] = pack_f16x2(f16_bits_to_f32(w[e] & 0xffffu) * qs,
                                      f16_bits_to_f32(w[e] >> 16) * qs);
                else
                    w[e] = pack_bf16x2(__uint_as_float(w[e] << 16) * qs,
                                       __uint_as_float(w[e] & 0xffff0000u) * qs);
            }
            st.qop[ks] = w;
        }
        if (qi < lq) pf_key_range(qi, lq, lk, a.wl, a.wr, st.qlo, st.qhi);
        else st.qlo = st.qhi = 0;
        st.m_run = -__builtin_inff();
        st.thr = -__builtin_inff();
        st.l_run = 0.0f;
        st.negm = 0.0f;
        st.negv = f32x16{};
#pragma unroll
        for (int md = 0; md < G::MD; ++md) st.acc[md] = f32x16{};
    }

    const uint16_t *kplane = a.k + sq.k0 + (int64_t)hk * a.k_sh;
    const uint16_t *vtplane = a.vt + ((int64_t)b * a.kv_heads + hk) * D * a.vt_len;
    PfLogit lg = {};
    if (LOGIT) {
        lg.cap2 = a.softcap2;
        lg.e2 = a.softcap2 > 0.0f ? 2.0f * kLog2e / a.softcap2 : 0.0f;
        lg.slope2 = a.alibi && wave_live ? a.alibi[(int64_t)b * a.alibi_bs + head] * kLog2e : 0.0f;
        lg.pos = q0 + 32 * qhalf + qr + lk - lq;
    }
    PF_WAIT_VMCNT(0);  // the Q loads above must not be counted by the copy waits below

    // Tile t lives in stage t % 4 of both rings. Its copies are issued in step t - 3, after
    // barrier t - 3 (tiles 0-2 before the loop); barrier t (at the top of step t) follows this
    // wavefront's copies of tile t + 1, so K(t + 1) and V(t) are in LDS for every wavefront
    // after it, and stage (t + 3) % 4 has no reader left: K(t - 1) was read in step t - 2,
    // V(t - 1) in step t - 1.
#define PF_KS(k) ((k) == 0 ? ks0 : (k) == 1 ? ks1 : (k) == 2 ? ks2 : ks3)
#define PF_VS(k) ((k) == 0 ? vs0 : (k) == 1 ? vs1 : (k) == 2 ? vs2 : vs3)
    uint32_t koff[G::KCP], voff[G::VCP];
    pf_copy_offsets<D>(koff, voff, a.k_st, a.vt_len, wave, lane);
    // Every step issues the copies of one tile; past the last tile they are dummies with a
    // zero-size resource (no memory access; zeros land in a stage nobody reads again), so each
    // wavefront always has the copies of exactly the next two tiles in flight at a barrier.
#define PF_ISSUE(k, t)                                                                       \
    pf_issue_tile<D>(PF_KS(k), PF_VS(k), kplane, vtplane, a.k_st, a.vt_len, koff, voff,      \
                  kt_begin + (t), lk, wave, (t) < ntiles)
    PF_ISSUE(0, 0);
    PF_ISSUE(1, 1);
    PF_ISSUE(2, 2);
    PF_WAIT_VMCNT(2 * G::CP);
    __builtin_amdgcn_s_barrier();

    // Barrier t: this wavefront's copies of tile t + 1 have landed (those of tile t + 2 may be
    // in flight); the copies of tile t + 3 follow within the step.
#define PF_SYNC(k, t)                                                                        \
    {                                                                                        \
        PF_WAIT_VMCNT(G::CP);                                                                \
        __builtin_amdgcn_s_barrier();                                                        \
    }
    if (!wave_live) {  // heads past the group: copies and barriers only
        for (int t = 0; t < ntiles;) {
            PF_SYNC(0, t) PF_ISSUE(3, t + 3); if (++t == ntiles) break;
            PF_SYNC(1, t) PF_ISSUE(0, t + 3); if (++t == ntiles) break;
            PF_SYNC(2, t) PF_ISSUE(1, t + 3); if (++t == ntiles) break;
            PF_SYNC(3, t) PF_ISSUE(2, t + 3); ++t;
        }
        PF_WAIT_VMCNT(0);
        return;
    }

    const auto tile_masked = [&](int kt) {
        const int k0 = (kt_begin + kt) * G::BK;
        return !(k0 >= lo_last && k0 + G::BK <= hi_first);
    };
    f32x16 sa[G::MB], sb[G::MB];
    u32x4 pop[2 * G::MB];
    PfAddr<D> ad;
    pf_addr_init<D>(ad, lane);
    if (ntiles > 0) {
        pf_qk<F16, D>(sa, st, ks0, ad, f32x16{});  // (negm is 0 here)
        if (LOGIT) {
            if constexpr (G::QRAW) pf_scale<G::MB>(sa, st.c2);
            pf_logit<G::MB>(sa, lg, kt_begin * G::BK, lane);
        }
        if (G::QRAW && !LOGIT) pf_shift_scaled<G::MB>(sa, st.c2, st.negm);
        else pf_shift<G::MB>(sa, st.negm);
        if (tile_masked(0)) pf_mask(sa, st, kt_begin * G::BK, lane);
        const float mx = pf_max_halves(pf_rowmax<G::MB>(sa));
        const bool need = mx > st.thr;
        if (__any(need)) pf_rescale(sa, st, mx, need);
    }
    // Step t: S(t) in CUR, stage t % 4 holds V(t), stage (t + 1) % 4 holds K(t + 1); the
    // copies of tile t + 3 go into stage (t + 3) % 4 in block 2. The last tile leaves the loop
    // (its stage in `last`) and is finished after it.
#define PF_STEP(k, CUR, NXT)                                                                 \
    {                                                                                        \
        pf_addr_opaque(ad);                                                                  \
        PF_SYNC(k, t)                                                                        \
        if (t + 1 == ntiles) {                                                               \
            last = k;                                                                        \
            break;                                                                           \
        }                                                                                    \
        pf_tile<LOGIT, F16, D>(CUR, NXT, pop, st, PF_KS(((k) + 1) & 3), PF_VS(k), ad,        \
                       tile_masked(t + 1), (kt_begin + t + 1) * G::BK, lane, lg, [&] {       \
                    PF_ISSUE(((k) + 3) & 3, t + 3);                                          \
                });                                                                          \
        ++t;                                                                                 \
    }
    int last = 0;
    if (ntiles > 0) {
        for (int t = 0;;) {
            PF_STEP(0, sa, sb)
            PF_STEP(1, sb, sa)
            PF_STEP(2, sa, sb)
            PF_STEP(3, sb, sa)
        }
        PF_WAIT_VMCNT(0);  // the dummy copies past the end
        pf_addr_opaque(ad);
        switch (last) {
            case 0: pf_last_tile<F16, D>(sa, pop, st, vs0, ad); break;
            case 1: pf_last_tile<F16, D>(sb, pop, st, vs1, ad); break;
            case 2: pf_last_tile<F16, D>(sa, pop, st, vs2, ad); break;
            default: pf_last_tile<F16, D>(sb, pop, st, vs3, ad); break;
        }
    }
#undef PF_STEP
#undef PF_SYNC
#undef PF_ISSUE
#undef PF_KS
#undef PF_VS

    // ---- normalise and write O (bf16): lane (qr, h), d = 32 md + 8 (j / 4) + 4 h + j % 4 ----
    const float l = pf_sum_halves(st.l_run);
    const float om = a.o_mul * (a.o_mul_dev ? a.o_mul_dev[0] : 1.0f);
    const float inv = l > 0.0f ? om / l : 0.0f;
    const int qi = q0 + 32 * qhalf + qr;
    if (qi >= lq) return;
    uint16_t *orow = a.out + sq.o0 + (int64_t)qi * a.o_st + (int64_t)head * a.o_sh;
#pragma unroll
    for (int md = 0; md < G::MD; ++md)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            u32x2 w;
            if constexpr (F16) {
                w.x = pack_f16x2(st.acc[md][4 * j + 0] * inv, st.acc[md][4 * j + 1] * inv);
                w.y = pack_f16x2(st.acc[md][4 * j + 2] * inv, st.acc[md][4 * j + 3] * inv);
            } else {
                w.x = pack_bf16x2(st.acc[md][4 * j + 0] * inv, st.acc[md][4 * j + 1] * inv);
                w.y = pack_bf16x2(st.acc[md][4 * j + 2] * inv, st.acc[md][4 * j + 3] * inv);
            }
            *(u32x2 *)(orow + 32 * md + 8 * j + 4 * h) = w;
        }
}

// Pre-pass, one workgroup per 64-key tile of a (batch, kv head) plane, through LDS:
//  * V (batch, kv_len, kv heads, D) -> V^T (batch, kv head, D, vt_len) with the keys of each
//    16-key group in S^T register order (key bits 2 and 3 swapped) and zeros past kv_len;
//  * with a.append, the FP8 quantize-and-append of K and V into the cache at a.position (a
//    multiple of 8): per token s = absmax / 448 (1 for an all-zero row), codes e4m3(x / s) -
//    RowCodec::quantize_row's FP8 branch (candle-core/src/accel/turbo.rs:366-374) as in
//    cqkv_quant_append - key codes row-major, value codes in 8-token transposed tiles.
PF_INLINE float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
PF_INLINE float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// LDS row stride of the pre-pass tiles in 32-bit words: the row plus 16 bytes (272 B at D = 128)
template <int D>
constexpr int st_row() { return D / 2 + 4; }

// 8 E4M3 codes (byte order) -> 8 bf16 or f16 values (exact), one conversion per pair
PF_INLINE u32x4 pf_widen_e4m3(u32x2 c, bool f16) {
    u32x4 r;
    if (f16) {
        r.x = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(c.x, 1.0f, false));
        r.y = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(c.x, 1.0f, true));
        r.z = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(c.y, 1.0f, false));
        r.w = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(c.y, 1.0f, true));
    } else {
        r.x = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(c.x, 1.0f, false));
        r.y = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(c.x, 1.0f, true));
        r.z = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(c.y, 1.0f, false));
        r.w = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(c.y, 1.0f, true));
    }
    return r;
}

template <int D>
__global__ __launch_bounds__(256) void prefill_stage_kernel(PrefillArgs a) {
    constexpr int kStRow = st_row<D>(), CPR = D / 8;  // 16-byte chunks per row
    // (the fused FP8 append and the E4M3 widening are D = 128 only: the host passes neither
    // at D = 64)
    constexpr bool kFull = D == kPfD;
    __shared__ __attribute__((aligned(16))) uint32_t vtile[kPfBK * kStRow];
    __shared__ float vscale[kPfBK], vrcp[kPfBK];
    const int kt = blockIdx.x, hk = blockIdx.y, b = blockIdx.z;
    const int tid = threadIdx.x;
    const PfSeq sq = pf_sequence(a, b);
    const int kv_len = sq.lk;  // this sequence's keys (the V^T row is zero-filled past them)
    const uint16_t *vplane = a.v + sq.v0 + (int64_t)hk * a.v_sh;
    const uint16_t *kplane = a.k + sq.k0 + (int64_t)hk * a.k_sh;
    u32x4 vreg[D / 32], kreg[D / 32];  // every load of the tile is issued before the first use
#pragma unroll
    for (int i = 0; i < D / 32; ++i) {
        const int id = tid + 256 * i, row = id / CPR, c = id % CPR;
        const int key = kt * kPfBK + row;
        u32x4 w = {0u, 0u, 0u, 0u};
        if (key < kv_len) {
            if (kFull && a.e4m3) {  // dense batches: the sequence is batch row b
                const uint8_t *kp = a.k8 + (int64_t)b * a.k8_sb + (int64_t)hk * a.k8_sh;
                const uint8_t *vp = a.v8 + (int64_t)b * a.v8_sb + (int64_t)hk * a.v8_sh;
                w = pf_widen_e4m3(*(const u32x2 *)(vp + (int64_t)key * a.v8_st + 8 * c), a.f16);
                const u32x4 kw = pf_widen_e4m3(*(const u32x2 *)(kp + (int64_t)key * a.k8_st + 8 * c), a.f16);
                *(u32x4 *)(a.kst + (((int64_t)b * a.kv_heads + hk) * a.kv_len + key) * kPfD + 8 * c) = kw;
            } else {
                w = *(const u32x4 *)(vplane + (int64_t)key * a.v_st + 8 * c);
            }
        }
        vreg[i] = w;
        if (kFull && a.append) {
            u32x4 wk = {0u, 0u, 0u, 0u};
            if (key < kv_len) wk = *(const u32x4 *)(kplane + (int64_t)key * a.k_st + 8 * c);
            kreg[i] = wk;
        }
    }
    const int64_t plane = (int64_t)b * a.kv_heads + hk;
#pragma unroll
    for (int i = 0; i < D / 32; ++i) {
        const int id = tid + 256 * i, row = id / CPR, c = id % CPR;
        *(u32x4 *)&vtile[row * kStRow + 4 * c] = vreg[i];
        if (kFull && a.append) {
            // ---- the row's scales from the CPR consecutive lanes that hold it, and its key
            // codes straight from the registers (8 per lane, row-major) ----
            const int t = kt * kPfBK + row;
            const uint32_t kw[4] = {kreg[i].x, kreg[i].y, kreg[i].z, kreg[i].w};
            const uint32_t vw[4] = {vreg[i].x, vreg[i].y, vreg[i].z, vreg[i].w};
            float kmax = 0.0f, vmax = 0.0f;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                kmax = fmaxf(kmax, fmaxf(__builtin_fabsf(bf16_lo(kw[e])), __builtin_fabsf(bf16_hi(kw[e]))));
                vmax = fmaxf(vmax, fmaxf(__builtin_fabsf(bf16_lo(vw[e])), __builtin_fabsf(bf16_hi(vw[e]))));
            }
#pragma unroll
            for (int o = 1; o < CPR; o <<= 1) {
                kmax = fmaxf(kmax, __shfl_xor(kmax, o, 64));
                vmax = fmaxf(vmax, __shfl_xor(vmax, o, 64));
            }
            const float ksc = kmax > 0.0f ? kmax / 448.0f : 1.0f;
            const float vsc = vmax > 0.0f ? vmax / 448.0f : 1.0f;
            const bool live = t < kv_len;
            if (c == 0) {
                vscale[row] = vsc;
                vrcp[row] = 1.0f / vsc;
                if (live) {
                    ((float *)(a.ks + plane * a.ks_plane))[a.position + t] = ksc;
                    ((float *)(a.vs + plane * a.vs_plane))[a.position + t] = vsc;
                }
            }
            if (live) {
                const float kr = 1.0f / ksc;
                u32x2 cw;
                cw.x = fp8_row_codes(bf16_lo(kw[0]), bf16_hi(kw[0]), ksc, kr) |
                       (fp8_row_codes(bf16_lo(kw[1]), bf16_hi(kw[1]), ksc, kr) << 16);
                cw.y = fp8_row_codes(bf16_lo(kw[2]), bf16_hi(kw[2]), ksc, kr) |
                       (fp8_row_codes(bf16_lo(kw[3]), bf16_hi(kw[3]), ksc, kr) << 16);
                *(u32x2 *)(a.kc + plane * a.kc_plane + (int64_t)(a.position + t) * kPfD + 8 * c) = cw;
            }
        }
    }
    __syncthreads();
    // V^T: thread (d, j) writes keys 8j .. 8j+7 (in register order) of head dim d
    uint16_t *out = (uint16_t *)a.vt + ((int64_t)b * a.kv_heads + hk) * D * a.vt_len;
#pragma unroll
    for (int i = 0; i < D / 32; ++i) {
        const int id = tid + 256 * i, d = id >> 3, j = id & 7;
        uint32_t w[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int p0 = 8 * j + 2 * e, p1 = p0 + 1;  // positions -> keys: swap bits 2 and 3
            const int k0 = (p0 & ~12) | ((p0 & 4) << 1) | ((p0 & 8) >> 1);
            const int k1 = (p1 & ~12) | ((p1 & 4) << 1) | ((p1 & 8) >> 1);
            const uint32_t w0 = vtile[k0 * kStRow + (d >> 1)], w1 = vtile[k1 * kStRow + (d >> 1)];
            w[e] = (d & 1) ? ((w0 >> 16) | (w1 & 0xffff0000u)) : ((w0 & 0xffffu) | (w1 << 16));
        }
        *(u32x4 *)(out + (int64_t)d * a.vt_len + kt * kPfBK + 8 * j) = u32x4{w[0], w[1], w[2], w[3]};
    }
    if (!kFull || !a.append) return;
    // ---- value codes: thread (dim pair dp, groups g, g + 4) of 8 tokens, 8-token tiles (the
    // row scales were written before the barrier above) ----
    const int dp = tid & 63;
    uint8_t *vc = a.vc + plane * a.vc_plane;
#pragma unroll
    for (int gi = 0; gi < 2; ++gi) {
        const int g = (tid >> 6) + 4 * gi, t0 = kt * kPfBK + 8 * g;
        if (t0 >= kv_len) continue;
        uint64_t vw0 = 0, vw1 = 0;
        uint32_t mask = 0;
#pragma unroll
        for (int sl = 0; sl < 8; ++sl) {
            if (t0 + sl < kv_len) {
                const uint32_t x = vtile[(8 * g + sl) * kStRow + dp];
                const float sc = vscale[8 * g + sl], rc = vrcp[8 * g + sl];
                const uint32_t c01 = fp8_row_codes(bf16_lo(x), bf16_hi(x), sc, rc);
                vw0 |= (uint64_t)(c01 & 0xffu) << (8 * sl);
                vw1 |= (uint64_t)(c01 >> 8) << (8 * sl);
                mask |= 1u << sl;
            }
        }
        // (position + t0) is a multiple of 8: the group is one value tile of the cache
        uint64_t *dst = (uint64_t *)(vc + (int64_t)((a.position + t0) >> 3) * kPfD * 8 + dp * 16);
        if (mask != 0xffu) {  // keep the codes of the tokens past the end
            uint64_t keep = 0;
            for (int sl = 0; sl < 8; ++sl)
                if (!((mask >> sl) & 1u)) keep |= 0xffull << (8 * sl);
            vw0 |= dst[0] & keep;
            vw1 |= dst[1] & keep;
        }
        *(u32x4 *)dst = u32x4{(uint32_t)vw0, (uint32_t)(vw0 >> 32), (uint32_t)vw1, (uint32_t)(vw1 >> 32)};
    }
}

int fa_plain_run(FaArgs a, const char *who, void *workspace, size_t workspace_bytes,
                 hipStream_t st);

int quant_append_launch(const cqkv_side *side, const void *x, int32_t x_dtype,
                        const int64_t xs[3], int32_t batch, int32_t tokens,
                        const int32_t *positions, int32_t position, hipStream_t stream,
                        int32_t clip_rows);

}  // namespace cqkv

using namespace cqkv;

namespace cqkv {

// The whole prefill call; descales (q_mul / o_mul and their device factors) are those of the FP8
// K / V path (fp8_attn.hip), 1 / null for bf16 K / V.
// Whether a call takes the MFMA prefill kernel (bf16 / f16, head dim 64, 128 or 256, more than 16
// queries); every other call runs the plain-dtype kernel of flash_plain.h.
static bool pf_fast_path(int32_t dtype, int32_t head_dim, int32_t q_len) {
    return (dtype == CQKV_BF16 || dtype == CQKV_F16) &&
           (head_dim == 128 || head_dim == 64 || head_dim == 256) && q_len > 16;
}

// V^T scratch of the MFMA prefill: (batch, kv heads, D, kv_len rounded up to the key tile) bf16.
static size_t pf_vt_bytes(int32_t batch, int32_t kv_len, int32_t kv_heads, int32_t head_dim) {
    return (size_t)batch * kv_heads * head_dim * ((kv_len + kPfBK - 1) / kPfBK * kPfBK) * 2;
}
// K widened from E4M3: (batch, kv heads, kv_len, D) of the dtype.
static size_t pf_kst_bytes(int32_t batch, int32_t kv_len, int32_t kv_heads) {
    return (size_t)batch * kv_heads * kv_len * kPfD * 2;
}

bool prefill_takes(int32_t dtype, int32_t head_dim, int32_t q_len, const void *q,
                   const int64_t q_strides[3], const void *out, const int64_t out_strides[3]) {
    auto aligned = [](const void *p, const int64_t st[3], int bytes) {
        const int64_t e = bytes / 2;
        return (uintptr_t)p % bytes == 0 && st[0] % e == 0 && st[1] % e == 0 && st[2] % e == 0;
    };
    // (the E4M3 widening of the pre-pass is written for head dim 128)
    return head_dim == kPfD && pf_fast_path(dtype, head_dim, q_len) && aligned(q, q_strides, 16) &&
           aligned(out, out_strides, 8);
}

size_t prefill_e4m3_workspace(int32_t batch, int32_t kv_len, int32_t kv_heads) {
    return (pf_vt_bytes(batch, kv_len, kv_heads, kPfD) + 255) / 256 * 256 +
           pf_kst_bytes(batch, kv_len, kv_heads);
}

size_t flash_attn_workspace(int32_t dtype, int32_t batch, int32_t q_len, int32_t kv_len,
                            int32_t q_heads, int32_t kv_heads, int32_t head_dim, bool varlen) {
    // (no query rows need nothing; no keys run the plain kernel, one split)
    if (batch <= 0 || q_len <= 0 || kv_len < 0 || q_heads <= 0 || kv_heads <= 0 ||
        q_heads % kv_heads != 0 || head_dim <= 0 || head_dim > 256)
        return 0;
    const size_t plain =
        fa_plain_workspace_bytes(batch, q_len, kv_len, q_heads, kv_heads, head_dim, varlen);
    // a call of the MFMA prefill's shape whose q / out rows are not aligned for it runs the
    // plain kernel: size for either
    if (kv_len > 0 && pf_fast_path(dtype, head_dim, q_len))
        return std::max(pf_vt_bytes(batch, kv_len, kv_heads, head_dim), plain);
    return plain;
}

template <int D>
static void pf_launch(bool f16, bool terms, dim3 grid, hipStream_t st, const PrefillArgs &a) {
    const dim3 block(PfGeom<D>::W * 64);
    if (f16) {
        if (terms) hipLaunchKernelGGL((prefill_kernel<true, true, D>), grid, block, 0, st, a);
        else hipLaunchKernelGGL((prefill_kernel<false, true, D>), grid, block, 0, st, a);
    } else {
        if (terms) hipLaunchKernelGGL((prefill_kernel<true, false, D>), grid, block, 0, st, a);
        else hipLaunchKernelGGL((prefill_kernel<false, false, D>), grid, block, 0, st, a);
    }
}

int flash_attn_impl(const void *q, const int64_t q_strides[3], const void *k,
                    const int64_t k_strides[3], const void *v, const int64_t v_strides[3],
                    void *out, const int64_t out_strides[3], int32_t dtype, int32_t kv_dtype,
                    int32_t batch, int32_t q_len, int32_t kv_len, int32_t q_heads,
                    int32_t kv_heads, int32_t head_dim, float softmax_scale, int32_t window_left,
                    int32_t window_right, float softcap, const float *alibi_slopes,
                    int32_t alibi_batch_stride, const int32_t *cu_seqlens_q,
                    const int32_t *cu_seqlens_k, int32_t total_q, int32_t total_k,
                    const cqkv_side *k_cache, const cqkv_side *v_cache, int32_t position,
                    void *workspace, size_t workspace_bytes, cqkv_stream_t stream, float q_mul,
                    const float *q_mul_dev, float o_mul, const float *o_mul_dev) {
    // Empty inputs as the reference: no output rows (batch or q_len 0) give an empty output
    // (rocm_backend/accel.rs:87) - only a cache append of the K / V rows remains; no keys
    // (kv_len 0) give zero rows (every key range is empty). Empty tensors may have null data.
    if (!q_strides || !k_strides || !v_strides || !out_strides)
        return fail(CQKV_ERR_ARG, "cqkv_flash_attn: null strides");
    if (batch < 0 || q_len < 0 || kv_len < 0)
        return fail(CQKV_ERR_ARG, "cqkv_flash_attn: batch %d q_len %d kv_len %d", batch, q_len,
                    kv_len);
    const bool no_rows = batch == 0 || q_len == 0, no_keys = batch == 0 || kv_len == 0;
    if ((!no_rows && (!q || !out)) || (!no_keys && (!k || !v)))
        return fail(CQKV_ERR_ARG, "cqkv_flash_attn: null tensor");
    // 16-byte row loads of K / V in both kernels, of q in the MFMA prefill (which also stores
    // 8-byte pieces of out rows); a batch stride is unused with variable-length batches
    const bool vl = cu_seqlens_q != nullptr;
    auto aligned = [vl](const void *p, const int64_t s[3], int bytes) {
        const int64_t e = bytes / 2;  // elements per aligned piece
        return (uintptr_t)p % bytes == 0 && (vl || s[0] % e == 0) && s[1] % e == 0 && s[2] % e == 0;
    };
    // E4M3 K / V under bf16 / f16 queries (cqkv_flash_attn_fp8 passes them only when the MFMA
    // prefill takes the call; 8-byte aligned code rows, checked there)
    const bool e4m3 = kv_dtype == kKvE4M3 && dtype != CQKV_F32;
    // (the f32-query kernel checks its own, 4-element, alignment)
    if (dtype != CQKV_F32 && !e4m3 && !no_keys &&
        (!aligned(k, k_strides, 16) || !aligned(v, v_strides, 16)))
        return fail(CQKV_ERR_ARG,
                    "cqkv_flash_attn: K / V need 16-byte aligned rows (pointers and strides in "
                    "whole 8-element chunks)");
    const bool fast = !no_rows && !no_keys && (kv_dtype == dtype || e4m3) &&
                      pf_fast_path(dtype, head_dim, q_len) && aligned(q, q_strides, 16) &&
                      aligned(out, out_strides, 8);
    if (e4m3 && (!fast || head_dim != kPfD || cu_seqlens_q || k_cache))
        return fail(CQKV_ERR_ARG, "cqkv_flash_attn: E4M3 K / V under %s queries take the MFMA prefill only",
                    dtype == CQKV_F16 ? "f16" : "bf16");
    if (!fast) {
        if (int rc = fa_plain_check("cqkv_flash_attn", dtype, kv_dtype, head_dim, k_strides[1],
                                    v_strides[1], kv_len))
            return rc;
    }
    if (q_heads <= 0 || kv_heads <= 0 || q_heads % kv_heads != 0)
        return fail(CQKV_ERR_ARG, "cqkv_flash_attn: batch %d q_len %d kv_len %d heads %d / %d",
                    batch, q_len, kv_len, q_heads, kv_heads);
    if ((k_cache == nullptr) != (v_cache == nullptr))
        return fail(CQKV_ERR_ARG, "cqkv_flash_attn: give both cache sides or neither");
    if (!(softcap >= 0.0f) || softcap == __builtin_inff())
        return fail(CQKV_ERR_ARG, "cqkv_flash_attn: softcap %g (finite, >= 0; 0 disables it)",
                    (double)softcap);
    if (alibi_slopes && alibi_batch_stride != 0 && alibi_batch_stride != q_heads)
        return fail(CQKV_ERR_ARG, "cqkv_flash_attn: alibi slopes must be (%d) or (%d, %d) (batch stride %d)",
                    q_heads, batch, q_heads, alibi_batch_stride);
    const bool varlen = cu_seqlens_q != nullptr;
    if ((cu_seqlens_k != nullptr) != varlen)
        return fail(CQKV_ERR_ARG, "cqkv_flash_attn: give both cu_seqlens_q and cu_seqlens_k or neither");
    if (varlen && (total_q <= 0 || total_k <= 0))
        return fail(CQKV_ERR_ARG, "cqkv_flash_attn: variable-length rows total_q %d total_k %d",
                    total_q, total_k);
    if (varlen && k_cache)
        return fail(CQKV_ERR_ARG, "cqkv_flash_attn: the cache append takes dense batches only");
    // 32-bit byte offsets inside a key tile (64 token rows) and inside a V^T plane
    if (k_strides && (k_strides[1] <= 0 || k_strides[1] >= (1 << 25)))
        return fail(CQKV_ERR_ARG, "cqkv_flash_attn: key token stride %lld outside [1, 2^25)",
                    (long long)k_strides[1]);
    if (kv_len > (1 << 23))
        return fail(CQKV_ERR_ARG, "cqkv_flash_attn: kv_len %d above 2^23", kv_len);
    hipStream_t st = (hipStream_t)stream;
    if (k_cache) {
        if (int rc = check_side(k_cache, "cqkv_flash_attn (key cache)")) return rc;
        if (int rc = check_side(v_cache, "cqkv_flash_attn (value cache)")) return rc;
        if (k_cache->is_value != 0 || v_cache->is_value != 1 || k_cache->head_dim != head_dim ||
            v_cache->head_dim != head_dim || k_cache->kv_heads != kv_heads ||
            v_cache->kv_heads != kv_heads)
            return fail(CQKV_ERR_ARG, "cqkv_flash_attn: the cache sides must be a key and a value side of the attention's head dim and kv heads");
        if (position < 0 || (int64_t)position + kv_len > k_cache->capacity ||
            (int64_t)position + kv_len > v_cache->capacity)
            return fail(CQKV_ERR_ARG, "cqkv_flash_attn: append [%d, %d) exceeds the cache capacity",
                        position, position + kv_len);
    }
    if (!fast) {
        FaArgs f = {};
        f.q = (const uint16_t *)q;
        f.q_sb = q_strides[0];
        f.q_st = q_strides[1];
        f.q_sh = q_strides[2];
        f.out = out;
        f.o_sb = out_strides[0];
        f.o_st = out_strides[1];
        f.o_sh = out_strides[2];
        f.k = (const uint16_t *)k;
        f.v = (const uint16_t *)v;
        f.k_sb = k_strides[0];
        f.k_st = k_strides[1];
        f.k_sh = k_strides[2];
        f.v_sb = v_strides[0];
        f.v_st = v_strides[1];
        f.v_sh = v_strides[2];
        f.cu_q = cu_seqlens_q;
        f.cu_k = cu_seqlens_k;
        f.total_q = total_q;
        f.total_k = total_k;
        f.batch = batch;
        f.q_len = q_len;
        f.kv_len = kv_len;
        f.q_heads = q_heads;
        f.kv_heads = kv_heads;
        f.group = q_heads / kv_heads;
        f.head_dim = head_dim;
        f.dtype = dtype;
        f.kv_dtype = kv_dtype;
        f.wl = window_left;
        f.wr = window_right;
        f.scale_log2 = softmax_scale * q_mul * kLog2e;
        f.softcap2 = softcap * kLog2e;
        f.alibi = alibi_slopes;
        f.alibi_bs = alibi_batch_stride;
        f.o_mul = o_mul;
        f.q_mul_dev = q_mul_dev;
        f.o_mul_dev = o_mul_dev;
        if (!no_rows)
            if (int rc = fa_plain_run(f, "cqkv_flash_attn", workspace, workspace_bytes, st)) return rc;
        if (k_cache && !no_keys) {
            // K / V are (batch, kv_len, kv_heads, D): the append kernel's (batch, head, token)
            const int64_t ks[3] = {k_strides[0], k_strides[2], k_strides[1]};
            const int64_t vs[3] = {v_strides[0], v_strides[2], v_strides[1]};
            if (int rc = quant_append_launch(k_cache, k, kv_dtype, ks, batch, kv_len, nullptr, position, st, 0))
                return rc;
            if (int rc = quant_append_launch(v_cache, v, kv_dtype, vs, batch, kv_len, nullptr, position, st, 0))
                return rc;
        }
        return CQKV_OK;
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
    const int hpw = head_dim == 256 ? PfGeom<256>::W / 2 : PfGeom<128>::W / 2;  // heads per workgroup
    a.heads_per_wg = a.group < hpw ? a.group : hpw;
    a.q_blocks = (q_len + kPfBQ - 1) / kPfBQ;
    a.wl = window_left;
    a.wr = window_right;
    a.scale_log2 = softmax_scale * kLog2e;
    a.batch = batch;
    a.softcap2 = softcap * kLog2e;
    a.alibi = alibi_slopes;
    a.alibi_bs = alibi_batch_stride;
    a.cu_q = cu_seqlens_q;
    a.cu_k = cu_seqlens_k;
    a.total_q = total_q;
    a.total_k = total_k;
    a.q_mul = q_mul;
    a.o_mul = o_mul;
    a.q_mul_dev = q_mul_dev;
    a.o_mul_dev = o_mul_dev;
    // V^T scratch (stream-ordered: freed after the launches that use it), then, for E4M3 K / V,
    // the widened K
    a.vt_len = (kv_len + kPfBK - 1) / kPfBK * kPfBK;
    void *vt = workspace;
    const size_t vt_bytes = pf_vt_bytes(batch, kv_len, kv_heads, head_dim);
    const size_t kst_off = (vt_bytes + 255) / 256 * 256;
    const size_t ws_bytes = e4m3 ? kst_off + pf_kst_bytes(batch, kv_len, kv_heads) : vt_bytes;
    if (workspace && workspace_bytes < ws_bytes)
        return fail(CQKV_ERR_WORKSPACE, "cqkv_flash_attn: workspace %zu < %zu bytes",
                    workspace_bytes, ws_bytes);
    const bool vt_owned = workspace == nullptr;
    if (vt_owned) CQKV_HIP_CHECK(hipMallocAsync(&vt, ws_bytes, st));
    a.vt = (const uint16_t *)vt;
    if (e4m3) {
        a.e4m3 = 1;
        a.f16 = dtype == CQKV_F16 ? 1 : 0;
        a.k8 = (const uint8_t *)k;
        a.v8 = (const uint8_t *)v;
        a.k8_sb = k_strides[0];
        a.k8_st = k_strides[1];
        a.k8_sh = k_strides[2];
        a.v8_sb = v_strides[0];
        a.v8_st = v_strides[1];
        a.v8_sh = v_strides[2];
        a.kst = (uint16_t *)((char *)vt + kst_off);
        // the attention kernel reads the widened K: (batch, kv head, token) strides
        a.k = a.kst;
        a.v = a.kst;  // (unread)
        a.k_st = kPfD;
        a.k_sh = (int64_t)kv_len * kPfD;
        a.k_sb = (int64_t)kv_heads * kv_len * kPfD;
    }
    // an FP8 append runs inside the pre-pass when value tiles line up (position % 8 == 0) and
    // neither side rotates; any other append as two cqkv_quant_append launches after the attention
    const bool fused = k_cache != nullptr && dtype == CQKV_BF16 && head_dim == kPfD && position % 8 == 0 &&
                       k_cache->format == CQKV_FMT_FP8 &&
                       v_cache->format == CQKV_FMT_FP8 && !side_rotates(k_cache) &&
                       !side_rotates(v_cache);
    if (fused) {
        a.append = 1;
        a.position = position;
        a.kc = (uint8_t *)k_cache->codes;
        a.ks = (uint8_t *)k_cache->scales;
        a.vc = (uint8_t *)v_cache->codes;
        a.vs = (uint8_t *)v_cache->scales;
        a.kc_plane = (uint32_t)cqkv_codes_plane_bytes(CQKV_FMT_FP8, kPfD, k_cache->capacity);
        a.ks_plane = (uint32_t)cqkv_scales_plane_bytes(CQKV_FMT_FP8, kPfD, k_cache->capacity);
        a.vc_plane = (uint32_t)cqkv_codes_plane_bytes(CQKV_FMT_FP8, kPfD, v_cache->capacity);
        a.vs_plane = (uint32_t)cqkv_scales_plane_bytes(CQKV_FMT_FP8, kPfD, v_cache->capacity);
    }
    const dim3 sgrid(a.vt_len / kPfBK, kv_heads, batch);
    if (head_dim == 64) hipLaunchKernelGGL(prefill_stage_kernel<64>, sgrid, dim3(256), 0, st, a);
    else if (head_dim == 256) hipLaunchKernelGGL(prefill_stage_kernel<256>, sgrid, dim3(256), 0, st, a);
    else hipLaunchKernelGGL(prefill_stage_kernel<128>, sgrid, dim3(256), 0, st, a);
    const dim3 grid(a.q_blocks * kv_heads * ((a.group + a.heads_per_wg - 1) / a.heads_per_wg) * batch);
    const bool terms = softcap > 0.0f || alibi_slopes;
    if (head_dim == 64) pf_launch<64>(dtype == CQKV_F16, terms, grid, st, a);
    else if (head_dim == 256) pf_launch<256>(dtype == CQKV_F16, terms, grid, st, a);
    else pf_launch<128>(dtype == CQKV_F16, terms, grid, st, a);
    hipError_t le = hipGetLastError();
    hipError_t fe = vt_owned ? hipFreeAsync(vt, st) : hipSuccess;
    if (le != hipSuccess) return fail(CQKV_ERR_HIP, "cqkv_flash_attn: launch: %s", hipGetErrorString(le));
    CQKV_HIP_CHECK(fe);
    if (k_cache && !fused) {
        // K / V are (batch, kv_len, kv_heads, D): the append kernel's (batch, head, token)
        const int64_t ks[3] = {k_strides[0], k_strides[2], k_strides[1]};
        const int64_t vs[3] = {v_strides[0], v_strides[2], v_strides[1]};
        if (int rc = quant_append_launch(k_cache, k, dtype, ks, batch, kv_len, nullptr, position, st, 0))
            return rc;
        if (int rc = quant_append_launch(v_cache, v, dtype, vs, batch, kv_len, nullptr, position, st, 0))
            return rc;
    }
    return CQKV_OK;
}

}  // namespace cqkv

extern "C" size_t cqkv_flash_attn_workspace_bytes(int32_t dtype, int32_t batch, int32_t q_len,
                                                  int32_t kv_len, int32_t q_heads,
                                                  int32_t kv_heads, int32_t head_dim,
                                                  int32_t varlen) {
    return flash_attn_workspace(dtype, batch, q_len, kv_len, q_heads, kv_heads, head_dim,
                                varlen != 0);
}

extern "C" int cqkv_flash_attn_ext(const void *q, const int64_t q_strides[3], const void *k,
                                   const int64_t k_strides[3], const void *v,
                                   const int64_t v_strides[3], void *out,
                                   const int64_t out_strides[3], int32_t dtype,
                                   int32_t kv_dtype, int32_t batch, int32_t q_len,
                                   int32_t kv_len, int32_t q_heads, int32_t kv_heads,
                                   int32_t head_dim, float softmax_scale, int32_t window_left,
                                   int32_t window_right, float softcap,
                                   const float *alibi_slopes, int32_t alibi_batch_stride,
                                   const int32_t *cu_seqlens_q, const int32_t *cu_seqlens_k,
                                   int32_t total_q, int32_t total_k, const cqkv_side *k_cache,
                                   const cqkv_side *v_cache, int32_t position, void *workspace,
                                   size_t workspace_bytes, cqkv_stream_t stream) {
    clear_error();
    // E4M3 K / V come through cqkv_flash_attn_fp8 (which carries their descales)
    if (kv_dtype == kKvE4M3)
        return fail(CQKV_ERR_ARG, "cqkv_flash_attn_ext: kv_dtype %d (bf16, f16 or f32)", kv_dtype);
    return flash_attn_impl(q, q_strides, k, k_strides, v, v_strides, out, out_strides, dtype,
                           kv_dtype, batch, q_len, kv_len, q_heads, kv_heads, head_dim, softmax_scale,
                           window_left, window_right, softcap, alibi_slopes, alibi_batch_stride,
                           cu_seqlens_q, cu_seqlens_k, total_q, total_k, k_cache, v_cache,
                           position, workspace, workspace_bytes, stream, 1.0f, nullptr, 1.0f,
                           nullptr);
}

extern "C" int cqkv_flash_attn(const void *q, const int64_t q_strides[3], const void *k,
                               const int64_t k_strides[3], const void *v,
                               const int64_t v_strides[3], void *out,
                               const int64_t out_strides[3], int32_t dtype, int32_t batch,
                               int32_t q_len, int32_t kv_len, int32_t q_heads, int32_t kv_heads,
                               int32_t head_dim, float softmax_scale, int32_t window_left,
                               int32_t window_right, const cqkv_side *k_cache,
                               const cqkv_side *v_cache, int32_t position, cqkv_stream_t stream) {
    return cqkv_flash_attn_ext(q, q_strides, k, k_strides, v, v_strides, out, out_strides, dtype,
                               dtype, batch, q_len, kv_len, q_heads, kv_heads, head_dim, softmax_scale,
                               window_left, window_right, 0.0f, nullptr, 0, nullptr, nullptr, 0, 0,
                               k_cache, v_cache, position, nullptr, 0, stream);
}
