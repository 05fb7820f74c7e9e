// Split-K flash-decode kernels over the quantized cache (gfx950), templated on the key and the
// value format (included by decode_inst.hip, one object per key format, and by decode_attn.hip
// for the argument structs).
//
// Reference behaviour (paths relative to the reference repository root): TqAttn / tq_attention
// (candle-core/src/rocm_backend/accel.rs:425-571; kernels tq_attng_core and tq_combine_impl in
// candle-core/kernels/turbo_quant_impl.h:403-619, 659-685), masks of key_range
// (candle-core/src/accel/attention.rs:80-92), the q rotation / o unrotation of the fused
// TurboQuant path (candle-nn/src/turbo_quant.rs:1162-1167, 1263). Numerics follow the reference's
// CPU path (softmax(scale q k^T) v over the dequantized cache, f32 accumulation) within the bf16
// tolerance, not bit for bit.
//
// Kernel shape: one workgroup = 8 wavefronts = one (key split, kv head, batch).
//  * Both products run on v_mfma_f32_16x16x32_bf16. MFMA columns are the (query, head) pairs of
//    the GQA group, 16 per workgroup (more than 16 - chunked prefill or speculative decode over
//    the cache - take more workgroups along a column-block index); rows are keys (S^T = K Q^T)
//    or head dims (O^T = V^T P^T).
//  * A wavefront streams 32-key tiles with nontemporal buffer loads straight into operand
//    registers (two register sets, A/B, no copies) and decodes codes in registers: E4M3 -> bf16 exactly, E2M1
//    with its E8M0 block scale exactly, TurboQuant code bytes through a per-lane LDS table of
//    f16 pairs (TurboQuant runs its MFMAs in f16: codebook values are not bf16-exact).
//    Loads of tiles past the split's end are aimed past the buffer range, so the hardware
//    returns zeros without touching memory and the load schedule stays branch-free.
//  * Key rows are row-major, so lane (r, g) loads the codes of key r for head-dim group g.
//    Value codes are stored in 8-token transposed tiles, so lane (r, g) loads keys 8g..8g+7 of
//    one head dim - the A operand of V^T P^T with no shuffle.
//  * Online softmax runs in the exp2 domain on the S^T accumulator; lane (n, g) holds column n
//    for keys 8g..8g+7, which is the B operand layout P^T needs. Only the running maximum is
//    reduced across lanes. P^T enters the MFMA as a hi + lo pair of 16-bit operands.
//  * The wavefronts of a workgroup interleave tiles and merge through LDS. With one split the
//    workgroup writes the output; otherwise it writes its (o, lse) partial and combine_kernel
//    merges the splits (tq_combine's formula), unrotating TurboQuant values. (A fused "last
//    workgroup combines" variant needs agent-scope release fences, which write back the L2 of
//    the XCD each time; measured at 6x the whole decode time, so the kernel boundary is used.)
#pragma once

#include <type_traits>

#include "cqkv_device.h"
#include "cqkv_host.h"

namespace cqkv {

constexpr uint32_t kOOB = 0x80000000u;  // past every plane (planes are < 2 GiB)

// Paged decode: a run of whole 32-key tiles of one cache block, decoded by one split. The keys
// of the call are the blocks' valid rows concatenated (the reference's block table, PageTable
// in candle-core/src/accel/attention.rs:307-366, walked by attention_packed_blocks,
// candle-nn/src/turbo_quant.rs:1082-1114).
struct PagedSeg {
    const uint8_t *kc, *ks, *vc, *vs;                  // the block's planes
    uint32_t kc_plane, ks_plane, vc_plane, vs_plane;   // bytes per (sequence, kv head) plane
    int32_t tile_begin, tile_end;                      // tiles [begin, end) of the block
    int32_t key_offset;                                // key index of the block's row 0
    int32_t rows;                                      // valid rows of the block
};

struct DecodeArgs {
    const void *q;
    int64_t q_sb, q_sh, q_si;
    const uint8_t *kc, *ks, *vc, *vs;
    uint32_t kc_plane, ks_plane, vc_plane, vs_plane;
    const int32_t *kv_lens;
    int32_t kv_len, q_dtype;
    int32_t q_heads, kv_heads, group, q_len, ncols;
    int32_t col_blocks;  // workgroups along the columns: ceil(ncols / 16)
    float scale_log2;  // softmax scale * log2(e)
    int32_t wl, wr;
    int32_t tiles_per_split, splits, batch;
    float *part_o;       // (splits, rows, D) f32, normalised partial outputs
    float *part_lse;     // (splits, rows) f32, log2-domain lse of each split
    void *out;
    int32_t out_dtype, q_split;  // q_split: queries need a lo part (not bf16 inputs)
    int64_t o_sb, o_sh, o_si;
    int32_t rot_k, rot_v;  // key / value sides with the in-register Hadamard rotation: rotate q,
                           // unrotate o (rot_v: partials always, the combine unrotates)
    uint32_t ksign_bits[8], vsign_bits[8];  // their rotation signs (bit set -> -1)
    float rot_scale;                        // 1 / sqrt(D)
    int32_t head_dim;      // the head dim d <= D: query elements past it are zero, outputs not
                           // written
    float qjl_c;           // TURBOPROD keys: -sqrt(pi / 2) / d
    int32_t partials;      // write partials at any split count (the combine finishes the rows)
    // score terms (the TERMS kernels): soft-capping cap * log2(e) (0: off), ALiBi slopes
    // alibi[b * alibi_bs + head] (device f32, null: off)
    float cap2;
    const float *alibi;
    int32_t alibi_bs;
    float cent[16];  // the TURBO4 code table's codebook (keys', else values'; one per kernel)
    const PagedSeg *segs;  // paged: one segment per split (the planes above are unused)
    const float *qjl;      // TURBOPROD keys: the D x D QJL matrix S (device, row-major)
    float kcent[8];        // compact key table (TURBOPROD, kFmtTurboC keys): their codebook
    float vcent[8];        // compact value table (kFmtTurboC values): their codebook
    int32_t kfmt, vfmt;    // host: the kernel formats of the call (kFmtTurboC where it applies)
};

constexpr float kQjlConst = 1.2533141f;  // sqrt(pi / 2) as the reference's QJL_CONST (turbo.rs:26)

// Visible keys [lo, hi) of query i of lq over lk keys (bottom-right aligned).
__device__ inline void key_range(int i, int lq, int lk, int wl, int wr, int &lo, int &hi) {
    const int pos = i + lk - lq;
    lo = wl >= 0 ? max(pos - wl, 0) : 0;
    hi = wr >= 0 ? min(pos + wr + 1, lk) : lk;
    lo = min(lo, lk);
    hi = max(hi, lo);
}

template <int D>
__device__ inline void fwht_pairs_dec(float &v0, float &v1, int lane) {
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

// The same transform at D = 256, four elements per lane: (v0, v1) are elements 2 lane, 2 lane + 1
// and (v2, v3) elements 128 + 2 lane, 129 + 2 lane. H_256 = H_2 x H_128: the transform of each
// half, then the stride-128 stage inside the lane.
__device__ inline void fwht_quads_dec(float &v0, float &v1, float &v2, float &v3, int lane) {
    fwht_pairs_dec<128>(v0, v1, lane);
    fwht_pairs_dec<128>(v2, v3, lane);
    float a = v0 + v2, b = v0 - v2;
    v0 = a;
    v2 = b;
    a = v1 + v3;
    b = v1 - v3;
    v1 = a;
    v3 = b;
}

__device__ inline bool sign_bit(const uint32_t *bits, int j) { return (bits[j >> 5] >> (j & 31)) & 1u; }

// Kernel-internal format id: TurboMse values or keys whose codes have at most 3 bits, decoded
// through a compact per-side table (as TurboProd keys' codes are) when the other side's
// TurboMse codebook occupies the 64 KB code table (TurboKvCache::with_formats(TurboMse{4},
// TurboMse{3}, ..)).
constexpr int kFmtTurboC = 6;
// Kernel-internal format id: TurboProd{5} keys, whose 4-bit MSE codes go through the 64 KB code
// table (the TurboMse{4} codebook of the head dim) while the QJL part is TurboProd's.
constexpr int kFmtProd4 = 7;
// TurboMse codes (either table).
template <int FMT>
constexpr bool turbo_mse() { return FMT == CQKV_FMT_TURBO4 || FMT == kFmtTurboC; }
// TurboProd keys (either code table).
template <int FMT>
constexpr bool is_prod() { return FMT == CQKV_FMT_TURBOPROD || FMT == kFmtProd4; }
// Codes of at most 3 bits through the compact byte-indexed table.
template <int FMT>
constexpr bool compact_tab() { return FMT == CQKV_FMT_TURBOPROD || FMT == kFmtTurboC; }

// Byte codes (FP8, MXFP8) or nibbles (MXFP4, NVFP4, TurboQuant).
template <int FMT>
constexpr bool is8() { return FMT == CQKV_FMT_FP8 || FMT == CQKV_FMT_MXFP8; }

// Head dim held in k-slot e of MFMA chunk j by lane group g (the same for K and Q operands).
template <int FMT, int D>
__device__ inline int qdim(int j, int g, int e) {
    if constexpr (is8<FMT>()) return 64 * (j >> 1) + 16 * g + 8 * (j & 1) + e;
    else return (D / 4) * g + 8 * j + e;
}

// ---------------------------------------------------------------------------------------------
// per-format tile registers, loads and decoders
// ---------------------------------------------------------------------------------------------
template <int KF, int VF, int D>
struct Tile {
    // keys: 2 sub-tiles x D/32 code words (byte codes: D/16 words, 4 per 16-key row chunk pair)
    uint32_t k[2][is8<KF>() ? D / 16 : D / 32];
    // values: D/32 chunks of 2 head dims x 8 keys (byte codes 4 words, 4-bit 2 words)
    uint32_t v[D / 32][is8<VF>() ? 4 : 2];
    // per sub-tile, this lane's key: FP8 f32 scale; MXFP4 the E8M0 bytes of its head dims (one,
    // two at D = 256); MXFP8 all its E8M0 block bytes (kscale2: bytes 4-7 at D = 256); NVFP4 the
    // E4M3 block bytes of its 64 (D = 256) / 32 (D = 128) / 16 (D = 64) head dims
    uint32_t kscale[2], kscale2[2];
    // key lane % 32 (broadcast across lanes): the MX formats' value block bytes (vs2: bytes 4-7
    // at D = 256)
    uint32_t vs, vs2;
    // FP8 / TURBO4: the scale words of keys 8 g .. 8 g + 7 of the tile (lane group g), the ones the
    // lane's score and P rows need, read directly instead of broadcast across lanes
    uint32_t ks8[8], vs8[8];
    // NVFP4: the value block bytes (D / 64 words per key) and f32 scales of keys 8 g .. 8 g + 7,
    // read directly (config-2 shape 100-103 -> 99 us same-box)
    uint32_t nvb[D / 8], nvg[8];
    // TURBOPROD keys: |r| of keys 8 g .. 8 g + 7, and per sub-tile the lane key's sign bits of
    // its head dims (D / 4 bits: dims (D / 4) g ..; ksg2: bits 32-63 at D = 256)
    uint32_t kr1[8], ksg[2], ksg2[2];
};

// Formats whose per-key scale words are read as ks8 / vs8 (one 32-bit word per key). Same-box
// A/B against the cross-lane broadcast: TurboQuant-4 config 5 270-276 -> 257-264 us, FP8 config 2
// 94.7-95.9 -> 94.3-94.6 us; MXFP4 config 3 got 2 % slower and keeps the broadcast.
template <int FMT>
constexpr bool direct_scales() {
    return FMT == CQKV_FMT_FP8 || turbo_mse<FMT>();
}
// Key formats whose per-token scale multiplies the score after the dot of the bare codes (the
// TurboQuant norm, the NVFP4 token scale), as in the reference's fused kernel (sc = rsc * dot,
// candle-core/kernels/turbo_quant_impl.h:270-271); they read it as ks8.
template <int FMT>
constexpr bool row_scaled_keys() {
    return turbo_mse<FMT>() || FMT == CQKV_FMT_NVFP4;
}

// The 32-bit scale words of keys kb .. kb + 7 (kb a multiple of 8: two aligned 16-byte loads).
template <int BYTES>
__device__ inline void load_scales8(uint32_t *out, rsrc_t r, uint32_t kb, uint32_t oob) {
    static_assert(BYTES == 4, "32-bit scale words");
    const u32x4 a = ld128(r, (kb * 4) | oob), b = ld128(r, (kb * 4 + 16) | oob);
    out[0] = a.x; out[1] = a.y; out[2] = a.z; out[3] = a.w;
    out[4] = b.x; out[5] = b.y; out[6] = b.z; out[7] = b.w;
}

template <int KF, int VF, int D>
__device__ inline void load_tile(Tile<KF, VF, D> &r, int tile, bool live, int lane, rsrc_t kr,
                                 rsrc_t ksr, rsrc_t vr, rsrc_t vsr, uint32_t ktok_off,
                                 uint32_t vtok_off) {
    const int n = lane & 15, g = lane >> 4;
    const uint32_t t0 = (uint32_t)tile * 32u;
    const uint32_t oob = live ? 0u : kOOB;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
        const uint32_t key = t0 + 8 * (n >> 2) + 4 * s + (n & 3);
        if constexpr (is8<KF>()) {
#pragma unroll
            for (int i = 0; i < D / 64; ++i) {
                const u32x4 w = ld128_stream(kr, (key * D + 16 * g + 64 * i) | oob);
                r.k[s][4 * i + 0] = w.x;
                r.k[s][4 * i + 1] = w.y;
                r.k[s][4 * i + 2] = w.z;
                r.k[s][4 * i + 3] = w.w;
            }
            if constexpr (KF == CQKV_FMT_FP8) {
                r.kscale[s] = ld32(ksr, (key * 4) | oob);
            } else if constexpr (D == 256) {
                const u32x2 w = ld64(ksr, (key * 8) | oob);
                r.kscale[s] = w.x;
                r.kscale2[s] = w.y;
            } else if constexpr (D == 128) {
                r.kscale[s] = ld32(ksr, (key * 4) | oob);
            } else {
                r.kscale[s] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(ksr, (key * 2) | oob, 0, 0);
            }
        } else {
            if constexpr (D == 256) {  // head dims 64 g .. 64 g + 63: two 16-byte pieces
                const u32x4 w0 = ld128_stream(kr, (key * 128 + 32 * g) | oob);
                const u32x4 w1 = ld128_stream(kr, (key * 128 + 32 * g + 16) | oob);
                r.k[s][0] = w0.x;
                r.k[s][1] = w0.y;
                r.k[s][2] = w0.z;
                r.k[s][3] = w0.w;
                r.k[s][4] = w1.x;
                r.k[s][5] = w1.y;
                r.k[s][6] = w1.z;
                r.k[s][7] = w1.w;
            } else if constexpr (D == 128) {
                const u32x4 w = ld128_stream(kr, (key * 64 + 16 * g) | oob);
                r.k[s][0] = w.x;
                r.k[s][1] = w.y;
                r.k[s][2] = w.z;
                r.k[s][3] = w.w;
            } else {
                const u32x2 w = ld64_stream(kr, (key * 32 + 8 * g) | oob);
                r.k[s][0] = w.x;
                r.k[s][1] = w.y;
            }
            if constexpr (KF == CQKV_FMT_MXFP4) {
                if constexpr (D == 256)  // blocks 2 g, 2 g + 1
                    r.kscale[s] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(
                        ksr, (key * 8 + 2 * g) | oob, 0, 0);
                else
                    r.kscale[s] = __builtin_amdgcn_raw_buffer_load_b8(
                        ksr, (key * (D / 32) + (D == 128 ? g : g >> 1)) | oob, 0, 0);
            }
            if constexpr (KF == CQKV_FMT_NVFP4) {
                if constexpr (D == 256)  // blocks 4 g .. 4 g + 3
                    r.kscale[s] = ld32(ksr, (key * 16 + 4 * g) | oob);
                else if constexpr (D == 128)
                    r.kscale[s] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(
                        ksr, (key * 8 + 2 * g) | oob, 0, 0);
                else
                    r.kscale[s] = __builtin_amdgcn_raw_buffer_load_b8(ksr, (key * 4 + g) | oob, 0, 0);
            }
        }
    }
#pragma unroll
    for (int u = 0; u < D / 32; ++u) {
        if constexpr (is8<VF>()) {
            const u32x4 w = ld128_stream(vr, (((t0 / 8 + g) * D + 32 * u + 2 * n) * 8) | oob);
            r.v[u][0] = w.x;
            r.v[u][1] = w.y;
            r.v[u][2] = w.z;
            r.v[u][3] = w.w;
        } else {
            const u32x2 w = ld64_stream(vr, (((t0 / 8 + g) * D + 32 * u + 2 * n) * 4) | oob);
            r.v[u][0] = w.x;
            r.v[u][1] = w.y;
        }
    }
    const uint32_t kl = t0 + (lane & 31);
    if constexpr (KF == CQKV_FMT_NVFP4)  // the token scales follow the block bytes
        load_scales8<4>(r.ks8, ksr, ktok_off / 4 + t0 + 8 * g, oob);
    else if constexpr (row_scaled_keys<KF>() || is_prod<KF>())
        load_scales8<4>(r.ks8, ksr, t0 + 8 * g, oob);
    if constexpr (is_prod<KF>()) {
        // the scales plane: norms, |r| (at cap * 4), sign bits (at cap * 8, D / 8 per key)
        const uint32_t cap = ktok_off;  // load_tile's caller passes the capacity here
        load_scales8<4>(r.kr1, ksr, cap + t0 + 8 * g, oob);
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) {
            const uint32_t key = t0 + 8 * (n >> 2) + 4 * s2 + (n & 3);
            if constexpr (D == 256) {
                const u32x2 w = ld64(ksr, (cap * 8 + key * 32 + 8 * g) | oob);
                r.ksg[s2] = w.x;
                r.ksg2[s2] = w.y;
            } else if constexpr (D == 128)
                r.ksg[s2] = ld32(ksr, (cap * 8 + key * 16 + 4 * g) | oob);
            else
                r.ksg[s2] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(ksr, (cap * 8 + key * 8 + 2 * g) | oob, 0, 0);
        }
    }
    if constexpr (direct_scales<VF>()) {
        load_scales8<4>(r.vs8, vsr, t0 + 8 * g, oob);
    } else if constexpr (VF == CQKV_FMT_MXFP4 || VF == CQKV_FMT_MXFP8) {
        if constexpr (D == 256) {
            const u32x2 w = ld64(vsr, (kl * 8) | oob);
            r.vs = w.x;
            r.vs2 = w.y;
        } else {
            r.vs = D == 128 ? ld32(vsr, (kl * 4) | oob)
                            : (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(vsr, (kl * 2) | oob, 0, 0);
        }
    } else if constexpr (VF == CQKV_FMT_NVFP4) {
        const uint32_t kb = t0 + 8 * g;
        constexpr uint32_t kBpk = D / 16;  // block bytes per key
#pragma unroll
        for (int i = 0; i < (int)(8 * kBpk / 16); ++i) {
            const u32x4 w = ld128(vsr, (kb * kBpk + 16 * i) | oob);
            r.nvb[4 * i + 0] = w.x;
            r.nvb[4 * i + 1] = w.y;
            r.nvb[4 * i + 2] = w.z;
            r.nvb[4 * i + 3] = w.w;
        }
        load_scales8<4>(r.nvg, vsr, kb + vtok_off / 4, oob);
    }
}

__device__ inline uint32_t fp4x2_to_bf16x2(uint32_t w, int byte_sel, float scale) {
    bf16x2 v;
    switch (byte_sel) {  // the selector must be an immediate
    case 0: v = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 0); break;
    case 1: v = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 1); break;
    case 2: v = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 2); break;
    default: v = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 3); break;
    }
    return __builtin_bit_cast(uint32_t, v);
}

// MFMA operand type: bf16 for FP8 / MXFP4 (their codes decode exactly), f16 for TurboQuant
// (codebook values, rotated queries: 11 significant bits instead of 8).
template <int FMT>
using op_t = typename std::conditional<turbo_mse<FMT>() || is_prod<FMT>(), f16x8,
                                      bf16x8>::type;
// Key-side operand type (keys and queries): as op_t, except NVFP4 keys, whose E2M1 code times its
// E4M3 block scale is exact in f16 (at most 6 significant bits, magnitudes 2^-10 .. 2688); their
// f32 token scale then multiplies the score after the dot, as a TurboQuant norm does.
template <int FMT>
using kop_t = typename std::conditional<FMT == CQKV_FMT_NVFP4, f16x8, op_t<FMT>>::type;

typedef __attribute__((address_space(3))) const uint32_t lds_u32;

// TurboProd key codes: the f16 pair of code byte b (codes b & 7, b >> 4 & 7; bits 3 and 7 are
// zero) from a 15 KB table, entry (b, l) at byte 128 b + 4 (l % 32): a copy per half-wavefront
// lane, so a 64 KB TurboQuant value table and this one leave room for two workgroups per CU.
// The table is 16 KB-aligned, so the address is one shift-or of the code byte into ktab.
constexpr int kProdTabWords = 120 * 32;
template <int I>
__device__ inline uint32_t prod_pair(uint32_t ktab, uint32_t w) {
    const uint32_t b = (w >> (8 * I)) & 0xffu;
    return *(lds_u32 *)(size_t)(ktab | (b << 7));
}
// 8 sign bits (byte j of w) -> 8 f16 operands -1 (bit set) / +1: with t = u | u << 15, pair k
// (bits 2k, 2k + 1 of u) sits at bits 15 and 31 of t << (15 - 2k), the f16 sign positions
__device__ inline f16x8 signs_f16x8(uint32_t w, int j) {
    const uint32_t u = (w >> (8 * j)) & 0xffu, t = u | (u << 15);
    u32x4 r;
    uint32_t *rp = (uint32_t *)&r;
#pragma unroll
    for (int k = 0; k < 4; ++k) rp[k] = ((t << (15 - 2 * k)) & 0x80008000u) | 0x3C003C00u;
    return __builtin_bit_cast(f16x8, r);
}

// TurboQuant codebook lookups: code byte b (codes b & 15, b >> 4) of lane l reads the f16 pair of
// entry (b, l) at byte 256 b + 4 l of a 64 KB LDS table, a copy per lane, so every lane reads
// its own bank (random codes through one shared 1 KB table cost several passes per read in bank
// conflicts). The table is 64 KB-aligned and tab = its address + 4 l, so the address of byte I
// of code word w is tab with w's byte I as byte 1: one byte permute.
template <int I>
__device__ inline uint32_t turbo_pair(uint32_t tab, uint32_t w) {
    // v_perm_b32 selector bytes: 0-3 pick bytes of the second operand (tab), 4-7 of the first (w)
    constexpr uint32_t sel = 0x03020000u | ((4u + I) << 8);
    return *(lds_u32 *)(size_t)__builtin_amdgcn_perm(w, tab, sel);
}

// 8 codes of one code word (4-bit) or two words (FP8) -> 8 operand values.
template <int FMT>
__device__ inline op_t<FMT> decode8(uint32_t w0, uint32_t w1, float scale, uint32_t tab) {
    u32x4 r;
    if constexpr (FMT == CQKV_FMT_FP8) {
        return fp8x8_to_bf16x8(w0, w1);
    } else if constexpr (FMT == CQKV_FMT_MXFP4) {
        r.x = fp4x2_to_bf16x2(w0, 0, scale);
        r.y = fp4x2_to_bf16x2(w0, 1, scale);
        r.z = fp4x2_to_bf16x2(w0, 2, scale);
        r.w = fp4x2_to_bf16x2(w0, 3, scale);
    } else if constexpr (compact_tab<FMT>()) {  // tab: the side's compact table
        r.x = prod_pair<0>(tab, w0);
        r.y = prod_pair<1>(tab, w0);
        r.z = prod_pair<2>(tab, w0);
        r.w = prod_pair<3>(tab, w0);
    } else {
        r.x = turbo_pair<0>(tab, w0);
        r.y = turbo_pair<1>(tab, w0);
        r.z = turbo_pair<2>(tab, w0);
        r.w = turbo_pair<3>(tab, w0);
    }
    return __builtin_bit_cast(op_t<FMT>, r);
}

__device__ inline float e8m0_scale(uint32_t code) {  // code 0 marks an all-zero block
    return code == 0 ? 0.0f : __uint_as_float(code << 23);
}

// NVFP4 key operand: 8 E2M1 codes of one word times the E4M3 block scale in byte `bi` of `cs`, in
// f16 (exact): one conversion per code pair, one packed f16 multiply.
__device__ inline f16x8 nvfp4x8_f16x8(uint32_t w, uint32_t cs, int bi) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    const uint32_t c2 = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(cs >> (8 * (bi & 2)), 1.0f, false));
    // the block's f16 scale in both halves (one byte permute)
    const h2 sc = __builtin_bit_cast(h2, __builtin_amdgcn_perm(c2, c2, (bi & 1) ? 0x03020302u : 0x01000100u));
    h2 r[4];
    r[0] = __builtin_bit_cast(h2, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 1.0f, 0)) * sc;
    r[1] = __builtin_bit_cast(h2, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 1.0f, 1)) * sc;
    r[2] = __builtin_bit_cast(h2, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 1.0f, 2)) * sc;
    r[3] = __builtin_bit_cast(h2, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 1.0f, 3)) * sc;
    return __builtin_bit_cast(f16x8, r);
}

// NVFP4 value operand: 8 E2M1 codes of 8 keys (one head dim), key pair i's codes times the f16
// pair cs[i] of their E4M3 block scales: exact in f16, one conversion and one packed multiply per
// pair. The reference's dequantized value is fl(fl(fp4 * cs) * gs) (RowCodec::elem times rsc0,
// turbo.rs:383-395); fp4 * cs is exact here and gs goes into P.
__device__ inline f16x8 nvfp4_codes_f16x8(uint32_t w, const uint32_t *cs) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    h2 r[4];
    r[0] = __builtin_bit_cast(h2, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 1.0f, 0)) * __builtin_bit_cast(h2, cs[0]);
    r[1] = __builtin_bit_cast(h2, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 1.0f, 1)) * __builtin_bit_cast(h2, cs[1]);
    r[2] = __builtin_bit_cast(h2, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 1.0f, 2)) * __builtin_bit_cast(h2, cs[2]);
    r[3] = __builtin_bit_cast(h2, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 1.0f, 3)) * __builtin_bit_cast(h2, cs[3]);
    return __builtin_bit_cast(f16x8, r);
}

// QS: the queries carry a lo part (their own instantiation: no branch inside the key products)
template <int KF, int VF, int D, bool TERMS, bool QS>
__device__ inline void compute_tile(Tile<KF, VF, D> &cur, int tile, const DecodeArgs &a,
                                    const kop_t<KF> *qhi, const kop_t<KF> *qlo, int lane,
                                    int lo, int hi, int lo_max, int hi_min, int L, int koff,
                                    uint32_t tab, float &m_run, float &l_run,
                                    f32x4 *acc, const kop_t<KF> *qsop, uint32_t ktab,
                                    uint32_t vtab, float slope2, int qpos, float kscale2,
                                    int &e_run) {
    constexpr int NCH = D / 32;
    const int g = lane >> 4;
    // tile and L are rows of the current block (the whole cache when not paged); keys of the
    // call, for the masks, are koff further
    const int t0 = tile * 32;
    const bool full = koff + t0 >= lo_max && koff + t0 + 32 <= hi_min && t0 + 32 <= L;

    // S^T = K Q^T for the two 16-key sub-tiles (TurboProd: and Z (S q)^T, the QJL sign dots)
    f32x4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
    f32x4 z0 = {0.f, 0.f, 0.f, 0.f}, z1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
        kop_t<KF> k0, k1;
        if constexpr (KF == CQKV_FMT_FP8) {
            // bf16(scale * code): the reference's bf16 cache values (its CPU path, within whose
            // 2e-2 the outputs must stay; the fused kernel's f32 products scaled after the dot
            // move outputs of |x| >= 4 by more than the bf16 ulp leaves)
            k0 = fp8x8_scaled_bf16x8(cur.k[0][2 * j], cur.k[0][2 * j + 1], __uint_as_float(cur.kscale[0]));
            k1 = fp8x8_scaled_bf16x8(cur.k[1][2 * j], cur.k[1][2 * j + 1], __uint_as_float(cur.kscale[1]));
        } else if constexpr (KF == CQKV_FMT_MXFP8) {
            // chunk j holds head dims 64 (j >> 1) + 16 g + 8 (j & 1) + e: block 2 (j >> 1) + g / 2;
            // code times the E8M0 power of two is exact in bf16, one conversion per pair
            const int bi = 2 * (j >> 1) + (g >> 1);
            const uint32_t w0 = bi < 4 ? cur.kscale[0] : cur.kscale2[0];
            const uint32_t w1 = bi < 4 ? cur.kscale[1] : cur.kscale2[1];
            const float sc0 = e8m0_scale((w0 >> (8 * (bi & 3))) & 0xffu);
            const float sc1 = e8m0_scale((w1 >> (8 * (bi & 3))) & 0xffu);
            k0 = fp8x8_pow2_bf16x8(cur.k[0][2 * j], cur.k[0][2 * j + 1], sc0);
            k1 = fp8x8_pow2_bf16x8(cur.k[1][2 * j], cur.k[1][2 * j + 1], sc1);
        } else if constexpr (KF == CQKV_FMT_NVFP4) {
            // chunk j holds head dims (D/4) g + 8 j + e: the lane's block byte j / 2 (D >= 128);
            // code times block scale in f16 (exact), the token scale goes on the score
            const int bi = D >= 128 ? (j >> 1) : 0;
            k0 = nvfp4x8_f16x8(cur.k[0][j], cur.kscale[0], bi);
            k1 = nvfp4x8_f16x8(cur.k[1][j], cur.kscale[1], bi);
        } else {
            float sc0 = 1.0f, sc1 = 1.0f;
            if constexpr (KF == CQKV_FMT_MXFP4) {
                // D = 256: chunk j holds head dims 64 g + 8 j + e, block byte j / 4 of the two
                const uint32_t b0 = D == 256 ? (cur.kscale[0] >> (8 * (j >> 2))) & 0xffu : cur.kscale[0];
                const uint32_t b1 = D == 256 ? (cur.kscale[1] >> (8 * (j >> 2))) & 0xffu : cur.kscale[1];
                sc0 = b0 ? __uint_as_float(b0 << 23) : 1.0f;
                sc1 = b1 ? __uint_as_float(b1 << 23) : 1.0f;
            }
            if constexpr (compact_tab<KF>()) {
                k0 = __builtin_bit_cast(op_t<KF>, u32x4{prod_pair<0>(ktab, cur.k[0][j]),
                                                        prod_pair<1>(ktab, cur.k[0][j]),
                                                        prod_pair<2>(ktab, cur.k[0][j]),
                                                        prod_pair<3>(ktab, cur.k[0][j])});
                k1 = __builtin_bit_cast(op_t<KF>, u32x4{prod_pair<0>(ktab, cur.k[1][j]),
                                                        prod_pair<1>(ktab, cur.k[1][j]),
                                                        prod_pair<2>(ktab, cur.k[1][j]),
                                                        prod_pair<3>(ktab, cur.k[1][j])});
            } else {
                k0 = decode8<KF>(cur.k[0][j], 0, sc0, tab);
                k1 = decode8<KF>(cur.k[1][j], 0, sc1, tab);
            }
        }
        s0 = mfma16x16x32(k0, qhi[j], s0);
        s1 = mfma16x16x32(k1, qhi[j], s1);
        if constexpr (is_prod<KF>()) {  // byte j of the lane key's sign bits
            const uint32_t sw0 = j < 4 ? cur.ksg[0] : cur.ksg2[0];
            const uint32_t sw1 = j < 4 ? cur.ksg[1] : cur.ksg2[1];
            z0 = mfma16x16x32(signs_f16x8(sw0, j & 3), qsop[j], z0);
            z1 = mfma16x16x32(signs_f16x8(sw1, j & 3), qsop[j], z1);
        }
        if constexpr (QS) {
            s0 = mfma16x16x32(k0, qlo[j], s0);
            s1 = mfma16x16x32(k1, qlo[j], s1);
        }
    }
    float x[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
    const int kbase = t0 + 8 * g;  // x[e] is key kbase + e
    if constexpr (is_prod<KF>()) {
        // r0 (q . c + r1 sqrt(pi / 2) / D (S q) . z) (turbo_quant_impl.h:268-276); zk holds
        // -(S q) . z (the operands are -1 where the sign bit is set)
        const float zk[8] = {z0.x, z0.y, z0.z, z0.w, z1.x, z1.y, z1.z, z1.w};
        const float kc = a.qjl_c;  // -sqrt(pi / 2) / d
#pragma unroll
        for (int e = 0; e < 8; ++e)
            x[e] = (x[e] + __uint_as_float(cur.kr1[e]) * kc * zk[e]) *
                   __uint_as_float(cur.ks8[e]) * kscale2;
    } else if constexpr (!row_scaled_keys<KF>()) {  // scales are inside the operands
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] *= kscale2;
    } else {  // the key's row scale times the dot (TurboQuant norm)
#pragma unroll
        for (int e = 0; e < 8; ++e)
            x[e] = x[e] * __uint_as_float(cur.ks8[e]) * kscale2;
    }
    if constexpr (TERMS) {  // soft-capping, then ALiBi (tq_logit, turbo_quant_impl.h:37-41)
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] = fa_logit2(x[e], a.cap2, slope2, qpos - (koff + kbase + e));
    }
    if (!full) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int key = koff + kbase + e;  // rows past the block's valid rows are masked too
            if (!(key >= lo && key < hi && kbase + e < L)) x[e] = -__builtin_inff();
        }
    }
    float mx = x[0];
#pragma unroll
    for (int e = 1; e < 8; ++e) mx = fmaxf(mx, x[e]);
    mx = group16_max(mx);
    const float m_new = fmaxf(m_run, mx);
    const bool none = m_new == -__builtin_inff();
    const float alpha = none ? 1.0f : __builtin_amdgcn_exp2f(m_run - m_new);
    float alpha_o = alpha;  // O's factor (NVFP4 values: times 2^(old e_run - new e_run))
    // keys past the written length may hold any bytes: keep them out of PV
    const int nv = min(max(L - kbase, 0), 8);
    float gsw[8];  // NVFP4 values: the keys' f32 token scales times 2^(14 - e_run)
    if constexpr (VF == CQKV_FMT_NVFP4) {
        if (t0 + 32 > L) {  // uniform: only the tile holding the end of the keys
#pragma unroll
            for (int e = 0; e < 8; ++e)
                if (e >= nv) {
                    cur.nvg[e] = 0u;
#pragma unroll
                    for (int i = 0; i < D / 64; ++i) cur.nvb[(D / 64) * e + i] = 0u;
                }
        }
        // O is accumulated in units of 2^(e_run - 14), with e_run the largest binary exponent of
        // the token scales seen so far (uniform: every lane group reads 8 of the tile's 32 keys),
        // so the f16 operand P * g * 2^(14 - e_run) stays below 2^14 and products down to 2^-28 of
        // the largest remain normal f16 numbers; a larger exponent rescales O exactly.
        float gm = __uint_as_float(cur.nvg[0]);
#pragma unroll
        for (int e = 1; e < 8; ++e) gm = fmaxf(gm, __uint_as_float(cur.nvg[e]));
        gm = group16_max(gm);
        const int e_new = gm > 0.0f ? max(e_run, __builtin_amdgcn_frexp_expf(gm)) : e_run;
        if (e_new != e_run) {
            alpha_o = __builtin_ldexpf(alpha, e_run - e_new);
            e_run = e_new;
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) gsw[e] = __builtin_ldexpf(__uint_as_float(cur.nvg[e]), 14 - e_run);
    }
    float p[8], psum = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        p[e] = none ? 0.0f : __builtin_amdgcn_exp2f(x[e] - m_new);
        psum += p[e];
    }
    l_run = l_run * alpha + psum;
    m_run = m_new;
    if (__any(alpha_o != 1.0f)) {
#pragma unroll
        for (int t = 0; t < 2 * NCH; ++t) acc[t] *= alpha_o;
    }
    if (t0 + 32 > L) {  // uniform: only the tile holding the end of the keys
#pragma unroll
        for (int u = 0; u < NCH; ++u) {
            if constexpr (is8<VF>()) {
                const uint64_t keep = nv == 0 ? 0ull : (~0ull >> (64 - 8 * nv));
                const uint64_t w0 = (((uint64_t)cur.v[u][1] << 32) | cur.v[u][0]) & keep;
                const uint64_t w1 = (((uint64_t)cur.v[u][3] << 32) | cur.v[u][2]) & keep;
                cur.v[u][0] = (uint32_t)w0;
                cur.v[u][1] = (uint32_t)(w0 >> 32);
                cur.v[u][2] = (uint32_t)w1;
                cur.v[u][3] = (uint32_t)(w1 >> 32);
            } else {
                const uint32_t keep = nv == 0 ? 0u : (~0u >> (32 - 4 * nv));
                cur.v[u][0] &= keep;
                cur.v[u][1] &= keep;
            }
        }
    }
    // O^T += V^T P^T: d-tile 2u + h, row r <-> head dim 32u + 2r + h
    if constexpr (VF == CQKV_FMT_NVFP4) {
        // V: E2M1 code times its E4M3 block scale, exact in f16 (at most 6 significant bits,
        // 2^-10 .. 2688); the key's f32 token scale goes into P, one f16 operand
        // p * g * 2^(14 - e_run) (11 significant bits), as TurboQuant's norm does. Keys past the
        // length have zero codes and scales.
        float pv[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) pv[e] = p[e] * gsw[e];
        const f16x8 pf = __builtin_bit_cast(
            f16x8, u32x4{pack_f16x2(pv[0], pv[1]), pack_f16x2(pv[2], pv[3]), pack_f16x2(pv[4], pv[5]),
                         pack_f16x2(pv[6], pv[7])});
#pragma unroll
        for (int u = 0; u < NCH; ++u) {
            // rows 32u + 2n + h lie in block bi = 2u + n / 8 of every key: byte bi % 4 of the key's
            // word bi / 4; the pair (keys 2i, 2i + 1) gathered into bytes 0-1 by one byte permute
            const int bi = 2 * u + ((lane & 15) >> 3);
            const uint32_t sel = (uint32_t)(bi & 3) | ((uint32_t)(4 + (bi & 3)) << 8) | 0x0c0c0000u;
            uint32_t cs[4];
#pragma unroll
            for (int i = 0; i < 4; ++i)
                cs[i] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(
                                                         __builtin_amdgcn_perm(cur.nvb[(D / 64) * (2 * i + 1) + (bi >> 2)],
                                                                               cur.nvb[(D / 64) * (2 * i) + (bi >> 2)], sel),
                                                         1.0f, false));
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const f16x8 v = nvfp4_codes_f16x8(cur.v[u][h], cs);
                acc[2 * u + h] = mfma16x16x32(v, pf, acc[2 * u + h]);
            }
        }
    } else if constexpr (VF == CQKV_FMT_MXFP4) {
        // value block u: P scaled by the keys' block-u scales, one bf16 operand (the E2M1 codes
        // and E8M0 scales are exact; P rounds to 8 significant bits, as in a bf16 flash
        // attention). E8M0 code c is the scale 2^(c - 127). Each key pair's P is rounded to bf16
        // once, its exponent fields biased by -127; block u then adds the two keys' codes to the
        // exponent fields (a byte permute, a packed multiply-add and a packed clamp per pair and
        // block): the bits of rounding p * 2^(c - 127) wherever that is a normal bf16 number.
        // Results below the normal range clamp to zero. Masked keys (tiles across a range end)
        // take code 0, and p floored at 2^-100 then clamps to exactly zero; the floor keeps a p
        // that underflows in exp2 from meeting a large code, its operand then at most 2^-100 of
        // its value where the row's largest p is at least 1. A column with no visible key is
        // dropped by the rescale (alpha 0) or the epilogue (m -inf). Code 0 also marks an
        // all-zero block: its zero codes make any operand vanish. Above the bf16 range (p 2^(c -
        // 127) >= 2^128, blocks with |x| >= 2^122) the clamp gives zero too, where the
        // reference's dequantized f32 values already overflow to infinity.
        typedef uint16_t u16x2 __attribute__((ext_vector_type(2)));
        typedef short i16x2 __attribute__((ext_vector_type(2)));
        uint32_t vw[8], vw2[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            vw[e] = (uint32_t)__shfl((int)cur.vs, 8 * g + e);
            vw2[e] = D == 256 ? (uint32_t)__shfl((int)cur.vs2, 8 * g + e) : 0u;
        }
        if (t0 + 32 > L) {  // uniform: keys past the written length may hold any scale bytes
#pragma unroll
            for (int e = 0; e < 8; ++e)
                if (e >= nv) vw[e] = vw2[e] = 0u;
        }
        if (!full) {  // uniform: masked keys take code 0, so their operands clamp to exactly 0
#pragma unroll
            for (int e = 0; e < 8; ++e)
                if (x[e] == -__builtin_inff()) vw[e] = vw2[e] = 0u;
        }
        u16x2 pb[4];  // bf16 P of keys 2i, 2i + 1, exponent fields minus 127
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            // (the word made opaque: otherwise the compiler splits the pair conversion in two)
            uint32_t w = pack_bf16x2(fmaxf(p[2 * i], 0x1p-100f), fmaxf(p[2 * i + 1], 0x1p-100f));
            asm volatile("" : "+v"(w));
            pb[i] = __builtin_bit_cast(u16x2, w) - u16x2{0x3f80, 0x3f80};
        }
        const uint32_t k128 = 0x00800080u;  // 128 in both halves: c << 7 by the multiply-add
#pragma unroll
        for (int u = 0; u < NCH; ++u) {
            u32x4 pw;
            uint32_t *pwp = (uint32_t *)&pw;
            // byte u % 4 of the even key's word into byte 0, of the odd key's into byte 2
            const uint32_t sel = (uint32_t)(u & 3) | 0x0c00u | ((uint32_t)(4 + (u & 3)) << 16) | 0x0c000000u;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t w0 = u < 4 ? vw[2 * i] : vw2[2 * i];
                const uint32_t w1 = u < 4 ? vw[2 * i + 1] : vw2[2 * i + 1];
                const uint32_t c = __builtin_amdgcn_perm(w1, w0, sel);
                uint32_t r;  // c * 128 + pb per half, one v_pk_mad_u16 (the compiler emits a shift and an add)
                asm("v_pk_mad_u16 %0, %1, %2, %3" : "=v"(r) : "v"(c), "v"(k128), "v"(pb[i]));
                pwp[i] = __builtin_bit_cast(uint32_t, __builtin_elementwise_max(__builtin_bit_cast(i16x2, r), i16x2{0, 0}));
            }
            const op_t<VF> pb = __builtin_bit_cast(op_t<VF>, pw);
            const op_t<VF> v0 = decode8<VF>(cur.v[u][0], 0, 1.0f, tab);
            const op_t<VF> v1 = decode8<VF>(cur.v[u][1], 0, 1.0f, tab);
            acc[2 * u] = mfma16x16x32(v0, pb, acc[2 * u]);
            acc[2 * u + 1] = mfma16x16x32(v1, pb, acc[2 * u + 1]);
        }
    } else {
        // FP8 / MXFP8: the value scales are inside the V operand (rounded to bf16 as the
        // reference's dequantized cache), P goes in full precision as a bf16 hi + lo pair.
        // TURBO4: the norm goes into P, which enters as one f16 operand (11 significant bits;
        // the lo part cost 8 more MFMAs per tile: config 5 246-254 -> 236 us same-box).
        float pv[8], sv[8];
        uint32_t vw[8], vw2[8];  // MX: the keys' block scale bytes (vw2: bytes 4-7 at D = 256)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            // scales past the written length may be any bits
            if constexpr (direct_scales<VF>())
                vw[e] = e < nv ? cur.vs8[e] : 0u;
            else
                vw[e] = e < nv ? (uint32_t)__shfl((int)cur.vs, 8 * g + e) : 0u;
            sv[e] = __uint_as_float(vw[e]);  // FP8 scale, TURBO4 norm
            if constexpr (VF == CQKV_FMT_MXFP8 && D == 256)
                vw2[e] = e < nv ? (uint32_t)__shfl((int)cur.vs2, 8 * g + e) : 0u;
            if constexpr (turbo_mse<VF>())
                pv[e] = (e < nv && p[e] > 0.0f) ? p[e] * sv[e] : 0.0f;
            else
                pv[e] = (e < nv && p[e] > 0.0f) ? p[e] : 0.0f;
        }
        op_t<VF> phi, plo;
        split8(pv, phi, plo);
#pragma unroll
        for (int u = 0; u < NCH; ++u) {
            op_t<VF> v0, v1;
            if constexpr (VF == CQKV_FMT_FP8) {
                v0 = fp8x8_scaled_bf16x8(cur.v[u][0], cur.v[u][1], sv);
                v1 = fp8x8_scaled_bf16x8(cur.v[u][2], cur.v[u][3], sv);
            } else if constexpr (VF == CQKV_FMT_MXFP8) {
                // rows 32u + 2r + h: block u of every key
                float su[8];
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    su[e] = e8m0_scale(((u < 4 ? vw[e] : vw2[e]) >> (8 * (u & 3))) & 0xffu);
                v0 = fp8x8_scaled_bf16x8(cur.v[u][0], cur.v[u][1], su);
                v1 = fp8x8_scaled_bf16x8(cur.v[u][2], cur.v[u][3], su);
            } else {
                v0 = decode8<VF>(cur.v[u][0], 0, 1.0f, compact_tab<VF>() ? vtab : tab);
                v1 = decode8<VF>(cur.v[u][1], 0, 1.0f, compact_tab<VF>() ? vtab : tab);
            }
            acc[2 * u] = mfma16x16x32(v0, phi, acc[2 * u]);
            acc[2 * u + 1] = mfma16x16x32(v1, phi, acc[2 * u + 1]);
            if constexpr (!turbo_mse<VF>()) {  // TurboMse: P (times the norms) as one f16
                acc[2 * u] = mfma16x16x32(v0, plo, acc[2 * u]);
                acc[2 * u + 1] = mfma16x16x32(v1, plo, acc[2 * u + 1]);
            }
        }
    }
}

// Wavefronts per SIMD the register allocation must leave room for with MXFP4 keys and values:
// 3 at D = 128 (168 VGPRs; at 176 only two fit and BASELINE config 3 runs 30 % slower), 4 at
// D = 64; other formats, and D = 256 (one wavefront per SIMD, VGPRs and AGPRs), take what the
// allocation gives.
template <int KF, int VF, int D>
constexpr int decode_min_waves() {
    return KF == CQKV_FMT_MXFP4 && VF == CQKV_FMT_MXFP4 && D < 256 ? (D == 128 ? 3 : 4) : 1;
}

template <int KF, int VF, int D, int WAVES, bool TERMS, bool QS>
__global__ __launch_bounds__(WAVES * 64)
__attribute__((amdgpu_waves_per_eu(decode_min_waves<KF, VF, D>()))) void decode_kernel(DecodeArgs a) {
    constexpr int NCH = D / 32;
    constexpr int NT = WAVES * 64;
    constexpr bool kTurbo =
        KF == CQKV_FMT_TURBO4 || KF == kFmtProd4 || VF == CQKV_FMT_TURBO4;  // the code table
    // the per-wavefront outputs (and, before the tile loop, the queries) share their LDS with the
    // TurboQuant code table (64 KB-aligned, see turbo_pair), which is live only during the tile
    // loop
    constexpr int kOWords = WAVES * 16 * D, kTabWords = kTurbo ? 256 * 64 : 0;
    __shared__ __attribute__((aligned(65536))) float sm_buf[kOWords > kTabWords ? kOWords : kTabWords];
    float(*sm_o)[16][D] = (float(*)[16][D])sm_buf;
    uint32_t *sm_tab = (uint32_t *)sm_buf;
    __shared__ float sm_m[WAVES][16], sm_l[WAVES][16];
    constexpr bool kProd = is_prod<KF>();
    // compact code-pair tables (120 code bytes x 32 lanes) of keys (TurboProd, kFmtTurboC) and of
    // kFmtTurboC values
    __shared__ __attribute__((aligned(16384))) uint32_t sm_ktab[compact_tab<KF>() ? kProdTabWords : 1];
    __shared__ __attribute__((aligned(16384))) uint32_t sm_vtab[compact_tab<VF>() ? kProdTabWords : 1];

    // 1-D grid, plane fastest: workgroup ids are dealt round-robin to the 8 XCDs, so with
    // kv_heads a multiple of 8 each XCD takes whole planes of one kv head from every sequence -
    // the same length mix everywhere (a split-fastest order would send split i of every plane to
    // one XCD, and in a ragged batch the high splits are mostly empty)
    const int planes = a.batch * a.kv_heads;
    const int rest = (int)blockIdx.x / planes, plane_id = (int)blockIdx.x % planes;
    const int split = rest / a.col_blocks, cb = rest % a.col_blocks;
    // this workgroup's columns: global columns c0col .. c0col + ncb - 1 (query c / group, head
    // c % group of the group)
    const int c0col = 16 * cb, ncb = min(16, a.ncols - c0col);
    const int hk = plane_id % a.kv_heads, b = plane_id / a.kv_heads;
    // the wavefront index is uniform: keep it scalar so the tile loop stays a scalar loop
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n = lane & 15, g = lane >> 4;
    const int L = a.kv_lens ? __builtin_amdgcn_readfirstlane(min(max(a.kv_lens[b], 0), a.kv_len))
                            : a.kv_len;

    // visible key range of this lane's column, and the workgroup-wide bounds
    const bool col_ok = n < ncb;
    int lo, hi, lo_min, hi_max, lo_max, hi_min;
    key_range(col_ok ? (c0col + n) / a.group : 0, a.q_len, L, a.wl, a.wr, lo, hi);
    // score terms of this lane's column: its ALiBi slope and its query's key position
    float slope2 = 0.0f;
    int qpos = 0;
    if constexpr (TERMS) {
        const int c = c0col + (col_ok ? n : 0);
        qpos = c / a.group + L - a.q_len;
        if (a.alibi && col_ok)
            slope2 = a.alibi[(int64_t)b * a.alibi_bs + hk * a.group + c % a.group] * kLog2e;
    }
    if (!col_ok) lo = hi = 0;
    key_range(c0col / a.group, a.q_len, L, a.wl, a.wr, lo_min, hi_min);
    key_range((c0col + ncb - 1) / a.group, a.q_len, L, a.wl, a.wr, lo_max, hi_max);
    // the split's tiles and the planes they live in: a segment of one block (paged) or a range of
    // the cache's tiles
    const uint8_t *kc = a.kc, *ks = a.ks, *vc = a.vc, *vs = a.vs;
    uint32_t kc_plane = a.kc_plane, ks_plane = a.ks_plane, vc_plane = a.vc_plane, vs_plane = a.vs_plane;
    int koff = 0, Lb = L, tb, te;
    if (a.segs) {
        const PagedSeg sg = a.segs[split];
        kc = sg.kc;
        ks = sg.ks;
        vc = sg.vc;
        vs = sg.vs;
        kc_plane = sg.kc_plane;
        ks_plane = sg.ks_plane;
        vc_plane = sg.vc_plane;
        vs_plane = sg.vs_plane;
        koff = sg.key_offset;
        Lb = sg.rows;
        tb = max(sg.tile_begin, max(lo_min - koff, 0) / 32);
        te = min(sg.tile_end, (max(hi_max - koff, 0) + 31) / 32);
    } else {
        tb = max(split * a.tiles_per_split, lo_min / 32);
        te = min((split + 1) * a.tiles_per_split, (hi_max + 31) / 32);
    }

    // ---- queries (rotated keys: q Pi_k^T = sign-flip, Hadamard, 1/sqrt(D)) ----
    float(*sm_q)[D] = sm_o[0];
    for (int idx = threadIdx.x; idx < 16 * D; idx += NT) {
        const int c = idx / D, d = idx % D;
        float v = 0.0f;
        if (c < ncb && d < a.head_dim) {
            const int head = hk * a.group + (c0col + c) % a.group, qi = (c0col + c) / a.group;
            v = load_elem(a.q, (int64_t)b * a.q_sb + (int64_t)head * a.q_sh + (int64_t)qi * a.q_si + d,
                          a.q_dtype);
        }
        sm_q[c][d] = v;
    }
    __syncthreads();
    if (a.rot_k) {
        for (int c = wave; c < ncb; c += WAVES) {
            if constexpr (D == 256) {
                float v[4] = {sm_q[c][2 * lane], sm_q[c][2 * lane + 1], sm_q[c][128 + 2 * lane],
                              sm_q[c][129 + 2 * lane]};
                const int j[4] = {2 * lane, 2 * lane + 1, 128 + 2 * lane, 129 + 2 * lane};
#pragma unroll
                for (int k = 0; k < 4; ++k)
                    if (sign_bit(a.ksign_bits, j[k])) v[k] = -v[k];
                fwht_quads_dec(v[0], v[1], v[2], v[3], lane);
#pragma unroll
                for (int k = 0; k < 4; ++k) sm_q[c][j[k]] = v[k] * a.rot_scale;
            } else {
                const bool act = lane < D / 2;
                float v0 = act ? sm_q[c][2 * lane] : 0.0f, v1 = act ? sm_q[c][2 * lane + 1] : 0.0f;
                if (act && sign_bit(a.ksign_bits, 2 * lane)) v0 = -v0;
                if (act && sign_bit(a.ksign_bits, 2 * lane + 1)) v1 = -v1;
                fwht_pairs_dec<D>(v0, v1, lane);
                if (act) {
                    sm_q[c][2 * lane] = v0 * a.rot_scale;
                    sm_q[c][2 * lane + 1] = v1 * a.rot_scale;
                }
            }
        }
        __syncthreads();
    }
    kop_t<KF> qhi[NCH], qlo[NCH], qsop[kProd ? NCH : 1];
    // the scores' factor: scale * log2(e), times 2^qe for queries scaled by 2^-qe into f16 range
    float kscale2 = a.scale_log2;
    int qe = 0;
    if constexpr (KF == CQKV_FMT_NVFP4) {
        // f16 queries: 2^-qe brings the largest |q| of the workgroup's columns below 2^15 (every
        // wavefront reads all of them, so each finds the same qe); exact scaling both ways
        float m = 0.0f;
        for (int i = lane; i < 16 * D; i += 64) m = fmaxf(m, __builtin_fabsf(sm_q[i / D][i % D]));
        m = wave_max(m);
        qe = m < 16384.0f ? 0 : max(__builtin_amdgcn_frexp_expf(m) - 14, 0);  // m < 2^(qe + 14)
        kscale2 = __builtin_ldexpf(a.scale_log2, qe);
    }
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
        float qv[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) qv[e] = sm_q[n][qdim<KF, D>(j, g, e)];
        if constexpr (KF == CQKV_FMT_NVFP4) {
#pragma unroll
            for (int e = 0; e < 8; ++e) qv[e] = __builtin_ldexpf(qv[e], -qe);
        }
        split8(qv, qhi[j], qlo[j]);
    }
    if constexpr (kProd) {
        // S q of the (rotated) queries on v_mfma_f32_16x16x4_f32: (S q)^T (D x 16) = S Q^T,
        // 16 outputs per wavefront step; k-step e of a group of four takes column
        // 16 kk + 4 g + e in lane group g (16-byte reads of S and of the queries)
        float(*sm_qs)[D] = sm_o[1];
        for (int bi = wave; bi < D / 16; bi += WAVES) {
            f32x4 acc2 = {0.f, 0.f, 0.f, 0.f};
            const float *srow = a.qjl + (int64_t)(16 * bi + n) * D + 4 * g;
#pragma unroll 4
            for (int kk = 0; kk < D / 16; ++kk) {
                const f32x4 sa = *(const f32x4 *)(srow + 16 * kk);
                const f32x4 qb = *(const f32x4 *)(&sm_q[n][16 * kk + 4 * g]);
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    acc2 = __builtin_amdgcn_mfma_f32_16x16x4f32(sa[e], qb[e], acc2, 0, 0, 0);
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) sm_qs[n][16 * bi + 4 * g + e] = acc2[e];
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < NCH; ++j) {
            float qv[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) qv[e] = sm_qs[n][qdim<KF, D>(j, g, e)];
            op_t<KF> lo_unused;
            split8(qv, qsop[j], lo_unused);
        }
    }
    if constexpr (compact_tab<KF>()) {
        for (int i = threadIdx.x; i < kProdTabWords; i += NT)
            sm_ktab[i] = pack_f16x2(a.kcent[(i >> 5) & 7], a.kcent[(i >> 9) & 7]);
    }
    if constexpr (compact_tab<VF>()) {
        for (int i = threadIdx.x; i < kProdTabWords; i += NT)
            sm_vtab[i] = pack_f16x2(a.vcent[(i >> 5) & 7], a.vcent[(i >> 9) & 7]);
    }
    __syncthreads();
    if constexpr (kTurbo) {  // entry (b, l) at word 64 b + l: code pair (b & 15, b >> 4)
        for (int i = threadIdx.x; i < 256 * 64; i += NT)
            sm_tab[i] = pack_f16x2(a.cent[(i >> 6) & 15], a.cent[i >> 10]);
        __syncthreads();
    }

    // ---- stream the tiles of this split ----
    const int64_t plane = (int64_t)b * a.kv_heads + hk;
    const rsrc_t kr = make_rsrc(kc + plane * kc_plane, kc_plane);
    const rsrc_t ksr = make_rsrc(ks + plane * ks_plane, ks_plane);
    const rsrc_t vr = make_rsrc(vc + plane * vc_plane, vc_plane);
    const rsrc_t vsr = make_rsrc(vs + plane * vs_plane, vs_plane);
    // NVFP4: the per-token f32 scales follow the block bytes of all the plane's tokens
    uint32_t ktok_off = 0, vtok_off = 0;
    if constexpr (KF == CQKV_FMT_NVFP4) ktok_off = ks_plane / (D / 16 + 4) * (D / 16);
    if constexpr (kProd) ktok_off = ks_plane / (8 + D / 8);  // load_tile reads the capacity here
    if constexpr (VF == CQKV_FMT_NVFP4) vtok_off = vs_plane / (D / 16 + 4) * (D / 16);

    f32x4 acc[2 * NCH];
#pragma unroll
    for (int t = 0; t < 2 * NCH; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    const uint32_t tab = (uint32_t)(size_t)sm_tab + 4 * lane;
    const uint32_t ktab = (uint32_t)(size_t)sm_ktab + 4 * (lane & 31);
    const uint32_t vtab = (uint32_t)(size_t)sm_vtab + 4 * (lane & 31);
    float m_run = -__builtin_inff(), l_run = 0.0f;
    // NVFP4 values: O in units of 2^(e_run - 14) (below any f32 exponent until a scale is seen)
    int e_run = -1024;

    // Register sets A and B alternate; the scheduling barriers keep every load of one set
    // issued before the next set's, so each wait only covers the set about to be used.
    Tile<KF, VF, D> ta, tb2;
    int t = tb + wave;
    load_tile<KF, VF, D>(ta, t, t < te, lane, kr, ksr, vr, vsr, ktok_off, vtok_off);
    __builtin_amdgcn_sched_barrier(0);
    load_tile<KF, VF, D>(tb2, t + WAVES, t + WAVES < te, lane, kr, ksr, vr, vsr, ktok_off, vtok_off);
    __builtin_amdgcn_sched_barrier(0);
    for (; t < te; t += 2 * WAVES) {
        compute_tile<KF, VF, D, TERMS, QS>(ta, t, a, qhi, qlo, lane, lo, hi, lo_max, hi_min, Lb,
                                       koff, tab, m_run, l_run, acc, kProd ? qsop : qhi, ktab, vtab,
                                       slope2, qpos, kscale2, e_run);
        __builtin_amdgcn_sched_barrier(0);
        load_tile<KF, VF, D>(ta, t + 2 * WAVES, t + 2 * WAVES < te, lane, kr, ksr, vr, vsr, ktok_off, vtok_off);
        __builtin_amdgcn_sched_barrier(0);
        if (t + WAVES < te)
            compute_tile<KF, VF, D, TERMS, QS>(tb2, t + WAVES, a, qhi, qlo, lane, lo, hi, lo_max,
                                           hi_min, Lb, koff, tab, m_run, l_run, acc,
                                           kProd ? qsop : qhi, ktab, vtab, slope2, qpos, kscale2, e_run);
        __builtin_amdgcn_sched_barrier(0);
        load_tile<KF, VF, D>(tb2, t + 3 * WAVES, t + 3 * WAVES < te, lane, kr, ksr, vr, vsr, ktok_off, vtok_off);
        __builtin_amdgcn_sched_barrier(0);
    }

    // ---- merge the wavefronts ----
    if constexpr (VF == CQKV_FMT_NVFP4) {
#pragma unroll
        for (int t = 0; t < 2 * NCH; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[t][i] = __builtin_ldexpf(acc[t][i], e_run - 14);
    }
    if constexpr (kTurbo) __syncthreads();  // every wavefront is done with the code table
    const float l_col = group16_sum(l_run);
#pragma unroll
    for (int u = 0; u < NCH; ++u)
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int i = 0; i < 4; ++i) sm_o[wave][n][32 * u + 8 * g + 2 * i + h] = acc[2 * u + h][i];
    if (g == 0) {
        sm_m[wave][n] = m_run;
        sm_l[wave][n] = l_col;
    }
    __syncthreads();
    const int rows = a.batch * a.q_heads * a.q_len;
    // rotated values always leave partials: the combine unrotates them (an unrotation here costs
    // the MXFP4 kernel three VGPRs and its third wavefront per SIMD)
    const bool single = a.splits == 1 && !a.partials;
    for (int idx = threadIdx.x; idx < ncb * D; idx += NT) {
        const int c = idx / D, d = idx % D;
        float M = -__builtin_inff();
#pragma unroll
        for (int w = 0; w < WAVES; ++w) M = fmaxf(M, sm_m[w][c]);
        float o = 0.0f, lse = -__builtin_inff();
        if (M != -__builtin_inff()) {
            float wsum = 0.0f, osum = 0.0f;
#pragma unroll
            for (int w = 0; w < WAVES; ++w) {
                const float f = __builtin_amdgcn_exp2f(sm_m[w][c] - M);
                wsum += sm_l[w][c] * f;
                osum += sm_o[w][c][d] * f;
            }
            o = osum / wsum;
            lse = M + __builtin_log2f(wsum);
        }
        const int head = hk * a.group + (c0col + c) % a.group, qi = (c0col + c) / a.group;
        if (d >= a.head_dim) continue;  // plane row padding
        if (!single) {  // the partial of this split; combine_kernel merges the splits
            const int64_t row = ((int64_t)b * a.q_heads + head) * a.q_len + qi;
            a.part_o[((int64_t)split * rows + row) * D + d] = o;
            if (d == 0) a.part_lse[(int64_t)split * rows + row] = lse;
        } else {
            store_elem(a.out, (int64_t)b * a.o_sb + (int64_t)head * a.o_sh + (int64_t)qi * a.o_si + d,
                       a.out_dtype, o);
        }
    }
}

// Wavefronts per workgroup: 8 when both formats have byte codes (HBM-bound: one workgroup per
// plane fills a CU), 4 when either is a 4-bit format (its decode is VALU-heavy; two or three
// independent workgroups per CU hide each other's latencies better than one of 8 wavefronts: 10 %
// faster on BASELINE config 3). Plane rows of 256 (d: the plane row length) take 4 wavefronts of
// one per SIMD: two tiles in flight need more than 256 registers.
constexpr int kWaves = 8;
constexpr int waves_of(int kf, int vf, int d = 128) {
    return d < 256 && (kf == CQKV_FMT_FP8 || kf == CQKV_FMT_MXFP8) &&
                   (vf == CQKV_FMT_FP8 || vf == CQKV_FMT_MXFP8)
               ? kWaves
               : 4;
}

// d: the plane row length (64, 128 or 256); terms: soft-capping or ALiBi (the TERMS kernels)
template <int KF, int VF, bool TERMS, bool QS>
inline void launch_decode_kvtq(int d, dim3 grid, hipStream_t st, const DecodeArgs &a) {
    constexpr int W = waves_of(KF, VF), W256 = waves_of(KF, VF, 256);
    if (d == 64)
        hipLaunchKernelGGL((decode_kernel<KF, VF, 64, W, TERMS, QS>), grid, dim3(W * 64), 0, st, a);
    else if (d == 128)
        hipLaunchKernelGGL((decode_kernel<KF, VF, 128, W, TERMS, QS>), grid, dim3(W * 64), 0, st, a);
    else
        hipLaunchKernelGGL((decode_kernel<KF, VF, 256, W256, TERMS, QS>), grid, dim3(W256 * 64), 0, st, a);
}
// Queries with a lo part (f32 or rotated queries over non-TurboQuant keys; TurboQuant keys take
// one f16 query operand) get their own kernels, so the common bf16-query kernels have no branch
// inside the key products.
template <int KF, int VF, bool TERMS>
inline void launch_decode_kvt(int d, dim3 grid, hipStream_t st, const DecodeArgs &a) {
    if constexpr (!turbo_mse<KF>() && !is_prod<KF>()) {
        if (a.q_split) {
            launch_decode_kvtq<KF, VF, TERMS, true>(d, grid, st, a);
            return;
        }
    }
    launch_decode_kvtq<KF, VF, TERMS, false>(d, grid, st, a);
}
template <int KF, int VF>
inline void launch_decode_kv(int d, dim3 grid, hipStream_t st, const DecodeArgs &a) {
    if (a.cap2 > 0.0f || a.alibi) launch_decode_kvt<KF, VF, true>(d, grid, st, a);
    else launch_decode_kvt<KF, VF, false>(d, grid, st, a);
}

// Launches the kernel of key format KF and value format vf; false (nothing launched) for a
// pairing that has no kernel.
template <int KF>
inline bool launch_decode_k(int vf, int d, dim3 grid, hipStream_t st, const DecodeArgs &a) {
    if constexpr (KF == kFmtTurboC) {  // compact keys come with TURBO4-table values only
        if (vf != CQKV_FMT_TURBO4) return false;
        launch_decode_kv<KF, CQKV_FMT_TURBO4>(d, grid, st, a);
    } else {
        switch (vf) {
        case CQKV_FMT_FP8: launch_decode_kv<KF, CQKV_FMT_FP8>(d, grid, st, a); break;
        case CQKV_FMT_MXFP4: launch_decode_kv<KF, CQKV_FMT_MXFP4>(d, grid, st, a); break;
        case CQKV_FMT_MXFP8: launch_decode_kv<KF, CQKV_FMT_MXFP8>(d, grid, st, a); break;
        case CQKV_FMT_NVFP4: launch_decode_kv<KF, CQKV_FMT_NVFP4>(d, grid, st, a); break;
        case kFmtTurboC:  // compact values come with 64 KB-table keys only
            if constexpr (KF == CQKV_FMT_TURBO4 || KF == kFmtProd4) {
                launch_decode_kv<KF, kFmtTurboC>(d, grid, st, a);
                break;
            } else {
                return false;
            }
        case CQKV_FMT_TURBO4: launch_decode_kv<KF, CQKV_FMT_TURBO4>(d, grid, st, a); break;
        default: return false;
        }
    }
    return true;
}

// Per-key-format launchers, defined in decode_inst.hip (one object per key format).
#define CQKV_DECODE_LAUNCHER(F) \
    bool decode_launch_k##F(int vf, int d, dim3 grid, hipStream_t st, const DecodeArgs &a);
CQKV_DECODE_LAUNCHER(0)
CQKV_DECODE_LAUNCHER(1)
CQKV_DECODE_LAUNCHER(2)
CQKV_DECODE_LAUNCHER(3)
CQKV_DECODE_LAUNCHER(4)
CQKV_DECODE_LAUNCHER(5)
CQKV_DECODE_LAUNCHER(6)
CQKV_DECODE_LAUNCHER(7)

}  // namespace cqkv
