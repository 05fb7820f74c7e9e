// Split-K flash-decode over the quantized cache, and the split combine (gfx950).
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
//    the GQA group (q_len * group <= 16); rows are keys (S^T = K Q^T) or head dims
//    (O^T = V^T P^T).
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
#include <algorithm>
#include <mutex>
#include <vector>

#include "cqkv_device.h"
#include "cqkv_host.h"

#include <type_traits>

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
    float scale_log2;  // softmax scale * log2(e)
    int32_t wl, wr;
    int32_t tiles_per_split, splits, batch;
    float *part_o;       // (splits, rows, D) f32, normalised partial outputs
    float *part_lse;     // (splits, rows) f32, log2-domain lse of each split
    void *out;
    int32_t out_dtype, q_split;  // q_split: queries need a lo part (not bf16 inputs)
    int64_t o_sb, o_sh, o_si;
    uint32_t ksign_bits[4], vsign_bits[4];  // TURBO4 rotation signs (bit set -> -1)
    float rot_scale;
    float cent[16];  // TURBO4 codebook (the same for keys and values at one head dim)
    const PagedSeg *segs;  // paged: one segment per split (the planes above are unused)
};

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

__device__ inline bool sign_bit(const uint32_t *bits, int j) { return (bits[j >> 5] >> (j & 31)) & 1u; }

// Byte codes (FP8, MXFP8) or nibbles (MXFP4, NVFP4, TURBO4).
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
template <int FMT, int D>
struct Tile {
    // keys: 2 sub-tiles x D/32 code words (byte codes: D/16 words, 4 per 16-key row chunk pair)
    uint32_t k[2][is8<FMT>() ? D / 16 : D / 32];
    // values: D/32 chunks of 2 head dims x 8 keys (byte codes 4 words, 4-bit 2 words)
    uint32_t v[D / 32][is8<FMT>() ? 4 : 2];
    // per sub-tile, this lane's key: FP8 f32 scale; MXFP4 its E8M0 block byte; MXFP8 all its
    // E8M0 block bytes; NVFP4 the E4M3 block bytes of its 32 (D=128) / 16 (D=64) head dims
    uint32_t kscale[2];
    uint32_t ktok[2];  // NVFP4: the key's f32 scale
    // key lane % 32 (broadcast across lanes): the MX formats' value block bytes
    uint32_t vs;
    // FP8 / TURBO4: the scale words of keys 8 g .. 8 g + 7 of the tile (lane group g), the ones the
    // lane's score and P rows need, read directly instead of broadcast across lanes
    uint32_t ks8[8], vs8[8];
    // NVFP4: the value block bytes (two words per key at D = 128, one at D = 64) and f32 scales
    // of keys 8 g .. 8 g + 7, read directly (config-2 shape 100-103 -> 99 us same-box)
    uint32_t nvb[D == 128 ? 16 : 8], nvg[8];
};

// Formats whose per-key scale words are read as ks8 / vs8 (one 32-bit word per key). Same-box
// A/B against the cross-lane broadcast: TurboQuant-4 config 5 270-276 -> 257-264 us, FP8 config 2
// 94.7-95.9 -> 94.3-94.6 us; MXFP4 config 3 got 2 % slower and keeps the broadcast.
template <int FMT>
constexpr bool direct_scales() {
    return FMT == CQKV_FMT_FP8 || FMT == CQKV_FMT_TURBO4;
}

// The 32-bit scale words of keys kb .. kb + 7 (kb a multiple of 8: two aligned 16-byte loads).
template <int BYTES>
__device__ inline void load_scales8(uint32_t *out, rsrc_t r, uint32_t kb, uint32_t oob) {
    static_assert(BYTES == 4, "32-bit scale words");
    const u32x4 a = ld128(r, (kb * 4) | oob), b = ld128(r, (kb * 4 + 16) | oob);
    out[0] = a.x; out[1] = a.y; out[2] = a.z; out[3] = a.w;
    out[4] = b.x; out[5] = b.y; out[6] = b.z; out[7] = b.w;
}

template <int FMT, int D>
__device__ inline void load_tile(Tile<FMT, D> &r, int tile, bool live, int lane, rsrc_t kr,
                                 rsrc_t ksr, rsrc_t vr, rsrc_t vsr, uint32_t ktok_off,
                                 uint32_t vtok_off) {
    const int n = lane & 15, g = lane >> 4;
    const uint32_t t0 = (uint32_t)tile * 32u;
    const uint32_t oob = live ? 0u : kOOB;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
        const uint32_t key = t0 + 8 * (n >> 2) + 4 * s + (n & 3);
        if constexpr (is8<FMT>()) {
#pragma unroll
            for (int i = 0; i < D / 64; ++i) {
                const u32x4 w = ld128_stream(kr, (key * D + 16 * g + 64 * i) | oob);
                r.k[s][4 * i + 0] = w.x;
                r.k[s][4 * i + 1] = w.y;
                r.k[s][4 * i + 2] = w.z;
                r.k[s][4 * i + 3] = w.w;
            }
            if constexpr (FMT == CQKV_FMT_FP8)
                r.kscale[s] = ld32(ksr, (key * 4) | oob);
            else if constexpr (D == 128)
                r.kscale[s] = ld32(ksr, (key * 4) | oob);
            else
                r.kscale[s] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(ksr, (key * 2) | oob, 0, 0);
        } else {
            if constexpr (D == 128) {
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
            if constexpr (FMT == CQKV_FMT_MXFP4)
                r.kscale[s] = __builtin_amdgcn_raw_buffer_load_b8(
                    ksr, (key * (D / 32) + (D == 128 ? g : g >> 1)) | oob, 0, 0);
            if constexpr (FMT == CQKV_FMT_NVFP4) {
                if constexpr (D == 128)
                    r.kscale[s] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(
                        ksr, (key * 8 + 2 * g) | oob, 0, 0);
                else
                    r.kscale[s] = __builtin_amdgcn_raw_buffer_load_b8(ksr, (key * 4 + g) | oob, 0, 0);
                r.ktok[s] = ld32(ksr, (ktok_off + key * 4) | oob);
            }
        }
    }
#pragma unroll
    for (int u = 0; u < D / 32; ++u) {
        if constexpr (is8<FMT>()) {
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
    if constexpr (direct_scales<FMT>()) {
        const uint32_t kb = t0 + 8 * g;
        load_scales8<4>(r.vs8, vsr, kb, oob);
        if constexpr (FMT == CQKV_FMT_TURBO4) load_scales8<4>(r.ks8, ksr, kb, oob);
    } else if constexpr (FMT == CQKV_FMT_MXFP4 || FMT == CQKV_FMT_MXFP8) {
        r.vs = D == 128 ? ld32(vsr, (kl * 4) | oob)
                        : (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(vsr, (kl * 2) | oob, 0, 0);
    } else if constexpr (FMT == CQKV_FMT_NVFP4) {
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
using op_t = typename std::conditional<FMT == CQKV_FMT_TURBO4, f16x8, bf16x8>::type;

// TurboQuant codebook lookups: code byte b (codes b & 15, b >> 4) of lane l reads the f16 pair of
// entry (b, l) at byte 256 b + 4 l of a 64 KB LDS table, a copy per lane, so every lane reads
// its own bank (random codes through one shared 1 KB table cost several passes per read in bank
// conflicts). The table is 64 KB-aligned and tab = its address + 4 l, so the address of byte I
// of code word w is tab with w's byte I as byte 1: one byte permute.
typedef __attribute__((address_space(3))) const uint32_t lds_u32;
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

// NVFP4: 8 E2M1 codes of one word times the scale sg = fl(cs * gs) of their (token, block):
// the E4M3 block scale cs times the token's f32 scale gs, rounded once per block, then one
// multiply per element before the bf16 rounding. The reference's dequantized cache rounds
// fl(fl(fp4 * cs) * gs) instead (RowCodec::elem times rsc0, turbo.rs:383-395): the two agree
// except where the f32 values straddle a bf16 rounding boundary (one bf16 ulp, rarely). The codes
// are converted unscaled: the conversion's own scale operand is meant for the E8M0 powers of
// two of the MX formats, not for E4M3 values.
__device__ inline bf16x8 nvfp4x8_bf16x8(uint32_t w, float sg) {
    u32x4 r;
    uint32_t *rp = (uint32_t *)&r;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        f32x2 f;
        switch (i) {  // the selector must be an immediate
        case 0: f = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 0); break;
        case 1: f = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 1); break;
        case 2: f = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 2); break;
        default: f = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 3); break;
        }
        rp[i] = pack_bf16x2(f.x * sg, f.y * sg);
    }
    return __builtin_bit_cast(bf16x8, r);
}

// The same for 8 codes of 8 keys, key e scaled by sg[e].
__device__ inline bf16x8 nvfp4x8_keys_bf16x8(uint32_t w, const float *sg) {
    u32x4 r;
    uint32_t *rp = (uint32_t *)&r;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        f32x2 f;
        switch (i) {
        case 0: f = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 0); break;
        case 1: f = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 1); break;
        case 2: f = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 2); break;
        default: f = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 3); break;
        }
        rp[i] = pack_bf16x2(f.x * sg[2 * i], f.y * sg[2 * i + 1]);
    }
    return __builtin_bit_cast(bf16x8, r);
}

template <int FMT, int D>
__device__ inline void compute_tile(Tile<FMT, D> &cur, int tile, const DecodeArgs &a,
                                    const op_t<FMT> *qhi, const op_t<FMT> *qlo, bool q_split, int lane,
                                    int lo, int hi, int lo_max, int hi_min, int L, int koff,
                                    uint32_t tab, float &m_run, float &l_run,
                                    f32x4 *acc) {
    constexpr int NCH = D / 32;
    const int g = lane >> 4;
    // tile and L are rows of the current block (the whole cache when not paged); keys of the
    // call, for the masks, are koff further
    const int t0 = tile * 32;
    const bool full = koff + t0 >= lo_max && koff + t0 + 32 <= hi_min && t0 + 32 <= L;

    // S^T = K Q^T for the two 16-key sub-tiles
    f32x4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
        op_t<FMT> k0, k1;
        if constexpr (FMT == CQKV_FMT_FP8) {
            k0 = fp8x8_scaled_bf16x8(cur.k[0][2 * j], cur.k[0][2 * j + 1], __uint_as_float(cur.kscale[0]));
            k1 = fp8x8_scaled_bf16x8(cur.k[1][2 * j], cur.k[1][2 * j + 1], __uint_as_float(cur.kscale[1]));
        } else if constexpr (FMT == CQKV_FMT_MXFP8) {
            // chunk j holds head dims 64 (j >> 1) + 16 g + 8 (j & 1) + e: block 2 (j >> 1) + g / 2
            const int bi = 2 * (j >> 1) + (g >> 1);
            const float sc0 = e8m0_scale((cur.kscale[0] >> (8 * bi)) & 0xffu);
            const float sc1 = e8m0_scale((cur.kscale[1] >> (8 * bi)) & 0xffu);
            k0 = fp8x8_scaled_bf16x8(cur.k[0][2 * j], cur.k[0][2 * j + 1], sc0);
            k1 = fp8x8_scaled_bf16x8(cur.k[1][2 * j], cur.k[1][2 * j + 1], sc1);
        } else if constexpr (FMT == CQKV_FMT_NVFP4) {
            // chunk j holds head dims (D/4) g + 8 j + e: the lane's block byte j / 2 (D = 128)
            const int bi = D == 128 ? (j >> 1) : 0;
            const float sg0 = __builtin_amdgcn_cvt_f32_fp8(cur.kscale[0] >> (8 * bi), 0) *
                              __uint_as_float(cur.ktok[0]);
            const float sg1 = __builtin_amdgcn_cvt_f32_fp8(cur.kscale[1] >> (8 * bi), 0) *
                              __uint_as_float(cur.ktok[1]);
            k0 = nvfp4x8_bf16x8(cur.k[0][j], sg0);
            k1 = nvfp4x8_bf16x8(cur.k[1][j], sg1);
        } else {
            float sc0 = 1.0f, sc1 = 1.0f;
            if constexpr (FMT == CQKV_FMT_MXFP4) {
                sc0 = cur.kscale[0] ? __uint_as_float(cur.kscale[0] << 23) : 1.0f;
                sc1 = cur.kscale[1] ? __uint_as_float(cur.kscale[1] << 23) : 1.0f;
            }
            k0 = decode8<FMT>(cur.k[0][j], 0, sc0, tab);
            k1 = decode8<FMT>(cur.k[1][j], 0, sc1, tab);
        }
        s0 = mfma16x16x32(k0, qhi[j], s0);
        s1 = mfma16x16x32(k1, qhi[j], s1);
        if (q_split) {
            s0 = mfma16x16x32(k0, qlo[j], s0);
            s1 = mfma16x16x32(k1, qlo[j], s1);
        }
    }
    float x[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
    const int kbase = t0 + 8 * g;  // x[e] is key kbase + e
    if constexpr (FMT != CQKV_FMT_TURBO4) {  // scales are inside the operands
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] *= a.scale_log2;
    } else {
#pragma unroll
        for (int e = 0; e < 8; ++e)
            x[e] = x[e] * __uint_as_float(cur.ks8[e]) * a.scale_log2;
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
    float p[8], psum = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        p[e] = none ? 0.0f : __builtin_amdgcn_exp2f(x[e] - m_new);
        psum += p[e];
    }
    l_run = l_run * alpha + psum;
    m_run = m_new;
    if (__any(alpha != 1.0f)) {
#pragma unroll
        for (int t = 0; t < 2 * NCH; ++t) acc[t] *= alpha;
    }
    // keys past the written length may hold any bytes: keep them out of PV
    const int nv = min(max(L - kbase, 0), 8);
    if (t0 + 32 > L) {  // uniform: only the tile holding the end of the keys
#pragma unroll
        for (int u = 0; u < NCH; ++u) {
            if constexpr (is8<FMT>()) {
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
    if constexpr (FMT == CQKV_FMT_MXFP4) {
        // value block u: P scaled by the keys' block-u scales, one bf16 operand (the E2M1 codes
        // and E8M0 scales are exact; P rounds to 8 significant bits, as in a bf16 flash
        // attention). The scale of E8M0 code c is the float with exponent field c (code 0: 0).
        uint32_t vw[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) vw[e] = (uint32_t)__shfl((int)cur.vs, 8 * g + e);
        if (t0 + 32 > L) {  // uniform: keys past the written length may hold any scale bytes
#pragma unroll
            for (int e = 0; e < 8; ++e)
                if (e >= nv) vw[e] = 0u;
        }
#pragma unroll
        for (int u = 0; u < NCH; ++u) {
            u32x4 pw;
            uint32_t *pwp = (uint32_t *)&pw;
#pragma unroll
            for (int e = 0; e < 8; e += 2) {
                const float s0 = __uint_as_float(((vw[e] >> (8 * u)) & 0xffu) << 23);
                const float s1 = __uint_as_float(((vw[e + 1] >> (8 * u)) & 0xffu) << 23);
                pwp[e / 2] = pack_bf16x2(p[e] * s0, p[e + 1] * s1);
            }
            const op_t<FMT> pb = __builtin_bit_cast(op_t<FMT>, pw);
            const op_t<FMT> v0 = decode8<FMT>(cur.v[u][0], 0, 1.0f, tab);
            const op_t<FMT> v1 = decode8<FMT>(cur.v[u][1], 0, 1.0f, tab);
            acc[2 * u] = mfma16x16x32(v0, pb, acc[2 * u]);
            acc[2 * u + 1] = mfma16x16x32(v1, pb, acc[2 * u + 1]);
        }
    } else {
        // FP8 / MXFP8 / NVFP4: the value scales are inside the V operand (rounded to bf16 as the
        // reference's dequantized cache), P goes in full precision as a bf16 hi + lo pair.
        // TURBO4: the norm goes into P, which enters as one f16 operand (11 significant bits;
        // the lo part cost 8 more MFMAs per tile: config 5 246-254 -> 236 us same-box).
        float pv[8], sv[8];
        uint32_t vw[8], vw2[8];  // MX / NVFP4: the keys' block scale bytes
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            // scales past the written length may be any bits
            if constexpr (direct_scales<FMT>())
                vw[e] = e < nv ? cur.vs8[e] : 0u;
            else if constexpr (FMT == CQKV_FMT_NVFP4)
                vw[e] = e < nv ? cur.nvb[(D == 128 ? 2 : 1) * e] : 0u;
            else
                vw[e] = e < nv ? (uint32_t)__shfl((int)cur.vs, 8 * g + e) : 0u;
            sv[e] = __uint_as_float(vw[e]);  // FP8 scale, TURBO4 norm
            if constexpr (FMT == CQKV_FMT_NVFP4)
                vw2[e] = D == 128 && e < nv ? cur.nvb[2 * e + 1] : 0u;
            if constexpr (FMT == CQKV_FMT_TURBO4)
                pv[e] = (e < nv && p[e] > 0.0f) ? p[e] * sv[e] : 0.0f;
            else
                pv[e] = (e < nv && p[e] > 0.0f) ? p[e] : 0.0f;
        }
        float gk[8];  // NVFP4: the keys' f32 scales
        if constexpr (FMT == CQKV_FMT_NVFP4) {
#pragma unroll
            for (int e = 0; e < 8; ++e)
                gk[e] = e < nv ? __uint_as_float(cur.nvg[e]) : 0.0f;
        }
        op_t<FMT> phi, plo;
        split8(pv, phi, plo);
#pragma unroll
        for (int u = 0; u < NCH; ++u) {
            op_t<FMT> v0, v1;
            if constexpr (FMT == CQKV_FMT_FP8) {
                v0 = fp8x8_scaled_bf16x8(cur.v[u][0], cur.v[u][1], sv);
                v1 = fp8x8_scaled_bf16x8(cur.v[u][2], cur.v[u][3], sv);
            } else if constexpr (FMT == CQKV_FMT_MXFP8) {
                // rows 32u + 2r + h: block u of every key
                float su[8];
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    su[e] = e8m0_scale((vw[e] >> (8 * u)) & 0xffu);
                v0 = fp8x8_scaled_bf16x8(cur.v[u][0], cur.v[u][1], su);
                v1 = fp8x8_scaled_bf16x8(cur.v[u][2], cur.v[u][3], su);
            } else if constexpr (FMT == CQKV_FMT_NVFP4) {
                // this lane's rows 32u + 2n + h lie in block 2u + n / 8 of every key
                const int bi = 2 * u + ((lane & 15) >> 3);
                float sg[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const uint32_t w = bi < 4 ? vw[e] : vw2[e];
                    sg[e] = __builtin_amdgcn_cvt_f32_fp8(w >> (8 * (bi & 3)), 0) * gk[e];
                    if (e >= nv) sg[e] = 0.0f;
                }
                v0 = nvfp4x8_keys_bf16x8(cur.v[u][0], sg);
                v1 = nvfp4x8_keys_bf16x8(cur.v[u][1], sg);
            } else {
                v0 = decode8<FMT>(cur.v[u][0], 0, 1.0f, tab);
                v1 = decode8<FMT>(cur.v[u][1], 0, 1.0f, tab);
            }
            acc[2 * u] = mfma16x16x32(v0, phi, acc[2 * u]);
            acc[2 * u + 1] = mfma16x16x32(v1, phi, acc[2 * u + 1]);
            if constexpr (FMT != CQKV_FMT_TURBO4) {  // TURBO4: P (times the norms) as one f16
                acc[2 * u] = mfma16x16x32(v0, plo, acc[2 * u]);
                acc[2 * u + 1] = mfma16x16x32(v1, plo, acc[2 * u + 1]);
            }
        }
    }
}

template <int FMT, int D, int WAVES>
__global__ __launch_bounds__(WAVES * 64) void decode_kernel(DecodeArgs a) {
    constexpr int NCH = D / 32;
    constexpr int NT = WAVES * 64;
    constexpr bool kTurbo = FMT == CQKV_FMT_TURBO4;
    // the per-wavefront outputs (and, before the tile loop, the queries) share their LDS with the
    // TurboQuant code table (64 KB-aligned, see turbo_pair), which is live only during the tile
    // loop
    constexpr int kOWords = WAVES * 16 * D, kTabWords = kTurbo ? 256 * 64 : 0;
    __shared__ __attribute__((aligned(65536))) float sm_buf[kOWords > kTabWords ? kOWords : kTabWords];
    float(*sm_o)[16][D] = (float(*)[16][D])sm_buf;
    uint32_t *sm_tab = (uint32_t *)sm_buf;
    __shared__ float sm_fin[16][D];
    __shared__ float sm_m[WAVES][16], sm_l[WAVES][16];

    // 1-D grid, plane fastest: workgroup ids are dealt round-robin to the 8 XCDs, so with
    // kv_heads a multiple of 8 each XCD takes whole planes of one kv head from every sequence -
    // the same length mix everywhere (a split-fastest order would send split i of every plane to
    // one XCD, and in a ragged batch the high splits are mostly empty)
    const int planes = a.batch * a.kv_heads;
    const int split = (int)blockIdx.x / planes, plane_id = (int)blockIdx.x % planes;
    const int hk = plane_id % a.kv_heads, b = plane_id / a.kv_heads;
    // the wavefront index is uniform: keep it scalar so the tile loop stays a scalar loop
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n = lane & 15, g = lane >> 4;
    const int L = a.kv_lens ? __builtin_amdgcn_readfirstlane(min(max(a.kv_lens[b], 0), a.kv_len))
                            : a.kv_len;

    // visible key range of this lane's column, and the workgroup-wide bounds
    const bool col_ok = n < a.ncols;
    int lo, hi, lo_min, hi_max, lo_max, hi_min;
    key_range(col_ok ? n / a.group : 0, a.q_len, L, a.wl, a.wr, lo, hi);
    if (!col_ok) lo = hi = 0;
    key_range(0, a.q_len, L, a.wl, a.wr, lo_min, hi_min);
    key_range(a.q_len - 1, a.q_len, L, a.wl, a.wr, lo_max, hi_max);
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

    // ---- queries (TURBO4: rotated, q Pi_k^T = sign-flip, Hadamard, 1/sqrt(D)) ----
    float(*sm_q)[D] = sm_o[0];
    for (int idx = threadIdx.x; idx < 16 * D; idx += NT) {
        const int c = idx / D, d = idx % D;
        float v = 0.0f;
        if (c < a.ncols) {
            const int head = hk * a.group + c % a.group, qi = c / a.group;
            v = load_elem(a.q, (int64_t)b * a.q_sb + (int64_t)head * a.q_sh + (int64_t)qi * a.q_si + d,
                          a.q_dtype);
        }
        sm_q[c][d] = v;
    }
    __syncthreads();
    if constexpr (kTurbo) {
        for (int c = wave; c < a.ncols; c += WAVES) {
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
        __syncthreads();
    }
    op_t<FMT> qhi[NCH], qlo[NCH];
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
        float qv[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) qv[e] = sm_q[n][qdim<FMT, D>(j, g, e)];
        split8(qv, qhi[j], qlo[j]);
    }
    const bool q_split = a.q_split != 0;
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
    if constexpr (FMT == CQKV_FMT_NVFP4) {
        ktok_off = ks_plane / (D / 16 + 4) * (D / 16);
        vtok_off = vs_plane / (D / 16 + 4) * (D / 16);
    }

    f32x4 acc[2 * NCH];
#pragma unroll
    for (int t = 0; t < 2 * NCH; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    const uint32_t tab = (uint32_t)(size_t)sm_tab + 4 * lane;
    float m_run = -__builtin_inff(), l_run = 0.0f;

    // Register sets A and B alternate; the scheduling barriers keep every load of one set
    // issued before the next set's, so each wait only covers the set about to be used.
    Tile<FMT, D> ta, tb2;
    int t = tb + wave;
    load_tile<FMT, D>(ta, t, t < te, lane, kr, ksr, vr, vsr, ktok_off, vtok_off);
    __builtin_amdgcn_sched_barrier(0);
    load_tile<FMT, D>(tb2, t + WAVES, t + WAVES < te, lane, kr, ksr, vr, vsr, ktok_off, vtok_off);
    __builtin_amdgcn_sched_barrier(0);
    for (; t < te; t += 2 * WAVES) {
        compute_tile<FMT, D>(ta, t, a, qhi, qlo, q_split, lane, lo, hi, lo_max, hi_min, Lb, koff, tab,
                             m_run, l_run, acc);
        __builtin_amdgcn_sched_barrier(0);
        load_tile<FMT, D>(ta, t + 2 * WAVES, t + 2 * WAVES < te, lane, kr, ksr, vr, vsr, ktok_off, vtok_off);
        __builtin_amdgcn_sched_barrier(0);
        if (t + WAVES < te)
            compute_tile<FMT, D>(tb2, t + WAVES, a, qhi, qlo, q_split, lane, lo, hi, lo_max, hi_min,
                                 Lb, koff, tab, m_run, l_run, acc);
        __builtin_amdgcn_sched_barrier(0);
        load_tile<FMT, D>(tb2, t + 3 * WAVES, t + 3 * WAVES < te, lane, kr, ksr, vr, vsr, ktok_off, vtok_off);
        __builtin_amdgcn_sched_barrier(0);
    }

    // ---- merge the wavefronts ----
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
    const bool single = a.splits == 1;
    for (int idx = threadIdx.x; idx < a.ncols * D; idx += NT) {
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
        const int head = hk * a.group + c % a.group, qi = c / a.group;
        if (!single) {  // the partial of this split; combine_kernel merges the splits
            const int64_t row = ((int64_t)b * a.q_heads + head) * a.q_len + qi;
            a.part_o[((int64_t)split * rows + row) * D + d] = o;
            if (d == 0) a.part_lse[(int64_t)split * rows + row] = lse;
        } else if (kTurbo) {
            sm_fin[c][d] = o;
        } else {
            store_elem(a.out, (int64_t)b * a.o_sb + (int64_t)head * a.o_sh + (int64_t)qi * a.o_si + d,
                       a.out_dtype, o);
        }
    }
    if (!single || !kTurbo) return;
    __syncthreads();
    // ---- single split, TURBO4: unrotate with the value rotation, x = sign * H o / sqrt(D) ----
    for (int c = wave; c < a.ncols; c += WAVES) {
        const bool act = lane < D / 2;
        float v0 = act ? sm_fin[c][2 * lane] : 0.0f, v1 = act ? sm_fin[c][2 * lane + 1] : 0.0f;
        fwht_pairs_dec<D>(v0, v1, lane);
        v0 *= a.rot_scale;
        v1 *= a.rot_scale;
        if (act) {
            if (sign_bit(a.vsign_bits, 2 * lane)) v0 = -v0;
            if (sign_bit(a.vsign_bits, 2 * lane + 1)) v1 = -v1;
            const int head = hk * a.group + c % a.group, qi = c / a.group;
            const int64_t base =
                (int64_t)b * a.o_sb + (int64_t)head * a.o_sh + (int64_t)qi * a.o_si + 2 * lane;
            store_elem(a.out, base, a.out_dtype, v0);
            store_elem(a.out, base + 1, a.out_dtype, v1);
        }
    }
}

struct CombineArgs {
    const float *part_o, *part_lse;
    int32_t splits, rows, q_heads, q_len, out_dtype, rotate;
    void *out;
    int64_t o_sb, o_sh, o_si;
    uint32_t vsign_bits[4];
    float rot_scale;
};

// Split combine (the formula of tq_combine_impl, candle-core/kernels/turbo_quant_impl.h:659-685,
// in the log2 domain): o = sum_s w_s o_s / sum_s w_s, w_s = 2^(lse_s - max lse), empty splits
// skipped; then, for TurboQuant values, x = sign * (H o) / sqrt(D) (the unrotation y Pi).
// One wavefront per output row (lane l: head dims 2l, 2l+1), four rows per workgroup; the
// split loop keeps up to 8 splits' loads in flight.
template <int D>
__global__ __launch_bounds__(256) void combine_kernel(CombineArgs a) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= a.rows) return;
    const bool active = lane < D / 2;
    const float *lse = a.part_lse + row;
    float M = -__builtin_inff();
    for (int s = 0; s < a.splits; ++s) M = fmaxf(M, lse[(int64_t)s * a.rows]);
    float o0 = 0.0f, o1 = 0.0f;
    if (M != -__builtin_inff()) {
        float wsum = 0.0f, a0 = 0.0f, a1 = 0.0f;
        const float *po = a.part_o + (int64_t)row * D + 2 * (active ? lane : 0);
        const int64_t step = (int64_t)a.rows * D;
#pragma unroll 8
        for (int s = 0; s < a.splits; ++s) {
            const float e = lse[(int64_t)s * a.rows];
            const f32x2 v = *(const f32x2 *)(po + s * step);
            const float w = e == -__builtin_inff() ? 0.0f : __builtin_amdgcn_exp2f(e - M);
            wsum += w;
            a0 += w * v.x;
            a1 += w * v.y;
        }
        o0 = a0 / wsum;
        o1 = a1 / wsum;
    }
    if (a.rotate) {
        fwht_pairs_dec<D>(o0, o1, lane);
        o0 *= a.rot_scale;
        o1 *= a.rot_scale;
        if (active && sign_bit(a.vsign_bits, 2 * lane)) o0 = -o0;
        if (active && sign_bit(a.vsign_bits, 2 * lane + 1)) o1 = -o1;
    }
    if (!active) return;
    const int qi = row % a.q_len, head = (row / a.q_len) % a.q_heads;
    const int b = row / (a.q_len * a.q_heads);
    const int64_t base = (int64_t)b * a.o_sb + (int64_t)head * a.o_sh + (int64_t)qi * a.o_si + 2 * lane;
    store_elem(a.out, base, a.out_dtype, o0);
    store_elem(a.out, base + 1, a.out_dtype, o1);
}

int fill_turbo_args(const cqkv_side *s, uint32_t sign_bits[4], float *rot_scale, float bnd[16]);

static int tiles_of(int kv_len) { return (kv_len + 31) / 32; }

// Key splits per (batch, kv head). One 8-wavefront workgroup per plane fills a CU of the
// MI355X (256 CUs, two waves per SIMD at this register budget; twice as many workgroups of 4
// wavefronts): split only when there are fewer planes than that, and then into pieces of at
// least two tiles per wavefront. Ragged batches (per-sequence lengths) are split into pieces of
// at most 128 tiles (4096 keys) so long and short sequences even out across CUs.
constexpr int kWaves = 8;
constexpr int kCUs = 256;

static int auto_splits(int batch, int kv_heads, int kv_len, bool ragged, int waves = kWaves) {
    const int planes = batch * kv_heads;
    const int tiles = tiles_of(kv_len);
    const int wgs = kCUs * (kWaves / waves);  // workgroups that fill the chip
    int s = (wgs + planes - 1) / planes;
    if (ragged) s = max(s, (tiles + 127) / 128);
    s = min(s, max(1, tiles / (2 * waves)));
    s = max(1, min(s, 256));
    const int tps = (tiles + s - 1) / s;
    return max(1, (tiles + tps - 1) / tps);
}

// Wavefronts per workgroup: 8 for FP8 (HBM-bound: one workgroup per plane fills a CU), 4 for
// the 4-bit formats (their decode is VALU-heavy; two or three independent workgroups per CU
// hide each other's latencies better than one of 8 wavefronts: 10 % faster on BASELINE config 3).
constexpr int waves_of(int format) {
    return format == CQKV_FMT_FP8 || format == CQKV_FMT_MXFP8 ? kWaves : 4;
}

template <int FMT>
static void launch_decode(int d, dim3 grid, hipStream_t st, const DecodeArgs &a) {
    constexpr int W = waves_of(FMT);
    if (d == 64)
        hipLaunchKernelGGL((decode_kernel<FMT, 64, W>), grid, dim3(W * 64), 0, st, a);
    else
        hipLaunchKernelGGL((decode_kernel<FMT, 128, W>), grid, dim3(W * 64), 0, st, a);
}

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// Workspace: partial outputs (splits, rows, D) f32 | partial lse (splits, rows) f32.
static size_t workspace_layout(int32_t batch, int32_t q_heads, int32_t q_len, int32_t head_dim,
                               int32_t splits, size_t *lse_off) {
    const size_t rows = (size_t)batch * q_heads * q_len;
    *lse_off = align256((size_t)splits * rows * head_dim * 4);
    return *lse_off + align256((size_t)splits * rows * 4);
}

}  // namespace cqkv

using namespace cqkv;

extern "C" int32_t cqkv_decode_splits(int32_t format, int32_t batch, int32_t kv_heads,
                                      int32_t kv_len, int32_t ragged) {
    if (batch <= 0 || kv_heads <= 0 || kv_len <= 0) return 1;
    return auto_splits(batch, kv_heads, kv_len, ragged != 0, waves_of(format));
}

extern "C" size_t cqkv_decode_workspace_bytes(int32_t batch, int32_t q_heads, int32_t q_len,
                                              int32_t head_dim, int32_t splits) {
    if (batch <= 0 || q_heads <= 0 || q_len <= 0 || head_dim <= 0 || splits <= 0) return 0;
    size_t lse_off;
    return workspace_layout(batch, q_heads, q_len, head_dim, splits, &lse_off);
}

// Checks and fills what the dense and the paged calls share: queries, output, heads, scale,
// window, TurboQuant rotation and codebook. k / v give the format, head dim and kv heads.
static int decode_prepare(DecodeArgs &a, const char *who, const void *q, int32_t q_dtype,
                          const int64_t q_strides[3], const cqkv_side *k, const cqkv_side *v,
                          int32_t batch, int32_t q_heads, int32_t q_len, float softmax_scale,
                          int32_t window_left, int32_t window_right, void *out, int32_t out_dtype,
                          const int64_t out_strides[3]) {
    if (int rc = check_side(k, who)) return rc;
    if (int rc = check_side(v, who)) return rc;
    if (k->is_value != 0 || v->is_value != 1)
        return fail(CQKV_ERR_ARG, "%s: expected a key side and a value side", who);
    if (k->format != v->format || k->head_dim != v->head_dim || k->kv_heads != v->kv_heads)
        return fail(CQKV_ERR_ARG, "%s: key / value sides differ in format, D or heads", who);
    if (!q || !out || !q_strides || !out_strides)
        return fail(CQKV_ERR_ARG, "%s: null q / out / strides", who);
    if (q_dtype < CQKV_BF16 || q_dtype > CQKV_F32 || out_dtype < CQKV_BF16 || out_dtype > CQKV_F32)
        return fail(CQKV_ERR_ARG, "%s: dtypes q %d out %d", who, q_dtype, out_dtype);
    const int hkv = k->kv_heads, d = k->head_dim;
    if (batch <= 0 || q_heads <= 0 || q_len <= 0 || q_heads % hkv != 0)
        return fail(CQKV_ERR_ARG, "%s: batch %d q_heads %d q_len %d kv_heads %d", who, batch,
                    q_heads, q_len, hkv);
    const int group = q_heads / hkv;
    if (group * q_len > 16)
        return fail(CQKV_ERR_ARG, "%s: q_len * q_heads / kv_heads = %d > 16", who, group * q_len);
    a = DecodeArgs{};
    a.q = q;
    a.q_sb = q_strides[0];
    a.q_sh = q_strides[1];
    a.q_si = q_strides[2];
    a.q_dtype = q_dtype;
    a.q_heads = q_heads;
    a.kv_heads = hkv;
    a.group = group;
    a.q_len = q_len;
    a.ncols = group * q_len;
    a.scale_log2 = softmax_scale * kLog2e;
    a.wl = window_left;
    a.wr = window_right;
    a.batch = batch;
    a.out = out;
    a.out_dtype = out_dtype;
    // queries not representable in the operand type get a lo part (f16 / f32 inputs to the bf16
    // formats); TurboQuant's rotated queries enter as one f16 operand (2^-12 relative rounding:
    // config 5 216-225 -> 208-220 us same-box, its parity tests unchanged)
    a.q_split = q_dtype != CQKV_BF16 ? 1 : 0;
    a.o_sb = out_strides[0];
    a.o_sh = out_strides[1];
    a.o_si = out_strides[2];
    if (k->format == CQKV_FMT_TURBO4) {
        float bnd[16], cent[16];
        if (int rc = fill_turbo_args(k, a.ksign_bits, &a.rot_scale, bnd)) return rc;
        if (int rc = fill_turbo_args(v, a.vsign_bits, &a.rot_scale, bnd)) return rc;
        if (turbo_codebook(d, 4, cent, bnd) != 0)
            return fail(CQKV_ERR_ARG, "%s: turbo codebook D=%d", who, d);
        for (int i = 0; i < 16; ++i) a.cent[i] = cent[i];
    }
    return CQKV_OK;
}

// Launches the decode kernel over a.splits splits and, for more than one, the combine
// (partials at a.part_o / a.part_lse).
static hipError_t decode_launch(const DecodeArgs &a, int format, int d, hipStream_t st) {
    const dim3 grid(a.splits * a.kv_heads * a.batch);
    switch (format) {
    case CQKV_FMT_FP8: launch_decode<CQKV_FMT_FP8>(d, grid, st, a); break;
    case CQKV_FMT_MXFP4: launch_decode<CQKV_FMT_MXFP4>(d, grid, st, a); break;
    case CQKV_FMT_MXFP8: launch_decode<CQKV_FMT_MXFP8>(d, grid, st, a); break;
    case CQKV_FMT_NVFP4: launch_decode<CQKV_FMT_NVFP4>(d, grid, st, a); break;
    default: launch_decode<CQKV_FMT_TURBO4>(d, grid, st, a); break;
    }
    hipError_t e = hipGetLastError();
    if (e == hipSuccess && a.splits > 1) {
        CombineArgs c = {};
        c.part_o = a.part_o;
        c.part_lse = a.part_lse;
        c.splits = a.splits;
        c.rows = a.batch * a.q_heads * a.q_len;
        c.q_heads = a.q_heads;
        c.q_len = a.q_len;
        c.out_dtype = a.out_dtype;
        c.rotate = format == CQKV_FMT_TURBO4 ? 1 : 0;
        c.out = a.out;
        c.o_sb = a.o_sb;
        c.o_sh = a.o_sh;
        c.o_si = a.o_si;
        for (int i = 0; i < 4; ++i) c.vsign_bits[i] = a.vsign_bits[i];
        c.rot_scale = a.rot_scale;
        const dim3 cg((c.rows + 3) / 4);
        if (d == 64) hipLaunchKernelGGL(combine_kernel<64>, cg, dim3(256), 0, st, c);
        else hipLaunchKernelGGL(combine_kernel<128>, cg, dim3(256), 0, st, c);
        e = hipGetLastError();
    }
    return e;
}

// ---- allocation-free decode: split partials in a library-owned device array ----
// `scratch` is one array per GPU (each device that loads the library's code object holds its own
// copy at its own address), kept until the process ends. In host code its name is only a
// host-side stand-in: the device address comes from hipGetSymbolAddress, fetched once per device
// with that device current, and only that address is ever handed to kernels. Every
// cqkv_decode_attention_noalloc call on a GPU shares that GPU's array; calls that overlap on one
// GPU (concurrent streams) race on it.
static __device__ __attribute__((aligned(256))) uint8_t scratch[CQKV_DECODE_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static void *g_scratch_ptr[kMaxDevices];

static int scratch_address(void **out, const char *who) {
    int dev = -1;
    CQKV_HIP_CHECK(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxDevices)
        return fail(CQKV_ERR_ARG, "%s: device ordinal %d above %d", who, dev, kMaxDevices - 1);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return fail(CQKV_ERR_HIP, "%s: hipGetSymbolAddress(scratch) on device %d: %s", who,
                        dev, hipGetErrorString(e));
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return CQKV_OK;
}

// The dense decode of both entry points. noalloc: the partials go to the device `scratch` array
// (automatic splits are lowered until they fit; explicit ones that do not fit are refused);
// otherwise to `workspace`, or to a stream-ordered allocation when none is given.
static int decode_dense(const char *who, const void *q, int32_t q_dtype,
                        const int64_t q_strides[3], const cqkv_side *k, const cqkv_side *v,
                        int32_t batch, int32_t q_heads, int32_t q_len, const int32_t *kv_lens,
                        int32_t kv_len, float softmax_scale, int32_t window_left,
                        int32_t window_right, void *out, int32_t out_dtype,
                        const int64_t out_strides[3], int32_t splits, void *workspace,
                        size_t workspace_bytes, bool noalloc, cqkv_stream_t stream) {
    DecodeArgs a;
    if (int rc = decode_prepare(a, who, q, q_dtype, q_strides, k, v, batch, q_heads, q_len,
                                softmax_scale, window_left, window_right, out, out_dtype,
                                out_strides))
        return rc;
    if (k->capacity != v->capacity)
        return fail(CQKV_ERR_ARG, "%s: key / value capacities %d / %d differ", who, k->capacity,
                    v->capacity);
    if (kv_len < 0 || kv_len > k->capacity)
        return fail(CQKV_ERR_ARG, "%s: kv_len %d outside [0, capacity %d]", who, kv_len,
                    k->capacity);
    if (splits < 0) return fail(CQKV_ERR_ARG, "%s: splits %d", who, splits);
    const int hkv = k->kv_heads, d = k->head_dim;

    const int tiles = max(1, tiles_of(kv_len));
    int s = splits > 0 ? min(splits, tiles)
                       : auto_splits(batch, hkv, max(kv_len, 1), kv_lens != nullptr,
                                     waves_of(k->format));
    size_t lse_off = 0;
    if (noalloc) {
        if (s > 1 &&
            workspace_layout(batch, q_heads, q_len, d, s, &lse_off) > CQKV_DECODE_SCRATCH_BYTES) {
            if (splits > 0)
                return fail(CQKV_ERR_WORKSPACE,
                            "%s: %d splits need %zu bytes of partials, above the %zu-byte "
                            "device scratch",
                            who, s, workspace_layout(batch, q_heads, q_len, d, s, &lse_off),
                            (size_t)CQKV_DECODE_SCRATCH_BYTES);
            while (s > 1 && workspace_layout(batch, q_heads, q_len, d, s, &lse_off) >
                                CQKV_DECODE_SCRATCH_BYTES)
                --s;
        }
    }
    const int tps = (tiles + s - 1) / s;
    s = (tiles + tps - 1) / tps;

    a.kc = (const uint8_t *)k->codes;
    a.ks = (const uint8_t *)k->scales;
    a.vc = (const uint8_t *)v->codes;
    a.vs = (const uint8_t *)v->scales;
    a.kc_plane = (uint32_t)cqkv_codes_plane_bytes(k->format, d, k->capacity);
    a.ks_plane = (uint32_t)cqkv_scales_plane_bytes(k->format, d, k->capacity);
    a.vc_plane = (uint32_t)cqkv_codes_plane_bytes(v->format, d, v->capacity);
    a.vs_plane = (uint32_t)cqkv_scales_plane_bytes(v->format, d, v->capacity);
    a.kv_lens = kv_lens;
    a.kv_len = kv_len;
    a.tiles_per_split = tps;
    a.splits = s;

    hipStream_t st = (hipStream_t)stream;
    void *ws = workspace;
    bool owned = false;
    if (s > 1) {
        const size_t need = workspace_layout(batch, q_heads, q_len, d, s, &lse_off);
        if (noalloc) {
            if (int rc = scratch_address(&ws, who)) return rc;
        } else if (ws && workspace_bytes < need) {
            return fail(CQKV_ERR_WORKSPACE, "%s: workspace %zu < %zu bytes", who,
                        workspace_bytes, need);
        } else if (!ws) {
            CQKV_HIP_CHECK(hipMallocAsync(&ws, need, st));
            owned = true;
        }
        a.part_o = (float *)ws;
        a.part_lse = (float *)((char *)ws + lse_off);
    }
    hipError_t e = decode_launch(a, k->format, d, st);
    if (owned) {
        hipError_t fe = hipFreeAsync(ws, st);
        if (e == hipSuccess) e = fe;
    }
    if (e != hipSuccess) return fail(CQKV_ERR_HIP, "%s: launch failed: %s", who, hipGetErrorString(e));
    return CQKV_OK;
}

extern "C" int cqkv_decode_attention(const void *q, int32_t q_dtype, const int64_t q_strides[3],
                                     const cqkv_side *k, const cqkv_side *v, int32_t batch,
                                     int32_t q_heads, int32_t q_len, const int32_t *kv_lens,
                                     int32_t kv_len, float softmax_scale, int32_t window_left,
                                     int32_t window_right, void *out, int32_t out_dtype,
                                     const int64_t out_strides[3], int32_t splits,
                                     void *workspace, size_t workspace_bytes,
                                     cqkv_stream_t stream) {
    clear_error();
    return decode_dense("cqkv_decode_attention", q, q_dtype, q_strides, k, v, batch, q_heads,
                        q_len, kv_lens, kv_len, softmax_scale, window_left, window_right, out,
                        out_dtype, out_strides, splits, workspace, workspace_bytes, false, stream);
}

extern "C" int cqkv_decode_attention_noalloc(const void *q, int32_t q_dtype,
                                             const int64_t q_strides[3], const cqkv_side *k,
                                             const cqkv_side *v, int32_t batch, int32_t q_heads,
                                             int32_t q_len, const int32_t *kv_lens,
                                             int32_t kv_len, float softmax_scale,
                                             int32_t window_left, int32_t window_right,
                                             void *out, int32_t out_dtype,
                                             const int64_t out_strides[3], int32_t splits,
                                             cqkv_stream_t stream) {
    clear_error();
    return decode_dense("cqkv_decode_attention_noalloc", q, q_dtype, q_strides, k, v, batch,
                        q_heads, q_len, kv_lens, kv_len, softmax_scale, window_left,
                        window_right, out, out_dtype, out_strides, splits, nullptr, 0, true,
                        stream);
}

// ---- paged decode ----
// Segments of a block list: each block's valid rows, cut into runs of at most tps whole tiles;
// the run length is the dense split rule's for the total key count.
static int paged_segments(const cqkv_kv_block *blocks, int32_t n_blocks, int32_t batch,
                          std::vector<PagedSeg> *segs) {
    const cqkv_side *k0 = blocks[0].k;
    int64_t total = 0, tiles = 0;
    for (int i = 0; i < n_blocks; ++i) {
        total += blocks[i].rows;
        tiles += tiles_of(blocks[i].rows);
    }
    const int s = auto_splits(batch, k0->kv_heads, (int)std::max<int64_t>(total, 1), false,
                              waves_of(k0->format));
    const int tps = (int)std::max<int64_t>(1, (tiles + s - 1) / s);
    int key = 0, n = 0;
    for (int i = 0; i < n_blocks; ++i) {
        const cqkv_kv_block &bl = blocks[i];
        const int bt = tiles_of(bl.rows);
        for (int t = 0; t < bt; t += tps) {
            if (segs) {
                PagedSeg g = {};
                const int d = bl.k->head_dim;
                g.kc = (const uint8_t *)bl.k->codes;
                g.ks = (const uint8_t *)bl.k->scales;
                g.vc = (const uint8_t *)bl.v->codes;
                g.vs = (const uint8_t *)bl.v->scales;
                g.kc_plane = (uint32_t)cqkv_codes_plane_bytes(bl.k->format, d, bl.k->capacity);
                g.ks_plane = (uint32_t)cqkv_scales_plane_bytes(bl.k->format, d, bl.k->capacity);
                g.vc_plane = (uint32_t)cqkv_codes_plane_bytes(bl.v->format, d, bl.v->capacity);
                g.vs_plane = (uint32_t)cqkv_scales_plane_bytes(bl.v->format, d, bl.v->capacity);
                g.tile_begin = t;
                g.tile_end = min(t + tps, bt);
                g.key_offset = key;
                g.rows = bl.rows;
                segs->push_back(g);
            }
            ++n;
        }
        key += bl.rows;
    }
    return n;
}

// The segment table is written into the workspace by kernels that carry the segments by value
// in their arguments, kPagedSegsPerLaunch per launch: a captured HIP graph keeps kernel
// arguments by value, so replays see this call's table (a host -> device copy would keep a
// pointer to host memory freed when the call returns).
constexpr int kPagedSegsPerLaunch = 32;  // 32 x 64 B of kernel arguments
struct PagedTableArgs {
    PagedSeg seg[kPagedSegsPerLaunch];
    PagedSeg *dst;
    int32_t n;
};
__global__ __launch_bounds__(64) void paged_table_kernel(PagedTableArgs a) {
    // 16 words per segment; word w of segment i goes to lane w of iteration i
    const int lane = threadIdx.x;
    for (int i = lane / 16; i < a.n; i += 4)
        ((uint32_t *)(a.dst + i))[lane % 16] = ((const uint32_t *)(a.seg + i))[lane % 16];
}
static_assert(sizeof(PagedSeg) == 64, "paged_table_kernel copies 16 words per segment");

static hipError_t write_paged_table(const std::vector<PagedSeg> &segs, PagedSeg *dst,
                                    hipStream_t st) {
    for (size_t i0 = 0; i0 < segs.size(); i0 += kPagedSegsPerLaunch) {
        PagedTableArgs t = {};
        t.n = (int32_t)std::min<size_t>(kPagedSegsPerLaunch, segs.size() - i0);
        for (int i = 0; i < t.n; ++i) t.seg[i] = segs[i0 + i];
        t.dst = dst + i0;
        hipLaunchKernelGGL(paged_table_kernel, dim3(1), dim3(64), 0, st, t);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

// workspace: the segment table, then (more than one segment) the partials
static size_t paged_workspace(int nseg, int32_t batch, int32_t q_heads, int32_t q_len,
                              int32_t head_dim, size_t *part_off, size_t *lse_off) {
    *part_off = align256((size_t)nseg * sizeof(PagedSeg));
    size_t parts = 0;
    *lse_off = 0;
    if (nseg > 1) parts = workspace_layout(batch, q_heads, q_len, head_dim, nseg, lse_off);
    return *part_off + parts;
}

static int check_blocks(const cqkv_kv_block *blocks, int32_t n_blocks, int32_t batch,
                        const char *who) {
    if (!blocks || n_blocks <= 0) return fail(CQKV_ERR_ARG, "%s: no blocks", who);
    int64_t total = 0;
    for (int i = 0; i < n_blocks; ++i) {
        const cqkv_kv_block &bl = blocks[i];
        if (!bl.k || !bl.v) return fail(CQKV_ERR_ARG, "%s: block %d has a null side", who, i);
        if (int rc = check_side(bl.k, who)) return rc;
        if (int rc = check_side(bl.v, who)) return rc;
        if (bl.k->format != blocks[0].k->format || bl.k->head_dim != blocks[0].k->head_dim ||
            bl.k->kv_heads != blocks[0].k->kv_heads || bl.v->format != blocks[0].k->format ||
            bl.v->head_dim != blocks[0].k->head_dim || bl.v->kv_heads != blocks[0].k->kv_heads ||
            bl.k->is_value != 0 || bl.v->is_value != 1 || bl.k->seed != blocks[0].k->seed ||
            bl.v->seed != blocks[0].v->seed)
            return fail(CQKV_ERR_ARG,
                        "%s: block %d differs from block 0 in format, head dim, kv heads, side or seed",
                        who, i);
        if (bl.rows < 0 || bl.rows > bl.k->capacity || bl.rows > bl.v->capacity)
            return fail(CQKV_ERR_ARG, "%s: block %d has %d rows but capacities %d / %d", who, i,
                        bl.rows, bl.k->capacity, bl.v->capacity);
        total += bl.rows;
    }
    if (total == 0) return fail(CQKV_ERR_ARG, "%s: the blocks hold no keys", who);
    if (total > (1 << 30)) return fail(CQKV_ERR_ARG, "%s: %lld keys", who, (long long)total);
    (void)batch;
    return CQKV_OK;
}

extern "C" size_t cqkv_decode_paged_workspace_bytes(const cqkv_kv_block *blocks,
                                                    int32_t n_blocks, int32_t batch,
                                                    int32_t q_heads, int32_t q_len) {
    clear_error();
    if (check_blocks(blocks, n_blocks, batch, "cqkv_decode_paged_workspace_bytes") != CQKV_OK ||
        batch <= 0 || q_heads <= 0 || q_len <= 0)
        return 0;
    const int nseg = paged_segments(blocks, n_blocks, batch, nullptr);
    size_t part_off, lse_off;
    return paged_workspace(nseg, batch, q_heads, q_len, blocks[0].k->head_dim, &part_off, &lse_off);
}

extern "C" int cqkv_decode_attention_paged(const void *q, int32_t q_dtype,
                                           const int64_t q_strides[3], const cqkv_kv_block *blocks,
                                           int32_t n_blocks, int32_t batch, int32_t q_heads,
                                           int32_t q_len, float softmax_scale, int32_t window_left,
                                           int32_t window_right, void *out, int32_t out_dtype,
                                           const int64_t out_strides[3], void *workspace,
                                           size_t workspace_bytes, cqkv_stream_t stream) {
    clear_error();
    const char *who = "cqkv_decode_attention_paged";
    if (int rc = check_blocks(blocks, n_blocks, batch, who)) return rc;
    DecodeArgs a;
    if (int rc = decode_prepare(a, who, q, q_dtype, q_strides, blocks[0].k, blocks[0].v, batch,
                                q_heads, q_len, softmax_scale, window_left, window_right, out,
                                out_dtype, out_strides))
        return rc;
    std::vector<PagedSeg> segs;
    const int nseg = paged_segments(blocks, n_blocks, batch, &segs);
    int64_t total = 0;
    for (int i = 0; i < n_blocks; ++i) total += blocks[i].rows;
    const int d = blocks[0].k->head_dim;
    a.kv_len = (int32_t)total;
    a.splits = nseg;

    hipStream_t st = (hipStream_t)stream;
    size_t part_off, lse_off;
    const size_t need = paged_workspace(nseg, batch, q_heads, q_len, d, &part_off, &lse_off);
    void *ws = workspace;
    bool owned = false;
    if (ws && workspace_bytes < need)
        return fail(CQKV_ERR_WORKSPACE, "%s: workspace %zu < %zu bytes", who, workspace_bytes, need);
    if (!ws) {
        CQKV_HIP_CHECK(hipMallocAsync(&ws, need, st));
        owned = true;
    }
    hipError_t e = write_paged_table(segs, (PagedSeg *)ws, st);
    a.segs = (const PagedSeg *)ws;
    if (nseg > 1) {
        a.part_o = (float *)((char *)ws + part_off);
        a.part_lse = (float *)((char *)ws + part_off + lse_off);
    }
    if (e == hipSuccess) e = decode_launch(a, blocks[0].k->format, d, st);
    if (owned) {
        hipError_t fe = hipFreeAsync(ws, st);
        if (e == hipSuccess) e = fe;
    }
    if (e != hipSuccess) return fail(CQKV_ERR_HIP, "%s: %s", who, hipGetErrorString(e));
    return CQKV_OK;
}
