// Device code of the quantize-and-append path (included by append_inst.hip, one object per cache
// format, and by quant_append.hip for the argument structs): the row-parallel encoder
// (rows_block), the fused RoPE + append kernel and their launchers.
//
// Reference behaviour (paths relative to the reference repository root):
//   RowCodec::quantize_row, candle-core/src/accel/turbo.rs:293-381 (FP8 366-374, MX 324-347,
//   TurboMse 299-323) after TurboQuantizer::rotate (candle-nn/src/turbo_quant.rs:182-189), then
//   Cache::append (candle-nn/src/kv_cache.rs:68-99); rope / rope_i of candle-nn/src/rotary_emb.rs
//   (ROCm kernels candle-core/kernels/nn.hip:107-148).
//
// Work split (rows_block): D / 32 threads per token row, 32 elements each, so a 256-thread
// workgroup encodes 64 (D = 128) or 128 (D = 64) rows of one (batch, kv head) plane at once; key
// codes go straight to their row-major place, value codes pass through LDS into the
// token-transposed 8-token tiles. The fused RoPE + append runs the same encoder on the key and
// value planes (the keys rotated after their load) and rotates the queries beside them.
#pragma once

#include "cqkv_device.h"
#include "cqkv_host.h"

namespace cqkv {

struct AppendArgs {
    const void *x;
    int64_t sb, sh, st;  // element strides of x: batch, head, token
    uint8_t *codes;
    uint8_t *scales;
    uint32_t codes_plane, scales_plane;  // bytes per (batch, head) plane
    const int32_t *positions;            // device, per batch, or null
    int32_t position, tokens, capacity, kv_heads, x_dtype;
    int32_t rotate;         // Hadamard-rotate each row before encoding (side_fwht)
    uint32_t sign_bits[8];  // rotation: bit j set -> column j of the rotation has sign -1
    float rot_scale;        // rotation: 1 / sqrt(D) in f32
    float bnd[16];          // TURBO4: the 15 codebook boundaries (+inf padded); TURBOPROD: 7
    int32_t turbo_sym;      // TURBO4: bnd[7] == 0 and bnd[14 - i] == -bnd[i] (a symmetric codebook)
    float cent[16];         // TURBOPROD: the centroids of its (bits - 1)-bit codebook
    const float *qjl;       // TURBOPROD: device D x D QJL matrix S (row-major, the plane row
                            // length D; zero rows and columns past the head dim)
    int32_t dim;            // the head dim (TURBOPROD: residuals past it are zero)
    int32_t pair_loads;     // elements 2l, 2l+1 of every row are one aligned 4 / 8-byte word
    int32_t row_loads;      // rows_block: kRowBF16 / kRowF16 / kRowF32 (16-byte loads) or kRowAny
    const void *cos, *sin;  // rotary tables (cs_rows, D/2) in the dtype of x (fused RoPE only)
    int32_t cs_rows;        // fused RoPE: rows of the tables, positions past them are skipped
                            // (keys and values alike); 0 for a plain append
    int32_t cs_pair_loads;  // both tables aligned for paired loads
    int32_t cs_vec16;       // both tables 16-byte aligned (16-byte table loads in rope_row32)
};

// Elements idx, idx + 1 of x in two steps: load_raw only issues the loads (one when `pair` says
// they form an aligned word), raw_to_f32 converts. Batches of rows are loaded with load_raw
// before any conversion, so no branch on dtype / pairing sits between a load and the next one
// and the loads of a batch are in flight together.
struct RawPair {
    uint32_t w0, w1;
};

__device__ inline RawPair load_raw(const void *p, int64_t idx, int dtype, bool pair) {
    RawPair r = {0u, 0u};
    if (dtype == CQKV_F32) {
        if (pair) {
            const u32x2 w = *(const u32x2 *)((const float *)p + idx);
            r.w0 = w.x;
            r.w1 = w.y;
        } else {
            r.w0 = ((const uint32_t *)p)[idx];
            r.w1 = ((const uint32_t *)p)[idx + 1];
        }
    } else if (pair) {
        r.w0 = *(const uint32_t *)((const uint16_t *)p + idx);  // both halves
    } else {
        r.w0 = ((const uint16_t *)p)[idx];
        r.w1 = ((const uint16_t *)p)[idx + 1];
    }
    return r;
}

__device__ inline void raw_to_f32(const RawPair &r, int dtype, bool pair, float &x0, float &x1) {
    if (dtype == CQKV_F32) {
        x0 = __uint_as_float(r.w0);
        x1 = __uint_as_float(r.w1);
        return;
    }
    const uint32_t lo = pair ? (r.w0 & 0xffffu) : r.w0, hi = pair ? (r.w0 >> 16) : r.w1;
    x0 = dtype == CQKV_BF16 ? bf16_bits_to_f32(lo) : f16_bits_to_f32(lo);
    x1 = dtype == CQKV_BF16 ? bf16_bits_to_f32(hi) : f16_bits_to_f32(hi);
}

__device__ inline void load_pair(const void *p, int64_t idx, int dtype, bool pair, float &x0,
                                 float &x1) {
    raw_to_f32(load_raw(p, idx, dtype, pair), dtype, pair, x0, x1);
}

// W16: the launch guarantees a 16-bit dtype and pair-aligned rows (and tables), so every load is
// one dword with no branch around it.
template <bool W16>
__device__ inline RawPair load_raw_t(const void *p, int64_t idx, int dtype, bool pair) {
    if constexpr (W16) return RawPair{*(const uint32_t *)((const uint16_t *)p + idx), 0u};
    else return load_raw(p, idx, dtype, pair);
}


// Rotary embedding of the pair (x0, x1) = elements (2l, 2l+1) of a row at position `row` of the
// cos / sin tables ((rows, D/2), dtype of x), then rounded to that dtype: the reference's rope
// kernels (candle-core/kernels/nn.hip:107-148; candle-nn/src/rotary_emb.rs:585-611 `rope`,
// :275-303 `rope_i`) write their output in the input dtype, and the cache quantizes that.
//   CQKV_ROPE_HALVES:      y_i = x_i c_i - x_{i+D/2} s_i,  y_{i+D/2} = x_i s_i + x_{i+D/2} c_i
//   CQKV_ROPE_INTERLEAVED: y_2i = x_2i c_i - x_2i+1 s_i,  y_2i+1 = x_2i s_i + x_2i+1 c_i
// Products are rounded before the sum, as in the reference kernels (no fused multiply-add).
// rope_load fetches a lane's table entries (issued ahead with the row loads); rope_apply is
// called by every lane of the wave (the halves form exchanges pairs across lanes).
struct RopeCS {
    RawPair c, s;  // raw table words: interleaved one element each, halves a pair each
};

template <int D, int ROPE, bool W16>
__device__ inline RopeCS rope_load(const void *cos, const void *sin, int dtype, bool pair,
                                   int64_t row, int lane) {
    RopeCS r;
    if constexpr (ROPE == CQKV_ROPE_INTERLEAVED) {
        const int64_t i = row * (D / 2) + lane;
        if constexpr (W16) {
            r.c = RawPair{((const uint16_t *)cos)[i], 0u};
            r.s = RawPair{((const uint16_t *)sin)[i], 0u};
        } else {
            r.c = load_raw(cos, i, dtype, false);
            r.s = load_raw(sin, i, dtype, false);
        }
    } else {
        const int64_t i = row * (D / 2) + 2 * lane - (lane >= D / 4 ? D / 2 : 0);
        r.c = load_raw_t<W16>(cos, i, dtype, pair);
        r.s = load_raw_t<W16>(sin, i, dtype, pair);
    }
    return r;
}

template <int D, int ROPE>
__device__ inline void rope_apply(float &x0, float &x1, const RopeCS &t, int dtype, bool pair,
                                  int lane) {
#pragma clang fp contract(off)
    if constexpr (ROPE == CQKV_ROPE_INTERLEAVED) {
        float c, s, unused;
        raw_to_f32(RawPair{t.c.w0, t.c.w0}, dtype, false, c, unused);
        raw_to_f32(RawPair{t.s.w0, t.s.w0}, dtype, false, s, unused);
        const float y0 = x0 * c - x1 * s, y1 = x0 * s + x1 * c;
        x0 = y0;
        x1 = y1;
    } else {
        float c0, c1, s0, s1;
        raw_to_f32(t.c, dtype, pair, c0, c1);
        raw_to_f32(t.s, dtype, pair, s0, s1);
        const float p0 = shfl_xor(x0, D / 4), p1 = shfl_xor(x1, D / 4);
        if (lane < D / 4) {
            x0 = x0 * c0 - p0 * s0;
            x1 = x1 * c1 - p1 * s1;
        } else {
            x0 = p0 * s0 + x0 * c0;
            x1 = p1 * s1 + x1 * c1;
        }
    }
    if (dtype == CQKV_BF16) {
        x0 = bf16_bits_to_f32(f32_to_bf16_bits(x0));
        x1 = bf16_bits_to_f32(f32_to_bf16_bits(x1));
    } else if (dtype == CQKV_F16) {
        x0 = (float)(_Float16)x0;
        x1 = (float)(_Float16)x1;
    }
}

// ---------------------------------------------------------------------------------------------
// Row-parallel append (cqkv_quant_append): R = D / 32 threads per token row, thread q holding the
// 32 elements 32 q .. 32 q + 31, so a 256-thread workgroup encodes 256 / R rows at once. Row
// reductions (FP8 / NVFP4 maxima, TurboQuant norms and transform stages across threads) are one or
// two DPP steps inside a quad; an MX block is exactly one thread. Rows come in by 16-byte loads
// issued before any conversion, key codes go out as 16-byte row-major stores, and value codes are
// staged in LDS and written as whole 16-byte pieces of the 8-token tiles. The encoders compute
// the codes of RowCodec::quantize_row (candle-core/src/accel/turbo.rs:293-381) bit for bit, except
// TurboQuant's, whose rotation the reference computes as a matmul of unpinned summation order (here
// the Walsh-Hadamard stages in stride order 1, 2, ..., D / 2).
// ---------------------------------------------------------------------------------------------
// row load forms: 16-byte loads of bf16 / f16 / f32 rows (16-byte aligned), or element loads
enum { kRowBF16 = 0, kRowF32 = 1, kRowAny = 2, kRowF16 = 3 };

// v from the lane `lane ^ M` of the same quad (M = 1 or 2), by DPP quad_perm
template <int M>
__device__ inline float quad_xor(float v) {
    constexpr int ctrl = M == 1 ? 0xB1 : 0x4E;  // quad_perm [1,0,3,2] / [2,3,0,1]
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), ctrl, 0xF, 0xF, true));
}
template <int M>
__device__ inline uint32_t quad_xor_u(uint32_t v) {
    constexpr int ctrl = M == 1 ? 0xB1 : 0x4E;
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, ctrl, 0xF, 0xF, true);
}
// v from the lane `lane ^ 4` (the partner quad of a row of 8 threads at D = 256), by
// ds_swizzle in bit-mask mode (and 0x1f, xor 4)
__device__ inline uint32_t xor4_u(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_ds_swizzle((int)v, 0x101F);
}
__device__ inline float xor4(float v) { return __uint_as_float(xor4_u(__float_as_uint(v))); }
template <int R>
__device__ inline float row_max(float v) {
    v = fmaxf(v, quad_xor<1>(v));
    if constexpr (R >= 4) v = fmaxf(v, quad_xor<2>(v));
    if constexpr (R == 8) v = fmaxf(v, xor4(v));
    return v;
}
template <int R>
__device__ inline float row_sum(float v) {
    v += quad_xor<1>(v);
    if constexpr (R >= 4) v += quad_xor<2>(v);
    if constexpr (R == 8) v += xor4(v);
    return v;
}
template <int R>
__device__ inline uint32_t row_or(uint32_t v) {
    v |= quad_xor_u<1>(v);
    if constexpr (R >= 4) v |= quad_xor_u<2>(v);
    if constexpr (R == 8) v |= xor4_u(v);
    return v;
}

// The 32 elements of this thread: element offset `base` (the block's first row, uniform across the
// workgroup) plus `lane` (this thread's row and element 32 q first), issued as one batch of loads
// before any conversion. The 16-byte forms are buffer loads from `base`, with dead rows pointed
// past the buffer range (the hardware returns zeros): no branch around a load, so the loads of a
// batch are in flight together (the host takes these forms only when a block's rows lie within
// 2^31 bytes of `base`).
constexpr uint32_t kRowOOB = 0x80000000u;
template <int LOAD>
__device__ inline void load_row32(const AppendArgs &a, int64_t base, int64_t lane, bool live,
                                  float (&x)[32]) {
    if constexpr (LOAD == kRowBF16 || LOAD == kRowF16) {
        const rsrc_t r = make_rsrc((const uint16_t *)a.x + base, kRowOOB);
        const uint32_t off = live ? (uint32_t)lane * 2u : kRowOOB;
        u32x4 w[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) w[i] = ld128(r, off + 16 * i);
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t v = w[i][e];
                if constexpr (LOAD == kRowBF16) {
                    x[8 * i + 2 * e] = __uint_as_float(v << 16);
                    x[8 * i + 2 * e + 1] = __uint_as_float(v & 0xffff0000u);
                } else {
                    x[8 * i + 2 * e] = f16_bits_to_f32(v & 0xffffu);
                    x[8 * i + 2 * e + 1] = f16_bits_to_f32(v >> 16);
                }
            }
    } else if constexpr (LOAD == kRowF32) {
        const rsrc_t r = make_rsrc((const float *)a.x + base, kRowOOB);
        const uint32_t off = live ? (uint32_t)lane * 4u : kRowOOB;
        u32x4 w[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) w[i] = ld128(r, off + 16 * i);
#pragma unroll
        for (int i = 0; i < 8; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e) x[4 * i + e] = __uint_as_float(w[i][e]);
    } else {
#pragma unroll
        for (int i = 0; i < 32; ++i) x[i] = live ? load_elem(a.x, base + lane + i, a.x_dtype) : 0.0f;
    }
}

// Codebook index of u, #{boundaries <= u} (Codebook::index, candle-core/src/accel/turbo.rs:40-44),
// for a symmetric codebook (bnd[7] = 0, bnd[14 - i] = -bnd[i]) and a finite u, by a three-step
// search over the 7 positive boundaries p[k] = bnd[8 + k]: for u >= 0 the index is
// 8 + #{p[k] <= u}; for u < 0 it is 7 - #{p[k] < |u|} = 7 - #{p[k] <= pred(|u|)}, pred the next
// float below. Non-negative floats order as their bit patterns, so each comparison is an integer
// subtraction whose sign gives a 0 / -1 mask, and each boundary choice a bitfield select: no
// branch and no lane-mask register (pb: the boundaries' bit patterns, in scalar registers).
__device__ inline int32_t sel_mask(int32_t m, int32_t if_set, int32_t if_clear) {
    return (if_set & m) | (if_clear & ~m);
}
__device__ inline uint32_t turbo_index_sym(float u, const int32_t (&pb)[7]) {
    const int32_t bits = __float_as_int(u + 0.0f);      // -0 -> +0
    const int32_t neg = (int32_t)((uint32_t)bits >> 31);  // u < 0 (then |u| > 0)
    const int32_t bx = (bits & 0x7fffffff) - neg;       // pattern of |u|, or of pred(|u|)
    // the sign of a wrapping subtraction (never out of range here: both patterns are below
    // 2^31); written so the compiler keeps it arithmetic instead of a compare and a select
    auto below = [bx](int32_t p) { return (int32_t)((uint32_t)bx - (uint32_t)p) >> 31; };
    const int32_t m3 = below(pb[3]);  // -1: below p3
    const int32_t m2 = below(sel_mask(m3, pb[1], pb[5]));
    const int32_t b1 = sel_mask(m3, sel_mask(m2, pb[0], pb[2]), sel_mask(m2, pb[4], pb[6]));
    const int32_t m1 = below(b1);
    const int32_t t = 4 * m3 + 2 * m2 + m1;              // #{p <= x} - 7, in [-7, 0]
    // 8 + #{p <= x} = 15 + t; for u < 0, 7 - #{p <= x} = (15 + t) ^ 15
    return (uint32_t)((15 + t) ^ (neg * 15));
}

// Rotary embedding of this thread's 32 elements at table row p (the token's cache position),
// rounded to the dtype as the reference's rope output is (see rope_apply). Halves: element j pairs
// with j + D / 2, which sits in thread q ^ (R / 2) at the same slot; interleaved: pairs (2i, 2i+1)
// are in the thread. Products are rounded before the sum (no fused multiply-add).
template <int D, int ROPE>
__device__ inline void rope_row32(const AppendArgs &a, int64_t p, int q, bool live,
                                  float (&x)[32]) {
#pragma clang fp contract(off)
    constexpr int R = D / 32;
    constexpr int NT = ROPE == CQKV_ROPE_HALVES ? 32 : 16;  // table entries of this thread
    const int64_t e0 = p * (D / 2) + (ROPE == CQKV_ROPE_HALVES ? 32 * (q % (R / 2)) : 16 * q);
    float c[NT], s[NT];
    if (a.cs_vec16 && a.x_dtype != CQKV_F32) {
        u32x4 cw[NT / 8], sw[NT / 8];
#pragma unroll
        for (int i = 0; i < NT / 8; ++i) {
            cw[i] = live ? *(const u32x4 *)((const uint16_t *)a.cos + e0 + 8 * i) : u32x4{0u, 0u, 0u, 0u};
            sw[i] = live ? *(const u32x4 *)((const uint16_t *)a.sin + e0 + 8 * i) : u32x4{0u, 0u, 0u, 0u};
        }
        const bool bf = a.x_dtype == CQKV_BF16;
#pragma unroll
        for (int i = 0; i < NT; ++i) {
            const uint32_t cb = (cw[i / 8][(i % 8) / 2] >> (16 * (i % 2))) & 0xffffu;
            const uint32_t sbits = (sw[i / 8][(i % 8) / 2] >> (16 * (i % 2))) & 0xffffu;
            c[i] = bf ? bf16_bits_to_f32(cb) : f16_bits_to_f32(cb);
            s[i] = bf ? bf16_bits_to_f32(sbits) : f16_bits_to_f32(sbits);
        }
    } else {
#pragma unroll
        for (int i = 0; i < NT; ++i) {
            c[i] = live ? load_elem(a.cos, e0 + i, a.x_dtype) : 0.0f;
            s[i] = live ? load_elem(a.sin, e0 + i, a.x_dtype) : 0.0f;
        }
    }
    if constexpr (ROPE == CQKV_ROPE_HALVES) {
        const bool upper = q >= R / 2;
#pragma unroll
        for (int i = 0; i < 32; ++i) {
            const float pv = R == 4 ? quad_xor<2>(x[i]) : quad_xor<1>(x[i]);
            x[i] = upper ? pv * s[i] + x[i] * c[i] : x[i] * c[i] - pv * s[i];
        }
    } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const float x0 = x[2 * i], x1 = x[2 * i + 1];
            x[2 * i] = x0 * c[i] - x1 * s[i];
            x[2 * i + 1] = x0 * s[i] + x1 * c[i];
        }
    }
#pragma unroll
    for (int i = 0; i < 32; ++i) {
        if (a.x_dtype == CQKV_BF16) x[i] = bf16_bits_to_f32(f32_to_bf16_bits(x[i]));
        else if (a.x_dtype == CQKV_F16) x[i] = (float)(_Float16)x[i];
    }
}

// y = H (sign * x) / sqrt(D) of this thread's 32 elements of a row (rotation_matrix(D, Hadamard,
// seed), candle-core/src/accel/turbo.rs:180-203, applied as TurboQuantizer::rotate does,
// candle-nn/src/turbo_quant.rs:182-189): the sign flip, the Walsh-Hadamard stages in element-stride
// order 1, 2, ..., D / 2 (1..16 in the thread, 32 and 64 across the row's threads by DPP, 128
// by ds_swizzle), then 1 / sqrt(D).
template <int D>
__device__ inline void hadamard_row32(const AppendArgs &a, int q, float (&x)[32]) {
    constexpr int R = D / 32;
    const uint32_t sb = a.sign_bits[q];
#pragma unroll
    for (int i = 0; i < 32; ++i)
        x[i] = __uint_as_float(__float_as_uint(x[i]) ^ ((sb << (31 - i)) & 0x80000000u));
#pragma unroll
    for (int m = 1; m < 32; m <<= 1)
#pragma unroll
        for (int i = 0; i < 32; ++i)
            if (!(i & m)) {
                const float u = x[i], v = x[i + m];
                x[i] = u + v;
                x[i + m] = u - v;
            }
    {
        const float sg = (q & 1) ? -1.0f : 1.0f;  // stride 32: partner thread q ^ 1
#pragma unroll
        for (int i = 0; i < 32; ++i) x[i] = __builtin_fmaf(sg, x[i], quad_xor<1>(x[i]));
    }
    if constexpr (R >= 4) {
        const float sg = (q & 2) ? -1.0f : 1.0f;  // stride 64: partner thread q ^ 2
#pragma unroll
        for (int i = 0; i < 32; ++i) x[i] = __builtin_fmaf(sg, x[i], quad_xor<2>(x[i]));
    }
    if constexpr (R == 8) {
        const float sg = (q & 4) ? -1.0f : 1.0f;  // stride 128: partner thread q ^ 4
#pragma unroll
        for (int i = 0; i < 32; ++i) x[i] = __builtin_fmaf(sg, x[i], xor4(x[i]));
    }
#pragma unroll
    for (int i = 0; i < 32; ++i) x[i] *= a.rot_scale;
}

// NR token rows of plane (b, h) from cache position c0 = first tile of the range + bx * NR, by
// the first NR * D / 32 threads of a 256-thread workgroup (all 256 threads must call it: the
// value tiles pass through LDS). ROPE != 0 rotates each row first (the fused RoPE + append).
// TurboProd's QJL stage for the block's rows (RowCodec::quantize_row, candle-core/src/accel/
// turbo.rs:311-320): residual r = u - centroid[code] of the unit row u = y / norm, rsc1 = |r|,
// and the sign bits of p = S r. Only signs are kept, so r is scaled by 64 (exact) into the range
// where its f16 hi + lo split keeps 22 significant bits; p = S_hi r_hi + S_hi r_lo + S_lo r_hi
// on v_mfma_f32_16x16x32_f16 (products exact, f32 sums; the dropped S_lo r_lo is 2^-22 of a
// term). Wavefront w owns outputs [w D / 4, (w + 1) D / 4): its rows of S stay in registers as
// A operands, the rows' r (hi, lo) come from LDS as B operands, and lane (row n, group g) gets p
// of outputs 16 bo + 4 g + i: bits OR-ed across g into the wavefront's D / 4 bits of the row.
constexpr int kProdResidStride = 8;  // f16 padding per LDS row: conflict-free 16-byte reads
__device__ inline void f16_split8(const float *v, f16x8 &hi, f16x8 &lo) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const _Float16 h = (_Float16)v[e];
        hi[e] = h;
        lo[e] = (_Float16)(v[e] - (float)h);
    }
}
template <int D, int NR>
__device__ inline void prod_qjl(const AppendArgs &a, const float (&x)[32], float inv,
                                const uint32_t (&cw)[4], bool live, int t, int r, int q,
                                uint8_t *scales, uint16_t *sm_r, float *sm_cent) {
    constexpr int R = D / 32, LD = D + kProdResidStride;  // f16 per LDS row
    constexpr int NB = D / 64;                            // 16-output blocks per wavefront
    constexpr int NC = D / 32;                            // 32-wide k chunks
    const int tid = threadIdx.x;
    if (tid < 16) sm_cent[tid] = a.cent[tid];
    __syncthreads();
    float rr = 0.0f, res[32];
#pragma unroll
    for (int i = 0; i < 32; ++i) {
        const uint32_t code = (cw[i / 8] >> (4 * (i % 8))) & 15u;
        // elements past the head dim (zero padding) have no residual
        res[i] = live && 32 * q + i < a.dim ? x[i] * inv - sm_cent[code] : 0.0f;
        rr += res[i] * res[i];
    }
    const float r1 = __builtin_sqrtf(row_sum<R>(rr));
    if (r < NR) {
        uint16_t *hrow = sm_r + r * LD + 32 * q, *lrow = sm_r + (NR + r) * LD + 32 * q;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            float v[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] = 64.0f * res[8 * j + e];
            f16x8 hi, lo;
            f16_split8(v, hi, lo);
            *(f16x8 *)(hrow + 8 * j) = hi;
            *(f16x8 *)(lrow + 8 * j) = lo;
        }
    }
    if (live && q == 0) ((float *)(scales + (int64_t)a.capacity * 4))[t] = r1;
    const int lane = tid & 63, wave = tid >> 6, n = lane & 15, g = lane >> 4;
    const int o0 = wave * (D / 4);
    const int pos = a.positions ? a.positions[blockIdx.z] : a.position;
    int end = min(pos + a.tokens, a.capacity);
    if (a.cs_rows > 0) end = min(end, a.cs_rows);
    const int c0 = t - r;  // the block's first cache position
    uint8_t *signs = scales + (int64_t)a.capacity * 8;
    if constexpr (D == 256) {
        // S does not fit the registers whole at D = 256 (256 VGPRs of operands): one 16-output
        // block of the wavefront's rows at a time, every row block against it; the 64 sign bits
        // of a row gather in a 64-bit word
        __syncthreads();
        uint64_t words[NR / 16];
#pragma unroll
        for (int rb = 0; rb < NR / 16; ++rb) words[rb] = 0;
#pragma unroll 1
        for (int bo = 0; bo < NB; ++bo) {
            f16x8 shi[NC], slo[NC];
#pragma unroll
            for (int c = 0; c < NC; ++c) {
                const float *src = a.qjl + (int64_t)(o0 + 16 * bo + n) * D + 32 * c + 8 * g;
                const f32x4 v0 = *(const f32x4 *)src, v1 = *(const f32x4 *)(src + 4);
                const float v[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
                f16_split8(v, shi[c], slo[c]);
            }
#pragma unroll
            for (int rb = 0; rb < NR / 16; ++rb) {
                f32x4 acc = {0.f, 0.f, 0.f, 0.f};
                const uint16_t *hrow = sm_r + (16 * rb + n) * LD + 8 * g;
                const uint16_t *lrow = sm_r + (NR + 16 * rb + n) * LD + 8 * g;
#pragma unroll
                for (int c = 0; c < NC; ++c) {
                    const f16x8 rhi = *(const f16x8 *)(hrow + 32 * c), rlo = *(const f16x8 *)(lrow + 32 * c);
                    acc = mfma16x16x32(shi[c], rhi, acc);
                    acc = mfma16x16x32(shi[c], rlo, acc);
                    acc = mfma16x16x32(slo[c], rhi, acc);
                }
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    words[rb] |= (uint64_t)(acc[i] >= 0.0f ? 1u : 0u) << (16 * bo + 4 * g + i);
            }
        }
#pragma unroll
        for (int rb = 0; rb < NR / 16; ++rb) {
            uint32_t lo = (uint32_t)words[rb], hi = (uint32_t)(words[rb] >> 32);
            lo |= (uint32_t)__shfl_xor((int)lo, 16, 64);
            hi |= (uint32_t)__shfl_xor((int)hi, 16, 64);
            lo |= (uint32_t)__shfl_xor((int)lo, 32, 64);
            hi |= (uint32_t)__shfl_xor((int)hi, 32, 64);
            // outputs past the head dim (zero rows of the padded S): no sign bits
            const int valid = a.dim - o0;
            if (valid < 32) lo &= valid <= 0 ? 0u : (1u << valid) - 1u;
            if (valid < 64) hi &= valid <= 32 ? 0u : (1u << (valid - 32)) - 1u;
            const int tr = c0 + 16 * rb + n;
            if (g == 0 && tr >= pos && tr < end)
                *(u32x2 *)(signs + (int64_t)tr * (D / 8) + wave * (D / 32)) = u32x2{lo, hi};
        }
        return;
    }
    // this wavefront's rows of S as A operands: lane (m, g) of block bo, chunk c holds
    // S[o0 + 16 bo + m][32 c + 8 g .. + 7]
    f16x8 shi[NB][NC], slo[NB][NC];
#pragma unroll
    for (int bo = 0; bo < NB; ++bo)
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            const float *src = a.qjl + (int64_t)(o0 + 16 * bo + n) * D + 32 * c + 8 * g;
            const f32x4 v0 = *(const f32x4 *)src, v1 = *(const f32x4 *)(src + 4);
            const float v[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
            f16_split8(v, shi[bo][c], slo[bo][c]);
        }
    __syncthreads();
#pragma unroll 1
    for (int rb = 0; rb < NR / 16; ++rb) {
        f32x4 acc[NB];
#pragma unroll
        for (int bo = 0; bo < NB; ++bo) acc[bo] = f32x4{0.f, 0.f, 0.f, 0.f};
        const uint16_t *hrow = sm_r + (16 * rb + n) * LD + 8 * g;
        const uint16_t *lrow = sm_r + (NR + 16 * rb + n) * LD + 8 * g;
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            const f16x8 rhi = *(const f16x8 *)(hrow + 32 * c), rlo = *(const f16x8 *)(lrow + 32 * c);
#pragma unroll
            for (int bo = 0; bo < NB; ++bo) {
                acc[bo] = mfma16x16x32(shi[bo][c], rhi, acc[bo]);
                acc[bo] = mfma16x16x32(shi[bo][c], rlo, acc[bo]);
                acc[bo] = mfma16x16x32(slo[bo][c], rhi, acc[bo]);
            }
        }
        // acc[bo][i] = p of output o0 + 16 bo + 4 g + i, row 16 rb + n
        uint32_t word = 0;
#pragma unroll
        for (int bo = 0; bo < NB; ++bo)
#pragma unroll
            for (int i = 0; i < 4; ++i) word |= (acc[bo][i] >= 0.0f ? 1u : 0u) << (16 * bo + 4 * g + i);
        word |= (uint32_t)__shfl_xor((int)word, 16, 64);
        word |= (uint32_t)__shfl_xor((int)word, 32, 64);
        // outputs past the head dim (zero rows of the padded S): no sign bits
        const int valid = a.dim - o0;
        if (valid < D / 4) word &= valid <= 0 ? 0u : (1u << valid) - 1u;
        const int tr = c0 + 16 * rb + n;
        if (g == 0 && tr >= pos && tr < end) {
            uint8_t *dst = signs + (int64_t)tr * (D / 8) + wave * (D / 32);
            if constexpr (D == 128) *(uint32_t *)dst = word;
            else *(uint16_t *)dst = (uint16_t)word;
        }
    }
}

// The 8-token value tiles of ROWS rows starting at cache position c0 (a multiple of 8), from
// their row-major codes in LDS (kRowBytes per row): a 16-byte piece of a tile holds 2 (byte
// codes) or 4 (nibble codes) elements of all 8 tokens. Positions outside [pos, end) keep the
// codes already in the cache. All NT threads of the workgroup take part.
template <bool kB8, int D, int ROWS, int NT = 256>
__device__ inline void write_value_tiles(uint8_t *codes, const uint8_t *sm_codes, int c0, int pos,
                                         int end, int tid) {
    constexpr int kRowBytes = kB8 ? D : D / 2;
    constexpr int kPer = kB8 ? 2 : 4;           // elements per piece
    constexpr int kPieces = ROWS / 8 * (D / kPer);
    for (int i = tid; i < kPieces; i += NT) {
        const int T = i / (D / kPer), e = i % (D / kPer);
        const int tt = c0 + 8 * T;  // first cache position of the tile
        uint32_t mask = 0;
#pragma unroll
        for (int s2 = 0; s2 < 8; ++s2) mask |= (tt + s2 >= pos && tt + s2 < end) ? 1u << s2 : 0u;
        if (!mask) continue;
        uint32_t wv[4] = {0u, 0u, 0u, 0u};
#pragma unroll
        for (int s2 = 0; s2 < 8; ++s2) {
            const uint32_t c2 = *(const uint16_t *)(sm_codes + (8 * T + s2) * kRowBytes + 2 * e);
            if constexpr (kB8) {  // elements 2e (low byte), 2e + 1: bytes e*16 + s2, + 8
                wv[s2 / 4] |= (c2 & 0xffu) << (8 * (s2 % 4));
                wv[2 + s2 / 4] |= (c2 >> 8) << (8 * (s2 % 4));
            } else {  // elements 4e .. 4e + 3: nibble k of c2, word k, nibble s2
#pragma unroll
                for (int k = 0; k < 4; ++k) wv[k] |= ((c2 >> (4 * k)) & 15u) << (4 * s2);
            }
        }
        u32x4 *dst = (u32x4 *)(codes + (int64_t)(tt / 8) * (kB8 ? D * 8 : D * 4) + 16 * e);
        if (mask != 0xffu) {  // keep the codes of tokens this call does not write
            uint32_t keep[4];
            if constexpr (kB8) {
                uint32_t kb = 0;
#pragma unroll
                for (int s2 = 0; s2 < 4; ++s2) kb |= ((mask >> s2) & 1u) ? 0u : 0xffu << (8 * s2);
                uint32_t kh = 0;
#pragma unroll
                for (int s2 = 0; s2 < 4; ++s2) kh |= ((mask >> (s2 + 4)) & 1u) ? 0u : 0xffu << (8 * s2);
                keep[0] = keep[2] = kb;
                keep[1] = keep[3] = kh;
            } else {
                uint32_t kn = 0;
#pragma unroll
                for (int s2 = 0; s2 < 8; ++s2) kn |= ((mask >> s2) & 1u) ? 0u : 0xfu << (4 * s2);
                keep[0] = keep[1] = keep[2] = keep[3] = kn;
            }
            const u32x4 old = *dst;
#pragma unroll
            for (int k = 0; k < 4; ++k) wv[k] = (wv[k] & ~keep[k]) | (old[k] & keep[k]);
        }
        *dst = u32x4{wv[0], wv[1], wv[2], wv[3]};
    }
}

template <int FMT, int IS_VALUE, int D, int LOAD, int ROPE, int NR>
__device__ inline void rows_block(const AppendArgs &a, int h, int b, int bx) {
    constexpr int R = D / 32, ROWS = NR;
    static_assert(NR * R <= 256, "rows of one workgroup");
    constexpr bool kB8 = FMT == CQKV_FMT_FP8 || FMT == CQKV_FMT_MXFP8;
    constexpr int kRowBytes = kB8 ? D : D / 2;  // code bytes per token
    __shared__ __attribute__((aligned(16))) uint8_t sm_codes[IS_VALUE ? ROWS * kRowBytes : 16];
    constexpr bool kProd = FMT == CQKV_FMT_TURBOPROD;
    static_assert(!kProd || !IS_VALUE, "TurboProd is a key format");
    // TurboProd: the rows' scaled residuals (f16 hi rows, then lo rows) for the S r projection,
    // and the centroids of its MSE codebook
    __shared__ __attribute__((aligned(16))) uint16_t
        sm_resid[kProd ? 2 * ROWS * (D + kProdResidStride) : 8];
    __shared__ float sm_cent[16];

    const int pos = a.positions ? a.positions[b] : a.position;
    if (pos < 0) return;
    // cache positions [c0, c0 + ROWS): whole 8-token value tiles from the first tile of the range
    const int c0 = pos / 8 * 8 + bx * ROWS;
    int end = min(pos + a.tokens, a.capacity);
    if (a.cs_rows > 0) end = min(end, a.cs_rows);
    if (c0 >= end) return;  // the whole workgroup
    const int tid = threadIdx.x, r = tid / R, q = tid % R;
    const int t = c0 + r;
    const bool live = r < ROWS && t >= pos && t < end;
    const int64_t plane = (int64_t)b * a.kv_heads + h;
    uint8_t *codes = a.codes + plane * a.codes_plane;
    uint8_t *scales = a.scales + plane * a.scales_plane;

    float x[32];
    load_row32<LOAD>(a, (int64_t)b * a.sb + (int64_t)h * a.sh + (int64_t)(c0 - pos) * a.st,
                     (int64_t)r * a.st + 32 * q, live, x);
    if constexpr (ROPE != 0) rope_row32<D, ROPE>(a, t, q, live, x);
    if (a.rotate) hadamard_row32<D>(a, q, x);

    uint32_t cw[kB8 ? 8 : 4];  // this thread's 32 codes, element order
    float tok_scale = 0.0f;    // FP8 / TURBO4 / NVFP4: the token's f32
    uint32_t blk = 0;          // MX: the block's E8M0 byte; NVFP4: the two E4M3 block bytes
    if constexpr (FMT == CQKV_FMT_FP8) {
        float m = 0.0f, chk = 0.0f;  // chk: NaN iff an element is not finite
#pragma unroll
        for (int i = 0; i < 32; ++i) {
            m = fmaxf(m, __builtin_fabsf(x[i]));
            chk = __builtin_fmaf(x[i], 0.0f, chk);
        }
        const float amax = row_max<R>(m);
        const float sc = amax > 0.0f ? amax / 448.0f : 1.0f;
        const float rc = 1.0f / sc;
        if (chk == chk && amax >= kFp8FastRowMin && amax <= 3.0e38f) {  // an ordinary row
#pragma unroll
            for (int w = 0; w < 8; ++w)
                cw[w] = fp8_row_codes_fast(x[4 * w], x[4 * w + 1], sc, rc) |
                        (fp8_row_codes_fast(x[4 * w + 2], x[4 * w + 3], sc, rc) << 16);
        } else {
#pragma unroll
            for (int w = 0; w < 8; ++w)
                cw[w] = fp8_row_codes(x[4 * w], x[4 * w + 1], sc, rc) |
                        (fp8_row_codes(x[4 * w + 2], x[4 * w + 3], sc, rc) << 16);
        }
        tok_scale = sc;
    } else if constexpr (FMT == CQKV_FMT_MXFP4 || FMT == CQKV_FMT_MXFP8) {
        constexpr bool kFp4 = FMT == CQKV_FMT_MXFP4;
        float m = 0.0f;
        bool nan = false;
#pragma unroll
        for (int i = 0; i < 32; ++i) {
            m = fmaxf(m, __builtin_fabsf(x[i]));
            nan |= x[i] != x[i];
        }
        const uint32_t sc = mx_scale_code(m, kFp4 ? 2 : 8);
        blk = sc;
        const float scale = e8m0_to_f32(sc);
        const float rs = 1.0f / scale;  // a power of two: x * rs is x / scale exactly
#pragma unroll
        for (int w = 0; w < (kFp4 ? 4 : 8); ++w) cw[w] = 0u;
        if (sc != 0 && !nan) {
            if constexpr (kFp4) {
#pragma unroll
                for (int w = 0; w < 4; ++w)
                    cw[w] = fp4_encode_hw(x[8 * w] * rs, x[8 * w + 1] * rs) |
                            (fp4_encode_hw(x[8 * w + 2] * rs, x[8 * w + 3] * rs) << 8) |
                            (fp4_encode_hw(x[8 * w + 4] * rs, x[8 * w + 5] * rs) << 16) |
                            (fp4_encode_hw(x[8 * w + 6] * rs, x[8 * w + 7] * rs) << 24);
            } else {
                // |x / scale| < 512; the conversion equals e4m3_encode up to 449 and the
                // reference saturates from 448 on, so clamp to +-448 first
#pragma unroll
                for (int w = 0; w < 8; ++w) {
                    float y[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        y[e] = fminf(fmaxf(x[4 * w + e] * rs, -448.0f), 448.0f);
                    cw[w] = e4m3_encode2(y[0], y[1]) | (e4m3_encode2(y[2], y[3]) << 16);
                }
            }
        } else if (sc != 0) {  // a NaN in the block: the software encoders
#pragma unroll
            for (int i = 0; i < 32; ++i) {
                const uint32_t c = kFp4 ? fp4_encode(x[i] / scale) : e4m3_encode(x[i] / scale);
                cw[kFp4 ? i / 8 : i / 4] |= c << (kFp4 ? 4 * (i % 8) : 8 * (i % 4));
            }
        }
    } else if constexpr (FMT == CQKV_FMT_NVFP4) {
        // g = row absmax / 2688; per 16 elements an E4M3 scale of bmax / 6 / g; codes E2M1 of
        // x / (e4m3(cs) g) (turbo.rs:348-365)
        float bm[2] = {0.0f, 0.0f}, chk[2] = {0.0f, 0.0f};  // chk: NaN iff not all finite
#pragma unroll
        for (int i = 0; i < 32; ++i) {
            bm[i / 16] = fmaxf(bm[i / 16], __builtin_fabsf(x[i]));
            chk[i / 16] = __builtin_fmaf(x[i], 0.0f, chk[i / 16]);
        }
        const float amax = row_max<R>(fmaxf(bm[0], bm[1]));
        const float gs = amax > 0.0f ? amax / 2688.0f : 1.0f;
#pragma unroll
        for (int w = 0; w < 4; ++w) cw[w] = 0u;
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const uint32_t cs = e4m3_encode(bm[k] / 6.0f / gs);
            blk |= cs << (8 * k);
            const float eff = __builtin_amdgcn_cvt_f32_fp8(cs, 0) * gs;
            if (!(eff > 0.0f)) continue;
            if (chk[k] == chk[k] && bm[k] >= kNvfp4FastBlockMin) {  // an ordinary block
                const float re = 1.0f / eff;
#pragma unroll
                for (int i = 0; i < 16; i += 2)
                    cw[2 * k + i / 8] |= nvfp4_codes2_fast(x[16 * k + i], x[16 * k + i + 1], eff, re)
                                         << (4 * (i % 8));
            } else {
#pragma unroll
                for (int i = 0; i < 16; ++i)
                    cw[2 * k + i / 8] |= fp4_encode(x[16 * k + i] / eff) << (4 * (i % 8));
            }
        }
        tok_scale = gs;
    } else {  // TURBO4: the (rotated) row's norm, codebook index of y / norm
        float ss = 0.0f;
#pragma unroll
        for (int i = 0; i < 32; ++i) ss += x[i] * x[i];
        const float norm = __builtin_sqrtf(row_sum<R>(ss));
        const float inv = norm > 0.0f ? 1.0f / norm : 0.0f;
        if (a.turbo_sym && norm <= 3.0e38f && inv <= 3.0e38f) {
            // finite norm and 1 / norm: every u = y / norm is finite
            int32_t p[7];
#pragma unroll
            for (int k = 0; k < 7; ++k) p[k] = __float_as_int(a.bnd[8 + k]);
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                uint32_t c = 0;
#pragma unroll
                for (int e = 0; e < 8; ++e) c |= turbo_index_sym(x[8 * w + e] * inv, p) << (4 * e);
                cw[w] = c;
            }
        } else {  // the count itself: NaN -> 0, infinities, any codebook
            float bnd[15];
#pragma unroll
            for (int k = 0; k < 15; ++k) bnd[k] = a.bnd[k];
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                uint32_t c = 0;
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float u = x[8 * w + e] * inv;
                    uint32_t k = 0;
#pragma unroll
                    for (int i = 0; i < 15; ++i) k += u >= bnd[i] ? 1u : 0u;
                    c |= k << (4 * e);
                }
                cw[w] = c;
            }
        }
        tok_scale = norm;
        if constexpr (kProd) prod_qjl<D, NR>(a, x, inv, cw, live, t, r, q, scales, sm_resid, sm_cent);
        if (32 * q + 32 > a.dim) {  // elements past the head dim (zero padding): zero codes
#pragma unroll
            for (int i = 0; i < 32; ++i)
                if (32 * q + i >= a.dim) cw[i / 8] &= ~(15u << (4 * (i % 8)));
        }
    }

    // ---- scales ----
    if constexpr (FMT == CQKV_FMT_FP8 || FMT == CQKV_FMT_TURBO4 || FMT == CQKV_FMT_NVFP4 || kProd) {
        constexpr int kBlockBytes = FMT == CQKV_FMT_NVFP4 ? D / 16 : 0;
        if (live && q == 0) ((float *)(scales + (int64_t)a.capacity * kBlockBytes))[t] = tok_scale;
    }
    if constexpr (FMT == CQKV_FMT_MXFP4 || FMT == CQKV_FMT_MXFP8) {
        // block q's byte at byte q of the token's D / 32
        const uint32_t lo = row_or<R>(q < 4 ? blk << (8 * q) : 0u);
        if constexpr (R == 8) {
            const uint32_t hi = row_or<R>(q >= 4 ? blk << (8 * (q - 4)) : 0u);
            if (live && q == 0) *(u32x2 *)(scales + (int64_t)t * 8) = u32x2{lo, hi};
        } else if (live && q == 0) {
            if constexpr (R == 4) *(uint32_t *)(scales + (int64_t)t * 4) = lo;
            else *(uint16_t *)(scales + (int64_t)t * 2) = (uint16_t)lo;
        }
    }
    if constexpr (FMT == CQKV_FMT_NVFP4) {
        // blocks 2q, 2q + 1: bytes 2q, 2q + 1 of the token's D / 16; word w from threads 2w, 2w + 1
        uint32_t w[R / 2];
#pragma unroll
        for (int k = 0; k < R / 2; ++k) w[k] = row_or<R>(q / 2 == k ? blk << (16 * (q % 2)) : 0u);
        if (live && q == 0) {
            if constexpr (R == 8) *(u32x4 *)(scales + (int64_t)t * 16) = u32x4{w[0], w[1], w[2], w[3]};
            else if constexpr (R == 4) *(u32x2 *)(scales + (int64_t)t * 8) = u32x2{w[0], w[1]};
            else *(uint32_t *)(scales + (int64_t)t * 4) = w[0];
        }
    }

    // ---- codes ----
    if constexpr (!IS_VALUE) {
        if (live) {
            uint8_t *dst = codes + (int64_t)t * kRowBytes + q * (kRowBytes / R);
            if constexpr (kB8) {
                *(u32x4 *)dst = u32x4{cw[0], cw[1], cw[2], cw[3]};
                *(u32x4 *)(dst + 16) = u32x4{cw[4], cw[5], cw[6], cw[7]};
            } else {
                *(u32x4 *)dst = u32x4{cw[0], cw[1], cw[2], cw[3]};
            }
        }
    } else {
        if (r < ROWS) {
            uint8_t *row = sm_codes + r * kRowBytes + q * (kRowBytes / R);
            *(u32x4 *)row = u32x4{cw[0], cw[1], cw[2], cw[3]};
            if constexpr (kB8) *(u32x4 *)(row + 16) = u32x4{cw[4], cw[5], cw[6], cw[7]};
        }
        __syncthreads();
        write_value_tiles<kB8, D, ROWS>(codes, sm_codes, c0, pos, end, tid);
    }
}

template <int FMT, int IS_VALUE, int D, int LOAD>
__global__ __launch_bounds__(256) void append_rows_kernel(AppendArgs a) {
    rows_block<FMT, IS_VALUE, D, LOAD, 0, 256 / (D / 32)>(a, blockIdx.y, blockIdx.z, blockIdx.x);
}

template <int FMT, int IS_VALUE, int D>
inline void launch_rows_d(int load, dim3 grid, hipStream_t st, const AppendArgs &a) {
    if (load == kRowBF16)
        hipLaunchKernelGGL((append_rows_kernel<FMT, IS_VALUE, D, kRowBF16>), grid, dim3(256), 0, st, a);
    else if (load == kRowF16)
        hipLaunchKernelGGL((append_rows_kernel<FMT, IS_VALUE, D, kRowF16>), grid, dim3(256), 0, st, a);
    else if (load == kRowF32)
        hipLaunchKernelGGL((append_rows_kernel<FMT, IS_VALUE, D, kRowF32>), grid, dim3(256), 0, st, a);
    else
        hipLaunchKernelGGL((append_rows_kernel<FMT, IS_VALUE, D, kRowAny>), grid, dim3(256), 0, st, a);
}

// The MFMA-rotation form of the TurboMse append (append_turbo.hip); false when the case is not
// one it takes (then the row-parallel encoder runs).
bool turbo_mfma_launch(const cqkv_side *s, int32_t tokens, int32_t batch, hipStream_t st,
                       const AppendArgs &a);
// The MFMA form of the TurboProd key append (append_turbo.hip); false when it does not take the
// case.
bool prod_mfma_launch(const cqkv_side *s, int32_t tokens, int32_t batch, hipStream_t st,
                      const AppendArgs &a);

template <int FMT>
inline void launch_rows(const cqkv_side *s, int32_t tokens, int32_t batch, hipStream_t st,
                        const AppendArgs &a) {
    if constexpr (FMT == CQKV_FMT_TURBO4) {
        if (turbo_mfma_launch(s, tokens, batch, st, a)) return;
    }
    if constexpr (FMT == CQKV_FMT_TURBOPROD) {
        if (prod_mfma_launch(s, tokens, batch, st, a)) return;
    }
    const int dk = kernel_dim(s->head_dim);
    const int rows = 256 / (dk / 32);
    const dim3 grid((unsigned)(((int64_t)tokens + 7 + rows - 1) / rows), s->kv_heads, batch);
    if constexpr (FMT == CQKV_FMT_TURBOPROD) {  // keys only (check_side refuses value sides)
        if (dk == 64) launch_rows_d<FMT, 0, 64>(a.row_loads, grid, st, a);
        else if (dk == 128) launch_rows_d<FMT, 0, 128>(a.row_loads, grid, st, a);
        else launch_rows_d<FMT, 0, 256>(a.row_loads, grid, st, a);
    } else if (dk == 64) {
        if (s->is_value) launch_rows_d<FMT, 1, 64>(a.row_loads, grid, st, a);
        else launch_rows_d<FMT, 0, 64>(a.row_loads, grid, st, a);
    } else if (dk == 128) {
        if (s->is_value) launch_rows_d<FMT, 1, 128>(a.row_loads, grid, st, a);
        else launch_rows_d<FMT, 0, 128>(a.row_loads, grid, st, a);
    } else {
        if (s->is_value) launch_rows_d<FMT, 1, 256>(a.row_loads, grid, st, a);
        else launch_rows_d<FMT, 0, 256>(a.row_loads, grid, st, a);
    }
}

// ---------------------------------------------------------------------------------------------
// Fused RoPE + quantize-append: one launch rotates the queries (written out in their dtype for
// the attention call), rotates the keys and quantizes them into the key side, and quantizes the
// values into the value side. Grid ((tiles / 4) * units, 1, batch) with units = kv_heads +
// v_units + q_units: unit y < kv_heads is a key plane, the next v_units (kv_heads, or 0 when the
// value side has another format and its own launch) value planes, the rest query head units.
// ---------------------------------------------------------------------------------------------
struct RopeAppendArgs {
    AppendArgs k, v;  // k carries the cos / sin tables
    const void *q;
    void *q_out;
    int64_t qsb, qsh, qst, osb, osh, ost;  // element strides: batch, head, token
    int32_t q_pair_loads, o_pair_stores, q_heads;
    int32_t q_vec16;  // query rows by rope_query_rows16
    int32_t q_units;  // grid units of the queries: q_heads, or head groups with q_vec16
    int32_t v_units;  // grid units of the values: kv_heads, or 0 (values appended separately)
};

template <int D, int ROPE, bool W16>
__device__ inline void rope_query_rows(const RopeAppendArgs &r, int h, int b, int bx, int wave,
                                       int lane) {
    const AppendArgs &a = r.k;
    const int pos = a.positions ? a.positions[b] : a.position;
    const int i_lo = (bx * 4 + wave) * 8, i_hi = min(i_lo + 8, a.tokens);
    if (pos < 0) return;
    const bool active = lane < D / 2;
    const int64_t in0 = (int64_t)b * r.qsb + (int64_t)h * r.qsh + 2 * lane;
    const int64_t out0 = (int64_t)b * r.osb + (int64_t)h * r.osh + 2 * lane;
    const int i_end = min(i_hi, a.cs_rows - pos);
    const bool pair = W16 || r.q_pair_loads != 0, cs_pair = W16 || a.cs_pair_loads != 0;
    RawPair raw[8];
    RopeCS cs[8];
#pragma unroll
    for (int s = 0; s < 8; ++s) {
        const int i = i_lo + s;
        raw[s] = RawPair{0u, 0u};
        cs[s] = RopeCS{{0u, 0u}, {0u, 0u}};
        if (active && i < i_end) {
            raw[s] = load_raw_t<W16>(r.q, in0 + (int64_t)i * r.qst, a.x_dtype, pair);
            cs[s] = rope_load<D, ROPE, W16>(a.cos, a.sin, a.x_dtype, cs_pair, pos + i, lane);
        }
    }
#pragma unroll
    for (int s = 0; s < 8; ++s) {
        const int i = i_lo + s;
        if (i >= i_end) break;
        float x0, x1;
        raw_to_f32(raw[s], a.x_dtype, pair, x0, x1);
        rope_apply<D, ROPE>(x0, x1, cs[s], a.x_dtype, cs_pair, lane);
        if (!active) continue;
        const int64_t o = out0 + (int64_t)i * r.ost;
        if (r.o_pair_stores && a.x_dtype != CQKV_F32) {
            *(uint32_t *)((uint16_t *)r.q_out + o) =
                a.x_dtype == CQKV_BF16 ? pack_bf16x2(x0, x1) : pack_f16x2(x0, x1);
        } else {
            store_elem(r.q_out, o, a.x_dtype, x0);
            store_elem(r.q_out, o + 1, a.x_dtype, x1);
        }
    }
}

// Query rows with 16-byte lanes (16-bit dtype, rows and tables 16-byte aligned): lane l holds
// elements 8c..8c+7 (c = l % (D/8)) of head g * (64 / (D/8)) + l / (D/8), so one load covers
// 4 heads (D = 128) or 8 heads (D = 64) of a token and a lane's table chunk serves 8 elements.
// Halves: the partner chunk c ^ (D/16) sits in lane l ^ (D/16). A wave takes 8 tokens in two
// batches of 4 (all loads of a batch issued before its first conversion).
template <int D, int ROPE>
__device__ inline void rope_query_rows16(const RopeAppendArgs &r, int g, int b, int bx, int wave,
                                         int lane) {
#pragma clang fp contract(off)
    const AppendArgs &a = r.k;
    constexpr int LPR = D / 8, RPW = 64 / LPR;
    const int pos = a.positions ? a.positions[b] : a.position;
    if (pos < 0) return;
    const int h = g * RPW + lane / LPR, c = lane % LPR;
    const bool live = h < r.q_heads;
    const int i_lo = (bx * 4 + wave) * 8, i_end = min(min(i_lo + 8, a.tokens), a.cs_rows - pos);
    if (i_lo >= i_end) return;
    const uint16_t *qp = (const uint16_t *)r.q + (int64_t)b * r.qsb + (int64_t)h * r.qsh + 8 * c;
    uint16_t *op = (uint16_t *)r.q_out + (int64_t)b * r.osb + (int64_t)h * r.osh + 8 * c;
    const bool bf = a.x_dtype == CQKV_BF16;
    const bool upper = c >= LPR / 2;
    // table offset of this lane's elements in a row of D/2 entries
    const int tofs = ROPE == CQKV_ROPE_HALVES ? 8 * (c % (LPR / 2)) : 4 * c;
    auto f32_of = [bf](uint32_t bits16) {
        return bf ? bf16_bits_to_f32(bits16) : f16_bits_to_f32(bits16);
    };
#pragma unroll
    for (int s0 = 0; s0 < 8; s0 += 4) {
        u32x4 xv[4], cv[4], sv[4];
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const int i = i_lo + s0 + s;
            xv[s] = u32x4{0u, 0u, 0u, 0u};
            cv[s] = sv[s] = u32x4{0u, 0u, 0u, 0u};
            if (i < i_end) {
                const int64_t trow = (int64_t)(pos + i) * (D / 2) + tofs;
                if (live) xv[s] = *(const u32x4 *)(qp + (int64_t)i * r.qst);
                if constexpr (ROPE == CQKV_ROPE_HALVES) {
                    cv[s] = *(const u32x4 *)((const uint16_t *)a.cos + trow);
                    sv[s] = *(const u32x4 *)((const uint16_t *)a.sin + trow);
                } else {
                    const u32x2 c2 = *(const u32x2 *)((const uint16_t *)a.cos + trow);
                    const u32x2 s2 = *(const u32x2 *)((const uint16_t *)a.sin + trow);
                    cv[s] = u32x4{c2.x, c2.y, 0u, 0u};
                    sv[s] = u32x4{s2.x, s2.y, 0u, 0u};
                }
            }
        }
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const int i = i_lo + s0 + s;
            if (i >= i_end) break;
            float x[8], y[8];
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                x[2 * w] = f32_of(xv[s][w] & 0xffffu);
                x[2 * w + 1] = f32_of(xv[s][w] >> 16);
            }
            if constexpr (ROPE == CQKV_ROPE_HALVES) {
                u32x4 pv;
#pragma unroll
                for (int w = 0; w < 4; ++w)
                    pv[w] = (uint32_t)__shfl_xor((int)xv[s][w], LPR / 2, kWave);
#pragma unroll
                for (int w = 0; w < 4; ++w) {
#pragma unroll
                    for (int k = 0; k < 2; ++k) {
                        const uint32_t cb = k ? cv[s][w] >> 16 : cv[s][w] & 0xffffu;
                        const uint32_t sb = k ? sv[s][w] >> 16 : sv[s][w] & 0xffffu;
                        const float cc = f32_of(cb), ss = f32_of(sb);
                        const float p = f32_of(k ? pv[w] >> 16 : pv[w] & 0xffffu);
                        const float xe = x[2 * w + k];
                        y[2 * w + k] = upper ? p * ss + xe * cc : xe * cc - p * ss;
                    }
                }
            } else {
#pragma unroll
                for (int m = 0; m < 4; ++m) {
                    const uint32_t cw = cv[s][m >> 1], sw = sv[s][m >> 1];
                    const float cc = f32_of((m & 1) ? cw >> 16 : cw & 0xffffu);
                    const float ss = f32_of((m & 1) ? sw >> 16 : sw & 0xffffu);
                    y[2 * m] = x[2 * m] * cc - x[2 * m + 1] * ss;
                    y[2 * m + 1] = x[2 * m] * ss + x[2 * m + 1] * cc;
                }
            }
            if (!live) continue;
            u32x4 ov;
#pragma unroll
            for (int w = 0; w < 4; ++w)
                ov[w] = bf ? pack_bf16x2(y[2 * w], y[2 * w + 1]) : pack_f16x2(y[2 * w], y[2 * w + 1]);
            *(u32x4 *)(op + (int64_t)i * r.ost) = ov;
        }
    }
}

// Query rows of the halves layout with 16-byte lanes (16-bit dtype, rows and tables 16-byte
// aligned), the same head groups as rope_query_rows16 (64 / (D/8) heads): lane l holds elements
// 8c..8c+7 and D/2 + 8c..+7 (c = l % (D/16)) of head g * (64 / (D/8)) + (l / (D/16)) % (64 / (D/8))
// of token 2s + l / 32 of the pair s, so each pair of elements is in one lane (no exchange across
// lanes) and a lane's 16-byte cos / sin chunks serve 16 outputs. A wave takes its 8 tokens as four
// token pairs, every load issued before the first conversion. Products are rounded before the sum,
// as in rope_query_rows16. The query rows are read and written once: nontemporal loads and stores
// (config-4 shape 83.5 -> 74.4 us same-box; the same hint on the key / value row loads of
// rows_block measured slower, 89-90 us).
template <int D>
__device__ inline void rope_query_rows16h(const RopeAppendArgs &r, int g, int b, int bx, int wave,
                                          int lane) {
#pragma clang fp contract(off)
    const AppendArgs &a = r.k;
    constexpr int LPH = D / 16, RPW = 64 / (D / 8), HALF = D / 2;  // lanes per head, heads per group
    static_assert(LPH * RPW == 32, "a token's heads of the group take half the wave");
    const int pos = a.positions ? a.positions[b] : a.position;
    if (pos < 0) return;
    const int h = g * RPW + (lane / LPH) % RPW, c = lane % LPH, ts = lane >> 5;
    const bool live = h < r.q_heads;
    const int i_lo = (bx * 4 + wave) * 8, i_end = min(min(i_lo + 8, a.tokens), a.cs_rows - pos);
    if (i_lo >= i_end) return;
    const uint16_t *qp = (const uint16_t *)r.q + (int64_t)b * r.qsb + (int64_t)h * r.qsh + 8 * c;
    uint16_t *op = (uint16_t *)r.q_out + (int64_t)b * r.osb + (int64_t)h * r.osh + 8 * c;
    const bool bf = a.x_dtype == CQKV_BF16;
    auto f32_of = [bf](uint32_t bits16) {
        return bf ? bf16_bits_to_f32(bits16) : f16_bits_to_f32(bits16);
    };
    u32x4 xl[4], xh[4], cv[4], sv[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        const int i = i_lo + 2 * s + ts;
        xl[s] = xh[s] = cv[s] = sv[s] = u32x4{0u, 0u, 0u, 0u};
        if (i < i_end) {
            const int64_t trow = (int64_t)(pos + i) * HALF + 8 * c;
            cv[s] = *(const u32x4 *)((const uint16_t *)a.cos + trow);
            sv[s] = *(const u32x4 *)((const uint16_t *)a.sin + trow);
            if (live) {
                xl[s] = __builtin_nontemporal_load((const u32x4 *)(qp + (int64_t)i * r.qst));
                xh[s] = __builtin_nontemporal_load((const u32x4 *)(qp + (int64_t)i * r.qst + HALF));
            }
        }
    }
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        const int i = i_lo + 2 * s + ts;
        if (i >= i_end || !live) continue;
        u32x4 ol, oh;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            float lo[2], hi[2];
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                const float cc = f32_of(k ? cv[s][w] >> 16 : cv[s][w] & 0xffffu);
                const float ss = f32_of(k ? sv[s][w] >> 16 : sv[s][w] & 0xffffu);
                const float x0 = f32_of(k ? xl[s][w] >> 16 : xl[s][w] & 0xffffu);
                const float x1 = f32_of(k ? xh[s][w] >> 16 : xh[s][w] & 0xffffu);
                lo[k] = x0 * cc - x1 * ss;
                hi[k] = x0 * ss + x1 * cc;
            }
            ol[w] = bf ? pack_bf16x2(lo[0], lo[1]) : pack_f16x2(lo[0], lo[1]);
            oh[w] = bf ? pack_bf16x2(hi[0], hi[1]) : pack_f16x2(hi[0], hi[1]);
        }
        __builtin_nontemporal_store(ol, (u32x4 *)(op + (int64_t)i * r.ost));
        __builtin_nontemporal_store(oh, (u32x4 *)(op + (int64_t)i * r.ost + HALF));
    }
}

// Blocks of 64 tokens: key and value planes by the row-parallel encoder (the keys rotated after
// their load), query head groups as two 32-token halves.
constexpr int kRopeBlockTokens = 64;

template <int FMT, int D, int ROPE, int LOAD>
__global__ __launch_bounds__(256) void rope_append_kernel(RopeAppendArgs r) {
    // head index fastest in dispatch order: the blocks in flight together read whole projection
    // rows (all heads of the same tokens) instead of one head's pieces 12 KB apart
    const int hkv = r.k.kv_heads, qy = hkv + r.v_units, units = qy + r.q_units;
    const int y = (int)(blockIdx.x % (unsigned)units), bx = (int)(blockIdx.x / (unsigned)units);
    const int b = blockIdx.z, wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (y < hkv) {
        rows_block<FMT, 0, D, LOAD, ROPE, kRopeBlockTokens>(r.k, y, b, bx);
    } else if (y < qy) {
        // TurboProd keys always take values of another format, appended by their own launch
        if constexpr (FMT != CQKV_FMT_TURBOPROD)
            rows_block<FMT, 1, D, LOAD, 0, kRopeBlockTokens>(r.v, y - hkv, b, bx);
    } else {
#pragma unroll
        for (int k = 0; k < 2; ++k) {  // rope_query_rows* cover 32 tokens per block index
            if (LOAD != kRowF32 && r.q_vec16 && ROPE == CQKV_ROPE_HALVES)
                rope_query_rows16h<D>(r, y - qy, b, 2 * bx + k, wave, lane);
            else if (LOAD != kRowF32 && r.q_vec16)
                rope_query_rows16<D, ROPE>(r, y - qy, b, 2 * bx + k, wave, lane);
            else rope_query_rows<D, ROPE, false>(r, y - qy, b, 2 * bx + k, wave, lane);
        }
    }
}

template <int FMT, int ROPE, int LOAD>
inline void launch_rope_append_l(int d, dim3 grid, hipStream_t st, const RopeAppendArgs &r) {
    if (d == 64)
        hipLaunchKernelGGL((rope_append_kernel<FMT, 64, ROPE, LOAD>), grid, dim3(256), 0, st, r);
    else
        hipLaunchKernelGGL((rope_append_kernel<FMT, 128, ROPE, LOAD>), grid, dim3(256), 0, st, r);
}

template <int FMT, int ROPE>
inline void launch_rope_append(int d, dim3 grid, hipStream_t st, const RopeAppendArgs &r) {
    // one row-load form for both sides (the most general one when they differ)
    const int load = !r.v_units || r.k.row_loads == r.v.row_loads ? r.k.row_loads : kRowAny;
    if (load == kRowBF16) launch_rope_append_l<FMT, ROPE, kRowBF16>(d, grid, st, r);
    else if (load == kRowF16) launch_rope_append_l<FMT, ROPE, kRowF16>(d, grid, st, r);
    else if (load == kRowF32) launch_rope_append_l<FMT, ROPE, kRowF32>(d, grid, st, r);
    else launch_rope_append_l<FMT, ROPE, kRowAny>(d, grid, st, r);
}

template <int FMT>
inline void launch_rope_append_fmt(int rope, int d, dim3 grid, hipStream_t st,
                                   const RopeAppendArgs &r) {
    if (rope == CQKV_ROPE_INTERLEAVED) launch_rope_append<FMT, CQKV_ROPE_INTERLEAVED>(d, grid, st, r);
    else launch_rope_append<FMT, CQKV_ROPE_HALVES>(d, grid, st, r);
}

// Per-format launchers, defined in append_inst.hip (one object per format).
#define CQKV_APPEND_LAUNCHERS(F)                                                                  \
    void append_rows_launch_##F(const cqkv_side *s, int32_t tokens, int32_t batch, hipStream_t st, \
                                const AppendArgs &a);                                              \
    void rope_append_launch_##F(int rope, int d, dim3 grid, hipStream_t st, const RopeAppendArgs &r);
CQKV_APPEND_LAUNCHERS(0)
CQKV_APPEND_LAUNCHERS(1)
CQKV_APPEND_LAUNCHERS(2)
CQKV_APPEND_LAUNCHERS(3)
CQKV_APPEND_LAUNCHERS(4)
CQKV_APPEND_LAUNCHERS(5)

}  // namespace cqkv
