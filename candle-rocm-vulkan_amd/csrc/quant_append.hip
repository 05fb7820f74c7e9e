// KV quantize-and-append into the FP8 / MXFP4 / MXFP8 / NVFP4 / TURBO4 cache layouts (gfx950).
//
// Reference behaviour (paths relative to the reference repository root):
//   RowCodec::quantize_row, candle-core/src/accel/turbo.rs:293-381 (FP8 366-374, MX 324-347,
//   TurboMse 299-323) after TurboQuantizer::rotate (candle-nn/src/turbo_quant.rs:182-189), then
//   Cache::append (candle-nn/src/kv_cache.rs:68-99). One launch here replaces the reference's
//   cast + rotation matmul + tq_quant + slice_set copy.
//
// Work split: one wavefront per 8-token tile of one (batch, kv head) plane. Lane l owns elements
// 2l and 2l+1 of every row (D = 128: all 64 lanes; D = 64: lanes 0..31). Per token the wave
// reduces the row (FP8: absmax over the wave; MXFP4: absmax over the 16 lanes of a 32-element
// block; TURBO4: in-register Walsh-Hadamard transform then sum of squares), encodes its two
// elements and stores them; key rows go straight to their row-major place, value codes are
// gathered in registers for the whole tile and stored once in the token-transposed layout.
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
    uint32_t sign_bits[4];  // TURBO4: bit j set -> column j of the rotation has sign -1
    float rot_scale;        // TURBO4: 1 / sqrt(D) in f32
    float bnd[16];          // TURBO4: the 15 codebook boundaries (+inf padded)
    int32_t pair_loads;     // elements 2l, 2l+1 of every row are one aligned 4 / 8-byte word
    const void *cos, *sin;  // rotary tables (cs_rows, D/2) in the dtype of x (fused RoPE only)
    int32_t cs_rows;        // fused RoPE: rows of the tables, positions past them are skipped
                            // (keys and values alike); 0 for a plain append
    int32_t cs_pair_loads;  // both tables aligned for paired loads
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

// One wave: the tokens of one 8-token cache tile of plane (b, h), bx / wave as in the grid of
// quant_append_launch. ROPE != 0 rotates each row (position = its cache position) first.
template <int FMT, int IS_VALUE, int D, int ROPE, bool W16>
__device__ inline void append_tile(const AppendArgs &a, int h, int b, int bx, int wave, int lane) {
    const int pos = a.positions ? a.positions[b] : a.position;
    const int tile = pos / 8 + bx * 4 + wave;
    const int t_lo = max(tile * 8, pos);
    int t_hi = min(min(tile * 8 + 8, pos + a.tokens), a.capacity);
    // the fused RoPE call skips positions past its cos / sin tables on both sides, so a K / V
    // slot is written for both or neither (cs_rows is 0 for a plain append)
    if (a.cs_rows > 0) t_hi = min(t_hi, a.cs_rows);
    if (pos < 0 || t_lo >= t_hi) return;

    const bool active = lane < D / 2;
    const int64_t plane = (int64_t)b * a.kv_heads + h;
    uint8_t *codes = a.codes + plane * a.codes_plane;
    uint8_t *scales = a.scales + plane * a.scales_plane;
    const int64_t xrow0 = (int64_t)b * a.sb + (int64_t)h * a.sh;

    // value tile words owned by this lane: elements 2l and 2l+1 of the 8 tokens
    uint64_t vw0 = 0, vw1 = 0;      // FP8: 8 code bytes per element
    uint32_t vn0 = 0, vn1 = 0;      // 4-bit: 8 code nibbles per element
    uint32_t new_mask = 0;          // tokens of this tile written by this call (bit t % 8)

    const bool pair = W16 || a.pair_loads != 0, cs_pair = W16 || a.cs_pair_loads != 0;
    constexpr bool kB8 = FMT == CQKV_FMT_FP8 || FMT == CQKV_FMT_MXFP8;  // byte codes
    // encodes one token (x0, x1) at cache position t, tile slot `slot`
    auto encode = [&](float x0, float x1, int t, int slot) {
        uint32_t c0, c1;
        float row_scale = 0.0f;
        if constexpr (FMT == CQKV_FMT_FP8) {
            const float amax = wave_max(fmaxf(__builtin_fabsf(x0), __builtin_fabsf(x1)));
            const float s = amax > 0.0f ? amax / 448.0f : 1.0f;
            const float r = 1.0f / s;
            const uint32_t c01 = fp8_row_codes(x0, x1, s, r);
            c0 = c01 & 0xffu;
            c1 = c01 >> 8;
            row_scale = s;
        } else if constexpr (FMT == CQKV_FMT_MXFP4 || FMT == CQKV_FMT_MXFP8) {
            // E8M0 per 32 elements: floor_log2(amax) - emax of the element format (turbo.rs:324-347)
            constexpr bool kFp4 = FMT == CQKV_FMT_MXFP4;
            const float amax = group_max(fmaxf(__builtin_fabsf(x0), __builtin_fabsf(x1)), 16);
            const uint32_t sc = mx_scale_code(amax, kFp4 ? 2 : 8);
            const float scale = e8m0_to_f32(sc);
            if constexpr (kFp4) {
                c0 = sc == 0 ? 0u : fp4_encode(x0 / scale);
                c1 = sc == 0 ? 0u : fp4_encode(x1 / scale);
            } else {
                c0 = sc == 0 ? 0u : e4m3_encode(x0 / scale);
                c1 = sc == 0 ? 0u : e4m3_encode(x1 / scale);
            }
            if (active && (lane & 15) == 0) scales[(int64_t)t * (D / 32) + lane / 16] = (uint8_t)sc;
        } else if constexpr (FMT == CQKV_FMT_NVFP4) {
            // g = row absmax / 2688 (= 448 * 6); per 16 elements an E4M3 scale of bmax / 6 / g;
            // codes E2M1 of x / (e4m3(cs) * g) (turbo.rs:348-365)
            const float ax = fmaxf(__builtin_fabsf(x0), __builtin_fabsf(x1));
            const float amax = wave_max(ax);
            const float gs = amax > 0.0f ? amax / 2688.0f : 1.0f;
            const float bmax = group_max(ax, 8);
            const uint32_t cs = e4m3_encode(bmax / 6.0f / gs);
            const float eff = __builtin_amdgcn_cvt_f32_fp8(cs, 0) * gs;
            c0 = eff > 0.0f ? fp4_encode(x0 / eff) : 0u;
            c1 = eff > 0.0f ? fp4_encode(x1 / eff) : 0u;
            if (active && (lane & 7) == 0) scales[(int64_t)t * (D / 16) + lane / 8] = (uint8_t)cs;
            row_scale = gs;
        } else {  // TURBO4: y = H (sign * x) / sqrt(D), norm, codebook index of y / norm
            const int j0 = 2 * lane, j1 = 2 * lane + 1;
            if (active) {
                if ((a.sign_bits[j0 >> 5] >> (j0 & 31)) & 1u) x0 = -x0;
                if ((a.sign_bits[j1 >> 5] >> (j1 & 31)) & 1u) x1 = -x1;
            }
            fwht_pairs<D>(x0, x1, lane);
            const float y0 = x0 * a.rot_scale, y1 = x1 * a.rot_scale;
            const float ss = wave_sum(active ? y0 * y0 + y1 * y1 : 0.0f);
            const float norm = __builtin_sqrtf(ss);
            const float inv = norm > 0.0f ? 1.0f / norm : 0.0f;
            const float u0 = y0 * inv, u1 = y1 * inv;
            c0 = 0;
            c1 = 0;
#pragma unroll
            for (int i = 0; i < 15; ++i) {
                c0 += u0 >= a.bnd[i] ? 1u : 0u;
                c1 += u1 >= a.bnd[i] ? 1u : 0u;
            }
            row_scale = norm;
        }
        if constexpr (FMT == CQKV_FMT_FP8 || FMT == CQKV_FMT_TURBO4 || FMT == CQKV_FMT_NVFP4) {
            // the per-token f32 follows the block bytes of all `capacity` tokens
            constexpr int kBlockBytes = FMT == CQKV_FMT_NVFP4 ? D / 16 : 0;
            if (lane == 0) ((float *)(scales + (int64_t)a.capacity * kBlockBytes))[t] = row_scale;
        }
        new_mask |= 1u << slot;
        if (!active) return;
        if constexpr (!IS_VALUE) {
            if constexpr (kB8)
                *(uint16_t *)(codes + (int64_t)t * D + 2 * lane) = (uint16_t)(c0 | (c1 << 8));
            else
                codes[(int64_t)t * (D / 2) + lane] = (uint8_t)(c0 | (c1 << 4));
        } else {
            if constexpr (kB8) {
                vw0 |= (uint64_t)c0 << (8 * slot);
                vw1 |= (uint64_t)c1 << (8 * slot);
            } else {
                vn0 |= c0 << (4 * slot);
                vn1 |= c1 << (4 * slot);
            }
        }
    };
    for (int t = t_lo; t < t_hi; ++t) {
        RawPair raw = {0u, 0u};
        RopeCS cs = {{0u, 0u}, {0u, 0u}};
        if (active) {
            raw = load_raw_t<W16>(a.x, xrow0 + (int64_t)(t - pos) * a.st + 2 * lane,
                                  a.x_dtype, pair);
            if constexpr (ROPE != 0)
                cs = rope_load<D, ROPE, W16>(a.cos, a.sin, a.x_dtype, cs_pair, t, lane);
        }
        float x0, x1;
        raw_to_f32(raw, a.x_dtype, pair, x0, x1);
        if constexpr (ROPE != 0) rope_apply<D, ROPE>(x0, x1, cs, a.x_dtype, cs_pair, lane);
        encode(x0, x1, t, t & 7);
    }
    if constexpr (IS_VALUE) {
        if (!active) return;
        if constexpr (kB8) {
            uint64_t *dst = (uint64_t *)(codes + (int64_t)tile * D * 8 + 2 * lane * 8);
            if (new_mask != 0xffu) {  // keep the codes of tokens this call does not write
                uint64_t keep = 0;
                for (int s = 0; s < 8; ++s)
                    if (!((new_mask >> s) & 1u)) keep |= 0xffull << (8 * s);
                vw0 |= dst[0] & keep;
                vw1 |= dst[1] & keep;
            }
            dst[0] = vw0;
            dst[1] = vw1;
        } else {
            uint32_t *dst = (uint32_t *)(codes + (int64_t)tile * D * 4 + 2 * lane * 4);
            if (new_mask != 0xffu) {
                uint32_t keep = 0;
                for (int s = 0; s < 8; ++s)
                    if (!((new_mask >> s) & 1u)) keep |= 0xfu << (4 * s);
                vn0 |= dst[0] & keep;
                vn1 |= dst[1] & keep;
            }
            dst[0] = vn0;
            dst[1] = vn1;
        }
    }
}

template <int FMT, int IS_VALUE, int D, bool W16>
__global__ __launch_bounds__(256) void quant_append_kernel(AppendArgs a) {
    append_tile<FMT, IS_VALUE, D, 0, W16>(a, blockIdx.y, blockIdx.z, blockIdx.x, threadIdx.x >> 6,
                                     threadIdx.x & 63);
}

template <int FMT, int IS_VALUE, bool W16>
static void launch_append_w(int d, dim3 grid, hipStream_t st, const AppendArgs &a) {
    if (d == 64)
        hipLaunchKernelGGL((quant_append_kernel<FMT, IS_VALUE, 64, W16>), grid, dim3(256), 0, st, a);
    else
        hipLaunchKernelGGL((quant_append_kernel<FMT, IS_VALUE, 128, W16>), grid, dim3(256), 0, st, a);
}

template <int FMT, int IS_VALUE>
static void launch_append_dim(int d, dim3 grid, hipStream_t st, const AppendArgs &a) {
    if (a.x_dtype != CQKV_F32 && a.pair_loads) launch_append_w<FMT, IS_VALUE, true>(d, grid, st, a);
    else launch_append_w<FMT, IS_VALUE, false>(d, grid, st, a);
}

template <int FMT>
static void launch_append(const cqkv_side *s, dim3 grid, hipStream_t st, const AppendArgs &a) {
    if (s->is_value) launch_append_dim<FMT, 1>(s->head_dim, grid, st, a);
    else launch_append_dim<FMT, 0>(s->head_dim, grid, st, a);
}

// Fills the TURBO4 fields of `a` for a side (signs from the side's seed, codebook of its D).
int fill_turbo_args(const cqkv_side *s, uint32_t sign_bits[4], float *rot_scale, float bnd[16]) {
    float signs[128], cent[16];
    turbo_signs(s->head_dim, s->seed, signs);
    for (int i = 0; i < 4; ++i) sign_bits[i] = 0;
    for (int j = 0; j < s->head_dim; ++j)
        if (signs[j] < 0.0f) sign_bits[j >> 5] |= 1u << (j & 31);
    *rot_scale = 1.0f / sqrtf((float)s->head_dim);
    for (int i = 0; i < 16; ++i) bnd[i] = __builtin_inff();
    if (turbo_codebook(s->head_dim, 4, cent, bnd) != 0)
        return fail(CQKV_ERR_ARG, "turbo codebook for D=%d", s->head_dim);
    return CQKV_OK;
}

// Elements 2l, 2l+1 of every row form one aligned 4- / 8-byte word.
static bool pair_aligned(const int64_t s[3], const void *p, int32_t dtype) {
    const size_t esz = dtype == CQKV_F32 ? 4 : 2;
    return s[0] % 2 == 0 && s[1] % 2 == 0 && s[2] % 2 == 0 && ((uintptr_t)p % (2 * esz)) == 0;
}

// Fills the append fields of `a` for one side and input x (shared by both entry points).
static int fill_append_args(AppendArgs &a, const cqkv_side *side, const void *x,
                            int32_t x_dtype, const int64_t xs[3], int32_t tokens,
                            const int32_t *positions, int32_t position) {
    a.x = x;
    a.x_dtype = x_dtype;
    a.sb = xs[0];
    a.sh = xs[1];
    a.st = xs[2];
    a.pair_loads = pair_aligned(xs, x, x_dtype) ? 1 : 0;
    a.codes = (uint8_t *)side->codes;
    a.scales = (uint8_t *)side->scales;
    a.codes_plane = (uint32_t)cqkv_codes_plane_bytes(side->format, side->head_dim, side->capacity);
    a.scales_plane = (uint32_t)cqkv_scales_plane_bytes(side->format, side->head_dim, side->capacity);
    a.positions = positions;
    a.position = position;
    a.tokens = tokens;
    a.capacity = side->capacity;
    a.kv_heads = side->kv_heads;
    if (side->format == CQKV_FMT_TURBO4) return fill_turbo_args(side, a.sign_bits, &a.rot_scale, a.bnd);
    return CQKV_OK;
}

// Launch used by cqkv_quant_append and by the prefill's fused append.
int quant_append_launch(const cqkv_side *side, const void *x, int32_t x_dtype,
                        const int64_t xs[3], int32_t batch, int32_t tokens,
                        const int32_t *positions, int32_t position, hipStream_t stream) {
    AppendArgs a = {};
    if (int rc = fill_append_args(a, side, x, x_dtype, xs, tokens, positions, position)) return rc;
    const int tiles = (tokens + 7) / 8 + 1;  // an unaligned start spans one more tile
    dim3 grid((tiles + 3) / 4, side->kv_heads, batch);
    switch (side->format) {
    case CQKV_FMT_FP8: launch_append<CQKV_FMT_FP8>(side, grid, stream, a); break;
    case CQKV_FMT_MXFP4: launch_append<CQKV_FMT_MXFP4>(side, grid, stream, a); break;
    case CQKV_FMT_MXFP8: launch_append<CQKV_FMT_MXFP8>(side, grid, stream, a); break;
    case CQKV_FMT_NVFP4: launch_append<CQKV_FMT_NVFP4>(side, grid, stream, a); break;
    default: launch_append<CQKV_FMT_TURBO4>(side, grid, stream, a); break;
    }
    CQKV_HIP_CHECK(hipGetLastError());
    return CQKV_OK;
}

// ---------------------------------------------------------------------------------------------
// Fused RoPE + quantize-append: one launch rotates the queries (written out in their dtype for
// the attention call), rotates the keys and quantizes them into the key side, and quantizes the
// values into the value side. Grid ((tiles / 4) * units, 1, batch) with units = 2 * kv_heads +
// q_heads: unit y < kv_heads is a key plane, the next kv_heads value planes, the rest query heads.
// ---------------------------------------------------------------------------------------------
struct RopeAppendArgs {
    AppendArgs k, v;  // k carries the cos / sin tables
    const void *q;
    void *q_out;
    int64_t qsb, qsh, qst, osb, osh, ost;  // element strides: batch, head, token
    int32_t q_pair_loads, o_pair_stores, q_heads;
    int32_t q_vec16;  // query rows by rope_query_rows16
    int32_t q_units;  // grid units of the queries: q_heads, or head groups with q_vec16
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

template <int FMT, int D, int ROPE, bool W16>
__global__ __launch_bounds__(256) void rope_append_kernel(RopeAppendArgs r) {
    // head index fastest in dispatch order: the blocks in flight together read whole projection
    // rows (all heads of the same tokens) instead of one head's 256-byte pieces 12 KB apart
    const int hkv = r.k.kv_heads, units = 2 * hkv + r.q_units;
    const int y = (int)(blockIdx.x % (unsigned)units), bx = (int)(blockIdx.x / (unsigned)units);
    const int b = blockIdx.z, wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (y < hkv) append_tile<FMT, 0, D, ROPE, W16>(r.k, y, b, bx, wave, lane);
    else if (y < 2 * hkv) append_tile<FMT, 1, D, 0, W16>(r.v, y - hkv, b, bx, wave, lane);
    else if (W16 && r.q_vec16) rope_query_rows16<D, ROPE>(r, y - 2 * hkv, b, bx, wave, lane);
    else rope_query_rows<D, ROPE, W16>(r, y - 2 * hkv, b, bx, wave, lane);
}

template <int FMT, int ROPE, bool W16>
static void launch_rope_append_w(int d, dim3 grid, hipStream_t st, const RopeAppendArgs &r) {
    if (d == 64)
        hipLaunchKernelGGL((rope_append_kernel<FMT, 64, ROPE, W16>), grid, dim3(256), 0, st, r);
    else
        hipLaunchKernelGGL((rope_append_kernel<FMT, 128, ROPE, W16>), grid, dim3(256), 0, st, r);
}

template <int FMT, int ROPE>
static void launch_rope_append(int d, dim3 grid, hipStream_t st, const RopeAppendArgs &r) {
    const bool w16 = r.k.x_dtype != CQKV_F32 && r.k.pair_loads && r.v.pair_loads &&
                     r.q_pair_loads && r.k.cs_pair_loads;
    if (w16) launch_rope_append_w<FMT, ROPE, true>(d, grid, st, r);
    else launch_rope_append_w<FMT, ROPE, false>(d, grid, st, r);
}

template <int FMT>
static void launch_rope_append_fmt(int rope, int d, dim3 grid, hipStream_t st,
                                   const RopeAppendArgs &r) {
    if (rope == CQKV_ROPE_INTERLEAVED) launch_rope_append<FMT, CQKV_ROPE_INTERLEAVED>(d, grid, st, r);
    else launch_rope_append<FMT, CQKV_ROPE_HALVES>(d, grid, st, r);
}

}  // namespace cqkv

extern "C" int cqkv_rope_quant_append(const cqkv_side *k_side, const cqkv_side *v_side,
                                      const void *q, const int64_t q_strides[3], const void *k,
                                      const int64_t k_strides[3], const void *v,
                                      const int64_t v_strides[3], int32_t dtype, int32_t batch,
                                      int32_t tokens, int32_t q_heads, const void *cos,
                                      const void *sin, int32_t cs_rows, int32_t rope_kind,
                                      const int32_t *positions, int32_t position, void *q_out,
                                      const int64_t q_out_strides[3], cqkv_stream_t stream) {
    using namespace cqkv;
    clear_error();
    static const char *who = "cqkv_rope_quant_append";
    if (int rc = check_side(k_side, who)) return rc;
    if (int rc = check_side(v_side, who)) return rc;
    if (k_side->is_value || !v_side->is_value)
        return fail(CQKV_ERR_ARG, "%s: k_side must be a key side and v_side a value side", who);
    if (k_side->format != v_side->format || k_side->head_dim != v_side->head_dim ||
        k_side->kv_heads != v_side->kv_heads || k_side->capacity != v_side->capacity)
        return fail(CQKV_ERR_ARG, "%s: key / value sides differ in format, D, heads or capacity", who);
    if (!q || !k || !v || !q_out || !q_strides || !k_strides || !v_strides || !q_out_strides ||
        !cos || !sin)
        return fail(CQKV_ERR_ARG, "%s: null pointer argument", who);
    if (dtype < CQKV_BF16 || dtype > CQKV_F32) return fail(CQKV_ERR_ARG, "%s: dtype %d", who, dtype);
    if (rope_kind != CQKV_ROPE_HALVES && rope_kind != CQKV_ROPE_INTERLEAVED)
        return fail(CQKV_ERR_ARG, "%s: rope kind %d", who, rope_kind);
    const int hkv = k_side->kv_heads;
    if (batch <= 0 || tokens < 0 || q_heads <= 0 || q_heads % hkv != 0)
        return fail(CQKV_ERR_ARG, "%s: batch %d tokens %d q_heads %d kv_heads %d", who, batch,
                    tokens, q_heads, hkv);
    if (cs_rows <= 0) return fail(CQKV_ERR_ARG, "%s: cos / sin rows %d", who, cs_rows);
    if (tokens == 0) return CQKV_OK;
    if (!positions) {
        const int64_t end = (int64_t)position + tokens;
        if (position < 0 || end > k_side->capacity)
            return fail(CQKV_ERR_ARG, "%s: positions [%d, %lld) exceed the capacity %d", who,
                        position, (long long)end, k_side->capacity);
        if (end > cs_rows)
            return fail(CQKV_ERR_ARG, "%s: positions [%d, %lld) exceed the %d cos / sin rows", who,
                        position, (long long)end, cs_rows);
    }
    RopeAppendArgs r = {};
    if (int rc = fill_append_args(r.k, k_side, k, dtype, k_strides, tokens, positions, position)) return rc;
    if (int rc = fill_append_args(r.v, v_side, v, dtype, v_strides, tokens, positions, position)) return rc;
    r.k.cos = cos;
    r.k.sin = sin;
    r.k.cs_rows = cs_rows;
    r.v.cs_rows = cs_rows;
    {
        const uintptr_t al = dtype == CQKV_F32 ? 8 : 4;
        r.k.cs_pair_loads = ((uintptr_t)cos % al == 0 && (uintptr_t)sin % al == 0) ? 1 : 0;
    }
    r.q = q;
    r.q_out = q_out;
    r.qsb = q_strides[0];
    r.qsh = q_strides[1];
    r.qst = q_strides[2];
    r.osb = q_out_strides[0];
    r.osh = q_out_strides[1];
    r.ost = q_out_strides[2];
    r.q_pair_loads = pair_aligned(q_strides, q, dtype) ? 1 : 0;
    r.o_pair_stores = pair_aligned(q_out_strides, q_out, dtype) ? 1 : 0;
    r.q_heads = q_heads;
    {
        auto al16 = [](const void *p, const int64_t st[3]) {
            return (uintptr_t)p % 16 == 0 && st[0] % 8 == 0 && st[1] % 8 == 0 && st[2] % 8 == 0;
        };
        r.q_vec16 = dtype != CQKV_F32 && al16(q, q_strides) && al16(q_out, q_out_strides) &&
                    (uintptr_t)cos % 16 == 0 && (uintptr_t)sin % 16 == 0 ? 1 : 0;
        const int rpw = 64 / (k_side->head_dim / 8);  // heads per 16-byte-lane load
        r.q_units = r.q_vec16 ? (q_heads + rpw - 1) / rpw : q_heads;
    }
    const int64_t tiles = ((int64_t)tokens + 7) / 8 + 1;  // an unaligned start spans one more tile
    const int64_t blocks = (tiles + 3) / 4 * (2 * hkv + r.q_units);
    if (blocks * 256 > (int64_t)UINT32_MAX)  // threads along x of one launch
        return fail(CQKV_ERR_ARG, "%s: %d tokens x %d heads exceed one launch", who, tokens,
                    2 * hkv + q_heads);
    dim3 grid((uint32_t)blocks, 1, batch);
    const hipStream_t st = (hipStream_t)stream;
    const int d = k_side->head_dim;
    switch (k_side->format) {
    case CQKV_FMT_FP8: launch_rope_append_fmt<CQKV_FMT_FP8>(rope_kind, d, grid, st, r); break;
    case CQKV_FMT_MXFP4: launch_rope_append_fmt<CQKV_FMT_MXFP4>(rope_kind, d, grid, st, r); break;
    case CQKV_FMT_MXFP8: launch_rope_append_fmt<CQKV_FMT_MXFP8>(rope_kind, d, grid, st, r); break;
    case CQKV_FMT_NVFP4: launch_rope_append_fmt<CQKV_FMT_NVFP4>(rope_kind, d, grid, st, r); break;
    default: launch_rope_append_fmt<CQKV_FMT_TURBO4>(rope_kind, d, grid, st, r); break;
    }
    CQKV_HIP_CHECK(hipGetLastError());
    return CQKV_OK;
}

extern "C" int cqkv_quant_append(const cqkv_side *side, const void *x, int32_t x_dtype,
                                 const int64_t x_strides[3], int32_t batch, int32_t tokens,
                                 const int32_t *positions, int32_t position,
                                 cqkv_stream_t stream) {
    using namespace cqkv;
    clear_error();
    if (int rc = check_side(side, "cqkv_quant_append")) return rc;
    if (!x || !x_strides) return fail(CQKV_ERR_ARG, "cqkv_quant_append: null x / strides");
    if (x_dtype < CQKV_BF16 || x_dtype > CQKV_F32)
        return fail(CQKV_ERR_ARG, "cqkv_quant_append: x dtype %d", x_dtype);
    if (batch <= 0 || tokens < 0) return fail(CQKV_ERR_ARG, "cqkv_quant_append: batch %d tokens %d", batch, tokens);
    if (tokens == 0) return CQKV_OK;
    if (!positions && (position < 0 || (int64_t)position + tokens > side->capacity))
        return fail(CQKV_ERR_ARG, "cqkv_quant_append: positions [%d, %d) exceed the capacity %d",
                    position, position + tokens, side->capacity);
    return quant_append_launch(side, x, x_dtype, x_strides, batch, tokens, positions, position,
                               (hipStream_t)stream);
}
