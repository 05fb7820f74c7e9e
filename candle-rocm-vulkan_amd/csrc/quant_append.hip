// KV quantize-and-append into the FP8 / MXFP4 / TURBO4 cache layouts (gfx950).
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
};

// elements idx, idx + 1 of x as floats (one load when `pair` says they form an aligned word)
__device__ inline void load_pair(const void *p, int64_t idx, int dtype, bool pair, float &x0,
                                 float &x1) {
    if (pair) {
        if (dtype == 2) {
            const f32x2 w = *(const f32x2 *)((const float *)p + idx);
            x0 = w.x;
            x1 = w.y;
        } else {
            const uint32_t w = *(const uint32_t *)((const uint16_t *)p + idx);
            x0 = dtype == 0 ? bf16_bits_to_f32(w & 0xffffu) : f16_bits_to_f32(w & 0xffffu);
            x1 = dtype == 0 ? bf16_bits_to_f32(w >> 16) : f16_bits_to_f32(w >> 16);
        }
    } else {
        x0 = load_elem(p, idx, dtype);
        x1 = load_elem(p, idx + 1, dtype);
    }
}

// In-register Walsh-Hadamard transform over 2 * `lanes` elements held as (v0, v1) = elements
// (2l, 2l+1): y_i = sum_j (-1)^popcount(i & j) x_j (Sylvester order, unnormalised).
template <int D>
__device__ inline void fwht_pairs(float &v0, float &v1, int lane) {
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

template <int FMT, int IS_VALUE, int D>
__global__ __launch_bounds__(256) void quant_append_kernel(AppendArgs a) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int h = blockIdx.y, b = blockIdx.z;
    const int pos = a.positions ? a.positions[b] : a.position;
    const int tile = pos / 8 + (int)blockIdx.x * 4 + wave;
    const int t_lo = max(tile * 8, pos);
    const int t_hi = min(min(tile * 8 + 8, pos + a.tokens), a.capacity);
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

    for (int t = t_lo; t < t_hi; ++t) {
        float x0 = 0.0f, x1 = 0.0f;
        if (active)
            load_pair(a.x, xrow0 + (int64_t)(t - pos) * a.st + 2 * lane, a.x_dtype,
                      a.pair_loads != 0, x0, x1);
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
        } else if constexpr (FMT == CQKV_FMT_MXFP4) {
            const float amax = group_max(fmaxf(__builtin_fabsf(x0), __builtin_fabsf(x1)), 16);
            const uint32_t sc = mx_scale_code(amax, 2);
            const float scale = e8m0_to_f32(sc);
            c0 = sc == 0 ? 0u : fp4_encode(x0 / scale);
            c1 = sc == 0 ? 0u : fp4_encode(x1 / scale);
            if (active && (lane & 15) == 0) scales[(int64_t)t * (D / 32) + lane / 16] = (uint8_t)sc;
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
        if constexpr (FMT != CQKV_FMT_MXFP4) {
            if (lane == 0) ((float *)scales)[t] = row_scale;
        }
        const int slot = t & 7;
        new_mask |= 1u << slot;
        if (!active) continue;
        if constexpr (!IS_VALUE) {
            if constexpr (FMT == CQKV_FMT_FP8)
                *(uint16_t *)(codes + (int64_t)t * D + 2 * lane) = (uint16_t)(c0 | (c1 << 8));
            else
                codes[(int64_t)t * (D / 2) + lane] = (uint8_t)(c0 | (c1 << 4));
        } else {
            if constexpr (FMT == CQKV_FMT_FP8) {
                vw0 |= (uint64_t)c0 << (8 * slot);
                vw1 |= (uint64_t)c1 << (8 * slot);
            } else {
                vn0 |= c0 << (4 * slot);
                vn1 |= c1 << (4 * slot);
            }
        }
    }
    if constexpr (IS_VALUE) {
        if (!active) return;
        if constexpr (FMT == CQKV_FMT_FP8) {
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

template <int FMT, int IS_VALUE>
static void launch_append_dim(int d, dim3 grid, hipStream_t st, const AppendArgs &a) {
    if (d == 64)
        hipLaunchKernelGGL((quant_append_kernel<FMT, IS_VALUE, 64>), grid, dim3(256), 0, st, a);
    else
        hipLaunchKernelGGL((quant_append_kernel<FMT, IS_VALUE, 128>), grid, dim3(256), 0, st, a);
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

// Launch used by cqkv_quant_append and by the prefill's fused append.
int quant_append_launch(const cqkv_side *side, const void *x, int32_t x_dtype,
                        const int64_t xs[3], int32_t batch, int32_t tokens,
                        const int32_t *positions, int32_t position, hipStream_t stream) {
    AppendArgs a = {};
    a.x = x;
    a.x_dtype = x_dtype;
    a.sb = xs[0];
    a.sh = xs[1];
    a.st = xs[2];
    {
        const size_t esz = x_dtype == CQKV_F32 ? 4 : 2;
        a.pair_loads = (xs[0] % 2 == 0 && xs[1] % 2 == 0 && xs[2] % 2 == 0 &&
                        ((uintptr_t)x % (2 * esz)) == 0) ? 1 : 0;
    }
    a.codes = (uint8_t *)side->codes;
    a.scales = (uint8_t *)side->scales;
    a.codes_plane = (uint32_t)cqkv_codes_plane_bytes(side->format, side->head_dim, side->capacity);
    a.scales_plane = (uint32_t)cqkv_scales_plane_bytes(side->format, side->head_dim, side->capacity);
    a.positions = positions;
    a.position = position;
    a.tokens = tokens;
    a.capacity = side->capacity;
    a.kv_heads = side->kv_heads;
    if (side->format == CQKV_FMT_TURBO4) {
        const int rc = fill_turbo_args(side, a.sign_bits, &a.rot_scale, a.bnd);
        if (rc) return rc;
    }
    const int tiles = (tokens + 7) / 8 + 1;  // an unaligned start spans one more tile
    dim3 grid((tiles + 3) / 4, side->kv_heads, batch);
    switch (side->format) {
    case CQKV_FMT_FP8: launch_append<CQKV_FMT_FP8>(side, grid, stream, a); break;
    case CQKV_FMT_MXFP4: launch_append<CQKV_FMT_MXFP4>(side, grid, stream, a); break;
    default: launch_append<CQKV_FMT_TURBO4>(side, grid, stream, a); break;
    }
    CQKV_HIP_CHECK(hipGetLastError());
    return CQKV_OK;
}

}  // namespace cqkv

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
