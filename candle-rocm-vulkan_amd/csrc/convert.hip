// Converters between the cache layout of include/cqkv.h and the reference's packed rows
// [codes][aux][rsc0][rsc1] (u32 words; candle-core/src/accel/formats.rs:206-242, written by
// RowCodec::quantize_row, candle-core/src/accel/turbo.rs:366-381):
//   FP8    D/4 code words (byte j = element j), rsc0 = f32 scale, rsc1 = 0
//   MXFP4  D/8 code words (nibble j = element j), ceil(D/32 / 4) aux words (byte b = E8M0 of
//          block b), rsc0 = 1.0, rsc1 = 0
//   TURBO4 D/8 code words, rsc0 = f32 norm, rsc1 = 0
//   MXFP8  D/4 code words, ceil(D/32 / 4) aux words (E8M0 bytes), rsc0 = 1.0, rsc1 = 0
//   NVFP4  D/8 code words, ceil(D/16 / 4) aux words (E4M3 block scales), rsc0 = f32 global
//          scale, rsc1 = 0
//   TURBO4 at bits b < 4 (TurboMse{b}): ceil(b D / 32) code words (b-bit codes, LSB first),
//          rsc0 = f32 norm, rsc1 = 0
//   TURBOPROD{b} (keys) ceil((b - 1) D / 32) code words ((b - 1)-bit codes, LSB first), D/32 aux
//          words (the QJL sign bits), rsc0 = f32 norm, rsc1 = f32 |r|
// The cache keeps TurboQuant codes of every width as nibbles.
// One wavefront per 8-token tile of a (batch, head) plane; lane l owns elements 2l, 2l+1, so
// the value tiles are read and written whole by one lane (no cross-lane read-modify-write).
#include <algorithm>

#include "cqkv_device.h"
#include "cqkv_host.h"

namespace cqkv {

struct ConvertArgs {
    uint32_t *rows;  // (batch, kv_heads, tokens, row_words)
    uint8_t *codes, *scales;
    uint32_t codes_plane, scales_plane;
    int32_t kv_heads, tokens, position, row_words, format, is_value;
    int32_t dk;           // plane row length (64, 128, 256)
    int32_t dim;          // head dim (<= dk): the reference row's elements
    int32_t b8;           // 8-bit codes (FP8, MXFP8), else 4-bit
    int32_t nblk;         // block scale bytes per token in the plane (MX, NVFP4), else 0
    int32_t nblk_ref;     // ... in the reference row (blocks of the head dim)
    int32_t tok_scale;    // an f32 per token (FP8, TURBO4, NVFP4), after the block bytes
    int32_t capacity;
    int32_t cbits;        // TurboQuant codes packed at cbits < 4 per element, or TURBOPROD; else 0
};

// One workgroup of max(64, dk / 2) threads per 8-token tile of a (batch, head) plane; thread l
// owns elements 2l, 2l+1 of the plane row, so the value tiles are read and written whole by one
// thread (no cross-thread read-modify-write). Elements past the head dim are zero codes in the
// plane and absent from the reference row (whose last code / sign word is zero-filled).
template <bool EXPORT>
__global__ __launch_bounds__(128) void convert_kernel(ConvertArgs a) {
    const int lane = threadIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int D = a.dk, dim = a.dim;
    const int tile = a.position / 8 + (int)blockIdx.x;
    const int t_lo = max(tile * 8, a.position), t_hi = min(tile * 8 + 8, a.position + a.tokens);
    if (t_lo >= t_hi) return;
    const bool active = lane < D / 2;
    const bool fp8 = a.b8 != 0;  // 8-bit code layout
    const int64_t plane = (int64_t)b * a.kv_heads + h;
    uint8_t *codes = a.codes + plane * a.codes_plane;
    uint8_t *scales = a.scales + plane * a.scales_plane;
    const int code_words = fp8 ? (dim + 3) / 4 : (dim + 7) / 8;
    const int nb = a.nblk, nbr = a.nblk_ref, aux_words = (nbr + 3) / 4;
    float *tscale = (float *)(scales + (int64_t)a.capacity * nb);
    const bool in0 = 2 * lane < dim, in1 = 2 * lane + 1 < dim;  // real elements of this thread

    // value tile words of this thread (elements 2l, 2l+1)
    uint64_t vw0 = 0, vw1 = 0;
    uint32_t vn0 = 0, vn1 = 0;
    if (a.is_value && active) {
        if (fp8) {
            const uint64_t *src = (const uint64_t *)(codes + (int64_t)tile * D * 8 + 2 * lane * 8);
            vw0 = src[0];
            vw1 = src[1];
        } else {
            const uint32_t *src = (const uint32_t *)(codes + (int64_t)tile * D * 4 + 2 * lane * 4);
            vn0 = src[0];
            vn1 = src[1];
        }
    }
    if (a.cbits) {  // TurboQuant codes of cbits < 4 bits, or TURBOPROD: nibbles <-> packed bits
        __shared__ uint8_t sm_c[256];
        const int cb = a.cbits, cw = (dim * cb + 31) / 32;
        const bool prod = a.format == CQKV_FMT_TURBOPROD;
        const int sw = prod ? (dim + 31) / 32 : 0;  // sign words of the reference row
        // TurboProd: |r| and the sign words follow the norms (TurboMse sides end at the norms)
        const float *r1 = (const float *)(scales + (int64_t)a.capacity * 4);
        uint32_t *signs = (uint32_t *)(scales + (int64_t)a.capacity * 8);
        const int swp = prod ? D / 32 : 0;  // sign words per token in the plane
        const uint32_t mask = (1u << cb) - 1u;
        // sign bits of the last reference word past the head dim are zero
        const uint32_t last_mask = dim % 32 ? (1u << (dim % 32)) - 1u : ~0u;
        for (int t = t_lo; t < t_hi; ++t) {
            uint32_t *row = a.rows + ((plane * a.tokens) + (t - a.position)) * (int64_t)a.row_words;
            const int s = t & 7;
            if (EXPORT) {
                if (active) {  // this thread's codes of elements 2 lane, 2 lane + 1
                    uint32_t c0, c1;
                    if (!a.is_value) {
                        const uint32_t by = codes[(int64_t)t * (D / 2) + lane];
                        c0 = by & 15u;
                        c1 = by >> 4;
                    } else {
                        c0 = (vn0 >> (4 * s)) & 15u;
                        c1 = (vn1 >> (4 * s)) & 15u;
                    }
                    sm_c[2 * lane] = (uint8_t)(c0 & mask);
                    sm_c[2 * lane + 1] = (uint8_t)(c1 & mask);
                }
                __syncthreads();
                if (lane < cw) {  // word `lane`: bits [32 lane, 32 lane + 32) of the packed codes
                    uint32_t w = 0;
                    const int j0 = (32 * lane) / cb, j1 = min((32 * lane + 31) / cb, dim - 1);
                    for (int j = j0; j <= j1; ++j) {
                        const uint32_t c = sm_c[j];
                        const int bit = cb * j - 32 * lane;  // -(cb - 1) .. 31
                        w |= bit >= 0 ? c << bit : c >> (-bit);
                    }
                    row[lane] = w;
                }
                __syncthreads();
                if (lane < sw) {
                    const uint32_t w = signs[(int64_t)t * swp + lane];
                    row[cw + lane] = lane == sw - 1 ? w & last_mask : w;
                }
                if (lane == 0) {
                    row[cw + sw] = __float_as_uint(tscale[t]);
                    row[cw + sw + 1] = prod ? __float_as_uint(r1[t]) : 0u;
                }
            } else {
                if (active) {  // elements 2 lane, 2 lane + 1
                    uint32_t c[2];
                    for (int e = 0; e < 2; ++e) {
                        c[e] = 0;
                        if (2 * lane + e >= dim) continue;
                        const int pos = cb * (2 * lane + e);
                        const uint64_t two = (uint64_t)row[pos >> 5] |
                                             ((pos >> 5) + 1 < cw ? (uint64_t)row[(pos >> 5) + 1] << 32 : 0ull);
                        c[e] = (uint32_t)(two >> (pos & 31)) & mask;
                    }
                    if (!a.is_value) {
                        codes[(int64_t)t * (D / 2) + lane] = (uint8_t)(c[0] | (c[1] << 4));
                    } else {
                        vn0 = (vn0 & ~(15u << (4 * s))) | (c[0] << (4 * s));
                        vn1 = (vn1 & ~(15u << (4 * s))) | (c[1] << (4 * s));
                    }
                }
                if (prod && lane < swp) {  // only TurboProd sides have a sign area
                    const uint32_t w = lane < sw ? row[cw + lane] : 0u;
                    signs[(int64_t)t * swp + lane] = lane == sw - 1 ? w & last_mask : w;
                }
                if (lane == 0) {
                    tscale[t] = __uint_as_float(row[cw + sw]);
                    if (prod) ((float *)r1)[t] = __uint_as_float(row[cw + sw + 1]);
                }
            }
        }
        if (!EXPORT && a.is_value && active) {
            uint32_t *dst = (uint32_t *)(codes + (int64_t)tile * D * 4 + 2 * lane * 4);
            dst[0] = vn0;
            dst[1] = vn1;
        }
        return;
    }
    for (int t = t_lo; t < t_hi; ++t) {
        uint32_t *row = a.rows + ((plane * a.tokens) + (t - a.position)) * (int64_t)a.row_words;
        uint8_t *rowb = (uint8_t *)row;
        const int s = t & 7;
        if (active) {
            if (EXPORT) {
                uint32_t c0, c1;
                if (!a.is_value) {
                    if (fp8) {
                        c0 = codes[(int64_t)t * D + 2 * lane];
                        c1 = codes[(int64_t)t * D + 2 * lane + 1];
                    } else {
                        const uint32_t by = codes[(int64_t)t * (D / 2) + lane];
                        c0 = by & 15u;
                        c1 = by >> 4;
                    }
                } else if (fp8) {
                    c0 = (uint32_t)(vw0 >> (8 * s)) & 0xffu;
                    c1 = (uint32_t)(vw1 >> (8 * s)) & 0xffu;
                } else {
                    c0 = (vn0 >> (4 * s)) & 15u;
                    c1 = (vn1 >> (4 * s)) & 15u;
                }
                if (!in0) c0 = 0;  // the zero fill of the last code word
                if (!in1) c1 = 0;
                // bytes of the code words only (past them lie the aux and scale words)
                if (fp8) {
                    if (2 * lane < 4 * code_words) rowb[2 * lane] = (uint8_t)c0;
                    if (2 * lane + 1 < 4 * code_words) rowb[2 * lane + 1] = (uint8_t)c1;
                } else if (lane < 4 * code_words) {
                    rowb[lane] = (uint8_t)(c0 | (c1 << 4));
                }
            } else {
                uint32_t c0 = 0, c1 = 0;
                if (fp8) {
                    if (in0) c0 = rowb[2 * lane];
                    if (in1) c1 = rowb[2 * lane + 1];
                } else {
                    if (in0) c0 = rowb[lane] & 15u;
                    if (in1) c1 = rowb[lane] >> 4;
                }
                if (!a.is_value) {
                    if (fp8) {
                        codes[(int64_t)t * D + 2 * lane] = (uint8_t)c0;
                        codes[(int64_t)t * D + 2 * lane + 1] = (uint8_t)c1;
                    } else {
                        codes[(int64_t)t * (D / 2) + lane] = (uint8_t)(c0 | (c1 << 4));
                    }
                } else if (fp8) {
                    vw0 = (vw0 & ~(0xffull << (8 * s))) | ((uint64_t)c0 << (8 * s));
                    vw1 = (vw1 & ~(0xffull << (8 * s))) | ((uint64_t)c1 << (8 * s));
                } else {
                    vn0 = (vn0 & ~(15u << (4 * s))) | (c0 << (4 * s));
                    vn1 = (vn1 & ~(15u << (4 * s))) | (c1 << (4 * s));
                }
            }
        }
        if (lane == 0) {
            uint32_t *aux = row + code_words;
            uint32_t *rsc = aux + aux_words;
            if (EXPORT) {
                for (int w = 0; w < aux_words; ++w) aux[w] = 0;
                for (int k = 0; k < nbr; ++k)
                    aux[k >> 2] |= (uint32_t)scales[(int64_t)t * nb + k] << (8 * (k & 3));
                rsc[0] = a.tok_scale ? __float_as_uint(tscale[t]) : __float_as_uint(1.0f);
                rsc[1] = 0;
            } else {
                for (int k = 0; k < nb; ++k)  // blocks past the head dim: zero scales
                    scales[(int64_t)t * nb + k] = k < nbr ? (uint8_t)(aux[k >> 2] >> (8 * (k & 3))) : 0;
                if (a.tok_scale) tscale[t] = __uint_as_float(rsc[0]);
            }
        }
    }
    if (!EXPORT && a.is_value && active) {
        if (fp8) {
            uint64_t *dst = (uint64_t *)(codes + (int64_t)tile * D * 8 + 2 * lane * 8);
            dst[0] = vw0;
            dst[1] = vw1;
        } else {
            uint32_t *dst = (uint32_t *)(codes + (int64_t)tile * D * 4 + 2 * lane * 4);
            dst[0] = vn0;
            dst[1] = vn1;
        }
    }
}

static int convert(const cqkv_side *side, uint32_t *rows, int32_t batch, int32_t tokens,
                   int32_t position, hipStream_t st, bool to_rows, const char *what) {
    clear_error();
    if (int rc = check_side(side, what)) return rc;
    if (!rows) return fail(CQKV_ERR_ARG, "%s: null rows", what);
    if (batch <= 0 || tokens < 0 || position < 0 || (int64_t)position + tokens > side->capacity)
        return fail(CQKV_ERR_ARG, "%s: batch %d, tokens [%d, %d) outside the capacity %d", what,
                    batch, position, position + tokens, side->capacity);
    if (tokens == 0) return CQKV_OK;
    ConvertArgs a = {};
    a.rows = rows;
    a.codes = (uint8_t *)side->codes;
    a.scales = (uint8_t *)side->scales;
    a.codes_plane = (uint32_t)cqkv_codes_plane_bytes(side->format, side->head_dim, side->capacity);
    a.scales_plane = (uint32_t)cqkv_scales_plane_bytes(side->format, side->head_dim, side->capacity);
    a.kv_heads = side->kv_heads;
    a.tokens = tokens;
    a.position = position;
    a.row_words = cqkv_reference_row_words(side->format, side->bits, side->head_dim);
    a.format = side->format;
    a.b8 = code_bits(side->format) == 8 ? 1 : 0;
    a.tok_scale = token_scale(side->format) ? 1 : 0;
    a.capacity = side->capacity;
    a.is_value = side->is_value;
    a.dim = side->head_dim;
    a.dk = kernel_dim(side->head_dim);
    a.nblk = block_elems(side->format) ? a.dk / block_elems(side->format) : 0;
    a.nblk_ref = block_elems(side->format) ? a.dim / block_elems(side->format) : 0;
    a.cbits = side->format == CQKV_FMT_TURBOPROD || turbo_code_bits(side) < 4 ? turbo_code_bits(side) : 0;
    dim3 grid((tokens + 7) / 8 + 1, side->kv_heads, batch);
    const dim3 block(a.dk == 256 ? 128 : 64);
    if (to_rows) hipLaunchKernelGGL(convert_kernel<true>, grid, block, 0, st, a);
    else hipLaunchKernelGGL(convert_kernel<false>, grid, block, 0, st, a);
    CQKV_HIP_CHECK(hipGetLastError());
    return CQKV_OK;
}

}  // namespace cqkv

extern "C" int cqkv_rows_import(const cqkv_side *side, const uint32_t *rows, int32_t batch,
                                int32_t tokens, int32_t position, cqkv_stream_t stream) {
    return cqkv::convert(side, const_cast<uint32_t *>(rows), batch, tokens, position,
                         (hipStream_t)stream, false, "cqkv_rows_import");
}

extern "C" int cqkv_rows_export(const cqkv_side *side, uint32_t *rows, int32_t batch,
                                int32_t tokens, int32_t position, cqkv_stream_t stream) {
    return cqkv::convert(side, rows, batch, tokens, position, (hipStream_t)stream, true,
                         "cqkv_rows_export");
}

// ---------------------------------------------------------------------------------------------
// Cache growth: the first `tokens` positions of every (batch, kv head) plane of src into dst,
// sides of different capacities (Cache::append's copy of the old contents into the grown buffer,
// candle-nn/src/kv_cache.rs:56-99). A codes plane is a prefix of whole rows (keys) or whole
// 8-token tiles (values); a scales plane holds the block-scale bytes of all `capacity` tokens,
// then the f32 token scales, so it is two prefixes at capacity-dependent offsets. Each region is
// one strided device copy over all planes (no kernel, nothing allocated).
// ---------------------------------------------------------------------------------------------
extern "C" int cqkv_side_copy(const cqkv_side *dst, const cqkv_side *src, int32_t batch,
                              int32_t tokens, cqkv_stream_t stream) {
    using namespace cqkv;
    clear_error();
    static const char *who = "cqkv_side_copy";
    if (int rc = check_side(dst, who)) return rc;
    if (int rc = check_side(src, who)) return rc;
    if (dst->format != src->format || dst->is_value != src->is_value ||
        dst->head_dim != src->head_dim || dst->kv_heads != src->kv_heads ||
        side_rotation(dst) != side_rotation(src) || side_bits(dst) != side_bits(src) ||
        ((side_rotates(src) || src->format == CQKV_FMT_TURBOPROD) && dst->seed != src->seed))
        return fail(CQKV_ERR_ARG,
                    "%s: sides differ in format, bits, side, head dim, kv heads, rotation or seed", who);
    if (batch <= 0 || tokens < 0 || tokens > src->capacity || tokens > dst->capacity)
        return fail(CQKV_ERR_ARG, "%s: batch %d, %d tokens for capacities %d -> %d", who, batch,
                    tokens, src->capacity, dst->capacity);
    if (tokens == 0) return CQKV_OK;
    const int fmt = src->format, d = kernel_dim(src->head_dim);  // the plane row length
    const size_t planes = (size_t)batch * src->kv_heads;
    const size_t row_bytes = (size_t)d * code_bits(fmt) / 8;
    // values: whole 8-token tiles, at most the smaller capacity (both are multiples of 32)
    const int ctok = src->is_value ? std::min((tokens + 7) / 8 * 8, std::min(src->capacity, dst->capacity))
                                   : tokens;
    const size_t src_cp = cqkv_codes_plane_bytes(fmt, src->head_dim, src->capacity);
    const size_t dst_cp = cqkv_codes_plane_bytes(fmt, src->head_dim, dst->capacity);
    const size_t src_sp = cqkv_scales_plane_bytes(fmt, src->head_dim, src->capacity);
    const size_t dst_sp = cqkv_scales_plane_bytes(fmt, src->head_dim, dst->capacity);
    const size_t bb = block_elems(fmt) ? (size_t)d / block_elems(fmt) : 0;  // block bytes per token
    const hipStream_t st = (hipStream_t)stream;
    CQKV_HIP_CHECK(hipMemcpy2DAsync(dst->codes, dst_cp, src->codes, src_cp, row_bytes * ctok,
                                    planes, hipMemcpyDeviceToDevice, st));
    if (bb)
        CQKV_HIP_CHECK(hipMemcpy2DAsync(dst->scales, dst_sp, src->scales, src_sp, bb * tokens,
                                        planes, hipMemcpyDeviceToDevice, st));
    if (token_scale(fmt))
        CQKV_HIP_CHECK(hipMemcpy2DAsync((uint8_t *)dst->scales + bb * dst->capacity, dst_sp,
                                        (const uint8_t *)src->scales + bb * src->capacity, src_sp,
                                        (size_t)4 * tokens, planes, hipMemcpyDeviceToDevice, st));
    if (fmt == CQKV_FMT_TURBOPROD) {  // |r| and the sign bits behind the norms
        CQKV_HIP_CHECK(hipMemcpy2DAsync((uint8_t *)dst->scales + 4 * (size_t)dst->capacity, dst_sp,
                                        (const uint8_t *)src->scales + 4 * (size_t)src->capacity,
                                        src_sp, (size_t)4 * tokens, planes,
                                        hipMemcpyDeviceToDevice, st));
        CQKV_HIP_CHECK(hipMemcpy2DAsync((uint8_t *)dst->scales + 8 * (size_t)dst->capacity, dst_sp,
                                        (const uint8_t *)src->scales + 8 * (size_t)src->capacity,
                                        src_sp, (size_t)(d / 8) * tokens, planes,
                                        hipMemcpyDeviceToDevice, st));
    }
    return CQKV_OK;
}
