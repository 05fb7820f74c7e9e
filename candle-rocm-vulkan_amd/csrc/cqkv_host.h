// Host-side helpers shared by the C-ABI entry points: per-thread error text, side checks,
// plane sizes.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "../../include/cqkv.h"

namespace cqkv {

void set_error(const std::string &msg);
void clear_error();

// Formats an error, stores it for cqkv_last_error() and returns `code`.
int fail(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));

#define CQKV_HIP_CHECK(expr)                                                                   \
    do {                                                                                       \
        hipError_t e_ = (expr);                                                                \
        if (e_ != hipSuccess)                                                                  \
            return ::cqkv::fail(CQKV_ERR_HIP, "%s failed: %s", #expr, hipGetErrorString(e_)); \
    } while (0)

// Code bits per element, or 0 for an unknown format.
inline int code_bits(int32_t format) {
    switch (format) {
    case CQKV_FMT_FP8:
    case CQKV_FMT_MXFP8: return 8;
    case CQKV_FMT_MXFP4:
    case CQKV_FMT_NVFP4:
    case CQKV_FMT_TURBO4:
    case CQKV_FMT_TURBOPROD: return 4;  // TURBOPROD: 3-bit codes stored as nibbles
    default: return 0;
    }
}

// Elements per block scale (MX: E8M0 per 32, NVFP4: E4M3 per 16), 0 without block scales.
inline int block_elems(int32_t format) {
    return format == CQKV_FMT_MXFP4 || format == CQKV_FMT_MXFP8 ? 32
           : format == CQKV_FMT_NVFP4                           ? 16
                                                                : 0;
}

// Formats with an f32 scale per token (FP8 absmax/448, TurboQuant norm, NVFP4 global scale);
// in the scales plane it follows the block-scale bytes of all `capacity` tokens.
inline bool token_scale(int32_t format) {
    return format == CQKV_FMT_FP8 || format == CQKV_FMT_TURBO4 || format == CQKV_FMT_NVFP4 ||
           format == CQKV_FMT_TURBOPROD;
}

// TurboQuant formats (codebook codes of the rotated unit row times its norm).
inline bool is_turbo(int32_t format) {
    return format == CQKV_FMT_TURBO4 || format == CQKV_FMT_TURBOPROD;
}

// Plane row length of head dim d: the smallest of 64, 128, 256 that holds it (0 past 256). The
// kernels are instantiated at these lengths; elements past d are zero codes.
inline int kernel_dim(int32_t d) { return d < 1 ? 0 : d <= 64 ? 64 : d <= 128 ? 128 : d <= 256 ? 256 : 0; }

// Head dims a cache side of `format` takes: 1-256 (the reference's fused attention bound,
// FA_MAX_HEAD_DIM), MX formats a multiple of 32 and NVFP4 of 16 (QuantFormat::validate,
// candle-core/src/accel/formats.rs:166-187).
inline bool supported_dim(int32_t format, int32_t d) {
    if (d < 1 || d > 256) return false;
    if ((format == CQKV_FMT_MXFP4 || format == CQKV_FMT_MXFP8) && d % 32 != 0) return false;
    if (format == CQKV_FMT_NVFP4 && d % 16 != 0) return false;
    return true;
}

// TurboQuant width of a side (QuantFormat::TurboMse{bits} / TurboProd{bits}; 0 selects 4), 0 for
// the other formats.
// K / V element type of the f32-query attention beyond the CQKV_* dtypes: E4M3 codes (the FP8
// K / V path with f32 queries).
constexpr int kKvE4M3 = 3;

inline int side_bits(const cqkv_side *s) {
    return is_turbo(s->format) ? (s->bits ? s->bits : 4) : 0;
}
// Bits of a TurboQuant side's codebook codes (TurboProd: bits - 1), 0 for the other formats.
// The cache stores them as nibbles whatever the width.
inline int turbo_code_bits(const cqkv_side *s) {
    return s->format == CQKV_FMT_TURBOPROD ? side_bits(s) - 1 : side_bits(s);
}

// RotationKind::resolve (candle-core/src/accel/config.rs:131-138) of a side's rotation at head
// dim d: CQKV_ROT_NONE, CQKV_ROT_HADAMARD or CQKV_ROT_DENSE; DEFAULT is AUTO for the TurboQuant
// formats and NONE for the others; -1 for an unknown kind.
inline int resolve_rotation(int32_t format, int32_t kind, int32_t d) {
    const bool pow2 = d > 0 && (d & (d - 1)) == 0;
    switch (kind) {
    case CQKV_ROT_DEFAULT:
        return is_turbo(format) ? (pow2 ? CQKV_ROT_HADAMARD : CQKV_ROT_DENSE) : CQKV_ROT_NONE;
    case CQKV_ROT_NONE: return CQKV_ROT_NONE;
    case CQKV_ROT_AUTO:
    case CQKV_ROT_HADAMARD: return pow2 ? CQKV_ROT_HADAMARD : CQKV_ROT_DENSE;
    case CQKV_ROT_DENSE: return CQKV_ROT_DENSE;
    default: return -1;
    }
}
inline int side_rotation(const cqkv_side *s) { return resolve_rotation(s->format, s->rotation, s->head_dim); }

// The side's rows are rotated before quantization.
inline bool side_rotates(const cqkv_side *s) {
    const int r = side_rotation(s);
    return r == CQKV_ROT_HADAMARD || r == CQKV_ROT_DENSE;
}
// ... by the in-register Walsh-Hadamard transform (a Hadamard side whose head dim is a plane row
// length); the other rotating sides multiply by their matrix cqkv_side.rot.
inline bool side_fwht(const cqkv_side *s) {
    return side_rotation(s) == CQKV_ROT_HADAMARD && s->head_dim == kernel_dim(s->head_dim);
}
inline bool side_matrix_rot(const cqkv_side *s) { return side_rotates(s) && !side_fwht(s); }
// The side's rows reach the encoders through the f32 staging pass (rowmat.hip): rotation by the
// matrix, or a head dim shorter than the plane row (zero padding).
inline bool side_staged(const cqkv_side *s) {
    return side_matrix_rot(s) || s->head_dim != kernel_dim(s->head_dim);
}

// Validates a cache side; returns CQKV_OK or an error (message set).
int check_side(const cqkv_side *s, const char *what);

// Host tables of the TurboQuant format (see cqkv.h).
int turbo_codebook(int dim, int bits, float *centroids, float *boundaries);
void turbo_signs(int dim, uint64_t seed, float *signs);
void qjl_matrix(int dim, uint64_t seed, float *out);
void rotation_matrix(int dim, int kind, uint64_t seed, float *out);

// The dense / variable-length flash attention (prefill_attn.hip) behind cqkv_flash_attn_ext and
// the FP8 K / V path: dtype is q's and out's, kv_dtype K's and V's (dtype itself, or with f32
// queries CQKV_F16 / CQKV_BF16 / kKvE4M3); q_mul / o_mul and their device factors are the FP8
// descales (1 / null otherwise).
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
                    const float *q_mul_dev, float o_mul, const float *o_mul_dev);
size_t flash_attn_workspace(int32_t dtype, int32_t batch, int32_t q_len, int32_t kv_len,
                            int32_t q_heads, int32_t kv_heads, int32_t head_dim, bool varlen);
// Whether a dense call of these queries / output takes the MFMA prefill (bf16 / f16, D = 128,
// more than 16 queries, 16-byte aligned q rows, 8-byte aligned out rows), and the workspace of
// such a call over E4M3 K / V (V^T and the widened K).
bool prefill_takes(int32_t dtype, int32_t head_dim, int32_t q_len, const void *q,
                   const int64_t q_strides[3], const void *out, const int64_t out_strides[3]);
size_t prefill_e4m3_workspace(int32_t batch, int32_t kv_len, int32_t kv_heads);

// Plain-dtype attention (flash_plain.hip): argument checks, workspace, bytes per K / V element.
int fa_plain_check(const char *who, int32_t dtype, int32_t kv_dtype, int32_t head_dim,
                   int64_t k_row_stride, int64_t v_row_stride, int64_t kv_len);
size_t fa_plain_workspace_bytes(int32_t batch, int32_t q_len, int32_t kv_len, int32_t q_heads,
                                int32_t kv_heads, int32_t head_dim, bool ragged);
int fa_kv_esz(int32_t kv_dtype);

}  // namespace cqkv
