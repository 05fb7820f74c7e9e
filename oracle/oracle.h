/*
 * CPU oracle of the quantized-KV attention path: a plain-C restatement of the reference's CPU
 * algorithms (codecs, row quantizers, TurboQuant rotation and codebook, the unfused attention
 * and the split combine). TEST INFRASTRUCTURE ONLY: tests, the smoke check and bench.py's
 * cpu_baseline leg may call it as the checker; the product library never links or loads it.
 *
 * Every function names the reference file:line it follows (paths relative to the reference
 * repository root). Parity status of each function is listed in oracle/README.md.
 */
#ifndef CQKV_ORACLE_H
#define CQKV_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Format ids: the kernel mode ids of candle-core/src/accel/formats.rs:41-48. */
enum { ORC_TURBO_MSE = 0, ORC_TURBO_PROD = 1, ORC_MXFP4 = 2, ORC_NVFP4 = 3, ORC_MXFP8 = 4, ORC_FP8 = 5 };
/* Rotation kinds (candle-core/src/accel/config.rs RotationKind, resolved). */
enum { ORC_ROT_NONE = 0, ORC_ROT_HADAMARD = 1, ORC_ROT_DENSE = 2 };

/* ---- SplitMix64 + Box-Muller (candle-core/src/accel/turbo.rs:150-176) ---- */
uint64_t orc_splitmix_next(uint64_t *state);
double orc_splitmix_f64(uint64_t *state);
double orc_splitmix_normal(uint64_t *state);
/* n values of `next_normal() as f32` from SplitMix64::new(seed). */
void orc_fill_normal(uint64_t seed, float *out, size_t n);

/* ---- 16-bit floats (half 2.7 bf16 / f16, round to nearest even) ---- */
uint16_t orc_f32_to_bf16(float f);
float orc_bf16_to_f32(uint16_t b);

/* ---- element codecs (candle-core/src/accel/formats.rs:248-407) ---- */
float orc_pow2i(int e);
int orc_floor_log2(float a);
float orc_e4m3_to_f32(uint8_t c);
uint8_t orc_f32_to_e4m3(float f);
float orc_fp4_to_f32(uint32_t c);
uint32_t orc_f32_to_fp4(float f);
float orc_e8m0_to_f32(uint8_t c);
uint8_t orc_mx_scale_code(float amax, int emax_elem);
uint32_t orc_get_bits(const uint32_t *words, size_t pos, uint32_t bits);
void orc_put_bits(uint32_t *words, size_t pos, uint32_t bits, uint32_t v);

/* ---- row layout (formats.rs:206-242). Returns 0, or -1 for an invalid format/dim. ---- */
typedef struct {
    int dim, code_bits, code_words, aux_words, row_words;
} orc_layout;
int orc_row_layout(int mode, int bits, int dim, orc_layout *out);

/* ---- TurboQuant codebook (turbo.rs:58-129): 2^bits centroids, 2^bits - 1 boundaries ---- */
int orc_lloyd_max(int dim, int bits, float *centroids, float *boundaries);

/* ---- rotation matrix Π, row-major dim x dim (turbo.rs:180-233) ---- */
int orc_rotation_matrix(int dim, int kind, uint64_t seed, float *m);
/* y = x Πᵀ (turbo_quant.rs:182-189), rows x dim, sequential f32 sums over j. */
void orc_rotate_rows(const float *pi, int dim, const float *x, size_t rows, float *y);
/* x = y Π (turbo_quant.rs:191-196). */
void orc_unrotate_rows(const float *pi, int dim, const float *y, size_t rows, float *x);

/* ---- row codec (turbo.rs:293-424) ----
 * TurboProd: qjl = the row-major dim x dim QJL matrix S (turbo.rs:236-239), or NULL for the
 * codec without it (RowCodec::without_qjl, turbo.rs:273-286: codes and norm only). */
typedef struct {
    int mode, bits;
    orc_layout l;
    float centroids[16];
    float boundaries[16];
    const float *qjl;
} orc_codec;
/* S = SplitMix64((seed + 1) ^ 0x514a4c5f534b4554) normals, row-major dim x dim (turbo.rs:236-239). */
void orc_qjl_matrix(int dim, uint64_t seed, float *s);
/* TurboProd{bits} rows with the QJL matrix s (quantize: y already rotated). */
int orc_quantize_rows_qjl(int bits, int dim, size_t rows, const float *y, const float *s, uint32_t *out,
                          int threads);
int orc_dequantize_rows_qjl(int bits, int dim, size_t rows, const uint32_t *words, const float *s,
                            float *out, int threads);
int orc_codec_init(orc_codec *c, int mode, int bits, int dim);
void orc_quantize_row(const orc_codec *c, const float *y, uint32_t *out);
float orc_elem(const orc_codec *c, const uint32_t *row, int j);
void orc_dequantize_row(const orc_codec *c, const uint32_t *row, float *out);
/* rows x dim (already rotated) -> rows x row_words, `threads` worker threads (0 = 1). */
int orc_quantize_rows(int mode, int bits, int dim, size_t rows, const float *y, uint32_t *out, int threads);
int orc_dequantize_rows(int mode, int bits, int dim, size_t rows, const uint32_t *words, float *out, int threads);

/* ---- masks (candle-core/src/accel/attention.rs:80-92) ---- */
void orc_key_range(int64_t i, int64_t lq, int64_t lk, int wl, int wr, int64_t *lo, int64_t *hi);

/* ---- attention ----
 * Unfused CPU path (candle-nn/src/flash_attn.rs:930-1000 with ops.rs:315-352 softmax):
 *   q: (b, hq, lq, d) f32, k / v: (b, hkv, lk, d) f32 (already converted to the query dtype),
 *   out: (b, hq, lq, d) f32. Mask -1e30, ALiBi slopes (hq) when non-null, rows with no visible
 *   key give zeros. kv_lens (b) overrides lk per batch when non-null (keys [0, kv_lens[b]) of the
 *   lk-capacity K/V are attended, bottom-right aligned against kv_lens[b]).
 */
int orc_attention_unfused(const float *q, const float *k, const float *v, int b, int hq, int hkv,
                          int lq, int lk, int d, const int32_t *kv_lens, float scale, float softcap,
                          int wl, int wr, const float *alibi, float *out, int threads);

/* The reference's CPU decode path over packed rows (turbo_quant.rs:948-990 then
 * flash_attn.rs:930-1000): dequantize K/V rows (b, hkv, cap, row_words), unrotate, round to
 * bf16 (the appended dtype), attend with bf16 queries q (b, hq, lq, d) given as bf16 bits.
 * pi_k / pi_v: rotation matrices or NULL; softcap / alibi (per-head slopes or NULL) as in
 * orc_attention_unfused. Output f32 (b, hq, lq, d) (round to bf16 to compare). */
int orc_cache_attention(const uint16_t *q_bf16, const uint32_t *k_rows, const uint32_t *v_rows,
                        int k_mode, int k_bits, int v_mode, int v_bits, const float *pi_k,
                        const float *pi_v, const float *qjl_k, int b, int hq, int hkv, int lq,
                        int cap, int d, const int32_t *kv_lens, int lk, float scale, int wl, int wr,
                        float softcap, const float *alibi, float *out, int threads);

/* Split combine (candle-core/kernels/turbo_quant_impl.h:659-685). part_o (splits, rows, d),
 * part_lse (splits, rows). */
void orc_combine(const float *part_o, const float *part_lse, float *o, size_t rows, int d, int splits);

/* Split rules of the reference (candle-core/src/accel/attention.rs:486-506, 586-592). */
/* vectorised encoders (exhaustive sweeps in the tests) */
void orc_e4m3_encode_n(const float *x, uint8_t *out, size_t n);
void orc_fp4_encode_n(const float *x, uint8_t *out, size_t n);

int orc_split_count_grouped(size_t rows, int group, size_t lk, int policy_fixed, int compute_units);
int orc_row_group(int hq, int hkv);

#ifdef __cplusplus
}
#endif
#endif
