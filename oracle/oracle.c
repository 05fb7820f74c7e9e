/*
 * CPU oracle of the quantized-KV attention path (TEST INFRASTRUCTURE: only tests, the smoke
 * check and bench.py's cpu_baseline leg use it, as the checker). Restates the reference's CPU
 * algorithms in plain C; every function cites the reference file:line it follows. Built with
 * -ffp-contract=off so that a*b+c is never fused, matching the reference's Rust arithmetic.
 *
 * Parity unpinned: the f32 bits of orc_rotate_rows / orc_unrotate_rows. The reference rotates
 * with the CPU `gemm` crate (0.18.2 / 0.19.0, not part of the reference tree), whose summation
 * order is not restated here (this sums in index order); the rotation is pinned by its structure
 * (Hadamard signs, orthogonality) and TurboQuant codes by the reference's own flip criterion, not
 * bit for bit. Likewise the last bits of orc_attention_unfused / orc_cache_attention (gemm and
 * SIMD sum order) are pinned against float64 attention within tolerance, not bit for bit.
 */
#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

static inline uint32_t f2u(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}
static inline float u2f(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* ------------------------------------------------------------------------------------------ */
/* tiny parallel-for over [0, n) in contiguous chunks                                         */
/* ------------------------------------------------------------------------------------------ */
typedef void (*orc_body)(void *ctx, size_t lo, size_t hi);
typedef struct {
    orc_body fn;
    void *ctx;
    size_t lo, hi;
} orc_job;
static void *orc_job_run(void *p) {
    orc_job *j = (orc_job *)p;
    j->fn(j->ctx, j->lo, j->hi);
    return NULL;
}
static void orc_parallel(size_t n, int threads, orc_body fn, void *ctx) {
    if (threads <= 1 || n < 2) {
        fn(ctx, 0, n);
        return;
    }
    if ((size_t)threads > n) threads = (int)n;
    pthread_t *th = (pthread_t *)malloc(sizeof(pthread_t) * threads);
    orc_job *jobs = (orc_job *)malloc(sizeof(orc_job) * threads);
    for (int t = 0; t < threads; ++t) {
        jobs[t].fn = fn;
        jobs[t].ctx = ctx;
        jobs[t].lo = n * t / threads;
        jobs[t].hi = n * (t + 1) / threads;
        pthread_create(&th[t], NULL, orc_job_run, &jobs[t]);
    }
    for (int t = 0; t < threads; ++t) pthread_join(th[t], NULL);
    free(th);
    free(jobs);
}

/* ------------------------------------------------------------------------------------------ */
/* SplitMix64 + Box-Muller: candle-core/src/accel/turbo.rs:150-176                             */
/* ------------------------------------------------------------------------------------------ */
uint64_t orc_splitmix_next(uint64_t *s) {
    *s += 0x9e3779b97f4a7c15ULL;
    uint64_t z = *s;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
    return z ^ (z >> 31);
}

double orc_splitmix_f64(uint64_t *s) {
    return ((double)(orc_splitmix_next(s) >> 11) + 0.5) / (double)(1ULL << 53);
}

double orc_splitmix_normal(uint64_t *s) {
    const double u1 = orc_splitmix_f64(s);
    const double u2 = orc_splitmix_f64(s);
    return sqrt(-2.0 * log(u1)) * cos(2.0 * 3.14159265358979323846 * u2);
}

void orc_fill_normal(uint64_t seed, float *out, size_t n) {
    uint64_t s = seed;
    for (size_t i = 0; i < n; ++i) out[i] = (float)orc_splitmix_normal(&s);
}

/* ------------------------------------------------------------------------------------------ */
/* bf16 (half 2.7 `bf16::from_f32`: NaN keeps a quiet payload, else round to nearest even)     */
/* ------------------------------------------------------------------------------------------ */
uint16_t orc_f32_to_bf16(float f) {
    uint32_t x = f2u(f);
    if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x0040u);
    const uint32_t round_bit = 0x00008000u;
    if ((x & round_bit) != 0 && (x & (3 * round_bit - 1)) != 0) return (uint16_t)((x >> 16) + 1);
    return (uint16_t)(x >> 16);
}

float orc_bf16_to_f32(uint16_t b) { return u2f((uint32_t)b << 16); }

/* ------------------------------------------------------------------------------------------ */
/* element codecs: candle-core/src/accel/formats.rs:248-407                                    */
/* ------------------------------------------------------------------------------------------ */
float orc_pow2i(int e) { return u2f((uint32_t)(e + 127) << 23); } /* formats.rs:250-252 */

int orc_floor_log2(float a) { /* formats.rs:256-263 */
    const int e = (int)((f2u(a) >> 23) & 0xff);
    return e == 0 ? -127 : e - 127;
}

float orc_e4m3_to_f32(uint8_t c) { /* formats.rs:267-284 */
    const uint32_t s = c & 0x80;
    const uint32_t e = (c >> 3) & 0xf;
    const uint32_t m = c & 7;
    if (e == 15 && m == 7) return NAN;
    const float v = e == 0 ? (float)m * 0.001953125f : u2f(((e + 120) << 23) | (m << 20));
    return s ? -v : v;
}

uint8_t orc_f32_to_e4m3(float f) { /* formats.rs:288-308 */
    const uint32_t x = f2u(f);
    const uint8_t s = (uint8_t)((x >> 24) & 0x80);
    const uint32_t ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) return s | 0x7f;
    const float a = u2f(ax);
    if (a >= 448.0f) return s | 0x7e;
    if (a < 0.015625f) return s | (uint8_t)rintf(a * 512.0f);
    const uint32_t r = ax + 0x7ffffu + ((ax >> 20) & 1u);
    const uint32_t e = (r >> 23) - 120u;
    const uint32_t m = (r >> 20) & 7u;
    uint32_t code = (e << 3) | m;
    if (code > 0x7e) code = 0x7e;
    return s | (uint8_t)code;
}

float orc_fp4_to_f32(uint32_t c) { /* formats.rs:312-325 */
    const uint32_t e = (c >> 1) & 3;
    const uint32_t m = c & 1;
    const float v = e == 0 ? 0.5f * (float)m : u2f(((e + 126) << 23) | (m << 22));
    return (c & 8) ? -v : v;
}

uint32_t orc_f32_to_fp4(float f) { /* formats.rs:329-350 */
    const uint32_t s = (f2u(f) >> 28) & 8;
    const float a = fabsf(f);
    uint32_t c;
    if (isnan(a) || a <= 0.25f) c = 0;
    else if (a < 0.75f) c = 1;
    else if (a <= 1.25f) c = 2;
    else if (a < 1.75f) c = 3;
    else if (a <= 2.5f) c = 4;
    else if (a < 3.5f) c = 5;
    else if (a <= 5.0f) c = 6;
    else c = 7;
    return s | c;
}

float orc_e8m0_to_f32(uint8_t c) { /* formats.rs:354-360 */
    return c == 0 ? u2f(0x00400000u) : u2f((uint32_t)c << 23);
}

uint8_t orc_mx_scale_code(float amax, int emax_elem) { /* formats.rs:365-372 */
    int e = (amax > 0.0f && isfinite(amax)) ? orc_floor_log2(amax) - emax_elem : -127;
    if (e < -127) e = -127;
    if (e > 127) e = 127;
    return (uint8_t)(e + 127);
}

uint32_t orc_get_bits(const uint32_t *words, size_t pos, uint32_t bits) { /* formats.rs:376-385 */
    const size_t w = pos >> 5;
    const uint32_t sh = (uint32_t)(pos & 31);
    const uint32_t mask = (1u << bits) - 1u;
    uint32_t v = words[w] >> sh;
    if (sh + bits > 32) v |= words[w + 1] << (32 - sh);
    return v & mask;
}

void orc_put_bits(uint32_t *words, size_t pos, uint32_t bits, uint32_t v) { /* formats.rs:389-397 */
    const size_t w = pos >> 5;
    const uint32_t sh = (uint32_t)(pos & 31);
    v &= (1u << bits) - 1u;
    words[w] |= v << sh;
    if (sh + bits > 32) words[w + 1] |= v >> (32 - sh);
}

static uint8_t get_byte(const uint32_t *w, size_t k) { return (uint8_t)(w[k >> 2] >> ((k & 3) * 8)); }
static void put_byte(uint32_t *w, size_t k, uint8_t b) { w[k >> 2] |= (uint32_t)b << ((k & 3) * 8); }

/* ------------------------------------------------------------------------------------------ */
/* row layout: formats.rs:86-96 (bit checks), 166-187 (validate), 224-242 (layout)             */
/* ------------------------------------------------------------------------------------------ */
static int block_size(int mode) {
    return (mode == ORC_MXFP4 || mode == ORC_MXFP8) ? 32 : (mode == ORC_NVFP4 ? 16 : 0);
}

int orc_row_layout(int mode, int bits, int dim, orc_layout *out) {
    int code_bits;
    switch (mode) {
    case ORC_TURBO_MSE:
        if (bits < 1 || bits > 4) return -1;
        code_bits = bits;
        break;
    case ORC_TURBO_PROD:
        if (bits < 2 || bits > 5) return -1;
        code_bits = bits - 1;
        break;
    case ORC_MXFP4:
    case ORC_NVFP4: code_bits = 4; break;
    case ORC_MXFP8:
    case ORC_FP8: code_bits = 8; break;
    default: return -1;
    }
    if (dim <= 0 || dim > 1024) return -1;
    const int bs = block_size(mode);
    if (bs > 0 && dim % bs != 0) return -1;
    out->dim = dim;
    out->code_bits = code_bits;
    out->code_words = (dim * code_bits + 31) / 32;
    if (mode == ORC_TURBO_PROD) out->aux_words = (dim + 31) / 32;
    else if (bs > 0) out->aux_words = (dim / bs + 3) / 4;
    else out->aux_words = 0;
    out->row_words = out->code_words + out->aux_words + 2;
    return 0;
}

/* ------------------------------------------------------------------------------------------ */
/* Lloyd-Max codebook: candle-core/src/accel/turbo.rs:58-129                                   */
/* ------------------------------------------------------------------------------------------ */
/* first index i with xs[i] >= b (Rust partition_point(|x| x < b)) */
static size_t partition_lt(const double *xs, size_t n, double b) {
    size_t lo = 0, hi = n;
    while (lo < hi) {
        const size_t mid = lo + (hi - lo) / 2;
        if (xs[mid] < b) lo = mid + 1;
        else hi = mid;
    }
    return lo;
}

int orc_lloyd_max(int dim, int bits, float *centroids, float *boundaries) {
    if (bits < 1 || bits > 4 || dim < 2) return -1;
    const int k = 1 << bits;
    double lim = 12.0 / sqrt((double)dim);
    if (lim > 1.0) lim = 1.0;
    const size_t n = (size_t)1 << 16;
    const double h = 2.0 * lim / (double)n;
    const double expo = ((double)dim - 3.0) / 2.0;
    double *xs = (double *)malloc(n * sizeof(double));
    double *w = (double *)malloc(n * sizeof(double));
    double *cw = (double *)malloc((n + 1) * sizeof(double));
    double *cx = (double *)malloc((n + 1) * sizeof(double));
    for (size_t i = 0; i < n; ++i) xs[i] = -lim + ((double)i + 0.5) * h;
    double total = 0.0;
    for (size_t i = 0; i < n; ++i) {
        double t = 1.0 - xs[i] * xs[i];
        if (t < 1e-300) t = 1e-300;
        w[i] = exp(expo * log(t));
    }
    for (size_t i = 0; i < n; ++i) total += w[i];
    for (size_t i = 0; i < n; ++i) w[i] /= total;
    cw[0] = 0.0;
    cx[0] = 0.0;
    for (size_t i = 0; i < n; ++i) {
        cw[i + 1] = cw[i] + w[i];
        cx[i + 1] = cx[i] + w[i] * xs[i];
    }
    double c[16], bnd[16];
    for (int i = 0; i < k; ++i) {
        const double p = ((double)i + 0.5) / (double)k;
        size_t j = partition_lt(cw, n + 1, p);
        if (j < 1) j = 1;
        if (j > n) j = n;
        c[i] = xs[j - 1];
    }
    for (int it = 0; it < 2000; ++it) {
        for (int i = 0; i + 1 < k; ++i) bnd[i] = 0.5 * (c[i] + c[i + 1]);
        double delta = 0.0;
        size_t lo = 0;
        for (int i = 0; i < k; ++i) {
            const size_t hi = (i + 1 < k) ? partition_lt(xs, n, bnd[i]) : n;
            const double mass = cw[hi] - cw[lo];
            if (mass > 0.0) {
                const double m = (cx[hi] - cx[lo]) / mass;
                const double dd = fabs(m - c[i]);
                if (dd > delta) delta = dd;
                c[i] = m;
            }
            lo = hi;
        }
        if (delta < 1e-12) break;
    }
    for (int i = 0; i < k / 2; ++i) {
        const double v = 0.5 * (c[k - 1 - i] - c[i]);
        c[i] = -v;
        c[k - 1 - i] = v;
    }
    for (int i = 0; i < k; ++i) centroids[i] = (float)c[i];
    for (int i = 0; i + 1 < k; ++i) boundaries[i] = (float)(0.5 * (c[i] + c[i + 1]));
    free(xs);
    free(w);
    free(cw);
    free(cx);
    return 0;
}

/* ------------------------------------------------------------------------------------------ */
/* rotation matrix: candle-core/src/accel/turbo.rs:180-233                                     */
/* ------------------------------------------------------------------------------------------ */
int orc_rotation_matrix(int dim, int kind, uint64_t seed, float *m) {
    memset(m, 0, sizeof(float) * (size_t)dim * dim);
    if (kind == ORC_ROT_NONE) {
        for (int i = 0; i < dim; ++i) m[(size_t)i * dim + i] = 1.0f;
        return 0;
    }
    if (kind == ORC_ROT_HADAMARD) {
        if (dim <= 0 || (dim & (dim - 1)) != 0) return -1;
        /* seed ^ 0x4841_4441_4d41_5244 (turbo.rs:192) */
        uint64_t s = seed ^ 0x484144414d415244ULL;
        float *signs = (float *)malloc(sizeof(float) * dim);
        for (int j = 0; j < dim; ++j) signs[j] = (orc_splitmix_next(&s) & 1) == 0 ? 1.0f : -1.0f;
        const float sc = 1.0f / sqrtf((float)dim);
        for (int i = 0; i < dim; ++i)
            for (int j = 0; j < dim; ++j) {
                const float hv = (__builtin_popcount((unsigned)(i & j)) % 2 == 0) ? sc : -sc;
                m[(size_t)i * dim + j] = hv * signs[j];
            }
        free(signs);
        return 0;
    }
    if (kind == ORC_ROT_DENSE) {
        uint64_t s = seed ^ 0x524f544154452121ULL;
        double *rows = (double *)malloc(sizeof(double) * (size_t)dim * dim);
        for (size_t i = 0; i < (size_t)dim * dim; ++i) rows[i] = orc_splitmix_normal(&s);
        for (int pass = 0; pass < 2; ++pass)
            for (int i = 0; i < dim; ++i) {
                double *ri = rows + (size_t)i * dim;
                for (int j = 0; j < i; ++j) {
                    const double *rj = rows + (size_t)j * dim;
                    double dot = 0.0;
                    for (int t = 0; t < dim; ++t) dot += ri[t] * rj[t];
                    for (int t = 0; t < dim; ++t) ri[t] -= dot * rj[t];
                }
                double nn = 0.0;
                for (int t = 0; t < dim; ++t) nn += ri[t] * ri[t];
                nn = sqrt(nn);
                for (int t = 0; t < dim; ++t) ri[t] /= nn;
            }
        for (size_t i = 0; i < (size_t)dim * dim; ++i) m[i] = (float)rows[i];
        free(rows);
        return 0;
    }
    return -1;
}

/* y[r][i] = sum_j x[r][j] * pi[i][j]  (x · Πᵀ, turbo_quant.rs:182-189) */
void orc_rotate_rows(const float *pi, int dim, const float *x, size_t rows, float *y) {
    for (size_t r = 0; r < rows; ++r)
        for (int i = 0; i < dim; ++i) {
            float acc = 0.0f;
            const float *pr = pi + (size_t)i * dim;
            const float *xr = x + r * dim;
            for (int j = 0; j < dim; ++j) acc += xr[j] * pr[j];
            y[r * dim + i] = acc;
        }
}

/* x[r][j] = sum_i y[r][i] * pi[i][j]  (y · Π, turbo_quant.rs:191-196) */
void orc_unrotate_rows(const float *pi, int dim, const float *y, size_t rows, float *x) {
    float *acc = (float *)malloc(sizeof(float) * dim);
    for (size_t r = 0; r < rows; ++r) {
        for (int j = 0; j < dim; ++j) acc[j] = 0.0f;
        for (int i = 0; i < dim; ++i) {
            const float yi = y[r * dim + i];
            const float *pr = pi + (size_t)i * dim;
            for (int j = 0; j < dim; ++j) acc[j] += yi * pr[j];
        }
        memcpy(x + r * dim, acc, sizeof(float) * dim);
    }
    free(acc);
}

/* ------------------------------------------------------------------------------------------ */
/* row codec: candle-core/src/accel/turbo.rs:293-430                                           */
/* ------------------------------------------------------------------------------------------ */
void orc_qjl_matrix(int dim, uint64_t seed, float *s) { /* turbo.rs:236-239 */
    orc_fill_normal((seed + 1) ^ 0x514a4c5f534b4554ull, s, (size_t)dim * dim);
}

int orc_codec_init(orc_codec *c, int mode, int bits, int dim) {
    memset(c, 0, sizeof(*c));
    if (orc_row_layout(mode, bits, dim, &c->l) != 0) return -1;
    c->mode = mode;
    c->bits = bits;
    for (int i = 0; i < 16; ++i) c->boundaries[i] = INFINITY;
    /* the MSE codebook of the code bits (bits for TurboMse, bits - 1 for TurboProd;
       RowCodec::new, turbo.rs:252-258) */
    if ((mode == ORC_TURBO_MSE || mode == ORC_TURBO_PROD) &&
        orc_lloyd_max(dim, c->l.code_bits, c->centroids, c->boundaries) != 0)
        return -1;
    return 0;
}

void orc_quantize_row(const orc_codec *c, const float *y, uint32_t *out) {
    const orc_layout *l = &c->l;
    const int d = l->dim;
    memset(out, 0, sizeof(uint32_t) * l->row_words);
    float rsc0 = 1.0f, rsc1 = 0.0f;
    if (c->mode == ORC_TURBO_MSE || c->mode == ORC_TURBO_PROD) { /* turbo.rs:299-323 */
        const int nb = (1 << l->code_bits) - 1;
        float ss = 0.0f;
        for (int j = 0; j < d; ++j) ss += y[j] * y[j];
        const float norm = sqrtf(ss);
        const float inv = norm > 0.0f ? 1.0f / norm : 0.0f;
        float *resid = (float *)malloc(sizeof(float) * d);
        for (int j = 0; j < d; ++j) {
            const float u = y[j] * inv;
            uint32_t idx = 0;
            for (int b = 0; b < nb; ++b) idx += u >= c->boundaries[b] ? 1u : 0u;
            orc_put_bits(out, (size_t)j * l->code_bits, (uint32_t)l->code_bits, idx);
            resid[j] = u - c->centroids[idx];
        }
        rsc0 = norm;
        if (c->mode == ORC_TURBO_PROD && c->qjl) { /* turbo.rs:311-320 */
            float rr = 0.0f;
            for (int j = 0; j < d; ++j) rr += resid[j] * resid[j];
            rsc1 = sqrtf(rr);
            uint32_t *signs = out + l->code_words;
            for (int i = 0; i < d; ++i) {
                float pr = 0.0f;
                for (int j = 0; j < d; ++j) pr += c->qjl[(size_t)i * d + j] * resid[j];
                if (pr >= 0.0f) signs[i >> 5] |= 1u << (i & 31);
            }
        }
        free(resid);
    } else if (c->mode == ORC_MXFP4 || c->mode == ORC_MXFP8) { /* turbo.rs:324-347 */
        const int fp4 = c->mode == ORC_MXFP4;
        for (int b = 0; b < d / 32; ++b) {
            const float *blk = y + b * 32;
            float amax = 0.0f;
            for (int t = 0; t < 32; ++t) amax = fmaxf(amax, fabsf(blk[t]));
            const uint8_t code = orc_mx_scale_code(amax, fp4 ? 2 : 8);
            const float scale = orc_e8m0_to_f32(code);
            put_byte(out + l->code_words, (size_t)b, code);
            for (int t = 0; t < 32; ++t) {
                uint32_t e;
                if (code == 0) e = 0;
                else if (fp4) e = orc_f32_to_fp4(blk[t] / scale);
                else e = orc_f32_to_e4m3(blk[t] / scale);
                orc_put_bits(out, (size_t)(b * 32 + t) * l->code_bits, (uint32_t)l->code_bits, e);
            }
        }
    } else if (c->mode == ORC_NVFP4) { /* turbo.rs:348-365 */
        float amax = 0.0f;
        for (int j = 0; j < d; ++j) amax = fmaxf(amax, fabsf(y[j]));
        const float g = amax > 0.0f ? amax / 2688.0f : 1.0f;
        for (int b = 0; b < d / 16; ++b) {
            const float *blk = y + b * 16;
            float bmax = 0.0f;
            for (int t = 0; t < 16; ++t) bmax = fmaxf(bmax, fabsf(blk[t]));
            const uint8_t cs = orc_f32_to_e4m3(bmax / 6.0f / g);
            const float eff = orc_e4m3_to_f32(cs) * g;
            put_byte(out + l->code_words, (size_t)b, cs);
            for (int t = 0; t < 16; ++t) {
                const uint32_t e = eff > 0.0f ? orc_f32_to_fp4(blk[t] / eff) : 0;
                orc_put_bits(out, (size_t)(b * 16 + t) * 4, 4, e);
            }
        }
        rsc0 = g;
    } else { /* FP8, turbo.rs:366-374 */
        float amax = 0.0f;
        for (int j = 0; j < d; ++j) amax = fmaxf(amax, fabsf(y[j]));
        const float s = amax > 0.0f ? amax / 448.0f : 1.0f;
        for (int j = 0; j < d; ++j) orc_put_bits(out, (size_t)j * 8, 8, orc_f32_to_e4m3(y[j] / s));
        rsc0 = s;
    }
    const int o = l->code_words + l->aux_words;
    out[o] = f2u(rsc0);
    out[o + 1] = f2u(rsc1);
}

float orc_elem(const orc_codec *c, const uint32_t *row, int j) { /* turbo.rs:383-396 */
    const orc_layout *l = &c->l;
    const uint32_t code = orc_get_bits(row, (size_t)j * l->code_bits, (uint32_t)l->code_bits);
    const uint32_t *aux = row + l->code_words;
    switch (c->mode) {
    case ORC_TURBO_MSE:
    case ORC_TURBO_PROD: return c->centroids[code];
    case ORC_MXFP4: return orc_fp4_to_f32(code) * orc_e8m0_to_f32(get_byte(aux, (size_t)(j / 32)));
    case ORC_NVFP4: return orc_fp4_to_f32(code) * orc_e4m3_to_f32(get_byte(aux, (size_t)(j / 16)));
    case ORC_MXFP8: return orc_e4m3_to_f32((uint8_t)code) * orc_e8m0_to_f32(get_byte(aux, (size_t)(j / 32)));
    default: return orc_e4m3_to_f32((uint8_t)code);
    }
}

void orc_dequantize_row(const orc_codec *c, const uint32_t *row, float *out) { /* turbo.rs:401-424 */
    const int d = c->l.dim;
    const float r0 = u2f(row[c->l.code_words + c->l.aux_words]);
    for (int j = 0; j < d; ++j) out[j] = r0 * orc_elem(c, row, j);
    if (c->mode == ORC_TURBO_PROD && c->qjl) {
        const float r1 = u2f(row[c->l.code_words + c->l.aux_words + 1]);
        const float cq = r0 * r1 * 1.2533141f / (float)d; /* QJL_CONST, turbo.rs:26 */
        const uint32_t *signs = row + c->l.code_words;
        for (int i = 0; i < d; ++i) {
            const float z = ((signs[i >> 5] >> (i & 31)) & 1u) ? cq : -cq;
            for (int j = 0; j < d; ++j) out[j] += z * c->qjl[(size_t)i * d + j];
        }
    }
}

typedef struct {
    orc_codec c;
    const float *y;
    const uint32_t *w;
    uint32_t *out_w;
    float *out_f;
} rows_ctx;

static void quant_body(void *p, size_t lo, size_t hi) {
    rows_ctx *r = (rows_ctx *)p;
    for (size_t i = lo; i < hi; ++i)
        orc_quantize_row(&r->c, r->y + i * r->c.l.dim, r->out_w + i * r->c.l.row_words);
}
static void dequant_body(void *p, size_t lo, size_t hi) {
    rows_ctx *r = (rows_ctx *)p;
    for (size_t i = lo; i < hi; ++i)
        orc_dequantize_row(&r->c, r->w + i * r->c.l.row_words, r->out_f + i * r->c.l.dim);
}

int orc_quantize_rows(int mode, int bits, int dim, size_t rows, const float *y, uint32_t *out, int threads) {
    rows_ctx r;
    if (orc_codec_init(&r.c, mode, bits, dim) != 0) return -1;
    r.y = y;
    r.out_w = out;
    orc_parallel(rows, threads, quant_body, &r);
    return 0;
}

int orc_dequantize_rows(int mode, int bits, int dim, size_t rows, const uint32_t *words, float *out, int threads) {
    rows_ctx r;
    if (orc_codec_init(&r.c, mode, bits, dim) != 0) return -1;
    r.w = words;
    r.out_f = out;
    orc_parallel(rows, threads, dequant_body, &r);
    return 0;
}

int orc_quantize_rows_qjl(int bits, int dim, size_t rows, const float *y, const float *s, uint32_t *out,
                          int threads) {
    rows_ctx r;
    if (orc_codec_init(&r.c, ORC_TURBO_PROD, bits, dim) != 0) return -1;
    r.c.qjl = s;
    r.y = y;
    r.out_w = out;
    orc_parallel(rows, threads, quant_body, &r);
    return 0;
}

int orc_dequantize_rows_qjl(int bits, int dim, size_t rows, const uint32_t *words, const float *s,
                            float *out, int threads) {
    rows_ctx r;
    if (orc_codec_init(&r.c, ORC_TURBO_PROD, bits, dim) != 0) return -1;
    r.c.qjl = s;
    r.w = words;
    r.out_f = out;
    orc_parallel(rows, threads, dequant_body, &r);
    return 0;
}

/* ------------------------------------------------------------------------------------------ */
/* masks: candle-core/src/accel/attention.rs:80-92                                             */
/* ------------------------------------------------------------------------------------------ */
void orc_key_range(int64_t i, int64_t lq, int64_t lk, int wl, int wr, int64_t *plo, int64_t *phi) {
    const int64_t pos = i + lk - lq;
    int64_t lo = wl >= 0 ? (pos - wl > 0 ? pos - wl : 0) : 0;
    int64_t hi = wr >= 0 ? (pos + wr + 1 < lk ? pos + wr + 1 : lk) : lk;
    if (lo > lk) lo = lk;
    if (hi < lo) hi = lo;
    *plo = lo;
    *phi = hi;
}

/* ------------------------------------------------------------------------------------------ */
/* unfused attention: candle-nn/src/flash_attn.rs:930-1000, softmax candle-nn/src/ops.rs:315-352 */
/* ------------------------------------------------------------------------------------------ */
typedef struct {
    const float *q, *k, *v, *alibi;
    const int32_t *kv_lens;
    int b, hq, hkv, lq, lk, d, wl, wr;
    float scale, softcap;
    float *out;
} attn_ctx;

static void attn_body(void *p, size_t lo_row, size_t hi_row) {
    attn_ctx *a = (attn_ctx *)p;
    const int d = a->d, g = a->hq / a->hkv;
    float *s = (float *)malloc(sizeof(float) * (a->lk > 0 ? a->lk : 1));
    for (size_t row = lo_row; row < hi_row; ++row) {
        /* row = (bi * hq + h) * lq + i */
        const int i = (int)(row % a->lq);
        const int h = (int)((row / a->lq) % a->hq);
        const int bi = (int)(row / ((size_t)a->lq * a->hq));
        const int hk = h / g;
        const int lk_b = a->kv_lens ? a->kv_lens[bi] : a->lk;
        const float *qv = a->q + row * d;
        float *o = a->out + row * d;
        for (int t = 0; t < d; ++t) o[t] = 0.0f;
        int64_t lo, hi;
        orc_key_range(i, a->lq, lk_b, a->wl, a->wr, &lo, &hi);
        const int valid = lo < hi;
        const float slope = a->alibi ? a->alibi[h] : 0.0f;
        const int64_t pos = (int64_t)i + lk_b - a->lq;
        /* s = q k^T * scale, softcap, additive mask, alibi (flash_attn.rs:965-995) */
        float mx = -INFINITY;
        for (int j = 0; j < lk_b; ++j) {
            const float *kr = a->k + (((size_t)bi * a->hkv + hk) * a->lk + j) * d;
            float dot = 0.0f;
            for (int t = 0; t < d; ++t) dot += qv[t] * kr[t];
            float x = dot * a->scale;
            if (a->softcap > 0.0f) x = tanhf(x / a->softcap) * a->softcap;
            if (j < lo || j >= hi) x += -1e30f;
            if (a->alibi) {
                const int64_t dist = pos - j;
                x -= slope * (float)(dist < 0 ? -dist : dist);
            }
            s[j] = x;
            if (x > mx) mx = x;
        }
        /* softmax_last_dim: max, exp(x - max), sum, divide (ops.rs:315-345) */
        float sum = 0.0f;
        for (int j = 0; j < lk_b; ++j) {
            s[j] = expf(s[j] - mx);
            sum += s[j];
        }
        for (int j = 0; j < lk_b; ++j) s[j] = s[j] / sum;
        if (!valid || lk_b == 0) continue;
        for (int j = 0; j < lk_b; ++j) {
            const float pj = s[j];
            const float *vr = a->v + (((size_t)bi * a->hkv + hk) * a->lk + j) * d;
            for (int t = 0; t < d; ++t) o[t] += pj * vr[t];
        }
    }
    free(s);
}

int orc_attention_unfused(const float *q, const float *k, const float *v, int b, int hq, int hkv,
                          int lq, int lk, int d, const int32_t *kv_lens, float scale, float softcap,
                          int wl, int wr, const float *alibi, float *out, int threads) {
    if (hkv <= 0 || hq % hkv != 0) return -1;
    attn_ctx a = {q, k, v, alibi, kv_lens, b, hq, hkv, lq, lk, d, wl, wr, scale, softcap, out};
    orc_parallel((size_t)b * hq * lq, threads, attn_body, &a);
    return 0;
}

/* ------------------------------------------------------------------------------------------ */
/* the CPU decode path over packed rows: turbo_quant.rs:948-990 -> flash_attn.rs:930-1000      */
/* ------------------------------------------------------------------------------------------ */
typedef struct {
    orc_codec c;
    const uint32_t *rows;
    const float *pi;
    int cap, lk, hkv;
    const int32_t *kv_lens;
    float *out; /* (b, hkv, lk, d) f32 of bf16-rounded values */
} deq_ctx;

static void deq_cache_body(void *p, size_t lo, size_t hi) {
    deq_ctx *c = (deq_ctx *)p;
    const int d = c->c.l.dim, rw = c->c.l.row_words;
    float *tmp = (float *)malloc(sizeof(float) * d);
    float *tmp2 = (float *)malloc(sizeof(float) * d);
    for (size_t bh = lo; bh < hi; ++bh) {
        const int bi = (int)(bh / c->hkv);
        const int n = c->kv_lens ? c->kv_lens[bi] : c->lk;
        for (int t = 0; t < c->lk; ++t) {
            float *dst = c->out + (bh * c->lk + t) * d;
            if (t >= n) {
                memset(dst, 0, sizeof(float) * d);
                continue;
            }
            orc_dequantize_row(&c->c, c->rows + (bh * c->cap + t) * rw, tmp);
            const float *x = tmp;
            if (c->pi) {
                orc_unrotate_rows(c->pi, d, tmp, 1, tmp2);
                x = tmp2;
            }
            for (int j = 0; j < d; ++j) dst[j] = orc_bf16_to_f32(orc_f32_to_bf16(x[j]));
        }
    }
    free(tmp);
    free(tmp2);
}

int orc_cache_attention(const uint16_t *q_bf16, const uint32_t *k_rows, const uint32_t *v_rows,
                        int k_mode, int k_bits, int v_mode, int v_bits, const float *pi_k,
                        const float *pi_v, const float *qjl_k, int b, int hq, int hkv, int lq,
                        int cap, int d, const int32_t *kv_lens, int lk, float scale, int wl, int wr,
                        float softcap, const float *alibi, float *out, int threads) {
    deq_ctx kc, vc;
    if (orc_codec_init(&kc.c, k_mode, k_bits, d) != 0 || orc_codec_init(&vc.c, v_mode, v_bits, d) != 0)
        return -1;
    if (k_mode == ORC_TURBO_PROD) {
        if (!qjl_k) return -1;
        kc.c.qjl = qjl_k;
    }
    if (v_mode == ORC_TURBO_PROD) return -1; /* values use the MSE codebooks (turbo_quant.rs:869-871) */
    const size_t kv_elems = (size_t)b * hkv * lk * d;
    float *k = (float *)malloc(sizeof(float) * kv_elems);
    float *v = (float *)malloc(sizeof(float) * kv_elems);
    float *q = (float *)malloc(sizeof(float) * (size_t)b * hq * lq * d);
    if (!k || !v || !q) {
        free(k);
        free(v);
        free(q);
        return -2;
    }
    kc.rows = k_rows;
    kc.pi = pi_k;
    vc.rows = v_rows;
    vc.pi = pi_v;
    kc.cap = vc.cap = cap;
    kc.lk = vc.lk = lk;
    kc.hkv = vc.hkv = hkv;
    kc.kv_lens = vc.kv_lens = kv_lens;
    kc.out = k;
    vc.out = v;
    orc_parallel((size_t)b * hkv, threads, deq_cache_body, &kc);
    orc_parallel((size_t)b * hkv, threads, deq_cache_body, &vc);
    for (size_t i = 0; i < (size_t)b * hq * lq * d; ++i) q[i] = orc_bf16_to_f32(q_bf16[i]);
    const int rc = orc_attention_unfused(q, k, v, b, hq, hkv, lq, lk, d, kv_lens, scale, softcap, wl,
                                         wr, alibi, out, threads);
    free(k);
    free(v);
    free(q);
    return rc;
}

/* ------------------------------------------------------------------------------------------ */
/* split combine: candle-core/kernels/turbo_quant_impl.h:659-685                               */
/* ------------------------------------------------------------------------------------------ */
void orc_combine(const float *part_o, const float *part_lse, float *o, size_t rows, int d, int splits) {
    float *w = (float *)malloc(sizeof(float) * (splits > 0 ? splits : 1));
    for (size_t row = 0; row < rows; ++row) {
        float mx = -INFINITY;
        for (int s = 0; s < splits; ++s) mx = fmaxf(mx, part_lse[(size_t)s * rows + row]);
        for (int s = 0; s < splits; ++s) {
            const float e = part_lse[(size_t)s * rows + row];
            w[s] = e == -INFINITY ? 0.0f : expf(e - mx);
        }
        float wsum = 0.0f;
        for (int s = 0; s < splits; ++s) wsum += w[s];
        for (int t = 0; t < d; ++t) {
            float acc = 0.0f;
            for (int s = 0; s < splits; ++s)
                if (w[s] != 0.0f) acc += w[s] * part_o[((size_t)s * rows + row) * d + t];
            o[row * d + t] = wsum > 0.0f ? acc / wsum : 0.0f;
        }
    }
    free(w);
}

/* ------------------------------------------------------------------------------------------ */
/* split rules: candle-core/src/accel/attention.rs:486-506, row_group :586-592                 */
/* ------------------------------------------------------------------------------------------ */
int orc_split_count_grouped(size_t rows, int group, size_t lk, int policy_fixed, int compute_units) {
    if (policy_fixed > 0) return policy_fixed > 64 ? 64 : policy_fixed; /* SplitKv::Fixed */
    if (policy_fixed < 0) return 1;                                    /* SplitKv::Off */
    if (group < 1) group = 1;
    size_t wgs = rows / (size_t)group;
    if (wgs < 1) wgs = 1;
    const size_t cus = compute_units > 1 ? (size_t)compute_units : 1;
    const size_t by_occ = (64 * cus + wgs - 1) / wgs;
    const size_t keys = group > 1 ? 64 : 128;
    size_t by_keys = (lk + keys - 1) / keys;
    if (by_keys < 1) by_keys = 1;
    size_t n = by_occ < by_keys ? by_occ : by_keys;
    if (n < 1) n = 1;
    if (n > 64) n = 64;
    return (int)n;
}

int orc_row_group(int hq, int hkv) {
    const int g = hq / (hkv > 1 ? hkv : 1);
    const int cands[3] = {8, 4, 2};
    for (int i = 0; i < 3; ++i)
        if (g >= cands[i] && g % cands[i] == 0) return cands[i];
    return 1;
}

/* vectorised element encoders for exhaustive sweeps in the tests */
void orc_e4m3_encode_n(const float *x, uint8_t *out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = orc_f32_to_e4m3(x[i]);
}
void orc_fp4_encode_n(const float *x, uint8_t *out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = (uint8_t)orc_f32_to_fp4(x[i]);
}
