// Host side of the C ABI that launches nothing: error text, plane sizes, side checks and the
// TurboQuant tables (Lloyd-Max codebook, Hadamard signs).
#include <math.h>
#include <stdarg.h>
#include <stdio.h>

#include <algorithm>
#include <map>
#include <mutex>
#include <vector>

#include "cqkv_host.h"

namespace cqkv {

static thread_local std::string g_error;

void set_error(const std::string &msg) { g_error = msg; }
void clear_error() { g_error.clear(); }

int fail(int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_error = buf;
    return code;
}

int check_side(const cqkv_side *s, const char *what) {
    if (!s) return fail(CQKV_ERR_ARG, "%s: null cache side", what);
    if (!code_bits(s->format)) return fail(CQKV_ERR_ARG, "%s: unknown format %d", what, s->format);
    if (!supported_dim(s->format, s->head_dim))
        return fail(CQKV_ERR_ARG,
                    "%s: head_dim %d not supported (1-256; MX formats a multiple of 32, NVFP4 of 16)",
                    what, s->head_dim);
    if (s->kv_heads <= 0) return fail(CQKV_ERR_ARG, "%s: kv_heads %d", what, s->kv_heads);
    if (s->capacity <= 0 || s->capacity % 32 != 0)
        return fail(CQKV_ERR_ARG, "%s: capacity %d is not a positive multiple of 32", what,
                    s->capacity);
    if (!s->codes || !s->scales) return fail(CQKV_ERR_ARG, "%s: null codes / scales", what);
    if (s->is_value != 0 && s->is_value != 1)
        return fail(CQKV_ERR_ARG, "%s: is_value must be 0 or 1", what);
    if (s->rotation < CQKV_ROT_DEFAULT || s->rotation > CQKV_ROT_AUTO)
        return fail(CQKV_ERR_ARG, "%s: rotation %d (default, none, Hadamard, dense or auto)", what,
                    s->rotation);
    if (side_matrix_rot(s) && !s->rot)
        return fail(CQKV_ERR_ARG,
                    "%s: a %s rotation at head_dim %d needs the side's rotation matrix (rot)", what,
                    side_rotation(s) == CQKV_ROT_DENSE ? "dense" : "Hadamard", s->head_dim);
    if (s->format == CQKV_FMT_TURBO4 && (s->bits < 0 || s->bits > 4))
        return fail(CQKV_ERR_ARG, "%s: TurboMse bits %d (1-4, 0: 4)", what, s->bits);
    if (s->format == CQKV_FMT_TURBOPROD && (s->bits < 0 || s->bits == 1 || s->bits > 5))
        return fail(CQKV_ERR_ARG, "%s: TurboProd bits %d (2-5, 0: 4)", what, s->bits);
    if (!is_turbo(s->format) && s->bits != 0)
        return fail(CQKV_ERR_ARG, "%s: bits %d given for a format without a width (0)", what,
                    s->bits);
    if (s->format == CQKV_FMT_TURBOPROD) {
        if (s->is_value)
            return fail(CQKV_ERR_ARG,
                        "%s: TURBOPROD is a key format (values use the MSE codebooks)", what);
        if (!s->qjl) return fail(CQKV_ERR_ARG, "%s: TURBOPROD side without its QJL matrix", what);
    }
    const size_t cb = cqkv_codes_plane_bytes(s->format, s->head_dim, s->capacity);
    if (cb > 0x7fffffffull)
        return fail(CQKV_ERR_ARG, "%s: a plane of %zu bytes exceeds 2 GiB", what, cb);
    return CQKV_OK;
}

// Lloyd-Max quantizer of one coordinate of a uniform random unit vector in R^dim, whose density
// is proportional to (1 - x^2)^((dim - 3) / 2). Same algorithm and constants as the reference
// (candle-core/src/accel/turbo.rs:58-129): a 2^16-point midpoint grid over
// |x| < min(1, 12 / sqrt(dim)), quantile initialisation, at most 2000 Lloyd iterations stopped
// at a 1e-12 centroid move, exact symmetrisation, f32 centroids and midpoint boundaries. The
// float64 sums run in index order so that the f32 tables come out identical.
static int turbo_codebook_compute(int dim, int bits, float *centroids, float *boundaries) {
    const int k = 1 << bits;
    const size_t n = size_t(1) << 16;
    const double lim = std::min(1.0, 12.0 / sqrt((double)dim));
    const double step = 2.0 * lim / (double)n;
    const double expo = ((double)dim - 3.0) / 2.0;
    std::vector<double> grid(n), mass(n), cmass(n + 1, 0.0), cmom(n + 1, 0.0);
    double total = 0.0;
    for (size_t i = 0; i < n; ++i) {
        grid[i] = -lim + ((double)i + 0.5) * step;
        mass[i] = exp(expo * log(std::max(1.0 - grid[i] * grid[i], 1e-300)));
    }
    for (size_t i = 0; i < n; ++i) total += mass[i];
    for (size_t i = 0; i < n; ++i) mass[i] /= total;
    for (size_t i = 0; i < n; ++i) {
        cmass[i + 1] = cmass[i] + mass[i];
        cmom[i + 1] = cmom[i] + mass[i] * grid[i];
    }
    auto first_not_below = [](const std::vector<double> &v, size_t len, double x) {
        return (size_t)(std::lower_bound(v.begin(), v.begin() + len, x) - v.begin());
    };
    double c[16], b[16];
    for (int i = 0; i < k; ++i) {
        const double p = ((double)i + 0.5) / (double)k;
        size_t j = first_not_below(cmass, n + 1, p);
        j = std::min(std::max(j, (size_t)1), n);
        c[i] = grid[j - 1];
    }
    for (int it = 0; it < 2000; ++it) {
        for (int i = 0; i + 1 < k; ++i) b[i] = 0.5 * (c[i] + c[i + 1]);
        double moved = 0.0;
        size_t lo = 0;
        for (int i = 0; i < k; ++i) {
            const size_t hi = i + 1 < k ? first_not_below(grid, n, b[i]) : n;
            const double m = cmass[hi] - cmass[lo];
            if (m > 0.0) {
                const double mean = (cmom[hi] - cmom[lo]) / m;
                moved = std::max(moved, fabs(mean - c[i]));
                c[i] = mean;
            }
            lo = hi;
        }
        if (moved < 1e-12) break;
    }
    for (int i = 0; i < k / 2; ++i) {
        const double h = 0.5 * (c[k - 1 - i] - c[i]);
        c[i] = -h;
        c[k - 1 - i] = h;
    }
    for (int i = 0; i < k; ++i) centroids[i] = (float)c[i];
    for (int i = 0; i + 1 < k; ++i) boundaries[i] = (float)(0.5 * (c[i] + c[i + 1]));
    return 0;
}

// The codebook of (dim, bits), computed once per process and cached (the reference caches it
// per (dim, bits) too, candle-core/src/accel/turbo.rs:131-146): every quantize / decode call
// needs it, and computing it takes milliseconds.
int turbo_codebook(int dim, int bits, float *centroids, float *boundaries) {
    if (bits < 1 || bits > 4 || dim < 2 || dim > 1024) return -1;
    struct Entry {
        float c[16], b[16];
    };
    static std::mutex mu;
    static std::map<std::pair<int, int>, Entry> cache;
    std::lock_guard<std::mutex> lock(mu);
    auto it = cache.find({dim, bits});
    if (it == cache.end()) {
        Entry e;
        if (turbo_codebook_compute(dim, bits, e.c, e.b) != 0) return -1;
        it = cache.emplace(std::make_pair(dim, bits), e).first;
    }
    const int k = 1 << bits;
    for (int i = 0; i < k; ++i) centroids[i] = it->second.c[i];
    for (int i = 0; i + 1 < k; ++i) boundaries[i] = it->second.b[i];
    return 0;
}

// rotation_matrix (candle-core/src/accel/turbo.rs:180-233) of a resolved kind: the identity, the
// sign-flipped Sylvester Hadamard matrix / sqrt(dim), or the Dense matrix - dim x dim normals of
// SplitMix64(seed ^ "ROTATE!!") (Box-Muller in f64), two passes of modified Gram-Schmidt in f64
// with the dot products and norms summed in index order and no fused multiply-add (this file is
// built with -ffp-contract=off, as the reference's Rust arithmetic rounds every operation),
// rounded to f32. Row-major, y = Pi x.
void rotation_matrix(int dim, int kind, uint64_t seed, float *out) {
    const size_t n = (size_t)dim * dim;
    for (size_t i = 0; i < n; ++i) out[i] = 0.0f;
    if (kind == CQKV_ROT_NONE) {
        for (int i = 0; i < dim; ++i) out[(size_t)i * dim + i] = 1.0f;
    } else if (kind == CQKV_ROT_HADAMARD) {
        std::vector<float> signs(dim);
        turbo_signs(dim, seed, signs.data());
        const float sc = 1.0f / sqrtf((float)dim);
        for (int i = 0; i < dim; ++i)
            for (int j = 0; j < dim; ++j)
                out[(size_t)i * dim + j] = (__builtin_popcount((unsigned)(i & j)) & 1 ? -sc : sc) * signs[j];
    } else {
        uint64_t state = seed ^ 0x524f544154452121ull;
        auto next = [&state]() {
            state += 0x9e3779b97f4a7c15ull;
            uint64_t z = state;
            z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
            z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
            return z ^ (z >> 31);
        };
        const double two_pi = 2.0 * 3.141592653589793;
        std::vector<double> rows(n);
        for (size_t i = 0; i < n; ++i) {
            const double u1 = ((double)(next() >> 11) + 0.5) / 9007199254740992.0;
            const double u2 = ((double)(next() >> 11) + 0.5) / 9007199254740992.0;
            rows[i] = sqrt(-2.0 * log(u1)) * cos(two_pi * u2);
        }
        for (int pass = 0; pass < 2; ++pass)
            for (int i = 0; i < dim; ++i) {
                double *ri = rows.data() + (size_t)i * dim;
                for (int j = 0; j < i; ++j) {
                    const double *rj = rows.data() + (size_t)j * dim;
                    double dot = 0.0;
                    for (int t = 0; t < dim; ++t) dot += ri[t] * rj[t];
                    for (int t = 0; t < dim; ++t) ri[t] -= dot * rj[t];
                }
                double nn = 0.0;
                for (int t = 0; t < dim; ++t) nn += ri[t] * ri[t];
                nn = sqrt(nn);
                for (int t = 0; t < dim; ++t) ri[t] /= nn;
            }
        for (size_t i = 0; i < n; ++i) out[i] = (float)rows[i];
    }
}

// Column signs of the seeded Hadamard rotation: SplitMix64 seeded with seed ^ "HADAMARD"
// (0x484144414d415244 in ASCII), one draw per column, even draw -> +1
// (candle-core/src/accel/turbo.rs:150-163, 188-196).
void turbo_signs(int dim, uint64_t seed, float *signs) {
    uint64_t state = seed ^ 0x484144414d415244ull;
    for (int j = 0; j < dim; ++j) {
        state += 0x9e3779b97f4a7c15ull;
        uint64_t z = state;
        z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
        z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
        z ^= z >> 31;
        signs[j] = (z & 1) == 0 ? 1.0f : -1.0f;
    }
}

// The QJL matrix: SplitMix64 at (seed + 1) ^ "QJL_SKET", one Box-Muller normal (two uniforms
// ((u >> 11) + 0.5) / 2^53, f64 log / sqrt / cos) per entry, rounded to f32
// (candle-core/src/accel/turbo.rs:150-176, 236-239).
void qjl_matrix(int dim, uint64_t seed, float *out) {
    uint64_t state = (seed + 1) ^ 0x514a4c5f534b4554ull;
    auto next = [&state]() {
        state += 0x9e3779b97f4a7c15ull;
        uint64_t z = state;
        z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
        z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
        return z ^ (z >> 31);
    };
    const double two_pi = 2.0 * 3.141592653589793;
    for (size_t i = 0; i < (size_t)dim * dim; ++i) {
        const double u1 = ((double)(next() >> 11) + 0.5) / 9007199254740992.0;
        const double u2 = ((double)(next() >> 11) + 0.5) / 9007199254740992.0;
        out[i] = (float)(sqrt(-2.0 * log(u1)) * cos(two_pi * u2));
    }
}

}  // namespace cqkv

extern "C" {

// Planes hold rows of the plane row length kernel_dim(head_dim).
size_t cqkv_codes_plane_bytes(int32_t format, int32_t head_dim, int32_t capacity) {
    const int bits = cqkv::code_bits(format);
    if (!bits || !cqkv::supported_dim(format, head_dim) || capacity <= 0) return 0;
    return (size_t)capacity * (size_t)cqkv::kernel_dim(head_dim) * (size_t)bits / 8;
}

size_t cqkv_scales_plane_bytes(int32_t format, int32_t head_dim, int32_t capacity) {
    if (!cqkv::code_bits(format) || !cqkv::supported_dim(format, head_dim) || capacity <= 0) return 0;
    const int dk = cqkv::kernel_dim(head_dim);
    if (format == CQKV_FMT_TURBOPROD)  // norms, |r|, sign bits
        return (size_t)capacity * (8 + (size_t)dk / 8);
    const int be = cqkv::block_elems(format);
    const size_t blocks = be ? (size_t)capacity * (size_t)(dk / be) : 0;
    return blocks + (cqkv::token_scale(format) ? (size_t)capacity * 4 : 0);
}

int32_t cqkv_reference_row_words(int32_t format, int32_t bits, int32_t head_dim) {
    const int cb = cqkv::code_bits(format);
    if (!cb || !cqkv::supported_dim(format, head_dim)) return 0;
    if (cqkv::is_turbo(format)) {  // formats.rs:226-240: b-bit (prod: b - 1) codes, prod signs
        const int b = bits ? bits : 4;
        if (format == CQKV_FMT_TURBO4 && (b < 1 || b > 4)) return 0;
        if (format == CQKV_FMT_TURBOPROD && (b < 2 || b > 5)) return 0;
        const int code = format == CQKV_FMT_TURBOPROD ? b - 1 : b;
        return (head_dim * code + 31) / 32 +
               (format == CQKV_FMT_TURBOPROD ? (head_dim + 31) / 32 : 0) + 2;
    }
    if (bits != 0) return 0;
    const int code_words = (head_dim * cb + 31) / 32;
    const int be = cqkv::block_elems(format);
    const int aux_words = be ? (head_dim / be + 3) / 4 : 0;  // formats.rs:229-233
    return code_words + aux_words + 2;
}

int cqkv_turbo_codebook(int32_t head_dim, int32_t bits, float *centroids, float *boundaries) {
    if (!centroids || !boundaries)
        return cqkv::fail(CQKV_ERR_ARG, "cqkv_turbo_codebook: null output");
    if (cqkv::turbo_codebook(head_dim, bits, centroids, boundaries) != 0)
        return cqkv::fail(CQKV_ERR_ARG, "cqkv_turbo_codebook: bits %d / dim %d", bits, head_dim);
    return CQKV_OK;
}

int cqkv_turbo_signs(int32_t head_dim, uint64_t seed, float *signs) {
    if (!signs || head_dim <= 0 || (head_dim & (head_dim - 1)) != 0)
        return cqkv::fail(CQKV_ERR_ARG, "cqkv_turbo_signs: head_dim %d", head_dim);
    cqkv::turbo_signs(head_dim, seed, signs);
    return CQKV_OK;
}

int32_t cqkv_resolve_rotation(int32_t format, int32_t kind, int32_t head_dim) {
    if (head_dim < 1 || head_dim > 1024) return -1;
    return cqkv::resolve_rotation(format, kind, head_dim);
}

int cqkv_rotation_matrix(int32_t head_dim, int32_t kind, uint64_t seed, float *out) {
    if (!out || head_dim < 1 || head_dim > 1024)
        return cqkv::fail(CQKV_ERR_ARG, "cqkv_rotation_matrix: head_dim %d / null output", head_dim);
    // DEFAULT as AUTO (the TurboQuant formats' own rotation)
    const int r = cqkv::resolve_rotation(CQKV_FMT_TURBO4, kind, head_dim);
    if (r < 0) return cqkv::fail(CQKV_ERR_ARG, "cqkv_rotation_matrix: rotation %d", kind);
    cqkv::rotation_matrix(head_dim, r, seed, out);
    return CQKV_OK;
}

int cqkv_qjl_matrix(int32_t head_dim, uint64_t seed, float *out) {
    if (!out || head_dim <= 0 || head_dim > 1024)
        return cqkv::fail(CQKV_ERR_ARG, "cqkv_qjl_matrix: head_dim %d / null output", head_dim);
    cqkv::qjl_matrix(head_dim, seed, out);
    return CQKV_OK;
}

const char *cqkv_last_error(void) { return cqkv::g_error.c_str(); }

const char *cqkv_version(void) { return "cqkv 0.1 gfx950"; }

}  // extern "C"
