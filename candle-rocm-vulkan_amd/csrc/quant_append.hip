// Host side of the quantize-and-append entry points (cqkv_quant_append, cqkv_rope_quant_append):
// argument checks, the per-side argument blocks and the dispatch to the per-format launchers of
// append_inst.hip. The kernels are in append_rows.h.
#include "append_rows.h"
#include "rowmat.h"

namespace cqkv {

// bnd[7] == 0 and bnd[14 - i] == -bnd[i]: the codebook turbo_index may search by halves
static int turbo_symmetric(const float bnd[16]) {
    if (bnd[7] != 0.0f) return 0;
    for (int i = 0; i < 7; ++i)
        if (bnd[14 - i] != -bnd[i]) return 0;
    return 1;
}

// The in-register Hadamard rotation of a side (its seed's sign vector as bits, bit j set ->
// column j has sign -1, and 1 / sqrt(D)); zeros when the side takes no Walsh-Hadamard transform.
void fill_rotation(const cqkv_side *s, uint32_t sign_bits[8], float *rot_scale) {
    for (int i = 0; i < 8; ++i) sign_bits[i] = 0;
    *rot_scale = 1.0f;
    if (!side_fwht(s)) return;
    float signs[256];
    turbo_signs(s->head_dim, s->seed, signs);
    for (int j = 0; j < s->head_dim; ++j)
        if (signs[j] < 0.0f) sign_bits[j >> 5] |= 1u << (j & 31);
    *rot_scale = 1.0f / sqrtf((float)s->head_dim);
}

// The TurboQuant-4 codebook boundaries of the side's head dim (+inf padded to 16).
int fill_turbo_bounds(const cqkv_side *s, float bnd[16], float *cent_out) {
    float cent[16];
    for (int i = 0; i < 16; ++i) bnd[i] = __builtin_inff();
    // TurboMse{b}: the b-bit codebook; TurboProd{b}: the (b - 1)-bit one; boundaries past the
    // codebook's stay +inf, so the general count never passes them
    const int bits = turbo_code_bits(s);
    if (turbo_codebook(s->head_dim, bits, cent, bnd) != 0)
        return fail(CQKV_ERR_ARG, "turbo codebook for D=%d", s->head_dim);
    if (cent_out)
        for (int i = 0; i < (1 << bits); ++i) cent_out[i] = cent[i];
    return CQKV_OK;
}

// Elements 2l, 2l+1 of every row form one aligned 4- / 8-byte word.
static bool pair_aligned(const int64_t s[3], const void *p, int32_t dtype) {
    const size_t esz = dtype == CQKV_F32 ? 4 : 2;
    return s[0] % 2 == 0 && s[1] % 2 == 0 && s[2] % 2 == 0 && ((uintptr_t)p % (2 * esz)) == 0;
}

// Fills the append fields of `a` for one side and input x (shared by both entry points); staged:
// x holds the side's rows already rotated and padded to the plane row (f32, the staging pass).
static int fill_append_args(AppendArgs &a, const cqkv_side *side, const void *x,
                            int32_t x_dtype, const int64_t xs[3], int32_t tokens,
                            const int32_t *positions, int32_t position, bool staged = false) {
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
    {
        // 16-byte row loads when every thread's 32 elements start 16-byte aligned and the rows of
        // a workgroup (at most 256, token stride xs[2]) lie within 2^31 bytes of its first row
        const int64_t v = x_dtype == CQKV_F32 ? 4 : 8;
        const bool al = (uintptr_t)x % 16 == 0 && xs[0] % v == 0 && xs[1] % v == 0 && xs[2] % v == 0 &&
                        xs[2] >= 0 && (256 * xs[2] + 256) * (x_dtype == CQKV_F32 ? 4 : 2) < (int64_t)1 << 31;
        a.row_loads = !al                     ? kRowAny
                      : x_dtype == CQKV_F32   ? kRowF32
                      : x_dtype == CQKV_BF16  ? kRowBF16
                                              : kRowF16;
    }
    a.rotate = !staged && side_fwht(side) ? 1 : 0;
    fill_rotation(side, a.sign_bits, &a.rot_scale);
    a.dim = side->head_dim;
    if (side->format == CQKV_FMT_TURBO4) {
        if (int rc = fill_turbo_bounds(side, a.bnd, nullptr)) return rc;
        a.turbo_sym = turbo_symmetric(a.bnd);
    } else if (side->format == CQKV_FMT_TURBOPROD) {
        if (int rc = fill_turbo_bounds(side, a.bnd, a.cent)) return rc;
        a.turbo_sym = 0;  // at most 7 boundaries: the general count
        a.qjl = side->qjl;
    }
    return CQKV_OK;
}

static void launch_append_fmt(const cqkv_side *side, int32_t batch, int32_t tokens,
                              hipStream_t stream, const AppendArgs &a) {
    switch (side->format) {
    case CQKV_FMT_FP8: append_rows_launch_5(side, tokens, batch, stream, a); break;
    case CQKV_FMT_MXFP4: append_rows_launch_2(side, tokens, batch, stream, a); break;
    case CQKV_FMT_MXFP8: append_rows_launch_4(side, tokens, batch, stream, a); break;
    case CQKV_FMT_NVFP4: append_rows_launch_3(side, tokens, batch, stream, a); break;
    case CQKV_FMT_TURBOPROD: append_rows_launch_1(side, tokens, batch, stream, a); break;
    default: append_rows_launch_0(side, tokens, batch, stream, a); break;
    }
}

// Sides whose rows need the staging pass (a rotation by the matrix, or a head dim shorter than
// the plane row): the rows are rotated (x Pi^T, sums in index order) or copied into a
// stream-ordered f32 buffer of plane-row length with zero padding, and encoded from there.
static int staged_append_launch(const cqkv_side *side, const void *x, int32_t x_dtype,
                                const int64_t xs[3], int32_t batch, int32_t tokens,
                                const int32_t *positions, int32_t position, hipStream_t st,
                                int32_t clip_rows) {
    const int d = side->head_dim, dk = kernel_dim(d), hkv = side->kv_heads;
    float *rows = nullptr;
    CQKV_HIP_CHECK(hipMallocAsync((void **)&rows, (size_t)batch * hkv * tokens * dk * 4, st));
    const int64_t ys[3] = {(int64_t)hkv * tokens * dk, (int64_t)tokens * dk, dk};
    RowMatArgs r = rowmat_args(x, x_dtype, xs, batch, hkv, tokens, d, rows, CQKV_F32, ys, dk);
    if (side_matrix_rot(side)) {
        r.m = side->rot;
        r.transpose = 1;
    }
    int rc = CQKV_OK;
    const float *qjl = nullptr;
    float *qjl_tmp = nullptr;
    if (hipError_t e = rowmat_launch(r, st)) {
        rc = fail(CQKV_ERR_HIP, "staging rows: %s", hipGetErrorString(e));
    } else if ((rc = qjl_for_kernels(side, st, &qjl, &qjl_tmp)) == CQKV_OK) {
        AppendArgs a = {};
        rc = fill_append_args(a, side, rows, CQKV_F32, ys, tokens, positions, position, true);
        if (rc == CQKV_OK) {
            a.cs_rows = clip_rows;
            if (qjl) a.qjl = qjl;
            launch_append_fmt(side, batch, tokens, st, a);
            if (hipError_t e = hipGetLastError())
                rc = fail(CQKV_ERR_HIP, "append launch: %s", hipGetErrorString(e));
        }
    }
    hipError_t fe = qjl_tmp ? hipFreeAsync(qjl_tmp, st) : hipSuccess;
    const hipError_t fe2 = hipFreeAsync(rows, st);
    if (fe == hipSuccess) fe = fe2;
    if (rc == CQKV_OK && fe != hipSuccess)
        rc = fail(CQKV_ERR_HIP, "staging buffers: %s", hipGetErrorString(fe));
    return rc;
}

// Launch used by cqkv_quant_append, the prefill's unfused append and the value side of a fused
// RoPE append whose sides differ in format; clip_rows > 0 skips positions at or past it (the
// rotary table end of the fused RoPE append).
int quant_append_launch(const cqkv_side *side, const void *x, int32_t x_dtype,
                        const int64_t xs[3], int32_t batch, int32_t tokens,
                        const int32_t *positions, int32_t position, hipStream_t stream,
                        int32_t clip_rows) {
    if (side_staged(side))
        return staged_append_launch(side, x, x_dtype, xs, batch, tokens, positions, position,
                                    stream, clip_rows);
    AppendArgs a = {};
    if (int rc = fill_append_args(a, side, x, x_dtype, xs, tokens, positions, position)) return rc;
    a.cs_rows = clip_rows;
    launch_append_fmt(side, batch, tokens, stream, a);
    CQKV_HIP_CHECK(hipGetLastError());
    return CQKV_OK;
}

// Rotary embedding of rows (batch, heads, tokens, d) of `dtype` into y (same shape and dtype),
// the reference's rope / rope_i (candle-core/kernels/nn.hip:107-148): token t of batch b at
// position p = positions[b] + t (or position + t) takes row p of the (cs_rows, d / 2) tables;
// products rounded before the sum, then rounded to the dtype. Tokens past the tables are not
// written. One thread per rotated pair. The unfused form of cqkv_rope_quant_append, for the
// sides the fused kernel does not take (plane rows of 256, staged sides).
struct RopeRowsArgs {
    const void *x;
    void *y;
    int64_t xs0, xs1, xs2, ys0, ys1, ys2;
    const void *cos, *sin;
    const int32_t *positions;
    int32_t heads, tokens, d, dtype, cs_rows, kind, position;
};

__global__ __launch_bounds__(256) void rope_rows_kernel(RopeRowsArgs a) {
#pragma clang fp contract(off)
    const int half = a.d / 2;
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t per_b = (int64_t)a.heads * a.tokens * half;
    const int b = blockIdx.y;
    if (i >= per_b) return;
    const int pr = (int)(i % half);
    const int64_t ht = i / half;
    const int t = (int)(ht % a.tokens), h = (int)(ht / a.tokens);
    const int base = a.positions ? a.positions[b] : a.position;
    const int64_t p = (int64_t)base + t;
    if (base < 0 || p >= a.cs_rows) return;
    const int j0 = a.kind == CQKV_ROPE_INTERLEAVED ? 2 * pr : pr;
    const int j1 = a.kind == CQKV_ROPE_INTERLEAVED ? 2 * pr + 1 : pr + half;
    const int64_t xo = b * a.xs0 + h * a.xs1 + t * a.xs2, yo = b * a.ys0 + h * a.ys1 + t * a.ys2;
    const float x0 = load_elem(a.x, xo + j0, a.dtype), x1 = load_elem(a.x, xo + j1, a.dtype);
    const float c = load_elem(a.cos, p * half + pr, a.dtype), sn = load_elem(a.sin, p * half + pr, a.dtype);
    const float c0 = x0 * c, s1 = x1 * sn, s0 = x0 * sn, c1 = x1 * c;
    store_elem(a.y, yo + j0, a.dtype, c0 - s1);
    store_elem(a.y, yo + j1, a.dtype, s0 + c1);
}

static hipError_t rope_rows_launch(const void *x, const int64_t xs[3], void *y, const int64_t ys[3],
                                   int32_t batch, int32_t heads, int32_t tokens, int32_t d,
                                   int32_t dtype, const void *cos, const void *sin, int32_t cs_rows,
                                   int32_t kind, const int32_t *positions, int32_t position,
                                   hipStream_t st) {
    RopeRowsArgs a = {x, y, xs[0], xs[1], xs[2], ys[0], ys[1], ys[2], cos, sin, positions,
                      heads, tokens, d, dtype, cs_rows, kind, position};
    const int64_t n = (int64_t)heads * tokens * (d / 2);
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(rope_rows_kernel, dim3((unsigned)((n + 255) / 256), batch), dim3(256), 0, st, a);
    return hipGetLastError();
}

// cqkv_rope_quant_append as separate launches: q rotated into q_out, k rotated into a
// stream-ordered buffer, then the appends of both sides with the tables' end as the clip.
static int rope_append_unfused(const cqkv_side *k_side, const cqkv_side *v_side, const void *q,
                               const int64_t qs[3], const void *k, const int64_t ks[3],
                               const void *v, const int64_t vs[3], int32_t dtype, int32_t batch,
                               int32_t tokens, int32_t q_heads, const void *cos, const void *sin,
                               int32_t cs_rows, int32_t kind, const int32_t *positions,
                               int32_t position, void *q_out, const int64_t qos[3],
                               hipStream_t st) {
    const int d = k_side->head_dim, hkv = k_side->kv_heads;
    const size_t esz = dtype == CQKV_F32 ? 4 : 2;
    if (hipError_t e = rope_rows_launch(q, qs, q_out, qos, batch, q_heads, tokens, d, dtype, cos,
                                        sin, cs_rows, kind, positions, position, st))
        return fail(CQKV_ERR_HIP, "rope of q: %s", hipGetErrorString(e));
    void *kr = nullptr;
    CQKV_HIP_CHECK(hipMallocAsync(&kr, (size_t)batch * hkv * tokens * d * esz, st));
    const int64_t krs[3] = {(int64_t)hkv * tokens * d, (int64_t)tokens * d, d};
    int rc = CQKV_OK;
    if (hipError_t e = rope_rows_launch(k, ks, kr, krs, batch, hkv, tokens, d, dtype, cos, sin,
                                        cs_rows, kind, positions, position, st))
        rc = fail(CQKV_ERR_HIP, "rope of k: %s", hipGetErrorString(e));
    if (rc == CQKV_OK)
        rc = quant_append_launch(k_side, kr, dtype, krs, batch, tokens, positions, position, st,
                                 cs_rows);
    const hipError_t fe = hipFreeAsync(kr, st);
    if (rc == CQKV_OK && fe != hipSuccess)
        rc = fail(CQKV_ERR_HIP, "rotated keys: %s", hipGetErrorString(fe));
    if (rc == CQKV_OK)
        rc = quant_append_launch(v_side, v, dtype, vs, batch, tokens, positions, position, st,
                                 cs_rows);
    return rc;
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
    if (k_side->head_dim != v_side->head_dim || k_side->kv_heads != v_side->kv_heads ||
        k_side->capacity != v_side->capacity)
        return fail(CQKV_ERR_ARG, "%s: key / value sides differ in D, heads or capacity", who);
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
    if (k_side->head_dim % 2 != 0)
        return fail(CQKV_ERR_ARG, "%s: rotary embedding of an odd head_dim %d", who,
                    k_side->head_dim);
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
    if (side_staged(k_side) || side_staged(v_side) || kernel_dim(k_side->head_dim) == 256)
        return rope_append_unfused(k_side, v_side, q, q_strides, k, k_strides, v, v_strides, dtype,
                                   batch, tokens, q_heads, cos, sin, cs_rows, rope_kind, positions,
                                   position, q_out, q_out_strides, (hipStream_t)stream);
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
        r.k.cs_vec16 = ((uintptr_t)cos % 16 == 0 && (uintptr_t)sin % 16 == 0) ? 1 : 0;
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
    // values of another format than the keys: their own append launch after this one
    const bool same = k_side->format == v_side->format;
    r.v_units = same ? hkv : 0;
    // an unaligned start spans up to 7 more positions
    const int64_t blocks = ((int64_t)tokens + 7 + kRopeBlockTokens - 1) / kRopeBlockTokens *
                           (hkv + r.v_units + r.q_units);
    if (blocks * 256 > (int64_t)UINT32_MAX)  // threads along x of one launch
        return fail(CQKV_ERR_ARG, "%s: %d tokens x %d heads exceed one launch", who, tokens,
                    2 * hkv + q_heads);
    dim3 grid((uint32_t)blocks, 1, batch);
    const hipStream_t st = (hipStream_t)stream;
    const int d = k_side->head_dim;
    switch (k_side->format) {
    case CQKV_FMT_FP8: rope_append_launch_5(rope_kind, d, grid, st, r); break;
    case CQKV_FMT_MXFP4: rope_append_launch_2(rope_kind, d, grid, st, r); break;
    case CQKV_FMT_TURBOPROD: rope_append_launch_1(rope_kind, d, grid, st, r); break;
    case CQKV_FMT_MXFP8: rope_append_launch_4(rope_kind, d, grid, st, r); break;
    case CQKV_FMT_NVFP4: rope_append_launch_3(rope_kind, d, grid, st, r); break;
    default: rope_append_launch_0(rope_kind, d, grid, st, r); break;
    }
    CQKV_HIP_CHECK(hipGetLastError());
    if (!same)
        return quant_append_launch(v_side, v, dtype, v_strides, batch, tokens, positions, position,
                                   st, cs_rows);
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
                               (hipStream_t)stream, 0);
}
