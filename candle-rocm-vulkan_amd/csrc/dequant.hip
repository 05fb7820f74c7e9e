// Dequantization of cache rows (cqkv_dequantize_rows): the device half of TqDequant /
// TurboQuantizer::dequantize_rows and TurboKvCache::keys_values.
//
// Reference behaviour (paths relative to the reference repository root): RowCodec::elem and
// dequantize_row (candle-core/src/accel/turbo.rs:383-424), TqDequant (candle-nn/src/
// turbo_quant.rs:612-689), dequantize_gpu + unrotate (turbo_quant.rs:250-300, 191-196),
// keys_values (turbo_quant.rs:948-966), RocmStorage::tq_dequantize
// (candle-core/src/rocm_backend/accel.rs:380-419).
//
// Each element is rsc0 * element_j in f32 with the reference's operation order, so the rotated-
// domain values are bit for bit those of dequantize_row. The TurboProd correction
// sum_i z_i S[i][j] and the unrotation y Pi run on the row-matrix kernel (rowmat.hip), terms
// summed in index order.
#include "cqkv_device.h"
#include "cqkv_host.h"
#include "rowmat.h"

namespace cqkv {

struct DequantArgs {
    const uint8_t *codes, *scales;
    uint32_t codes_plane, scales_plane;
    int32_t kv_heads, tokens, position, capacity;
    int32_t dk, dim, format, is_value;
    int32_t nblk;  // block scale bytes per token in the plane (MX, NVFP4)
    float cent[16];
    void *out;     // rows of dim elements: (batch, head, token) at strides os0 / os1 / os2
    int32_t out_dtype, pad_;
    int64_t os0, os1, os2;
    float *zs;     // TURBOPROD: +-rsc0 rsc1 sqrt(pi/2) / dim per sign bit, (rows, dim) f32
};

__device__ inline float e4m3_value(uint32_t c) { return __builtin_amdgcn_cvt_f32_fp8(c, 0); }
__device__ inline float fp4_value(uint32_t c) {
    const f32x2 v = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(c, 1.0f, 0);  // exact
    return v[0];  // the code in the low nibble
}
__device__ inline float e8m0_value(uint32_t c) {  // formats.rs:354-360: code 0 is 2^-127
    return c == 0 ? __uint_as_float(0x00400000u) : __uint_as_float(c << 23);
}

// One workgroup of max(64, dk / 2) threads per 8-token tile of a (batch, head) plane; thread l
// owns elements 2l, 2l+1 of the plane row.
__global__ __launch_bounds__(128) void dequant_kernel(DequantArgs a) {
#pragma clang fp contract(off)
    const int lane = threadIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int D = a.dk, dim = a.dim;
    const int tile = a.position / 8 + (int)blockIdx.x;
    const int t_lo = max(tile * 8, a.position), t_hi = min(tile * 8 + 8, a.position + a.tokens);
    if (t_lo >= t_hi || lane >= D / 2) return;
    const bool fp8 = a.format == CQKV_FMT_FP8 || a.format == CQKV_FMT_MXFP8;
    const int64_t plane = (int64_t)b * a.kv_heads + h;
    const uint8_t *codes = a.codes + plane * a.codes_plane;
    const uint8_t *scales = a.scales + plane * a.scales_plane;
    const float *tscale = (const float *)(scales + (int64_t)a.capacity * a.nblk);
    const bool prod = a.format == CQKV_FMT_TURBOPROD;
    for (int t = t_lo; t < t_hi; ++t) {
        const int s = t & 7;
        uint32_t c[2];
        if (!a.is_value) {
            if (fp8) {
                c[0] = codes[(int64_t)t * D + 2 * lane];
                c[1] = codes[(int64_t)t * D + 2 * lane + 1];
            } else {
                const uint32_t by = codes[(int64_t)t * (D / 2) + lane];
                c[0] = by & 15u;
                c[1] = by >> 4;
            }
        } else if (fp8) {  // 8-token tiles: element j at byte j * 8 + t % 8
            c[0] = codes[(int64_t)(t / 8) * D * 8 + 2 * lane * 8 + s];
            c[1] = codes[(int64_t)(t / 8) * D * 8 + (2 * lane + 1) * 8 + s];
        } else {           // nibble t % 8 of u32 j
            const uint32_t *w = (const uint32_t *)(codes + (int64_t)(t / 8) * D * 4) + 2 * lane;
            c[0] = (w[0] >> (4 * s)) & 15u;
            c[1] = (w[1] >> (4 * s)) & 15u;
        }
        // rsc0: the token's f32 (FP8 scale, TurboQuant norm, NVFP4 global scale) or 1.0 (MX)
        const bool tok = a.format != CQKV_FMT_MXFP4 && a.format != CQKV_FMT_MXFP8;
        const float r0 = tok ? tscale[t] : 1.0f;
        const int64_t row = ((int64_t)b * a.kv_heads + h) * a.tokens + (t - a.position);
        const int64_t o = (int64_t)b * a.os0 + (int64_t)h * a.os1 + (int64_t)(t - a.position) * a.os2;
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const int j = 2 * lane + e;
            if (j >= dim) break;
            float el;
            switch (a.format) {
            case CQKV_FMT_FP8: el = e4m3_value(c[e]); break;
            case CQKV_FMT_MXFP4: el = fp4_value(c[e]) * e8m0_value(scales[(int64_t)t * a.nblk + j / 32]); break;
            case CQKV_FMT_MXFP8: el = e4m3_value(c[e]) * e8m0_value(scales[(int64_t)t * a.nblk + j / 32]); break;
            case CQKV_FMT_NVFP4: el = fp4_value(c[e]) * e4m3_value(scales[(int64_t)t * a.nblk + j / 16]); break;
            default: el = a.cent[c[e] & 15u]; break;  // TurboQuant: the codebook centroid
            }
            store_elem(a.out, o + j, a.out_dtype, r0 * el);
        }
        if (prod) {  // the QJL coefficients z_i of sign bits i = 2 lane, 2 lane + 1
            const float r1 = ((const float *)(scales + (int64_t)a.capacity * 4))[t];
            const float cq = r0 * r1 * 1.2533141f / (float)dim;  // QJL_CONST, turbo.rs:26
            const uint32_t *sg = (const uint32_t *)(scales + (int64_t)a.capacity * 8) + (int64_t)t * (D / 32);
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const int i = 2 * lane + e;
                if (i >= dim) break;
                a.zs[row * dim + i] = ((sg[i >> 5] >> (i & 31)) & 1u) ? cq : -cq;
            }
        }
    }
}

int fill_turbo_bounds(const cqkv_side *s, float bnd[16], float *cent_out);

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// Workspace: the f32 rows before the correction / unrotation, then the QJL coefficients.
static size_t dequant_workspace(const cqkv_side *s, int32_t batch, int32_t tokens, bool unrotate,
                                size_t *zs_off) {
    const size_t rows = (size_t)batch * s->kv_heads * tokens, n = align256(rows * s->head_dim * 4);
    const bool prod = s->format == CQKV_FMT_TURBOPROD, unrot = unrotate && side_rotates(s);
    *zs_off = n;
    return prod ? 2 * n : unrot ? n : 0;
}

}  // namespace cqkv

using namespace cqkv;

extern "C" size_t cqkv_dequantize_workspace_bytes(const cqkv_side *side, int32_t batch,
                                                  int32_t tokens, int32_t unrotate) {
    clear_error();
    if (check_side(side, "cqkv_dequantize_workspace_bytes") != CQKV_OK || batch <= 0 || tokens <= 0)
        return 0;
    size_t zs_off;
    return dequant_workspace(side, batch, tokens, unrotate != 0, &zs_off);
}

extern "C" int cqkv_dequantize_rows(const cqkv_side *side, int32_t batch, int32_t position,
                                    int32_t tokens, int32_t unrotate, void *out, int32_t out_dtype,
                                    const int64_t out_strides[3], void *workspace,
                                    size_t workspace_bytes, cqkv_stream_t stream) {
    clear_error();
    static const char *who = "cqkv_dequantize_rows";
    if (int rc = check_side(side, who)) return rc;
    if (!out || !out_strides) return fail(CQKV_ERR_ARG, "%s: null out / strides", who);
    if (out_dtype < CQKV_BF16 || out_dtype > CQKV_F32)
        return fail(CQKV_ERR_ARG, "%s: out dtype %d", who, out_dtype);
    if (batch <= 0 || tokens < 0 || position < 0 || (int64_t)position + tokens > side->capacity)
        return fail(CQKV_ERR_ARG, "%s: batch %d, tokens [%d, %lld) outside the capacity %d", who,
                    batch, position, (long long)position + tokens, side->capacity);
    const bool unrot = unrotate != 0 && side_rotates(side);
    if (unrot && !side->rot)
        return fail(CQKV_ERR_ARG, "%s: unrotating a rotating side needs its matrix (rot)", who);
    if (tokens == 0) return CQKV_OK;
    const int d = side->head_dim, hkv = side->kv_heads;
    const bool prod = side->format == CQKV_FMT_TURBOPROD;
    size_t zs_off;
    const size_t need = dequant_workspace(side, batch, tokens, unrotate != 0, &zs_off);
    const hipStream_t st = (hipStream_t)stream;
    void *ws = workspace;
    bool owned = false;
    if (need) {
        if (ws && workspace_bytes < need)
            return fail(CQKV_ERR_WORKSPACE, "%s: workspace %zu < %zu bytes", who, workspace_bytes, need);
        if (!ws) {
            CQKV_HIP_CHECK(hipMallocAsync(&ws, need, st));
            owned = true;
        }
    }
    DequantArgs a = {};
    a.codes = (const uint8_t *)side->codes;
    a.scales = (const uint8_t *)side->scales;
    a.codes_plane = (uint32_t)cqkv_codes_plane_bytes(side->format, d, side->capacity);
    a.scales_plane = (uint32_t)cqkv_scales_plane_bytes(side->format, d, side->capacity);
    a.kv_heads = hkv;
    a.tokens = tokens;
    a.position = position;
    a.capacity = side->capacity;
    a.dk = kernel_dim(d);
    a.dim = d;
    a.format = side->format;
    a.is_value = side->is_value;
    a.nblk = block_elems(side->format) ? a.dk / block_elems(side->format) : 0;
    int rc = CQKV_OK;
    if (is_turbo(side->format)) {
        float bnd[16];
        rc = fill_turbo_bounds(side, bnd, a.cent);
    }
    // the f32 rows go to the workspace when a correction or an unrotation follows
    const int64_t fs[3] = {(int64_t)hkv * tokens * d, (int64_t)tokens * d, d};
    float *rows32 = (float *)ws;
    if (prod || unrot) {
        a.out = rows32;
        a.out_dtype = CQKV_F32;
        a.os0 = fs[0];
        a.os1 = fs[1];
        a.os2 = fs[2];
        a.zs = prod ? (float *)((char *)ws + zs_off) : nullptr;
    } else {
        a.out = out;
        a.out_dtype = out_dtype;
        a.os0 = out_strides[0];
        a.os1 = out_strides[1];
        a.os2 = out_strides[2];
    }
    hipError_t e = hipSuccess;
    if (rc == CQKV_OK) {
        const dim3 grid((unsigned)((tokens + (position % 8) + 7) / 8), hkv, batch);
        hipLaunchKernelGGL(dequant_kernel, grid, dim3(a.dk == 256 ? 128 : 64), 0, st, a);
        e = hipGetLastError();
    }
    if (rc == CQKV_OK && e == hipSuccess && prod) {
        // y = mse + z S, in place over the f32 rows (each output tile reads its own base first),
        // or straight into out when nothing follows
        const int64_t ys[3] = {unrot ? fs[0] : out_strides[0], unrot ? fs[1] : out_strides[1],
                               unrot ? fs[2] : out_strides[2]};
        RowMatArgs r = rowmat_args(a.zs, CQKV_F32, fs, batch, hkv, tokens, d, unrot ? (void *)rows32 : out,
                                   unrot ? CQKV_F32 : out_dtype, ys, d);
        r.m = side->qjl;
        r.transpose = 0;
        r.base = rows32;
        r.base_stride = d;
        e = rowmat_launch(r, st);
    }
    if (rc == CQKV_OK && e == hipSuccess && unrot) {  // y Pi into out
        RowMatArgs r = rowmat_args(rows32, CQKV_F32, fs, batch, hkv, tokens, d, out, out_dtype,
                                   out_strides, d);
        r.m = side->rot;
        r.transpose = 0;
        e = rowmat_launch(r, st);
    }
    if (owned) {
        const hipError_t fe = hipFreeAsync(ws, st);
        if (e == hipSuccess) e = fe;
    }
    if (rc != CQKV_OK) return rc;
    if (e != hipSuccess) return fail(CQKV_ERR_HIP, "%s: %s", who, hipGetErrorString(e));
    return CQKV_OK;
}
