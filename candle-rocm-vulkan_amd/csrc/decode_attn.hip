// Host side of the decode entry points (dense, allocation-free and paged decode) and the split
// combine kernel. The decode kernels are in decode_kernels.h.
#include <algorithm>
#include <mutex>
#include <vector>

#include "decode_kernels.h"
#include "rowmat.h"

namespace cqkv {

struct CombineArgs {
    const float *part_o, *part_lse;
    int32_t splits, rows, q_heads, q_len, out_dtype, rotate;
    void *out;
    int64_t o_sb, o_sh, o_si;
    uint32_t vsign_bits[8];
    float rot_scale;
    int32_t head_dim;  // outputs past it (plane row padding) are not written
};

// Split combine (the formula of tq_combine_impl, candle-core/kernels/turbo_quant_impl.h:659-685,
// in the log2 domain): o = sum_s w_s o_s / sum_s w_s, w_s = 2^(lse_s - max lse), empty splits
// skipped; then, for values with the in-register Hadamard rotation, x = sign * (H o) / sqrt(D)
// (the unrotation y Pi). One wavefront per output row (lane l: head dims 2l, 2l+1, and
// 128 + 2l, 129 + 2l at D = 256), four rows per workgroup; the split loop keeps up to 8 splits'
// loads in flight.
template <int D>
__global__ __launch_bounds__(256) void combine_kernel(CombineArgs a) {
    constexpr int NP = D == 256 ? 2 : 1;  // element pairs per lane
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= a.rows) return;
    const bool active = lane < D / 2 / NP;
    const float *lse = a.part_lse + row;
    float M = -__builtin_inff();
    for (int s = 0; s < a.splits; ++s) M = fmaxf(M, lse[(int64_t)s * a.rows]);
    float o[2 * NP] = {};
    if (M != -__builtin_inff()) {
        float wsum = 0.0f, acc[2 * NP] = {};
        const float *po = a.part_o + (int64_t)row * D + 2 * (active ? lane : 0);
        const int64_t step = (int64_t)a.rows * D;
#pragma unroll 8
        for (int s = 0; s < a.splits; ++s) {
            const float e = lse[(int64_t)s * a.rows];
            const float w = e == -__builtin_inff() ? 0.0f : __builtin_amdgcn_exp2f(e - M);
            wsum += w;
#pragma unroll
            for (int p = 0; p < NP; ++p) {
                const f32x2 v = *(const f32x2 *)(po + s * step + 128 * p);
                acc[2 * p] += w * v.x;
                acc[2 * p + 1] += w * v.y;
            }
        }
#pragma unroll
        for (int k = 0; k < 2 * NP; ++k) o[k] = acc[k] / wsum;
    }
    if (a.rotate) {
        if constexpr (D == 256) fwht_quads_dec(o[0], o[1], o[2], o[3], lane);
        else fwht_pairs_dec<D>(o[0], o[1], lane);
#pragma unroll
        for (int p = 0; p < NP; ++p)
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                o[2 * p + e] *= a.rot_scale;
                if (active && sign_bit(a.vsign_bits, 128 * p + 2 * lane + e)) o[2 * p + e] = -o[2 * p + e];
            }
    }
    if (!active) return;
    const int qi = row % a.q_len, head = (row / a.q_len) % a.q_heads;
    const int b = row / (a.q_len * a.q_heads);
    const int64_t base = (int64_t)b * a.o_sb + (int64_t)head * a.o_sh + (int64_t)qi * a.o_si;
#pragma unroll
    for (int p = 0; p < NP; ++p)
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const int j = 128 * p + 2 * lane + e;
            if (j < a.head_dim) store_elem(a.out, base + j, a.out_dtype, o[2 * p + e]);
        }
}

void fill_rotation(const cqkv_side *s, uint32_t sign_bits[8], float *rot_scale);

static int tiles_of(int kv_len) { return (kv_len + 31) / 32; }

// Compute units of the current device (hipDeviceAttributeMultiprocessorCount, cached per device;
// 256, the MI355X's, when there is no device to ask).
static int device_cus() {
    constexpr int kMaxDev = 64;
    static int cache[kMaxDev];
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDev) {
        (void)hipGetLastError();
        return 256;
    }
    if (!cache[dev]) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) {
            (void)hipGetLastError();
            n = 256;
        }
        cache[dev] = n;
    }
    return cache[dev];
}

// Key splits per (batch, kv head). One 8-wavefront workgroup per plane fills a CU (two waves per
// SIMD at this register budget; twice as many workgroups of 4 wavefronts): split only when
// there are fewer planes than the device's CUs take, and then into pieces of at least two tiles
// per wavefront. Ragged batches (per-sequence lengths) are split into pieces of at most 128 tiles
// (4096 keys) so long and short sequences even out across CUs.
static int auto_splits(int batch, int kv_heads, int kv_len, bool ragged, int waves = kWaves) {
    const int planes = batch * kv_heads;
    const int tiles = tiles_of(kv_len);
    const int wgs = device_cus() * (kWaves / waves);  // workgroups that fill the chip
    int s = (wgs + planes - 1) / planes;
    if (ragged) s = max(s, (tiles + 127) / 128);
    s = min(s, max(1, tiles / (2 * waves)));
    s = max(1, min(s, 256));
    const int tps = (tiles + s - 1) / s;
    return max(1, (tiles + tps - 1) / tps);
}


static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// Workspace (D' = the plane row length of head_dim): partial outputs (splits, rows, D') f32 |
// partial lse (splits, rows) f32 | rotated queries (rows, D') f32 | combined outputs before the
// matrix unrotation (rows, D') f32 | the padded QJL matrix (D', D') f32. The last three (extras)
// serve the sides that rotate by their matrix and TurboProd keys at a head dim below D'; the
// size query reserves them whatever the formats, so its answer depends on the shapes only, and a
// call that needs none of them uses only the partials.
struct DecodeWs {
    size_t lse, qrot, otmp, qjl, total;
};
static DecodeWs workspace_layout(int32_t batch, int32_t q_heads, int32_t q_len, int32_t head_dim,
                                 int32_t splits, bool extras = true) {
    const size_t rows = (size_t)batch * q_heads * q_len, dk = (size_t)kernel_dim(head_dim);
    DecodeWs w;
    w.lse = align256((size_t)splits * rows * dk * 4);
    w.qrot = w.lse + align256((size_t)splits * rows * 4);
    w.otmp = w.qrot + (extras ? align256(rows * dk * 4) : 0);
    w.qjl = w.otmp + (extras ? align256(rows * dk * 4) : 0);
    w.total = w.qjl + (extras ? align256(dk * dk * 4) : 0);
    return w;
}

}  // namespace cqkv

using namespace cqkv;

extern "C" int32_t cqkv_decode_splits(int32_t k_format, int32_t v_format, int32_t batch,
                                      int32_t kv_heads, int32_t kv_len, int32_t ragged) {
    if (batch <= 0 || kv_heads <= 0 || kv_len <= 0) return 1;
    return auto_splits(batch, kv_heads, kv_len, ragged != 0, waves_of(k_format, v_format));
}

extern "C" size_t cqkv_decode_workspace_bytes(int32_t batch, int32_t q_heads, int32_t q_len,
                                              int32_t head_dim, int32_t splits) {
    if (batch <= 0 || q_heads <= 0 || q_len <= 0 || head_dim <= 0 || head_dim > 256 || splits <= 0)
        return 0;
    return workspace_layout(batch, q_heads, q_len, head_dim, splits).total;
}

// Checks and fills what the dense and the paged calls share: queries, output, heads, scale,
// window, TurboQuant rotation and codebook. k / v give the format, head dim and kv heads.
// Host-side parts of a decode call beyond the kernel arguments: the matrix rotations.
struct DecodeHost {
    const float *k_rot = nullptr;  // rotate the queries by this matrix first (x Pi_k^T)
    const float *v_rot = nullptr;  // unrotate the combined output by this matrix (y Pi_v)
    const cqkv_side *k = nullptr;  // the key side (TURBOPROD at a padded head dim: S padded)
    int32_t head_dim = 0, q_dtype = 0;
    const void *q = nullptr;
    int64_t q_strides[3] = {0, 0, 0};
};

static int decode_prepare(DecodeArgs &a, DecodeHost &h, const char *who, const void *q,
                          int32_t q_dtype, const int64_t q_strides[3], const cqkv_side *k,
                          const cqkv_side *v, int32_t batch, int32_t q_heads, int32_t q_len,
                          float softmax_scale, int32_t window_left, int32_t window_right,
                          float softcap, const float *alibi_slopes, int32_t alibi_batch_stride,
                          void *out, int32_t out_dtype, const int64_t out_strides[3]) {
    if (int rc = check_side(k, who)) return rc;
    if (int rc = check_side(v, who)) return rc;
    if (k->is_value != 0 || v->is_value != 1)
        return fail(CQKV_ERR_ARG, "%s: expected a key side and a value side", who);
    if (k->head_dim != v->head_dim || k->kv_heads != v->kv_heads)
        return fail(CQKV_ERR_ARG, "%s: key / value sides differ in D or heads", who);
    // no query rows (batch or q_len 0): an empty output, as the reference's (rocm_backend/
    // accel.rs:481); q / out may then be null and the callers launch nothing
    const bool no_rows = batch == 0 || q_len == 0;
    if ((!no_rows && (!q || !out)) || !q_strides || !out_strides)
        return fail(CQKV_ERR_ARG, "%s: null q / out / strides", who);
    if (q_dtype < CQKV_BF16 || q_dtype > CQKV_F32 || out_dtype < CQKV_BF16 || out_dtype > CQKV_F32)
        return fail(CQKV_ERR_ARG, "%s: dtypes q %d out %d", who, q_dtype, out_dtype);
    const int hkv = k->kv_heads, d = k->head_dim;
    if (batch < 0 || q_heads <= 0 || q_len < 0 || q_heads % hkv != 0)
        return fail(CQKV_ERR_ARG, "%s: batch %d q_heads %d q_len %d kv_heads %d", who, batch,
                    q_heads, q_len, hkv);
    const int group = q_heads / hkv;
    if ((int64_t)group * q_len > (1 << 24))
        return fail(CQKV_ERR_ARG, "%s: q_len * q_heads / kv_heads = %lld above 2^24", who,
                    (long long)group * q_len);
    if (!(softcap >= 0.0f) || softcap == __builtin_inff())
        return fail(CQKV_ERR_ARG, "%s: softcap %g (finite, >= 0; 0 disables it)", who,
                    (double)softcap);
    if (alibi_slopes && alibi_batch_stride != 0 && alibi_batch_stride != q_heads)
        return fail(CQKV_ERR_ARG, "%s: alibi batch stride %d (0 or q_heads %d)", who,
                    alibi_batch_stride, q_heads);
    a = DecodeArgs{};
    h = DecodeHost{};
    a.cap2 = softcap * kLog2e;
    a.alibi = alibi_slopes;
    a.alibi_bs = alibi_batch_stride;
    a.q = q;
    a.q_sb = q_strides[0];
    a.q_sh = q_strides[1];
    a.q_si = q_strides[2];
    a.q_dtype = q_dtype;
    a.q_heads = q_heads;
    a.kv_heads = hkv;
    a.group = group;
    a.q_len = q_len;
    a.ncols = group * q_len;
    a.col_blocks = (a.ncols + 15) / 16;
    a.scale_log2 = softmax_scale * kLog2e;
    a.wl = window_left;
    a.wr = window_right;
    a.batch = batch;
    a.out = out;
    a.out_dtype = out_dtype;
    a.rot_k = side_fwht(k) ? 1 : 0;
    a.rot_v = side_fwht(v) ? 1 : 0;
    a.head_dim = d;
    a.qjl_c = -kQjlConst / (float)d;
    if (side_matrix_rot(k)) h.k_rot = k->rot;
    if (side_matrix_rot(v)) h.v_rot = v->rot;
    a.partials = a.rot_v || h.v_rot ? 1 : 0;
    h.k = k;
    h.head_dim = d;
    h.q = q;
    h.q_dtype = q_dtype;
    for (int i = 0; i < 3; ++i) h.q_strides[i] = q_strides[i];
    // queries not representable in the operand type get a lo part (f16 / f32 inputs, or rotated
    // queries, for the bf16 key formats); TurboQuant keys take the rotated queries as one f16
    // operand (2^-12 relative rounding: config 5 216-225 -> 208-220 us same-box, its parity tests
    // unchanged)
    a.q_split = !is_turbo(k->format) && (q_dtype != CQKV_BF16 || a.rot_k || h.k_rot) ? 1 : 0;
    a.o_sb = out_strides[0];
    a.o_sh = out_strides[1];
    a.o_si = out_strides[2];
    float rs;
    fill_rotation(k, a.ksign_bits, &rs);
    fill_rotation(v, a.vsign_bits, &rs);
    a.rot_scale = 1.0f / sqrtf((float)d);
    // kernel formats: TurboMse keys and values of different widths cannot share the 64 KB code
    // table, so the side with the narrower (at most 3-bit) codes takes a compact table of its own
    // TurboProd{5} keys (4-bit MSE codes) decode their codes through the 64 KB table
    const int kb = turbo_code_bits(k), vb = turbo_code_bits(v);
    a.kfmt = k->format == CQKV_FMT_TURBOPROD && kb == 4 ? kFmtProd4 : k->format;
    a.vfmt = v->format;
    const bool k_tab = a.kfmt == CQKV_FMT_TURBO4 || a.kfmt == kFmtProd4;  // keys on the 64 KB table
    if (k_tab && v->format == CQKV_FMT_TURBO4 && kb != vb) {
        if (kb <= 3) a.kfmt = kFmtTurboC;
        else a.vfmt = kFmtTurboC;
    }
    float bnd[16], cent[16];
    const bool k_tab2 = a.kfmt == CQKV_FMT_TURBO4 || a.kfmt == kFmtProd4;
    if (k_tab2 || a.vfmt == CQKV_FMT_TURBO4) {  // the 64 KB table's codebook
        if (turbo_codebook(d, k_tab2 ? kb : vb, cent, bnd) != 0)
            return fail(CQKV_ERR_ARG, "%s: turbo codebook D=%d", who, d);
        for (int i = 0; i < 16; ++i) a.cent[i] = cent[i];
    }
    if (a.kfmt == CQKV_FMT_TURBOPROD || a.kfmt == kFmtTurboC) {  // compact key codebook
        if (turbo_codebook(d, kb, cent, bnd) != 0)
            return fail(CQKV_ERR_ARG, "%s: turbo codebook D=%d", who, d);
        for (int i = 0; i < (1 << kb); ++i) a.kcent[i] = cent[i];
    }
    if (a.vfmt == kFmtTurboC) {  // compact value codebook
        if (turbo_codebook(d, vb, cent, bnd) != 0)
            return fail(CQKV_ERR_ARG, "%s: turbo codebook D=%d", who, d);
        for (int i = 0; i < (1 << vb); ++i) a.vcent[i] = cent[i];
    }
    if (k->format == CQKV_FMT_TURBOPROD) a.qjl = k->qjl;
    return CQKV_OK;
}

// Launches a decode over a.splits splits: the query rotation by the key side's matrix (into the
// workspace's rotated-query region), the decode kernel, the combine for more than one split or
// when a.partials, and the unrotation by the value side's matrix (from the workspace's combined
// output region). ws: the call's workspace (layout w) when one is needed.
static hipError_t decode_launch(DecodeArgs a, const DecodeHost &h, int kf, int vf, void *ws,
                                const DecodeWs &w, hipStream_t st) {
    const int d = h.head_dim, dk = kernel_dim(d);
    const int rows = a.batch * a.q_heads * a.q_len;
    if (h.k_rot) {  // q Pi_k^T, f32, padded to the plane row
        float *qr = (float *)((char *)ws + w.qrot);
        const int64_t ys[3] = {(int64_t)a.q_heads * a.q_len * dk, (int64_t)a.q_len * dk, dk};
        RowMatArgs r = rowmat_args(h.q, h.q_dtype, h.q_strides, a.batch, a.q_heads, a.q_len, d, qr,
                                   CQKV_F32, ys, dk);
        r.m = h.k_rot;
        r.transpose = 1;
        if (hipError_t e = rowmat_launch(r, st)) return e;
        a.q = qr;
        a.q_dtype = CQKV_F32;
        a.q_sb = ys[0];
        a.q_sh = ys[1];
        a.q_si = ys[2];
    }
    if (h.k->format == CQKV_FMT_TURBOPROD && d != dk) {  // S padded to the plane row
        float *sp = (float *)((char *)ws + w.qjl);
        const int64_t xs[3] = {0, 0, d}, ys[3] = {0, 0, dk};
        RowMatArgs r = rowmat_args(h.k->qjl, CQKV_F32, xs, 1, 1, dk, d, sp, CQKV_F32, ys, dk);
        r.xrows = d;
        if (hipError_t e = rowmat_launch(r, st)) return e;
        a.qjl = sp;
    }
    const int64_t wgs = (int64_t)a.splits * a.col_blocks * a.kv_heads * a.batch;
    if (wgs > 0x7fffffff) return hipErrorInvalidConfiguration;
    const dim3 grid((unsigned)wgs);
    bool ok = false;
    switch (kf) {
    case CQKV_FMT_FP8: ok = decode_launch_k5(vf, dk, grid, st, a); break;
    case CQKV_FMT_MXFP4: ok = decode_launch_k2(vf, dk, grid, st, a); break;
    case CQKV_FMT_MXFP8: ok = decode_launch_k4(vf, dk, grid, st, a); break;
    case CQKV_FMT_NVFP4: ok = decode_launch_k3(vf, dk, grid, st, a); break;
    case CQKV_FMT_TURBOPROD: ok = decode_launch_k1(vf, dk, grid, st, a); break;
    case kFmtTurboC: ok = decode_launch_k6(vf, dk, grid, st, a); break;
    case kFmtProd4: ok = decode_launch_k7(vf, dk, grid, st, a); break;
    case CQKV_FMT_TURBO4: ok = decode_launch_k0(vf, dk, grid, st, a); break;
    default: break;
    }
    if (!ok) return hipErrorInvalidValue;  // a key / value format pairing without a kernel
    hipError_t e = hipGetLastError();
    if (e == hipSuccess && (a.splits > 1 || a.partials)) {
        CombineArgs c = {};
        c.part_o = a.part_o;
        c.part_lse = a.part_lse;
        c.splits = a.splits;
        c.rows = rows;
        c.q_heads = a.q_heads;
        c.q_len = a.q_len;
        c.rotate = a.rot_v;
        c.head_dim = d;
        if (h.v_rot) {  // combined rows to the workspace, f32, for the unrotation below
            c.out = (char *)ws + w.otmp;
            c.out_dtype = CQKV_F32;
            c.o_sb = (int64_t)a.q_heads * a.q_len * d;
            c.o_sh = (int64_t)a.q_len * d;
            c.o_si = d;
        } else {
            c.out = a.out;
            c.out_dtype = a.out_dtype;
            c.o_sb = a.o_sb;
            c.o_sh = a.o_sh;
            c.o_si = a.o_si;
        }
        for (int i = 0; i < 8; ++i) c.vsign_bits[i] = a.vsign_bits[i];
        c.rot_scale = a.rot_scale;
        const dim3 cg((c.rows + 3) / 4);
        if (dk == 64) hipLaunchKernelGGL(combine_kernel<64>, cg, dim3(256), 0, st, c);
        else if (dk == 128) hipLaunchKernelGGL(combine_kernel<128>, cg, dim3(256), 0, st, c);
        else hipLaunchKernelGGL(combine_kernel<256>, cg, dim3(256), 0, st, c);
        e = hipGetLastError();
        if (e == hipSuccess && h.v_rot) {  // y Pi_v into the output
            const int64_t xs[3] = {c.o_sb, c.o_sh, c.o_si}, ys[3] = {a.o_sb, a.o_sh, a.o_si};
            RowMatArgs r = rowmat_args(c.out, CQKV_F32, xs, a.batch, a.q_heads, a.q_len, d, a.out,
                                       a.out_dtype, ys, d);
            r.m = h.v_rot;
            r.transpose = 0;
            e = rowmat_launch(r, st);
        }
    }
    return e;
}

// Whether a decode call needs the workspace's extra regions (matrix rotations, padded QJL matrix).
static bool needs_extras(const DecodeHost &h) {
    return h.k_rot || h.v_rot ||
           (h.k->format == CQKV_FMT_TURBOPROD && h.head_dim != kernel_dim(h.head_dim));
}

// Whether a decode call needs its workspace: partials, or the extra regions.
static bool needs_workspace(const DecodeArgs &a, const DecodeHost &h) {
    return a.splits > 1 || a.partials || needs_extras(h);
}

// ---- allocation-free decode: split partials in a library-owned device array ----
// `scratch` is one array per GPU (each device that loads the library's code object holds its own
// copy at its own address), kept until the process ends. In host code its name is only a
// host-side stand-in: the device address comes from hipGetSymbolAddress, fetched once per device
// with that device current, and only that address is ever handed to kernels. Every
// cqkv_decode_attention_noalloc call on a GPU shares that GPU's array; calls that overlap on one
// GPU (concurrent streams) race on it.
static __device__ __attribute__((aligned(256))) uint8_t scratch[CQKV_DECODE_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static void *g_scratch_ptr[kMaxDevices];

static int scratch_address(void **out, const char *who) {
    int dev = -1;
    CQKV_HIP_CHECK(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxDevices)
        return fail(CQKV_ERR_ARG, "%s: device ordinal %d above %d", who, dev, kMaxDevices - 1);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return fail(CQKV_ERR_HIP, "%s: hipGetSymbolAddress(scratch) on device %d: %s", who,
                        dev, hipGetErrorString(e));
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return CQKV_OK;
}

// The dense decode of both entry points. noalloc: the partials go to the device `scratch` array
// (automatic splits are lowered until they fit; explicit ones that do not fit are refused);
// otherwise to `workspace`, or to a stream-ordered allocation when none is given.
static int decode_dense(const char *who, const void *q, int32_t q_dtype,
                        const int64_t q_strides[3], const cqkv_side *k, const cqkv_side *v,
                        int32_t batch, int32_t q_heads, int32_t q_len, const int32_t *kv_lens,
                        int32_t kv_len, float softmax_scale, int32_t window_left,
                        int32_t window_right, float softcap, const float *alibi_slopes,
                        int32_t alibi_batch_stride, void *out, int32_t out_dtype,
                        const int64_t out_strides[3], int32_t splits, void *workspace,
                        size_t workspace_bytes, bool noalloc, cqkv_stream_t stream) {
    DecodeArgs a;
    DecodeHost h;
    if (int rc = decode_prepare(a, h, who, q, q_dtype, q_strides, k, v, batch, q_heads, q_len,
                                softmax_scale, window_left, window_right, softcap, alibi_slopes,
                                alibi_batch_stride, out, out_dtype, out_strides))
        return rc;
    if (k->capacity != v->capacity)
        return fail(CQKV_ERR_ARG, "%s: key / value capacities %d / %d differ", who, k->capacity,
                    v->capacity);
    if (kv_len < 0 || kv_len > k->capacity)
        return fail(CQKV_ERR_ARG, "%s: kv_len %d outside [0, capacity %d]", who, kv_len,
                    k->capacity);
    if (splits < 0) return fail(CQKV_ERR_ARG, "%s: splits %d", who, splits);
    if (batch == 0 || q_len == 0) return CQKV_OK;
    const int hkv = k->kv_heads, d = k->head_dim;

    const int tiles = max(1, tiles_of(kv_len));
    int s = splits > 0 ? min(splits, tiles)
                       : auto_splits(batch, hkv, max(kv_len, 1), kv_lens != nullptr,
                                     waves_of(k->format, v->format));
    const bool extras = needs_extras(h);
    if (noalloc) {  // everything the call needs must fit the device scratch
        auto fits = [&](int n) {
            a.splits = n;
            return !needs_workspace(a, h) || workspace_layout(batch, q_heads, q_len, d, n, extras)
                                                     .total <= CQKV_DECODE_SCRATCH_BYTES;
        };
        if (!fits(s) && splits > 0)
            return fail(CQKV_ERR_WORKSPACE,
                        "%s: %d splits need %zu bytes of partials, above the %zu-byte device "
                        "scratch",
                        who, s, workspace_layout(batch, q_heads, q_len, d, s, extras).total,
                        (size_t)CQKV_DECODE_SCRATCH_BYTES);
        while (s > 1 && !fits(s)) --s;
        if (!fits(s))
            return fail(CQKV_ERR_WORKSPACE,
                        "%s: %zu bytes of partials and rotation buffers exceed the %zu-byte "
                        "device scratch",
                        who, workspace_layout(batch, q_heads, q_len, d, s, extras).total,
                        (size_t)CQKV_DECODE_SCRATCH_BYTES);
    }
    const int tps = (tiles + s - 1) / s;
    s = (tiles + tps - 1) / tps;

    a.kc = (const uint8_t *)k->codes;
    a.ks = (const uint8_t *)k->scales;
    a.vc = (const uint8_t *)v->codes;
    a.vs = (const uint8_t *)v->scales;
    a.kc_plane = (uint32_t)cqkv_codes_plane_bytes(k->format, d, k->capacity);
    a.ks_plane = (uint32_t)cqkv_scales_plane_bytes(k->format, d, k->capacity);
    a.vc_plane = (uint32_t)cqkv_codes_plane_bytes(v->format, d, v->capacity);
    a.vs_plane = (uint32_t)cqkv_scales_plane_bytes(v->format, d, v->capacity);
    a.kv_lens = kv_lens;
    a.kv_len = kv_len;
    a.tiles_per_split = tps;
    a.splits = s;

    hipStream_t st = (hipStream_t)stream;
    void *ws = workspace;
    bool owned = false;
    const DecodeWs w = workspace_layout(batch, q_heads, q_len, d, s, extras);
    if (needs_workspace(a, h)) {
        if (noalloc) {
            if (int rc = scratch_address(&ws, who)) return rc;
        } else if (ws && workspace_bytes < w.total) {
            return fail(CQKV_ERR_WORKSPACE, "%s: workspace %zu < %zu bytes", who,
                        workspace_bytes, w.total);
        } else if (!ws) {
            CQKV_HIP_CHECK(hipMallocAsync(&ws, w.total, st));
            owned = true;
        }
        a.part_o = (float *)ws;
        a.part_lse = (float *)((char *)ws + w.lse);
    }
    hipError_t e = decode_launch(a, h, a.kfmt, a.vfmt, ws, w, st);
    if (owned) {
        hipError_t fe = hipFreeAsync(ws, st);
        if (e == hipSuccess) e = fe;
    }
    if (e != hipSuccess) return fail(CQKV_ERR_HIP, "%s: launch failed: %s", who, hipGetErrorString(e));
    return CQKV_OK;
}

extern "C" int cqkv_decode_attention(const void *q, int32_t q_dtype, const int64_t q_strides[3],
                                     const cqkv_side *k, const cqkv_side *v, int32_t batch,
                                     int32_t q_heads, int32_t q_len, const int32_t *kv_lens,
                                     int32_t kv_len, float softmax_scale, int32_t window_left,
                                     int32_t window_right, float softcap,
                                     const float *alibi_slopes, int32_t alibi_batch_stride,
                                     void *out, int32_t out_dtype, const int64_t out_strides[3],
                                     int32_t splits, void *workspace, size_t workspace_bytes,
                                     cqkv_stream_t stream) {
    clear_error();
    return decode_dense("cqkv_decode_attention", q, q_dtype, q_strides, k, v, batch, q_heads,
                        q_len, kv_lens, kv_len, softmax_scale, window_left, window_right, softcap,
                        alibi_slopes, alibi_batch_stride, out, out_dtype, out_strides, splits,
                        workspace, workspace_bytes, false, stream);
}

extern "C" int cqkv_decode_attention_noalloc(const void *q, int32_t q_dtype,
                                             const int64_t q_strides[3], const cqkv_side *k,
                                             const cqkv_side *v, int32_t batch, int32_t q_heads,
                                             int32_t q_len, const int32_t *kv_lens,
                                             int32_t kv_len, float softmax_scale,
                                             int32_t window_left, int32_t window_right,
                                             float softcap, const float *alibi_slopes,
                                             int32_t alibi_batch_stride, void *out,
                                             int32_t out_dtype, const int64_t out_strides[3],
                                             int32_t splits, cqkv_stream_t stream) {
    clear_error();
    return decode_dense("cqkv_decode_attention_noalloc", q, q_dtype, q_strides, k, v, batch,
                        q_heads, q_len, kv_lens, kv_len, softmax_scale, window_left,
                        window_right, softcap, alibi_slopes, alibi_batch_stride, out, out_dtype,
                        out_strides, splits, nullptr, 0, true, stream);
}

// ---- paged decode ----
// Segments of a block list: each block's valid rows, cut into runs of at most tps whole tiles;
// the run length is the dense split rule's for the total key count.
static int paged_segments(const cqkv_kv_block *blocks, int32_t n_blocks, int32_t batch,
                          std::vector<PagedSeg> *segs) {
    const cqkv_side *k0 = blocks[0].k;
    int64_t total = 0, tiles = 0;
    for (int i = 0; i < n_blocks; ++i) {
        total += blocks[i].rows;
        tiles += tiles_of(blocks[i].rows);
    }
    const int s = auto_splits(batch, k0->kv_heads, (int)std::max<int64_t>(total, 1), false,
                              waves_of(k0->format, blocks[0].v->format));
    const int tps = (int)std::max<int64_t>(1, (tiles + s - 1) / s);
    int key = 0, n = 0;
    for (int i = 0; i < n_blocks; ++i) {
        const cqkv_kv_block &bl = blocks[i];
        const int bt = tiles_of(bl.rows);
        for (int t = 0; t < bt; t += tps) {
            if (segs) {
                PagedSeg g = {};
                const int d = bl.k->head_dim;
                g.kc = (const uint8_t *)bl.k->codes;
                g.ks = (const uint8_t *)bl.k->scales;
                g.vc = (const uint8_t *)bl.v->codes;
                g.vs = (const uint8_t *)bl.v->scales;
                g.kc_plane = (uint32_t)cqkv_codes_plane_bytes(bl.k->format, d, bl.k->capacity);
                g.ks_plane = (uint32_t)cqkv_scales_plane_bytes(bl.k->format, d, bl.k->capacity);
                g.vc_plane = (uint32_t)cqkv_codes_plane_bytes(bl.v->format, d, bl.v->capacity);
                g.vs_plane = (uint32_t)cqkv_scales_plane_bytes(bl.v->format, d, bl.v->capacity);
                g.tile_begin = t;
                g.tile_end = min(t + tps, bt);
                g.key_offset = key;
                g.rows = bl.rows;
                segs->push_back(g);
            }
            ++n;
        }
        key += bl.rows;
    }
    return n;
}

// The segment table is written into the workspace by kernels that carry the segments by value
// in their arguments, kPagedSegsPerLaunch per launch: a captured HIP graph keeps kernel
// arguments by value, so replays see this call's table (a host -> device copy would keep a
// pointer to host memory freed when the call returns).
constexpr int kPagedSegsPerLaunch = 32;  // 32 x 64 B of kernel arguments
struct PagedTableArgs {
    PagedSeg seg[kPagedSegsPerLaunch];
    PagedSeg *dst;
    int32_t n;
};
__global__ __launch_bounds__(64) void paged_table_kernel(PagedTableArgs a) {
    // 16 words per segment; word w of segment i goes to lane w of iteration i
    const int lane = threadIdx.x;
    for (int i = lane / 16; i < a.n; i += 4)
        ((uint32_t *)(a.dst + i))[lane % 16] = ((const uint32_t *)(a.seg + i))[lane % 16];
}
static_assert(sizeof(PagedSeg) == 64, "paged_table_kernel copies 16 words per segment");

static hipError_t write_paged_table(const std::vector<PagedSeg> &segs, PagedSeg *dst,
                                    hipStream_t st) {
    for (size_t i0 = 0; i0 < segs.size(); i0 += kPagedSegsPerLaunch) {
        PagedTableArgs t = {};
        t.n = (int32_t)std::min<size_t>(kPagedSegsPerLaunch, segs.size() - i0);
        for (int i = 0; i < t.n; ++i) t.seg[i] = segs[i0 + i];
        t.dst = dst + i0;
        hipLaunchKernelGGL(paged_table_kernel, dim3(1), dim3(64), 0, st, t);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

// Workspace: the segment table, then the dense decode's workspace (partials, rotation buffers)
// for the segment count.
static size_t paged_workspace(int nseg, int32_t batch, int32_t q_heads, int32_t q_len,
                              int32_t head_dim, size_t *part_off, DecodeWs *w) {
    *part_off = align256((size_t)nseg * sizeof(PagedSeg));
    *w = workspace_layout(batch, q_heads, q_len, head_dim, nseg);
    return *part_off + w->total;
}

static int check_blocks(const cqkv_kv_block *blocks, int32_t n_blocks, int32_t batch,
                        const char *who) {
    if (!blocks || n_blocks <= 0) return fail(CQKV_ERR_ARG, "%s: no blocks", who);
    int64_t total = 0;
    for (int i = 0; i < n_blocks; ++i) {
        const cqkv_kv_block &bl = blocks[i];
        if (!bl.k || !bl.v) return fail(CQKV_ERR_ARG, "%s: block %d has a null side", who, i);
        if (int rc = check_side(bl.k, who)) return rc;
        if (int rc = check_side(bl.v, who)) return rc;
        const cqkv_kv_block &b0 = blocks[0];
        if (bl.k->format != b0.k->format || bl.v->format != b0.v->format ||
            side_bits(bl.k) != side_bits(b0.k) || side_bits(bl.v) != side_bits(b0.v) ||
            bl.k->head_dim != b0.k->head_dim || bl.v->head_dim != b0.k->head_dim ||
            bl.k->kv_heads != b0.k->kv_heads || bl.v->kv_heads != b0.k->kv_heads ||
            bl.k->is_value != 0 || bl.v->is_value != 1 || side_rotates(bl.k) != side_rotates(b0.k) ||
            side_rotates(bl.v) != side_rotates(b0.v) ||
            side_rotation(bl.k) != side_rotation(b0.k) || side_rotation(bl.v) != side_rotation(b0.v) ||
            (side_rotates(b0.k) && bl.k->seed != b0.k->seed) ||
            (side_rotates(b0.v) && bl.v->seed != b0.v->seed) ||
            (b0.k->format == CQKV_FMT_TURBOPROD && bl.k->qjl != b0.k->qjl))
            return fail(CQKV_ERR_ARG,
                        "%s: block %d differs from block 0 in format, head dim, kv heads, side, "
                        "rotation, seed or QJL matrix",
                        who, i);
        if (bl.rows < 0 || bl.rows > bl.k->capacity || bl.rows > bl.v->capacity)
            return fail(CQKV_ERR_ARG, "%s: block %d has %d rows but capacities %d / %d", who, i,
                        bl.rows, bl.k->capacity, bl.v->capacity);
        total += bl.rows;
    }
    if (total == 0) return fail(CQKV_ERR_ARG, "%s: the blocks hold no keys", who);
    if (total > (1 << 30)) return fail(CQKV_ERR_ARG, "%s: %lld keys", who, (long long)total);
    (void)batch;
    return CQKV_OK;
}

extern "C" size_t cqkv_decode_paged_workspace_bytes(const cqkv_kv_block *blocks,
                                                    int32_t n_blocks, int32_t batch,
                                                    int32_t q_heads, int32_t q_len) {
    clear_error();
    if (check_blocks(blocks, n_blocks, batch, "cqkv_decode_paged_workspace_bytes") != CQKV_OK ||
        batch <= 0 || q_heads <= 0 || q_len <= 0)
        return 0;
    const int nseg = paged_segments(blocks, n_blocks, batch, nullptr);
    size_t part_off;
    DecodeWs w;
    return paged_workspace(nseg, batch, q_heads, q_len, blocks[0].k->head_dim, &part_off, &w);
}

extern "C" int cqkv_decode_attention_paged(const void *q, int32_t q_dtype,
                                           const int64_t q_strides[3], const cqkv_kv_block *blocks,
                                           int32_t n_blocks, int32_t batch, int32_t q_heads,
                                           int32_t q_len, float softmax_scale, int32_t window_left,
                                           int32_t window_right, float softcap,
                                           const float *alibi_slopes, int32_t alibi_batch_stride,
                                           void *out, int32_t out_dtype,
                                           const int64_t out_strides[3], void *workspace,
                                           size_t workspace_bytes, cqkv_stream_t stream) {
    clear_error();
    const char *who = "cqkv_decode_attention_paged";
    if (int rc = check_blocks(blocks, n_blocks, batch, who)) return rc;
    DecodeArgs a;
    DecodeHost h;
    if (int rc = decode_prepare(a, h, who, q, q_dtype, q_strides, blocks[0].k, blocks[0].v, batch,
                                q_heads, q_len, softmax_scale, window_left, window_right, softcap,
                                alibi_slopes, alibi_batch_stride, out, out_dtype, out_strides))
        return rc;
    if (batch == 0 || q_len == 0) return CQKV_OK;
    std::vector<PagedSeg> segs;
    const int nseg = paged_segments(blocks, n_blocks, batch, &segs);
    int64_t total = 0;
    for (int i = 0; i < n_blocks; ++i) total += blocks[i].rows;
    const int d = blocks[0].k->head_dim;
    a.kv_len = (int32_t)total;
    a.splits = nseg;

    hipStream_t st = (hipStream_t)stream;
    size_t part_off;
    DecodeWs w;
    const size_t need = paged_workspace(nseg, batch, q_heads, q_len, d, &part_off, &w);
    void *ws = workspace;
    bool owned = false;
    if (ws && workspace_bytes < need)
        return fail(CQKV_ERR_WORKSPACE, "%s: workspace %zu < %zu bytes", who, workspace_bytes, need);
    if (!ws) {
        CQKV_HIP_CHECK(hipMallocAsync(&ws, need, st));
        owned = true;
    }
    hipError_t e = write_paged_table(segs, (PagedSeg *)ws, st);
    a.segs = (const PagedSeg *)ws;
    void *dws = (char *)ws + part_off;
    a.part_o = (float *)dws;
    a.part_lse = (float *)((char *)dws + w.lse);
    if (e == hipSuccess) e = decode_launch(a, h, a.kfmt, a.vfmt, dws, w, st);
    if (owned) {
        hipError_t fe = hipFreeAsync(ws, st);
        if (e == hipSuccess) e = fe;
    }
    if (e != hipSuccess) return fail(CQKV_ERR_HIP, "%s: %s", who, hipGetErrorString(e));
    return CQKV_OK;
}
