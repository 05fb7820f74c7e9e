// Host side of the plain-dtype flash attention (flash_plain.h): split planning, the workspace of
// the split partials, the launches, and the paged entry point cqkv_flash_attn_blocks.
#include <algorithm>
#include <vector>

#include "flash_plain.h"

namespace cqkv {

static int fa_dmax(int head_dim) { return head_dim <= 64 ? 64 : head_dim <= 128 ? 128 : 256; }

// Workgroups one CU holds: the row kernel keeps two stages of a K and a V tile per wavefront,
// the tile kernel three stages shared by its four wavefronts.
static int fa_wgs_per_cu(int dmax, bool tile = false) {
    const int w = dmax == 256 ? 2 : 4;
    const int lds = tile ? 3 * 2 * 32 * 2 * dmax : 2 * w * 2 * 32 * 2 * dmax;
    return std::max(1, (160 * 1024) / lds);
}

// Key splits: enough workgroups to fill the chip (256 CUs), at least two tiles per wavefront and
// split; with per-sequence lengths, pieces of at most 4096 keys.
static int fa_auto_splits(int planes_cols, int kv_len, int dmax, bool ragged, bool tile = false) {
    const int w = tile ? 1 : dmax == 256 ? 2 : 4;
    const int tiles = std::max(1, (kv_len + 31) / 32);
    const int target = 256 * fa_wgs_per_cu(dmax, tile);
    int s = (target + planes_cols - 1) / std::max(planes_cols, 1);
    if (ragged) s = std::max(s, (tiles + 127) / 128);
    s = std::min(s, std::max(1, tiles / (2 * w)));
    s = std::max(1, std::min(s, 256));
    const int tps = (tiles + s - 1) / s;
    return std::max(1, (tiles + tps - 1) / tps);
}

static size_t fa_align256(size_t x) { return (x + 255) & ~(size_t)255; }

// Partials (splits, rows, dmax) f32 then lse (splits, rows) f32.
static size_t fa_partials_bytes(int splits, int64_t rows, int dmax, size_t *lse_off) {
    *lse_off = fa_align256((size_t)splits * rows * dmax * 4);
    return *lse_off + fa_align256((size_t)splits * rows * 4);
}

// The f32-query kernels (flash_f32.hip).
void fa32_launch(const FaArgs &a, int dmax, bool tile, hipStream_t st);

template <bool F16, int D>
static void fa_launch_d(const FaArgs &a, bool tile, hipStream_t st) {
    constexpr int W = fa_waves<D>();
    const int64_t wgs = (int64_t)a.splits * a.col_blocks * a.kv_heads * a.batch;
    if (tile)
        hipLaunchKernelGGL((fa_tile_kernel<F16, D>), dim3((unsigned)wgs), dim3(256), 0, st, a);
    else
        hipLaunchKernelGGL((fa_row_kernel<F16, D, W>), dim3((unsigned)wgs), dim3(W * 64), 0, st, a);
    if (a.splits > 1) {
        const int64_t rows = (int64_t)a.batch * a.q_heads * a.q_len;
        hipLaunchKernelGGL(fa_combine_kernel<D>, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, st,
                           a);
    }
}

static void fa_launch(const FaArgs &a, int dmax, bool tile, hipStream_t st) {
    if (a.dtype == CQKV_F32) {
        fa32_launch(a, dmax, tile, st);
        return;
    }
    const bool f16 = a.dtype == CQKV_F16;
    if (dmax == 64) f16 ? fa_launch_d<true, 64>(a, tile, st) : fa_launch_d<false, 64>(a, tile, st);
    else if (dmax == 128) f16 ? fa_launch_d<true, 128>(a, tile, st) : fa_launch_d<false, 128>(a, tile, st);
    else f16 ? fa_launch_d<true, 256>(a, tile, st) : fa_launch_d<false, 256>(a, tile, st);
}

// The dense call's plan: the tile kernel (64 columns per workgroup) for more than 16 columns
// per kv head, else the row kernel; column groups, splits, tiles per split.
struct FaPlan {
    bool tile;
    int col_blocks, splits, tps;
};
static FaPlan fa_plan(int64_t batch, int64_t kv_heads, int64_t ncols, int kv_len, int dmax,
                      bool ragged) {
    FaPlan p;
    p.tile = ncols > 16;
    p.col_blocks = (int)std::min<int64_t>((ncols + (p.tile ? 63 : 15)) / (p.tile ? 64 : 16), 1 << 20);
    const int64_t planes_cols = batch * kv_heads * p.col_blocks;
    int s = fa_auto_splits((int)std::min<int64_t>(planes_cols, 1 << 30), kv_len, dmax, ragged,
                           p.tile);
    const int tiles = std::max(1, (kv_len + 31) / 32);
    p.tps = (tiles + s - 1) / s;
    p.splits = (tiles + p.tps - 1) / p.tps;
    return p;
}

// Whether a tensor's rows can be read as whole 16-byte chunks (`esz`-byte elements).
static bool fa_vec_ok(const void *p, const int64_t s[3], int esz = 2) {
    const int64_t e = 16 / esz;
    return (uintptr_t)p % 16 == 0 && s[0] % e == 0 && s[1] % e == 0 && s[2] % e == 0;
}

// Bytes per K / V element of a dtype pair.
int fa_kv_esz(int32_t kv_dtype) {
    return kv_dtype == CQKV_F32 ? 4 : kv_dtype == kKvE4M3 ? 1 : 2;
}

// Checks shared by the dense and the paged calls. The dtype pairs are the reference's
// (kv_dtype_supported, candle-core/src/accel/attention.rs:569-576): q / out and K / V of one
// dtype, or f32 queries over f16 / bf16 / E4M3 K / V.
int fa_plain_check(const char *who, int32_t dtype, int32_t kv_dtype, int32_t head_dim,
                   int64_t k_row_stride, int64_t v_row_stride, int64_t kv_len) {
    const bool same = (dtype == CQKV_BF16 || dtype == CQKV_F16 || dtype == CQKV_F32) &&
                      kv_dtype == dtype;
    const bool wide = dtype == CQKV_F32 &&
                      (kv_dtype == CQKV_F16 || kv_dtype == CQKV_BF16 || kv_dtype == kKvE4M3);
    if (!same && !wide)
        return fail(CQKV_ERR_ARG,
                    "%s: dtypes q %d, k / v %d (q / k / v of one of bf16, f16, f32, or f32 q with "
                    "f16 / bf16 k / v)", who, dtype, kv_dtype);
    if (head_dim <= 0 || head_dim > 256 || head_dim % 8 != 0)
        return fail(CQKV_ERR_ARG, "%s: head_dim %d (a multiple of 8 up to 256)", who, head_dim);
    // 32-bit byte offsets inside a 32-row tile (16-bit copies) or a 16-row tile (f32 kernel)
    const int64_t lim = dtype == CQKV_F32 ? (1 << 24) : (1 << 25);
    if (k_row_stride < head_dim || v_row_stride < head_dim || k_row_stride >= lim ||
        v_row_stride >= lim)
        return fail(CQKV_ERR_ARG, "%s: K / V row strides %lld / %lld (head_dim .. %lld)", who,
                    (long long)k_row_stride, (long long)v_row_stride, (long long)lim);
    if (kv_len > (1 << 30)) return fail(CQKV_ERR_ARG, "%s: %lld keys", who, (long long)kv_len);
    return CQKV_OK;
}

// The dense / variable-length call (flash_attn_impl's path for bf16 / f16 inputs the MFMA
// prefill does not take): `a` carries tensors, lengths, masks and terms.
int fa_plain_run(FaArgs a, const char *who, void *workspace, size_t workspace_bytes,
                 hipStream_t st) {
    // 16-bit kernels: 16-byte copies; f32 kernel: loads of 4 elements
    const bool f32 = a.dtype == CQKV_F32;
    const int esz = fa_kv_esz(a.kv_dtype);
    const int64_t ce = f32 ? 4 : 8;  // elements per aligned piece
    const uintptr_t cb = (uintptr_t)(ce * esz);
    if ((uintptr_t)a.k % cb != 0 || (uintptr_t)a.v % cb != 0 || a.k_st % ce != 0 ||
        a.v_st % ce != 0 || a.k_sh % ce != 0 || a.v_sh % ce != 0 ||
        (!a.cu_k && (a.k_sb % ce != 0 || a.v_sb % ce != 0)))
        return fail(CQKV_ERR_ARG,
                    "%s: K / V need %d-byte aligned rows (pointers and strides in whole %d-element "
                    "chunks)", who, (int)cb, (int)ce);
    const int dmax = fa_dmax(a.head_dim);
    const int64_t ncols = (int64_t)a.q_len * a.group;
    if ((ncols + 15) / 16 > (1 << 20))
        return fail(CQKV_ERR_ARG, "%s: %lld query columns per kv head", who, (long long)ncols);
    const FaPlan plan = fa_plan(a.batch, a.kv_heads, ncols, a.kv_len, dmax, a.cu_k != nullptr);
    a.col_blocks = plan.col_blocks;
    const int64_t planes_cols = (int64_t)a.batch * a.kv_heads * a.col_blocks;
    const int s = plan.splits;
    if (planes_cols * s > 0x7fffffff)
        return fail(CQKV_ERR_ARG, "%s: %lld workgroups", who, (long long)(planes_cols * s));
    a.splits = s;
    a.tiles_per_split = plan.tps;
    {
        const int64_t qs[3] = {a.cu_q ? 0 : a.q_sb, a.q_st, a.q_sh};
        const int64_t os[3] = {a.cu_q ? 0 : a.o_sb, a.o_st, a.o_sh};
        a.q_vec = fa_vec_ok(a.q, qs, f32 ? 4 : 2) ? 1 : 0;
        a.o_vec = f32 && fa_vec_ok(a.out, os, 4) ? 1 : 0;
    }
    void *ws = workspace;
    bool owned = false;
    if (s > 1) {
        size_t lse_off;
        const int64_t rows = (int64_t)a.batch * a.q_heads * a.q_len;
        const size_t need = fa_partials_bytes(s, rows, dmax, &lse_off);
        if (ws && workspace_bytes < need)
            return fail(CQKV_ERR_WORKSPACE, "%s: workspace %zu < %zu bytes", who, workspace_bytes,
                        need);
        if (!ws) {
            CQKV_HIP_CHECK(hipMallocAsync(&ws, need, st));
            owned = true;
        }
        a.part_o = (float *)ws;
        a.part_lse = (float *)((char *)ws + lse_off);
    }
    fa_launch(a, dmax, plan.tile, st);
    hipError_t e = hipGetLastError();
    if (owned) {
        const hipError_t fe = hipFreeAsync(ws, st);
        if (e == hipSuccess) e = fe;
    }
    if (e != hipSuccess) return fail(CQKV_ERR_HIP, "%s: launch failed: %s", who, hipGetErrorString(e));
    return CQKV_OK;
}

size_t fa_plain_workspace_bytes(int32_t batch, int32_t q_len, int32_t kv_len, int32_t q_heads,
                                int32_t kv_heads, int32_t head_dim, bool ragged) {
    const int dmax = fa_dmax(head_dim);
    const FaPlan p = fa_plan(batch, kv_heads, (int64_t)q_len * (q_heads / kv_heads), kv_len, dmax,
                             ragged);
    if (p.splits <= 1) return 0;
    size_t lse_off;
    return fa_partials_bytes(p.splits, (int64_t)batch * q_heads * q_len, dmax, &lse_off);
}

// ---- paged: blocks of plain K / V ----
struct FaPagedPlan {
    std::vector<FaSeg> segs;
    int64_t total = 0;
};

// One segment per split: each block's tiles in pieces, so the split count follows the total.
static void fa_paged_plan(const cqkv_plain_block *blocks, int n_blocks, int batch, int kv_heads,
                          int cols, int dmax, FaPagedPlan &p) {
    for (int i = 0; i < n_blocks; ++i) p.total += blocks[i].rows;
    const int w = dmax == 256 ? 2 : 4;
    const int64_t planes_cols = (int64_t)batch * kv_heads * cols;
    const int target = (int)((256 * fa_wgs_per_cu(dmax) + planes_cols - 1) / planes_cols);
    const int64_t tiles_total = std::max<int64_t>(1, (p.total + 31) / 32);
    // tiles per segment: the total spread over `target` splits, at least two per wavefront
    int64_t tps = std::max<int64_t>(2 * w, (tiles_total + target - 1) / std::max(target, 1));
    tps = std::max<int64_t>(tps, (tiles_total + 255) / 256);  // at most ~256 segments
    int64_t off = 0;
    for (int i = 0; i < n_blocks; ++i) {
        const cqkv_plain_block &bl = blocks[i];
        const int tiles = (bl.rows + 31) / 32;
        for (int t0 = 0; t0 < tiles; t0 += (int)tps) {
            FaSeg s = {};
            s.k = (const uint16_t *)bl.k;
            s.v = (const uint16_t *)bl.v;
            s.k_sb = bl.k_strides[0];
            s.k_sh = bl.k_strides[1];
            s.v_sb = bl.v_strides[0];
            s.v_sh = bl.v_strides[1];
            s.rows = bl.rows;
            s.key_offset = (int32_t)off;
            s.tile_begin = t0;
            s.tile_end = std::min<int>(tiles, t0 + (int)tps);
            p.segs.push_back(s);
        }
        off += bl.rows;
    }
}

struct FaSegTableArgs {
    FaSeg seg[32];
    FaSeg *dst;
    int32_t n;
};

// Writes up to 32 segments into the device table: the table travels as kernel arguments, so a
// captured call replays with its own copy.
__global__ void fa_seg_table_kernel(FaSegTableArgs a) {
    const int i = threadIdx.x;
    if (i < a.n) a.dst[i] = a.seg[i];
}

}  // namespace cqkv

using namespace cqkv;

extern "C" size_t cqkv_flash_attn_blocks_workspace_bytes(const cqkv_plain_block *blocks,
                                                         int32_t n_blocks, int32_t batch,
                                                         int32_t q_heads, int32_t q_len,
                                                         int32_t kv_heads, int32_t head_dim) {
    clear_error();
    if (!blocks || n_blocks <= 0 || batch <= 0 || q_heads <= 0 || q_len <= 0 || kv_heads <= 0 ||
        q_heads % kv_heads != 0 || head_dim <= 0 || head_dim > 256)
        return 0;
    const int dmax = fa_dmax(head_dim);
    const int cols = (int)(((int64_t)q_len * (q_heads / kv_heads) + 15) / 16);
    FaPagedPlan p;
    fa_paged_plan(blocks, n_blocks, batch, kv_heads, cols, dmax, p);
    const size_t table = fa_align256(p.segs.size() * sizeof(FaSeg));
    size_t lse_off = 0;
    const size_t parts = p.segs.size() > 1
                             ? fa_partials_bytes((int)p.segs.size(),
                                                 (int64_t)batch * q_heads * q_len, dmax, &lse_off)
                             : 0;
    return table + parts;
}

extern "C" int cqkv_flash_attn_blocks(const void *q, const int64_t q_strides[3],
                                      const cqkv_plain_block *blocks, int32_t n_blocks,
                                      int32_t dtype, int32_t kv_dtype, int32_t batch,
                                      int32_t q_heads,
                                      int32_t q_len, int32_t kv_heads, int32_t head_dim,
                                      float softmax_scale, int32_t window_left,
                                      int32_t window_right, float softcap,
                                      const float *alibi_slopes, int32_t alibi_batch_stride,
                                      void *out, const int64_t out_strides[3], void *workspace,
                                      size_t workspace_bytes, cqkv_stream_t stream) {
    clear_error();
    static const char *who = "cqkv_flash_attn_blocks";
    // no query rows (batch or q_len 0): an empty output once the blocks pass their checks, as
    // the reference's (rocm_backend/accel.rs:197); q / out may then be null
    const bool no_rows = batch == 0 || q_len == 0;
    if ((!no_rows && (!q || !out)) || !q_strides || !out_strides || !blocks)
        return fail(CQKV_ERR_ARG, "%s: null q / out / strides / blocks", who);
    if (n_blocks <= 0) return fail(CQKV_ERR_ARG, "%s: no blocks", who);
    if (batch < 0 || q_heads <= 0 || q_len < 0 || kv_heads <= 0 || q_heads % kv_heads != 0)
        return fail(CQKV_ERR_ARG, "%s: batch %d q_len %d heads %d / %d", who, batch, q_len,
                    q_heads, kv_heads);
    if (!(softcap >= 0.0f) || softcap == __builtin_inff())
        return fail(CQKV_ERR_ARG, "%s: softcap %g (finite, >= 0)", who, (double)softcap);
    if (alibi_slopes && alibi_batch_stride != 0 && alibi_batch_stride != q_heads)
        return fail(CQKV_ERR_ARG, "%s: alibi batch stride %d (0 or q_heads)", who,
                    alibi_batch_stride);
    const int64_t k_row = blocks[0].k_strides[2], v_row = blocks[0].v_strides[2];
    if (int rc = fa_plain_check(who, dtype, kv_dtype, head_dim, k_row, v_row, 0)) return rc;
    // 16-bit kernels: 16-byte copies; f32 kernel: loads of 4 elements
    const int64_t ce = dtype == CQKV_F32 ? 4 : 8;
    const uintptr_t cb = (uintptr_t)(ce * fa_kv_esz(kv_dtype));
    int64_t total = 0;
    for (int i = 0; i < n_blocks; ++i) {
        const cqkv_plain_block &bl = blocks[i];
        if (!bl.k || !bl.v) return fail(CQKV_ERR_ARG, "%s: block %d has a null K / V", who, i);
        if (bl.rows < 0) return fail(CQKV_ERR_ARG, "%s: block %d rows %d", who, i, bl.rows);
        if (bl.k_strides[2] != k_row || bl.v_strides[2] != v_row)
            return fail(CQKV_ERR_ARG, "%s: block %d row strides differ from block 0's", who, i);
        if ((uintptr_t)bl.k % cb || (uintptr_t)bl.v % cb || bl.k_strides[0] % ce ||
            bl.k_strides[1] % ce || bl.v_strides[0] % ce || bl.v_strides[1] % ce)
            return fail(CQKV_ERR_ARG, "%s: block %d K / V need %d-byte aligned rows", who, i,
                        (int)cb);
        total += bl.rows;
    }
    if (total == 0) return fail(CQKV_ERR_ARG, "%s: the blocks hold no keys", who);
    if (k_row % ce || v_row % ce)
        return fail(CQKV_ERR_ARG, "%s: K / V row strides must be whole %d-element chunks", who,
                    (int)ce);
    if (int rc = fa_plain_check(who, dtype, kv_dtype, head_dim, k_row, v_row, total)) return rc;
    if (no_rows) return CQKV_OK;
    const int dmax = fa_dmax(head_dim);
    const int cols = (int)(((int64_t)q_len * (q_heads / kv_heads) + 15) / 16);
    FaPagedPlan p;
    fa_paged_plan(blocks, n_blocks, batch, kv_heads, cols, dmax, p);
    const int nseg = (int)p.segs.size();
    if ((int64_t)nseg * cols * batch * kv_heads > 0x7fffffff)
        return fail(CQKV_ERR_ARG, "%s: too many workgroups", who);

    FaArgs a = {};
    a.q = (const uint16_t *)q;
    a.q_sb = q_strides[0];
    a.q_sh = q_strides[1];
    a.q_st = q_strides[2];
    a.out = out;
    a.o_sb = out_strides[0];
    a.o_sh = out_strides[1];
    a.o_st = out_strides[2];
    a.k_st = k_row;
    a.v_st = v_row;
    a.batch = batch;
    a.q_len = q_len;
    a.kv_len = (int32_t)total;
    a.q_heads = q_heads;
    a.kv_heads = kv_heads;
    a.group = q_heads / kv_heads;
    a.head_dim = head_dim;
    a.dtype = dtype;
    a.kv_dtype = kv_dtype;
    a.splits = nseg;
    a.tiles_per_split = 0;
    a.col_blocks = cols;
    a.wl = window_left;
    a.wr = window_right;
    a.scale_log2 = softmax_scale * kLog2e;
    a.softcap2 = softcap * kLog2e;
    a.alibi = alibi_slopes;
    a.alibi_bs = alibi_batch_stride;
    a.o_mul = 1.0f;
    a.q_vec = fa_vec_ok(q, q_strides, dtype == CQKV_F32 ? 4 : 2) ? 1 : 0;
    a.o_vec = dtype == CQKV_F32 && fa_vec_ok(out, out_strides, 4) ? 1 : 0;

    const hipStream_t st = (hipStream_t)stream;
    const size_t table = fa_align256((size_t)nseg * sizeof(FaSeg));
    size_t lse_off = 0;
    const size_t parts =
        nseg > 1 ? fa_partials_bytes(nseg, (int64_t)batch * q_heads * q_len, dmax, &lse_off) : 0;
    const size_t need = table + parts;
    void *ws = workspace;
    bool owned = false;
    if (ws && workspace_bytes < need)
        return fail(CQKV_ERR_WORKSPACE, "%s: workspace %zu < %zu bytes", who, workspace_bytes, need);
    if (!ws) {
        CQKV_HIP_CHECK(hipMallocAsync(&ws, need, st));
        owned = true;
    }
    hipError_t e = hipSuccess;
    for (int i0 = 0; i0 < nseg && e == hipSuccess; i0 += 32) {
        FaSegTableArgs t = {};
        t.n = std::min(32, nseg - i0);
        for (int i = 0; i < t.n; ++i) t.seg[i] = p.segs[i0 + i];
        t.dst = (FaSeg *)ws + i0;
        hipLaunchKernelGGL(fa_seg_table_kernel, dim3(1), dim3(64), 0, st, t);
        e = hipGetLastError();
    }
    a.segs = (const FaSeg *)ws;
    if (nseg > 1) {
        a.part_o = (float *)((char *)ws + table);
        a.part_lse = (float *)((char *)ws + table + lse_off);
    }
    if (e == hipSuccess) {
        fa_launch(a, dmax, false, st);
        e = hipGetLastError();
    }
    if (owned) {
        const hipError_t fe = hipFreeAsync(ws, st);
        if (e == hipSuccess) e = fe;
    }
    if (e != hipSuccess) return fail(CQKV_ERR_HIP, "%s: %s", who, hipGetErrorString(e));
    return CQKV_OK;
}
