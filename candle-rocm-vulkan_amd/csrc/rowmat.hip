// Rows times a D x D f32 matrix, and the f32 staging of cache rows: the rotations that are not the
// in-register Walsh-Hadamard transform (the Dense rotation, Hadamard at head dims other than the
// plane row lengths), the QJL correction of a TurboProd dequantization, and the zero padding of
// rows shorter than their plane row.
//
// Reference behaviour (paths relative to the reference repository root): TurboQuantizer::rotate
// x Pi^T and unrotate y Pi (candle-nn/src/turbo_quant.rs:182-196), the prod correction of
// RowCodec::dequantize_row (candle-core/src/accel/turbo.rs:401-424). The reference multiplies with
// a matmul of unpinned summation order; here every output sums its terms in index order, each
// product rounded before its add (no fused multiply-add), which is the order of the CPU
// restatement used as the checker.
#include "rowmat.h"

namespace cqkv {

constexpr int kRmTile = 64;  // rows x columns of a workgroup's output tile
constexpr int kRmK = 32;     // terms staged per step

// One 64 x 64 output tile per workgroup of 256 threads, 4 x 4 outputs per thread. The terms go
// through LDS in steps of 32, and each thread adds them to its outputs in index order.
__global__ __launch_bounds__(256) void rowmat_kernel(RowMatArgs a) {
#pragma clang fp contract(off)
    __shared__ float sm_a[kRmK][kRmTile + 1], sm_b[kRmK][kRmTile + 1];
    const int tid = threadIdx.x, tr = tid / 16, tc = tid % 16;
    const int64_t r0 = (int64_t)blockIdx.x * kRmTile;
    const int c0 = blockIdx.y * kRmTile;
    float acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int64_t row = r0 + 4 * tr + i;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int col = c0 + 4 * tc + j;
            acc[i][j] = a.base && row < a.rows && col < a.d ? a.base[row * a.base_stride + col] : 0.0f;
        }
    }
    for (int k0 = 0; k0 < a.d; k0 += kRmK) {
        for (int idx = tid; idx < kRmK * kRmTile; idx += 256) {
            const int kk = idx % kRmK, rr = idx / kRmK;  // consecutive threads: consecutive terms
            const int64_t row = r0 + rr;
            const int k = k0 + kk;
            float v = 0.0f;
            if (row < a.xrows && k < a.d) v = load_elem(a.x, rowmat_offset(a, row) + k, a.x_dtype);
            sm_a[kk][rr] = v;
        }
        for (int idx = tid; idx < kRmK * kRmTile; idx += 256) {
            int kk, cc;
            if (a.transpose) {  // B[k][c] = M[c][k]: consecutive threads read along a row of M
                kk = idx % kRmK;
                cc = idx / kRmK;
            } else {            // B[k][c] = M[k][c]
                cc = idx % kRmTile;
                kk = idx / kRmTile;
            }
            const int k = k0 + kk, col = c0 + cc;
            float v = 0.0f;
            if (k < a.d && col < a.d)
                v = a.transpose ? a.m[(int64_t)col * a.d + k] : a.m[(int64_t)k * a.d + col];
            sm_b[kk][cc] = v;
        }
        __syncthreads();
        const int kn = min(kRmK, a.d - k0);
        for (int kk = 0; kk < kn; ++kk) {
            float av[4], bv[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) av[i] = sm_a[kk][4 * tr + i];
#pragma unroll
            for (int j = 0; j < 4; ++j) bv[j] = sm_b[kk][4 * tc + j];
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float p = av[i] * bv[j];
                    acc[i][j] = acc[i][j] + p;
                }
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int64_t row = r0 + 4 * tr + i;
        if (row >= a.rows) continue;
        const int64_t yo = rowmat_out_offset(a, row);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int col = c0 + 4 * tc + j;
            if (col < a.ycols) store_elem(a.y, yo + col, a.y_dtype, col < a.d ? acc[i][j] : 0.0f);
        }
    }
}

// y = x with the columns from d to ycols zero (no matrix): one thread per output element.
__global__ __launch_bounds__(256) void rowcopy_kernel(RowMatArgs a) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= a.rows * a.ycols) return;
    const int64_t row = i / a.ycols;
    const int col = (int)(i % a.ycols);
    const float v = col < a.d && row < a.xrows ? load_elem(a.x, rowmat_offset(a, row) + col, a.x_dtype)
                                               : 0.0f;
    store_elem(a.y, rowmat_out_offset(a, row) + col, a.y_dtype, v);
}

hipError_t rowmat_launch(const RowMatArgs &a, hipStream_t st) {
    if (a.rows <= 0 || a.ycols <= 0) return hipSuccess;
    if (!a.m) {
        const int64_t n = a.rows * a.ycols;
        hipLaunchKernelGGL(rowcopy_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, a);
    } else {
        const dim3 grid((unsigned)((a.rows + kRmTile - 1) / kRmTile),
                        (unsigned)((a.ycols + kRmTile - 1) / kRmTile));
        hipLaunchKernelGGL(rowmat_kernel, grid, dim3(256), 0, st, a);
    }
    return hipGetLastError();
}

int qjl_for_kernels(const cqkv_side *side, hipStream_t st, const float **out, float **tmp) {
    *tmp = nullptr;
    *out = side->qjl;
    const int d = side->head_dim, dk = kernel_dim(d);
    if (side->format != CQKV_FMT_TURBOPROD || d == dk) return CQKV_OK;
    CQKV_HIP_CHECK(hipMallocAsync((void **)tmp, (size_t)dk * dk * 4, st));
    const int64_t xs[3] = {0, 0, d}, ys[3] = {0, 0, dk};
    RowMatArgs r = rowmat_args(side->qjl, CQKV_F32, xs, 1, 1, dk, d, *tmp, CQKV_F32, ys, dk);
    r.xrows = d;
    CQKV_HIP_CHECK(rowmat_launch(r, st));
    *out = *tmp;
    return CQKV_OK;
}

}  // namespace cqkv
