// Rows times a D x D f32 matrix, and the zero-padded f32 staging of rows (rowmat.hip): the
// argument block and the launcher shared by the append, decode and dequantize entry points.
#pragma once

#include "cqkv_device.h"
#include "cqkv_host.h"

namespace cqkv {

// Row r of x and y is (i0, i1, i2) with r = (i0 * n1 + i1) * n2 + i2 and element offsets
// i0 * s0 + i1 * s1 + i2 * s2 (the row's elements contiguous).
//   m == NULL:   y_c = x_c for c < d, 0 for d <= c < ycols (copy, padding);
//   transpose:   y_c = base_c + sum_k x_k m[c][k]  (x m^T: the rotation x Pi^T);
//   otherwise:   y_c = base_c + sum_k x_k m[k][c]  (x m: the unrotation y Pi, x S).
// Sums run over k = 0 .. d - 1 in index order, products rounded before each add. base (optional,
// f32, row r at r * base_stride) is the start value of each sum; columns d .. ycols - 1 are 0,
// and so are rows xrows .. rows - 1 of x (read as zeros).
struct RowMatArgs {
    const void *x;
    int32_t x_dtype, n1, n2, d;
    int64_t xs0, xs1, xs2, rows, xrows;
    const float *m;
    int32_t transpose, ycols;
    const float *base;
    int64_t base_stride;
    void *y;
    int32_t y_dtype, pad_;
    int64_t ys0, ys1, ys2;
};

__device__ inline int64_t rowmat_offset(const RowMatArgs &a, int64_t row) {
    const int64_t i2 = row % a.n2, r1 = row / a.n2, i1 = r1 % a.n1, i0 = r1 / a.n1;
    return i0 * a.xs0 + i1 * a.xs1 + i2 * a.xs2;
}
__device__ inline int64_t rowmat_out_offset(const RowMatArgs &a, int64_t row) {
    const int64_t i2 = row % a.n2, r1 = row / a.n2, i1 = r1 % a.n1, i0 = r1 / a.n1;
    return i0 * a.ys0 + i1 * a.ys1 + i2 * a.ys2;
}

hipError_t rowmat_launch(const RowMatArgs &a, hipStream_t st);

// Rows (n0, n1, n2) of d elements at x (strides xs) to rows of ycols at y (strides ys), no
// matrix (a copy with zero padding) until the caller sets m / transpose / base.
inline RowMatArgs rowmat_args(const void *x, int32_t x_dtype, const int64_t xs[3], int64_t n0,
                              int32_t n1, int32_t n2, int32_t d, void *y, int32_t y_dtype,
                              const int64_t ys[3], int32_t ycols) {
    RowMatArgs r = {};
    r.x = x;
    r.x_dtype = x_dtype;
    r.n1 = n1;
    r.n2 = n2;
    r.d = d;
    r.xs0 = xs[0];
    r.xs1 = xs[1];
    r.xs2 = xs[2];
    r.rows = n0 * n1 * n2;
    r.xrows = r.rows;
    r.y = y;
    r.y_dtype = y_dtype;
    r.ys0 = ys[0];
    r.ys1 = ys[1];
    r.ys2 = ys[2];
    r.ycols = ycols;
    return r;
}

// A TURBOPROD side's QJL matrix as the kernels read it: D' x D' (the plane row length) with zero
// rows and columns past the head dim. Returns side->qjl itself when D' is the head dim; else a
// padded copy, stream-ordered in *tmp (the caller frees it with hipFreeAsync after its launches).
int qjl_for_kernels(const cqkv_side *side, hipStream_t st, const float **out, float **tmp);

}  // namespace cqkv
