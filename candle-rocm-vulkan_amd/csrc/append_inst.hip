// One cache format's instantiations of the append kernels (compiled once per format with
// -DCQKV_APPEND_FMT=<format id>, so the formats build in parallel).
#include "append_rows.h"

#ifndef CQKV_APPEND_FMT
#error "compile with -DCQKV_APPEND_FMT=<format id>"
#endif

#define CQKV_CAT2(a, b) a##b
#define CQKV_CAT(a, b) CQKV_CAT2(a, b)

namespace cqkv {

void CQKV_CAT(append_rows_launch_, CQKV_APPEND_FMT)(const cqkv_side *s, int32_t tokens,
                                                   int32_t batch, hipStream_t st,
                                                   const AppendArgs &a) {
    launch_rows<CQKV_APPEND_FMT>(s, tokens, batch, st, a);
}

void CQKV_CAT(rope_append_launch_, CQKV_APPEND_FMT)(int rope, int d, dim3 grid, hipStream_t st,
                                                   const RopeAppendArgs &r) {
    launch_rope_append_fmt<CQKV_APPEND_FMT>(rope, d, grid, st, r);
}

}  // namespace cqkv
