// One key format's instantiations of the decode kernels (compiled once per key format with
// -DCQKV_DECODE_KF=<format id>, so the formats build in parallel; every value format each).
#include "decode_kernels.h"

#ifndef CQKV_DECODE_KF
#error "compile with -DCQKV_DECODE_KF=<format id>"
#endif

#define CQKV_CAT2(a, b) a##b
#define CQKV_CAT(a, b) CQKV_CAT2(a, b)

namespace cqkv {

bool CQKV_CAT(decode_launch_k, CQKV_DECODE_KF)(int vf, int d, dim3 grid, hipStream_t st,
                                               const DecodeArgs &a) {
    return launch_decode_k<CQKV_DECODE_KF>(vf, d, grid, st, a);
}

}  // namespace cqkv
