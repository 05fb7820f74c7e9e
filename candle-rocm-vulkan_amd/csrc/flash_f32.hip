// Launches of the f32-query flash attention (flash_f32.h): one instantiation per K / V element
// type, padded head dim (64, 128, 256) and mode (row: at most 16 columns per kv head; column:
// more), then the split combine of flash_plain.h in f32.
#include "flash_f32.h"

namespace cqkv {

template <int KV, int D>
static void fa32_launch_d(const FaArgs &a, bool tile, hipStream_t st) {
    const int64_t wgs = (int64_t)a.splits * a.col_blocks * a.kv_heads * a.batch;
    if (tile)
        hipLaunchKernelGGL((fa32_kernel<KV, D, true>), dim3((unsigned)wgs), dim3(256), 0, st, a);
    else
        hipLaunchKernelGGL((fa32_kernel<KV, D, false>), dim3((unsigned)wgs), dim3(256), 0, st, a);
    if (a.splits > 1) {
        const int64_t rows = (int64_t)a.batch * a.q_heads * a.q_len;
        hipLaunchKernelGGL(fa_combine_kernel<D>, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, st,
                           a);
    }
}

template <int KV>
static void fa32_launch_kv(const FaArgs &a, int dmax, bool tile, hipStream_t st) {
    if (dmax == 64) fa32_launch_d<KV, 64>(a, tile, st);
    else if (dmax == 128) fa32_launch_d<KV, 128>(a, tile, st);
    else fa32_launch_d<KV, 256>(a, tile, st);
}

// a.dtype is f32; a.kv_dtype one of CQKV_F32 / CQKV_F16 / CQKV_BF16 / kKvE4M3 (checked by the
// callers' fa_plain_check).
void fa32_launch(const FaArgs &a, int dmax, bool tile, hipStream_t st) {
    switch (a.kv_dtype) {
        case CQKV_F32: fa32_launch_kv<kFa32F32>(a, dmax, tile, st); break;
        case CQKV_F16: fa32_launch_kv<kFa32F16>(a, dmax, tile, st); break;
        case CQKV_BF16: fa32_launch_kv<kFa32BF16>(a, dmax, tile, st); break;
        default: fa32_launch_kv<kFa32E4M3>(a, dmax, tile, st); break;
    }
}

}  // namespace cqkv
