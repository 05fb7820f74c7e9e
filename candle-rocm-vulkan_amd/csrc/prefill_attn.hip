// Causal bf16 flash-attention prefill on MFMA (gfx950), with an optional fused FP8
// quantize-and-append of K / V into the decode cache.
#include "cqkv_device.h"
#include "cqkv_host.h"

extern "C" int cqkv_flash_attn(const void *q, const int64_t q_strides[3], const void *k,
                               const int64_t k_strides[3], const void *v,
                               const int64_t v_strides[3], void *out,
                               const int64_t out_strides[3], int32_t batch, int32_t q_len,
                               int32_t kv_len, int32_t q_heads, int32_t kv_heads,
                               int32_t head_dim, float softmax_scale, int32_t window_left,
                               int32_t window_right, const cqkv_side *k_cache,
                               const cqkv_side *v_cache, int32_t position, cqkv_stream_t stream) {
    return cqkv::fail(CQKV_ERR_ARG, "cqkv_flash_attn: not built yet");
}
