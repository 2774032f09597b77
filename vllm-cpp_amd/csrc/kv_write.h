// kv_write.h -- launch interface of the K/V page writer.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "vcpp_attention.h"

namespace vcpp {

struct KvWriteParams {
    int32_t dtype;
    int32_t block_size;
    int32_t num_kv_heads;
    int32_t head_dim;
    int64_t num_blocks;
    int64_t block_stride;        // elements
    int64_t scale_block_stride;  // fp16 elements
    void* k;
    void* v;
    uint16_t* k_scale;
    uint16_t* v_scale;
    const float* k_src;  // [num_tokens][num_kv_heads][head_dim]
    const float* v_src;
    const int64_t* slots;  // [num_tokens] block * block_size + pos, < 0 skips
    int32_t num_tokens;
    int32_t fp16_rne;  // 0: reference truncation, 1: round to nearest even
};

hipError_t launch_kv_write(const KvWriteParams& p, hipStream_t stream);

}  // namespace vcpp
