// dense.h -- launch interface of the contiguous-KV attention kernel.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace vcpp {

struct DenseParams {
    const float* q;      // [batch][heads][q_len][head_dim] (row 0 used)
    const float* k;      // [batch][heads][kv_len][head_dim]
    const float* v;
    float* out;          // [batch][heads][head_dim]
    float* attn_weights; // [batch * heads][kv_len]
    const float* mask;   // [kv_len] or nullptr
    int32_t batch, heads, head_dim, q_len, kv_len;
};

hipError_t launch_dense(const DenseParams& p, hipStream_t stream);

}  // namespace vcpp
