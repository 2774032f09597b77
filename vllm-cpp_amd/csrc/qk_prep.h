// qk_prep.h -- launch interface of the query/key preparation kernels (per-head
// RMS norm and rotary position embedding) that feed the attention kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "vcpp_attention.h"

namespace vcpp {

// One tensor [num_tokens][num_heads][head_dim] fp32, updated in place.
struct QkTensor {
    float* x;
    const float* norm_weight;  // [head_dim]; null: no norm
    int32_t num_heads;
};

struct QkPrepParams {
    QkTensor t[2];             // q, k (k.x null: one tensor)
    int32_t num_tokens;
    int32_t head_dim;
    float eps;
    const int32_t* positions;  // [num_tokens]; null: no rotation
    const float* inv_freq;     // [inv_freq_size]
    int32_t inv_freq_size;
    int32_t style;             // VCPP_ROPE_INTERLEAVED or VCPP_ROPE_HALF
};

hipError_t launch_qk_prep(const QkPrepParams& p, hipStream_t stream);

// apply_rope_cuda semantics: one cos/sin row [head_dim / 2] for every batch row,
// half-split pairs (d, d + head_dim / 2) inside each head of q and k.
struct RopeTableParams {
    float* q;
    float* k;
    const float* cos;
    const float* sin;
    int32_t total_dim;
    int32_t head_dim;
    int32_t batch_size;
};

hipError_t launch_rope_table(const RopeTableParams& p, hipStream_t stream);

}  // namespace vcpp
