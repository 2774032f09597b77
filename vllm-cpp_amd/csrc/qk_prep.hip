// qk_prep.hip -- query/key preparation in front of attention: the per-head RMS
// norm of Qwen3-style models and the rotary position embedding (RoPE).
//
// qk_prep_kernel: one wave per (token, head) row of q or k, lane i owning the
// rotation pair i (pairs per row <= 64 per pass, head_dim <= 256).  Each row is
// read once and written once: norm (optional) then rotation (optional), the
// order of Qwen3 (q_norm / k_norm before the rotary embedding).  Arithmetic
// follows the reference statement by statement with contraction off:
//   norm  inv = 1 / sqrt(sum(x^2) / head_dim + eps); y = (w * x) * inv
//         (src/paged_engine.cpp:14-20, applied per head);
//   rope  theta = inv_freq[min(i, size - 1)] * (float)pos, c = cos(theta),
//         s = sin(theta); (x0, x1) -> (x0 c - x1 s, x0 s + x1 c), with the pair
//         (2i, 2i + 1) (src/paged_engine.cpp:47-62) or (i, i + head_dim / 2)
//         (cuda/attention_kernels.cuh:249-287).
// The row reduction is a lane tree, so the norm matches the reference's
// sequential sum to fp32 rounding, not bit for bit.
//
// rope_table_kernel: apply_rope_cuda (cuda/attention.cu:130-145) -- one thread
// per (batch row, d) with d in the first half of its head, cos/sin indexed by
// the pair, the partner index clamped to d past total_dim as the reference does.
#include "qk_prep.h"

#pragma clang fp contract(off)

namespace vcpp {

namespace {

constexpr int kQkWaves = 4;

__global__ __launch_bounds__(kQkWaves * 64) void qk_prep_kernel(QkPrepParams p) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * kQkWaves + (threadIdx.x >> 6);
    const int64_t rows_q = (int64_t)p.num_tokens * p.t[0].num_heads;
    const int64_t rows_k = p.t[1].x ? (int64_t)p.num_tokens * p.t[1].num_heads : 0;
    if (row >= rows_q + rows_k) return;
    const int which = row >= rows_q;
    const QkTensor& T = p.t[which];
    const int64_t r = which ? row - rows_q : row;
    const int64_t tok = r / T.num_heads;
    float* x = T.x + r * p.head_dim;
    const int D = p.head_dim, P = D / 2;
    const bool half = p.style == VCPP_ROPE_HALF;
    constexpr int kMaxPairs = 2;  // head_dim <= 256
    float x0[kMaxPairs], x1[kMaxPairs];
#pragma unroll
    for (int j = 0; j < kMaxPairs; ++j) {
        const int i = lane + 64 * j;
        x0[j] = x1[j] = 0.f;
        if (i < P) {
            if (half) {
                x0[j] = x[i];
                x1[j] = x[i + P];
            } else {
                const float2 v = *reinterpret_cast<const float2*>(x + 2 * i);
                x0[j] = v.x;
                x1[j] = v.y;
            }
        }
    }
    if (T.norm_weight) {
        float ss = 0.f;
#pragma unroll
        for (int j = 0; j < kMaxPairs; ++j) ss += x0[j] * x0[j] + x1[j] * x1[j];
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) ss += __shfl_xor(ss, m, 64);
        const float inv = 1.0f / sqrtf(ss / (float)D + p.eps);
#pragma unroll
        for (int j = 0; j < kMaxPairs; ++j) {
            const int i = lane + 64 * j;
            if (i < P) {
                const int d0 = half ? i : 2 * i, d1 = half ? i + P : 2 * i + 1;
                x0[j] = T.norm_weight[d0] * x0[j] * inv;
                x1[j] = T.norm_weight[d1] * x1[j] * inv;
            }
        }
    }
    if (p.positions) {
        const float pos = (float)p.positions[tok];
#pragma unroll
        for (int j = 0; j < kMaxPairs; ++j) {
            const int i = lane + 64 * j;
            if (i < P) {
                const float theta = p.inv_freq[min(i, p.inv_freq_size - 1)] * pos;
                float s, c;
                sincosf(theta, &s, &c);
                const float a = x0[j], b = x1[j];
                x0[j] = a * c - b * s;
                x1[j] = a * s + b * c;
            }
        }
    }
#pragma unroll
    for (int j = 0; j < kMaxPairs; ++j) {
        const int i = lane + 64 * j;
        if (i < P) {
            if (half) {
                x[i] = x0[j];
                x[i + P] = x1[j];
            } else {
                *reinterpret_cast<float2*>(x + 2 * i) = make_float2(x0[j], x1[j]);
            }
        }
    }
}

__global__ __launch_bounds__(256) void rope_table_kernel(RopeTableParams p) {
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (int64_t)p.batch_size * p.total_dim) return;
    const int64_t b = idx / p.total_dim;
    const int d = (int)(idx - b * p.total_dim);
    const int hdim = d % p.head_dim;
    if (hdim >= p.head_dim / 2) return;
    const float c = p.cos[hdim], s = p.sin[hdim];
    const int i0 = d;
    int i1 = d + p.head_dim / 2;
    if (i1 >= p.total_dim) i1 = d;
    float* q = p.q + b * p.total_dim;
    float* k = p.k + b * p.total_dim;
    const float q0 = q[i0], q1 = q[i1], k0 = k[i0], k1 = k[i1];
    q[i0] = q0 * c - q1 * s;
    q[i1] = q0 * s + q1 * c;
    k[i0] = k0 * c - k1 * s;
    k[i1] = k0 * s + k1 * c;
}

}  // namespace

hipError_t launch_qk_prep(const QkPrepParams& p, hipStream_t stream) {
    const int64_t rows = (int64_t)p.num_tokens * p.t[0].num_heads +
                         (p.t[1].x ? (int64_t)p.num_tokens * p.t[1].num_heads : 0);
    if (rows == 0) return hipSuccess;
    const int64_t wg = (rows + kQkWaves - 1) / kQkWaves;
    hipLaunchKernelGGL(qk_prep_kernel, dim3((unsigned)wg), dim3(kQkWaves * 64), 0, stream, p);
    return hipGetLastError();
}

hipError_t launch_rope_table(const RopeTableParams& p, hipStream_t stream) {
    const int64_t n = (int64_t)p.batch_size * p.total_dim;
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(rope_table_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, p);
    return hipGetLastError();
}

}  // namespace vcpp
