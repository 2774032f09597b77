// dense.hip -- contiguous-KV attention behind the reference's
// flash_attention_cuda slot (cuda/attention.cu:58-124).
//
// The reference runs host loops over (batch, head), uses only query row 0 of
// each (b, h), writes the softmax probabilities to attn_weights and the
// weighted sum of V to out [B][H][D].  Here one workgroup per (b, h) does the
// same on the device: logits (and the mask, attn_mask[s] < 0 -> -1e9) into
// attn_weights, a workgroup max and sum, probabilities back into
// attn_weights, then out[d] = sum_s w[s] v[s][d] with one thread per d.
// fp32 throughout; this is not a hot path.
#include "dense.h"

namespace vcpp {

namespace {

constexpr int kThreads = 256;

__device__ float block_reduce(float x, bool is_max, float* red) {
    for (int m = 32; m > 0; m >>= 1) {
        const float y = __shfl_xor(x, m, 64);
        x = is_max ? fmaxf(x, y) : x + y;
    }
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (lane == 0) red[wave] = x;
    __syncthreads();
    float r = red[0];
    for (int w = 1; w < kThreads / 64; ++w) r = is_max ? fmaxf(r, red[w]) : r + red[w];
    __syncthreads();
    return r;
}

__global__ __launch_bounds__(kThreads) void dense_attention_kernel(DenseParams p) {
    extern __shared__ float qs[];  // query row 0, head_dim floats
    __shared__ float red[kThreads / 64];
    const int64_t bh = blockIdx.x;
    const int D = p.head_dim, S = p.kv_len;
    const float* q = p.q + bh * D * p.q_len;
    const float* k = p.k + bh * D * S;
    const float* v = p.v + bh * D * S;
    float* w = p.attn_weights + bh * S;
    for (int d = threadIdx.x; d < D; d += kThreads) qs[d] = q[d];
    __syncthreads();

    const float scale = 1.0f / sqrtf((float)D);
    float mx = -__builtin_inff();
    for (int s = threadIdx.x; s < S; s += kThreads) {
        float dot = 0.0f;
        for (int d = 0; d < D; ++d) dot += qs[d] * k[(int64_t)s * D + d];
        float l = dot * scale;
        if (p.mask && p.mask[s] < 0.0f) l = -1e9f;
        w[s] = l;
        mx = fmaxf(mx, l);
    }
    mx = block_reduce(mx, true, red);
    float sum = 0.0f;
    for (int s = threadIdx.x; s < S; s += kThreads) {
        const float e = expf(w[s] - mx);
        w[s] = e;
        sum += e;
    }
    sum = block_reduce(sum, false, red);
    const float inv = 1.0f / (sum + 1e-9f);
    for (int s = threadIdx.x; s < S; s += kThreads) w[s] *= inv;
    __syncthreads();  // this thread's later reads of w cover other threads' writes
    for (int d = threadIdx.x; d < D; d += kThreads) {
        float acc = 0.0f;
        for (int s = 0; s < S; ++s) acc += w[s] * v[(int64_t)s * D + d];
        p.out[bh * D + d] = acc;
    }
}

}  // namespace

hipError_t launch_dense(const DenseParams& p, hipStream_t stream) {
    hipLaunchKernelGGL(dense_attention_kernel, dim3(p.batch * p.heads), dim3(kThreads),
                       p.head_dim * sizeof(float), stream, p);
    return hipGetLastError();
}

}  // namespace vcpp
