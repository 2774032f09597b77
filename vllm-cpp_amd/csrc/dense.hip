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

// The same for head_dim % 16 == 0 (<= 128) and 16-byte aligned tensors, laid
// out for bandwidth.  Logits: lane (key lane / 4, quarter lane % 4) of each
// wave dots the D / 4 elements of its quarter of a key row (16-byte loads) and
// the quad sums them with two DPP steps: 16 keys per wave step.  Output: the
// four waves take a quarter of the keys each, lanes own dims lane and
// lane + 64, and the quarters are summed through LDS.  Same arithmetic as the
// generic kernel up to the order of the sums.
template <int D>
__global__ __launch_bounds__(kThreads) void dense_attention_vec_kernel(DenseParams p) {
    typedef float f4 __attribute__((ext_vector_type(4)));
    constexpr int EQ = D / 4;       // floats per lane per key row
    constexpr int NW = kThreads / 64;
    __shared__ float red[kThreads / 64];
    __shared__ float part[NW][D];
    const int64_t bh = blockIdx.x;
    const int S = p.kv_len;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const float* q = p.q + bh * D * p.q_len;
    const float* k = p.k + bh * D * S;
    const float* v = p.v + bh * D * S;
    float* w = p.attn_weights + bh * S;
    const int qq = lane & 3, r = lane >> 2;
    f4 qv[EQ / 4];
#pragma unroll
    for (int m = 0; m < EQ / 4; ++m) qv[m] = *reinterpret_cast<const f4*>(q + qq * EQ + 4 * m);
    const float scale = 1.0f / sqrtf((float)D);
    float mx = -__builtin_inff();
    for (int s0 = wave * 16; s0 < S; s0 += NW * 16) {
        const int s = min(s0 + r, S - 1);
        const float* krow = k + (int64_t)s * D + qq * EQ;
        float dot = 0.0f;
#pragma unroll
        for (int m = 0; m < EQ / 4; ++m) {
            const f4 x = *reinterpret_cast<const f4*>(krow + 4 * m);
#pragma unroll
            for (int i = 0; i < 4; ++i) dot += qv[m][i] * x[i];
        }
        dot += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, dot), 0xB1, 0xF, 0xF, false));
        dot += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, dot), 0x4E, 0xF, 0xF, false));
        float l = dot * scale;
        if (p.mask && p.mask[s] < 0.0f) l = -1e9f;
        if (qq == 0 && s0 + r < S) {
            w[s] = l;
            mx = fmaxf(mx, l);
        }
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
    const int sa = (int)(((int64_t)S * wave) / NW), sb = (int)(((int64_t)S * (wave + 1)) / NW);
    // lane (row slot lane / EQ, quad lane % EQ) adds w[s] * v[s][4 quad ..] for
    // the keys s of its slot (R slots per instruction, 16-byte loads)
    constexpr int R = 64 / EQ;
    const int slot = lane / EQ, quad = lane - slot * EQ;
    const bool act = slot < R;
    f4 acc[2] = {};
    int s = sa + slot;
    for (; s + R < sb; s += 2 * R) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int su = s + u * R;
            const float ws = w[su];
            const f4 x = act ? *reinterpret_cast<const f4*>(v + (int64_t)su * D + 4 * quad) : f4{};
            acc[u] += ws * x;
        }
    }
    if (s < sb && act) acc[0] += w[s] * *reinterpret_cast<const f4*>(v + (int64_t)s * D + 4 * quad);
    const f4 a = acc[0] + acc[1];
    // sum the R slots of each quad, then the waves, through LDS
    __shared__ f4 slots_all[NW][64];
    slots_all[wave][lane] = act ? a : f4{};
    __syncthreads();
    if (lane < EQ) {
        f4 t = {};
        for (int r = 0; r < R; ++r) t += slots_all[wave][r * EQ + lane];
#pragma unroll
        for (int i = 0; i < 4; ++i) part[wave][4 * lane + i] = t[i];
    }
    __syncthreads();
    for (int d = threadIdx.x; d < D; d += kThreads) {
        float o = 0.0f;
#pragma unroll
        for (int i = 0; i < NW; ++i) o += part[i][d];
        p.out[bh * D + d] = o;
    }
}

}  // namespace

hipError_t launch_dense(const DenseParams& p, hipStream_t stream) {
    const dim3 grid(p.batch * p.heads), block(kThreads);
    auto al = [](const void* x) { return reinterpret_cast<uintptr_t>(x) % 16 == 0; };
    const bool vec = al(p.q) && al(p.k) && al(p.v) && p.kv_len > 0;
    if (vec && p.head_dim == 64) hipLaunchKernelGGL(dense_attention_vec_kernel<64>, grid, block, 0, stream, p);
    else if (vec && p.head_dim == 80) hipLaunchKernelGGL(dense_attention_vec_kernel<80>, grid, block, 0, stream, p);
    else if (vec && p.head_dim == 128) hipLaunchKernelGGL(dense_attention_vec_kernel<128>, grid, block, 0, stream, p);
    else hipLaunchKernelGGL(dense_attention_kernel, grid, block, p.head_dim * sizeof(float), stream, p);
    return hipGetLastError();
}

}  // namespace vcpp
