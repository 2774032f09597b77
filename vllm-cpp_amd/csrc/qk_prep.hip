// qk_prep.hip -- query/key preparation in front of attention: the per-head RMS
// norm of Qwen3-style models and the rotary position embedding (RoPE).
//
// qk_prep_kernel: one wave per (token, 16 head rows of q or k), lane L owning
// elements L, L + 64, ... of each row.  Each
// row is read once and written once: norm (optional) then rotation
// (optional), the order of Qwen3 (q_norm / k_norm before the rotary
// embedding).  Arithmetic
// follows the reference statement by statement with contraction off:
//   norm  inv = 1 / sqrt(sum(x^2) / head_dim + eps); y = (w * x) * inv
//         (src/paged_engine.cpp:14-20, applied per head);
//   rope  theta = inv_freq[min(i, size - 1)] * (float)pos, c = cos(theta),
//         s = sin(theta); (x0, x1) -> (x0 c - x1 s, x0 s + x1 c), with the pair
//         (2i, 2i + 1) (src/paged_engine.cpp:47-62) or (i, i + head_dim / 2)
//         (cuda/attention_kernels.cuh:249-287).
// The row reduction is a lane tree and 1 / sqrt uses the hardware square root
// and reciprocal, so the norm matches the reference to a few fp32 ulps, not
// bit for bit; the rotation partner is
// the partner's normalised value, as in the reference's sequence of calls.
//
// rope_table_kernel: apply_rope_cuda (cuda/attention.cu:130-145) -- one thread
// per (batch row, d) with d in the first half of its head, cos/sin indexed by
// the pair, the partner index clamped to d past total_dim as the reference does.
#include "qk_prep.h"

#pragma clang fp contract(off)

namespace vcpp {

namespace {

constexpr int kQkWaves = 4;
constexpr int kRows = 16;  // head rows per wave

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL,
                                                                 0xF, 0xF, false));
}

// Sum over the wave's 64 lanes, bitwise identical in every lane (each step
// adds two equal-shape partial sums, and fp32 addition commutes): quad swaps,
// half-row and row mirrors (DPP), then the two cross-row steps.
__device__ __forceinline__ float wave_allsum(float v) {
    v += dpp<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp<0x141>(v);  // row_half_mirror
    v += dpp<0x140>(v);  // row_mirror
    v += __shfl_xor(v, 16, 64);
    v += __shfl_xor(v, 32, 64);
    return v;
}

// One wave per (token, group of kRows head rows of q or of k); the group
// shares the token's cos/sin.  Lane L owns
// element e = L + 64 j of each row (NE = ceil(head_dim / 64) per lane), so a
// row moves in fully coalesced 256-byte instructions.  The rotation partner of
// e is e ^ 1 (interleaved: the neighbouring lane, by a DPP quad swap) or
// e +- head_dim / 2 (half-split: loaded again, from cache).
template <int NE>
__global__ __launch_bounds__(kQkWaves * 64) void qk_prep_kernel(QkPrepParams p) {
    const int lane = threadIdx.x & 63;
    // wave-uniform work item (scalar registers, scalar branches)
    const int64_t item = (int64_t)blockIdx.x * kQkWaves + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int gq = (p.t[0].num_heads + kRows - 1) / kRows;
    const int gk = p.t[1].x ? (p.t[1].num_heads + kRows - 1) / kRows : 0;
    const int64_t tok = item / (gq + gk);
    if (tok >= p.num_tokens) return;
    const int grp = (int)(item - tok * (gq + gk));
    const int which = grp >= gq;
    const QkTensor T = p.t[which];
    const int h0 = (which ? grp - gq : grp) * kRows;
    const int nrows = min(kRows, T.num_heads - h0);
    const int D = p.head_dim, P = D / 2;
    const bool half = p.style == VCPP_ROPE_HALF;
    const bool rot = p.positions != nullptr;
    const bool norm = T.norm_weight != nullptr;
    float* base = T.x + (tok * T.num_heads + h0) * D;

    // Element e = lane + 64 j of each row; lanes past the row read a valid
    // element (discarded) instead of branching.
    int ei[NE], pe[NE];
    bool first[NE], valid[NE];
#pragma unroll
    for (int j = 0; j < NE; ++j) {
        const int e = lane + 64 * j;
        valid[j] = e < D;
        const int ec = valid[j] ? e : lane % D;
        ei[j] = ec;
        first[j] = half ? ec < P : (ec & 1) == 0;
        pe[j] = half ? (ec < P ? ec + P : ec - P) : (ec ^ 1);
    }
    float x[kRows][NE], xp[kRows][NE];
    // rows past nrows re-read the last row (cache hits) instead of branching
#pragma unroll
    for (int u = 0; u < kRows; ++u) {
        const int ur = min(u, nrows - 1);
#pragma unroll
        for (int j = 0; j < NE; ++j) {
            x[u][j] = base[ur * D + ei[j]];
            xp[u][j] = (half && rot) ? base[ur * D + pe[j]] : 0.f;
        }
    }
    float cs[NE], sn[NE], w[NE], wp[NE];
    const float pos = rot ? (float)p.positions[tok] : 0.f;
#pragma unroll
    for (int j = 0; j < NE; ++j) {
        cs[j] = 1.f;
        sn[j] = 0.f;
        w[j] = wp[j] = 1.f;
        if (rot) {
            const int pi = half ? (ei[j] < P ? ei[j] : ei[j] - P) : (ei[j] >> 1);
            sincosf(p.inv_freq[min(pi, p.inv_freq_size - 1)] * pos, &sn[j], &cs[j]);
        }
        if (norm) {
            w[j] = T.norm_weight[ei[j]];
            wp[j] = T.norm_weight[pe[j]];
        }
    }
    const float inv_d = 1.0f / (float)D;
#pragma unroll
    for (int u = 0; u < kRows; ++u) {
        float inv = 1.f;
        if (norm) {
            float ss = 0.f;
#pragma unroll
            for (int j = 0; j < NE; ++j) ss += valid[j] ? x[u][j] * x[u][j] : 0.f;
            ss = wave_allsum(ss);
            // hardware sqrt and reciprocal (about 1 ulp each)
            inv = __builtin_amdgcn_rcpf(__builtin_amdgcn_sqrtf(ss * inv_d + p.eps));
        }
#pragma unroll
        for (int j = 0; j < NE; ++j) {
            float y = norm ? w[j] * x[u][j] * inv : x[u][j];
            if (rot) {
                float yp;
                if (half) yp = norm ? wp[j] * xp[u][j] * inv : xp[u][j];
                else yp = dpp<0xB1>(y);  // the neighbour's (normalised) value
                // (x0, x1) -> (x0 c - x1 s, x0 s + x1 c)
                y = first[j] ? y * cs[j] - yp * sn[j] : yp * sn[j] + y * cs[j];
            }
            if (u < nrows && valid[j]) base[u * D + ei[j]] = y;
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
    if (p.num_tokens == 0) return hipSuccess;
    const int64_t groups = (p.t[0].num_heads + kRows - 1) / kRows +
                           (p.t[1].x ? (p.t[1].num_heads + kRows - 1) / kRows : 0);
    const int64_t wg = ((int64_t)p.num_tokens * groups + kQkWaves - 1) / kQkWaves;
    const dim3 grid((unsigned)wg), block(kQkWaves * 64);
    if (p.head_dim <= 64) hipLaunchKernelGGL(qk_prep_kernel<1>, grid, block, 0, stream, p);
    else if (p.head_dim <= 128) hipLaunchKernelGGL(qk_prep_kernel<2>, grid, block, 0, stream, p);
    else hipLaunchKernelGGL(qk_prep_kernel<4>, grid, block, 0, stream, p);
    return hipGetLastError();
}

hipError_t launch_rope_table(const RopeTableParams& p, hipStream_t stream) {
    const int64_t n = (int64_t)p.batch_size * p.total_dim;
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(rope_table_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, p);
    return hipGetLastError();
}

}  // namespace vcpp
