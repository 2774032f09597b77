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
#include "device_common.h"

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

// The same work for head_dim 64, 80 or 128 with 16-byte aligned rows, staged
// through LDS.  A wave's rows are one contiguous run of nrows * D floats: it
// moves in and out with fully coalesced 16-byte lane accesses.  Between the
// two, lane (row lane / 4, quarter lane % 4) owns the D / 4 consecutive
// elements of that quarter of the row, so
//  - the row's sum of squares is a two-step quad reduction (DPP),
//  - interleaved pairs (2i, 2i + 1) lie inside a lane, and the half-split
//    partner e +- D / 2 is the same slot of quarter q ^ 2 (a DPP quad swap),
//  - cos/sin of the token's D / 2 pair angles are formed once per wave into a
//    table beside the tile.
// Arithmetic per element is the generic kernel's, statement by statement.
template <int D>
__global__ __launch_bounds__(kQkWaves * 64) void qk_prep_lds_kernel(QkPrepParams p) {
    constexpr int P = D / 2, EQ = D / 4;          // pairs; elements per lane
    constexpr int NQ = kRows * D / 4;             // 16-byte units of a full tile
    constexpr int NK = (NQ + 63) / 64;            // per lane
    static_assert(EQ % 4 == 0, "a lane's quarter is whole 16-byte units");
    __shared__ __attribute__((aligned(16))) float tile_all[kQkWaves][kRows * D];
    typedef float f2 __attribute__((ext_vector_type(2)));
    __shared__ f2 cs_all[kQkWaves][P];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t item = (int64_t)blockIdx.x * kQkWaves + __builtin_amdgcn_readfirstlane(wave);
    const int gq = (p.t[0].num_heads + kRows - 1) / kRows;
    const int gk = p.t[1].x ? (p.t[1].num_heads + kRows - 1) / kRows : 0;
    const int64_t tok = item / (gq + gk);
    if (tok >= p.num_tokens) return;
    const int grp = (int)(item - tok * (gq + gk));
    const int which = grp >= gq;
    const QkTensor T = p.t[which];
    const int h0 = (which ? grp - gq : grp) * kRows;
    const int nrows = min(kRows, T.num_heads - h0);
    const int nq = nrows * (D / 4);
    const bool half = p.style == VCPP_ROPE_HALF;
    const bool rot = p.positions != nullptr;
    const bool norm = T.norm_weight != nullptr;
    f4* base = reinterpret_cast<f4*>(T.x + (tok * T.num_heads + h0) * D);
    auto* tile = (__attribute__((address_space(3))) float*)(tile_all[wave]);
    auto* cs = (__attribute__((address_space(3))) f2*)(cs_all[wave]);

    f4 in[NK];
#pragma unroll
    for (int k = 0; k < NK; ++k) {
        const int idx = 64 * k + lane;
        // Non-temporal: each unit is read once and written once (5.92 -> 6.23
        // TB/s on config 3's tokens; the dense and KV-write kernels measured
        // slower with it).
        in[k] = __builtin_nontemporal_load(base + min(idx, nq - 1));  // past the rows: a valid unit, not stored
    }
    if (rot && lane < P) {
        float sn, c;
        sincosf(p.inv_freq[min(lane, p.inv_freq_size - 1)] * (float)p.positions[tok], &sn, &c);
        cs[lane] = f2{c, sn};
    }
#pragma unroll
    for (int k = 0; k < NK; ++k) {
        const int idx = 64 * k + lane;
        if (idx < NQ) reinterpret_cast<__attribute__((address_space(3))) f4*>(tile)[idx] = in[k];
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    const int r = lane >> 2, qq = lane & 3, e0 = qq * EQ;
    __attribute__((address_space(3))) float* row = tile + r * D + e0;
    float x[EQ];
#pragma unroll
    for (int m = 0; m < EQ / 4; ++m) {
        const f4 v = reinterpret_cast<__attribute__((address_space(3))) f4*>(row)[m];
#pragma unroll
        for (int i = 0; i < 4; ++i) x[4 * m + i] = v[i];
    }
    float inv = 1.f;
    if (norm) {
        float ss = 0.f;
#pragma unroll
        for (int i = 0; i < EQ; ++i) ss += x[i] * x[i];
        ss += dpp<0xB1>(ss);  // quad_perm [1,0,3,2]
        ss += dpp<0x4E>(ss);  // quad_perm [2,3,0,1]
        inv = __builtin_amdgcn_rcpf(__builtin_amdgcn_sqrtf(ss * (1.0f / (float)D) + p.eps));
    }
    float y[EQ];
    if (norm) {
#pragma unroll
        for (int m = 0; m < EQ / 4; ++m) {
            const f4 wv = *reinterpret_cast<const f4*>(T.norm_weight + e0 + 4 * m);
#pragma unroll
            for (int i = 0; i < 4; ++i) y[4 * m + i] = wv[i] * x[4 * m + i] * inv;
        }
    } else {
#pragma unroll
        for (int i = 0; i < EQ; ++i) y[i] = x[i];
    }
    if (rot) {
        if (half) {
            // partner of e (quarter qq) is e +- P: the same slot of quarter qq ^ 2
            const bool lo = qq < 2;
#pragma unroll
            for (int i = 0; i < EQ; ++i) {
                const float yp = dpp<0x4E>(y[i]);
                const f2 t = cs[lo ? e0 + i : e0 + i - P];
                y[i] = lo ? y[i] * t.x - yp * t.y : yp * t.y + y[i] * t.x;
            }
        } else {
#pragma unroll
            for (int i = 0; i < EQ; i += 2) {
                const f2 t = cs[(e0 + i) >> 1];
                const float a = y[i], b = y[i + 1];
                y[i] = a * t.x - b * t.y;      // x0 c - x1 s
                y[i + 1] = a * t.y + b * t.x;  // x0 s + x1 c
            }
        }
    }
#pragma unroll
    for (int m = 0; m < EQ / 4; ++m)
        reinterpret_cast<__attribute__((address_space(3))) f4*>(row)[m] =
            f4{y[4 * m], y[4 * m + 1], y[4 * m + 2], y[4 * m + 3]};
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int k = 0; k < NK; ++k) {
        const int idx = 64 * k + lane;
        if (idx < nq) __builtin_nontemporal_store(reinterpret_cast<__attribute__((address_space(3))) f4*>(tile)[idx], base + idx);
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
    const bool aligned = reinterpret_cast<uintptr_t>(p.t[0].x) % 16 == 0 &&
                         reinterpret_cast<uintptr_t>(p.t[1].x) % 16 == 0 &&
                         reinterpret_cast<uintptr_t>(p.t[0].norm_weight) % 16 == 0 &&
                         reinterpret_cast<uintptr_t>(p.t[1].norm_weight) % 16 == 0;
    if (aligned && p.head_dim == 80) hipLaunchKernelGGL(qk_prep_lds_kernel<80>, grid, block, 0, stream, p);
    else if (aligned && p.head_dim == 64) hipLaunchKernelGGL(qk_prep_lds_kernel<64>, grid, block, 0, stream, p);
    else if (aligned && p.head_dim == 128) hipLaunchKernelGGL(qk_prep_lds_kernel<128>, grid, block, 0, stream, p);
    else if (p.head_dim <= 64) hipLaunchKernelGGL(qk_prep_kernel<1>, grid, block, 0, stream, p);
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
