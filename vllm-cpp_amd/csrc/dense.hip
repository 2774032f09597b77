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

#include <cstdlib>

#ifndef VCPP_DENSE_NW
#define VCPP_DENSE_NW 4
#endif

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

// The same (head_dim 64, 80, 96 or 128, 16-byte aligned q/k/v) as one pass
// over K and V through LDS.  Each wave owns the 16-key chunks wave,
// wave + NW, ... of the pair; a chunk's K rows and V rows are each one
// contiguous run, moved into the wave's own LDS ring with
// global_load_lds_dwordx4 (1 KiB of whole cache lines per instruction,
// non-temporal: every byte is read once), with the chunk's 16 mask values
// when there is a mask, and waited for on the wave's own vmcnt, so no loop
// iteration has a compiler-visible global load.  Lane (key lane / 4, quarter
// lane % 4) dots its quarter of the key row, the quad sums it, and the lane
// keeps an online softmax over its keys (running max, sum of exp, and the
// exp-weighted sum of its quarter of the V rows).  The logits stay in LDS, in
// segments of 4096 keys; a full segment is flushed to attn_weights before
// the next one reuses the space.  At the end the lanes and waves combine by
// log-sum-exp and the probabilities exp(l - max) / (sum + 1e-9) are written.
template <int D, int NW, bool MASK>
struct DenseDma {
    static constexpr int ROWB = D * 4;               // bytes of one key row
    static constexpr int CH = 16 * ROWB;             // one chunk of K (or of V)
    static constexpr int NI = CH / 1024;             // DMA instructions per chunk of K
    static constexpr int NM = MASK ? 1 : 0;          // mask instruction per chunk
    static constexpr int NPER = 2 * NI + NM;         // DMA instructions per chunk
    static constexpr int MAXS = 4096;                // logits held in LDS (one segment)
    static constexpr int SEGI = MAXS / 16 / NW;      // local chunks per segment
    static constexpr int RED = NW * (D + 2) * 4;     // per-wave partials
    static constexpr int STAGE = 2 * CH + (MASK ? 256 : 0);  // K, V, the mask dwords
    static constexpr int STAGES = NW * 3 * STAGE + MAXS * 4 + RED <= 160 * 1024 ? 3 : 2;
    static constexpr int WAVE = STAGES * STAGE;
    static constexpr int OFF_LOGIT = NW * WAVE;
    static constexpr int OFF_RED = OFF_LOGIT + MAXS * 4;
    static constexpr int LDS = OFF_RED + RED;
    static_assert(CH % 1024 == 0 && D % 16 == 0, "chunk shape");
    static_assert(LDS <= 160 * 1024, "LDS budget");
    static_assert((STAGES - 1) * NPER < 64, "vmcnt range");
};

__device__ __attribute__((aligned(16))) const uint32_t kDenseZero16[4] = {0, 0, 0, 0};

__device__ __forceinline__ void dense_dma16(const void* src, uint32_t lds_base) {
    uint32_t saved;
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %2, off nt\n\ts_mov_b32 m0, %0"
                 : "=&s"(saved) : "s"(lds_base), "v"(src) : "memory");
}

// 4 bytes per lane (lane l lands at lds_base + 4 l).
__device__ __forceinline__ void dense_dma4(const void* src, uint32_t lds_base) {
    uint32_t saved;
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\tglobal_load_lds_dword %2, off nt\n\ts_mov_b32 m0, %0"
                 : "=&s"(saved) : "s"(lds_base), "v"(src) : "memory");
}

template <int N>
__device__ __forceinline__ void dense_wait_vm() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

template <int D, int NW, bool MASK>
__global__ __launch_bounds__(NW * 64) void dense_attention_dma_kernel(DenseParams p) {
    using C = DenseDma<D, NW, MASK>;
    typedef float f4 __attribute__((ext_vector_type(4)));
    constexpr int EQ = D / 4, NQ = EQ / 4;
    extern __shared__ __attribute__((aligned(16))) char smem[];
    const int64_t bh = blockIdx.x;
    const int S = p.kv_len;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int qq = lane & 3, r = lane >> 2;
    const char* kb = reinterpret_cast<const char*>(p.k + bh * D * S);
    const char* vb = reinterpret_cast<const char*>(p.v + bh * D * S);
    const int64_t bytes = (int64_t)S * C::ROWB;
    const uint32_t wbase = (uint32_t)(uintptr_t)smem + wave * C::WAVE;
    const int nch = (S + 15) >> 4;
    // Every wave runs the same number of iterations (chunks past the last
    // one are zero loads and no keys), so that all of them reach each
    // segment flush.
    const int nit = (nch + NW - 1) / NW;
    float* logit = reinterpret_cast<float*>(smem + C::OFF_LOGIT);
    float* wout = p.attn_weights + bh * S;

    const float* q = p.q + bh * D * p.q_len;
    f4 qv[NQ];
#pragma unroll
    for (int m = 0; m < NQ; ++m) qv[m] = *reinterpret_cast<const f4*>(q + qq * EQ + 4 * m);
    // q must be in registers before the first DMA: a wait for it left to its
    // first use would be a vmcnt wait inside the loop, counted without the
    // DMAs, and would drain the ring.
#pragma unroll
    for (int m = 0; m < NQ; ++m) asm volatile("" : "+v"(qv[m]));

    // Local chunk i into ring stage i % STAGES; lanes past the pair's last
    // key read a zero chunk, so every issue is NPER instructions and the
    // waits below have fixed counts.
    auto issue = [&](int i) {
        const int c = wave + NW * i;
        const int64_t off0 = (int64_t)c * C::CH + lane * 16;
        const uint32_t sb = __builtin_amdgcn_readfirstlane(wbase + (i % C::STAGES) * C::STAGE);
#pragma unroll
        for (int j = 0; j < C::NI; ++j) {
            const int64_t off = off0 + j * 1024;
            dense_dma16(off < bytes ? (const void*)(kb + off) : (const void*)kDenseZero16, sb + j * 1024);
        }
#pragma unroll
        for (int j = 0; j < C::NI; ++j) {
            const int64_t off = off0 + j * 1024;
            dense_dma16(off < bytes ? (const void*)(vb + off) : (const void*)kDenseZero16, sb + C::CH + j * 1024);
        }
        if constexpr (MASK) {  // lanes 0-15: the chunk's mask values
            const int s = 16 * c + lane;
            dense_dma4(lane < 16 && s < S ? (const void*)(p.mask + s) : (const void*)kDenseZero16, sb + 2 * C::CH);
        }
    };
#pragma unroll
    for (int i = 0; i < C::STAGES - 1; ++i) issue(i);

    const float scale = 1.0f / sqrtf((float)D);
    float mx = -__builtin_inff(), sum = 0.0f;
    f4 acc[NQ];
#pragma unroll
    for (int m = 0; m < NQ; ++m) acc[m] = f4{0.f, 0.f, 0.f, 0.f};
    for (int i = 0; i < nit; ++i) {
        if (S > C::MAXS && i > 0 && i % C::SEGI == 0) {
            // Keys [i / SEGI - 1 segments, ...) are done: flush the segment's
            // logits.  The ring is drained first (the stores then wait on
            // nothing of it), and the chunks already issued stay in LDS.
            dense_wait_vm<0>();
            __syncthreads();
            const int seg0 = (i / C::SEGI - 1) * C::MAXS;
            for (int e = threadIdx.x; e < C::MAXS; e += NW * 64) wout[seg0 + e] = logit[e];
            __syncthreads();
        }
        // the stage about to be refilled was read in the previous iteration
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        issue(i + C::STAGES - 1);
        dense_wait_vm<(C::STAGES - 1) * C::NPER>();
        const char* sbase = smem + wave * C::WAVE + (i % C::STAGES) * C::STAGE;
        const char* st = sbase + r * C::ROWB + qq * EQ * 4;
        float dot = 0.0f;
#pragma unroll
        for (int m = 0; m < NQ; ++m) {
            const f4 x = *reinterpret_cast<const f4*>(st + 16 * m);
#pragma unroll
            for (int e = 0; e < 4; ++e) dot += qv[m][e] * x[e];
        }
        dot += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, dot), 0xB1, 0xF, 0xF, false));
        dot += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, dot), 0x4E, 0xF, 0xF, false));
        const int s = (wave + NW * i) * 16 + r;
        float l = dot * scale;
        if constexpr (MASK) {
            if (*reinterpret_cast<const float*>(sbase + 2 * C::CH + r * 4) < 0.0f) l = -1e9f;
        }
        if (s < S) {
            if (qq == 0) logit[s & (C::MAXS - 1)] = l;
            if (l > mx) {
                const float f = expf(mx - l);
                sum *= f;
#pragma unroll
                for (int m = 0; m < NQ; ++m) acc[m] *= f;
                mx = l;
            }
            const float e = expf(l - mx);
            sum += e;
#pragma unroll
            for (int m = 0; m < NQ; ++m) acc[m] += e * *reinterpret_cast<const f4*>(st + C::CH + 16 * m);
        }
    }
    dense_wait_vm<0>();  // the ring's padding loads and the segment flushes

    // Lanes -> wave: max over the wave, rescale, sum over the 16 key lanes of
    // each quarter.
    float wm = mx;
    for (int o = 1; o < 64; o <<= 1) wm = fmaxf(wm, __shfl_xor(wm, o, 64));
    const float f = mx == -__builtin_inff() ? 0.0f : expf(mx - wm);
    sum *= f;
#pragma unroll
    for (int m = 0; m < NQ; ++m) acc[m] *= f;
    for (int o = 4; o < 64; o <<= 1) {
        sum += __shfl_xor(sum, o, 64);
#pragma unroll
        for (int m = 0; m < NQ; ++m)
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[m][e] += __shfl_xor(acc[m][e], o, 64);
    }
    float* red = reinterpret_cast<float*>(smem + C::OFF_RED);  // [NW][D] sums, [NW] max, [NW] sum
    if (r == 0) {
#pragma unroll
        for (int m = 0; m < NQ; ++m) *reinterpret_cast<f4*>(red + wave * D + qq * EQ + 4 * m) = acc[m];
    }
    if (lane == 0) {
        red[NW * D + wave] = wm;
        red[NW * D + NW + wave] = sum;
    }
    __syncthreads();  // logits and the per-wave partials of every wave

    // Waves -> pair.
    float gm = red[NW * D];
#pragma unroll
    for (int w = 1; w < NW; ++w) gm = fmaxf(gm, red[NW * D + w]);
    float fw[NW], total = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
        const float mw = red[NW * D + w];
        fw[w] = mw == -__builtin_inff() ? 0.0f : expf(mw - gm);
        total += red[NW * D + NW + w] * fw[w];
    }
    const float inv = 1.0f / (total + 1e-9f);
    for (int d = threadIdx.x; d < D; d += NW * 64) {
        float o = 0.0f;
#pragma unroll
        for (int w = 0; w < NW; ++w) o += red[w * D + d] * fw[w];
        p.out[bh * D + d] = o * inv;
    }
    // Probabilities: the last segment's logits from LDS, earlier ones from
    // attn_weights (written above by this same thread: the same index map).
    const int last0 = ((S - 1) / C::MAXS) * C::MAXS;
    for (int s = threadIdx.x; s < S; s += NW * 64) {
        const float l = s >= last0 ? logit[s - last0] : wout[s];
        wout[s] = expf(l - gm) * inv;
    }
}

template <int D, bool MASK>
hipError_t launch_dense_dma(const DenseParams& p, hipStream_t stream) {
    constexpr int NW = VCPP_DENSE_NW;
    using C = DenseDma<D, NW, MASK>;
    // The LDS limit is a per-device property of the kernel: raise it once on
    // each device the library launches on (idempotent if two threads race).
    static bool attr_set[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64 || !attr_set[dev]) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(dense_attention_dma_kernel<D, NW, MASK>),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, C::LDS);
        if (e != hipSuccess) return e;
        if (dev >= 0 && dev < 64) attr_set[dev] = true;
    }
    hipLaunchKernelGGL((dense_attention_dma_kernel<D, NW, MASK>), dim3(p.batch * p.heads), dim3(NW * 64), C::LDS,
                       stream, p);
    return hipGetLastError();
}

template <int D>
hipError_t launch_dense_dma(const DenseParams& p, hipStream_t stream) {
    return p.mask ? launch_dense_dma<D, true>(p, stream) : launch_dense_dma<D, false>(p, stream);
}

}  // namespace

// VCPP_DENSE_DMA=0 keeps the register-load kernels (for measurement).
static bool dense_dma_off() {
    static const bool off = [] {
        const char* e = std::getenv("VCPP_DENSE_DMA");
        return e && e[0] == '0';
    }();
    return off;
}

hipError_t launch_dense(const DenseParams& p, hipStream_t stream) {
    const dim3 grid(p.batch * p.heads), block(kThreads);
    auto al = [](const void* x) { return reinterpret_cast<uintptr_t>(x) % 16 == 0; };
    const bool vec = al(p.q) && al(p.k) && al(p.v) && p.kv_len > 0;
    const bool dma = vec && !dense_dma_off();
    if (dma && p.head_dim == 64) return launch_dense_dma<64>(p, stream);
    if (dma && p.head_dim == 80) return launch_dense_dma<80>(p, stream);
    if (dma && p.head_dim == 96) return launch_dense_dma<96>(p, stream);
    if (dma && p.head_dim == 128) return launch_dense_dma<128>(p, stream);
    if (vec && p.head_dim == 64) hipLaunchKernelGGL(dense_attention_vec_kernel<64>, grid, block, 0, stream, p);
    else if (vec && p.head_dim == 80) hipLaunchKernelGGL(dense_attention_vec_kernel<80>, grid, block, 0, stream, p);
    else if (vec && p.head_dim == 128) hipLaunchKernelGGL(dense_attention_vec_kernel<128>, grid, block, 0, stream, p);
    else hipLaunchKernelGGL(dense_attention_kernel, grid, block, p.head_dim * sizeof(float), stream, p);
    return hipGetLastError();
}

}  // namespace vcpp
