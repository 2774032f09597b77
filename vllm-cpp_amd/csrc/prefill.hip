// prefill.hip -- the chunked causal prefill kernel: one workgroup per
// (query tile, chunk, kv head / head group), the work of prefill_tile
// (prefill_body.h).
#include "prefill_body.h"
#include "prefill_wide.h"
#include "profile.h"

#include <cstdlib>

namespace vcpp {

namespace {

// Workgroups are dealt to the 8 XCDs round-robin by linear id; remap so that
// each XCD walks a contiguous range of (tile, head group, chunk, kv head) ids
// and its L2 holds the K/V of the (chunk, kv head) pair it is serving.  slots: the
// workgroups one CU holds at once (a grid of at most slots per CU pairs the
// k-th heaviest tile of an XCD's share with its k-th lightest on one CU).
__device__ __forceinline__ void remap_ids(const PrefillParams& p, int slots, int& bx, int& by, int& bz) {
    bx = blockIdx.x, by = blockIdx.y, bz = blockIdx.z;
    const int nx = gridDim.x, ny = gridDim.y;
    const int total = nx * ny * gridDim.z;
    if ((total & 7) == 0) {
        const int lin = bx + nx * (by + ny * bz);
        const int per = total >> 3;  // ids per XCD
        int j = lin >> 3;            // dispatch order within the XCD
#ifndef VCPP_PF_NO_PAIRING
        // A grid that fits the GPU in one round (at most two workgroups per
        // CU): the dispatcher gives each CU of an XCD one workgroup before it
        // gives any a second, so local ids j and j + C (C CUs per XCD) share
        // a CU.  Reversing the order of the second ones puts the k-th
        // heaviest tile beside the k-th lightest of the XCD's share.
        // (Grids of several rounds keep heaviest-first order.)
        const int C = p.xcd_cus;
        if (slots == 2 && C > 0 && per > C && per <= 2 * C && j >= C) j = per + C - 1 - j;
#endif
        // m = tile + nx (head group + HG (chunk + ny (kv head, key part))):
        // an XCD's consecutive ids are the tiles of both head groups of one
        // (chunk, kv head), which read the same K/V pages, so its L2 serves
        // them to all of its concurrently running workgroups.
        const int m = (lin & 7) * per + j;
        const int HG = p.head_groups;
        bx = m % nx;
        int r = m / nx;
        const int hg = r % HG;
        r /= HG;
        by = r % ny;
        bz = (r / ny) * HG + hg;
    }
}

template <int KV, int D>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))
void prefill_dma_kernel(PrefillParams p) {
    extern __shared__ __attribute__((aligned(16))) char smem[];
    int bx, by, bz;
    remap_ids(p, 2, bx, by, bz);
    // z: (key part, kv head, head group)
    const int zh = p.num_kv_heads * p.head_groups;
    const int part = bz / zh;
    prefill_tile<KV, D, false>(p, bx, by, bz - part * zh, part,
                               reinterpret_cast<lds_char*>((__attribute__((address_space(3))) char*)smem));
}

// fp16 pages at head_dim 64 / 80: 128-row tiles, one wave per SIMD
// (prefill_wide_run).
template <int D>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
void prefill_wide_kernel(PrefillParams p) {
    extern __shared__ __attribute__((aligned(16))) char smem[];
    prefill_wide_run<D>(p, reinterpret_cast<lds_char*>((__attribute__((address_space(3))) char*)smem));
}

// Log-sum-exp merge of a split prefill's S parts: thread (row, head, 4 dims).
// S is a template argument so that the parts' loads are all issued before
// their first use, in exactly S registers' worth of values.
template <int S>
__global__ __launch_bounds__(256) void prefill_merge_kernel(PrefillParams p) {
    const int D4 = p.head_dim / 4;
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t per_row = (int64_t)p.num_heads * D4;
    const int row = (int)(idx / per_row);
    if (row >= p.q_start[p.num_chunks]) return;
    // Rows of a chunk longer than max_chunk_len (a caller error) that no
    // query tile of the grid covered are left unwritten, as the unsplit
    // kernel leaves them: the grid covers each chunk's last
    // ceil(max_chunk_len / tile_rows) tiles.
    {
        int lo = 0, hi = p.num_chunks - 1;  // chunk of the row: last c with q_start[c] <= row
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (p.q_start[mid] <= row) lo = mid;
            else hi = mid - 1;
        }
        const int q0 = p.q_start[lo], n = p.q_start[lo + 1] - q0;
        const int ntile = (n + p.tile_rows - 1) / p.tile_rows;
        const int first = ntile - (p.max_chunk_len + p.tile_rows - 1) / p.tile_rows;
        if (first > 0 && row - q0 < first * p.tile_rows) return;
    }
    const int rem = (int)(idx - row * per_row);
    const int head = rem / D4, d4 = rem - head * D4;
    float2 ml[S];
    float4 v[S];
    float M = -__builtin_inff();
#pragma unroll
    for (int s = 0; s < S; ++s) {
        const int64_t rh = ((int64_t)s * p.rows_cap + row) * p.num_heads + head;
        ml[s] = p.ws_ml[rh];
        v[s] = reinterpret_cast<const float4*>(p.ws_o + rh * p.head_dim)[d4];
    }
#pragma unroll
    for (int s = 0; s < S; ++s)
        if (ml[s].y > 0.f) M = fmaxf(M, ml[s].x);  // parts with no visible key (sum 0) weigh 0
    float L = 0.f;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int s = 0; s < S; ++s) {
        if (ml[s].y > 0.f) {
            const float w = exp2f(ml[s].x - M);
            L += w * ml[s].y;
            acc.x += w * v[s].x;
            acc.y += w * v[s].y;
            acc.z += w * v[s].z;
            acc.w += w * v[s].w;
        }
    }
    const float inv = 1.0f / (L + 1e-9f);
    reinterpret_cast<float4*>(p.out + ((int64_t)row * p.num_heads + head) * p.head_dim)[d4] =
        make_float4(acc.x * inv, acc.y * inv, acc.z * inv, acc.w * inv);
}

template <int S>
hipError_t launch_merge_s(const PrefillParams& p, hipStream_t stream) {
    if (p.splits != S) return launch_merge_s<S - 1>(p, stream);
    const int64_t threads = (int64_t)p.rows_cap * p.num_heads * (p.head_dim / 4);
    hipLaunchKernelGGL(prefill_merge_kernel<S>, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, stream, p);
    return hipGetLastError();
}
template <>
hipError_t launch_merge_s<1>(const PrefillParams&, hipStream_t) { return hipErrorInvalidValue; }

// VCPP_PF_WIDE=1: fp16 pages at head_dim 64 / 80 (power-of-two block size)
// run prefill_wide_kernel instead of prefill_dma_kernel.  Opt-in: on MI355X
// it measured about 10 % slower on config 3 (read at every launch, so a
// process can switch).
bool wide_requested() {
    const char* e = std::getenv("VCPP_PF_WIDE");
    return e && e[0] == '1';
}

template <int KV, int D>
constexpr bool use_wide_t() { return KV == VCPP_KV_F16 && wide_prefill_ok<D>(); }

bool pow2(int x) { return x > 0 && (x & (x - 1)) == 0; }

template <int KV, int D>
hipError_t launch_dma(const PrefillParams& p, hipStream_t stream) {
    const bool wide = prefill_uses_wide(KV, D, p.block_size);
    const int QT = prefill_tile_rows(KV, D, p.block_size);
    dim3 grid((p.max_chunk_len + QT - 1) / QT, p.num_chunks,
              p.num_kv_heads * p.head_groups * max(p.splits, 1));
    size_t lds = (wide ? (size_t)WDims<D>::STAGES * DmaDims<D>::STAGE + 1024 : prefill_ring_bytes(KV, D)) +
                 (size_t)p.max_blocks * 4;
#ifdef VCPP_PREFILL_LDS_PAD
    lds = std::max<size_t>(lds, VCPP_PREFILL_LDS_PAD);
#endif
    // Raise the kernel's dynamic LDS limit on this device only when a launch
    // needs more than it was last set to there (the attribute call is a host
    // round trip; the limit is per device).
    static size_t attr_lds[2][64] = {};
    int dev = 0;
    const bool known = hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < 64;
    const void* fn = (const void*)prefill_dma_kernel<KV, D>;
    if constexpr (use_wide_t<KV, D>()) {
        if (wide) fn = (const void*)prefill_wide_kernel<D>;
    }
    if (!known || lds > std::max<size_t>(attr_lds[wide][dev], 65536)) {
        const hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
        if (known) attr_lds[wide][dev] = lds;
    }
    if constexpr (use_wide_t<KV, D>()) {
        if (wide) {
            // A 1-D grid of all tiles (ordered by wide_tile_ids).
            const unsigned tiles = grid.x * grid.y * grid.z;
            hipLaunchKernelGGL((prefill_wide_kernel<D>), dim3(tiles), dim3(256), lds, stream, p);
            return hipGetLastError();
        }
    }
    hipLaunchKernelGGL((prefill_dma_kernel<KV, D>), grid, dim3(256), lds, stream, p);
    return hipGetLastError();
}


}  // namespace

bool prefill_uses_wide(int kv_dtype, int head_dim, int block_size) {
    return kv_dtype == VCPP_KV_F16 && (head_dim == 64 || head_dim == 80) && pow2(block_size) && wide_requested();
}

int prefill_tile_rows(int kv_dtype, int head_dim, int block_size) {
    if (prefill_uses_wide(kv_dtype, head_dim, block_size)) return WDims<80>::QT;
    switch (head_dim) {
        case 64: return 16 * PDims<64>::RB;
        case 80: return 16 * PDims<80>::RB;
        default: return 16 * PDims<128>::RB;
    }
}

int prefill_head_groups(int group) { return (group + kHeadsPerGroup - 1) / kHeadsPerGroup; }

// LDS of the ring of prefill_dma_kernel.
size_t prefill_ring_bytes(int kv_dtype, int head_dim) {
    auto ring = [&](auto d) -> size_t {
        constexpr int D = decltype(d)::value;
        if (kv_dtype == VCPP_KV_I8)
            return (size_t)ByteDims<D, true>::STAGES * ByteDims<D, true>::STAGE + 2 * (size_t)DmaDims<D>::STAGE;
        if (kv_dtype == VCPP_KV_FP8)
            return (size_t)ByteDims<D, false>::STAGES * ByteDims<D, false>::STAGE + 2 * (size_t)DmaDims<D>::STAGE;
        return (size_t)DmaDims<D>::STAGES * DmaDims<D>::STAGE;
    };
    switch (head_dim) {
        case 64: return ring(std::integral_constant<int, 64>{});
        case 80: return ring(std::integral_constant<int, 80>{});
        case 128: return ring(std::integral_constant<int, 128>{});
        default: return 0;
    }
}

size_t prefill_lds_bytes(int kv_dtype, int head_dim, int max_blocks) {
    size_t r = prefill_ring_bytes(kv_dtype, head_dim);
    if (r == 0) return 0;
    if (kv_dtype == VCPP_KV_F16 && head_dim == 64)
        r = std::max<size_t>(r, (size_t)WDims<64>::STAGES * DmaDims<64>::STAGE + 1024);
    if (kv_dtype == VCPP_KV_F16 && head_dim == 80)
        r = std::max<size_t>(r, (size_t)WDims<80>::STAGES * DmaDims<80>::STAGE + 1024);
    return r + (size_t)max_blocks * 4;
}

hipError_t launch_prefill(const PrefillParams& p, hipStream_t stream) {
    if (p.num_chunks == 0 || p.max_chunk_len == 0) return hipSuccess;
    const bool prof = prof_enabled();
    if (prof) prof_begin(kKernelPrefill, stream);
    hipError_t err = hipErrorInvalidValue;
#define VCPP_PF_D(KVT)                                      \
    switch (p.head_dim) {                                   \
        case 64: err = launch_dma<KVT, 64>(p, stream); break;   \
        case 80: err = launch_dma<KVT, 80>(p, stream); break;   \
        case 128: err = launch_dma<KVT, 128>(p, stream); break; \
        default: return hipErrorInvalidValue;               \
    }
    if (p.kv_dtype == VCPP_KV_F16) {
        VCPP_PF_D(VCPP_KV_F16)
    } else if (p.kv_dtype == VCPP_KV_FP8) {
        VCPP_PF_D(VCPP_KV_FP8)
    } else {
        VCPP_PF_D(VCPP_KV_I8)
    }
#undef VCPP_PF_D
    if (err != hipSuccess) return err;
    if (p.splits > 1) {
        if (p.splits > kMaxPrefillSplits) return hipErrorInvalidValue;
        PrefillParams pm = p;
        pm.tile_rows = prefill_tile_rows(p.kv_dtype, p.head_dim, p.block_size);
        err = launch_merge_s<kMaxPrefillSplits>(pm, stream);
        if (err != hipSuccess) return err;
    }
    if (prof) prof_end(kKernelPrefill, stream);
    return hipSuccess;
}

size_t prefill_split_bytes(int splits, int rows_cap, int num_heads, int head_dim) {
    if (splits <= 1) return 0;
    const size_t rows = (size_t)splits * rows_cap * num_heads;
    return ((rows * head_dim * sizeof(float) + 255) & ~size_t(255)) + rows * sizeof(float2);
}

}  // namespace vcpp

#ifdef VCPP_PF_TIMING
// Timing builds only: reads and clears the wide prefill's segment sums.
extern "C" int vcpp_pf_timing_read(unsigned long long* out) {
    if (hipMemcpyFromSymbol(out, HIP_SYMBOL(vcpp::g_pf_timing), 16 * sizeof(unsigned long long)) != hipSuccess)
        return -1;
    unsigned long long z[16] = {};
    return hipMemcpyToSymbol(HIP_SYMBOL(vcpp::g_pf_timing), z, sizeof(z)) == hipSuccess ? 0 : -1;
}
#endif
