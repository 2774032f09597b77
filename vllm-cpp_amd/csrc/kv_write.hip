// kv_write.hip -- writes new tokens' K/V rows (fp32 on the device) into the
// paged pool: the device side of KVCacheManager::write_kv /
// write_kv_token / write_kv_prefill (src/kv_cache_manager.cpp:297-314,
// src/paged_attention.cpp:127-168).
//
// One wave per (token, kv head) in general; a vector path (16-byte loads,
// several rows per wave) when head_dim % 4 == 0 and the pages are aligned.
// Encodings:
//   fp32  copied;
//   fp16  the reference encoder (src/kv_cache_manager.cpp:157-179): mantissa
//         truncated, exponents below the fp16 normal range flushed to +/-0,
//         overflow to +/-inf, NaN to an fp16 NaN -- or, on request, IEEE
//         round-to-nearest-even;
//   int8  symmetric per (token, kv head): scale = fp16_rne(max|x| / 127),
//         q = clamp(rne(x / scale), +/-127), q = 0 when the scale is 0;
//   fp8   the reference pool's E4M3 encoder (src/quantization.cpp:50-82 via
//         float_to_fp8_e4m3_batch): the finite code of the value's sign with
//         the smallest float error |a - |code||, the smaller code on a tie;
//         NaN -> 0xFF, +-inf -> 0x7E / 0xFE, +-0 -> 0x00.
#include "kv_write.h"

namespace vcpp {

namespace {

__device__ __forceinline__ uint32_t fbits(float x) { return __builtin_bit_cast(uint32_t, x); }

__device__ uint16_t f16_trunc(float x) {
    // The reference's truncating encoder on |x|'s bits: NaN keeps a quiet
    // payload of 1, exponents past fp16's (and inf) give inf, those below its
    // normal range give zero (no subnormals), the rest drop 13 mantissa bits
    // and rebias the exponent (fp32's bias 127 is 112 above fp16's).
    const uint32_t b = fbits(x), a = b & 0x7FFFFFFFu;
    const uint32_t mag = a > 0x7F800000u   ? 0x7C01u
                         : a >= 0x47800000u ? 0x7C00u
                         : a < 0x38800000u  ? 0u
                                            : (a >> 13) - (112u << 10);
    return (uint16_t)(((b >> 16) & 0x8000u) | mag);
}

__device__ uint16_t f16_rne(float x) { return __builtin_bit_cast(uint16_t, (_Float16)x); }

__device__ float f16_to_f32(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }

// Value of a finite E4M3 code 0x00..0x77 (bias 7, 3 mantissa bits).
__device__ float fp8_value(uint32_t c) {
    const uint32_t e = c >> 3, m = c & 7u;
    return e == 0 ? (float)m * (1.0f / 512.0f) : (1.0f + (float)m / 8.0f) * ldexpf(1.0f, (int)e - 7);
}

__device__ uint8_t fp8_encode(float v) {
    if (__builtin_isnan(v)) return 0xFF;
    if (__builtin_isinf(v)) return v > 0.f ? 0x7E : 0xFE;
    const uint32_t sign = v < 0.f ? 0x80u : 0u;
    const float a = fabsf(v);
    if (a == 0.f) return (uint8_t)sign;
    if (a > 240.f) {
        // Past the largest code the float errors a - code round, and several
        // codes can tie: the reference's search, over the finite codes.
        float best_err = __builtin_inff();
        uint32_t best = 0;
        for (uint32_t c = 0; c <= 0x77u; ++c) {
            const float err = fabsf(a - fp8_value(c));
            if (err < best_err) {
                best_err = err;
                best = c;
            }
        }
        return (uint8_t)(sign | best);
    }
    // Nearest code, a tie keeping the smaller one (the reference's search
    // takes the first minimum over ascending codes).  Normal codes: the
    // float's top 12 bits are (exponent, 3 mantissa bits), so adding half a
    // code step minus one unit and shifting rounds half down, a carry moving
    // into the exponent; E4M3's bias 7 is 120 below fp32's.  Subnormal codes
    // are multiples of 2^-9: ceil(x - 1/2) rounds x = 512 a half down (x - 1/2
    // is exact for x >= 1/4, and below that either way rounds to 0).
    const uint32_t c = a < 0.015625f ? (uint32_t)__builtin_ceilf(a * 512.0f - 0.5f)
                                     : ((fbits(a) + 0x7FFFFu) >> 20) - (120u << 3);
    return (uint8_t)(sign | c);
}

__global__ __launch_bounds__(256) void kv_write_kernel(KvWriteParams p) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int64_t item = (int64_t)blockIdx.x * 4 + wave;  // (token, kv head)
    if (item >= (int64_t)p.num_tokens * p.num_kv_heads) return;
    const int64_t tok = item / p.num_kv_heads;
    const int h = (int)(item - tok * p.num_kv_heads);
    const int64_t slot = p.slots[tok];
    if (slot < 0) return;
    const int64_t block = slot / p.block_size;
    if (block >= p.num_blocks) return;
    const int pos = (int)(slot - block * p.block_size);
    const int D = p.head_dim;
    const int64_t src_off = (tok * p.num_kv_heads + h) * D;
    const int64_t dst_off = block * p.block_stride + ((int64_t)pos * p.num_kv_heads + h) * D;
    for (int which = 0; which < 2; ++which) {
        const float* src = (which ? p.v_src : p.k_src) + src_off;
        void* base = which ? p.v : p.k;
        if (p.dtype == VCPP_KV_F32) {
            for (int d = lane; d < D; d += 64) static_cast<float*>(base)[dst_off + d] = src[d];
        } else if (p.dtype == VCPP_KV_FP8) {
            uint8_t* dst = static_cast<uint8_t*>(base) + dst_off;
            for (int d = lane; d < D; d += 64) dst[d] = fp8_encode(src[d]);
        } else if (p.dtype == VCPP_KV_F16) {
            uint16_t* dst = static_cast<uint16_t*>(base) + dst_off;
            for (int d = lane; d < D; d += 64) dst[d] = p.fp16_rne ? f16_rne(src[d]) : f16_trunc(src[d]);
        } else {
            float amax = 0.0f;
            for (int d = lane; d < D; d += 64) amax = fmaxf(amax, fabsf(src[d]));
            for (int m = 32; m > 0; m >>= 1) amax = fmaxf(amax, __shfl_xor(amax, m, 64));
            const uint16_t sh = f16_rne(amax / 127.0f);
            const float s = f16_to_f32(sh);
            int8_t* dst = static_cast<int8_t*>(base) + dst_off;
            for (int d = lane; d < D; d += 64) {
                float r = s > 0.0f ? rintf(src[d] / s) : 0.0f;
                r = fminf(fmaxf(r, -127.0f), 127.0f);
                dst[d] = (int8_t)r;
            }
            if (lane == 0) {
                uint16_t* sc = which ? p.v_scale : p.k_scale;
                sc[block * p.scale_block_stride + (int64_t)h * p.block_size + pos] = sh;
            }
        }
    }
}

// Vector path (head_dim % 4 == 0, aligned pages): a row of one (token, kv
// head) is owned by L = head_dim / 4 consecutive lanes, 4 values each (one
// 16-byte load per lane and K/V), rows_per_wave = 64 / L rows per wave.  Same
// encodings as kv_write_kernel; int8 forms the row's max |x| across its lane
// segment.
template <int KV>
__global__ __launch_bounds__(256) void kv_write_vec_kernel(KvWriteParams p, int L, int rows_per_wave) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int seg = lane / L, li = lane - seg * L;
    if (seg >= rows_per_wave) return;  // whole segments idle
    const int64_t item = ((int64_t)blockIdx.x * 4 + wave) * rows_per_wave + seg;
    if (item >= (int64_t)p.num_tokens * p.num_kv_heads) return;
    const int64_t tok = item / p.num_kv_heads;
    const int h = (int)(item - tok * p.num_kv_heads);
    const int64_t slot = p.slots[tok];
    if (slot < 0) return;
    const int64_t block = slot / p.block_size;
    if (block >= p.num_blocks) return;
    const int pos = (int)(slot - block * p.block_size);
    const int D = p.head_dim;
    const int64_t src_off = (tok * p.num_kv_heads + h) * D + 4 * li;
    const int64_t dst_off = block * p.block_stride + ((int64_t)pos * p.num_kv_heads + h) * D + 4 * li;
    for (int which = 0; which < 2; ++which) {
        const float4 x = *reinterpret_cast<const float4*>((which ? p.v_src : p.k_src) + src_off);
        void* base = which ? p.v : p.k;
        if constexpr (KV == VCPP_KV_F32) {
            *reinterpret_cast<float4*>(static_cast<float*>(base) + dst_off) = x;
        } else if constexpr (KV == VCPP_KV_F16) {
            uint16_t e[4];
            const float xs[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) e[i] = p.fp16_rne ? f16_rne(xs[i]) : f16_trunc(xs[i]);
            *reinterpret_cast<uint2*>(static_cast<uint16_t*>(base) + dst_off) =
                make_uint2(e[0] | ((uint32_t)e[1] << 16), e[2] | ((uint32_t)e[3] << 16));
        } else if constexpr (KV == VCPP_KV_FP8) {
            const uint32_t w = fp8_encode(x.x) | ((uint32_t)fp8_encode(x.y) << 8) |
                               ((uint32_t)fp8_encode(x.z) << 16) | ((uint32_t)fp8_encode(x.w) << 24);
            *reinterpret_cast<uint32_t*>(static_cast<uint8_t*>(base) + dst_off) = w;
        } else {
            float amax = fmaxf(fmaxf(fabsf(x.x), fabsf(x.y)), fmaxf(fabsf(x.z), fabsf(x.w)));
            float row_max = amax;
            if (L % 4 == 0) {
                // Segments of whole quads (a row's lanes all active or all
                // returned): the quad's max by two DPP quad permutes, then one
                // read per quad of the segment (max is exact in any order).
                float qm = fmaxf(amax, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                                           0, __builtin_bit_cast(int, amax), 0xB1, 0xF, 0xF, false)));
                qm = fmaxf(qm, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                                   0, __builtin_bit_cast(int, qm), 0x4E, 0xF, 0xF, false)));
                row_max = qm;
                for (int j = 0; j < L; j += 4) row_max = fmaxf(row_max, __shfl(qm, seg * L + j, 64));
            } else {
                for (int j = 0; j < L; ++j) row_max = fmaxf(row_max, __shfl(amax, seg * L + j, 64));
            }
            const uint16_t sh = f16_rne(row_max / 127.0f);
            const float sc = f16_to_f32(sh);
            const float xs[4] = {x.x, x.y, x.z, x.w};
            // rint(x / sc) with x / sc correctly rounded, as the oracle
            // computes it.  q = x * fl(1 / sc) is within 2 ulp of fl(x / sc)
            // (|q| <= 128: 2^-15); when q is more than 2^-14 from every
            // half-integer no half-integer lies between the two and their
            // rint agree, otherwise (rarely) divide.
            const float isc = sc > 0.0f ? 1.0f / sc : 0.0f;
            uint32_t w = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float qf = xs[i] * isc;
                float r = rintf(qf);
                if (sc > 0.0f && fabsf(fabsf(qf - r) - 0.5f) < 6.103515625e-05f) r = rintf(xs[i] / sc);
                if (!(sc > 0.0f)) r = 0.0f;
                r = fminf(fmaxf(r, -127.0f), 127.0f);
                w |= (uint32_t)(uint8_t)(int8_t)r << (8 * i);
            }
            *reinterpret_cast<uint32_t*>(static_cast<int8_t*>(base) + dst_off) = w;
            if (li == 0) {
                uint16_t* scp = which ? p.v_scale : p.k_scale;
                scp[block * p.scale_block_stride + (int64_t)h * p.block_size + pos] = sh;
            }
        }
    }
}

// fp16, int8 and FP8 pages with head_dim % 8 == 0: eight values per lane (two
// 16-byte loads of each of K and V), so a lane stores 16 bytes (fp16) or 8
// (int8, FP8) at once; D / 8 lanes own a row.  Same encoders, element by
// element; the int8 row max is exact in any order (a lane-pair DPP swap, then
// one read per pair: rows start on even lanes).
template <int KV>
__global__ __launch_bounds__(256) void kv_write_vec8_kernel(KvWriteParams p, int L, int rows_per_wave) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int seg = lane / L, li = lane - seg * L;
    if (seg >= rows_per_wave) return;  // whole segments idle
    const int64_t item = ((int64_t)blockIdx.x * 4 + wave) * rows_per_wave + seg;
    if (item >= (int64_t)p.num_tokens * p.num_kv_heads) return;
    const int64_t tok = item / p.num_kv_heads;
    const int h = (int)(item - tok * p.num_kv_heads);
    const int64_t slot = p.slots[tok];
    if (slot < 0) return;
    const int64_t block = slot / p.block_size;
    if (block >= p.num_blocks) return;
    const int pos = (int)(slot - block * p.block_size);
    const int D = p.head_dim;
    const int64_t src_off = (tok * p.num_kv_heads + h) * D + 8 * li;
    const int64_t dst_off = block * p.block_stride + ((int64_t)pos * p.num_kv_heads + h) * D + 8 * li;
    for (int which = 0; which < 2; ++which) {
        const float* src = (which ? p.v_src : p.k_src) + src_off;
        const float4 a = *reinterpret_cast<const float4*>(src);
        const float4 b = *reinterpret_cast<const float4*>(src + 4);
        const float xs[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
        void* base = which ? p.v : p.k;
        if constexpr (KV == VCPP_KV_F16) {
            uint32_t w[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint16_t e0 = p.fp16_rne ? f16_rne(xs[2 * i]) : f16_trunc(xs[2 * i]);
                const uint16_t e1 = p.fp16_rne ? f16_rne(xs[2 * i + 1]) : f16_trunc(xs[2 * i + 1]);
                w[i] = e0 | ((uint32_t)e1 << 16);
            }
            *reinterpret_cast<uint4*>(static_cast<uint16_t*>(base) + dst_off) = make_uint4(w[0], w[1], w[2], w[3]);
        } else if constexpr (KV == VCPP_KV_I8) {
            float amax = 0.0f;
#pragma unroll
            for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(xs[i]));
            const float pm = fmaxf(amax, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                                             0, __builtin_bit_cast(int, amax), 0xB1, 0xF, 0xF, false)));
            float row_max = pm;
            for (int j = 0; j < L; j += 2) row_max = fmaxf(row_max, __shfl(pm, seg * L + j, 64));
            const uint16_t sh = f16_rne(row_max / 127.0f);
            const float sc = f16_to_f32(sh);
            // rint(x / sc), x / sc correctly rounded: see kv_write_vec_kernel
            const float isc = sc > 0.0f ? 1.0f / sc : 0.0f;
            uint32_t w[2] = {0u, 0u};
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float qf = xs[i] * isc;
                float r = rintf(qf);
                if (sc > 0.0f && fabsf(fabsf(qf - r) - 0.5f) < 6.103515625e-05f) r = rintf(xs[i] / sc);
                if (!(sc > 0.0f)) r = 0.0f;
                r = fminf(fmaxf(r, -127.0f), 127.0f);
                w[i >> 2] |= (uint32_t)(uint8_t)(int8_t)r << (8 * (i & 3));
            }
            *reinterpret_cast<uint2*>(static_cast<int8_t*>(base) + dst_off) = make_uint2(w[0], w[1]);
            if (li == 0) {
                uint16_t* scp = which ? p.v_scale : p.k_scale;
                scp[block * p.scale_block_stride + (int64_t)h * p.block_size + pos] = sh;
            }
        } else {
            uint32_t w[2];
#pragma unroll
            for (int i = 0; i < 2; ++i)
                w[i] = fp8_encode(xs[4 * i]) | ((uint32_t)fp8_encode(xs[4 * i + 1]) << 8) |
                       ((uint32_t)fp8_encode(xs[4 * i + 2]) << 16) | ((uint32_t)fp8_encode(xs[4 * i + 3]) << 24);
            *reinterpret_cast<uint2*>(static_cast<uint8_t*>(base) + dst_off) = make_uint2(w[0], w[1]);
        }
    }
}

}  // namespace

hipError_t launch_kv_write(const KvWriteParams& p, hipStream_t stream) {
    const int64_t items = (int64_t)p.num_tokens * p.num_kv_heads;
    if (items == 0) return hipSuccess;
    const int es = p.dtype == VCPP_KV_F32 ? 4 : p.dtype == VCPP_KV_F16 ? 2 : 1;
    auto aligned = [](const void* q, int a) { return (reinterpret_cast<uintptr_t>(q) % a) == 0; };
    const bool vec = p.head_dim % 4 == 0 && p.head_dim <= 256 && p.block_stride % 4 == 0 &&
                     aligned(p.k_src, 16) && aligned(p.v_src, 16) && aligned(p.k, 4 * es) &&
                     aligned(p.v, 4 * es);
    // int8's pair-swap row max needs rows to start on even lanes: D / 8 even
    const bool vec8 = vec && p.dtype != VCPP_KV_F32 && p.head_dim % (p.dtype == VCPP_KV_I8 ? 16 : 8) == 0 &&
                      p.head_dim >= 16 &&
                      p.block_stride % 8 == 0 && aligned(p.k, 8 * es) && aligned(p.v, 8 * es);
    if (vec8) {
        const int L = p.head_dim / 8, rpw = 64 / L;
        const int64_t waves = (items + rpw - 1) / rpw;
        const dim3 grid((unsigned)((waves + 3) / 4)), block(256);
        if (p.dtype == VCPP_KV_F16)
            hipLaunchKernelGGL(kv_write_vec8_kernel<VCPP_KV_F16>, grid, block, 0, stream, p, L, rpw);
        else if (p.dtype == VCPP_KV_I8)
            hipLaunchKernelGGL(kv_write_vec8_kernel<VCPP_KV_I8>, grid, block, 0, stream, p, L, rpw);
        else
            hipLaunchKernelGGL(kv_write_vec8_kernel<VCPP_KV_FP8>, grid, block, 0, stream, p, L, rpw);
        return hipGetLastError();
    }
    if (vec) {
        const int L = p.head_dim / 4, rpw = 64 / L;
        const int64_t waves = (items + rpw - 1) / rpw;
        const dim3 grid((unsigned)((waves + 3) / 4)), block(256);
        switch (p.dtype) {
            case VCPP_KV_F32: hipLaunchKernelGGL(kv_write_vec_kernel<VCPP_KV_F32>, grid, block, 0, stream, p, L, rpw); break;
            case VCPP_KV_F16: hipLaunchKernelGGL(kv_write_vec_kernel<VCPP_KV_F16>, grid, block, 0, stream, p, L, rpw); break;
            case VCPP_KV_FP8: hipLaunchKernelGGL(kv_write_vec_kernel<VCPP_KV_FP8>, grid, block, 0, stream, p, L, rpw); break;
            default: hipLaunchKernelGGL(kv_write_vec_kernel<VCPP_KV_I8>, grid, block, 0, stream, p, L, rpw); break;
        }
        return hipGetLastError();
    }
    hipLaunchKernelGGL(kv_write_kernel, dim3((unsigned)((items + 3) / 4)), dim3(256), 0, stream, p);
    return hipGetLastError();
}

}  // namespace vcpp
