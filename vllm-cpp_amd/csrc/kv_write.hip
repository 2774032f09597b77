// kv_write.hip -- writes new tokens' K/V rows (fp32 on the device) into the
// paged pool: the device side of KVCacheManager::write_kv /
// write_kv_token / write_kv_prefill (src/kv_cache_manager.cpp:297-314,
// src/paged_attention.cpp:127-168).
//
// One wave per (token, kv head).  Encodings:
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
    const uint32_t b = fbits(x);
    const uint32_t s = b >> 31, e = (b >> 23) & 0xFFu, f = b & 0x7FFFFFu;
    if (e == 0xFFu) return (uint16_t)((s << 15) | (0x1Fu << 10) | (f ? 1u : 0u));
    const int ee = (int)e - 127 + 15;
    if (e == 0 || ee <= 0) return (uint16_t)(s << 15);
    if (ee >= 31) return (uint16_t)((s << 15) | (0x1Fu << 10));
    return (uint16_t)((s << 15) | ((uint32_t)ee << 10) | ((f >> 13) & 0x3FFu));
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
    // The largest code c with value <= a, and c + 1; both errors are exact
    // (the values lie within a factor 2 of a), so the nearest wins and a tie
    // keeps c, as the reference's first-minimum search does.
    uint32_t c;
    float lo, step;
    if (a < 0.015625f) {  // subnormal codes, multiples of 2^-9
        c = (uint32_t)(a * 512.0f);
        lo = (float)c * (1.0f / 512.0f);
        step = 1.0f / 512.0f;
    } else {
        const uint32_t b = fbits(a);
        const int e = (int)(b >> 23) - 127;  // -6 .. 7
        c = ((uint32_t)(e + 7) << 3) | ((b >> 20) & 7u);
        lo = __builtin_bit_cast(float, b & 0xFFF00000u);
        step = __builtin_bit_cast(float, (uint32_t)(e - 3 + 127) << 23);
    }
    const float hi = lo + step;
    return (uint8_t)(sign | ((hi - a) < (a - lo) ? c + 1 : c));
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

}  // namespace

hipError_t launch_kv_write(const KvWriteParams& p, hipStream_t stream) {
    const int64_t items = (int64_t)p.num_tokens * p.num_kv_heads;
    if (items == 0) return hipSuccess;
    hipLaunchKernelGGL(kv_write_kernel, dim3((unsigned)((items + 3) / 4)), dim3(256), 0, stream, p);
    return hipGetLastError();
}

}  // namespace vcpp
