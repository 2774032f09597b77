// host_util.h -- helpers shared by the host-side BlockPool / KVCacheManager /
// paged_attention implementation.
#pragma once

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstring>
#include <stdexcept>
#include <mutex>
#include <string>
#include <vector>

#include "vllm_cpp/kv_config.h"

namespace vcpp_host {

inline void check(hipError_t e, const char* what) {
    if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

inline void check_rc(int rc, const char* what) {
    if (rc != 0) throw std::runtime_error(std::string(what) + ": " + vcpp_last_error());
}

// True for device (or managed) memory; plain host memory -- pageable, which
// the runtime does not know, or pinned -- is false.
inline bool is_device(const void* p) {
    if (!p) return false;
    hipPointerAttribute_t a{};
    const hipError_t e = hipPointerGetAttributes(&a, p);
    if (e != hipSuccess) {
        (void)hipGetLastError();  // an unknown host pointer is not an error here
        return false;
    }
    return a.type == hipMemoryTypeDevice || a.type == hipMemoryTypeManaged;
}

// The reference's fp16 -> fp32 decoder (src/kv_cache_manager.cpp:120-143):
// exact for zeros, subnormals and normals; exponent 31 gives +/-inf.
// FP8 E4M3 as the reference KV pool stores it (src/quantization.cpp:25-48):
// bias 7, exponent 15 = inf (mantissa 6) or NaN.
inline float fp8_decode(uint8_t b) {
    const int sign = (b >> 7) & 1, e = (b >> 3) & 0xF, m = b & 7;
    if (e == 0xF) return m == 6 ? (sign ? -INFINITY : INFINITY) : NAN;
    const float v = e == 0 ? (float)m / 8.0f * std::ldexp(1.0f, -6)
                           : (1.0f + (float)m / 8.0f) * std::ldexp(1.0f, e - 7);
    return sign ? -v : v;
}

inline float f16_decode(uint16_t h) {
    const uint32_t s = (h >> 15) & 1u, e = (h >> 10) & 0x1Fu;
    uint32_t f = h & 0x3FFu;
    uint32_t bits;
    if (e == 0) {
        if (f == 0) {
            bits = s << 31;
        } else {
            int ee = 1;
            while ((f & 0x400u) == 0) {
                f <<= 1;
                --ee;
            }
            f &= 0x3FFu;
            bits = (s << 31) | ((uint32_t)(127 - 15 + ee) << 23) | (f << 13);
        }
    } else if (e == 31) {
        bits = (s << 31) | 0x7F800000u;
    } else {
        bits = (s << 31) | ((127 - 15 + e) << 23) | (f << 13);
    }
    float out;
    std::memcpy(&out, &bits, 4);
    return out;
}

// One row [kv_dim] of a pool's page, raw bytes of dtype, to floats exactly as
// the reference pool decodes it (fp16: src/kv_cache_manager.cpp:120-143;
// FP8: src/quantization.cpp:25-48); INT8 rows take their [kv_dim / head_dim]
// fp16 scales.
inline void decode_row(const uint8_t* raw, const uint16_t* scales, float* out, int32_t kv_dim,
                       int32_t head_dim, KVDtype dtype) {
    switch (dtype) {
        case KVDtype::FP32:
            std::memcpy(out, raw, sizeof(float) * kv_dim);
            break;
        case KVDtype::FP16: {
            uint16_t h;
            for (int32_t i = 0; i < kv_dim; ++i) {
                std::memcpy(&h, raw + 2 * i, 2);
                out[i] = f16_decode(h);
            }
            break;
        }
        case KVDtype::FP8_E4M3:
            for (int32_t i = 0; i < kv_dim; ++i) out[i] = fp8_decode(raw[i]);
            break;
        case KVDtype::INT8:
            for (int32_t i = 0; i < kv_dim; ++i)
                out[i] = (float)(int8_t)raw[i] * f16_decode(scales[i / head_dim]);
            break;
    }
}

// A device buffer that only grows.  Growing waits for `stream` first: work
// queued there may still read the old buffer.
struct DevBuf {
    void* p = nullptr;
    size_t n = 0;
    void* get(size_t bytes, hipStream_t stream) {
        if (bytes > n) {
            if (p) {
                check(hipStreamSynchronize(stream), "device scratch: wait before growing");
                (void)hipFree(p);
            }
            p = nullptr;
            n = 0;
            check(hipMalloc(&p, bytes), "device scratch allocation");
            n = bytes;
        }
        return p;
    }
    ~DevBuf() {
        if (p) (void)hipFree(p);
    }
};

}  // namespace vcpp_host

// Device staging of the host entry points (paged_attention.cpp) for one
// BlockPool: calls on a pool are queued on the pool's stream, so buffers kept
// per pool are never overwritten by work on another pool's stream.
struct PoolStaging {
    std::mutex mu;
    vcpp_host::DevBuf q, out, tables, ctx, ws, k, v, slots, rows;
    std::vector<uint8_t> host;  // read_kv_prefill: gathered raw rows
};

