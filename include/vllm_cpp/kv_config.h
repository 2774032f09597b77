// kv_config.h -- the KV-cache constants of the reference's src/config.h
// (BLOCK_SIZE, src/config.h:48; KVDtype, src/config.h:69-73) plus INT8.
//
// An engine that keeps its own config.h adds `INT8 = 3` to its KVDtype and
// defines VCPP_EXTERNAL_KV_CONFIG before including the vllm_cpp headers.
#pragma once

#include <cstdint>

#ifndef VCPP_EXTERNAL_KV_CONFIG
constexpr int32_t BLOCK_SIZE = 16;

enum class KVDtype : uint8_t {
    FP32 = 0,
    FP16 = 1,
    FP8_E4M3 = 2,  // the reference's E4M3 (src/quantization.cpp:25-82): VCPP_KV_FP8 pages
    INT8 = 3,      // symmetric int8, one fp16 scale per (token, kv head)
};
#endif
