// device_common.h -- gfx950 device helpers shared by the attention kernels.
//
// Matrix-core fragment conventions used throughout (wave64, lane l,
// g = l / 16 the lane group, c = l % 16 the lane in its 16-lane row):
//   v_mfma_f32_16x16x32_f16  A: row c, k = 8g..8g+7     B: col c, k = 8g..8g+7
//   v_mfma_f32_16x16x16_f16  A: row c, k = 4g..4g+3     B: col c, k = 4g..4g+3
//   accumulator (both)       D: row 4g + r (r = 0..3), col c
// Only the row/column placement matters for correctness: any k order that is
// the same for A and B gives the same sum.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "vcpp_attention.h"

namespace vcpp {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef int i4 __attribute__((ext_vector_type(4)));
typedef int i2 __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;
constexpr float kLog2e = 1.4426950408889634f;
// Running-max seed: finite so that exp2(m_old - m_new) never sees inf - inf.
constexpr float kMaxSeed = -1e30f;

__device__ __forceinline__ f4 mfma32(h8 a, h8 b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f4 mfma16(h4 a, h4 b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}

// Value of lane l ^ 1 (DPP quad_perm [1,0,3,2]).
__device__ __forceinline__ float dpp_swap1(float x) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0xB1, 0xF, 0xF, false));
}

// Value of lane (l ^ 8) within each 16-lane row (DPP row_ror:8).
__device__ __forceinline__ float dpp_ror8(float x) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x128, 0xF, 0xF, false));
}

__device__ __forceinline__ float shfl_xor(float x, int m) { return __shfl_xor(x, m, kWave); }
__device__ __forceinline__ float shfl(float x, int src) { return __shfl(x, src, kWave); }

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Eight signed int8 (two dwords) -> eight exact fp16 values.  Uses the
// 1024-bias trick: the fp16 with bits 0x6400 | u has value 1024 + u for
// u in [0, 255], so (x ^ 0x80) placed under 0x64 minus 1152 is exactly x.
__device__ __forceinline__ h8 i8x8_to_h8(uint32_t lo, uint32_t hi) {
    lo ^= 0x80808080u;
    hi ^= 0x80808080u;
    // v_perm_b32 selector bytes: 0..3 from src1, 4..7 from src0 (0x64 pad).
    uint32_t w0 = __builtin_amdgcn_perm(0x64646464u, lo, 0x05010400u);
    uint32_t w1 = __builtin_amdgcn_perm(0x64646464u, lo, 0x05030402u);
    uint32_t w2 = __builtin_amdgcn_perm(0x64646464u, hi, 0x05010400u);
    uint32_t w3 = __builtin_amdgcn_perm(0x64646464u, hi, 0x05030402u);
    i4 w = {(int)w0, (int)w1, (int)w2, (int)w3};
    h8 v = __builtin_bit_cast(h8, w);
    const h8 bias = {1152, 1152, 1152, 1152, 1152, 1152, 1152, 1152};
    return v - bias;
}

__device__ __forceinline__ h4 i8x4_to_h4(uint32_t x) {
    x ^= 0x80808080u;
    uint32_t w0 = __builtin_amdgcn_perm(0x64646464u, x, 0x05010400u);
    uint32_t w1 = __builtin_amdgcn_perm(0x64646464u, x, 0x05030402u);
    i2 w = {(int)w0, (int)w1};
    h4 v = __builtin_bit_cast(h4, w);
    const h4 bias = {1152, 1152, 1152, 1152};
    return v - bias;
}

// FP8 E4M3 bytes -> fp16 with the gfx950 converter (OCP E4M3, scale 1).  The
// reference's E4M3 (bias 7, max 240) has the same value for every code whose
// exponent field is below 15, so finite reference pages convert exactly.
__device__ __forceinline__ h4 fp8x4_to_h4(uint32_t x) {
    const h2 a = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(x, 1.0f, false);
    const h2 b = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(x, 1.0f, true);
    return h4{a[0], a[1], b[0], b[1]};
}

__device__ __forceinline__ h8 fp8x8_to_h8(uint32_t lo, uint32_t hi) {
    const h4 a = fp8x4_to_h4(lo), b = fp8x4_to_h4(hi);
    return h8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}

// Bytes of a KV page -> fp16 MFMA operands (int8: exact integers; FP8: values).
template <int KV>
__device__ __forceinline__ h8 bytes8_to_h8(uint32_t lo, uint32_t hi) {
    if constexpr (KV == VCPP_KV_FP8) return fp8x8_to_h8(lo, hi);
    else return i8x8_to_h8(lo, hi);
}
template <int KV>
__device__ __forceinline__ h4 bytes4_to_h4(uint32_t x) {
    if constexpr (KV == VCPP_KV_FP8) return fp8x4_to_h4(x);
    else return i8x4_to_h4(x);
}


// Gather-index dump (checker builds only, -DVCPP_GATHER_DUMP): every kernel
// that addresses K/V pages records, per (sequence or chunk, position), the
// physical block and slot it loads, into an int32 [rows][stride][2] buffer the
// test reads back and compares with the block table.
#ifdef VCPP_GATHER_DUMP
template <class P>
__device__ __forceinline__ void gather_record(const P& p, int row, int pos, int bid, int slot) {
    if (p.gather_dump && pos < p.gather_stride) {
        int32_t* e = p.gather_dump + 2 * ((int64_t)row * p.gather_stride + pos);
        e[0] = bid;
        e[1] = slot;
    }
}
#endif

}  // namespace vcpp
