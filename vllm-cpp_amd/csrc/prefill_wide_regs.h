// prefill_wide_regs.h -- the wide prefill's accumulation registers
// (prefill_wide.h).  The output accumulators and the Q fragments live in
// AGPRs that no C++ value names: output block I (= row block * NT + column
// block) in a[4I : 4I+3], Q fragment J in a[kWQBase + 4J : kWQBase + 4J + 3].
// Every instruction that touches them is inline assembly naming them by
// number, so the compiler neither moves nor copies them (it would, for
// values it can allocate, through VGPRs around every use).  kw_reserve()
// clobbers the highest one, which sizes the kernel's AGPR allocation; the
// compiler itself must use no AGPR in these kernels (no VGPR spilling to
// AGPRs: prefill.hip is built with -amdgpu-spill-vgpr-to-agpr=0, and
// build.py checks the kernels' assembly).
//
// The compiler's hazard recognizer does not see into inline assembly, so
// the callers keep every MFMA result and every AGPR write far from its
// first reader (a whole MFMA group, or explicit s_nop).
#pragma once

#include "device_common.h"

namespace vcpp {

namespace {

constexpr int kWQBase = 160;  // first Q fragment register
constexpr int kWTop = 239;    // highest register used

__device__ __forceinline__ void kw_reserve() { asm volatile("" ::: "a239"); }

// a[N] = 0
template <int N>
__device__ __forceinline__ void kw_zero() { asm volatile("v_accvgpr_write_b32 a%c0, 0" ::"n"(N)); }

// Q fragment J = q
template <int J>
__device__ __forceinline__ void kw_set_q(const h8& q) {
    const i4 w = __builtin_bit_cast(i4, q);
    asm volatile("v_accvgpr_write_b32 a%c4, %0\n\tv_accvgpr_write_b32 a%c5, %1\n\t"
                 "v_accvgpr_write_b32 a%c6, %2\n\tv_accvgpr_write_b32 a%c7, %3"
                 ::"v"(w[0]), "v"(w[1]), "v"(w[2]), "v"(w[3]), "n"(kWQBase + 4 * J), "n"(kWQBase + 4 * J + 1),
                   "n"(kWQBase + 4 * J + 2), "n"(kWQBase + 4 * J + 3));
}

// d = k q_J  /  d += k q_J
template <int J>
__device__ __forceinline__ void kw_s0(f4& d, const h8& k) {
    asm volatile("v_mfma_f32_16x16x32_f16 %0, %1, a[%c2:%c3], 0"
                 : "=&v"(d) : "v"(k), "n"(kWQBase + 4 * J), "n"(kWQBase + 4 * J + 3));
}
template <int J>
__device__ __forceinline__ void kw_s(f4& d, const h8& k) {
    asm volatile("v_mfma_f32_16x16x32_f16 %0, %1, a[%c2:%c3], %0"
                 : "+v"(d) : "v"(k), "n"(kWQBase + 4 * J), "n"(kWQBase + 4 * J + 3));
}

// o_I += p v
template <int I>
__device__ __forceinline__ void kw_pv(const h8& p, const h8& v) {
    asm volatile("v_mfma_f32_16x16x32_f16 a[%c2:%c3], %0, %1, a[%c2:%c3]"
                 ::"v"(p), "v"(v), "n"(4 * I), "n"(4 * I + 3));
}

// o_I *= (a0, a1, a2, a3) component-wise
template <int I>
__device__ __forceinline__ void kw_scale(float a0, float a1, float a2, float a3) {
    float t;
    asm volatile("v_accvgpr_read_b32 %0, a%c5\n\tv_mul_f32 %0, %0, %1\n\tv_accvgpr_write_b32 a%c5, %0\n\t"
                 "v_accvgpr_read_b32 %0, a%c6\n\tv_mul_f32 %0, %0, %2\n\tv_accvgpr_write_b32 a%c6, %0\n\t"
                 "v_accvgpr_read_b32 %0, a%c7\n\tv_mul_f32 %0, %0, %3\n\tv_accvgpr_write_b32 a%c7, %0\n\t"
                 "v_accvgpr_read_b32 %0, a%c8\n\tv_mul_f32 %0, %0, %4\n\tv_accvgpr_write_b32 a%c8, %0"
                 : "=&v"(t) : "v"(a0), "v"(a1), "v"(a2), "v"(a3), "n"(4 * I), "n"(4 * I + 1), "n"(4 * I + 2),
                   "n"(4 * I + 3));
}

// o_I as a value
template <int I>
__device__ __forceinline__ f4 kw_get() {
    float x0, x1, x2, x3;
    asm volatile("v_accvgpr_read_b32 %0, a%c4\n\tv_accvgpr_read_b32 %1, a%c5\n\t"
                 "v_accvgpr_read_b32 %2, a%c6\n\tv_accvgpr_read_b32 %3, a%c7"
                 : "=v"(x0), "=v"(x1), "=v"(x2), "=v"(x3) : "n"(4 * I), "n"(4 * I + 1), "n"(4 * I + 2), "n"(4 * I + 3));
    return f4{x0, x1, x2, x3};
}

}  // namespace

}  // namespace vcpp
