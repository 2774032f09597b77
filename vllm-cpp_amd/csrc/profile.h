// profile.h -- optional per-kernel HIP-event timing (vcpp_profile_* entry points).
#pragma once

#include <hip/hip_runtime.h>

namespace vcpp {

enum KernelId { kKernelDecode = 0, kKernelMerge = 1, kKernelPrefill = 2, kKernelMixed = 3, kKernelCount = 4 };

// True while vcpp_profile_enable(1) is in force.
bool prof_enabled();
// Record an event on `stream` before / after one launch of kernel `id`.
void prof_begin(KernelId id, hipStream_t stream);
void prof_end(KernelId id, hipStream_t stream);

}  // namespace vcpp
