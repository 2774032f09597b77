// noalloc.cpp -- vcpp_paged_decode_noalloc: the batched decode with its
// split-K partials in a static device array instead of a caller workspace, for
// callers that cannot allocate (graph capture, serving loops).  No counterpart
// in the reference.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <mutex>

#include "vcpp_attention.h"

namespace vcpp {
int record_error(int code, const char* msg);  // api.cpp
}

namespace {

// Decode partials of vcpp_paged_decode_noalloc.  Every GPU the library runs on
// holds its own copy until the process ends.  They need no initial value:
// each call writes every partial that its merge reads.
static __device__ __align__(256) char scratch[VCPP_NOALLOC_SCRATCH_BYTES];

int hip_error(hipError_t e, const char* what) {
    char buf[256];
    snprintf(buf, sizeof(buf), "vcpp_paged_decode_noalloc: %s: %s", what, hipGetErrorString(e));
    return vcpp::record_error(VCPP_E_HIP, buf);
}

// Device address of `scratch` on the current device, looked up once per
// device.  In host code the array's name is a host-side stand-in, never a
// device address: only this pointer is passed to kernels.
int scratch_ptr(void** out) {
    static std::mutex mu;
    static void* ptr[64] = {};
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_error(e, "hipGetDevice");
    if (dev < 0 || dev >= 64) return vcpp::record_error(VCPP_E_UNSUPPORTED, "device index out of range");
    std::lock_guard<std::mutex> lock(mu);
    if (!ptr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return hip_error(e, "hipGetSymbolAddress(scratch)");
        if (!p) return vcpp::record_error(VCPP_E_HIP, "vcpp_paged_decode_noalloc: scratch has no address");
        ptr[dev] = p;
    }
    *out = ptr[dev];
    return VCPP_OK;
}

}  // namespace

extern "C" int vcpp_paged_decode_noalloc(const vcpp_kv_pages* kv, const float* q, float* out,
                                         const int32_t* block_tables, int32_t max_blocks_per_seq,
                                         const int32_t* table_lens, const int32_t* context_lens,
                                         int32_t num_seqs, int32_t max_context_len,
                                         int32_t num_heads, int32_t partition_size, void* stream) {
    const size_t need =
        vcpp_decode_workspace_size(kv, num_seqs, num_heads, max_context_len, partition_size);
    if (need > (size_t)VCPP_NOALLOC_SCRATCH_BYTES) {
        char buf[256];
        snprintf(buf, sizeof(buf),
                 "vcpp_paged_decode_noalloc: this call needs %zu bytes of split-K scratch, more than "
                 "the static %zu (call vcpp_paged_decode with a workspace)",
                 need, (size_t)VCPP_NOALLOC_SCRATCH_BYTES);
        return vcpp::record_error(VCPP_E_UNSUPPORTED, buf);
    }
    void* ws = nullptr;
    if (need > 0) {
        const int rc = scratch_ptr(&ws);
        if (rc != VCPP_OK) return rc;
    }
    // Argument checks, planning and the launches are vcpp_paged_decode's.
    return vcpp_paged_decode(kv, q, out, block_tables, max_blocks_per_seq, table_lens,
                             context_lens, num_seqs, max_context_len, num_heads, partition_size,
                             ws, need > 0 ? (size_t)VCPP_NOALLOC_SCRATCH_BYTES : 0, stream);
}
