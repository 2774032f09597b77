// profile.cpp -- HIP-event timing of each kernel launch, on the launch stream.
//
// Enabled by vcpp_profile_enable(1); every launch of a kernel then records a
// start and a stop event on its own stream, so the measured span is that
// kernel alone.  vcpp_profile_read() waits for the events and sums them.
#include "profile.h"

#include <atomic>
#include <mutex>
#include <vector>

#include "vcpp_attention.h"

namespace vcpp {
namespace {

struct Span {
    hipEvent_t start, stop;
};

struct Profiler {
    std::mutex mu;
    std::atomic<bool> on{false};
    std::vector<Span> spans[kKernelCount];
    hipEvent_t pending[kKernelCount] = {};
    std::vector<hipEvent_t> free_events;

    hipEvent_t get() {
        if (!free_events.empty()) {
            hipEvent_t e = free_events.back();
            free_events.pop_back();
            return e;
        }
        hipEvent_t e = nullptr;
        if (hipEventCreate(&e) != hipSuccess) return nullptr;
        return e;
    }
    void reset() {
        for (auto& v : spans) {
            for (auto& s : v) {
                free_events.push_back(s.start);
                free_events.push_back(s.stop);
            }
            v.clear();
        }
        for (auto& p : pending) {
            if (p) free_events.push_back(p);
            p = nullptr;
        }
    }
};

Profiler& prof() {
    static Profiler p;
    return p;
}

}  // namespace

bool prof_enabled() { return prof().on.load(std::memory_order_relaxed); }

void prof_begin(KernelId id, hipStream_t stream) {
    Profiler& p = prof();
    std::lock_guard<std::mutex> lock(p.mu);
    hipEvent_t e = p.get();
    if (!e) return;
    if (hipEventRecord(e, stream) != hipSuccess) {
        p.free_events.push_back(e);
        return;
    }
    if (p.pending[id]) p.free_events.push_back(p.pending[id]);
    p.pending[id] = e;
}

void prof_end(KernelId id, hipStream_t stream) {
    Profiler& p = prof();
    std::lock_guard<std::mutex> lock(p.mu);
    if (!p.pending[id]) return;
    hipEvent_t e = p.get();
    if (!e) return;
    if (hipEventRecord(e, stream) != hipSuccess) {
        p.free_events.push_back(e);
        return;
    }
    p.spans[id].push_back(Span{p.pending[id], e});
    p.pending[id] = nullptr;
}

}  // namespace vcpp

extern "C" {

int vcpp_profile_enable(int on) {
    vcpp::Profiler& p = vcpp::prof();
    std::lock_guard<std::mutex> lock(p.mu);
    p.reset();
    p.on.store(on != 0);
    return VCPP_OK;
}

int vcpp_profile_read(int kernel_id, double* total_ms, int64_t* launches) {
    if (kernel_id < 0 || kernel_id >= vcpp::kKernelCount || !total_ms || !launches)
        return VCPP_E_INVALID;
    vcpp::Profiler& p = vcpp::prof();
    std::lock_guard<std::mutex> lock(p.mu);
    double total = 0.0;
    for (const auto& s : p.spans[kernel_id]) {
        if (hipEventSynchronize(s.stop) != hipSuccess) return VCPP_E_HIP;
        float ms = 0.f;
        if (hipEventElapsedTime(&ms, s.start, s.stop) != hipSuccess) return VCPP_E_HIP;
        total += ms;
    }
    *total_ms = total;
    *launches = (int64_t)p.spans[kernel_id].size();
    return VCPP_OK;
}

}  // extern "C"
