// ref_engine_harness.cpp -- C entry points around the reference engine's own
// inline math helpers, which are file-static in src/paged_engine.cpp.
//
// TEST INFRASTRUCTURE ONLY.  This translation unit includes
// src/paged_engine.cpp where it lies (oracle/Makefile links it with the other
// reference sources that file needs) into oracle/_ref/libref_engine.so, so the
// tests can pin the oracle's RoPE and per-head RMS norm against the real
// rope_single (src/paged_engine.cpp:47-62) and rms_norm (:14-20).
#include "paged_engine.cpp"

extern "C" {

// rope_single on one position: x [dim] = dim / head_dim heads, rotated in place.
void ref_rope_single(float* x, int32_t dim, int32_t head_dim, int32_t pos, const float* inv_freq,
                     int32_t inv_freq_size) {
    rope_single(x, dim, head_dim, pos, inv_freq, inv_freq_size);
}

// rms_norm of one row: out [dim] = weight * in / sqrt(mean(in^2) + eps).
void ref_rms_norm(const float* in, const float* weight, float* out, int32_t dim, float eps) {
    rms_norm(in, weight, out, dim, eps);
}

}  // extern "C"
