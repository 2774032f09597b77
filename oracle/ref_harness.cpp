// ref_harness.cpp -- C entry points around the reference's own CPU path.
//
// TEST INFRASTRUCTURE ONLY.  Compiled together with the reference sources
// src/paged_attention.cpp, src/kv_cache_manager.cpp and src/quantization.cpp
// where they lie (oracle/Makefile), into oracle/_ref/libref.so.  It lets the
// tests pin the oracle against the real reference, the golden-vector script
// write fixtures, and bench.py time the reference as the CPU baseline.
#include "paged_attention.h"
#include "kv_cache_manager.h"
#include "quantization.h"

#include <cstdint>
#include <vector>

extern "C" {

// dtype: 0 = KVDtype::FP32, 1 = KVDtype::FP16, 2 = KVDtype::FP8_E4M3
// (src/config.h:69-73).
void* ref_pool_create(int32_t num_blocks, int32_t num_layers, int32_t kv_dim, int32_t dtype) {
    return new KVCacheManager(num_layers, kv_dim, num_blocks,
                              dtype == 1 ? KVDtype::FP16
                                         : dtype == 2 ? KVDtype::FP8_E4M3 : KVDtype::FP32);
}

// The reference FP8 E4M3 codec of the KV pool's conversions
// (src/kv_cache_manager.cpp:145-146,180-181 -> src/quantization.cpp:176-188).
void ref_fp8_encode_n(const float* x, uint8_t* b, int64_t n) { float_to_fp8_e4m3_batch(x, b, n); }
void ref_fp8_decode_n(const uint8_t* b, float* x, int64_t n) { fp8_e4m3_to_float_batch(b, x, n); }

void ref_pool_destroy(void* m) { delete static_cast<KVCacheManager*>(m); }

// Write float K/V [num_blocks][BLOCK_SIZE][kv_dim] of one layer through the
// reference's KVCacheManager::write_kv (which encodes to the pool dtype).
void ref_pool_write(void* mp, int32_t layer, const float* k, const float* v) {
    auto* m = static_cast<KVCacheManager*>(mp);
    const int32_t kv_dim = m->block_pool().kv_dim();
    const int32_t nb = m->block_pool().num_blocks();
    for (int32_t b = 0; b < nb; b++)
        for (int32_t t = 0; t < BLOCK_SIZE; t++) {
            int64_t off = ((int64_t)b * BLOCK_SIZE + t) * kv_dim;
            m->write_kv(b, layer, t, k + off, v + off, kv_dim);
        }
}

// Copy the raw bytes of one layer slab of every block (K then V).
void ref_pool_read_raw(void* mp, int32_t layer, uint8_t* k, uint8_t* v) {
    auto* m = static_cast<KVCacheManager*>(mp);
    const BlockPool& p = m->block_pool();
    int64_t esize = kv_elem_size(p.kv_dtype());
    int64_t slab = (int64_t)BLOCK_SIZE * p.kv_dim() * esize;
    for (int32_t b = 0; b < p.num_blocks(); b++) {
        const uint8_t* ks = p.get_k_raw(b, layer);
        const uint8_t* vs = p.get_v_raw(b, layer);
        for (int64_t i = 0; i < slab; i++) { k[b * slab + i] = ks[i]; v[b * slab + i] = vs[i]; }
    }
}

// Batched decode through paged_attention (src/paged_attention.cpp:11-90), one
// call per sequence; table row b has min(table_lens[b], stride) entries.
void ref_decode(void* mp, int32_t layer, const float* q, const int32_t* tables, int64_t stride,
                const int32_t* table_lens, const int32_t* ctx, int32_t batch,
                int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, float* out) {
    auto* m = static_cast<KVCacheManager*>(mp);
    for (int32_t b = 0; b < batch; b++) {
        int64_t len = stride;
        if (table_lens && table_lens[b] < len) len = table_lens[b];
        std::vector<int32_t> table(tables + b * stride, tables + b * stride + len);
        paged_attention(q + (int64_t)b * num_heads * head_dim, table, ctx[b], m->block_pool(),
                        num_heads, num_kv_heads, head_dim, layer,
                        out + (int64_t)b * num_heads * head_dim);
    }
}

// Chunked causal prefill with the engine's per-position semantics: row i of
// chunk c calls paged_attention with seq_len = prefix[c] + i + 1.
void ref_prefill(void* mp, int32_t layer, const float* q, const int32_t* tables, int64_t stride,
                 const int32_t* q_start, const int32_t* prefix, int32_t num_chunks,
                 int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, float* out) {
    auto* m = static_cast<KVCacheManager*>(mp);
    const int64_t row = (int64_t)num_heads * head_dim;
    for (int32_t c = 0; c < num_chunks; c++) {
        std::vector<int32_t> table(tables + c * stride, tables + (c + 1) * stride);
        for (int32_t r = q_start[c]; r < q_start[c + 1]; r++)
            paged_attention(q + r * row, table, prefix[c] + (r - q_start[c]) + 1, m->block_pool(),
                            num_heads, num_kv_heads, head_dim, layer, out + r * row);
    }
}

}  // extern "C"
