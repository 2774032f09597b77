// paged_attention.h -- the reference's src/paged_attention.h:30-88 entry
// points over the device-resident BlockPool and the gfx950 kernels.
//
// Pointers to q / out / k_data / v_data may be host or device memory (the
// reference engine passes host buffers).  With host memory the call returns
// after the result is in host memory, as the reference's does; with device
// memory it is queued on the pool's stream.  Semantics are those of
// src/paged_attention.cpp: positions whose block index is at or past
// block_table.size() or whose block id is outside the pool are skipped; the
// pool's kv_dim must equal num_kv_heads * head_dim.
#pragma once

#include <cstdint>
#include <vector>

#include "kv_cache_manager.h"

void paged_attention(const float* q, const std::vector<int32_t>& block_table, int32_t seq_len,
                     const BlockPool& kv_manager, int32_t num_heads, int32_t num_kv_heads,
                     int32_t head_dim, int32_t layer, float* out);

// One launch over all requests with a table (null tables are skipped, as in
// src/paged_attention.cpp:96-121).
void paged_attention_batch(const std::vector<const float*>& q_ptrs,
                           const std::vector<const std::vector<int32_t>*>& block_tables,
                           const std::vector<int32_t>& seq_lens, const BlockPool& kv_manager,
                           int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                           int32_t layer, std::vector<float*> out_ptrs);

void write_kv_token(KVCacheManager& kv_manager, const std::vector<int32_t>& block_table,
                    int32_t seq_len, int32_t layer, const float* k_data, const float* v_data);

// All seq_len positions in one launch.
void write_kv_prefill(KVCacheManager& kv_manager, const std::vector<int32_t>& block_table,
                      int32_t seq_len, int32_t layer, const float* k_data, const float* v_data);

// Host outputs [seq_len][kv_dim] floats (positions past the table are left as is).
void read_kv_prefill(const BlockPool& kv_manager, const std::vector<int32_t>& block_table,
                     int32_t seq_len, int32_t layer, int32_t num_kv_heads, int32_t head_dim,
                     float* k_out, float* v_out);
