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

// Host outputs [seq_len][kv_dim] floats (positions past the table are left as
// is): one device gather of the rows and one copy to the host.
void read_kv_prefill(const BlockPool& kv_manager, const std::vector<int32_t>& block_table,
                     int32_t seq_len, int32_t layer, int32_t num_kv_heads, int32_t head_dim,
                     float* k_out, float* v_out);

// Causal attention of num_tokens new tokens of one sequence appended to
// prefix_len tokens already in its blocks: row i of q ([num_tokens][num_heads
// * head_dim] fp32, host or device) attends positions 0 .. prefix_len + i
// through block_table, into row i of out.  The chunk's K/V must be in the
// pool already (write_kv_prefill).  This is the engine's prefill loop of
// read_kv_prefill + compute_attention per position
// (src/paged_engine.cpp:381-384, src/paged_attention.cpp:174-201) as one
// launch: q is rounded to fp16 for the MFMA kernel (vcpp_paged_prefill_split,
// which splits each query tile's keys over several workgroups when few
// chunks sit on long prefixes) on FP16 / FP8 / INT8 pools; FP32 pools run
// every row as an fp32 decode query.
void paged_prefill(const float* q, const std::vector<int32_t>& block_table, int32_t prefix_len,
                   int32_t num_tokens, const BlockPool& kv_manager, int32_t num_heads,
                   int32_t num_kv_heads, int32_t head_dim, int32_t layer, float* out);

// Several sequences' chunks in one launch (a ScheduleOutput's prefills,
// src/scheduler.h:14-23).  Chunks without a table or tokens are skipped.
struct PrefillChunk {
    const float* q;                          // [num_tokens][num_heads * head_dim]
    const std::vector<int32_t>* block_table;
    int32_t prefix_len;
    int32_t num_tokens;
    float* out;                              // [num_tokens][num_heads * head_dim]
};
void paged_prefill_batch(const std::vector<PrefillChunk>& chunks, const BlockPool& kv_manager,
                         int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, int32_t layer);

// One engine step's attention for one layer: the decoding requests (as
// paged_attention_batch) and the prefill chunks (as paged_prefill_batch) of a
// ScheduleOutput (src/scheduler.h:14-23), served together as the engine's
// step serves them (src/paged_engine.cpp:254-269), through one
// vcpp_paged_mixed_step call: the decode kernel, its merge beside the
// prefill kernel.  Same skip rules and results as the two calls; FP32 pools,
// and steps with only one kind of work, run as those calls.
void paged_attention_step(const std::vector<const float*>& q_ptrs,
                          const std::vector<const std::vector<int32_t>*>& block_tables,
                          const std::vector<int32_t>& seq_lens, std::vector<float*> out_ptrs,
                          const std::vector<PrefillChunk>& chunks, const BlockPool& kv_manager,
                          int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, int32_t layer);
