// prefill.h -- internal launch interface of the chunked prefill kernel.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "vcpp_attention.h"

namespace vcpp {

struct PrefillParams {
    // KV pages (see vcpp_kv_pages)
    const void* k;
    const void* v;
    const uint16_t* k_scale;
    const uint16_t* v_scale;
    int64_t num_blocks;
    int64_t block_stride;
    int64_t scale_block_stride;
    int32_t block_size;
    int32_t num_kv_heads;
    int32_t head_dim;
    int32_t kv_dtype;
    // queries (fp16 [rows][num_heads][head_dim]) and fp32 outputs
    const uint16_t* q;
    float* out;
    int32_t num_heads;
    int32_t group;        // num_heads / num_kv_heads
    int32_t head_groups;  // workgroups per kv head (4 query heads each)
    // chunks
    const int32_t* block_tables;  // [num_chunks][max_blocks]
    const int32_t* q_start;       // [num_chunks + 1] device
    const int32_t* prefix_lens;   // [num_chunks] device
    int32_t max_blocks;
    int32_t num_chunks;
    int32_t max_chunk_len;
    float scale_log2;  // log2(e) / sqrt(head_dim)
    // split-K over the keys (1: none): part k of a tile's key blocks leaves
    // unnormalised outputs and (max, sum) in ws_o / ws_ml at row
    // k * rows_cap + row, for launch_prefill's merge
    int32_t splits;
    int32_t rows_cap;  // >= the rows of all chunks (num_chunks * max_chunk_len)
    float* ws_o;       // [splits][rows_cap][num_heads][head_dim]
    float2* ws_ml;     // [splits][rows_cap][num_heads] (max in log2 units, sum)
    uint64_t bs_magic; // ceil(2^40 / block_size): pos / block_size = (pos * bs_magic) >> 40
    int32_t xcd_cus;   // CUs per XCD (0: unknown; no pairing of heavy and light tiles)
    int32_t tile_rows; // query rows per workgroup tile (set by launch_prefill for the merge)
#ifdef VCPP_GATHER_DUMP
    int32_t* gather_dump;    // checker builds: [rows][gather_stride][2] (block, slot)
    int64_t gather_stride;
#endif
};

hipError_t launch_prefill(const PrefillParams& p, hipStream_t stream);
// Workspace bytes of a split prefill (0 when splits <= 1).
// Most key parts a split prefill cuts a query tile into.
constexpr int kMaxPrefillSplits = 16;
size_t prefill_split_bytes(int splits, int rows_cap, int num_heads, int head_dim);
int prefill_head_groups(int group);
// Whether fp16 pages of this shape run prefill_wide_kernel (128-row tiles)
// rather than prefill_dma_kernel, and the query rows per workgroup tile of
// the kernel that serves them.
bool prefill_uses_wide(int kv_dtype, int head_dim, int block_size);
int prefill_tile_rows(int kv_dtype, int head_dim, int block_size);
size_t prefill_ring_bytes(int kv_dtype, int head_dim);
// Dynamic LDS bytes of the prefill kernel for a table of max_blocks entries
// (the larger of the two kernels' needs where both serve the dtype).
size_t prefill_lds_bytes(int kv_dtype, int head_dim, int max_blocks);

}  // namespace vcpp
