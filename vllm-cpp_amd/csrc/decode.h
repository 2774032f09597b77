// decode.h -- internal launch interface of the decode kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "prefill.h"
#include "vcpp_attention.h"

namespace vcpp {

// Everything a decode launch needs, passed to the kernels by value.
struct DecodeParams {
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
    // queries / outputs
    const float* q;
    float* out;
    int32_t num_heads;
    int32_t num_seqs;
    int32_t group;    // num_heads / num_kv_heads
    int32_t qchunks;  // ceil(group / 8)
    int32_t pairs;    // num_kv_heads * qchunks (waves per (partition, seq))
    // tables
    const int32_t* block_tables;
    const int32_t* table_lens;
    const int32_t* context_lens;
    int32_t max_blocks;
    // fp16/int8: balanced split of the concatenated 16-token tiles over
    // num_wg workgroup ranges (per kv-head group)
    int32_t num_wg;
    // Cost of starting a sequence in a range, in tiles: the split divides
    // T + switch_tiles * (non-empty sequences) evenly, each sequence's tiles
    // preceded by switch_tiles units that hold no tile (0: plain tile split).
    int32_t switch_tiles;
    int32_t ctx_cap;       // context lengths are clamped to this
    // fp32: fixed partitions of `partition` tokens, max_parts per sequence
    int32_t partition;
    int32_t max_parts;
    // partials: fp16/int8 blocks [num_wg][2 slots][pairs] of [8 heads][head_dim] outputs and
    // 16 (m, l) pairs; fp32 [num_seqs][max_parts][num_heads]
    float* ws_o;     // (.., head_dim) unnormalised outputs
    float2* ws_ml;   // (max in log2 units, sum of exponentials)
    float scale_log2;  // log2(e) / sqrt(head_dim)
    int32_t pipeline;  // fp16/int8 pipeline shape (tuning; 0 = default)
    int32_t page_mode; // fp16/int8, Hkv 8: 8-wave workgroups staging whole tiles in LDS
    int32_t page_grid; // workgroups that walk the num_wg ranges (page mode: a run each; else num_wg)
    // Balanced page split (one range per workgroup), g1 > 0: ranges of
    // alternating size, the even positions of the axis taking g1_share / 256
    // of each neighbouring pair; workgroup w < num_wg / 2 walks position 2 w,
    // the others position 2 (w - num_wg / 2) + 1 (g1 == 0: equal ranges,
    // workgroup w at position w).
    int32_t g1;
    int32_t g1_share;
#ifdef VCPP_GATHER_DUMP
    int32_t* gather_dump;    // checker builds: [rows][gather_stride][2] (block, slot)
    int64_t gather_stride;
#endif
};

// Fork / join of the decode's merge onto a second stream: after the decode
// kernel, `fork` is recorded on the launch stream and `side` waits for it;
// the merge runs on `side`, which records `join` after it.  The caller makes
// its stream wait for `join` before anything that reads the outputs.
// *forked (if given) is set once `side` waits on `fork`; from then on `join`
// is recorded on `side` even when the merge launch fails.
struct MergeFork {
    hipStream_t side;
    hipEvent_t fork, join;
};
hipError_t launch_decode(const DecodeParams& p, hipStream_t stream, const MergeFork* mf = nullptr,
                         bool* forked = nullptr);

// The fused mixed step: one launch of 3 workgroups per CU (cus a multiple of
// 8), two prefill workers and one decode worker on each CU, then the decode
// merge.  dp is planned for the fused split (mixed_decode_grid); pp as for
// launch_prefill.
hipError_t launch_mixed(const DecodeParams& dp, const PrefillParams& pp, int cus, hipStream_t stream);
// Decode workgroups per kv-head group of the fused step (0: the shape has no
// fused step).
int mixed_decode_grid(int kv_dtype, int num_kv_heads, int group, int head_dim, int block_size, int cus);
// Dynamic LDS bytes of the fused kernel (prefill tables of max_blocks entries).
size_t mixed_lds_bytes(int kv_dtype, int head_dim, int max_blocks);
// Workgroups along y of the fp16/int8 grid (kv-head groups of up to 4 waves).
int decode_group_count(int pairs);
bool decode_head_dim_supported(int kv_dtype, int head_dim);
// kv heads per workgroup of the page-staged kernel for a shape (0: the
// shape runs the register-path kernel).
int decode_page_heads(int kv_dtype, int num_kv_heads, int head_dim);
// Workgroups of the page-staged kernel resident per CU for a shape.
int decode_page_wg_per_cu(int kv_dtype, int num_kv_heads, int head_dim);
// Shapes the page-staged kernel (decode_page_kernel) handles.

bool decode_page_mode_supported(int kv_dtype, int num_kv_heads, int group, int head_dim,
                                int block_size);

}  // namespace vcpp
