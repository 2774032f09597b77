// kv_cache_manager.h -- device-resident BlockPool / KVCacheManager with the
// interface of the reference src/kv_cache_manager.h:50-147.
//
// Same names, arguments and skip rules as the reference; what differs:
//   * block storage lives in HBM: one K and one V allocation laid out as the
//     reference's per-block vectors, [num_blocks][num_layers][BLOCK_SIZE][kv_dim]
//     (src/kv_cache_manager.cpp:12-34), so get_k_raw / get_v_raw return DEVICE
//     pointers at the reference's offsets;
//   * get_k / get_v return a host snapshot of the block's layer converted to
//     float (the reference returns a view that is writable for FP32 pools);
//   * INT8 pools (not in the reference) carry fp16 scale pages
//     [num_blocks][num_layers][num_kv_heads][BLOCK_SIZE]; they need head_dim;
//   * FP8_E4M3 pools hold the reference's E4M3 bytes (VCPP_KV_FP8 pages);
//     HIP failures throw std::runtime_error (the reference has no failure
//     mode there).
// Device work is queued on the pool's stream (default: the null stream).
#pragma once

#include <cstdint>
#include <memory>
#include <mutex>
#include <vector>

#include "kv_config.h"
#include "vcpp_attention.h"

struct PoolStaging;  // device staging of the paged_attention.h entry points

inline constexpr int32_t kv_elem_size(KVDtype dtype) {
    switch (dtype) {
        case KVDtype::FP32: return 4;
        case KVDtype::FP16: return 2;
        case KVDtype::FP8_E4M3: return 1;
        case KVDtype::INT8: return 1;
    }
    return 4;
}

// Book-keeping of one physical block (src/kv_cache_manager.h:33-47); the data
// is in the pool's device allocations.
struct KVsBlock {
    int32_t block_id = -1;
    int32_t ref_count = 0;
    bool free = true;
    KVDtype dtype = KVDtype::FP32;
};

class BlockPool {
public:
    // head_dim: required for INT8 (scales are per kv head), else optional
    // (defaults to kv_dim, i.e. one kv head).
    BlockPool(int32_t num_blocks, int32_t num_layers, int32_t kv_dim,
              KVDtype kv_dtype = KVDtype::FP32, int32_t head_dim = 0);
    ~BlockPool();
    BlockPool(const BlockPool&) = delete;
    BlockPool& operator=(const BlockPool&) = delete;

    int32_t alloc();                 // first free block (ref_count 1), or -1
    void free(int32_t block_id);     // ref_count - 1; at 0 the block is freed and zeroed
    void ref(int32_t block_id);      // ref_count + 1
    void deref(int32_t block_id);    // ref_count - 1; at 0 freed (not zeroed)

    // Device pointers to the block's slab of `layer` (nullptr when out of range).
    uint8_t* get_k_raw(int32_t block_id, int32_t layer);
    uint8_t* get_v_raw(int32_t block_id, int32_t layer);
    const uint8_t* get_k_raw(int32_t block_id, int32_t layer) const;
    const uint8_t* get_v_raw(int32_t block_id, int32_t layer) const;
    // INT8 scale pages of the block's layer ([num_kv_heads][BLOCK_SIZE] fp16).
    uint16_t* get_k_scale_raw(int32_t block_id, int32_t layer) const;
    uint16_t* get_v_scale_raw(int32_t block_id, int32_t layer) const;

    // Host snapshot of the block's layer as float [BLOCK_SIZE][kv_dim]
    // (a buffer owned by the pool, overwritten by the next call).
    float* get_k(int32_t block_id, int32_t layer);
    float* get_v(int32_t block_id, int32_t layer);
    const float* get_k(int32_t block_id, int32_t layer) const;
    const float* get_v(int32_t block_id, int32_t layer) const;

    void copy_to(int32_t dst, int32_t src);  // all layers (and scales) of src -> dst

    // Bytes of one block's pages in host memory: K and V of every layer, then
    // the INT8 scales.  copy_out / copy_in move them between a block and host
    // memory on the pool's stream (asynchronous; the host buffer must be
    // pinned and live until the stream has passed the copy).
    size_t block_host_bytes() const;
    void copy_out(int32_t block_id, void* host) const;
    void copy_in(int32_t block_id, const void* host);

    int32_t free_count() const;
    int32_t used_count() const;
    void reset();  // every block free, all data zero

    KVsBlock& get_block(int32_t block_id);
    const KVsBlock& get_block(int32_t block_id) const;

    int32_t num_blocks() const { return (int32_t)blocks_.size(); }
    int32_t kv_dim() const { return kv_dim_; }
    int32_t num_layers() const { return num_layers_; }
    KVDtype kv_dtype() const { return kv_dtype_; }
    int32_t head_dim() const { return head_dim_; }
    int32_t num_kv_heads() const { return kv_dim_ / head_dim_; }

    // ---- device extensions (no reference counterpart) ----
    // Page descriptor of one layer for the vcpp_* kernels.
    vcpp_kv_pages pages(int32_t layer) const;
    // Work queued by later calls goes to `stream`; set_stream first waits
    // for the previous stream, which the pool's staging buffers may be in use on.
    void set_stream(void* stream);
    void* stream() const { return stream_; }
    PoolStaging& staging() const { return *staging_; }

private:
    void zero_block(int32_t block_id);

    std::vector<KVsBlock> blocks_;
    int32_t kv_dim_;
    int32_t num_layers_;
    KVDtype kv_dtype_;
    int32_t head_dim_;
    int64_t layer_bytes_;  // BLOCK_SIZE * kv_dim * elem_size
    int64_t block_bytes_;  // num_layers * layer_bytes_
    int64_t scale_layer_;  // fp16 elements of one block's layer of scales
    uint8_t* k_ = nullptr;
    uint8_t* v_ = nullptr;
    uint16_t* k_scale_ = nullptr;
    uint16_t* v_scale_ = nullptr;
    void* stream_ = nullptr;

    std::unique_ptr<PoolStaging> staging_;
    mutable std::vector<float> k_convert_buf_;
    mutable std::vector<float> v_convert_buf_;
    mutable std::mutex mtx_;
};

// Pages of some blocks kept in pinned host memory by KVCacheManager::swap_out.
class KVSwap {
public:
    ~KVSwap();  // waits for the stream that filled it, then frees the memory
    KVSwap(const KVSwap&) = delete;
    KVSwap& operator=(const KVSwap&) = delete;
    int32_t num_blocks() const { return num_blocks_; }

private:
    friend class KVCacheManager;
    KVSwap() = default;
    void* host_ = nullptr;
    size_t block_bytes_ = 0;
    int32_t num_blocks_ = 0;
    void* stream_ = nullptr;
};

class KVCacheManager {
public:
    KVCacheManager(int32_t num_layers, int32_t kv_dim, int32_t num_blocks,
                   KVDtype kv_dtype = KVDtype::FP32, int32_t head_dim = 0);
    ~KVCacheManager();

    bool alloc_blocks(int32_t num_blocks, std::vector<int32_t>& out);
    void free_blocks(const std::vector<int32_t>& blocks_to_free);
    void copy_blocks(const std::vector<int32_t>& src, const std::vector<int32_t>& dst);

    // Preemption that keeps the data (no counterpart in the reference, whose
    // Scheduler keeps only block ids across a preemption and restores by
    // copy_blocks from blocks it has already freed, i.e. zeroed:
    // src/scheduler.cpp:87-153).  swap_out copies the blocks' pages (every
    // layer, K, V and INT8 scales) to pinned host memory, queued on the pool's
    // stream ahead of the free that may follow; swap_in copies them into the
    // same number of (newly allocated) blocks.  Invalid ids are skipped;
    // swap_in returns false when the counts differ.
    std::unique_ptr<KVSwap> swap_out(const std::vector<int32_t>& blocks);
    bool swap_in(const KVSwap& swap, const std::vector<int32_t>& blocks);

    BlockPool& block_pool() { return pool_; }
    const BlockPool& block_pool() const { return pool_; }

    // One token's K/V row ([kv_dim] floats, host or device memory) into slot
    // pos_in_block of the block's layer, encoded for the pool's dtype
    // (vcpp_write_kv: the reference's truncating fp16 encoder for FP16).
    void write_kv(int32_t block_id, int32_t layer, int32_t pos_in_block,
                  const float* k_data, const float* v_data, int32_t kv_dim);
    // One token's K/V row as floats into host memory.
    void read_kv(int32_t block_id, int32_t layer, int32_t pos_in_block,
                 float* k_data, float* v_data, int32_t kv_dim) const;

    int32_t free_blocks_count() const;
    int32_t used_blocks_count() const;
    KVDtype kv_dtype() const { return pool_.kv_dtype(); }

private:
    BlockPool pool_;
};
