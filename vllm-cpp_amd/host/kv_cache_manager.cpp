// kv_cache_manager.cpp -- BlockPool / KVCacheManager on device memory with the
// interface and book-keeping of the reference src/kv_cache_manager.cpp.
#include "vllm_cpp/kv_cache_manager.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <stdexcept>

#include "host_util.h"

using vcpp_host::check;

namespace {

// Bit-exact float view of one block layer slab (host copy of the raw bytes).
void decode_rows(const uint8_t* raw, const uint16_t* scales, float* out, int32_t kv_dim,
                 int32_t head_dim, KVDtype dtype) {
    const int32_t n = BLOCK_SIZE * kv_dim;
    switch (dtype) {
        case KVDtype::FP32:
            std::memcpy(out, raw, sizeof(float) * n);
            break;
        case KVDtype::FP16: {
            const uint16_t* h = reinterpret_cast<const uint16_t*>(raw);
            for (int32_t i = 0; i < n; ++i) out[i] = vcpp_host::f16_decode(h[i]);
            break;
        }
        case KVDtype::FP8_E4M3:
            for (int32_t i = 0; i < n; ++i) out[i] = vcpp_host::fp8_decode(raw[i]);
            break;
        case KVDtype::INT8: {
            const int8_t* q = reinterpret_cast<const int8_t*>(raw);
            const int32_t hkv = kv_dim / head_dim;
            for (int32_t t = 0; t < BLOCK_SIZE; ++t)
                for (int32_t h = 0; h < hkv; ++h) {
                    const float s = vcpp_host::f16_decode(scales[h * BLOCK_SIZE + t]);
                    for (int32_t d = 0; d < head_dim; ++d) {
                        const int32_t i = (t * hkv + h) * head_dim + d;
                        out[i] = (float)q[i] * s;
                    }
                }
            break;
        }
        default:
            throw std::invalid_argument("unsupported KV dtype");
    }
}

// Zero n bytes at p: 16-byte stores over the aligned middle, byte stores at
// the ends.  Pool pages are cleared with this kernel rather than with
// hipMemsetAsync, so a step that frees or resets blocks can be recorded in a
// HIP graph (a memset node recorded there has given wrong results on replays).
__global__ void zero_bytes_kernel(uint8_t* p, int64_t n) {
    const int64_t head = std::min<int64_t>(n, (16 - ((uintptr_t)p & 15)) & 15);
    const int64_t nv = (n - head) / 16;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    uint4* v = reinterpret_cast<uint4*>(p + head);
    for (int64_t i = t; i < nv; i += stride) v[i] = make_uint4(0, 0, 0, 0);
    const int64_t tail0 = head + nv * 16;
    if (t < head) p[t] = 0;
    if (t < n - tail0) p[tail0 + t] = 0;
}

void zero_bytes(void* p, size_t n, hipStream_t s, const char* what) {
    if (n == 0) return;
    const int64_t nv = (int64_t)(n / 16) + 1;
    const unsigned blocks = (unsigned)std::min<int64_t>((nv + 255) / 256, 4096);
    hipLaunchKernelGGL(zero_bytes_kernel, dim3(blocks), dim3(256), 0, s, static_cast<uint8_t*>(p), (int64_t)n);
    check(hipGetLastError(), what);
}

}  // namespace

// ---- BlockPool --------------------------------------------------------------

BlockPool::BlockPool(int32_t num_blocks, int32_t num_layers, int32_t kv_dim, KVDtype kv_dtype,
                     int32_t head_dim)
    : kv_dim_(kv_dim), num_layers_(num_layers), kv_dtype_(kv_dtype),
      head_dim_(head_dim > 0 ? head_dim : kv_dim), staging_(new PoolStaging()) {
    if (num_blocks < 0 || num_layers <= 0 || kv_dim <= 0 || kv_dim % head_dim_ != 0)
        throw std::invalid_argument("BlockPool: bad shape");
    if (kv_dtype == KVDtype::INT8 && head_dim <= 0)
        throw std::invalid_argument("BlockPool: INT8 pools need head_dim");
    layer_bytes_ = (int64_t)BLOCK_SIZE * kv_dim * kv_elem_size(kv_dtype);
    block_bytes_ = (int64_t)num_layers * layer_bytes_;
    scale_layer_ = (int64_t)(kv_dim / head_dim_) * BLOCK_SIZE;
    blocks_.resize(num_blocks);
    for (int32_t i = 0; i < num_blocks; ++i) {
        blocks_[i].block_id = i;
        blocks_[i].dtype = kv_dtype;
    }
    const size_t bytes = (size_t)block_bytes_ * (size_t)std::max(num_blocks, 1);
    check(hipMalloc(&k_, bytes), "BlockPool K pages");
    check(hipMalloc(&v_, bytes), "BlockPool V pages");
    check(hipMemset(k_, 0, bytes), "BlockPool zero K");
    check(hipMemset(v_, 0, bytes), "BlockPool zero V");
    if (kv_dtype == KVDtype::INT8) {
        const size_t sb = sizeof(uint16_t) * scale_layer_ * num_layers * std::max(num_blocks, 1);
        check(hipMalloc(&k_scale_, sb), "BlockPool K scales");
        check(hipMalloc(&v_scale_, sb), "BlockPool V scales");
        check(hipMemset(k_scale_, 0, sb), "BlockPool zero K scales");
        check(hipMemset(v_scale_, 0, sb), "BlockPool zero V scales");
    }
    k_convert_buf_.resize((size_t)BLOCK_SIZE * kv_dim);
    v_convert_buf_.resize((size_t)BLOCK_SIZE * kv_dim);
}

BlockPool::~BlockPool() {
    (void)hipStreamSynchronize(static_cast<hipStream_t>(stream_));
    staging_.reset();
    for (void* p : {(void*)k_, (void*)v_, (void*)k_scale_, (void*)v_scale_})
        if (p) (void)hipFree(p);
}

void BlockPool::set_stream(void* stream) {
    if (stream != stream_) check(hipStreamSynchronize(static_cast<hipStream_t>(stream_)), "set_stream");
    stream_ = stream;
}

int32_t BlockPool::alloc() {
    std::lock_guard<std::mutex> lock(mtx_);
    for (int32_t i = 0; i < (int32_t)blocks_.size(); ++i) {
        if (blocks_[i].free) {
            blocks_[i].free = false;
            blocks_[i].ref_count = 1;
            return i;
        }
    }
    return -1;
}

void BlockPool::zero_block(int32_t id) {
    hipStream_t s = static_cast<hipStream_t>(stream_);
    zero_bytes(k_ + (int64_t)id * block_bytes_, block_bytes_, s, "zero block K");
    zero_bytes(v_ + (int64_t)id * block_bytes_, block_bytes_, s, "zero block V");
    if (k_scale_) {
        const size_t n = sizeof(uint16_t) * scale_layer_ * num_layers_;
        zero_bytes(k_scale_ + (int64_t)id * scale_layer_ * num_layers_, n, s, "zero scales");
        zero_bytes(v_scale_ + (int64_t)id * scale_layer_ * num_layers_, n, s, "zero scales");
    }
}

void BlockPool::free(int32_t block_id) {
    std::lock_guard<std::mutex> lock(mtx_);
    if (block_id < 0 || (size_t)block_id >= blocks_.size()) return;
    KVsBlock& b = blocks_[block_id];
    b.ref_count--;
    if (b.ref_count <= 0) {
        b.ref_count = 0;
        b.free = true;
        zero_block(block_id);  // the reference clears a freed block's data
    }
}

void BlockPool::ref(int32_t block_id) {
    std::lock_guard<std::mutex> lock(mtx_);
    if (block_id < 0 || (size_t)block_id >= blocks_.size()) return;
    blocks_[block_id].ref_count++;
}

void BlockPool::deref(int32_t block_id) {
    std::lock_guard<std::mutex> lock(mtx_);
    if (block_id < 0 || (size_t)block_id >= blocks_.size()) return;
    KVsBlock& b = blocks_[block_id];
    b.ref_count--;
    if (b.ref_count <= 0) {
        b.ref_count = 0;
        b.free = true;
    }
}

uint8_t* BlockPool::get_k_raw(int32_t block_id, int32_t layer) {
    if (block_id < 0 || (size_t)block_id >= blocks_.size() || layer < 0 || layer >= num_layers_)
        return nullptr;
    return k_ + (int64_t)block_id * block_bytes_ + (int64_t)layer * layer_bytes_;
}

uint8_t* BlockPool::get_v_raw(int32_t block_id, int32_t layer) {
    if (block_id < 0 || (size_t)block_id >= blocks_.size() || layer < 0 || layer >= num_layers_)
        return nullptr;
    return v_ + (int64_t)block_id * block_bytes_ + (int64_t)layer * layer_bytes_;
}

const uint8_t* BlockPool::get_k_raw(int32_t block_id, int32_t layer) const {
    return const_cast<BlockPool*>(this)->get_k_raw(block_id, layer);
}

const uint8_t* BlockPool::get_v_raw(int32_t block_id, int32_t layer) const {
    return const_cast<BlockPool*>(this)->get_v_raw(block_id, layer);
}

uint16_t* BlockPool::get_k_scale_raw(int32_t block_id, int32_t layer) const {
    if (!k_scale_ || block_id < 0 || (size_t)block_id >= blocks_.size() || layer < 0 ||
        layer >= num_layers_)
        return nullptr;
    return k_scale_ + ((int64_t)block_id * num_layers_ + layer) * scale_layer_;
}

uint16_t* BlockPool::get_v_scale_raw(int32_t block_id, int32_t layer) const {
    if (!v_scale_ || block_id < 0 || (size_t)block_id >= blocks_.size() || layer < 0 ||
        layer >= num_layers_)
        return nullptr;
    return v_scale_ + ((int64_t)block_id * num_layers_ + layer) * scale_layer_;
}

float* BlockPool::get_k(int32_t block_id, int32_t layer) {
    const uint8_t* raw = get_k_raw(block_id, layer);
    if (!raw) return nullptr;
    std::vector<uint8_t> host((size_t)layer_bytes_);
    std::vector<uint16_t> sc((size_t)scale_layer_);
    std::lock_guard<std::mutex> lock(mtx_);
    hipStream_t s = static_cast<hipStream_t>(stream_);
    check(hipStreamSynchronize(s), "get_k sync");
    check(hipMemcpy(host.data(), raw, layer_bytes_, hipMemcpyDeviceToHost), "get_k copy");
    if (k_scale_)
        check(hipMemcpy(sc.data(), get_k_scale_raw(block_id, layer), sizeof(uint16_t) * scale_layer_,
                        hipMemcpyDeviceToHost), "get_k scales");
    decode_rows(host.data(), sc.data(), k_convert_buf_.data(), kv_dim_, head_dim_, kv_dtype_);
    return k_convert_buf_.data();
}

float* BlockPool::get_v(int32_t block_id, int32_t layer) {
    const uint8_t* raw = get_v_raw(block_id, layer);
    if (!raw) return nullptr;
    std::vector<uint8_t> host((size_t)layer_bytes_);
    std::vector<uint16_t> sc((size_t)scale_layer_);
    std::lock_guard<std::mutex> lock(mtx_);
    hipStream_t s = static_cast<hipStream_t>(stream_);
    check(hipStreamSynchronize(s), "get_v sync");
    check(hipMemcpy(host.data(), raw, layer_bytes_, hipMemcpyDeviceToHost), "get_v copy");
    if (v_scale_)
        check(hipMemcpy(sc.data(), get_v_scale_raw(block_id, layer), sizeof(uint16_t) * scale_layer_,
                        hipMemcpyDeviceToHost), "get_v scales");
    decode_rows(host.data(), sc.data(), v_convert_buf_.data(), kv_dim_, head_dim_, kv_dtype_);
    return v_convert_buf_.data();
}

const float* BlockPool::get_k(int32_t block_id, int32_t layer) const {
    return const_cast<BlockPool*>(this)->get_k(block_id, layer);
}

const float* BlockPool::get_v(int32_t block_id, int32_t layer) const {
    return const_cast<BlockPool*>(this)->get_v(block_id, layer);
}

void BlockPool::copy_to(int32_t dst, int32_t src) {
    std::lock_guard<std::mutex> lock(mtx_);
    if (dst < 0 || dst >= (int32_t)blocks_.size()) return;
    if (src < 0 || src >= (int32_t)blocks_.size()) return;
    hipStream_t s = static_cast<hipStream_t>(stream_);
    check(hipMemcpyAsync(k_ + (int64_t)dst * block_bytes_, k_ + (int64_t)src * block_bytes_,
                         block_bytes_, hipMemcpyDeviceToDevice, s), "copy_to K");
    check(hipMemcpyAsync(v_ + (int64_t)dst * block_bytes_, v_ + (int64_t)src * block_bytes_,
                         block_bytes_, hipMemcpyDeviceToDevice, s), "copy_to V");
    if (k_scale_) {
        const int64_t n = scale_layer_ * num_layers_;
        check(hipMemcpyAsync(k_scale_ + dst * n, k_scale_ + src * n, sizeof(uint16_t) * n,
                             hipMemcpyDeviceToDevice, s), "copy_to K scales");
        check(hipMemcpyAsync(v_scale_ + dst * n, v_scale_ + src * n, sizeof(uint16_t) * n,
                             hipMemcpyDeviceToDevice, s), "copy_to V scales");
    }
}

int32_t BlockPool::free_count() const {
    int32_t c = 0;
    for (const auto& b : blocks_) c += b.free ? 1 : 0;
    return c;
}

int32_t BlockPool::used_count() const { return (int32_t)blocks_.size() - free_count(); }

void BlockPool::reset() {
    std::lock_guard<std::mutex> lock(mtx_);
    for (auto& b : blocks_) {
        b.ref_count = 0;
        b.free = true;
    }
    hipStream_t s = static_cast<hipStream_t>(stream_);
    const size_t nb = std::max<size_t>(blocks_.size(), 1);
    zero_bytes(k_, (size_t)block_bytes_ * nb, s, "reset K");
    zero_bytes(v_, (size_t)block_bytes_ * nb, s, "reset V");
    if (k_scale_) {
        const size_t n = sizeof(uint16_t) * scale_layer_ * num_layers_ * nb;
        zero_bytes(k_scale_, n, s, "reset K scales");
        zero_bytes(v_scale_, n, s, "reset V scales");
    }
}

KVsBlock& BlockPool::get_block(int32_t block_id) { return blocks_[block_id]; }

const KVsBlock& BlockPool::get_block(int32_t block_id) const { return blocks_[block_id]; }

vcpp_kv_pages BlockPool::pages(int32_t layer) const {
    vcpp_kv_pages p{};
    switch (kv_dtype_) {
        case KVDtype::FP32: p.dtype = VCPP_KV_F32; break;
        case KVDtype::FP16: p.dtype = VCPP_KV_F16; break;
        case KVDtype::FP8_E4M3: p.dtype = VCPP_KV_FP8; break;
        default: p.dtype = VCPP_KV_I8; break;
    }
    p.block_size = BLOCK_SIZE;
    p.num_kv_heads = kv_dim_ / head_dim_;
    p.head_dim = head_dim_;
    p.num_blocks = (int64_t)blocks_.size();
    p.block_stride = block_bytes_ / kv_elem_size(kv_dtype_);
    p.scale_block_stride = scale_layer_ * num_layers_;
    p.k = k_ + (int64_t)layer * layer_bytes_;
    p.v = v_ + (int64_t)layer * layer_bytes_;
    p.k_scale = k_scale_ ? k_scale_ + (int64_t)layer * scale_layer_ : nullptr;
    p.v_scale = v_scale_ ? v_scale_ + (int64_t)layer * scale_layer_ : nullptr;
    return p;
}

size_t BlockPool::block_host_bytes() const {
    size_t n = 2 * (size_t)block_bytes_;
    if (k_scale_) n += 2 * sizeof(uint16_t) * (size_t)(scale_layer_ * num_layers_);
    return n;
}

void BlockPool::copy_out(int32_t block_id, void* host) const {
    if (block_id < 0 || block_id >= (int32_t)blocks_.size()) return;
    hipStream_t s = static_cast<hipStream_t>(stream_);
    uint8_t* h = static_cast<uint8_t*>(host);
    check(hipMemcpyAsync(h, k_ + (int64_t)block_id * block_bytes_, block_bytes_, hipMemcpyDeviceToHost, s),
          "copy_out K");
    check(hipMemcpyAsync(h + block_bytes_, v_ + (int64_t)block_id * block_bytes_, block_bytes_,
                         hipMemcpyDeviceToHost, s), "copy_out V");
    if (k_scale_) {
        const int64_t n = scale_layer_ * num_layers_;
        uint8_t* hs = h + 2 * block_bytes_;
        check(hipMemcpyAsync(hs, k_scale_ + block_id * n, sizeof(uint16_t) * n, hipMemcpyDeviceToHost, s),
              "copy_out K scales");
        check(hipMemcpyAsync(hs + sizeof(uint16_t) * n, v_scale_ + block_id * n, sizeof(uint16_t) * n,
                             hipMemcpyDeviceToHost, s), "copy_out V scales");
    }
}

void BlockPool::copy_in(int32_t block_id, const void* host) {
    if (block_id < 0 || block_id >= (int32_t)blocks_.size()) return;
    hipStream_t s = static_cast<hipStream_t>(stream_);
    const uint8_t* h = static_cast<const uint8_t*>(host);
    check(hipMemcpyAsync(k_ + (int64_t)block_id * block_bytes_, h, block_bytes_, hipMemcpyHostToDevice, s),
          "copy_in K");
    check(hipMemcpyAsync(v_ + (int64_t)block_id * block_bytes_, h + block_bytes_, block_bytes_,
                         hipMemcpyHostToDevice, s), "copy_in V");
    if (k_scale_) {
        const int64_t n = scale_layer_ * num_layers_;
        const uint8_t* hs = h + 2 * block_bytes_;
        check(hipMemcpyAsync(k_scale_ + block_id * n, hs, sizeof(uint16_t) * n, hipMemcpyHostToDevice, s),
              "copy_in K scales");
        check(hipMemcpyAsync(v_scale_ + block_id * n, hs + sizeof(uint16_t) * n, sizeof(uint16_t) * n,
                             hipMemcpyHostToDevice, s), "copy_in V scales");
    }
}

// ---- KVSwap / KVCacheManager -------------------------------------------------

KVSwap::~KVSwap() {
    if (host_) {
        (void)hipStreamSynchronize(static_cast<hipStream_t>(stream_));
        (void)hipHostFree(host_);
    }
}

std::unique_ptr<KVSwap> KVCacheManager::swap_out(const std::vector<int32_t>& blocks) {
    std::unique_ptr<KVSwap> sw(new KVSwap());
    sw->block_bytes_ = pool_.block_host_bytes();
    sw->num_blocks_ = (int32_t)blocks.size();
    sw->stream_ = pool_.stream();
    if (!blocks.empty())
        check(hipHostMalloc(&sw->host_, sw->block_bytes_ * blocks.size(), hipHostMallocDefault),
              "swap_out host memory");
    for (size_t i = 0; i < blocks.size(); ++i)
        pool_.copy_out(blocks[i], static_cast<uint8_t*>(sw->host_) + i * sw->block_bytes_);
    return sw;
}

bool KVCacheManager::swap_in(const KVSwap& swap, const std::vector<int32_t>& blocks) {
    if ((int32_t)blocks.size() != swap.num_blocks_ || swap.block_bytes_ != pool_.block_host_bytes())
        return false;
    for (size_t i = 0; i < blocks.size(); ++i)
        pool_.copy_in(blocks[i], static_cast<const uint8_t*>(swap.host_) + i * swap.block_bytes_);
    return true;
}

// ---- KVCacheManager ---------------------------------------------------------

KVCacheManager::KVCacheManager(int32_t num_layers, int32_t kv_dim, int32_t num_blocks,
                               KVDtype kv_dtype, int32_t head_dim)
    : pool_(num_blocks, num_layers, kv_dim, kv_dtype, head_dim) {}

KVCacheManager::~KVCacheManager() {}

bool KVCacheManager::alloc_blocks(int32_t num_blocks, std::vector<int32_t>& out) {
    out.clear();
    out.reserve(num_blocks);
    for (int32_t i = 0; i < num_blocks; ++i) {
        const int32_t bid = pool_.alloc();
        if (bid < 0) return false;
        out.push_back(bid);
    }
    return true;
}

void KVCacheManager::free_blocks(const std::vector<int32_t>& blocks_to_free) {
    for (int32_t bid : blocks_to_free) pool_.free(bid);
}

void KVCacheManager::copy_blocks(const std::vector<int32_t>& src, const std::vector<int32_t>& dst) {
    for (size_t i = 0; i < src.size() && i < dst.size(); ++i) pool_.copy_to(dst[i], src[i]);
}

void write_kv_rows(KVCacheManager& m, int32_t layer, const std::vector<int64_t>& slots,
                   const float* k_data, const float* v_data);  // paged_attention.cpp

void KVCacheManager::write_kv(int32_t block_id, int32_t layer, int32_t pos_in_block,
                              const float* k_data, const float* v_data, int32_t kv_dim) {
    if (pos_in_block < 0 || pos_in_block >= BLOCK_SIZE) return;
    if (!pool_.get_k_raw(block_id, layer) || kv_dim != pool_.kv_dim()) return;
    write_kv_rows(*this, layer, {(int64_t)block_id * BLOCK_SIZE + pos_in_block}, k_data, v_data);
}

void KVCacheManager::read_kv(int32_t block_id, int32_t layer, int32_t pos_in_block,
                             float* k_data, float* v_data, int32_t kv_dim) const {
    if (pos_in_block < 0 || pos_in_block >= BLOCK_SIZE) return;
    if (!pool_.get_k_raw(block_id, layer) || kv_dim != pool_.kv_dim()) return;
    const float* k = pool_.get_k(block_id, layer);
    std::memcpy(k_data, k + (int64_t)pos_in_block * kv_dim, sizeof(float) * kv_dim);
    const float* v = pool_.get_v(block_id, layer);
    std::memcpy(v_data, v + (int64_t)pos_in_block * kv_dim, sizeof(float) * kv_dim);
}

int32_t KVCacheManager::free_blocks_count() const { return pool_.free_count(); }

int32_t KVCacheManager::used_blocks_count() const { return pool_.used_count(); }
