// paged_attention.cpp -- the reference's src/paged_attention.h entry points
// (src/paged_attention.cpp:11-201) over the device-resident BlockPool: each
// call packs its arguments into device buffers and runs vcpp_paged_decode /
// vcpp_write_kv on the pool's stream.
#include "vllm_cpp/paged_attention.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <mutex>
#include <vector>

#include "host_util.h"

using vcpp_host::check;
using vcpp_host::check_rc;
using vcpp_host::DevBuf;
using vcpp_host::is_device;

namespace {

// Device staging shared by the host entry points of this process (one device).
struct Staging {
    std::mutex mu;
    DevBuf q, out, tables, ctx, ws, k, v, slots;
};

Staging& staging() {
    static Staging s;
    return s;
}

// A layer's descriptor with the call's head split (the pool itself only knows
// kv_dim; INT8 pools fix head_dim).
bool attention_pages(const BlockPool& pool, int32_t layer, int32_t num_kv_heads, int32_t head_dim,
                     vcpp_kv_pages* out) {
    if (layer < 0 || layer >= pool.num_layers()) return false;
    if (num_kv_heads <= 0 || head_dim <= 0 || num_kv_heads * head_dim != pool.kv_dim()) return false;
    if (pool.kv_dtype() == KVDtype::INT8 && head_dim != pool.head_dim()) return false;
    *out = pool.pages(layer);
    out->num_kv_heads = num_kv_heads;
    out->head_dim = head_dim;
    return true;
}

}  // namespace

void paged_attention(const float* q, const std::vector<int32_t>& block_table, int32_t seq_len,
                     const BlockPool& kv_manager, int32_t num_heads, int32_t num_kv_heads,
                     int32_t head_dim, int32_t layer, float* out) {
    std::vector<const float*> qs{q};
    std::vector<const std::vector<int32_t>*> ts{&block_table};
    paged_attention_batch(qs, ts, {seq_len}, kv_manager, num_heads, num_kv_heads, head_dim, layer,
                          {out});
}

void paged_attention_batch(const std::vector<const float*>& q_ptrs,
                           const std::vector<const std::vector<int32_t>*>& block_tables,
                           const std::vector<int32_t>& seq_lens, const BlockPool& kv_manager,
                           int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                           int32_t layer, std::vector<float*> out_ptrs) {
    if (num_heads <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads != 0) return;
    vcpp_kv_pages pages;
    if (!attention_pages(kv_manager, layer, num_kv_heads, head_dim, &pages)) return;
    hipStream_t s = static_cast<hipStream_t>(kv_manager.stream());
    const size_t row = (size_t)num_heads * head_dim;

    // Requests with a table; the others are skipped as in the reference.
    std::vector<size_t> live;
    int32_t max_blocks = 1, max_ctx = 0;
    const size_t n = std::min({q_ptrs.size(), block_tables.size(), seq_lens.size(), out_ptrs.size()});
    for (size_t i = 0; i < n; ++i) {
        if (!block_tables[i]) continue;
        live.push_back(i);
        max_blocks = std::max<int32_t>(max_blocks, (int32_t)block_tables[i]->size());
        max_ctx = std::max(max_ctx, seq_lens[i]);
    }
    if (live.empty()) return;
    const int32_t B = (int32_t)live.size();

    std::vector<int32_t> tables((size_t)B * max_blocks, -1), tlens(B), ctx(B);
    for (int32_t b = 0; b < B; ++b) {
        const auto& t = *block_tables[live[b]];
        std::copy(t.begin(), t.end(), tables.begin() + (size_t)b * max_blocks);
        tlens[b] = (int32_t)t.size();
        ctx[b] = std::max(seq_lens[live[b]], 0);
    }

    Staging& st = staging();
    std::lock_guard<std::mutex> lock(st.mu);
    float* qd = static_cast<float*>(st.q.get(row * B * sizeof(float)));
    float* od = static_cast<float*>(st.out.get(row * B * sizeof(float)));
    int32_t* td = static_cast<int32_t*>(st.tables.get(tables.size() * sizeof(int32_t)));
    int32_t* cd = static_cast<int32_t*>(st.ctx.get(2 * B * sizeof(int32_t)));
    bool any_host = false;
    for (int32_t b = 0; b < B; ++b) {
        const float* src = q_ptrs[live[b]];
        const bool dev = is_device(src);
        any_host |= !dev;
        check(hipMemcpyAsync(qd + row * b, src, row * sizeof(float),
                             dev ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice, s), "q");
    }
    check(hipMemcpyAsync(td, tables.data(), tables.size() * sizeof(int32_t), hipMemcpyHostToDevice, s),
          "tables");
    check(hipMemcpyAsync(cd, ctx.data(), B * sizeof(int32_t), hipMemcpyHostToDevice, s), "context lens");
    check(hipMemcpyAsync(cd + B, tlens.data(), B * sizeof(int32_t), hipMemcpyHostToDevice, s),
          "table lens");
    const size_t wsb = vcpp_decode_workspace_size(&pages, B, num_heads, max_ctx, 0);
    void* ws = wsb ? st.ws.get(wsb) : nullptr;
    check_rc(vcpp_paged_decode(&pages, qd, od, td, max_blocks, cd + B, cd, B, max_ctx, num_heads, 0,
                               ws, wsb, s),
             "paged_attention");
    for (int32_t b = 0; b < B; ++b) {
        float* dst = out_ptrs[live[b]];
        const bool dev = is_device(dst);
        any_host |= !dev;
        check(hipMemcpyAsync(dst, od + row * b, row * sizeof(float),
                             dev ? hipMemcpyDeviceToDevice : hipMemcpyDeviceToHost, s), "out");
    }
    // Host inputs or outputs: return with the work done (the staging buffers
    // are reused by the next call and host results must be in place).
    if (any_host) check(hipStreamSynchronize(s), "paged_attention sync");
}

// Writes rows of k/v ([slots.size()][kv_dim], host or device) to the given
// physical slots (block * BLOCK_SIZE + position; < 0 skips) of one layer.
void write_kv_rows(KVCacheManager& m, int32_t layer, const std::vector<int64_t>& slots,
                   const float* k_data, const float* v_data) {
    BlockPool& pool = m.block_pool();
    if (slots.empty() || layer < 0 || layer >= pool.num_layers()) return;
    hipStream_t s = static_cast<hipStream_t>(pool.stream());
    const vcpp_kv_pages pages = pool.pages(layer);
    const size_t rows = slots.size(), bytes = rows * pool.kv_dim() * sizeof(float);
    Staging& st = staging();
    std::lock_guard<std::mutex> lock(st.mu);
    const float* kd = k_data;
    const float* vd = v_data;
    if (!is_device(k_data)) {
        float* b = static_cast<float*>(st.k.get(bytes));
        check(hipMemcpyAsync(b, k_data, bytes, hipMemcpyHostToDevice, s), "k rows");
        kd = b;
    }
    if (!is_device(v_data)) {
        float* b = static_cast<float*>(st.v.get(bytes));
        check(hipMemcpyAsync(b, v_data, bytes, hipMemcpyHostToDevice, s), "v rows");
        vd = b;
    }
    int64_t* sd = static_cast<int64_t*>(st.slots.get(rows * sizeof(int64_t)));
    check(hipMemcpyAsync(sd, slots.data(), rows * sizeof(int64_t), hipMemcpyHostToDevice, s), "slots");
    check_rc(vcpp_write_kv(&pages, kd, vd, sd, (int32_t)rows, 0, s), "write_kv");
    // The staging buffers are reused by the next call, and host callers
    // expect the write to be done when it returns.
    check(hipStreamSynchronize(s), "write_kv sync");
}

void write_kv_token(KVCacheManager& kv_manager, const std::vector<int32_t>& block_table,
                    int32_t seq_len, int32_t layer, const float* k_data, const float* v_data) {
    const int32_t block_idx = (seq_len - 1) / BLOCK_SIZE;
    const int32_t pos = (seq_len - 1) % BLOCK_SIZE;
    if (seq_len <= 0 || block_idx < 0 || (size_t)block_idx >= block_table.size()) return;
    const int32_t kv_dim = kv_manager.block_pool().kv_dim();
    kv_manager.write_kv(block_table[block_idx], layer, pos, k_data, v_data, kv_dim);
}

void write_kv_prefill(KVCacheManager& kv_manager, const std::vector<int32_t>& block_table,
                      int32_t seq_len, int32_t layer, const float* k_data, const float* v_data) {
    if (seq_len <= 0) return;
    const int32_t nb = kv_manager.block_pool().num_blocks();
    std::vector<int64_t> slots(seq_len, -1);
    for (int32_t p = 0; p < seq_len; ++p) {
        const int32_t bi = p / BLOCK_SIZE;
        if ((size_t)bi >= block_table.size()) continue;
        const int32_t bid = block_table[bi];
        if (bid < 0 || bid >= nb) continue;
        slots[p] = (int64_t)bid * BLOCK_SIZE + p % BLOCK_SIZE;
    }
    write_kv_rows(kv_manager, layer, slots, k_data, v_data);
}

void read_kv_prefill(const BlockPool& kv_manager, const std::vector<int32_t>& block_table,
                     int32_t seq_len, int32_t layer, int32_t /*num_kv_heads*/, int32_t /*head_dim*/,
                     float* k_out, float* v_out) {
    const int32_t kv_dim = kv_manager.kv_dim();
    for (int32_t p0 = 0; p0 < seq_len; p0 += BLOCK_SIZE) {
        const int32_t bi = p0 / BLOCK_SIZE;
        if ((size_t)bi >= block_table.size()) continue;
        const float* k = kv_manager.get_k(block_table[bi], layer);
        if (!k) continue;
        const int32_t n = std::min(BLOCK_SIZE, seq_len - p0);
        std::copy(k, k + (size_t)n * kv_dim, k_out + (size_t)p0 * kv_dim);
        const float* v = kv_manager.get_v(block_table[bi], layer);
        std::copy(v, v + (size_t)n * kv_dim, v_out + (size_t)p0 * kv_dim);
    }
}
