// paged_attention.cpp -- the reference's src/paged_attention.h entry points
// (src/paged_attention.cpp:11-201) over the device-resident BlockPool: each
// call packs its arguments into the pool's device staging buffers and runs
// vcpp_paged_decode / vcpp_paged_prefill / vcpp_write_kv on the pool's stream.
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

// Raw rows of some positions of one layer gathered into a dense buffer:
// K rows, then V rows ([n][row_bytes] each), then for INT8 pools the K and V
// scales of each row ([n][num_kv_heads] fp16 each).  One workgroup per row.
__global__ void gather_rows_kernel(const uint8_t* k, const uint8_t* v, const uint16_t* ks,
                                   const uint16_t* vs, const int64_t* src, int32_t n,
                                   int32_t row_bytes, int32_t hkv, int64_t scale_stride,
                                   uint8_t* dst) {
    const int32_t i = blockIdx.x;
    if (i >= n) return;
    const int64_t off = src[2 * i];  // byte offset of the row in the layer's pages
    const int64_t soff = src[2 * i + 1];  // element offset of the row's first scale
    uint8_t* dk = dst + (int64_t)i * row_bytes;
    uint8_t* dv = dst + ((int64_t)n + i) * row_bytes;
    if ((row_bytes & 3) == 0) {  // whole 32-bit words (every row offset is then word aligned)
        const int32_t words = row_bytes / 4;
        const uint32_t* k4 = reinterpret_cast<const uint32_t*>(k + off);
        const uint32_t* v4 = reinterpret_cast<const uint32_t*>(v + off);
        for (int32_t w = threadIdx.x; w < words; w += blockDim.x) {
            reinterpret_cast<uint32_t*>(dk)[w] = k4[w];
            reinterpret_cast<uint32_t*>(dv)[w] = v4[w];
        }
    } else {  // rows of an odd byte count (FP8 / INT8 with kv_dim % 4 != 0, or odd fp16 rows)
        for (int32_t b = threadIdx.x; b < row_bytes; b += blockDim.x) {
            dk[b] = k[off + b];
            dv[b] = v[off + b];
        }
    }
    if (ks) {
        uint16_t* ds = reinterpret_cast<uint16_t*>(dst + 2 * (int64_t)n * row_bytes);
        for (int32_t h = threadIdx.x; h < hkv; h += blockDim.x) {
            ds[(int64_t)i * hkv + h] = ks[soff + h * scale_stride];
            ds[((int64_t)n + i) * hkv + h] = vs[soff + h * scale_stride];
        }
    }
}

// fp32 -> fp16 (round to nearest even), the prefill kernel's q operand.
__global__ void f32_to_f16_kernel(const float* x, _Float16* y, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = (_Float16)x[i];
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

    PoolStaging& st = kv_manager.staging();
    std::lock_guard<std::mutex> lock(st.mu);
    float* qd = static_cast<float*>(st.q.get(row * B * sizeof(float), s));
    float* od = static_cast<float*>(st.out.get(row * B * sizeof(float), s));
    int32_t* td = static_cast<int32_t*>(st.tables.get(tables.size() * sizeof(int32_t), s));
    int32_t* cd = static_cast<int32_t*>(st.ctx.get(2 * B * sizeof(int32_t), s));
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
    void* ws = wsb ? st.ws.get(wsb, s) : nullptr;
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
    // Host inputs or outputs: return with the work done (host results must be
    // in place).  Device ones: the pool's next call reuses the staging
    // buffers behind this one on the same stream.
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
    PoolStaging& st = pool.staging();
    std::lock_guard<std::mutex> lock(st.mu);
    const float* kd = k_data;
    const float* vd = v_data;
    if (!is_device(k_data)) {
        float* b = static_cast<float*>(st.k.get(bytes, s));
        check(hipMemcpyAsync(b, k_data, bytes, hipMemcpyHostToDevice, s), "k rows");
        kd = b;
    }
    if (!is_device(v_data)) {
        float* b = static_cast<float*>(st.v.get(bytes, s));
        check(hipMemcpyAsync(b, v_data, bytes, hipMemcpyHostToDevice, s), "v rows");
        vd = b;
    }
    int64_t* sd = static_cast<int64_t*>(st.slots.get(rows * sizeof(int64_t), s));
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
    if (seq_len <= 0 || layer < 0 || layer >= kv_manager.num_layers()) return;
    const int32_t kv_dim = kv_manager.kv_dim();
    const int32_t hkv = kv_manager.num_kv_heads();
    const vcpp_kv_pages pages = kv_manager.pages(layer);
    const int32_t esize = kv_elem_size(kv_manager.kv_dtype());
    const int32_t row_bytes = kv_dim * esize;
    // Positions with a block in the pool (the reference skips the others,
    // leaving their output rows as they are).
    std::vector<int32_t> pos;
    std::vector<int64_t> src;
    for (int32_t p = 0; p < seq_len; ++p) {
        const int32_t bi = p / BLOCK_SIZE;
        if ((size_t)bi >= block_table.size()) continue;
        const int32_t bid = block_table[bi];
        if (bid < 0 || bid >= kv_manager.num_blocks()) continue;
        pos.push_back(p);
        src.push_back((int64_t)bid * pages.block_stride * esize + (int64_t)(p % BLOCK_SIZE) * row_bytes);
        src.push_back((int64_t)bid * pages.scale_block_stride + p % BLOCK_SIZE);
    }
    const int32_t n = (int32_t)pos.size();
    if (n == 0) return;
    const bool scaled = pages.k_scale != nullptr;
    const size_t bytes = 2 * (size_t)n * row_bytes + (scaled ? 2 * (size_t)n * hkv * 2 : 0);
    hipStream_t s = static_cast<hipStream_t>(kv_manager.stream());
    PoolStaging& st = kv_manager.staging();
    std::lock_guard<std::mutex> lock(st.mu);
    int64_t* sd = static_cast<int64_t*>(st.slots.get(src.size() * sizeof(int64_t), s));
    uint8_t* rows = static_cast<uint8_t*>(st.rows.get(bytes, s));
    check(hipMemcpyAsync(sd, src.data(), src.size() * sizeof(int64_t), hipMemcpyHostToDevice, s),
          "read_kv_prefill offsets");
    hipLaunchKernelGGL(gather_rows_kernel, dim3(n), dim3(256), 0, s,
                       static_cast<const uint8_t*>(pages.k), static_cast<const uint8_t*>(pages.v),
                       pages.k_scale, pages.v_scale, sd, n, row_bytes, hkv, (int64_t)BLOCK_SIZE, rows);
    check(hipGetLastError(), "read_kv_prefill gather");
    st.host.resize(bytes);
    check(hipMemcpyAsync(st.host.data(), rows, bytes, hipMemcpyDeviceToHost, s), "read_kv_prefill copy");
    check(hipStreamSynchronize(s), "read_kv_prefill sync");
    const uint8_t* h = st.host.data();
    const uint16_t* hs = reinterpret_cast<const uint16_t*>(h + 2 * (size_t)n * row_bytes);
    const KVDtype dt = kv_manager.kv_dtype();
    const int32_t d = kv_manager.head_dim();
    for (int32_t i = 0; i < n; ++i) {
        const size_t o = (size_t)pos[i] * kv_dim;
        vcpp_host::decode_row(h + (size_t)i * row_bytes, scaled ? hs + (size_t)i * hkv : nullptr,
                              k_out + o, kv_dim, d, dt);
        vcpp_host::decode_row(h + ((size_t)n + i) * row_bytes,
                              scaled ? hs + ((size_t)n + i) * hkv : nullptr, v_out + o, kv_dim, d, dt);
    }
}

void paged_prefill(const float* q, const std::vector<int32_t>& block_table, int32_t prefix_len,
                   int32_t num_tokens, const BlockPool& kv_manager, int32_t num_heads,
                   int32_t num_kv_heads, int32_t head_dim, int32_t layer, float* out) {
    const PrefillChunk c{q, &block_table, prefix_len, num_tokens, out};
    paged_prefill_batch({c}, kv_manager, num_heads, num_kv_heads, head_dim, layer);
}

void paged_prefill_batch(const std::vector<PrefillChunk>& chunks, const BlockPool& kv_manager,
                         int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, int32_t layer) {
    if (num_heads <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads != 0) return;
    vcpp_kv_pages pages;
    if (!attention_pages(kv_manager, layer, num_kv_heads, head_dim, &pages)) return;
    hipStream_t s = static_cast<hipStream_t>(kv_manager.stream());
    const size_t row = (size_t)num_heads * head_dim;
    // Chunks with a table and at least one token; rows of chunk j are
    // rows0[j] .. rows0[j + 1] - 1 of the staged q / out.
    std::vector<size_t> live;
    std::vector<int32_t> rows0{0};
    int32_t max_blocks = 1, max_len = 0;
    for (size_t i = 0; i < chunks.size(); ++i) {
        const PrefillChunk& c = chunks[i];
        if (!c.block_table || c.num_tokens <= 0 || c.prefix_len < 0 || !c.q || !c.out) continue;
        live.push_back(i);
        rows0.push_back(rows0.back() + c.num_tokens);
        max_blocks = std::max<int32_t>(max_blocks, (int32_t)c.block_table->size());
        max_len = std::max(max_len, c.num_tokens);
    }
    if (live.empty()) return;
    const int32_t C = (int32_t)live.size(), R = rows0.back();
    const bool fp32 = pages.dtype == VCPP_KV_F32;

    PoolStaging& st = kv_manager.staging();
    std::lock_guard<std::mutex> lock(st.mu);
    float* qd = static_cast<float*>(st.q.get(row * R * sizeof(float), s));
    float* od = static_cast<float*>(st.out.get(row * R * sizeof(float), s));
    bool any_host = false;
    for (int32_t j = 0; j < C; ++j) {
        const PrefillChunk& c = chunks[live[j]];
        const bool dev = is_device(c.q);
        any_host |= !dev;
        check(hipMemcpyAsync(qd + row * rows0[j], c.q, row * c.num_tokens * sizeof(float),
                             dev ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice, s), "prefill q");
    }
    if (fp32) {
        // fp32 pages: every row is a decode query over positions
        // 0 .. prefix + i of its chunk's table (the engine's per-position
        // semantics), run by the fp32 decode kernel.
        std::vector<int32_t> tables((size_t)R * max_blocks, -1), tlens(R), ctx(R);
        int32_t max_ctx = 0;
        for (int32_t j = 0; j < C; ++j) {
            const PrefillChunk& c = chunks[live[j]];
            for (int32_t i = 0; i < c.num_tokens; ++i) {
                const int32_t r = rows0[j] + i;
                std::copy(c.block_table->begin(), c.block_table->end(), tables.begin() + (size_t)r * max_blocks);
                tlens[r] = (int32_t)c.block_table->size();
                ctx[r] = c.prefix_len + i + 1;
                max_ctx = std::max(max_ctx, ctx[r]);
            }
        }
        int32_t* td = static_cast<int32_t*>(st.tables.get(tables.size() * sizeof(int32_t), s));
        int32_t* cd = static_cast<int32_t*>(st.ctx.get(2 * (size_t)R * sizeof(int32_t), s));
        check(hipMemcpyAsync(td, tables.data(), tables.size() * sizeof(int32_t), hipMemcpyHostToDevice, s),
              "prefill tables");
        check(hipMemcpyAsync(cd, ctx.data(), R * sizeof(int32_t), hipMemcpyHostToDevice, s), "prefill lens");
        check(hipMemcpyAsync(cd + R, tlens.data(), R * sizeof(int32_t), hipMemcpyHostToDevice, s),
              "prefill table lens");
        const size_t wsb = vcpp_decode_workspace_size(&pages, R, num_heads, max_ctx, 0);
        void* ws = wsb ? st.ws.get(wsb, s) : nullptr;
        check_rc(vcpp_paged_decode(&pages, qd, od, td, max_blocks, cd + R, cd, R, max_ctx, num_heads, 0,
                                   ws, wsb, s),
                 "paged_prefill (fp32 pages)");
    } else {
        std::vector<int32_t> tables((size_t)C * max_blocks, -1), meta(2 * (size_t)C + 1);
        int32_t max_prefix = 0;
        for (int32_t j = 0; j < C; ++j) {
            const PrefillChunk& c = chunks[live[j]];
            std::copy(c.block_table->begin(), c.block_table->end(), tables.begin() + (size_t)j * max_blocks);
            meta[C + 1 + j] = c.prefix_len;
            max_prefix = std::max(max_prefix, c.prefix_len);
        }
        for (int32_t j = 0; j <= C; ++j) meta[j] = rows0[j];
        uint16_t* q16 = static_cast<uint16_t*>(st.k.get(row * R * sizeof(uint16_t), s));
        int32_t* td = static_cast<int32_t*>(st.tables.get(tables.size() * sizeof(int32_t), s));
        int32_t* md = static_cast<int32_t*>(st.ctx.get(meta.size() * sizeof(int32_t), s));
        check(hipMemcpyAsync(td, tables.data(), tables.size() * sizeof(int32_t), hipMemcpyHostToDevice, s),
              "prefill tables");
        check(hipMemcpyAsync(md, meta.data(), meta.size() * sizeof(int32_t), hipMemcpyHostToDevice, s),
              "prefill chunk starts");
        const int64_t nq = (int64_t)row * R;
        hipLaunchKernelGGL(f32_to_f16_kernel, dim3((unsigned)((nq + 255) / 256)), dim3(256), 0, s, qd,
                           reinterpret_cast<_Float16*>(q16), nq);
        check(hipGetLastError(), "prefill q to fp16");
        // Few chunks on long prefixes split each tile's keys over several
        // workgroups (the size is 0 when the chunks fill the GPU already).
        const size_t wsb = vcpp_prefill_workspace_size(&pages, C, max_len, max_prefix, num_heads);
        void* ws = wsb ? st.ws.get(wsb, s) : nullptr;
        check_rc(vcpp_paged_prefill_split(&pages, q16, od, td, max_blocks, md, md + C + 1, C, max_len, max_prefix,
                                          num_heads, ws, wsb, s),
                 "paged_prefill");
    }
    for (int32_t j = 0; j < C; ++j) {
        const PrefillChunk& c = chunks[live[j]];
        const bool dev = is_device(c.out);
        any_host |= !dev;
        check(hipMemcpyAsync(c.out, od + row * rows0[j], row * c.num_tokens * sizeof(float),
                             dev ? hipMemcpyDeviceToDevice : hipMemcpyDeviceToHost, s), "prefill out");
    }
    if (any_host) check(hipStreamSynchronize(s), "paged_prefill sync");
}

void paged_attention_step(const std::vector<const float*>& q_ptrs,
                          const std::vector<const std::vector<int32_t>*>& block_tables,
                          const std::vector<int32_t>& seq_lens, std::vector<float*> out_ptrs,
                          const std::vector<PrefillChunk>& chunks, const BlockPool& kv_manager,
                          int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, int32_t layer) {
    if (num_heads <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads != 0) return;
    vcpp_kv_pages pages;
    if (!attention_pages(kv_manager, layer, num_kv_heads, head_dim, &pages)) return;
    // Decoding requests with a table, prefill chunks with a table and tokens
    // (the others are skipped, as by the two calls).
    std::vector<size_t> dl, pl;
    int32_t dmb = 1, max_ctx = 0, pmb = 1, max_len = 0;
    const size_t n = std::min({q_ptrs.size(), block_tables.size(), seq_lens.size(), out_ptrs.size()});
    for (size_t i = 0; i < n; ++i) {
        if (!block_tables[i]) continue;
        dl.push_back(i);
        dmb = std::max<int32_t>(dmb, (int32_t)block_tables[i]->size());
        max_ctx = std::max(max_ctx, seq_lens[i]);
    }
    for (size_t i = 0; i < chunks.size(); ++i) {
        const PrefillChunk& c = chunks[i];
        if (!c.block_table || c.num_tokens <= 0 || c.prefix_len < 0 || !c.q || !c.out) continue;
        pl.push_back(i);
        pmb = std::max<int32_t>(pmb, (int32_t)c.block_table->size());
        max_len = std::max(max_len, c.num_tokens);
    }
    if (pages.dtype == VCPP_KV_F32 || dl.empty() || pl.empty()) {
        if (!dl.empty())
            paged_attention_batch(q_ptrs, block_tables, seq_lens, kv_manager, num_heads, num_kv_heads, head_dim,
                                  layer, out_ptrs);
        if (!pl.empty()) paged_prefill_batch(chunks, kv_manager, num_heads, num_kv_heads, head_dim, layer);
        return;
    }
    hipStream_t s = static_cast<hipStream_t>(kv_manager.stream());
    const size_t row = (size_t)num_heads * head_dim;
    const int32_t B = (int32_t)dl.size(), C = (int32_t)pl.size();
    // Host-side argument blocks: decode tables then prefill tables; decode
    // context lengths, table lengths, then the chunks' row starts and
    // prefix lengths.
    std::vector<int32_t> tables((size_t)B * dmb + (size_t)C * pmb, -1), meta(2 * (size_t)B + 2 * C + 1);
    for (int32_t b = 0; b < B; ++b) {
        const auto& t = *block_tables[dl[b]];
        std::copy(t.begin(), t.end(), tables.begin() + (size_t)b * dmb);
        meta[b] = std::max(seq_lens[dl[b]], 0);
        meta[B + b] = (int32_t)t.size();
    }
    std::vector<int32_t> rows0{0};
    for (int32_t j = 0; j < C; ++j) {
        const PrefillChunk& c = chunks[pl[j]];
        std::copy(c.block_table->begin(), c.block_table->end(), tables.begin() + (size_t)B * dmb + (size_t)j * pmb);
        rows0.push_back(rows0.back() + c.num_tokens);
        meta[2 * B + C + 1 + j] = c.prefix_len;
    }
    for (int32_t j = 0; j <= C; ++j) meta[2 * B + j] = rows0[j];
    const int32_t R = rows0.back();

    PoolStaging& st = kv_manager.staging();
    std::lock_guard<std::mutex> lock(st.mu);
    float* qd = static_cast<float*>(st.q.get(row * ((size_t)B + R) * sizeof(float), s));
    float* od = static_cast<float*>(st.out.get(row * ((size_t)B + R) * sizeof(float), s));
    uint16_t* q16 = static_cast<uint16_t*>(st.k.get(row * R * sizeof(uint16_t), s));
    int32_t* td = static_cast<int32_t*>(st.tables.get(tables.size() * sizeof(int32_t), s));
    int32_t* md = static_cast<int32_t*>(st.ctx.get(meta.size() * sizeof(int32_t), s));
    float* qp = qd + row * B;
    float* op = od + row * B;
    bool any_host = false;
    for (int32_t b = 0; b < B; ++b) {
        const float* src = q_ptrs[dl[b]];
        const bool dev = is_device(src);
        any_host |= !dev;
        check(hipMemcpyAsync(qd + row * b, src, row * sizeof(float),
                             dev ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice, s), "step decode q");
    }
    for (int32_t j = 0; j < C; ++j) {
        const PrefillChunk& c = chunks[pl[j]];
        const bool dev = is_device(c.q);
        any_host |= !dev;
        check(hipMemcpyAsync(qp + row * rows0[j], c.q, row * c.num_tokens * sizeof(float),
                             dev ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice, s), "step prefill q");
    }
    check(hipMemcpyAsync(td, tables.data(), tables.size() * sizeof(int32_t), hipMemcpyHostToDevice, s),
          "step tables");
    check(hipMemcpyAsync(md, meta.data(), meta.size() * sizeof(int32_t), hipMemcpyHostToDevice, s), "step lens");
    const int64_t nq = (int64_t)row * R;
    hipLaunchKernelGGL(f32_to_f16_kernel, dim3((unsigned)((nq + 255) / 256)), dim3(256), 0, s, qp,
                       reinterpret_cast<_Float16*>(q16), nq);
    check(hipGetLastError(), "step q to fp16");
    const size_t wsb = vcpp_mixed_workspace_size(&pages, B, num_heads, max_ctx, pmb);
    void* ws = wsb ? st.ws.get(wsb, s) : nullptr;
    check_rc(vcpp_paged_mixed_step(&pages, qd, od, td, dmb, md + B, md, B, max_ctx, q16, op, td + (size_t)B * dmb,
                                   pmb, md + 2 * B, md + 2 * B + C + 1, C, max_len, num_heads, ws, wsb, s),
             "paged_attention_step");
    for (int32_t b = 0; b < B; ++b) {
        float* dst = out_ptrs[dl[b]];
        const bool dev = is_device(dst);
        any_host |= !dev;
        check(hipMemcpyAsync(dst, od + row * b, row * sizeof(float),
                             dev ? hipMemcpyDeviceToDevice : hipMemcpyDeviceToHost, s), "step decode out");
    }
    for (int32_t j = 0; j < C; ++j) {
        const PrefillChunk& c = chunks[pl[j]];
        const bool dev = is_device(c.out);
        any_host |= !dev;
        check(hipMemcpyAsync(c.out, op + row * rows0[j], row * c.num_tokens * sizeof(float),
                             dev ? hipMemcpyDeviceToDevice : hipMemcpyDeviceToHost, s), "step prefill out");
    }
    if (any_host) check(hipStreamSynchronize(s), "paged_attention_step sync");
}
