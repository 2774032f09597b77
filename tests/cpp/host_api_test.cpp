// host_api_test.cpp -- drives the C++ BlockPool / KVCacheManager /
// paged_attention mirror (include/vllm_cpp) the way the reference engine
// does (src/paged_engine.cpp:329-384,460-508) and checks every result
// against the CPU oracle (oracle/oracle.h) on the same data.  Test
// infrastructure: links liboracle.so as the checker.
//
// Prints one line per check and "ALL PASSED" at the end; exit status 1 on
// the first failure.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <vector>

#include "oracle.h"
#include "vllm_cpp/paged_attention.h"

namespace {

int g_checks = 0;

#define CHECK(cond, ...)                                                   \
    do {                                                                   \
        ++g_checks;                                                        \
        if (!(cond)) {                                                     \
            std::printf("FAIL %s:%d: ", __FILE__, __LINE__);               \
            std::printf(__VA_ARGS__);                                      \
            std::printf("\n");                                             \
            std::exit(1);                                                  \
        }                                                                  \
    } while (0)

std::vector<float> normal(uint64_t seed, size_t n, double std = 1.0) {
    std::vector<float> x(n);
    orc_fill_normal(seed, x.data(), (int64_t)n, 0.0, std);
    return x;
}

// The parity bar: max |got - want| <= atol outright, and the normwise
// relative error ||got - want|| / ||want|| <= rtol.
void close(const float* got, const float* want, size_t n, double atol, double rtol, const char* what) {
    double worst = 0, e2 = 0, w2 = 0;
    size_t at = 0;
    for (size_t i = 0; i < n; ++i) {
        CHECK(std::isfinite(got[i]), "%s: non-finite at %zu", what, i);
        const double err = std::fabs((double)got[i] - want[i]);
        if (err > worst) {
            worst = err;
            at = i;
        }
        e2 += err * err;
        w2 += (double)want[i] * want[i];
    }
    CHECK(worst <= atol, "%s: max abs err %.3g > %.3g at index %zu (got %.7g want %.7g)", what, worst, atol, at,
          got[at], want[at]);
    const double rel = w2 > 0 ? std::sqrt(e2 / w2) : std::sqrt(e2);
    CHECK(rel <= rtol, "%s: normwise relative err %.3g > %.3g", what, rel, rtol);
    std::printf("ok   %-58s max abs err %.3g, rel %.3g\n", what, worst, rel);
}

// Host image of one layer of a pool in the reference slab layout, encoded by
// the oracle, for orc_paged_attention.
struct HostLayer {
    KVDtype dtype;
    int32_t nb, num_layers, hkv, d;
    std::vector<uint8_t> k, v;       // [nb][num_layers][16][kv_dim] elements
    std::vector<uint16_t> ks, vs;    // [nb][num_layers][hkv][16]
    HostLayer(KVDtype t, int32_t nb_, int32_t nl, int32_t hkv_, int32_t d_)
        : dtype(t), nb(nb_), num_layers(nl), hkv(hkv_), d(d_) {
        const size_t n = (size_t)nb * nl * 16 * hkv * d * kv_elem_size(t);
        k.assign(n, 0);
        v.assign(n, 0);
        ks.assign((size_t)nb * nl * hkv * 16, 0);
        vs.assign((size_t)nb * nl * hkv * 16, 0);
    }
    int64_t row_off(int32_t block, int32_t layer, int32_t pos) const {
        return (((int64_t)block * num_layers + layer) * 16 + pos) * hkv * d;  // elements
    }
    void write(int32_t block, int32_t layer, int32_t pos, const float* kr, const float* vr) {
        const int64_t off = row_off(block, layer, pos);
        for (int which = 0; which < 2; ++which) {
            const float* src = which ? vr : kr;
            std::vector<uint8_t>& dst = which ? v : k;
            if (dtype == KVDtype::FP32) {
                std::memcpy(dst.data() + off * 4, src, sizeof(float) * hkv * d);
            } else if (dtype == KVDtype::FP16) {
                orc_f16_encode_trunc_n(src, reinterpret_cast<uint16_t*>(dst.data()) + off, (int64_t)hkv * d);
            } else if (dtype == KVDtype::FP8_E4M3) {
                orc_fp8_encode_n(src, dst.data() + off, (int64_t)hkv * d);
            } else {
                std::vector<uint16_t>& sc = which ? vs : ks;
                for (int32_t h = 0; h < hkv; ++h) {
                    uint16_t s;
                    orc_quant_i8(src + h * d, d, reinterpret_cast<int8_t*>(dst.data()) + off + h * d, &s);
                    sc[(((int64_t)block * num_layers + layer) * hkv + h) * 16 + pos] = s;
                }
            }
        }
    }
    orc_pool pool(int32_t layer) const {
        orc_pool p{};
        p.kind = dtype == KVDtype::FP32       ? ORC_F32
                 : dtype == KVDtype::FP16     ? ORC_F16
                 : dtype == KVDtype::FP8_E4M3 ? ORC_FP8
                                              : ORC_I8;
        const int64_t esz = kv_elem_size(dtype);
        p.k = k.data() + (int64_t)layer * 16 * hkv * d * esz;
        p.v = v.data() + (int64_t)layer * 16 * hkv * d * esz;
        p.k_scale = ks.data() + (int64_t)layer * hkv * 16;
        p.v_scale = vs.data() + (int64_t)layer * hkv * 16;
        p.num_blocks = nb;
        p.block_stride = (int64_t)num_layers * 16 * hkv * d;
        p.scale_block_stride = (int64_t)num_layers * hkv * 16;
        p.block_size = 16;
        p.num_kv_heads = hkv;
        p.head_dim = d;
        return p;
    }
};

void test_bookkeeping() {
    BlockPool pool(6, 2, 32, KVDtype::FP32);
    CHECK(pool.alloc() == 0 && pool.alloc() == 1 && pool.alloc() == 2, "alloc order");
    CHECK(pool.free_count() == 3 && pool.used_count() == 3, "counts");
    pool.ref(1);
    pool.free(1);  // ref 2 -> 1: still used
    CHECK(!pool.get_block(1).free && pool.get_block(1).ref_count == 1, "free with ref");
    pool.deref(1);
    CHECK(pool.get_block(1).free, "deref to zero frees");
    CHECK(pool.alloc() == 1, "lowest free block first");
    pool.free(-3);
    pool.free(99);  // out of range: ignored
    CHECK(pool.used_count() == 3, "out-of-range free ignored");
    CHECK(pool.get_k_raw(6, 0) == nullptr && pool.get_k_raw(0, 2) == nullptr, "raw bounds");
    CHECK(pool.get_k_raw(1, 1) == pool.get_k_raw(1, 0) + 16 * 32 * 4, "layer slab offset");
    CHECK(pool.get_k_raw(2, 0) == pool.get_k_raw(1, 0) + 2 * 16 * 32 * 4, "block offset");
    pool.reset();
    CHECK(pool.free_count() == 6, "reset frees all");
    std::printf("ok   %-58s\n", "BlockPool book-keeping (alloc/free/ref/deref/reset)");
}

void test_write_read(KVDtype dt) {
    const int32_t L = 3, H = 4, D = 80, kv = H * D;
    KVCacheManager m(L, kv, 5, dt, D);
    HostLayer host(dt, 5, L, H, D);
    std::vector<int32_t> blocks;
    CHECK(m.alloc_blocks(3, blocks), "alloc_blocks");
    auto k = normal(11, kv * 4, 2.0), v = normal(12, kv * 4, 2.0);
    const int32_t pos[4] = {0, 5, 15, 7};
    for (int i = 0; i < 4; ++i) {
        m.write_kv(blocks[i % 3], i % L, pos[i], k.data() + i * kv, v.data() + i * kv, kv);
        host.write(blocks[i % 3], i % L, pos[i], k.data() + i * kv, v.data() + i * kv);
    }
    m.write_kv(blocks[0], 0, 16, k.data(), v.data(), kv);  // slot out of range: ignored
    m.write_kv(77, 0, 0, k.data(), v.data(), kv);          // block out of range: ignored
    // Raw device bytes equal the oracle's encoding.
    const BlockPool& p = m.block_pool();
    for (int32_t b = 0; b < 5; ++b)
        for (int32_t l = 0; l < L; ++l) {
            const size_t bytes = (size_t)16 * kv * kv_elem_size(dt);
            std::vector<uint8_t> got(bytes);
            CHECK(hipMemcpy(got.data(), p.get_k_raw(b, l), bytes, hipMemcpyDeviceToHost) == hipSuccess, "copy");
            CHECK(std::memcmp(got.data(), host.k.data() + host.row_off(b, l, 0) * kv_elem_size(dt), bytes) == 0,
                  "K bytes of block %d layer %d", b, l);
        }
    // read_kv returns the decoded values.
    std::vector<float> rk(kv), rv(kv);
    for (int i = 0; i < 4; ++i) {
        m.read_kv(blocks[i % 3], i % L, pos[i], rk.data(), rv.data(), kv);
        orc_pool op = host.pool(i % L);
        std::vector<float> want(kv);
        for (int32_t j = 0; j < kv; ++j) {
            if (dt == KVDtype::FP32) want[j] = k[i * kv + j];
            else if (dt == KVDtype::FP16) want[j] = orc_f16_decode(orc_f16_encode_trunc(k[i * kv + j]));
            else if (dt == KVDtype::FP8_E4M3) want[j] = orc_fp8_decode(orc_fp8_encode(k[i * kv + j]));
            else {
                const int32_t h = j / D;
                const int8_t q = reinterpret_cast<const int8_t*>(op.k)[blocks[i % 3] * op.block_stride + pos[i] * kv + j];
                want[j] = (float)q * orc_f16_decode(op.k_scale[blocks[i % 3] * op.scale_block_stride + h * 16 + pos[i]]);
            }
        }
        CHECK(std::memcmp(rk.data(), want.data(), sizeof(float) * kv) == 0, "read_kv row %d", i);
    }
    // free zeroes the block; copy_blocks copies all layers.
    m.copy_blocks({blocks[1]}, {blocks[2]});
    std::vector<float> a(kv), b2(kv), c(kv);
    m.read_kv(blocks[2], 1, pos[1], a.data(), b2.data(), kv);
    m.read_kv(blocks[1], 1, pos[1], c.data(), b2.data(), kv);
    CHECK(std::memcmp(a.data(), c.data(), sizeof(float) * kv) == 0, "copy_blocks");
    m.free_blocks({blocks[0]});
    m.read_kv(blocks[0], 0, pos[0], a.data(), b2.data(), kv);
    bool zero = true;
    for (float x : a) zero &= (x == 0.0f);
    CHECK(zero, "freed block zeroed");
    static const char* names[] = {"FP32", "FP16", "FP8", "INT8"};
    std::printf("ok   write_kv / read_kv / copy_blocks / free on %-12s (bit-exact)\n", names[(int)dt]);
}

// Preemption that keeps the data: swap_out before free, swap_in into the
// blocks allocated on restore (which the free zeroed or another request used).
void test_swap(KVDtype dt) {
    const int32_t L = 3, H = 4, D = 80, kv = H * D;
    KVCacheManager m(L, kv, 6, dt, D);
    std::vector<int32_t> blocks;
    CHECK(m.alloc_blocks(3, blocks), "alloc_blocks");
    auto k = normal(31, kv * 6, 2.0), v = normal(32, kv * 6, 2.0);
    for (int i = 0; i < 6; ++i)
        m.write_kv(blocks[i % 3], i % L, 2 * i, k.data() + i * kv, v.data() + i * kv, kv);
    std::vector<float> before(6 * kv), vb(6 * kv);
    for (int i = 0; i < 6; ++i)
        m.read_kv(blocks[i % 3], i % L, 2 * i, before.data() + i * kv, vb.data() + i * kv, kv);
    auto sw = m.swap_out(blocks);
    m.free_blocks(blocks);  // zeroes them (after the copy, same stream)
    std::vector<int32_t> other, again;
    CHECK(m.alloc_blocks(2, other), "alloc other");  // reuses freed ids
    auto junk = normal(33, kv, 5.0);
    for (int32_t b : other) m.write_kv(b, 0, 0, junk.data(), junk.data(), kv);
    CHECK(m.alloc_blocks(3, again), "alloc restore");
    CHECK(m.swap_in(*sw, again), "swap_in");
    CHECK(!m.swap_in(*sw, other), "swap_in rejects a different block count");
    std::vector<float> after(kv), va(kv);
    for (int i = 0; i < 6; ++i) {
        m.read_kv(again[i % 3], i % L, 2 * i, after.data(), va.data(), kv);
        CHECK(std::memcmp(after.data(), before.data() + i * kv, sizeof(float) * kv) == 0 &&
                  std::memcmp(va.data(), vb.data() + i * kv, sizeof(float) * kv) == 0,
              "swapped-in row %d", i);
    }
    static const char* names[] = {"FP32", "FP16", "FP8", "INT8"};
    std::printf("ok   swap_out / free / swap_in on %-12s (bit-exact)\n", names[(int)dt]);
}

void test_attention(KVDtype dt) {
    const int32_t L = 2, layer = 1, H = 64, HKV = 8, D = 80, kv = HKV * D, NB = 160;
    KVCacheManager m(L, kv, NB, dt, D);
    HostLayer host(dt, NB, L, HKV, D);
    // Reserve a few blocks so tables are not the identity.
    std::vector<int32_t> junk;
    CHECK(m.alloc_blocks(7, junk), "alloc");
    const int32_t lens[4] = {1, 300, 17, 1777};
    std::vector<std::vector<int32_t>> tables(4);
    std::vector<std::vector<float>> ks, vs;
    for (int r = 0; r < 4; ++r) {
        CHECK(m.alloc_blocks((lens[r] + 15) / 16 + 1, tables[r]), "alloc request %d", r);
        ks.push_back(normal(100 + r, (size_t)lens[r] * kv));
        vs.push_back(normal(200 + r, (size_t)lens[r] * kv));
        // prefill all but the last token, then append it as a decode step
        write_kv_prefill(m, tables[r], lens[r] - 1, layer, ks[r].data(), vs[r].data());
        write_kv_token(m, tables[r], lens[r], layer, ks[r].data() + (size_t)(lens[r] - 1) * kv,
                       vs[r].data() + (size_t)(lens[r] - 1) * kv);
        for (int32_t p = 0; p < lens[r]; ++p)
            host.write(tables[r][p / 16], layer, p % 16, ks[r].data() + (size_t)p * kv,
                       vs[r].data() + (size_t)p * kv);
        tables[r].pop_back();  // one spare block removed: table covers exactly the context
    }
    tables[2][0] = NB + 5;     // a bad block id: skipped by both sides
    const double tol = dt == KVDtype::FP32 ? 1e-4 : 2e-3, rtol = dt == KVDtype::FP32 ? 1e-4 : 1e-2;
    orc_pool op = host.pool(layer);
    std::vector<float> q = normal(300, (size_t)4 * H * D), want((size_t)4 * H * D);
    for (int r = 0; r < 4; ++r)
        orc_paged_attention(&op, q.data() + (size_t)r * H * D, tables[r].data(), (int32_t)tables[r].size(),
                            lens[r], H, want.data() + (size_t)r * H * D);
    // 1. one request at a time, host buffers (the reference engine's call)
    std::vector<float> out((size_t)4 * H * D, NAN);
    for (int r = 0; r < 4; ++r)
        paged_attention(q.data() + (size_t)r * H * D, tables[r], lens[r], m.block_pool(), H, HKV, D, layer,
                        out.data() + (size_t)r * H * D);
    close(out.data(), want.data(), out.size(), tol, rtol, "paged_attention, host buffers");
    // 2. one launch for the batch, device buffers
    float *qd, *od;
    CHECK(hipMalloc(&qd, q.size() * 4) == hipSuccess && hipMalloc(&od, q.size() * 4) == hipSuccess, "malloc");
    CHECK(hipMemcpy(qd, q.data(), q.size() * 4, hipMemcpyHostToDevice) == hipSuccess, "copy");
    std::vector<const float*> qp;
    std::vector<float*> opp;
    std::vector<const std::vector<int32_t>*> tp;
    std::vector<int32_t> sl;
    for (int r = 0; r < 4; ++r) {
        qp.push_back(qd + (size_t)r * H * D);
        opp.push_back(od + (size_t)r * H * D);
        tp.push_back(&tables[r]);
        sl.push_back(lens[r]);
    }
    paged_attention_batch(qp, tp, sl, m.block_pool(), H, HKV, D, layer, opp);
    CHECK(hipDeviceSynchronize() == hipSuccess, "sync");
    std::vector<float> out2(q.size());
    CHECK(hipMemcpy(out2.data(), od, q.size() * 4, hipMemcpyDeviceToHost) == hipSuccess, "copy");
    close(out2.data(), want.data(), out2.size(), tol, rtol, "paged_attention_batch, device buffers");
    // 3. a null table is skipped: its output stays untouched
    std::vector<float> keep(H * D, 42.0f);
    std::vector<const float*> q3{q.data(), q.data() + H * D};
    std::vector<float*> o3{out.data(), keep.data()};
    std::vector<const std::vector<int32_t>*> t3{&tables[0], nullptr};
    paged_attention_batch(q3, t3, {lens[0], lens[1]}, m.block_pool(), H, HKV, D, layer, o3);
    CHECK(keep[0] == 42.0f && keep[H * D - 1] == 42.0f, "null table skipped");
    // 4. a table shorter than seq_len: positions past it are skipped
    std::vector<int32_t> short_t(tables[3].begin(), tables[3].begin() + 10);
    std::vector<float> w4(H * D), g4(H * D);
    orc_paged_attention(&op, q.data(), short_t.data(), 10, lens[3], H, w4.data());
    paged_attention(q.data(), short_t, lens[3], m.block_pool(), H, HKV, D, layer, g4.data());
    close(g4.data(), w4.data(), g4.size(), tol, rtol, "paged_attention, table shorter than seq_len");
    // 5. read_kv_prefill gathers the decoded rows
    std::vector<float> rk((size_t)lens[1] * kv), rv((size_t)lens[1] * kv);
    read_kv_prefill(m.block_pool(), tables[1], lens[1], layer, HKV, D, rk.data(), rv.data());
    for (int32_t p = 0; p < lens[1]; p += 37) {
        for (int32_t j = 0; j < kv; j += 13) {
            float want_k;
            const int64_t e = tables[1][p / 16] * op.block_stride + (int64_t)(p % 16) * kv + j;
            if (dt == KVDtype::FP32) want_k = reinterpret_cast<const float*>(op.k)[e];
            else if (dt == KVDtype::FP16) want_k = orc_f16_decode(reinterpret_cast<const uint16_t*>(op.k)[e]);
            else if (dt == KVDtype::FP8_E4M3) want_k = orc_fp8_decode(reinterpret_cast<const uint8_t*>(op.k)[e]);
            else want_k = (float)reinterpret_cast<const int8_t*>(op.k)[e] *
                          orc_f16_decode(op.k_scale[tables[1][p / 16] * op.scale_block_stride + (j / D) * 16 + p % 16]);
            CHECK(rk[(size_t)p * kv + j] == want_k, "read_kv_prefill pos %d dim %d", p, j);
        }
    }
    std::printf("ok   %-58s\n", "read_kv_prefill");
    // 6. paged_prefill: the last 100 tokens of request 3 as one chunk on its
    // 1677-token prefix (few workgroups on a long prefix: the keys of each
    // tile are split), host fp32 q and out (the engine's prefill buffers);
    // row i is the reference's per-position attention over 0 .. 1677 + i.
    {
        const int32_t n = 100, pre = lens[3] - n;
        std::vector<float> qc = normal(400, (size_t)n * H * D), wc((size_t)n * H * D), gc((size_t)n * H * D, NAN);
        for (int32_t i = 0; i < n; ++i)
            orc_paged_attention(&op, qc.data() + (size_t)i * H * D, tables[3].data(), (int32_t)tables[3].size(),
                                pre + i + 1, H, wc.data() + (size_t)i * H * D);
        paged_prefill(qc.data(), tables[3], pre, n, m.block_pool(), H, HKV, D, layer, gc.data());
        close(gc.data(), wc.data(), gc.size(), tol, rtol, "paged_prefill, host buffers");
        // 7. two chunks in one launch, device q / out: request 1 whole
        // (prefix 0) and request 3's chunk again.
        const int32_t n1 = lens[1];
        std::vector<float> q1 = normal(401, (size_t)n1 * H * D), w1((size_t)n1 * H * D);
        for (int32_t i = 0; i < n1; ++i)
            orc_paged_attention(&op, q1.data() + (size_t)i * H * D, tables[1].data(), (int32_t)tables[1].size(),
                                i + 1, H, w1.data() + (size_t)i * H * D);
        float *q1d, *o1d, *qcd, *ocd;
        CHECK(hipMalloc(&q1d, q1.size() * 4) == hipSuccess && hipMalloc(&o1d, q1.size() * 4) == hipSuccess &&
                  hipMalloc(&qcd, qc.size() * 4) == hipSuccess && hipMalloc(&ocd, qc.size() * 4) == hipSuccess,
              "malloc");
        CHECK(hipMemcpy(q1d, q1.data(), q1.size() * 4, hipMemcpyHostToDevice) == hipSuccess &&
                  hipMemcpy(qcd, qc.data(), qc.size() * 4, hipMemcpyHostToDevice) == hipSuccess,
              "copy");
        paged_prefill_batch({{q1d, &tables[1], 0, n1, o1d}, {qcd, &tables[3], pre, n, ocd}}, m.block_pool(), H,
                            HKV, D, layer);
        CHECK(hipDeviceSynchronize() == hipSuccess, "sync");
        std::vector<float> g1(q1.size());
        CHECK(hipMemcpy(g1.data(), o1d, g1.size() * 4, hipMemcpyDeviceToHost) == hipSuccess &&
                  hipMemcpy(gc.data(), ocd, gc.size() * 4, hipMemcpyDeviceToHost) == hipSuccess,
              "copy");
        close(g1.data(), w1.data(), g1.size(), tol, rtol, "paged_prefill_batch chunk 0, device buffers");
        close(gc.data(), wc.data(), gc.size(), tol, rtol, "paged_prefill_batch chunk 1, device buffers");
        // 8. one step with both kinds of work (paged_attention_step): the four
        // decode queries (host buffers) and the two chunks (host buffers).
        {
            std::vector<float> gd((size_t)4 * H * D, NAN), g1s(q1.size(), NAN), gcs(qc.size(), NAN);
            std::vector<const float*> sq;
            std::vector<float*> so;
            std::vector<const std::vector<int32_t>*> stb;
            std::vector<int32_t> ssl;
            for (int r = 0; r < 4; ++r) {
                sq.push_back(q.data() + (size_t)r * H * D);
                so.push_back(gd.data() + (size_t)r * H * D);
                stb.push_back(&tables[r]);
                ssl.push_back(lens[r]);
            }
            paged_attention_step(sq, stb, ssl, so,
                                 {{q1.data(), &tables[1], 0, n1, g1s.data()}, {qc.data(), &tables[3], pre, n, gcs.data()}},
                                 m.block_pool(), H, HKV, D, layer);
            close(gd.data(), want.data(), gd.size(), tol, rtol, "paged_attention_step decodes, host buffers");
            close(g1s.data(), w1.data(), g1s.size(), tol, rtol, "paged_attention_step chunk 0, host buffers");
            close(gcs.data(), wc.data(), gcs.size(), tol, rtol, "paged_attention_step chunk 1, host buffers");
            // the same step on device buffers (queued on the pool's stream)
            CHECK(hipMemset(od, 0xFF, q.size() * 4) == hipSuccess && hipMemset(o1d, 0xFF, q1.size() * 4) == hipSuccess &&
                      hipMemset(ocd, 0xFF, qc.size() * 4) == hipSuccess,
                  "poison");
            paged_attention_step(qp, tp, sl, opp, {{q1d, &tables[1], 0, n1, o1d}, {qcd, &tables[3], pre, n, ocd}},
                                 m.block_pool(), H, HKV, D, layer);
            CHECK(hipDeviceSynchronize() == hipSuccess, "sync");
            CHECK(hipMemcpy(gd.data(), od, gd.size() * 4, hipMemcpyDeviceToHost) == hipSuccess &&
                      hipMemcpy(g1s.data(), o1d, g1s.size() * 4, hipMemcpyDeviceToHost) == hipSuccess &&
                      hipMemcpy(gcs.data(), ocd, gcs.size() * 4, hipMemcpyDeviceToHost) == hipSuccess,
                  "copy");
            close(gd.data(), want.data(), gd.size(), tol, rtol, "paged_attention_step decodes, device buffers");
            close(g1s.data(), w1.data(), g1s.size(), tol, rtol, "paged_attention_step chunk 0, device buffers");
            close(gcs.data(), wc.data(), gcs.size(), tol, rtol, "paged_attention_step chunk 1, device buffers");
        }
        for (float* p : {q1d, o1d, qcd, ocd}) (void)hipFree(p);
    }
    (void)hipFree(qd);
    (void)hipFree(od);
}

// Two pools on two streams, device q / out, calls queued back to back with no
// wait between them: each pool stages its own arguments, so neither call can
// see the other's tables, lengths or partials.
void test_two_pools_two_streams() {
    const int32_t L = 1, H = 64, HKV = 8, D = 80, kv = HKV * D, NB = 120;
    const int32_t lens[2][3] = {{1000, 33, 400}, {17, 1500, 260}};
    hipStream_t st[2];
    CHECK(hipStreamCreate(&st[0]) == hipSuccess && hipStreamCreate(&st[1]) == hipSuccess, "streams");
    KVCacheManager m0(L, kv, NB, KVDtype::FP16, D), m1(L, kv, NB, KVDtype::FP16, D);
    KVCacheManager* ms[2] = {&m0, &m1};
    std::vector<HostLayer> hosts{HostLayer(KVDtype::FP16, NB, L, HKV, D), HostLayer(KVDtype::FP16, NB, L, HKV, D)};
    std::vector<std::vector<int32_t>> tables[2];
    std::vector<float> want[2], q[2];
    float *qd[2], *od[2];
    for (int i = 0; i < 2; ++i) {
        tables[i].resize(3);
        for (int r = 0; r < 3; ++r) {
            CHECK(ms[i]->alloc_blocks((lens[i][r] + 15) / 16, tables[i][r]), "alloc");
            auto k = normal(500 + 10 * i + r, (size_t)lens[i][r] * kv), v = normal(600 + 10 * i + r, (size_t)lens[i][r] * kv);
            write_kv_prefill(*ms[i], tables[i][r], lens[i][r], 0, k.data(), v.data());
            for (int32_t p = 0; p < lens[i][r]; ++p)
                hosts[i].write(tables[i][r][p / 16], 0, p % 16, k.data() + (size_t)p * kv, v.data() + (size_t)p * kv);
        }
        ms[i]->block_pool().set_stream(st[i]);
        q[i] = normal(700 + i, (size_t)3 * H * D);
        want[i].resize(q[i].size());
        orc_pool op = hosts[i].pool(0);
        for (int r = 0; r < 3; ++r)
            orc_paged_attention(&op, q[i].data() + (size_t)r * H * D, tables[i][r].data(),
                                (int32_t)tables[i][r].size(), lens[i][r], H, want[i].data() + (size_t)r * H * D);
        CHECK(hipMalloc(&qd[i], q[i].size() * 4) == hipSuccess && hipMalloc(&od[i], q[i].size() * 4) == hipSuccess,
              "malloc");
        CHECK(hipMemcpy(qd[i], q[i].data(), q[i].size() * 4, hipMemcpyHostToDevice) == hipSuccess, "copy");
    }
    CHECK(hipDeviceSynchronize() == hipSuccess, "sync");
    for (int rep = 0; rep < 4; ++rep)
        for (int i = 0; i < 2; ++i) {
            std::vector<const float*> qp;
            std::vector<float*> opp;
            std::vector<const std::vector<int32_t>*> tp;
            std::vector<int32_t> sl;
            for (int r = 0; r < 3; ++r) {
                qp.push_back(qd[i] + (size_t)r * H * D);
                opp.push_back(od[i] + (size_t)r * H * D);
                tp.push_back(&tables[i][r]);
                sl.push_back(lens[i][r]);
            }
            paged_attention_batch(qp, tp, sl, ms[i]->block_pool(), H, HKV, D, 0, opp);
        }
    CHECK(hipDeviceSynchronize() == hipSuccess, "sync");
    for (int i = 0; i < 2; ++i) {
        std::vector<float> got(q[i].size());
        CHECK(hipMemcpy(got.data(), od[i], got.size() * 4, hipMemcpyDeviceToHost) == hipSuccess, "copy");
        close(got.data(), want[i].data(), got.size(), 2e-3, 1e-2,
              i ? "two pools on two streams: pool 1" : "two pools on two streams: pool 0");
        (void)hipFree(qd[i]);
        (void)hipFree(od[i]);
        ms[i]->block_pool().set_stream(nullptr);
    }
    (void)hipStreamDestroy(st[0]);
    (void)hipStreamDestroy(st[1]);
}


// read_kv_prefill on rows whose byte count is not a multiple of 4 (FP8 and
// FP16 pools of odd kv_dim) and on an INT8 pool with more kv heads (300) than
// the gather's workgroup has threads: every byte and scale of each row comes
// back.  The pages are filled with raw bytes, so the expected rows are the
// oracle's decode of exactly those bytes.
void test_read_kv_prefill_odd_rows() {
    struct Case { KVDtype dt; int32_t kv, hd; const char* name; };
    const Case cases[] = {{KVDtype::FP8_E4M3, 37, 37, "FP8 kv_dim 37"},
                          {KVDtype::FP16, 37, 37, "FP16 kv_dim 37"},
                          {KVDtype::INT8, 300, 1, "INT8 300 kv heads of dim 1"}};
    for (const Case& cs : cases) {
        const int32_t L = 2, NB = 4, layer = 1, seq = 40;
        KVCacheManager m(L, cs.kv, NB, cs.dt, cs.hd);
        const BlockPool& p = m.block_pool();
        const int32_t esz = kv_elem_size(cs.dt), hkv = cs.kv / cs.hd;
        const size_t slab = (size_t)16 * cs.kv * esz;
        std::mt19937 rng(7);
        std::vector<std::vector<uint8_t>> kb(NB), vb(NB);
        std::vector<std::vector<uint16_t>> ksc(NB), vsc(NB);
        for (int32_t b = 0; b < NB; ++b) {
            kb[b].resize(slab);
            vb[b].resize(slab);
            for (size_t i = 0; i < slab; ++i) {
                kb[b][i] = (uint8_t)rng();
                vb[b][i] = (uint8_t)rng();
            }
            if (cs.dt == KVDtype::FP8_E4M3)  // keep codes finite (exponent field below 15)
                for (size_t i = 0; i < slab; ++i) {
                    kb[b][i] &= 0xF7;
                    vb[b][i] &= 0xF7;
                }
            if (cs.dt == KVDtype::FP16)  // finite halves: clear the top exponent bit
                for (size_t i = 1; i < slab; i += 2) {
                    kb[b][i] &= 0xBF;
                    vb[b][i] &= 0xBF;
                }
            CHECK(hipMemcpy(const_cast<uint8_t*>(p.get_k_raw(b, layer)), kb[b].data(), slab, hipMemcpyHostToDevice) == hipSuccess, "fill K");
            CHECK(hipMemcpy(const_cast<uint8_t*>(p.get_v_raw(b, layer)), vb[b].data(), slab, hipMemcpyHostToDevice) == hipSuccess, "fill V");
            if (cs.dt == KVDtype::INT8) {
                ksc[b].resize((size_t)hkv * 16);
                vsc[b].resize((size_t)hkv * 16);
                for (size_t i = 0; i < ksc[b].size(); ++i) {
                    ksc[b][i] = (uint16_t)(0x2000 + (rng() & 0x1FFF));  // positive normal halves
                    vsc[b][i] = (uint16_t)(0x2000 + (rng() & 0x1FFF));
                }
                const vcpp_kv_pages pg = p.pages(layer);
                CHECK(hipMemcpy(const_cast<uint16_t*>(pg.k_scale) + b * pg.scale_block_stride, ksc[b].data(), ksc[b].size() * 2, hipMemcpyHostToDevice) == hipSuccess, "fill K scales");
                CHECK(hipMemcpy(const_cast<uint16_t*>(pg.v_scale) + b * pg.scale_block_stride, vsc[b].data(), vsc[b].size() * 2, hipMemcpyHostToDevice) == hipSuccess, "fill V scales");
            }
        }
        const std::vector<int32_t> table = {2, 0, 3};  // 40 positions over 3 blocks
        std::vector<float> rk((size_t)seq * cs.kv, -7.f), rv((size_t)seq * cs.kv, -7.f);
        read_kv_prefill(p, table, seq, layer, hkv, cs.hd, rk.data(), rv.data());
        for (int32_t pos = 0; pos < seq; ++pos) {
            const int32_t b = table[pos / 16], slot = pos % 16;
            for (int32_t j = 0; j < cs.kv; ++j) {
                const size_t e = (size_t)slot * cs.kv + j;
                float wk, wv;
                if (cs.dt == KVDtype::FP8_E4M3) {
                    wk = orc_fp8_decode(kb[b][e]);
                    wv = orc_fp8_decode(vb[b][e]);
                } else if (cs.dt == KVDtype::FP16) {
                    wk = orc_f16_decode((uint16_t)(kb[b][2 * e] | kb[b][2 * e + 1] << 8));
                    wv = orc_f16_decode((uint16_t)(vb[b][2 * e] | vb[b][2 * e + 1] << 8));
                } else {
                    const int32_t h = j / cs.hd;
                    wk = (float)(int8_t)kb[b][e] * orc_f16_decode(ksc[b][h * 16 + slot]);
                    wv = (float)(int8_t)vb[b][e] * orc_f16_decode(vsc[b][h * 16 + slot]);
                }
                CHECK(rk[(size_t)pos * cs.kv + j] == wk && rv[(size_t)pos * cs.kv + j] == wv,
                      "%s: read_kv_prefill pos %d dim %d", cs.name, pos, j);
            }
        }
        std::printf("ok   read_kv_prefill, %-42s (bit-exact)\n", cs.name);
    }
}

}  // namespace

int main() {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n == 0) {
        std::printf("no GPU\n");
        return 2;
    }
    test_bookkeeping();
    const KVDtype all[] = {KVDtype::FP32, KVDtype::FP16, KVDtype::FP8_E4M3, KVDtype::INT8};
    static const char* names[] = {"FP32", "FP16", "FP8", "INT8"};
    for (KVDtype dt : all) test_write_read(dt);
    for (KVDtype dt : all) test_swap(dt);
    for (KVDtype dt : all) {
        std::printf("---- attention on %s pages\n", names[(int)dt]);
        test_attention(dt);
    }
    test_two_pools_two_streams();
    test_read_kv_prefill_odd_rows();
    std::printf("ALL PASSED (%d checks)\n", g_checks);
    return 0;
}
