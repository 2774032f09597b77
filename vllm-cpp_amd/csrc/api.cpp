// api.cpp -- extern "C" entry points of libvcpp_attn.so (include/vcpp_attention.h).
//
// Argument checking, workspace sizing and the v1 shims live here; the kernels
// live in decode.hip / prefill.hip.  Errors never terminate the process: v2
// returns a VCPP_E* code, v1 (void, like cuda/attention.h) records it, and
// both leave the message in a thread-local string for vcpp_last_error().
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "decode.h"
#include "prefill.h"
#include "dense.h"
#include "kv_write.h"
#include "qk_prep.h"
#include "vcpp_attention.h"

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

}  // namespace

#ifdef VCPP_GATHER_DUMP
// Checker builds: the dump buffer every following decode / prefill launch writes.
int32_t* g_gather_dump = nullptr;
int64_t g_gather_stride = 0;
#endif

namespace vcpp {
// Records a failure for vcpp_last_error() from other sources of the library.
int record_error(int code, const char* msg) { return fail(code, "%s", msg); }
}  // namespace vcpp

namespace {

bool eps_ok(float eps) { return std::isfinite(eps) && eps >= 0.f; }

int hip_fail(hipError_t e, const char* what) {
    return fail(VCPP_E_HIP, "%s: %s", what, hipGetErrorString(e));
}

constexpr int32_t kDefaultPartition = 256;
constexpr int32_t kMaxPartition = 1024;
// fp16/int8 split: at least one 64-token step per range; grid.x limit.
constexpr int64_t kMinTilesPerRange = 4;
constexpr int64_t kMaxRanges = 1 << 20;
// Page-staged decode: the balanced split charges each sequence this many
// 16-token tiles for starting it (its Q load, the previous one's outputs).  A
// sweep of 0, 2, 4, 6, 8 on BASELINE config 2 put the step's best at 2; byte
// pages (half the bytes per tile) measured the same at 2, 3 and 4.
constexpr int kSwitchTiles = 2;
// Byte pages' alternating ranges: the first dispatch round's share of each
// pair of neighbouring ranges, / 256, per page dtype.  int8 on BASELINE
// config 5: 164 (step 0.233 ms against 0.238 at 180, 2.6 % over equal
// ranges); FP8 on config 2's sequences: 180 (kernel 40.7-41.1 us against
// 41.3 at 164 and 42.1-42.3 with equal ranges).
constexpr int kRoundShareI8 = 164;
constexpr int kRoundShareFp8 = 180;

int32_t ceil_div(int64_t a, int64_t b) { return (int32_t)((a + b - 1) / b); }

int32_t num_parts(int32_t max_context_len, int32_t partition) {
    return max_context_len <= 0 ? 1 : ceil_div(max_context_len, partition);
}

size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

// Compute units of the current device (cached per device).
int device_cus() {
    static int cus[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cus[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            n <= 0)
            n = 256;
        cus[dev] = n;
    }
    return cus[dev];
}

// The mixed step's side streams (default priority) and fork / join events:
// one set per (device, caller stream), made on first use and kept for the
// process.  Each caller stream forks onto its own side stream, so steps on
// different streams never share one (a side stream joined to one stream's
// graph capture is never used by another stream meanwhile).  Calls on one
// stream are serialised by the caller, as for every entry point; g_fork_mu
// guards only the table.
std::mutex g_fork_mu;

const vcpp::MergeFork* merge_fork(hipStream_t stream) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0) return nullptr;
    // Only for a stream of the current device (the side stream is made there).
    hipDevice_t sdev = -1;
    if (stream && (hipStreamGetDevice(stream, &sdev) != hipSuccess || sdev != dev)) {
        (void)hipGetLastError();
        return nullptr;
    }
    struct Entry {
        vcpp::MergeFork mf;
        bool ok;
    };
    static std::map<std::pair<int, hipStream_t>, Entry> table;
    std::lock_guard<std::mutex> lock(g_fork_mu);
    auto it = table.find({dev, stream});
    if (it == table.end()) {
        Entry en{};
        bool ok = hipStreamCreateWithFlags(&en.mf.side, hipStreamNonBlocking) == hipSuccess;
        ok = ok && hipEventCreateWithFlags(&en.mf.fork, hipEventDisableTiming) == hipSuccess;
        ok = ok && hipEventCreateWithFlags(&en.mf.join, hipEventDisableTiming) == hipSuccess;
        if (!ok) (void)hipGetLastError();
        en.ok = ok;
        it = table.emplace(std::make_pair(dev, stream), en).first;
    }
    return it->second.ok ? &it->second.mf : nullptr;
}

// VCPP_NO_MERGE_FORK=1: the mixed step's merge stays on the caller's stream
// (for measurement).
bool no_merge_fork() {
    const char* e = std::getenv("VCPP_NO_MERGE_FORK");
    return e && e[0] == '1';
}

// Launch geometry and workspace layout of one decode call.
struct DecodePlan {
    int32_t num_wg = 0;      // fp16/int8: workgroup ranges per kv-head group
    bool page_mode = false;  // fp16/int8, Hkv 8: page-staged kernel
    int32_t page_grid = 0;   // page mode: workgroups (one per range, or a run of ranges each)
    int32_t partition = 0;   // fp32: tokens per partition
    int32_t max_parts = 0;   // fp32: partitions per sequence
    int32_t g1 = 0, g1_share = 0;  // page mode: unequal ranges (see DecodeParams)
    size_t off_o = 0, off_ml = 0, bytes = 0;
};

// fused_grid > 0: the decode side of the fused mixed step, whose decode
// workers (fused_grid per kv-head group of 4) walk the balanced split.
DecodePlan plan_decode(const vcpp_kv_pages* kv, int32_t num_seqs, int32_t num_heads,
                       int32_t max_context_len, int32_t partition_size, int32_t fused_grid = 0) {
    DecodePlan pl;
    const int D = kv->head_dim;
    if (kv->dtype == VCPP_KV_F32) {
        // Default: partitions of 32..256 tokens, so that the workgroups
        // (partition, sequence, kv head, 8-head chunk) fill about two per CU.
        int32_t dflt = kDefaultPartition;
        if (partition_size == 0 && max_context_len > 0 && kv->num_kv_heads > 0 && num_heads > 0) {
            const int64_t chunks = (int64_t)kv->num_kv_heads * ((num_heads / kv->num_kv_heads + 7) / 8);
            const int64_t want = (int64_t)max_context_len * num_seqs * chunks / (2 * (int64_t)device_cus());
            dflt = (int32_t)std::min<int64_t>(kDefaultPartition, std::max<int64_t>(32, (want + 31) / 32 * 32));
        }
        pl.partition = partition_size > 0 ? partition_size : dflt;
        pl.max_parts = num_parts(max_context_len, pl.partition);
        if (pl.max_parts > 1) {
            const size_t rows = (size_t)num_seqs * pl.max_parts * num_heads;
            pl.off_o = 0;
            pl.off_ml = align256(rows * D * sizeof(float));
            pl.bytes = pl.off_ml + align256(rows * sizeof(float2));
        }
        return pl;
    }
    const int group = num_heads / kv->num_kv_heads;
    const int pairs = kv->num_kv_heads * ((group + 7) / 8);
    const int wpw = pairs < 4 ? pairs : 4;
    const int groups = vcpp::decode_group_count(pairs);
    // The page-staged kernel (balanced split only) unless VCPP_DECODE_PAGE=0.
    const char* pe = getenv("VCPP_DECODE_PAGE");
    // Its 16-byte DMA of byte pages (and int8 scales) needs 16-byte aligned
    // bases and strides (fp16 pages already must be).
    const bool bytes = kv->dtype == VCPP_KV_I8 || kv->dtype == VCPP_KV_FP8;
    const bool dma_aligned =
        !bytes ||
        (kv->block_stride % 16 == 0 && reinterpret_cast<uintptr_t>(kv->k) % 16 == 0 &&
         reinterpret_cast<uintptr_t>(kv->v) % 16 == 0 &&
         (kv->dtype != VCPP_KV_I8 ||
          (kv->scale_block_stride % 8 == 0 && reinterpret_cast<uintptr_t>(kv->k_scale) % 16 == 0 &&
           reinterpret_cast<uintptr_t>(kv->v_scale) % 16 == 0)));
    pl.page_mode = !(pe && pe[0] == '0') && dma_aligned &&
                   vcpp::decode_page_mode_supported(kv->dtype, kv->num_kv_heads, group, D,
                                                    kv->block_size);
    // Ranges that are all resident at once: 2 waves per SIMD, 4 SIMDs per CU
    // (page mode: 8-wave workgroups that each cover every kv head, one per CU
    // for fp16 pages and two for byte pages).
    const int64_t slots = (int64_t)device_cus() * (8 / wpw);
    // Page mode: each range is walked by num_kv_heads / HW workgroups (one per
    // head group), so ranges = resident workgroups / head groups.
    const int page_hw = vcpp::decode_page_heads(kv->dtype, kv->num_kv_heads, D);
    const int64_t page_slots = (int64_t)device_cus() * vcpp::decode_page_wg_per_cu(kv->dtype, kv->num_kv_heads, D);
    const int64_t page_ranges = page_hw > 0 ? std::max<int64_t>(1, page_slots / (kv->num_kv_heads / page_hw)) : 1;
    int64_t G = pl.page_mode ? page_ranges : slots / groups;
    if (fused_grid > 0) {
        pl.page_mode = true;
        G = fused_grid;
    }
    const int64_t tiles_upper = (int64_t)num_seqs * ((max_context_len + 15) / 16);
    if (partition_size > 0) {
        G = (tiles_upper * 16 + partition_size - 1) / partition_size;
    } else {
        G = std::min<int64_t>(G, (tiles_upper + kMinTilesPerRange - 1) / kMinTilesPerRange);
    }
    G = std::max<int64_t>(1, std::min<int64_t>(G, kMaxRanges));
    pl.num_wg = (int32_t)G;
    // Page mode: the balanced split has one resident workgroup per range;
    // fixed partitions (more ranges than fit at once) are walked by that many
    // workgroups, each taking a contiguous run of ranges.
    pl.page_grid = pl.page_mode ? (int32_t)std::min<int64_t>(G, fused_grid > 0 ? fused_grid : page_ranges)
                                : pl.num_wg;
    // Byte pages at two workgroups per CU: the dispatcher places ids 0 ..
    // CUs - 1 first, and those start their rings while the second round's
    // workgroups still build their tile lists.  Ranges alternate in size
    // along the split axis, the first round's taking kRoundShareI8 (int8) or
    // kRoundShareFp8 (FP8) 256ths of each pair of neighbours
    // (VCPP_DECODE_ROUND_SHARE overrides; 128: equal ranges).
    if (pl.page_mode && fused_grid == 0 && partition_size == 0 && pl.page_grid == pl.num_wg &&
        vcpp::decode_page_wg_per_cu(kv->dtype, kv->num_kv_heads, D) == 2 && bytes &&
        pl.num_wg == page_ranges && pl.num_wg % 2 == 0) {
        const char* rs = getenv("VCPP_DECODE_ROUND_SHARE");
        const int share = rs ? atoi(rs) : kv->dtype == VCPP_KV_FP8 ? kRoundShareFp8 : kRoundShareI8;
        if (share > 0 && share < 256 && share != 128) {
            pl.g1 = pl.num_wg / 2;
            pl.g1_share = share;
        }
    }
    pl.off_o = 0;
    const size_t blocks = (size_t)G * 2 * pairs;  // [range][slot][kv-head slot]
    pl.off_ml = pl.off_o + align256(blocks * 8 * D * sizeof(float));
    pl.bytes = pl.off_ml + align256(blocks * 16 * sizeof(float2));
    return pl;
}

int check_pages(const vcpp_kv_pages* kv) {
    if (!kv) return fail(VCPP_E_INVALID, "kv pages descriptor is NULL");
    if (kv->dtype != VCPP_KV_F32 && kv->dtype != VCPP_KV_F16 && kv->dtype != VCPP_KV_I8 &&
        kv->dtype != VCPP_KV_FP8)
        return fail(VCPP_E_INVALID, "unknown kv dtype %d", kv->dtype);
    if (kv->block_size <= 0 || kv->block_size % 16 != 0)
        return fail(VCPP_E_UNSUPPORTED, "block_size %d is not a positive multiple of 16",
                    kv->block_size);
    if (kv->num_kv_heads <= 0) return fail(VCPP_E_INVALID, "num_kv_heads must be positive");
    if (kv->num_blocks < 0) return fail(VCPP_E_INVALID, "num_blocks must be >= 0");
    if (kv->head_dim > 256 || !vcpp::decode_head_dim_supported(kv->dtype, kv->head_dim))
        return fail(VCPP_E_UNSUPPORTED, "head_dim %d not supported for kv dtype %d",
                    kv->head_dim, kv->dtype);
    if (kv->num_blocks > 0 && (!kv->k || !kv->v))
        return fail(VCPP_E_INVALID, "K/V page base is NULL");
    const int64_t esize = kv->dtype == VCPP_KV_F32 ? 4 : kv->dtype == VCPP_KV_F16 ? 2 : 1;
    const int64_t align = esize == 1 ? 8 : 16;
    if ((kv->block_stride * esize) % align != 0 || (kv->head_dim * esize) % align != 0 ||
        (reinterpret_cast<uintptr_t>(kv->k) % align) != 0 ||
        (reinterpret_cast<uintptr_t>(kv->v) % align) != 0)
        return fail(VCPP_E_INVALID, "K/V pages must be %lld-byte aligned (bases and strides)",
                    (long long)align);
    if (kv->block_stride < (int64_t)kv->block_size * kv->num_kv_heads * kv->head_dim)
        return fail(VCPP_E_INVALID, "block_stride %lld smaller than one page",
                    (long long)kv->block_stride);
    if (kv->dtype == VCPP_KV_I8) {
        if (kv->num_blocks > 0 && (!kv->k_scale || !kv->v_scale))
            return fail(VCPP_E_INVALID, "int8 pages need k_scale and v_scale");
        if (kv->scale_block_stride < (int64_t)kv->num_kv_heads * kv->block_size ||
            kv->scale_block_stride % 4 != 0 ||
            reinterpret_cast<uintptr_t>(kv->k_scale) % 8 != 0 ||
            reinterpret_cast<uintptr_t>(kv->v_scale) % 8 != 0)
            return fail(VCPP_E_INVALID,
                        "scale pages must be 8-byte aligned with scale_block_stride a multiple "
                        "of 4 and >= num_kv_heads * block_size");
    }
    return VCPP_OK;
}

}  // namespace

// ---- v2: query / key preparation ------------------------------------------

int vcpp_qk_norm_rope(float* q, float* k, int32_t num_tokens, int32_t num_heads,
                      int32_t num_kv_heads, int32_t head_dim, const float* q_norm_weight,
                      const float* k_norm_weight, float eps, const int32_t* positions,
                      const float* inv_freq, int32_t inv_freq_size, int32_t style, void* stream) {
    g_last_error.clear();
    if (num_tokens < 0 || num_heads <= 0 || (k && num_kv_heads <= 0))
        return fail(VCPP_E_INVALID, "num_tokens %d, num_heads %d, num_kv_heads %d", num_tokens,
                    num_heads, num_kv_heads);
    if (head_dim <= 0 || head_dim % 2 != 0 || head_dim > 256)
        return fail(VCPP_E_UNSUPPORTED, "head_dim %d must be even and <= 256", head_dim);
    if (style != VCPP_ROPE_INTERLEAVED && style != VCPP_ROPE_HALF)
        return fail(VCPP_E_INVALID, "unknown rope style %d", style);
    if (positions && (!inv_freq || inv_freq_size <= 0))
        return fail(VCPP_E_INVALID, "rotation needs inv_freq with inv_freq_size > 0");
    if (!eps_ok(eps)) return fail(VCPP_E_INVALID, "eps must be finite and >= 0");
    if (num_tokens == 0) return VCPP_OK;
    if (!q) return fail(VCPP_E_INVALID, "q is NULL");
    if (reinterpret_cast<uintptr_t>(q) % 8 != 0 || reinterpret_cast<uintptr_t>(k) % 8 != 0)
        return fail(VCPP_E_INVALID, "q and k must be 8-byte aligned");
    const int64_t rows = (int64_t)num_tokens * num_heads + (k ? (int64_t)num_tokens * num_kv_heads : 0);
    if (rows > (int64_t)INT32_MAX * 4) return fail(VCPP_E_UNSUPPORTED, "too many rows");
    vcpp::QkPrepParams p{};
    p.t[0] = {q, q_norm_weight, num_heads};
    p.t[1] = {k, k_norm_weight, k ? num_kv_heads : 0};
    p.num_tokens = num_tokens;
    p.head_dim = head_dim;
    p.eps = eps;
    p.positions = positions;
    p.inv_freq = inv_freq;
    p.inv_freq_size = inv_freq_size;
    p.style = style;
    const hipError_t e = vcpp::launch_qk_prep(p, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "qk_prep launch");
    return VCPP_OK;
}

int vcpp_rope(float* x, int32_t num_tokens, int32_t num_heads, int32_t head_dim,
              const int32_t* positions, const float* inv_freq, int32_t inv_freq_size,
              int32_t style, void* stream) {
    if (!positions && num_tokens > 0) {
        g_last_error.clear();
        return fail(VCPP_E_INVALID, "positions is NULL");
    }
    return vcpp_qk_norm_rope(x, nullptr, num_tokens, num_heads, 0, head_dim, nullptr, nullptr, 0.f,
                             positions, inv_freq, inv_freq_size, style, stream);
}

int vcpp_head_norm(float* x, const float* weight, float eps, int32_t num_rows, int32_t head_dim,
                   void* stream) {
    if (!weight && num_rows > 0) {
        g_last_error.clear();
        return fail(VCPP_E_INVALID, "weight is NULL");
    }
    // Rows go to the kernel's waves in runs of up to 16 (one "token" each).
    int run = 16;
    while (run > 1 && num_rows % run != 0) run /= 2;
    return vcpp_qk_norm_rope(x, nullptr, num_rows / run, run, 0, head_dim, weight, nullptr, eps,
                             nullptr, nullptr, 0, VCPP_ROPE_INTERLEAVED, stream);
}

// ---- v1 shims: library-owned buffers ---------------------------------------

namespace {
// Library-owned device buffers of the v1 entry points (grown, never shrunk).
struct V1State {
    std::mutex mu;
    void* ws = nullptr;
    size_t ws_bytes = 0;
    int32_t* ctx = nullptr;
    size_t ctx_count = 0;
};
V1State& v1_state() {
    static V1State s;
    return s;
}

// Whole blocks of block_bytes from base to the end of the device allocation
// that contains it (INT32_MAX when the runtime does not know the pointer).
int64_t v1_num_blocks(const void* base, int64_t block_bytes) {
    if (!base || block_bytes <= 0) return 0;
    hipDeviceptr_t start = nullptr;
    size_t size = 0;
    if (hipMemGetAddressRange(&start, &size, const_cast<void*>(base)) != hipSuccess || !start) {
        (void)hipGetLastError();
        return INT32_MAX;
    }
    const int64_t left = (int64_t)((const char*)start + size - (const char*)base);
    return std::min<int64_t>(left / block_bytes, INT32_MAX);
}
}  // namespace


extern "C" {

const char* vcpp_last_error(void) { return g_last_error.c_str(); }

#ifdef VCPP_GATHER_DUMP
// Checker builds only (not declared in include/): set (or clear, with NULL)
// the device buffer [rows][stride][2] int32 that decode and prefill launches
// record their (block, slot) gather indices into.
void vcpp_debug_gather_dump(int32_t* buf, int64_t stride) {
    g_gather_dump = buf;
    g_gather_stride = buf ? stride : 0;
}
#endif

const char* vcpp_version(void) { return "vcpp_attn 0.1 gfx950"; }

size_t vcpp_decode_workspace_size(const vcpp_kv_pages* kv, int32_t num_seqs, int32_t num_heads,
                                  int32_t max_context_len, int32_t partition_size) {
    if (!kv || kv->num_kv_heads <= 0 || num_heads <= 0 || num_seqs <= 0) return 0;
    return plan_decode(kv, num_seqs, num_heads, max_context_len, partition_size).bytes;
}

}  // extern "C"

namespace {

// Validates a decode call's arguments (not its workspace).
int check_decode(const vcpp_kv_pages* kv, const float* q, float* out, const int32_t* block_tables,
                 int32_t max_blocks_per_seq, const int32_t* context_lens, int32_t num_seqs,
                 int32_t max_context_len, int32_t num_heads, int32_t partition_size) {
    int rc = check_pages(kv);
    if (rc != VCPP_OK) return rc;
    if (num_seqs < 0) return fail(VCPP_E_INVALID, "num_seqs must be >= 0");
    if (num_seqs == 0) return VCPP_OK;
    if (!q || !out || !context_lens) return fail(VCPP_E_INVALID, "q/out/context_lens is NULL");
    if (max_blocks_per_seq < 0) return fail(VCPP_E_INVALID, "max_blocks_per_seq must be >= 0");
    if (max_blocks_per_seq > 0 && !block_tables)
        return fail(VCPP_E_INVALID, "block_tables is NULL");
    if (num_heads <= 0 || num_heads % kv->num_kv_heads != 0)
        return fail(VCPP_E_INVALID, "num_heads %d is not a positive multiple of num_kv_heads %d",
                    num_heads, kv->num_kv_heads);
    if (max_context_len < 0) return fail(VCPP_E_INVALID, "max_context_len must be >= 0");
    if (partition_size < 0 || partition_size % 16 != 0 || partition_size > kMaxPartition)
        return fail(VCPP_E_INVALID, "partition_size %d must be 0 or a multiple of 16 <= %d",
                    partition_size, kMaxPartition);
    if (kv->dtype != VCPP_KV_F32 && (int64_t)kv->num_kv_heads * ((num_heads / kv->num_kv_heads + 7) / 8) > 65535 * 8)
        return fail(VCPP_E_UNSUPPORTED, "too many kv heads");
    if (kv->dtype == VCPP_KV_F32 && (int64_t)kv->num_kv_heads * ((num_heads / kv->num_kv_heads + 7) / 8) > 65535)
        return fail(VCPP_E_UNSUPPORTED, "too many kv heads");
    if (kv->dtype == VCPP_KV_F32 && num_seqs > 65535)
        return fail(VCPP_E_UNSUPPORTED, "fp32 pages: too many sequences (%d)", num_seqs);
    return VCPP_OK;
}

// The launch parameters of a checked decode call under plan pl.
vcpp::DecodeParams decode_params(const vcpp_kv_pages* kv, const float* q, float* out,
                                 const int32_t* block_tables, int32_t max_blocks_per_seq,
                                 const int32_t* table_lens, const int32_t* context_lens, int32_t num_seqs,
                                 int32_t max_context_len, int32_t num_heads, int32_t partition_size,
                                 const DecodePlan& pl, void* workspace) {
    vcpp::DecodeParams p{};
    p.k = kv->k;
    p.v = kv->v;
    p.k_scale = kv->k_scale;
    p.v_scale = kv->v_scale;
    p.num_blocks = kv->num_blocks;
    p.block_stride = kv->block_stride;
    p.scale_block_stride = kv->scale_block_stride;
    p.block_size = kv->block_size;
    p.num_kv_heads = kv->num_kv_heads;
    p.head_dim = kv->head_dim;
    p.kv_dtype = kv->dtype;
    p.q = q;
    p.out = out;
    p.num_heads = num_heads;
    p.num_seqs = num_seqs;
    p.group = num_heads / kv->num_kv_heads;
    p.qchunks = (p.group + 7) / 8;
    p.pairs = kv->num_kv_heads * p.qchunks;
    p.block_tables = block_tables;
    p.table_lens = table_lens;
    p.context_lens = context_lens;
    p.max_blocks = max_blocks_per_seq;
    char* ws = static_cast<char*>(workspace);
    p.partition = pl.partition;
    p.max_parts = pl.max_parts;
    p.num_wg = pl.num_wg;
    p.page_mode = pl.page_mode ? 1 : 0;
    p.page_grid = pl.page_grid;
    p.g1 = pl.g1;
    p.g1_share = pl.g1_share;
    // Switch units only for the balanced page split (the merge kernel maps
    // tiles to ranges on the same axis).
    p.switch_tiles = pl.page_mode && partition_size == 0 ? kSwitchTiles : 0;
    p.ctx_cap = max_context_len;
    if (pl.bytes > 0) {
        p.ws_o = reinterpret_cast<float*>(ws + pl.off_o);
        p.ws_ml = reinterpret_cast<float2*>(ws + pl.off_ml);
    }
    {
        const char* e = getenv("VCPP_DECODE_PIPELINE");
        p.pipeline = e ? atoi(e) : 0;
    }
    p.scale_log2 = (1.0f / std::sqrt((float)kv->head_dim)) * 1.4426950408889634f;
#ifdef VCPP_GATHER_DUMP
    p.gather_dump = g_gather_dump;
    p.gather_stride = g_gather_stride;
#endif
    return p;
}

int check_workspace(const DecodePlan& pl, void* workspace, size_t workspace_bytes) {
    if (pl.bytes > 0 && (!workspace || workspace_bytes < pl.bytes))
        return fail(VCPP_E_WORKSPACE, "decode needs %zu workspace bytes, got %zu", pl.bytes,
                    workspace ? workspace_bytes : (size_t)0);
    return VCPP_OK;
}

// Validates a prefill call's arguments.
int check_prefill(const vcpp_kv_pages* kv, const uint16_t* q, float* out, const int32_t* block_tables,
                  int32_t max_blocks_per_seq, const int32_t* q_start, const int32_t* prefix_lens,
                  int32_t num_chunks, int32_t max_chunk_len, int32_t num_heads) {
    int rc = check_pages(kv);
    if (rc != VCPP_OK) return rc;
    if (kv->dtype == VCPP_KV_F32)
        return fail(VCPP_E_UNSUPPORTED, "prefill supports fp16, int8 and fp8 pages (got fp32)");
    if (kv->head_dim != 64 && kv->head_dim != 80 && kv->head_dim != 128)
        return fail(VCPP_E_UNSUPPORTED, "prefill head_dim %d (64, 80 or 128)", kv->head_dim);
    if (num_chunks < 0 || max_chunk_len < 0)
        return fail(VCPP_E_INVALID, "num_chunks and max_chunk_len must be >= 0");
    if (num_chunks == 0 || max_chunk_len == 0) return VCPP_OK;
    if (!q || !out || !q_start || !prefix_lens)
        return fail(VCPP_E_INVALID, "q/out/q_start/prefix_lens is NULL");
    if (max_blocks_per_seq <= 0 || !block_tables)
        return fail(VCPP_E_INVALID, "block_tables missing");
    if (num_heads <= 0 || num_heads % kv->num_kv_heads != 0)
        return fail(VCPP_E_INVALID, "num_heads %d is not a positive multiple of num_kv_heads %d",
                    num_heads, kv->num_kv_heads);
    if (num_chunks > 65535) return fail(VCPP_E_UNSUPPORTED, "too many chunks (%d)", num_chunks);
    // The kernel stages a tile's block table in LDS (160 KiB per workgroup).
    if (vcpp::prefill_lds_bytes(kv->dtype, kv->head_dim, max_blocks_per_seq) > 160 * 1024)
        return fail(VCPP_E_UNSUPPORTED, "prefill block table of %d entries exceeds the LDS budget",
                    max_blocks_per_seq);
    if ((int64_t)kv->num_kv_heads * vcpp::prefill_head_groups(num_heads / kv->num_kv_heads) > 65535)
        return fail(VCPP_E_UNSUPPORTED, "too many heads");
    return VCPP_OK;
}

vcpp::PrefillParams prefill_params(const vcpp_kv_pages* kv, const uint16_t* q, float* out,
                                   const int32_t* block_tables, int32_t max_blocks_per_seq,
                                   const int32_t* q_start, const int32_t* prefix_lens, int32_t num_chunks,
                                   int32_t max_chunk_len, int32_t num_heads) {
    vcpp::PrefillParams p{};
    p.k = kv->k;
    p.v = kv->v;
    p.k_scale = kv->k_scale;
    p.v_scale = kv->v_scale;
    p.num_blocks = kv->num_blocks;
    p.block_stride = kv->block_stride;
    p.scale_block_stride = kv->scale_block_stride;
    p.block_size = kv->block_size;
    p.num_kv_heads = kv->num_kv_heads;
    p.head_dim = kv->head_dim;
    p.kv_dtype = kv->dtype;
    p.q = q;
    p.out = out;
    p.num_heads = num_heads;
    p.group = num_heads / kv->num_kv_heads;
    p.head_groups = vcpp::prefill_head_groups(p.group);
    p.block_tables = block_tables;
    p.q_start = q_start;
    p.prefix_lens = prefix_lens;
    p.max_blocks = max_blocks_per_seq;
    p.num_chunks = num_chunks;
    p.max_chunk_len = max_chunk_len;
    p.scale_log2 = (1.0f / std::sqrt((float)kv->head_dim)) * 1.4426950408889634f;
    p.bs_magic = ((1ull << 40) + kv->block_size - 1) / kv->block_size;
    p.splits = 1;
    p.xcd_cus = device_cus() / 8;
    p.rows_cap = (int32_t)std::min<int64_t>((int64_t)num_chunks * max_chunk_len, INT32_MAX);
#ifdef VCPP_GATHER_DUMP
    p.gather_dump = g_gather_dump;
    p.gather_stride = g_gather_stride;
#endif
    return p;
}

// Decode workgroups per kv-head group of the fused mixed step for this call
// (0: run decode and prefill as two launches).  The fused launch is opt-in
// (VCPP_MIXED_FUSED=1): on BASELINE config 5 it measured 388 us against
// 291 us for the two launches.  Its decode side needs the page-staged
// kernel's alignment, its prefill side three workgroups' LDS per CU.
int32_t mixed_grid(const vcpp_kv_pages* kv, int32_t num_heads, int32_t p_max_blocks) {
    const char* e = getenv("VCPP_MIXED_FUSED");
    if (!e || e[0] != '1') return 0;
    if (kv->dtype == VCPP_KV_F32 || num_heads % kv->num_kv_heads != 0) return 0;
    const bool bytes = kv->dtype == VCPP_KV_I8 || kv->dtype == VCPP_KV_FP8;
    if (bytes && (kv->block_stride % 16 != 0 || reinterpret_cast<uintptr_t>(kv->k) % 16 != 0 ||
                  reinterpret_cast<uintptr_t>(kv->v) % 16 != 0))
        return 0;
    if (kv->dtype == VCPP_KV_I8 &&
        (kv->scale_block_stride % 8 != 0 || reinterpret_cast<uintptr_t>(kv->k_scale) % 16 != 0 ||
         reinterpret_cast<uintptr_t>(kv->v_scale) % 16 != 0))
        return 0;
    if (vcpp::mixed_lds_bytes(kv->dtype, kv->head_dim, p_max_blocks) * 3 > 160 * 1024) return 0;
    return vcpp::mixed_decode_grid(kv->dtype, kv->num_kv_heads, num_heads / kv->num_kv_heads,
                                   kv->head_dim, kv->block_size, device_cus());
}

}  // namespace

extern "C" {

int vcpp_paged_decode(const vcpp_kv_pages* kv, const float* q, float* out,
                      const int32_t* block_tables, int32_t max_blocks_per_seq,
                      const int32_t* table_lens, const int32_t* context_lens, int32_t num_seqs,
                      int32_t max_context_len, int32_t num_heads, int32_t partition_size,
                      void* workspace, size_t workspace_bytes, void* stream) {
    g_last_error.clear();
    int rc = check_decode(kv, q, out, block_tables, max_blocks_per_seq, context_lens, num_seqs,
                          max_context_len, num_heads, partition_size);
    if (rc != VCPP_OK || num_seqs == 0) return rc;
    const DecodePlan pl = plan_decode(kv, num_seqs, num_heads, max_context_len, partition_size);
    if (pl.max_parts > 65535) return fail(VCPP_E_UNSUPPORTED, "too many partitions (%d)", pl.max_parts);
    rc = check_workspace(pl, workspace, workspace_bytes);
    if (rc != VCPP_OK) return rc;
    const vcpp::DecodeParams p = decode_params(kv, q, out, block_tables, max_blocks_per_seq, table_lens,
                                               context_lens, num_seqs, max_context_len, num_heads,
                                               partition_size, pl, workspace);
    hipError_t e = vcpp::launch_decode(p, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "decode launch");
    return VCPP_OK;
}

int vcpp_paged_prefill(const vcpp_kv_pages* kv, const uint16_t* q, float* out,
                       const int32_t* block_tables, int32_t max_blocks_per_seq,
                       const int32_t* q_start, const int32_t* prefix_lens, int32_t num_chunks,
                       int32_t max_chunk_len, int32_t num_heads, void* stream) {
    g_last_error.clear();
    int rc = check_prefill(kv, q, out, block_tables, max_blocks_per_seq, q_start, prefix_lens, num_chunks,
                           max_chunk_len, num_heads);
    if (rc != VCPP_OK || num_chunks == 0 || max_chunk_len == 0) return rc;
    const vcpp::PrefillParams p = prefill_params(kv, q, out, block_tables, max_blocks_per_seq, q_start,
                                                 prefix_lens, num_chunks, max_chunk_len, num_heads);
    hipError_t e = vcpp::launch_prefill(p, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "prefill launch");
    return VCPP_OK;
}

// Key parts of a split prefill: enough workgroups to fill two per CU, each
// part at least 16 key blocks (512 keys) of the longest chunk, at most 16.
static int32_t prefill_splits(const vcpp_kv_pages* kv, int32_t num_chunks, int32_t max_chunk_len,
                              int32_t max_prefix_len, int32_t num_heads) {
    if (num_chunks <= 0 || max_chunk_len <= 0 || max_prefix_len < 0) return 1;
    const int64_t qt = kv->head_dim <= 80 ? 64 : 32;  // query rows per workgroup
    const int64_t items = (max_chunk_len + qt - 1) / qt * num_chunks * kv->num_kv_heads *
                          vcpp::prefill_head_groups(num_heads / kv->num_kv_heads);
    const int64_t slots = 2 * (int64_t)device_cus();
    if (items >= slots) return 1;
    const int64_t want = (slots + items - 1) / items;
    const int64_t by_len = ((int64_t)max_prefix_len + max_chunk_len) / (16 * 32);
    return (int32_t)std::max<int64_t>(1, std::min<int64_t>({want, by_len, (int64_t)vcpp::kMaxPrefillSplits}));
}

size_t vcpp_prefill_workspace_size(const vcpp_kv_pages* kv, int32_t num_chunks, int32_t max_chunk_len,
                                   int32_t max_prefix_len, int32_t num_heads) {
    if (!kv || kv->num_kv_heads <= 0 || num_heads <= 0 || num_heads % kv->num_kv_heads != 0) return 0;
    const int32_t s = prefill_splits(kv, num_chunks, max_chunk_len, max_prefix_len, num_heads);
    return vcpp::prefill_split_bytes(s, (int32_t)std::min<int64_t>((int64_t)num_chunks * max_chunk_len, INT32_MAX),
                                     num_heads, kv->head_dim);
}

int vcpp_paged_prefill_split(const vcpp_kv_pages* kv, const uint16_t* q, float* out,
                             const int32_t* block_tables, int32_t max_blocks_per_seq, const int32_t* q_start,
                             const int32_t* prefix_lens, int32_t num_chunks, int32_t max_chunk_len,
                             int32_t max_prefix_len, int32_t num_heads, void* workspace, size_t workspace_bytes,
                             void* stream) {
    g_last_error.clear();
    int rc = check_prefill(kv, q, out, block_tables, max_blocks_per_seq, q_start, prefix_lens, num_chunks,
                           max_chunk_len, num_heads);
    if (rc != VCPP_OK || num_chunks == 0 || max_chunk_len == 0) return rc;
    if (max_prefix_len < 0) return fail(VCPP_E_INVALID, "max_prefix_len must be >= 0");
    vcpp::PrefillParams p = prefill_params(kv, q, out, block_tables, max_blocks_per_seq, q_start, prefix_lens,
                                           num_chunks, max_chunk_len, num_heads);
    p.splits = prefill_splits(kv, num_chunks, max_chunk_len, max_prefix_len, num_heads);
    if ((int64_t)kv->num_kv_heads * p.head_groups * p.splits > 65535)
        return fail(VCPP_E_UNSUPPORTED, "too many heads x key parts");
    if (p.splits > 1) {
        const size_t need = vcpp::prefill_split_bytes(p.splits, p.rows_cap, num_heads, kv->head_dim);
        if (!workspace || workspace_bytes < need)
            return fail(VCPP_E_WORKSPACE, "split prefill needs %zu workspace bytes, got %zu", need,
                        workspace ? workspace_bytes : (size_t)0);
        const size_t rows = (size_t)p.splits * p.rows_cap * num_heads;
        p.ws_o = static_cast<float*>(workspace);
        p.ws_ml = reinterpret_cast<float2*>(static_cast<char*>(workspace) +
                                            ((rows * kv->head_dim * sizeof(float) + 255) & ~size_t(255)));
    }
    hipError_t e = vcpp::launch_prefill(p, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "prefill launch");
    return VCPP_OK;
}

size_t vcpp_mixed_workspace_size(const vcpp_kv_pages* kv, int32_t num_seqs, int32_t num_heads,
                                 int32_t max_context_len, int32_t max_blocks_per_chunk) {
    if (!kv || kv->num_kv_heads <= 0 || num_heads <= 0 || num_seqs <= 0) return 0;
    const size_t two = plan_decode(kv, num_seqs, num_heads, max_context_len, 0).bytes;
    const int32_t fg = mixed_grid(kv, num_heads, max_blocks_per_chunk);
    const size_t one = fg > 0 ? plan_decode(kv, num_seqs, num_heads, max_context_len, 0, fg).bytes : 0;
    return std::max(one, two);
}

int vcpp_paged_mixed_step(const vcpp_kv_pages* kv, const float* dq, float* dout,
                          const int32_t* d_block_tables, int32_t d_max_blocks_per_seq,
                          const int32_t* d_table_lens, const int32_t* d_context_lens, int32_t num_seqs,
                          int32_t max_context_len, const uint16_t* pq, float* pout,
                          const int32_t* p_block_tables, int32_t p_max_blocks_per_seq,
                          const int32_t* q_start, const int32_t* prefix_lens, int32_t num_chunks,
                          int32_t max_chunk_len, int32_t num_heads, void* workspace,
                          size_t workspace_bytes, void* stream) {
    g_last_error.clear();
    int rc = check_decode(kv, dq, dout, d_block_tables, d_max_blocks_per_seq, d_context_lens, num_seqs,
                          max_context_len, num_heads, 0);
    if (rc != VCPP_OK) return rc;
    rc = check_prefill(kv, pq, pout, p_block_tables, p_max_blocks_per_seq, q_start, prefix_lens, num_chunks,
                       max_chunk_len, num_heads);
    if (rc != VCPP_OK) return rc;
    const bool has_p = num_chunks > 0 && max_chunk_len > 0;
    const int32_t fg = num_seqs > 0 && has_p ? mixed_grid(kv, num_heads, p_max_blocks_per_seq) : 0;
    if (fg == 0 && num_seqs > 0 && has_p && kv->dtype != VCPP_KV_F32 && !no_merge_fork()) {
        // Decode, then the prefill on the caller's stream, with the decode's
        // merge on a side stream between them (it depends on the decode
        // only, and overlaps the prefill); the caller's stream waits for it
        // at the end.
        const DecodePlan pl = plan_decode(kv, num_seqs, num_heads, max_context_len, 0);
        if (pl.max_parts > 65535) return fail(VCPP_E_UNSUPPORTED, "too many partitions (%d)", pl.max_parts);
        rc = check_workspace(pl, workspace, workspace_bytes);
        if (rc != VCPP_OK) return rc;
        const vcpp::DecodeParams dp = decode_params(kv, dq, dout, d_block_tables, d_max_blocks_per_seq,
                                                    d_table_lens, d_context_lens, num_seqs, max_context_len,
                                                    num_heads, 0, pl, workspace);
        const vcpp::PrefillParams pp = prefill_params(kv, pq, pout, p_block_tables, p_max_blocks_per_seq,
                                                      q_start, prefix_lens, num_chunks, max_chunk_len, num_heads);
        const hipStream_t s = static_cast<hipStream_t>(stream);
        const vcpp::MergeFork* mf = merge_fork(s);
        bool forked = false;
        hipError_t e = vcpp::launch_decode(dp, s, mf, &forked);
        // Once the merge is forked, the caller's stream joins it whatever
        // fails later, so the stream stays ordered after the merge (and a
        // capture ends with the side stream joined).
        const hipError_t ep = e == hipSuccess ? vcpp::launch_prefill(pp, s) : hipSuccess;
        const hipError_t ej = forked ? hipStreamWaitEvent(s, mf->join, 0) : hipSuccess;
        if (e != hipSuccess) return hip_fail(e, "decode launch");
        if (ep != hipSuccess) return hip_fail(ep, "prefill launch");
        if (ej != hipSuccess) return hip_fail(ej, "merge join");
        return VCPP_OK;
    }
    if (fg == 0) {  // two launches on the stream: decode, then prefill
        if (num_seqs > 0) {
            rc = vcpp_paged_decode(kv, dq, dout, d_block_tables, d_max_blocks_per_seq, d_table_lens,
                                   d_context_lens, num_seqs, max_context_len, num_heads, 0, workspace,
                                   workspace_bytes, stream);
            if (rc != VCPP_OK) return rc;
        }
        if (!has_p) return VCPP_OK;
        return vcpp_paged_prefill(kv, pq, pout, p_block_tables, p_max_blocks_per_seq, q_start, prefix_lens,
                                  num_chunks, max_chunk_len, num_heads, stream);
    }
    const DecodePlan pl = plan_decode(kv, num_seqs, num_heads, max_context_len, 0, fg);
    rc = check_workspace(pl, workspace, workspace_bytes);
    if (rc != VCPP_OK) return rc;
    const vcpp::DecodeParams dp = decode_params(kv, dq, dout, d_block_tables, d_max_blocks_per_seq, d_table_lens,
                                                d_context_lens, num_seqs, max_context_len, num_heads, 0, pl,
                                                workspace);
    const vcpp::PrefillParams pp = prefill_params(kv, pq, pout, p_block_tables, p_max_blocks_per_seq, q_start,
                                                  prefix_lens, num_chunks, max_chunk_len, num_heads);
    hipError_t e = vcpp::launch_mixed(dp, pp, device_cus(), static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "mixed step launch");
    return VCPP_OK;
}

int vcpp_write_kv(const vcpp_kv_pages* kv, const float* k, const float* v, const int64_t* slots,
                  int32_t num_tokens, int32_t fp16_round_nearest, void* stream) {
    g_last_error.clear();
    // Writing needs less than attention: any head split and block size.
    if (!kv) return fail(VCPP_E_INVALID, "kv pages descriptor is NULL");
    if (kv->dtype != VCPP_KV_F32 && kv->dtype != VCPP_KV_F16 && kv->dtype != VCPP_KV_I8 &&
        kv->dtype != VCPP_KV_FP8)
        return fail(VCPP_E_INVALID, "unknown kv dtype %d", kv->dtype);
    if (kv->block_size <= 0 || kv->num_kv_heads <= 0 || kv->head_dim <= 0 || kv->num_blocks < 0)
        return fail(VCPP_E_INVALID, "bad page shape");
    if (kv->block_stride < (int64_t)kv->block_size * kv->num_kv_heads * kv->head_dim)
        return fail(VCPP_E_INVALID, "block_stride %lld smaller than one page", (long long)kv->block_stride);
    if (kv->num_blocks > 0 && (!kv->k || !kv->v)) return fail(VCPP_E_INVALID, "K/V page base is NULL");
    if (kv->dtype == VCPP_KV_I8 && kv->num_blocks > 0 &&
        (!kv->k_scale || !kv->v_scale ||
         kv->scale_block_stride < (int64_t)kv->num_kv_heads * kv->block_size))
        return fail(VCPP_E_INVALID, "int8 pages need scale pages of num_kv_heads * block_size per block");
    if (num_tokens < 0) return fail(VCPP_E_INVALID, "num_tokens must be >= 0");
    if (num_tokens == 0) return VCPP_OK;
    if (!k || !v || !slots) return fail(VCPP_E_INVALID, "k/v/slots is NULL");
    if ((int64_t)num_tokens * kv->num_kv_heads > (int64_t)INT32_MAX * 4)
        return fail(VCPP_E_UNSUPPORTED, "too many tokens (%d)", num_tokens);
    vcpp::KvWriteParams p{};
    p.dtype = kv->dtype;
    p.block_size = kv->block_size;
    p.num_kv_heads = kv->num_kv_heads;
    p.head_dim = kv->head_dim;
    p.num_blocks = kv->num_blocks;
    p.block_stride = kv->block_stride;
    p.scale_block_stride = kv->scale_block_stride;
    p.k = const_cast<void*>(kv->k);  // the pages are written: they must be writable
    p.v = const_cast<void*>(kv->v);
    p.k_scale = const_cast<uint16_t*>(kv->k_scale);
    p.v_scale = const_cast<uint16_t*>(kv->v_scale);
    p.k_src = k;
    p.v_src = v;
    p.slots = slots;
    p.num_tokens = num_tokens;
    p.fp16_rne = fp16_round_nearest ? 1 : 0;
    const hipError_t e = vcpp::launch_kv_write(p, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "write_kv launch");
    return VCPP_OK;
}

void paged_attention_cuda(const float* q, const uint16_t* kv_cache, const int32_t* block_tables,
                          const int32_t* context_lens, float* out, int32_t num_heads,
                          int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                          int32_t batch_size) {
    g_last_error.clear();
    if (block_size != 16 && block_size != 32) {
        fail(VCPP_E_UNSUPPORTED, "paged_attention_cuda: block_size %d (only 16 and 32)",
             block_size);
        return;
    }
    if (batch_size <= 0) return;
    if (!context_lens) {
        fail(VCPP_E_INVALID, "paged_attention_cuda: context_lens is NULL");
        return;
    }
    if (num_kv_heads <= 0 || num_heads <= 0 || num_heads % num_kv_heads != 0) {
        fail(VCPP_E_INVALID, "paged_attention_cuda: num_heads %d is not a positive multiple of "
             "num_kv_heads %d", num_heads, num_kv_heads);
        return;
    }
    if (head_dim <= 0 || head_dim > 256 || !vcpp::decode_head_dim_supported(VCPP_KV_F16, head_dim)) {
        fail(VCPP_E_UNSUPPORTED, "paged_attention_cuda: head_dim %d not supported", head_dim);
        return;
    }
    // Host read of the lengths, as cuda/attention.cu:25-28 does.
    int32_t max_ctx = 0;
    for (int32_t b = 0; b < batch_size; b++) max_ctx = context_lens[b] > max_ctx ? context_lens[b] : max_ctx;
    const int32_t max_blocks = max_ctx > 0 ? (max_ctx + block_size - 1) / block_size : 0;

    vcpp_kv_pages kv{};
    kv.dtype = VCPP_KV_F16;
    kv.block_size = block_size;
    kv.num_kv_heads = num_kv_heads;
    kv.head_dim = head_dim;
    const int64_t page = (int64_t)block_size * num_kv_heads * head_dim;
    // v1 passes no block count: bound block ids by the device allocation that
    // holds kv_cache (ids whose pages would end past it are skipped, as
    // get_k skips ids outside the pool, src/kv_cache_manager.cpp:90-95).
    kv.num_blocks = v1_num_blocks(kv_cache, 2 * page * (int64_t)sizeof(uint16_t));
    kv.block_stride = 2 * page;
    kv.k = kv_cache;
    kv.v = kv_cache ? kv_cache + page : nullptr;

    V1State& st = v1_state();
    std::lock_guard<std::mutex> lock(st.mu);
    const size_t need = plan_decode(&kv, batch_size, num_heads, max_ctx, 0).bytes;
    if (need > st.ws_bytes) {
        if (st.ws) (void)hipFree(st.ws);
        st.ws = nullptr;
        st.ws_bytes = 0;
        if (hipMalloc(&st.ws, need) != hipSuccess) {
            fail(VCPP_E_HIP, "paged_attention_cuda: workspace allocation of %zu bytes", need);
            return;
        }
        st.ws_bytes = need;
    }
    if ((size_t)batch_size > st.ctx_count) {
        if (st.ctx) (void)hipFree(st.ctx);
        st.ctx = nullptr;
        st.ctx_count = 0;
        if (hipMalloc(&st.ctx, sizeof(int32_t) * batch_size) != hipSuccess) {
            fail(VCPP_E_HIP, "paged_attention_cuda: context_lens staging allocation");
            return;
        }
        st.ctx_count = batch_size;
    }
    hipError_t e = hipMemcpyAsync(st.ctx, context_lens, sizeof(int32_t) * batch_size,
                                  hipMemcpyHostToDevice, nullptr);
    if (e != hipSuccess) {
        hip_fail(e, "paged_attention_cuda: context_lens copy");
        return;
    }
    vcpp_paged_decode(&kv, q, out, block_tables, max_blocks, nullptr, st.ctx, batch_size,
                      max_ctx, num_heads, 0, st.ws, st.ws_bytes, nullptr);
}

void flash_attention_cuda(const float* q, const float* k, const float* v, float* out,
                          float* attn_weights, int32_t batch_size, int32_t num_heads,
                          int32_t head_dim, int32_t q_len, int32_t kv_len, const float* attn_mask) {
    g_last_error.clear();
    if (batch_size <= 0 || num_heads <= 0) return;
    if (!q || !k || !v || !out || !attn_weights) {
        fail(VCPP_E_INVALID, "flash_attention_cuda: q/k/v/out/attn_weights is NULL");
        return;
    }
    if (head_dim <= 0 || q_len <= 0 || kv_len <= 0) {
        // kv_len 0 would make the reference read an unset logit (cuda/attention.cu:100).
        fail(VCPP_E_INVALID, "flash_attention_cuda: head_dim %d, q_len %d, kv_len %d must be > 0",
             head_dim, q_len, kv_len);
        return;
    }
    if ((int64_t)batch_size * num_heads > INT32_MAX || head_dim > 16384) {
        fail(VCPP_E_UNSUPPORTED, "flash_attention_cuda: shape too large");
        return;
    }
    vcpp::DenseParams p{q, k, v, out, attn_weights, attn_mask, batch_size, num_heads, head_dim, q_len, kv_len};
    const hipError_t e = vcpp::launch_dense(p, nullptr);
    if (e != hipSuccess) hip_fail(e, "flash_attention_cuda launch");
}

void apply_rope_cuda(float* q, float* k, const float* cos, const float* sin, int32_t total_dim,
                     int32_t head_dim, int32_t batch_size) {
    g_last_error.clear();
    if (batch_size <= 0 || total_dim <= 0) return;
    if (!q || !k || !cos || !sin) {
        fail(VCPP_E_INVALID, "apply_rope_cuda: q/k/cos/sin is NULL");
        return;
    }
    if (head_dim < 2) {
        fail(VCPP_E_INVALID, "apply_rope_cuda: head_dim %d must be >= 2", head_dim);
        return;
    }
    if ((int64_t)batch_size * total_dim > (int64_t)INT32_MAX * 256) {
        fail(VCPP_E_UNSUPPORTED, "apply_rope_cuda: shape too large");
        return;
    }
    vcpp::RopeTableParams p{q, k, cos, sin, total_dim, head_dim, batch_size};
    hipError_t e = vcpp::launch_rope_table(p, nullptr);
    if (e == hipSuccess) e = hipStreamSynchronize(nullptr);
    if (e != hipSuccess) hip_fail(e, "apply_rope_cuda");
}

void head_norm_cuda(float* x, const float* weight, float eps, int32_t num_heads, int32_t head_dim,
                    int32_t batch_size) {
    if (batch_size <= 0 || num_heads <= 0) {
        g_last_error.clear();
        return;
    }
    if ((int64_t)batch_size * num_heads > INT32_MAX) {
        g_last_error.clear();
        fail(VCPP_E_UNSUPPORTED, "head_norm_cuda: shape too large");
        return;
    }
    if (!weight) {
        g_last_error.clear();
        fail(VCPP_E_INVALID, "head_norm_cuda: weight is NULL");
        return;
    }
    if (vcpp_qk_norm_rope(x, nullptr, batch_size, num_heads, 0, head_dim, weight, nullptr, eps,
                          nullptr, nullptr, 0, VCPP_ROPE_INTERLEAVED, nullptr) != VCPP_OK)
        return;
    const hipError_t e = hipStreamSynchronize(nullptr);
    if (e != hipSuccess) hip_fail(e, "head_norm_cuda");
}

}  // extern "C"
