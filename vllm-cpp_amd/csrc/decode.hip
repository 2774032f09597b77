// decode.hip -- batched paged decode attention for gfx950.
//
// Reference behaviour: src/paged_attention.cpp:11-90 (one query token per
// sequence, GQA map kv_h = h / (H / Hkv), scale 1/sqrt(D), max seeded at
// -1e9, sum + 1e-9, positions past the table or on an invalid block skipped).
// The reference's GPU slot is cuda/attention.cu:11-52; its kernel
// (cuda/attention_kernels.cuh:9-123) is not followed.
//
// fp16 / int8 / FP8 pages (the HBM-bound path) run one of two kernels with the
// same split, MFMA step and merge (below).
//  * decode_page_kernel -- Hkv = 8, <= 8 query heads per kv head, D 64 or 80:
//    a workgroup of 8 waves (one per kv head) walks its range of 16-token
//    tiles (balanced split), or a run of fixed-partition ranges.  Each tile's K rows and V rows (16 tokens x all kv
//    heads: one contiguous run of the page each) are DMA'd into an LDS ring
//    with global_load_lds_dwordx4 (1 KiB of whole lines per instruction,
//    explicit vmcnt bookkeeping), chunk order XOR-swizzled by token, one
//    barrier per tile.  fp16: a 3-tile ring, one workgroup per CU.  Byte
//    pages: a 3-tile ring per workgroup and two workgroups per CU; K widened
//    in registers, V read transposed straight from the byte tile with
//    ds_read_b64_tr_b8, int8 scales in one more DMA instruction per tile.
//  * decode_mfma_kernel -- every other shape: one wave
//    per (kv head, chunk of <= 8 query heads of its GQA group); workgroups hold
//    4 waves = 4 kv heads = 640 contiguous bytes of each token row.  Its loads
//    are described at the end of this comment.
// Both kernels:
//  * Every K/V page is read from HBM once for a kv head's whole GQA group.
//  * Balanced split: the 16-token tiles of all sequences are laid end to end
//    and every resident workgroup takes an equal contiguous range of them, so
//    ragged batches keep the whole GPU busy to the end.  A range touches one
//    or more sequences (1-3 for 64 sequences of U[128, 4096] tokens over 256
//    ranges); a sequence wholly inside one range is finished in place, and
//    at most two fragments per range (the sequence continuing from the
//    previous range, the one continuing into the next) leave (m, l, o)
//    partials that a log-sum-exp merge kernel combines.
//  * A 16-token tile is one MFMA step:
//      S^T[16 tok][16] = K_tile[16 tok][D] x Qs^T   (16x16x32 f16; a 16-dim
//                                                    remainder as 16x16x16 into
//                                                    its own accumulator)
//      O[16][D]       += P[16][16 tok] x V_tile      (16x16x16 f16)
//    The 16 MFMA rows hold the fp16 "hi" part of the 8 query heads (rows 0-7)
//    and the fp16 residual q - hi (rows 8-15); likewise P = p_hi + p_lo, so
//    q and p keep about 22 significant bits while K/V stay exact fp16, with
//    fp32 accumulation: the rows an 8-head group would waste carry the low
//    halves instead.
//  * decode_mfma_kernel: K fragments come straight from HBM into registers (one 16-byte buffer
//    load per lane per 32 dims).  V is staged row-major in LDS and read back
//    with ds_read_b64_tr_b16, which hands each lane four tokens of one dim --
//    the P x V operand -- in one instruction.
//  * Loads go through buffer descriptors sized to the tile (zero-sized for an
//    invalid block, which then reads as zeros), so every load is issued
//    unconditionally, two 64-token steps are kept in flight in ping-pong
//    register buffers and the wait counts stay static.
// fp32 pages use a plain VALU kernel over fixed partitions (parity path).
#include "decode.h"
#include "device_common.h"
#include "prefill_body.h"
#include "profile.h"

#include <cstdlib>
#include <type_traits>

namespace vcpp {

namespace {

constexpr int kTile = 16;          // tokens per MFMA tile
// Page-staged decode's lazy running max (log2 units): the max moves when a
// tile's scores pass it by more than kPageLazy, and is looked at only when a
// lane's sum of P over its 4 tokens passes kPageLazySum.
constexpr float kPageLazy = 8.0f;
constexpr float kPageLazySum = 1024.0f;
// Pipeline shape (template parameters of the kernel): TPS tiles per step
// (one softmax update), NBUF register buffers, loads issued NBUF-1 steps ahead.
// Waves (kv heads) per workgroup: 4 kv heads x 80 dims x 2 B = 640 B, five
// whole 128-byte lines of every token row.
constexpr int kWavesPerGroup = 4;

typedef short s4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) char lds_char;

template <int D>
struct Dims {
    static constexpr int NC32 = D / 32;  // 16x16x32 steps over head_dim
    // A trailing 16-dim remainder runs as a 16x16x16 step into its own
    // accumulator.  One opcode per accumulation chain: a 16x16x16 step
    // chained straight onto a 16x16x32 accumulator was measured to drop the
    // previous step's contribution on gfx950 with this toolchain.
    static constexpr int REM = (D % 32) / 16;
    static constexpr int NT = D / 16;    // output 16-column tiles
    static_assert(D % 16 == 0 && D <= 256, "head_dim must be a multiple of 16");
};

// Registers of one 16-token tile for one lane (token c, head_dim chunk g).
template <int KV, int D>
struct Tile;

template <int D>
struct Tile<VCPP_KV_F16, D> {
    h8 k[Dims<D>::NC32 > 0 ? Dims<D>::NC32 : 1];
    h4 kr;  // dims 32*NC32 + 4g .. +3
    h8 v[Dims<D>::NC32 > 0 ? Dims<D>::NC32 : 1];
    h4 vr;
};

template <int D>
struct Tile<VCPP_KV_I8, D> {
    i2 k[Dims<D>::NC32 > 0 ? Dims<D>::NC32 : 1];
    uint32_t kr;
    i2 v[Dims<D>::NC32 > 0 ? Dims<D>::NC32 : 1];
    uint32_t vr;
    i2 ks;  // fp16 K scales of tokens 4g..4g+3
    i2 vs;  // fp16 V scales of tokens 4g..4g+3
};

template <int D>
struct Tile<VCPP_KV_FP8, D> {
    i2 k[Dims<D>::NC32 > 0 ? Dims<D>::NC32 : 1];
    uint32_t kr;
    i2 v[Dims<D>::NC32 > 0 ? Dims<D>::NC32 : 1];
    uint32_t vr;
};

// Per-lane byte offsets of the lane's share of a tile, identical for every
// tile: only the buffer base moves.
struct LaneOffsets {
    int k[4];   // 16x16x32 chunks (head_dim <= 128)
    int rem;    // 16x16x16 remainder chunk
    int scale;  // int8: fp16 scales of tokens 4g..4g+3
};

template <int KV, int D>
__device__ __forceinline__ LaneOffsets lane_offsets(const DecodeParams& p, int kvh, int g, int c) {
    constexpr int ES = KV == VCPP_KV_F16 ? 2 : 1;
    LaneOffsets o;
    const int row = (c * p.num_kv_heads + kvh) * D;
#pragma unroll
    for (int cc = 0; cc < 4; ++cc) o.k[cc] = (row + 32 * cc + 8 * g) * ES;
    o.rem = (row + 32 * Dims<D>::NC32 + 4 * g) * ES;
    o.scale = (kvh * p.block_size + 4 * g) * 2;
    return o;
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int bytes) {
    // dword3 0x00020000: raw 32-bit data format, the gfx9 setting for untyped
    // buffer loads; out-of-range offsets read as zero.
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, bytes, 0x00020000);
}

// Issues the lane's loads of one tile through buffer descriptors whose size is
// the tile's 16 token rows (and the block's scale page), or zero for an
// invalid block: the hardware then returns zeros without touching memory.
template <int KV, int D>
__device__ __forceinline__ void load_tile(Tile<KV, D>& t, const DecodeParams& p, int bid,
                                          int tok_in_block, const LaneOffsets& lo) {
    constexpr int NC32 = Dims<D>::NC32;
    constexpr int ES = KV == VCPP_KV_F16 ? 2 : 1;
    const bool ok = bid >= 0;
    const int64_t elem = (int64_t)(ok ? bid : 0) * p.block_stride +
                         (int64_t)tok_in_block * p.num_kv_heads * D;
    const int bytes = ok ? kTile * p.num_kv_heads * D * ES : 0;
    const auto kr = make_rsrc(static_cast<const char*>(p.k) + elem * ES, bytes);
    const auto vr = make_rsrc(static_cast<const char*>(p.v) + elem * ES, bytes);
    if constexpr (KV == VCPP_KV_F16) {
#pragma unroll
        for (int cc = 0; cc < NC32; ++cc) {
            t.k[cc] = __builtin_bit_cast(h8, __builtin_amdgcn_raw_buffer_load_b128(kr, lo.k[cc], 0, 0));
            t.v[cc] = __builtin_bit_cast(h8, __builtin_amdgcn_raw_buffer_load_b128(vr, lo.k[cc], 0, 0));
        }
        if constexpr (Dims<D>::REM) {
            t.kr = __builtin_bit_cast(h4, __builtin_amdgcn_raw_buffer_load_b64(kr, lo.rem, 0, 0));
            t.vr = __builtin_bit_cast(h4, __builtin_amdgcn_raw_buffer_load_b64(vr, lo.rem, 0, 0));
        }
    } else {
#pragma unroll
        for (int cc = 0; cc < NC32; ++cc) {
            t.k[cc] = __builtin_bit_cast(i2, __builtin_amdgcn_raw_buffer_load_b64(kr, lo.k[cc], 0, 0));
            t.v[cc] = __builtin_bit_cast(i2, __builtin_amdgcn_raw_buffer_load_b64(vr, lo.k[cc], 0, 0));
        }
        if constexpr (Dims<D>::REM) {
            t.kr = __builtin_amdgcn_raw_buffer_load_b32(kr, lo.rem, 0, 0);
            t.vr = __builtin_amdgcn_raw_buffer_load_b32(vr, lo.rem, 0, 0);
        }
    }
    if constexpr (KV == VCPP_KV_I8) {
        const int64_t se = (int64_t)(ok ? bid : 0) * p.scale_block_stride + tok_in_block;
        const int sbytes = ok ? (p.num_kv_heads * p.block_size - tok_in_block) * 2 : 0;
        const auto ksr = make_rsrc(p.k_scale + se, sbytes);
        const auto vsr = make_rsrc(p.v_scale + se, sbytes);
        t.ks = __builtin_bit_cast(i2, __builtin_amdgcn_raw_buffer_load_b64(ksr, lo.scale, 0, 0));
        t.vs = __builtin_bit_cast(i2, __builtin_amdgcn_raw_buffer_load_b64(vsr, lo.scale, 0, 0));
    }
}

// Decodes a tile's K chunk to fp16 MFMA operands.
template <int KV, int D>
__device__ __forceinline__ h8 k_chunk(const Tile<KV, D>& t, int cc) {
    if constexpr (KV == VCPP_KV_F16) return t.k[cc];
    else return bytes8_to_h8<KV>((uint32_t)t.k[cc].x, (uint32_t)t.k[cc].y);
}
template <int KV, int D>
__device__ __forceinline__ h4 k_rem(const Tile<KV, D>& t) {
    if constexpr (KV == VCPP_KV_F16) return t.kr;
    else return bytes4_to_h4<KV>(t.kr);
}

// Writes the lane's V row chunk (token c) into the wave's row-major LDS tile
// [16 tok][D]; rows of masked tokens are written as zeros so 0 * garbage
// cannot produce NaN in P x V.
template <int KV, int D>
__device__ __forceinline__ void stage_v(lds_char* tile, const Tile<KV, D>& t, bool valid, int g,
                                        int c) {
    constexpr int NC32 = Dims<D>::NC32;
    lds_char* row = tile + c * D * 2;
#pragma unroll
    for (int cc = 0; cc < NC32; ++cc) {
        h8 x;
        if constexpr (KV == VCPP_KV_F16) x = t.v[cc];
        else x = bytes8_to_h8<KV>((uint32_t)t.v[cc].x, (uint32_t)t.v[cc].y);
        if (!valid) x = h8{};
        *reinterpret_cast<__attribute__((address_space(3))) h8*>(row + (32 * cc + 8 * g) * 2) = x;
    }
    if constexpr (Dims<D>::REM) {
        h4 x;
        if constexpr (KV == VCPP_KV_F16) x = t.vr;
        else x = bytes4_to_h4<KV>(t.vr);
        if (!valid) x = h4{};
        *reinterpret_cast<__attribute__((address_space(3))) h4*>(row + (32 * NC32 + 4 * g) * 2) = x;
    }
}

// P x V operand of output columns 16t..16t+15: lane (g, c) receives
// V[4g + r][16t + c], r = 0..3.  ds_read_b64_tr_b16 gives lane i of each
// 16-lane group element (i mod 4) of the 8-byte read of lane 4j + i/4, so
// lane (g, c) reads row 4g + c/4, columns 16t + 4(c mod 4) .. +3.
template <int D>
__device__ __forceinline__ h4 read_v_tr(lds_char* tile, int t, int g, int c) {
    lds_char* a = tile + ((4 * g + (c >> 2)) * D + 16 * t + 4 * (c & 3)) * 2;
    const s4 x = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        reinterpret_cast<__attribute__((address_space(3))) s4*>(a));
    return __builtin_bit_cast(h4, x);
}

__device__ __forceinline__ float h_to_f(uint32_t bits16) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
}

__device__ __forceinline__ int tiles_of(const DecodeParams& p, int s) {
    const int ctx = min(max(p.context_lens[s], 0), p.ctx_cap);
    return (ctx + kTile - 1) / kTile;
}

// First tile of workgroup range w: floor(w * T / G).
__device__ __forceinline__ int range_start(int w, int T, int G) {
    return (int)(((int64_t)w * T) / G);
}

// Cross-lane steps on DPP (VALU, no LDS round trip): lanes whose source is
// outside its row, or whose row / bank is masked off, read 0.
template <int CTRL, int ROW_MASK = 0xF, int BANK_MASK = 0xF>
__device__ __forceinline__ int dpp_or0(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, ROW_MASK, BANK_MASK, false);
}

// Inclusive prefix sum over the wave's 64 lanes: Hillis-Steele within each
// row of 16 (row_shr 1, 2, 4, 8), then row 0's total into row 1 and row 2's
// into row 3 (row_bcast:15), then rows 0-1's total into rows 2 and 3
// (row_bcast:31).
__device__ __forceinline__ int wave_incl_scan(int x) {
    x += dpp_or0<0x111>(x);
    x += dpp_or0<0x112>(x);
    x += dpp_or0<0x114>(x);
    x += dpp_or0<0x118>(x);
    x += dpp_or0<0x142, 0xA>(x);
    x += dpp_or0<0x143, 0xC>(x);
    return x;
}

// Sum over the wave's lanes, returned as a scalar (provably uniform).
__device__ __forceinline__ int wave_sum(int x) {
    return __builtin_amdgcn_readlane(wave_incl_scan(x), 63);
}

// Exclusive prefix sum over the wave's lanes.
__device__ __forceinline__ int wave_excl_scan(int x, int /*lane*/) {
    return wave_incl_scan(x) - x;
}

// Range holding tile t (0 <= t < T): the largest w with floor(w T / G) <= t.
__device__ __forceinline__ int range_of(int t, int T, int G) {
    return (int)(((int64_t)(t + 1) * G - 1) / T);
}

__device__ __forceinline__ bool range_live(int w, int T, int G) {
    return T >= G || range_start(w, T, G) < range_start(w + 1, T, G);
}

// Partial block of fragment i (range w0 + i) of a sequence for kv-head slot
// `pair`: the first range holds the sequence in slot 1 (it starts inside it),
// every later one in slot 0.  Blocks are [8 heads][head_dim] floats for the
// outputs (32 * head_dim bytes, whole 128-byte lines as head_dim % 16 == 0)
// and 16 (m, l) pairs (128 bytes) for the softmax state, so no cache line is
// shared by two blocks.
__device__ __forceinline__ int64_t frag_block(int w0, int i, int pairs, int pair) {
    return ((int64_t)(w0 + i) * 2 + (i == 0 ? 1 : 0)) * pairs + pair;
}

// Log-sum-exp merge of the fragments (ranges w0..w1) of sequence s for one
// wave's heads head_base .. head_base+gc-1.  Each chunk of 8 fragments is one
// round of loads: every (m, l) and every partial output of the chunk is
// requested before any is used, then folded in with an online rescale.
// Lane (i8, h) = (lane / 8, lane % 8) owns fragment weights; output element
// e = lane + 64 k (head e / D) of the 8 x D block is lane-owned.  `wts` is the
// wave's LDS scratch (>= 80 floats).
// Workgroup spans of the split axis (Tv tiles, G ranges walked by WG
// workgroups, WG <= G): workgroup w covers ranges [range_start(w, G, WG),
// range_start(w + 1, G, WG)).  With WG == G a span is one range.
// The ranges of the split axis (Tv units, G ranges): equal ones
// [floor(r Tv / G), floor((r + 1) Tv / G)), or, with g1 > 0 (G even),
// alternating sizes: positions 2k take share / 256 of each pair's units and
// positions 2k + 1 the rest, so position r starts at
// Tv cum(r) / (128 G) with cum(r) = 256 (r / 2) + share (r % 2).
struct Split {
    int Tv, G, share;
    __device__ Split(int tv, int g, int g1, int sh) : Tv(tv), G(g), share(g1 > 0 && g % 2 == 0 ? sh : 0) {}
    __device__ int rstart(int r) const {
        if (share == 0) return range_start(r, Tv, G);
        const int64_t cum = (int64_t)(r >> 1) * 256 + (r & 1) * share;
        return (int)((int64_t)Tv * cum / ((int64_t)G * 128));
    }
    __device__ int rof(int t) const {  // the largest r with rstart(r) <= t (0 <= t < Tv)
        if (share == 0) return range_of(t, Tv, G);
        const int64_t u = ((int64_t)t * G * 128) / Tv;  // weight units before t, rounded down
        int r = (int)(u >> 8) * 2 + ((u & 255) >= share ? 1 : 0);
        while (r + 1 < G && rstart(r + 1) <= t) ++r;
        while (r > 0 && rstart(r) > t) --r;
        return r;
    }
    // every range holds at least one unit
    __device__ bool all_live() const {
        return share == 0 ? Tv >= G : (int64_t)Tv * min(share, 256 - share) >= (int64_t)G * 128;
    }
};

struct Spans {
    Split sp;
    int WG;  // workgroups walking the G ranges (G: a span is one range)
    __device__ int start(int w) const { return sp.rstart(WG == sp.G ? w : range_start(w, sp.G, WG)); }
    __device__ int span_of(int t) const {
        const int r = sp.rof(t);
        return WG == sp.G ? r : range_of(r, sp.G, WG);
    }
    // Every span holds a tile when every range does (WG <= G).
    __device__ bool live(int w) const { return sp.all_live() || start(w) < start(w + 1); }
};

template <int D>
__device__ __forceinline__ void merge_fragments(const DecodeParams& p, int s, int w0, int w1,
                                                int pair, int head_base, int gc, const Spans& sp,
                                                int lane,
                                                __attribute__((address_space(3))) float* wts) {
    // output element e = 4 lane + 256 k4 (.. +3, all in head e / D since D % 4 == 0)
    constexpr int K4 = (8 * D + 255) / 256;
    const int nfr = w1 - w0 + 1;
    const int i8 = lane >> 3, h = lane & 7;
    const int n_out = gc * D;
    const auto mlr = make_rsrc(p.ws_ml, 0x7FFFFFFF);
    float M = kMaxSeed, L = 0.f;  // of head h
    f4 acc[K4];
#pragma unroll
    for (int k = 0; k < K4; ++k) acc[k] = f4{0.f, 0.f, 0.f, 0.f};
    for (int i0 = 0; i0 < nfr; i0 += 8) {
        // one round of loads for the chunk
        float2 ml = make_float2(kMaxSeed, 0.f);
        {
            const int i = i0 + i8;
            const bool ok = i < nfr && h < gc && sp.live(w0 + i);
            const int64_t idx = frag_block(w0, ok ? i : 0, p.pairs, pair) * 16 + h;
            const float2 x = __builtin_bit_cast(
                float2, __builtin_amdgcn_raw_buffer_load_b64(mlr, (int)(idx * 8), 0, 0));
            if (ok) ml = x;
        }
        f4 v[8][K4];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            // an empty or missing fragment reads fragment 0 (weight 0 below)
            const int i = i0 + j;
            const bool ok = i < nfr && sp.live(w0 + i);
            const float* row = p.ws_o + frag_block(w0, ok ? i : 0, p.pairs, pair) * (8 * D);
            const auto rr = make_rsrc(row, n_out * 4);
#pragma unroll
            for (int k = 0; k < K4; ++k)
                v[j][k] = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(
                                                     rr, (4 * lane + 256 * k) * 4, 0, 0));
        }
        // running max / sum of head h, chunk weights
        float cm = ml.x;
        cm = fmaxf(cm, __shfl_xor(cm, 8, 64));
        cm = fmaxf(cm, __shfl_xor(cm, 16, 64));
        cm = fmaxf(cm, __shfl_xor(cm, 32, 64));
        const float Mn = fmaxf(M, cm);
        const float wt = fast_exp2(ml.x - Mn);  // 0 for empty fragments
        float cl = wt * ml.y;
        cl += __shfl_xor(cl, 8, 64);
        cl += __shfl_xor(cl, 16, 64);
        cl += __shfl_xor(cl, 32, 64);
        const float resc = fast_exp2(M - Mn);
        L = L * resc + cl;
        M = Mn;
        wts[lane] = wt;                       // wts[i8 * 8 + h]
        if (lane < 8) wts[64 + lane] = resc;  // rescale of head `lane`
#pragma unroll
        for (int k = 0; k < K4; ++k) {
            const int hk = min((4 * lane + 256 * k) / D, 7);
            f4 a = acc[k] * wts[64 + hk];
#pragma unroll
            for (int j = 0; j < 8; ++j) a += wts[j * 8 + hk] * v[j][k];
            acc[k] = a;
        }
    }
    if (lane < 8) wts[72 + lane] = 1.0f / (L + 1e-9f);
    float* out = p.out + ((int64_t)s * p.num_heads + head_base) * D;
#pragma unroll
    for (int k = 0; k < K4; ++k) {
        const int e = 4 * lane + 256 * k;
        if (e < n_out) *reinterpret_cast<f4*>(out + e) = acc[k] * wts[72 + e / D];
    }
}

template <int KV, int D, int TPS, int NBUF>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))
void decode_mfma_kernel(DecodeParams p) {
    constexpr int NC32 = Dims<D>::NC32, NT = Dims<D>::NT;
    extern __shared__ char lds_raw[];

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int g = lane >> 4, c = lane & 15;
    const int pair = blockIdx.y * (blockDim.x >> 6) + wave;
    if (pair >= p.pairs) return;  // whole waves only; no workgroup barriers below
    const int w = blockIdx.x, G = p.num_wg;

    const int kvh = pair / p.qchunks, qc = pair - kvh * p.qchunks;
    const int head_base = kvh * p.group + qc * 8;
    const int gc = min(8, p.group - qc * 8);
    const LaneOffsets lofs = lane_offsets<KV, D>(p, kvh, g, c);
    lds_char* lds = reinterpret_cast<lds_char*>((__attribute__((address_space(3))) char*)lds_raw) +
                    wave * (TPS * kTile * D * 2);

    // Tiles of all sequences laid end to end: total T, this workgroup's range
    // [a, b) = [floor(w T / G), floor((w + 1) T / G)).
    int T = 0;
    for (int base = 0; base < p.num_seqs; base += 64)
        T += wave_sum(base + lane < p.num_seqs ? tiles_of(p, base + lane) : 0);
    const int a = range_start(w, T, G), b = range_start(w + 1, T, G);
    // Zero-tile sequences are zeroed by the range their start falls into (the
    // last range for those at T, range 0 when every sequence is empty).
    const bool zero_owner_tail = (T == 0 && w == 0) || (T > 0 && w == G - 1);

    auto process_fragment = [&](int s, int S, int E) {
        const int t0 = max(a, S) - S, t1 = min(b, E) - S;
        const bool complete = S >= a && E <= b;
        const int slot = S < a ? 0 : 1;

        const int ctx = min(max(p.context_lens[s], 0), p.ctx_cap);
        int tlen = p.max_blocks;
        if (p.table_lens) tlen = min(tlen, p.table_lens[s]);
        const int end = (int)min((int64_t)ctx, (int64_t)tlen * p.block_size);

        // Query fragment: row c = hi (c < 8) or lo (c >= 8) of head c & 7.
        h8 qa[NC32 > 0 ? NC32 : 1];
        h4 qr = {};
        {
            const bool qv = (c & 7) < gc;
            const float* qrow = p.q + ((int64_t)s * p.num_heads + head_base + (c & 7)) * D;
#pragma unroll
            for (int cc = 0; cc < NC32; ++cc) {
                f4 x0 = {}, x1 = {};
                if (qv) {
                    x0 = *reinterpret_cast<const f4*>(qrow + 32 * cc + 8 * g);
                    x1 = *reinterpret_cast<const f4*>(qrow + 32 * cc + 8 * g + 4);
                }
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const float x = i < 4 ? x0[i] : x1[i - 4];
                    const _Float16 hi = (_Float16)x;
                    qa[cc][i] = c < 8 ? hi : (_Float16)(x - (float)hi);
                }
            }
            if constexpr (Dims<D>::REM) {
                f4 x = {};
                if (qv) x = *reinterpret_cast<const f4*>(qrow + 32 * NC32 + 4 * g);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const _Float16 hi = (_Float16)x[i];
                    qr[i] = c < 8 ? hi : (_Float16)(x[i] - (float)hi);
                }
            }
        }

        f4 o[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t) o[t] = f4{0.f, 0.f, 0.f, 0.f};
        float m_run = kMaxSeed, l_run = 0.f;

        for (int ch = t0; ch < t1; ch += 64) {
            const int ntiles = min(64, t1 - ch);
            // Physical block of tile ch + j in lane j (-1: past the table or
            // an id outside the pool).
            int my_bid = -1, my_off = 0;
            if (lane < ntiles) {
                const int pos = (ch + lane) * kTile;
                const int lb = pos / p.block_size;
                my_off = pos - lb * p.block_size;
                if (lb < tlen) {
                    const int id = p.block_tables[(int64_t)s * p.max_blocks + lb];
                    if (id >= 0 && (int64_t)id < p.num_blocks) my_bid = id;
                }
            }

            auto load_step = [&](Tile<KV, D>(&buf)[TPS], int it) {
#pragma unroll
                for (int j = 0; j < TPS; ++j) {
                    const int tt = it * TPS + j;
                    const int bid = tt < ntiles ? __builtin_amdgcn_readlane(my_bid, tt & 63) : -1;
                    const int off = __builtin_amdgcn_readlane(my_off, tt & 63);
#ifdef VCPP_GATHER_DUMP
                    const int gpos = (ch + tt) * kTile + lane;
                    if (pair == 0 && tt < ntiles && lane < kTile && bid >= 0 && gpos < end)
                        gather_record(p, s, gpos, bid, off + lane);
#endif
                    load_tile<KV, D>(buf[j], p, bid, off, lofs);
                }
            };

            // FULL: every tile of the step is a valid block lying wholly below `end`,
            // so no masking code runs (the common case).
            auto compute_step = [&](const Tile<KV, D>(&cur)[TPS], int it, auto full_tag) {
                constexpr bool FULL = decltype(full_tag)::value;
                float sc[TPS][4];
                float mx = kMaxSeed;
#pragma unroll
                for (int j = 0; j < TPS; ++j) {
                    const int tt = it * TPS + j;
                    const int bid = tt < ntiles ? __builtin_amdgcn_readlane(my_bid, tt & 63) : -1;
                    const int pos0 = (ch + tt) * kTile;
                    const bool full = FULL || (bid >= 0 && pos0 + kTile <= end);  // wave-uniform
                    f4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int cc = 0; cc < NC32; ++cc)
                        acc = mfma32(k_chunk<KV, D>(cur[j], cc), qa[cc], acc);
                    if constexpr (Dims<D>::REM) {
                        // Own accumulator, summed on the VALU (see Dims).
                        const f4 zero = {0.f, 0.f, 0.f, 0.f};
                        const f4 acc2 = mfma16(k_rem<KV, D>(cur[j]), qr, zero);
                        acc += acc2;
                    }
                    stage_v<KV, D>(lds + j * kTile * D * 2, cur[j], full || pos0 + c < end, g, c);
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        float x = acc[r] + dpp_ror8(acc[r]);
                        float f = p.scale_log2;
                        if constexpr (KV == VCPP_KV_I8) {
                            const uint32_t wd = (uint32_t)(r < 2 ? cur[j].ks.x : cur[j].ks.y);
                            f *= h_to_f((r & 1) ? (wd >> 16) : (wd & 0xFFFFu));
                        }
                        x *= f;
                        if (!full) x = (bid >= 0 && pos0 + 4 * g + r < end) ? x : -__builtin_inff();
                        sc[j][r] = x;
                        mx = fmaxf(mx, x);
                    }
                }
                mx = fmaxf(mx, shfl_xor(mx, 16));
                mx = fmaxf(mx, shfl_xor(mx, 32));
                const float m_new = fmaxf(m_run, mx);
                const float alpha = fast_exp2(m_run - m_new);
                m_run = m_new;
                if (__any(alpha != 1.0f)) {
                    // Accumulator row 4g + r belongs to head (4g + r) & 7.
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const float al = shfl(alpha, (4 * g + r) & 7);
#pragma unroll
                        for (int t = 0; t < NT; ++t) o[t][r] *= al;
                    }
                }
                float lsum = 0.f;
#pragma unroll
                for (int j = 0; j < TPS; ++j) {
                    h4 pa;
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        float pr = fast_exp2(sc[j][r] - m_new);
                        lsum += pr;
                        if constexpr (KV == VCPP_KV_I8) {
                            const uint32_t wd = (uint32_t)(r < 2 ? cur[j].vs.x : cur[j].vs.y);
                            // masked tokens have pr == 0; the select keeps 0 * garbage out
                            pr = pr > 0.f ? pr * h_to_f((r & 1) ? (wd >> 16) : (wd & 0xFFFFu)) : 0.f;
                        }
                        const _Float16 hi = (_Float16)pr;
                        pa[r] = c < 8 ? hi : (_Float16)(pr - (float)hi);
                    }
                    lds_char* vt = lds + j * kTile * D * 2;
#pragma unroll
                    for (int t = 0; t < NT; ++t) o[t] = mfma16(pa, read_v_tr<D>(vt, t, g, c), o[t]);
                }
                l_run = l_run * alpha + lsum;
            };

            // NBUF register buffers in rotation: steps it+1 .. it+NBUF-1 are in
            // flight while step it computes; no buffer is copied (a copy would
            // wait on its loads).  Steps past the end load zero-sized (free) tiles.
            Tile<KV, D> buf[NBUF][TPS];
            const int niters = (ntiles + TPS - 1) / TPS;
            // Whole steps of valid blocks below `end` (tiles are in order).
            int nfull = 0;
            {
                const int last_ok = (ch * kTile + ntiles * kTile <= end);
                const bool all_valid = __builtin_amdgcn_read_exec() ==
                                       (uint64_t)__ballot(lane >= ntiles || my_bid >= 0);
                const int full_tiles = all_valid ? (last_ok ? ntiles : ntiles - 1) : 0;
                nfull = full_tiles / TPS;
            }
#pragma unroll
            for (int k = 0; k < NBUF - 1; ++k) load_step(buf[k], k);
            for (int it = 0; it < niters; it += NBUF) {
#pragma unroll
                for (int k = 0; k < NBUF; ++k) {
                    if (it + k >= niters) break;
                    load_step(buf[(k + NBUF - 1) % NBUF], it + k + NBUF - 1);
                    if (it + k < nfull) compute_step(buf[k], it + k, std::true_type{});
                    else compute_step(buf[k], it + k, std::false_type{});
                }
            }
        }

        // Per-head totals: l over the four lane groups; O rows h (hi) + h + 8 (lo).
        float lt = l_run;
        lt += shfl_xor(lt, 16);
        lt += shfl_xor(lt, 32);
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) o[t][r] += shfl_xor(o[t][r], 32);
        float lh[4], mh[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            lh[r] = shfl(lt, (4 * g + r) & 7);
            mh[r] = shfl(m_run, (4 * g + r) & 7);
        }
        if (g < 2) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int h = 4 * g + r;
                if (h >= gc) continue;
                const int head = head_base + h;
                if (complete) {
                    const float inv = 1.0f / (lh[r] + 1e-9f);
                    float* orow = p.out + ((int64_t)s * p.num_heads + head) * D;
#pragma unroll
                    for (int t = 0; t < NT; ++t) orow[16 * t + c] = o[t][r] * inv;
                } else {
                    const int64_t blk = ((int64_t)w * 2 + slot) * p.pairs + pair;
                    float* orow = p.ws_o + (blk * 8 + h) * D;
#pragma unroll
                    for (int t = 0; t < NT; ++t) orow[16 * t + c] = o[t][r];
                    if (c == 0) p.ws_ml[blk * 16 + h] = make_float2(mh[r], lh[r]);
                }
            }
        }
    };

    int carry = 0;
    for (int base = 0; base < p.num_seqs; base += 64) {
        const int sl = base + lane;
        const int nt = sl < p.num_seqs ? tiles_of(p, sl) : 0;
        const int Sl = carry + wave_excl_scan(nt, lane);
        carry += wave_sum(nt);
        const bool overlap = a < b && sl < p.num_seqs && nt > 0 && Sl < b && Sl + nt > a;
        const bool zero_here = sl < p.num_seqs && nt == 0 &&
                               ((Sl >= a && Sl < b) || (zero_owner_tail && Sl >= T));
        uint64_t todo = __ballot(overlap || zero_here);
        while (todo) {
            const int j = __builtin_ctzll(todo);
            todo &= todo - 1;
            const int s = base + j;
            // readlane keeps S / E in scalar registers: everything derived
            // from them (tile counts, buffer descriptors) stays provably
            // uniform, with no per-load waterfall loops.
            const int S = __builtin_amdgcn_readlane(Sl, j);
            const int E = S + __builtin_amdgcn_readlane(nt, j);
            if (E == S) {  // no tiles: zero output
                float* orow = p.out + ((int64_t)s * p.num_heads + head_base) * D;
                for (int e = lane; e < gc * D; e += 64) orow[e] = 0.f;
                continue;
            }
            process_fragment(s, S, E);
        }
        if (carry >= b && !zero_owner_tail) break;
    }
}

// One wave per (sequence, kv-head slot): sequences split over several ranges
// get their partial blocks merged; everything else was finished in place.
template <int D>
__global__ __launch_bounds__(256) void merge_split_kernel(DecodeParams p) {
    __shared__ float wts_all[4][80];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int pair = blockIdx.y * 4 + wave;
    const int s = blockIdx.x;
    if (pair >= p.pairs) return;
    const int G = p.num_wg, X = p.switch_tiles;
    int T = 0, S = 0, K = 0, KS = 0;  // tiles and non-empty sequences: all, before s
    for (int base = 0; base < p.num_seqs; base += 64) {
        const int sl = base + lane;
        const int nt = sl < p.num_seqs ? tiles_of(p, sl) : 0;
        T += wave_sum(nt);
        S += wave_sum(sl < s ? nt : 0);
        K += wave_sum(nt > 0 ? 1 : 0);
        KS += wave_sum(sl < s && nt > 0 ? 1 : 0);
    }
    const int E = S + tiles_of(p, s);
    if (E <= S) return;  // no tiles: zeroed by the decode kernel
    // the split's axis: tile t of s sits at t + X (non-empty sequences up to s)
    const int Tv = T + X * K, shift = X * (KS + 1);
    const Spans sp{Split(Tv, G, p.g1, p.g1_share), p.page_grid};
    const int w0 = sp.span_of(S + shift), w1 = sp.span_of(E - 1 + shift);
    if (w0 == w1) return;  // finished in place
    const int kvh = pair / p.qchunks, qc = pair - kvh * p.qchunks;
    merge_fragments<D>(p, s, w0, w1, pair, kvh * p.group + qc * 8, min(8, p.group - qc * 8), sp,
                       lane, reinterpret_cast<__attribute__((address_space(3))) float*>(
                                 (__attribute__((address_space(3))) float*)wts_all[wave]));
}

// ---- fp32 pages -----------------------------------------------------------

// Plain VALU kernel, one wave per (partition, sequence, head).  Logits of the
// partition live in LDS; the exp2/log2-scaled partials match the merge below.
// fp32 pages: one workgroup per (partition, sequence, kv head, chunk of up to
// 8 query heads of its group).  The partition's positions go through LDS in
// 32-token tiles: the workgroup gathers a tile's K and V rows of its kv head
// (16-byte lanes, through the block table) once for all of its query heads;
// thread (head h, token j) forms one score (a D-long dot in fp32, in order),
// the heads' running max / sum move per tile, and thread (h, dims d, d + 32,
// ..) accumulates the weighted V rows.  Partitions of a sequence leave
// (m, l, o) partials for merge_parts_kernel when there are several.
constexpr int kF32Tile = 32;
constexpr int kF32Heads = 8;

__global__ __launch_bounds__(256) void decode_f32_kernel(DecodeParams p) {
    extern __shared__ __attribute__((aligned(16))) float f32_lds[];
    const int D = p.head_dim;
    const int tid = threadIdx.x;
    const int seq = blockIdx.y, part = blockIdx.x;
    const int kvh = blockIdx.z / p.qchunks, qc = blockIdx.z - kvh * p.qchunks;
    const int h0 = kvh * p.group + qc * kF32Heads;             // first query head
    const int nh = min(kF32Heads, p.group - qc * kF32Heads);   // query heads here
    const int ctx = min(p.context_lens[seq], p.max_parts * p.partition);
    const int P = p.partition;
    const int np = ctx <= 0 ? 1 : min((ctx + P - 1) / P, p.max_parts);
    if (part >= np) return;  // whole workgroup
    int tlen = p.max_blocks;
    if (p.table_lens) tlen = min(tlen, p.table_lens[seq]);
    const int start = part * P;
    const int stop = max(min(start + P, ctx), start);
    const int end = (int)min((int64_t)stop, (int64_t)tlen * p.block_size);  // usable positions

    // LDS: q [8][D], K tile [32][D + 1], V tile [32][D], P [8][32], per-head (m, l, alpha)
    const int KP = D + 1;  // K row pitch (odd: the 32 rows of a dot fall on distinct banks)
    float* qs = f32_lds;
    float* ks = qs + kF32Heads * D;
    float* vs = ks + kF32Tile * KP;
    float* ps = vs + kF32Tile * D;
    float* st = ps + kF32Heads * kF32Tile;  // [8] m, [8] l, [8] alpha
    for (int e = tid; e < nh * D; e += 256)
        qs[e] = p.q[((int64_t)seq * p.num_heads + h0) * D + e];
    if (tid < kF32Heads) {
        st[tid] = kMaxSeed;
        st[8 + tid] = 0.f;
    }
    // output ownership: thread (h = tid / 32, d = tid % 32 + 32 k)
    const int oh = tid >> 5, od = tid & 31;
    float acc[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) acc[k] = 0.f;
    const float* kbase = reinterpret_cast<const float*>(p.k);
    const float* vbase = reinterpret_cast<const float*>(p.v);
    const int chunks = D / 4;  // 16-byte pieces of a row
    for (int t0 = start; t0 < stop; t0 += kF32Tile) {
        __syncthreads();  // previous tile's K, V, P no longer read
        // gather: piece (row j, chunk c4) of K and V
        for (int e = tid; e < kF32Tile * chunks; e += 256) {
            const int j = e / chunks, c4 = e - j * chunks;
            const int pos = t0 + j;
            float4 kx = make_float4(0.f, 0.f, 0.f, 0.f), vx = kx;
            if (pos < end) {
                const int lb = pos / p.block_size;
                const int id = p.block_tables[(int64_t)seq * p.max_blocks + lb];
                if (id >= 0 && (int64_t)id < p.num_blocks) {
                    const int64_t off = (int64_t)id * p.block_stride +
                                        ((int64_t)(pos - lb * p.block_size) * p.num_kv_heads + kvh) * D + 4 * c4;
                    kx = *reinterpret_cast<const float4*>(kbase + off);
                    vx = *reinterpret_cast<const float4*>(vbase + off);
#ifdef VCPP_GATHER_DUMP
                    if (c4 == 0 && blockIdx.z == 0) gather_record(p, seq, pos, id, pos - lb * p.block_size);
#endif
                }
            }
            float* kr = ks + j * KP + 4 * c4;
            kr[0] = kx.x;
            kr[1] = kx.y;
            kr[2] = kx.z;
            kr[3] = kx.w;
            *reinterpret_cast<float4*>(vs + j * D + 4 * c4) = vx;
        }
        __syncthreads();
        // scores: thread (head h = tid / 32, token j = tid % 32), skipped
        // positions -inf; then the head's new max (a 32-lane reduction)
        {
            const int h = tid >> 5, j = tid & 31;
            const int pos = t0 + j;
            float s = -__builtin_inff();
            bool ok = h < nh && pos < end;
            if (ok) {
                const int lb = pos / p.block_size;
                const int id = p.block_tables[(int64_t)seq * p.max_blocks + lb];
                ok = id >= 0 && (int64_t)id < p.num_blocks;
            }
            if (ok) {
                const float* qr = qs + h * D;
                const float* kr = ks + j * KP;
                float a = 0.f;
                for (int d = 0; d < D; ++d) a = fmaf(qr[d], kr[d], a);
                s = a * p.scale_log2;
            }
            float mx = s;
#pragma unroll
            for (int k = 16; k >= 1; k >>= 1) mx = fmaxf(mx, shfl_xor(mx, k));
            const float m_old = st[h];
            const float m_new = fmaxf(m_old, mx);
            const float e = ok ? fast_exp2(s - m_new) : 0.f;
            ps[h * kF32Tile + j] = e;
            float sum = e;
#pragma unroll
            for (int k = 16; k >= 1; k >>= 1) sum += shfl_xor(sum, k);
            __syncthreads();  // every lane of the head read st[h] before it moves
            if (j == 0) {
                const float alpha = fast_exp2(m_old - m_new);
                st[h] = m_new;
                st[8 + h] = st[8 + h] * alpha + sum;
                st[16 + h] = alpha;
            }
        }
        __syncthreads();
        // outputs: rescale, then the tile's weighted V rows
        if (oh < nh) {
            const float alpha = st[16 + oh];
            const float* pr = ps + oh * kF32Tile;
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const int d = od + 32 * k;
                if (d < D) {
                    float a = acc[k] * alpha;
                    for (int j = 0; j < kF32Tile; ++j) a = fmaf(pr[j], vs[j * D + d], a);
                    acc[k] = a;
                }
            }
        }
    }
    __syncthreads();
    if (oh < nh) {
        const int head = h0 + oh;
        const float m = st[oh], l = st[8 + oh];
        if (np == 1) {
            const float inv = 1.0f / (l + 1e-9f);
            float* orow = p.out + ((int64_t)seq * p.num_heads + head) * D;
#pragma unroll
            for (int k = 0; k < 8; ++k)
                if (od + 32 * k < D) orow[od + 32 * k] = acc[k] * inv;
        } else {
            const int64_t idx = ((int64_t)seq * p.max_parts + part) * p.num_heads + head;
#pragma unroll
            for (int k = 0; k < 8; ++k)
                if (od + 32 * k < D) p.ws_o[idx * D + od + 32 * k] = acc[k];
            if (od == 0) p.ws_ml[idx] = make_float2(m, l);
        }
    }
}

// Log-sum-exp merge of the fixed partitions of one (sequence, head) per wave.
__global__ __launch_bounds__(256) void merge_parts_kernel(DecodeParams p) {
    const int lane = threadIdx.x & 63;
    const int head = blockIdx.y * 4 + (threadIdx.x >> 6);
    const int seq = blockIdx.x;
    if (head >= p.num_heads) return;
    const int ctx = min(p.context_lens[seq], p.max_parts * p.partition);
    const int P = p.partition;
    const int np = ctx <= 0 ? 1 : min((ctx + P - 1) / P, p.max_parts);
    if (np <= 1) return;
    const int D = p.head_dim;
    const int64_t base = (int64_t)seq * p.max_parts * p.num_heads + head;
    float M = kMaxSeed, L = 0.f;
    for (int i0 = 0; i0 < np; i0 += 64) {
        const int i = i0 + lane;
        float2 ml = make_float2(kMaxSeed, 0.f);
        if (i < np) ml = p.ws_ml[base + (int64_t)i * p.num_heads];
        float m = ml.x;
        for (int k = 32; k >= 1; k >>= 1) m = fmaxf(m, shfl_xor(m, k));
        const float Mn = fmaxf(M, m);
        float l = fast_exp2(ml.x - Mn) * ml.y;
        for (int k = 32; k >= 1; k >>= 1) l += shfl_xor(l, k);
        L = L * fast_exp2(M - Mn) + l;
        M = Mn;
    }
    const float inv = 1.0f / (L + 1e-9f);
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    for (int i0 = 0; i0 < np; i0 += 64) {
        const int n = min(64, np - i0);
        float wt = 0.f;
        if (i0 + lane < np) wt = fast_exp2(p.ws_ml[base + (int64_t)(i0 + lane) * p.num_heads].x - M);
        for (int j = 0; j < n; ++j) {
            const float wj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wt), j));
            const float* orow = p.ws_o + (base + (int64_t)(i0 + j) * p.num_heads) * D;
#pragma unroll
            for (int k = 0; k < 4; ++k)
                if (lane + 64 * k < D) acc[k] += wj * orow[lane + 64 * k];
        }
    }
    float* out = p.out + ((int64_t)seq * p.num_heads + head) * D;
#pragma unroll
    for (int k = 0; k < 4; ++k)
        if (lane + 64 * k < D) out[lane + 64 * k] = acc[k] * inv;
}

// ---------------------------------------------------------------------------
// fp16 or int8 pages, Hkv = 8: whole 16-token tiles staged through LDS.
//
// One workgroup (8 waves, one per kv head) per CU takes a balanced range of
// the concatenated tiles.  A tile's K rows (16 tokens x 8 heads x D values)
// and V rows are each one contiguous run in the page, so the workgroup moves
// them into LDS with global_load_lds_dwordx4 -- every instruction 1 KiB of
// whole cache lines -- through a ring of tiles, one barrier per tile.  Within
// every SWZ-chunk group (16-byte chunks; a token row is a whole number of
// groups) the chunk order is XOR-swizzled by the group's token, so the K
// fragment reads (16 tokens of one head) and the V reads spread over the
// banks.  Each wave then runs the MFMA tile step of decode_mfma_kernel on its
// head and writes complete sequences or (m, l, o) partials for
// merge_split_kernel.
//
// int8 and FP8 pages (one byte per value): K fragments are widened to fp16 in
// registers (int8: exact integers; FP8: its values), and V is read transposed
// straight from the byte tile (ds_read_b64_tr_b8) and widened likewise.  int8
// pages also carry the tile's 8 x 16 K and V scales (fp16, [head][token]) in
// one more DMA instruction: the K scale multiplies the fp32 score, the V scale
// fp32 P before its fp16 split.


struct PageEntry {
    int bid;     // physical block (-1: zeros)
    int tok;     // first token of the tile in its block
    int seq;     // sequence
    int tis;     // tile index within the sequence
    int ntiles;  // tiles of the sequence
    int end;     // usable positions of the sequence
    int pad0, pad1;
};

// Shape of the page-staged kernel: HW kv heads per workgroup (one wave
// each); a tile region is the 16 tokens' slice of those heads' rows.
//  * HW 8, D 64 / 80 (BASELINE shapes): fp16 a 3-tile ring, one workgroup per
//    CU (2 waves per SIMD); byte pages two workgroups per CU (4 waves per
//    SIMD), whose second workgroup hides the first one's per-tile latency
//    (a deeper single ring does not).
//  * HW 4 (head groups of 4 kv heads, and head_dim 128): fp16 D <= 80 two
//    workgroups per CU with 3-tile rings; fp16 D 128 (32 KiB per tile) two
//    workgroups per CU with 2-tile rings; byte pages D <= 80 four workgroups
//    per CU, D 128 two.
// F: the decode side of the fused mixed-step kernel (HW 4, three workgroups
// per CU): byte pages a 4-tile ring, fp16 a 2-tile ring, 128 tiles listed at
// a time, so that its LDS stays within a third of a CU.
template <int KV, int D, int HW, bool F = false>
struct PageCfg {
    static constexpr bool BYTES = KV != VCPP_KV_F16;   // int8 or FP8: one byte per value
    static constexpr bool SCALED = KV == VCPP_KV_I8;   // per-(token, head) fp16 scales
    static constexpr int ES = BYTES ? 1 : 2;
    static constexpr int RC = HW * D * ES / 16;           // 16-byte chunks per token row slice
    static constexpr int HC = D * ES / 16;                // chunks of one head in a row
    static constexpr int SWZ = RC % 16 == 0 ? 16 : RC % 8 == 0 ? 8 : 4;  // swizzle group (chunks)
    static constexpr int REG = 16 * RC * 16;              // bytes of one region (K or V) of a tile
    static constexpr int NI = REG / 1024;                 // DMA instructions per region
    static constexpr int NREAL = 2 * NI + (SCALED ? 1 : 0);  // + the scale instruction
    static constexpr int PERW = (NREAL + HW - 1) / HW;
    static constexpr int STAGE = 2 * REG + (SCALED ? 1024 : 0);
    static constexpr bool BIG = !BYTES && HW == 4 && D > 80;   // fp16 head_dim 128
    static constexpr int WPC = F ? 3 : HW == 8 ? (BYTES ? 2 : 1) : (BYTES && D <= 80 ? 4 : 2);  // workgroups per CU
    static constexpr int WPE = WPC * HW / 4;              // waves per SIMD
    static constexpr int STAGES = F ? (BYTES ? 4 : 2) : BIG ? 2 : 3;
    static constexpr int WINDOW = F || WPC == 4 ? 128 : (BIG ? 256 : 512);  // tiles listed at a time
    static constexpr int OFF_JUNK = STAGES * STAGE;       // target of padding DMAs
    static constexpr int OFF_LIST = OFF_JUNK + (PERW * HW > NREAL ? 1024 : 0);
    static constexpr int LDS = OFF_LIST + WINDOW * (int)sizeof(PageEntry);
    static_assert(RC % SWZ == 0 && REG % 1024 == 0 && (D * ES) % 16 == 0, "tile shape");
    static_assert(LDS * WPC <= 160 * 1024, "LDS budget");
};

__device__ __attribute__((aligned(16))) const uint32_t kZeroChunk16[4] = {0, 0, 0, 0};

// One 16-byte lane of a tile DMA.  The load is non-temporal (nt): every
// K/V byte of a decode is read once, and streaming it without the normal
// allocation policy raised config 2's kernel from 0.62 to 0.70 of the HBM
// peak (71.8 -> 62.7 us) and config 4's from 0.72 to 0.81.  (Prefill re-reads
// each page from several workgroups and keeps the default policy.)
__device__ __forceinline__ void dma16_page(const void* src, uint32_t lds_base) {
    uint32_t saved;
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %2, off nt\n\ts_mov_b32 m0, %0"
                 : "=&s"(saved) : "s"(lds_base), "v"(src) : "memory");
}

template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// LDS slot of chunk gc (16-byte units) of a tile region whose token rows are
// rc chunks long: XOR of the low bits (group of SWZ) with the token.
template <int SWZ>
__device__ __forceinline__ int page_slot(int gc, int rc) {
    return (gc & ~(SWZ - 1)) | ((gc & (SWZ - 1)) ^ ((gc / rc) & (SWZ - 1)));
}

// One workgroup of the page-staged decode: it walks ranges [r_lo, r_hi) of
// the split (bx of the nbx workgroups per kv-head group) for kv heads
// by * HW .. + HW - 1.
template <int KV, int D, int HW, bool F>
__device__ __forceinline__ void decode_page_body(const DecodeParams& p, int bx, int by, int nbx) {
    using C = PageCfg<KV, D, HW, F>;
    constexpr bool BYTES = C::BYTES, SCALED = C::SCALED;
    constexpr int NC32 = Dims<D>::NC32, NT = Dims<D>::NT;
    constexpr int kPageWindow = C::WINDOW;
    constexpr int RC = C::RC, HC = C::HC, SWZ = C::SWZ, REG = C::REG, NI = C::NI;
    constexpr int PERW = C::PERW, STAGE = C::STAGE, STAGES = C::STAGES;
    extern __shared__ __attribute__((aligned(16))) char smem[];
    lds_char* lds = reinterpret_cast<lds_char*>((__attribute__((address_space(3))) char*)smem);
    PageEntry* list = reinterpret_cast<PageEntry*>(smem + C::OFF_LIST);
    const uint32_t lds_addr = (uint32_t)(uintptr_t)lds;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, c = lane & 15;
    // Every argument the range start reads, in scalar registers before the
    // first use: one batch of kernel-argument loads and one wait, instead of
    // a load and a wait wherever the compiler first needs a field.
    asm volatile("" ::"s"(p.context_lens), "s"(p.table_lens), "s"(p.block_tables), "s"(p.q), "s"(p.out),
                 "s"(p.num_seqs), "s"(p.ctx_cap), "s"(p.max_blocks), "s"(p.num_wg), "s"(p.switch_tiles),
                 "s"(p.block_size), "s"(p.num_blocks), "s"(p.num_heads), "s"(p.group), "s"(p.k), "s"(p.v),
                 "s"(p.block_stride));
    // Ranges of the split: G in all.  Workgroup w walks the contiguous ranges
    // [r_lo, r_hi) with one DMA ring: one range for the balanced split; with
    // fixed partitions (G > workgroups, no switch units) a run of whole
    // partitions, whose online softmax combines them in registers.  Either
    // way a workgroup leaves at most one fragment per sequence end, indexed
    // by the workgroup (span_of in the merge kernel).
    const int G = p.num_wg, WG = nbx;
    // With alternating range sizes the first dispatch round (ids below WG / 2)
    // takes the even positions of the axis, the second the odd ones; partial
    // blocks are indexed by position.
    const int posn = !F && p.g1 > 0 ? (bx < WG / 2 ? 2 * bx : 2 * (bx - WG / 2) + 1) : bx;
    const int r_lo = range_start(posn, G, WG), r_hi = range_start(posn + 1, G, WG);
    // This workgroup's kv heads: hb .. hb + HW - 1, one per wave (global
    // head kvh; local slot `wave` in the LDS tile).  group <= 8: one query
    // chunk per kv head.
    const int hb = by * HW;
    const int kvh = hb + wave, pair = kvh;
    const int head_base = kvh * p.group;
    const int gc = p.group;

    // The split: ranges divide T + X K evenly, where sequence j's tiles are
    // preceded by X units that hold no tile (the cost of starting it), and
    // each range's bounds map back to real tile indices a, b.
    const int X = p.switch_tiles;
    // Context lengths of the first 128 sequences stay in registers (lane l:
    // sequences l and 64 + l) from this first scan on: every later scan (the
    // range bounds, the empty-sequence zeroing, the tile list) reads them
    // from there instead of with a dependent round trip to memory of its own.
    int ctx_c0 = 0, ctx_c1 = 0, tl_c0 = 0, tl_c1 = 0;
    auto lane_ctx = [&](int base) -> int {  // context length of sequence base + lane
        if (base == 0) return ctx_c0;
        if (base == 64) return ctx_c1;
        const int sl = base + lane;
        return sl < p.num_seqs ? min(max(p.context_lens[sl], 0), p.ctx_cap) : 0;
    };
    auto load_tlen = [&](int base) -> int {  // usable table length of sequence base + lane
        const int sl = base + lane;
        return sl < p.num_seqs && p.table_lens ? min(p.max_blocks, p.table_lens[sl]) : p.max_blocks;
    };
    auto lane_tlen = [&](int base) -> int {
        if (base == 0) return tl_c0;
        if (base == 64) return tl_c1;
        return load_tlen(base);
    };
    {
        // The first 128 sequences' lengths: four loads with clamped indices
        // in one batch, one wait.
        const int n1 = max(p.num_seqs - 1, 0);
        const int r0 = p.context_lens[min(lane, n1)], r1 = p.context_lens[min(64 + lane, n1)];
        int u0 = p.max_blocks, u1 = p.max_blocks;
        if (p.table_lens) {
            u0 = p.table_lens[min(lane, n1)];
            u1 = p.table_lens[min(64 + lane, n1)];
        }
        ctx_c0 = lane < p.num_seqs ? min(max(r0, 0), p.ctx_cap) : 0;
        ctx_c1 = 64 + lane < p.num_seqs ? min(max(r1, 0), p.ctx_cap) : 0;
        tl_c0 = lane < p.num_seqs ? min(p.max_blocks, u0) : p.max_blocks;
        tl_c1 = 64 + lane < p.num_seqs ? min(p.max_blocks, u1) : p.max_blocks;
    }
    int T = 0, K = 0;
    for (int base = 0; base < p.num_seqs; base += 64) {
        const int nt = (lane_ctx(base) + kTile - 1) / kTile;
        T += wave_sum(nt);
        K += wave_sum(nt > 0 ? 1 : 0);
    }
    const int Tv = T + X * K;
    // first real tile at or past virtual position V
    auto real_of = [&](int V) -> int {
        if (X == 0 || V <= 0) return max(V, 0);
        if (V >= Tv) return T;
        int cs = 0, ck = 0;
        for (int base = 0; base < p.num_seqs; base += 64) {
            const int nt = (lane_ctx(base) + kTile - 1) / kTile;
            const int Sl = cs + wave_excl_scan(nt, lane);
            const int kl = ck + wave_excl_scan(nt > 0 ? 1 : 0, lane);
            const int vfirst = Sl + X * (kl + 1);  // virtual position of its first tile
            const uint64_t hit = __ballot(nt > 0 && V >= vfirst - X && V < vfirst + nt);
            if (hit) {
                const int j = __builtin_ctzll(hit);
                const int Sj = __builtin_amdgcn_readlane(Sl, j), kj = __builtin_amdgcn_readlane(kl, j);
                return max(Sj, V - X * (kj + 1));
            }
            cs += wave_sum(nt);
            ck += wave_sum(nt > 0 ? 1 : 0);
        }
        return T;
    };
    const Split spl(Tv, G, F ? 0 : p.g1, p.g1_share);
    const int a = real_of(spl.rstart(r_lo)), b = real_of(spl.rstart(r_hi));
    const bool zero_owner_tail = (T == 0 && bx == 0) || (T > 0 && bx == WG - 1);

    // Zero the outputs of empty sequences this range owns (wave 0).
    if (wave == 0) {
        int carry = 0;
        for (int base = 0; base < p.num_seqs; base += 64) {
            const int sl = base + lane;
            const int nt = (lane_ctx(base) + kTile - 1) / kTile;
            const int Sl = carry + wave_excl_scan(nt, lane);
            carry += wave_sum(nt);
            const bool zero_here = sl < p.num_seqs && nt == 0 &&
                                   ((Sl >= a && Sl < b) || (zero_owner_tail && Sl >= T));
            uint64_t todo = __ballot(zero_here);
            while (todo) {
                const int j = __builtin_ctzll(todo);
                todo &= todo - 1;
                // this workgroup's heads only
                float* orow = p.out + ((int64_t)(base + j) * p.num_heads + hb * p.group) * D;
                for (int e = lane; e < HW * p.group * D; e += 64) orow[e] = 0.f;
            }
        }
    }

    // Per-wave DMA lanes: instruction j = wave * PERW + i fills bytes
    // [1024 j', 1024 j' + 1024) of region j / NI (j' = j mod NI); int8 adds
    // instruction 2 NI for the scales; the rest pad every wave to PERW.
    auto issue = [&](int tau, int win0, int win1) {
        const uint32_t sbase = lds_addr + (tau % STAGES) * STAGE;
        int bid = -1, tok = 0;
        if (tau < win1) {
            const PageEntry& e = list[tau - win0];
            bid = e.bid;
            tok = e.tok;
#ifdef VCPP_GATHER_DUMP
            const int gpos = e.tis * kTile + lane;
            if (by == 0 && wave == 0 && lane < kTile && bid >= 0 && gpos < e.end)
                gather_record(p, e.seq, gpos, bid, tok + lane);
#endif
        }
        // The workgroup's slice of each token row: rows are num_kv_heads * D
        // elements apart and the slice starts hb * D into one (the whole row
        // when HW == num_kv_heads, one contiguous run for the tile).
        const int64_t row = (int64_t)p.num_kv_heads * D;
        const int64_t elem = (int64_t)(bid >= 0 ? bid : 0) * p.block_stride + (int64_t)tok * row + (int64_t)hb * D;
#pragma unroll
        for (int i = 0; i < PERW; ++i) {
            const int j = wave * PERW + i;  // uniform
            if (j < 2 * NI) {
                const int which = j >= NI;
                const int pos = (j - which * NI) * 64 + lane;  // slot in the region
                const int grp = pos & ~(SWZ - 1);
                const int gcn = grp | ((pos & (SWZ - 1)) ^ ((grp / RC) & (SWZ - 1)));  // source chunk
                const int gtok = gcn / RC, gch = gcn - gtok * RC;           // its token, chunk in the slice
                const char* base = static_cast<const char*>(which ? p.v : p.k);
                const void* src = bid >= 0 ? (const void*)(base + (elem + gtok * row) * C::ES + (int64_t)gch * 16)
                                           : (const void*)kZeroChunk16;
                dma16_page(src, __builtin_amdgcn_readfirstlane(sbase + which * REG + (j - which * NI) * 1024));
            } else if (SCALED && j == 2 * NI) {
                // lanes 0 .. 2 HW - 1: K scales of local head lane / 2 (32 B =
                // 2 chunks), lanes 2 HW .. 4 HW - 1: V scales likewise
                const bool vsc = lane >= 2 * HW;
                const int head = hb + ((vsc ? lane - 2 * HW : lane) >> 1), half = lane & 1;
                const uint16_t* sp = vsc ? p.v_scale : p.k_scale;
                const void* src = bid >= 0 && lane < 4 * HW
                    ? (const void*)(sp + (int64_t)bid * p.scale_block_stride + head * p.block_size + tok + 8 * half)
                    : (const void*)kZeroChunk16;
                dma16_page(src, __builtin_amdgcn_readfirstlane(sbase + 2 * REG));
            } else {
                dma16_page(kZeroChunk16, lds_addr + C::OFF_JUNK);
            }
        }
    };

    // Fragment state of this wave's head.
    int cur = -1, first_tis = 0, last_tis = 0, cur_ntiles = 0, cur_end = 0;
    h8 qa[NC32 > 0 ? NC32 : 1];
    h4 qr = {};
    f4 o[NT];
    float m_run = kMaxSeed, l_run = 0.f;

    auto finalize = [&]() {
        float lt = l_run;
        lt += shfl_xor(lt, 16);
        lt += shfl_xor(lt, 32);
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) o[t][r] += shfl_xor(o[t][r], 32);
        float lh[4], mh[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            lh[r] = shfl(lt, (4 * g + r) & 7);
            mh[r] = shfl(m_run, (4 * g + r) & 7);
        }
        const bool complete = first_tis == 0 && last_tis == cur_ntiles - 1;
        const int slot = first_tis == 0 ? 1 : 0;
        // Rows 4 (g & 1) + r hold head rows; after the half-wave sum every
        // lane has its row's values, so all lanes store: pass k takes register
        // r = k + 2 (g >> 1), even lanes store pass 0 and odd lanes pass 1 as
        // column pairs (the pair's other value one DPP swap away).  One float2
        // store per 16 columns keeps the finalize off the memory queue that
        // the DMA ring fills.
        const int rk0 = 2 * (g >> 1), rk1 = rk0 + 1;
        const bool odd = (c & 1) != 0;
        const int rr = odd ? rk1 : rk0;
        const int h = 4 * (g & 1) + rr;
        const int64_t blk = ((int64_t)posn * 2 + slot) * p.pairs + pair;
        float* orow = complete ? p.out + ((int64_t)cur * p.num_heads + head_base + h) * D
                               : p.ws_o + (blk * 8 + h) * D;
        float lsel = lh[0];
#pragma unroll
        for (int r = 1; r < 4; ++r) lsel = rr == r ? lh[r] : lsel;
        const float scl = complete ? 1.0f / (lsel + 1e-9f) : 1.0f;
        // The swap runs on every lane: with an odd group size the partner of
        // the last even head's lane stores nothing but must still supply its
        // value.
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            float x0 = o[t][0], x1 = o[t][1];
            if (rk0 == 2) {
                x0 = o[t][2];
                x1 = o[t][3];
            }
            const float y = dpp_swap1(odd ? x0 : x1);  // neighbour in the pair
            const float2 v = odd ? make_float2(y * scl, x1 * scl) : make_float2(x0 * scl, y * scl);
            if (h < gc) *reinterpret_cast<float2*>(orow + 16 * t + (c & ~1)) = v;
        }
        // (m, l) of the partial: lanes c < 4 of the first two groups, row 4 g + c
        if (!complete && g < 2 && c < 4 && 4 * g + c < gc) {
            float ms = mh[0], ls = lh[0];
#pragma unroll
            for (int r = 1; r < 4; ++r) {
                ms = c == r ? mh[r] : ms;
                ls = c == r ? lh[r] : ls;
            }
            p.ws_ml[blk * 16 + 4 * g + c] = make_float2(ms, ls);
        }
    };

    // Raw q rows of this wave's heads for sequence `seq` (lane (g, c): head
    // c & 7, dims 32 cc + 8 g .. + 7 and the remainder's 4 g .. + 3), and
    // their hi/lo fp16 split into the MFMA operands.
    constexpr int QN = 2 * NC32 + (Dims<D>::REM ? 1 : 0);
    auto load_q = [&](int seq, f4 (&xq)[QN]) {
        const bool qv = (c & 7) < gc;
        const float* qrow = p.q + ((int64_t)seq * p.num_heads + head_base + (c & 7)) * D;
#pragma unroll
        for (int cc = 0; cc < NC32; ++cc) {
            xq[2 * cc] = qv ? *reinterpret_cast<const f4*>(qrow + 32 * cc + 8 * g) : f4{};
            xq[2 * cc + 1] = qv ? *reinterpret_cast<const f4*>(qrow + 32 * cc + 8 * g + 4) : f4{};
        }
        if constexpr (Dims<D>::REM)
            xq[2 * NC32] = qv ? *reinterpret_cast<const f4*>(qrow + 32 * NC32 + 4 * g) : f4{};
    };
    auto split_q = [&](const f4 (&xq)[QN]) {
#pragma unroll
        for (int cc = 0; cc < NC32; ++cc) {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float x = i < 4 ? xq[2 * cc][i] : xq[2 * cc + 1][i - 4];
                const _Float16 hi = (_Float16)x;
                qa[cc][i] = c < 8 ? hi : (_Float16)(x - (float)hi);
            }
        }
        if constexpr (Dims<D>::REM) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float x = xq[2 * NC32][i];
                const _Float16 hi = (_Float16)x;
                qr[i] = c < 8 ? hi : (_Float16)(x - (float)hi);
            }
        }
    };
    // fp16 pages: q of the first two sequences of the range (the one holding
    // its first tile, the next one to start in it) is loaded with the tile
    // list (its wait is the list's), so neither start waits for the DMA ring
    // the way a later start_seq's load does.  (Byte pages run 4 waves per
    // SIMD and have no registers for it.)
    constexpr bool PRE_Q = !BYTES;
    f4 qpre[PRE_Q ? QN : 1], qpre2[PRE_Q ? QN : 1];
    int pre_seq = -1, pre_seq2 = -1;

    auto start_seq = [&](const PageEntry& e) {
        cur = e.seq;
        first_tis = e.tis;
        cur_ntiles = e.ntiles;
        cur_end = e.end;
        if (PRE_Q && e.seq == pre_seq) {
            if constexpr (PRE_Q) split_q(qpre);
            pre_seq = -1;
        } else if (PRE_Q && e.seq == pre_seq2) {
            if constexpr (PRE_Q) split_q(qpre2);
            pre_seq2 = -1;
        } else {
            f4 xq[QN];
            load_q(cur, xq);
            split_q(xq);
        }
#pragma unroll
        for (int t = 0; t < NT; ++t) o[t] = f4{0.f, 0.f, 0.f, 0.f};
        m_run = kMaxSeed;
        l_run = 0.f;
    };

    // LDS byte offset of chunk `chunk` of this lane's token row c, head kvh
    // (the same in the K and V regions).
    auto kofs = [&](int chunk) { return page_slot<SWZ>(c * RC + wave * HC + chunk, RC) * 16; };
    // fp16: transposing V reads (tokens 4g + c/4 [+ 0..3], dims 16t + 4(c&3)).
    auto vofs = [&](int t) {
        const int tok = 4 * g + (c >> 2);
        const int dim = 16 * t + 4 * (c & 3);
        return REG + page_slot<SWZ>(tok * RC + wave * HC + dim / 8, RC) * 16 + (dim & 7) * 2;
    };
    typedef __attribute__((address_space(3))) uint32_t lds_u32;
    typedef __attribute__((address_space(3))) i2 lds_i2;

    const float lo_sel = c < 8 ? 0.f : -1.f;
    auto compute_tile = [&](int tau, const PageEntry& e) {
        lds_char* sb = lds + (tau % STAGES) * STAGE;
        const int pos0 = e.tis * kTile;
        const bool full = e.bid >= 0 && pos0 + kTile <= cur_end;  // uniform
        f4 acc = {0.f, 0.f, 0.f, 0.f};
        i2 ksw = {}, vsw = {};
        if constexpr (BYTES) {
            if constexpr (SCALED) {
                // K scales of tokens 4g..4g+3 (head kvh), V scales likewise
                ksw = *reinterpret_cast<lds_i2*>(sb + 2 * REG + wave * 32 + 8 * g);
                vsw = *reinterpret_cast<lds_i2*>(sb + 2 * REG + 32 * HW + wave * 32 + 8 * g);
            }
#pragma unroll
            for (int cc = 0; cc < NC32; ++cc) {
                const i2 kw = *reinterpret_cast<lds_i2*>(sb + kofs(2 * cc + (g >> 1)) + 8 * (g & 1));
                acc = mfma32(bytes8_to_h8<KV>((uint32_t)kw.x, (uint32_t)kw.y), qa[cc], acc);
            }
            if constexpr (Dims<D>::REM) {
                const uint32_t kw = *reinterpret_cast<lds_u32*>(sb + kofs(2 * NC32) + 4 * g);
                const f4 zero = {0.f, 0.f, 0.f, 0.f};
                acc += mfma16(bytes4_to_h4<KV>(kw), qr, zero);
            }
        } else {
#pragma unroll
            for (int cc = 0; cc < NC32; ++cc) {
                const h8 kf = *reinterpret_cast<__attribute__((address_space(3))) h8*>(sb + kofs(4 * cc + g));
                acc = mfma32(kf, qa[cc], acc);
            }
            if constexpr (Dims<D>::REM) {
                const h4 kf = *reinterpret_cast<__attribute__((address_space(3))) h4*>(
                    sb + kofs(4 * NC32 + (g >> 1)) + (g & 1) * 8);
                const f4 zero = {0.f, 0.f, 0.f, 0.f};
                acc += mfma16(kf, qr, zero);
            }
        }
        // V operands, read here so that their LDS latency overlaps the S
        // MFMAs and the softmax.  Byte pages: one ds_read_b64_tr_b8 per pair
        // of output blocks (t, t+1): lane i of each 16-lane group gets byte
        // i mod 8 of the read of lane 2j + i/8, j = 0..7.  Lanes 2j, 2j+1 of
        // group g read token 4g + (j & 3), dims 16u .. 16u+15 of head kvh
        // (one 16-byte chunk), u = t for j < 4 and t+1 above, so lane (g, c)
        // gets V[4g + r][16t + c] in bytes r and V[4g + r][16(t+1) + c] in
        // bytes 4 + r.  An odd last block reads itself twice.  fp16 pages:
        // one ds_read_b64_tr_b16 per output block.
        i2 vx[BYTES ? (NT + 1) / 2 : 1];
        s4 vh[BYTES ? 1 : NT];
        if constexpr (BYTES) {
#pragma unroll
            for (int t = 0; t < NT; t += 2) {
                const int j = c >> 1;
                const int u = (j < 4 || t + 1 == NT) ? t : t + 1;
                const int ofs = REG + page_slot<SWZ>((4 * g + (j & 3)) * RC + wave * HC + u, RC) * 16 + 8 * (c & 1);
                vx[t / 2] = __builtin_amdgcn_ds_read_tr8_b64_v2i32(reinterpret_cast<lds_i2*>(sb + ofs));
            }
        } else {
#pragma unroll
            for (int t = 0; t < NT; ++t)
                vh[t] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                    reinterpret_cast<__attribute__((address_space(3))) s4*>(sb + vofs(t)));
        }
        // Visible tokens of the tile (uniform): all 16, the sequence's
        // remainder, or none on a missing page.
        const int lim = full ? kTile : (e.bid >= 0 ? cur_end - pos0 : 0);
        float sc[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            float x = acc[r] + dpp_ror8(acc[r]);
            float f = p.scale_log2;
            if constexpr (SCALED) {
                const uint32_t wd = (uint32_t)(r < 2 ? ksw.x : ksw.y);
                f *= h_to_f((r & 1) ? (wd >> 16) : (wd & 0xFFFFu));
            }
            x *= f;
            sc[r] = 4 * g + r < lim ? x : -__builtin_inff();
        }
        // Lazy running max: P against the current max; only when a lane's
        // sum of P passes 2^10 (so some P may exceed it, or is inf / NaN)
        // is the tile's max formed, and the max moves when it grows by more
        // than 2^kPageLazy -- so P stays <= 2^10 (fp16 hi/lo split exact to
        // ~22 bits) and most tiles need no cross-lane reduction.
        float pr[4], lsum = 0.f;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            pr[r] = fast_exp2(sc[r] - m_run);
            lsum += pr[r];
        }
        if (__builtin_expect(__any(!(lsum <= kPageLazySum)), 0)) {
            float mx = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
            mx = fmaxf(mx, shfl_xor(mx, 16));
            mx = fmaxf(mx, shfl_xor(mx, 32));
            const bool grow = mx > m_run + kPageLazy;
            const float m_new = grow ? mx : m_run;
            const float alpha = fast_exp2(m_run - m_new);
            m_run = m_new;
            if (__any(alpha != 1.0f)) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float al = shfl(alpha, (4 * g + r) & 7);
#pragma unroll
                    for (int t = 0; t < NT; ++t) o[t][r] *= al;
                }
            }
            l_run *= alpha;
            lsum = 0.f;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                pr[r] = fast_exp2(sc[r] - m_run);
                lsum += pr[r];
            }
        }
        if constexpr (SCALED) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const uint32_t wd = (uint32_t)(r < 2 ? vsw.x : vsw.y);
                // masked tokens have pr == 0; the select keeps 0 * garbage out
                pr[r] = pr[r] > 0.f ? pr[r] * h_to_f((r & 1) ? (wd >> 16) : (wd & 0xFFFFu)) : 0.f;
            }
        }
        // Rows 0-7 carry fp16(p), rows 8-15 p - fp16(p): x = p - lo_sel * fp16(p).
        h4 pa;
#pragma unroll
        for (int r = 0; r < 4; r += 2) {
            const h2 hi = {(_Float16)pr[r], (_Float16)pr[r + 1]};
            const float x0 = fmaf(lo_sel, (float)hi[0], pr[r]), x1 = fmaf(lo_sel, (float)hi[1], pr[r + 1]);
            pa[r] = (_Float16)x0;
            pa[r + 1] = (_Float16)x1;
        }
        if constexpr (BYTES) {
#pragma unroll
            for (int t = 0; t < NT; t += 2) {
                o[t] = mfma16(pa, bytes4_to_h4<KV>((uint32_t)vx[t / 2].x), o[t]);
                if (t + 1 < NT) o[t + 1] = mfma16(pa, bytes4_to_h4<KV>((uint32_t)vx[t / 2].y), o[t + 1]);
            }
        } else {
#pragma unroll
            for (int t = 0; t < NT; ++t) o[t] = mfma16(pa, __builtin_bit_cast(h4, vh[t]), o[t]);
        }
        l_run += lsum;
    };

    for (int win0 = a; win0 < b; win0 += kPageWindow) {
        const int win1 = min(b, win0 + kPageWindow);
        __syncthreads();  // the previous window's list is no longer read
        // List the window's tiles: every wave scans the sequences; the
        // workgroup fills the entries of each overlapping one.
        {
            int carry = 0;
            for (int base = 0; base < p.num_seqs; base += 64) {
                const int sl = base + lane;
                // This lane's sequence: its context length (tiles) and table
                // length, loaded together; the sequences the window overlaps
                // read them by lane below instead of with loads of their own.
                const bool in = sl < p.num_seqs;
                const int ctx_l = lane_ctx(base);
                const int tlen_l = lane_tlen(base);
                const int nt = (ctx_l + kTile - 1) / kTile;
                const int Sl = carry + wave_excl_scan(nt, lane);
                carry += wave_sum(nt);
                uint64_t todo = __ballot(in && nt > 0 && Sl < win1 && Sl + nt > win0);
                while (todo) {
                    const int j = __builtin_ctzll(todo);
                    todo &= todo - 1;
                    const int s = base + j;
                    const int S = __builtin_amdgcn_readlane(Sl, j);
                    const int n = __builtin_amdgcn_readlane(nt, j);
                    const int ctx = __builtin_amdgcn_readlane(ctx_l, j);
                    const int tlen = __builtin_amdgcn_readlane(tlen_l, j);
                    const int end = (int)min((int64_t)ctx, (int64_t)tlen * p.block_size);
                    const int t0 = max(win0, S), t1 = min(win1, S + n);
                    if constexpr (PRE_Q) {
                        if (win0 == a && t0 == a) {  // the range's first tile
                            pre_seq = s;
                            load_q(s, qpre);
                        } else if (win0 == a && t0 == S && pre_seq2 < 0) {  // next start
                            pre_seq2 = s;
                            load_q(s, qpre2);
                        }
                    }
                    for (int tt = t0 + tid; tt < t1; tt += HW * 64) {
                        const int tis = tt - S;
                        const int pos = tis * kTile;
                        const int lb = pos / p.block_size;
                        int bid = -1;
                        if (lb < tlen) {
                            const int id = p.block_tables[(int64_t)s * p.max_blocks + lb];
                            if (id >= 0 && (int64_t)id < p.num_blocks) bid = id;
                        }
                        PageEntry& e = list[tt - win0];
                        e.bid = bid;
                        e.tok = pos - lb * p.block_size;
                        e.seq = s;
                        e.tis = tis;
                        e.ntiles = n;
                        e.end = end;
                    }
                }
                if (carry >= win1) break;
            }
        }
        // Table and length loads land here in a wait the compiler sees (the
        // DMA ring below is invisible to its counters).
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
        __syncthreads();
#pragma unroll
        for (int i = 0; i < STAGES - 1; ++i) issue(win0 + i, win0, win1);
        for (int tau = win0; tau < win1; ++tau) {
            wait_vm<(STAGES - 2) * PERW>();
            __syncthreads();  // tile tau landed for every wave; tile tau - 1 consumed
            issue(tau + STAGES - 1, win0, win1);
            const PageEntry e = list[tau - win0];
            if (e.seq != cur) {
                if (cur >= 0) finalize();
                start_seq(e);
            }
            last_tis = e.tis;
            compute_tile(tau, e);
        }
        wait_vm<0>();
    }
    if (cur >= 0) finalize();
}

template <int KV, int D, int HW>
__global__ __launch_bounds__(HW * 64) __attribute__((amdgpu_waves_per_eu(PageCfg<KV, D, HW>::WPE, PageCfg<KV, D, HW>::WPE)))
void decode_page_kernel(DecodeParams p) {
    decode_page_body<KV, D, HW, false>(p, blockIdx.x, blockIdx.y, gridDim.x);
}

template <int KV, int D, int HW>
hipError_t launch_page(const DecodeParams& p, hipStream_t stream) {
    const size_t lds = PageCfg<KV, D, HW>::LDS;
    // The LDS limit is a per-device property of the kernel: set it once on
    // each device the library launches on (idempotent if two threads race).
    static bool attr_set[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64 || !attr_set[dev]) {
        const hipError_t e = hipFuncSetAttribute((const void*)decode_page_kernel<KV, D, HW>,
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
        if (dev >= 0 && dev < 64) attr_set[dev] = true;
    }
    hipLaunchKernelGGL((decode_page_kernel<KV, D, HW>), dim3(p.page_grid, p.num_kv_heads / HW), dim3(HW * 64),
                       lds, stream, p);
    return hipGetLastError();
}

// ---- fused mixed step ------------------------------------------------------
//
// A scheduler step that carries decodes and prefill chunks together
// (src/scheduler.h:14-23; the engine serves them in one step,
// src/paged_engine.cpp:254-269) as one launch (opt-in; vcpp_paged_mixed_step
// runs two launches by default, which measured faster).  Decode is HBM-bound
// and prefill MFMA-bound, so the launch puts both on every CU at once: three
// 4-wave workgroups per CU (168 VGPRs, 3 waves per SIMD), one of them a
// decode worker walking the balanced split with 4 kv heads
// (decode_page_body), two of them prefill workers taking query tiles of 32
// rows (prefill_tile, heaviest tiles first) in a fixed stride.  Workgroups
// are dealt to the 8 XCDs by linear id, and within an XCD the roles repeat
// every three workgroups, so with the launch sized to three per CU each CU
// holds one decode and two prefill workers whatever order the CUs are filled
// in.
constexpr int kMixedWpc = 3;    // workgroups per CU
constexpr int kMixedPrefill = 2;  // of them prefill workers
struct MixedGrid {
    int pf_items;  // prefill work items: tiles x chunks x (kv head, head group)
    int pf_nyz;    // chunks x (kv head, head group)
    int pf_nz;     // (kv head, head group) pairs
    int dec_hg;    // kv-head groups of 4 (decode workgroups per range)
};

template <int KV, int D>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(kMixedWpc, kMixedWpc)))
void mixed_step_kernel(DecodeParams dp, PrefillParams pp, MixedGrid mg) {
    constexpr int W = kMixedWpc, NPF = kMixedPrefill, NDEC = W - NPF;
    const int id = blockIdx.x, xcd = id & 7, local = id >> 3;
    const int per_cu = (gridDim.x >> 3) / W;  // CUs per XCD
    const int trip = local / W, role = local - W * trip;
    if (role >= NDEC) {
        extern __shared__ __attribute__((aligned(16))) char smem[];
        lds_char* lds = reinterpret_cast<lds_char*>((__attribute__((address_space(3))) char*)smem);
        const int workers = NPF * (gridDim.x / W);
        for (int it = xcd * NPF * per_cu + NPF * trip + role - NDEC; it < mg.pf_items; it += workers) {
            const int bx = it / mg.pf_nyz, r = it - bx * mg.pf_nyz;
            const int by = r / mg.pf_nz, bz = r - by * mg.pf_nz;
            prefill_tile<KV, D, true>(pp, bx, by, bz, 0, lds);
            __syncthreads();  // the next item reuses the LDS
        }
    } else {
        // decode worker 0 .. NDEC CUs - 1, the head groups of one range adjacent
        const int di = xcd * NDEC * per_cu + NDEC * trip + role;
        const int bx = di / mg.dec_hg, by = di - bx * mg.dec_hg;
        if (bx < dp.page_grid) decode_page_body<KV, D, 4, true>(dp, bx, by, dp.page_grid);
    }
}

template <int KV, int D>
size_t mixed_lds(int max_blocks) {
    constexpr bool BYTES = KV != VCPP_KV_F16;
    constexpr size_t pf = BYTES ? (size_t)ByteDims<D, KV == VCPP_KV_I8, true>::STAGES *
                                          ByteDims<D, KV == VCPP_KV_I8, true>::STAGE +
                                      2 * (size_t)DmaDims<D, true>::STAGE
                                : (size_t)DmaDims<D, true>::STAGES * DmaDims<D, true>::STAGE;
    return std::max<size_t>(PageCfg<KV, D, 4, true>::LDS, pf + (size_t)max_blocks * 4);
}

template <int KV, int D>
hipError_t launch_mixed_kd(const DecodeParams& dp, const PrefillParams& pp, int cus, hipStream_t stream) {
    const size_t lds = mixed_lds<KV, D>(pp.max_blocks);
    static bool attr_set[64] = {};
    int dev = 0;
    if (lds > 65536 && (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64 || !attr_set[dev])) {
        const hipError_t e = hipFuncSetAttribute((const void*)mixed_step_kernel<KV, D>,
                                                 hipFuncAttributeMaxDynamicSharedMemorySize,
                                                 160 * 1024 / kMixedWpc);
        if (e != hipSuccess) return e;
        if (dev >= 0 && dev < 64) attr_set[dev] = true;
    }
    MixedGrid mg;
    constexpr int QT = 16 * PDims<D, true>::RB;
    mg.pf_nz = pp.num_kv_heads * pp.head_groups;
    mg.pf_nyz = pp.num_chunks * mg.pf_nz;
    mg.pf_items = (pp.max_chunk_len + QT - 1) / QT * mg.pf_nyz;
    mg.dec_hg = dp.num_kv_heads / 4;
    hipLaunchKernelGGL((mixed_step_kernel<KV, D>), dim3(kMixedWpc * cus), dim3(256), lds, stream, dp, pp, mg);
    return hipGetLastError();
}

template <int KV>
hipError_t launch_page_kv(const DecodeParams& p, hipStream_t stream) {
    switch (decode_page_heads(p.kv_dtype, p.num_kv_heads, p.head_dim)) {
        case 8: return p.head_dim == 64 ? launch_page<KV, 64, 8>(p, stream) : launch_page<KV, 80, 8>(p, stream);
        case 4:
            if (p.head_dim == 64) return launch_page<KV, 64, 4>(p, stream);
            if (p.head_dim == 80) return launch_page<KV, 80, 4>(p, stream);
            return launch_page<KV, 128, 4>(p, stream);
        default: return hipErrorInvalidValue;
    }
}

template <int KV, int D, int TPS, int NBUF>
hipError_t launch_shape(const DecodeParams& p, hipStream_t stream) {
    const int wpw = p.pairs < kWavesPerGroup ? p.pairs : kWavesPerGroup;
    dim3 grid(p.num_wg, (p.pairs + wpw - 1) / wpw);
    const size_t lds = (size_t)wpw * TPS * kTile * D * sizeof(_Float16);
    hipLaunchKernelGGL((decode_mfma_kernel<KV, D, TPS, NBUF>), grid, dim3(wpw * 64), lds, stream, p);
    return hipGetLastError();
}

template <int KV, int D>
hipError_t launch_mfma(const DecodeParams& p, hipStream_t stream) {
    switch (p.pipeline) {
        case 2: return launch_shape<KV, D, 2, 4>(p, stream);
        case 3: return launch_shape<KV, D, 1, 6>(p, stream);
        case 4: return launch_shape<KV, D, 1, 8>(p, stream);
        case 5: return launch_shape<KV, D, 4, 2>(p, stream);
        default:
            // 2 tiles x 3 buffers fits 256 VGPRs without spills up to
            // head_dim 80; wider heads take 1 tile x 4 buffers.
            if constexpr (D <= 80) return launch_shape<KV, D, 2, 3>(p, stream);
            else return launch_shape<KV, D, 1, 4>(p, stream);
    }
}

}  // namespace

int decode_group_count(int pairs) {
    const int wpw = pairs < kWavesPerGroup ? pairs : kWavesPerGroup;
    return (pairs + wpw - 1) / wpw;
}

hipError_t launch_decode(const DecodeParams& p, hipStream_t stream, const MergeFork* mf, bool* forked) {
    if (p.num_seqs == 0) return hipSuccess;
    hipError_t err;
    const bool prof = prof_enabled();
    if (p.kv_dtype == VCPP_KV_F32) {
        if (prof) prof_begin(kKernelDecode, stream);
        const int qchunks = (p.group + kF32Heads - 1) / kF32Heads;
        dim3 grid(p.max_parts, p.num_seqs, p.num_kv_heads * qchunks);
        DecodeParams pf = p;
        pf.qchunks = qchunks;
        const size_t lds = sizeof(float) * ((size_t)kF32Heads * p.head_dim + (size_t)kF32Tile * (p.head_dim + 1) +
                                            (size_t)kF32Tile * p.head_dim + kF32Heads * kF32Tile + 24);
        if (lds > 65536) {  // head_dim > 128: raise the kernel's dynamic LDS limit (per device)
            static bool attr_set[64] = {};
            int dev = 0;
            if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64 || !attr_set[dev]) {
                const hipError_t e = hipFuncSetAttribute((const void*)decode_f32_kernel,
                                                         hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
                if (e != hipSuccess) return e;
                if (dev >= 0 && dev < 64) attr_set[dev] = true;
            }
        }
        hipLaunchKernelGGL(decode_f32_kernel, grid, dim3(256), lds, stream, pf);
        err = hipGetLastError();
        if (err != hipSuccess) return err;
        if (prof) prof_end(kKernelDecode, stream);
        if (p.max_parts > 1) {
            if (prof) prof_begin(kKernelMerge, stream);
            dim3 mg(p.num_seqs, (p.num_heads + 3) / 4);
            hipLaunchKernelGGL(merge_parts_kernel, mg, dim3(256), 0, stream, p);
            err = hipGetLastError();
            if (prof) prof_end(kKernelMerge, stream);
        }
        return err;
    }
    if (prof) prof_begin(kKernelDecode, stream);
#define VCPP_DISPATCH_D(KVT)                                              \
    switch (p.head_dim) {                                                 \
        case 64: err = launch_mfma<KVT, 64>(p, stream); break;            \
        case 80: err = launch_mfma<KVT, 80>(p, stream); break;            \
        case 128: err = launch_mfma<KVT, 128>(p, stream); break;          \
        default: return hipErrorInvalidValue;                             \
    }
    if (p.page_mode) {
        if (p.kv_dtype == VCPP_KV_I8) err = launch_page_kv<VCPP_KV_I8>(p, stream);
        else if (p.kv_dtype == VCPP_KV_FP8) err = launch_page_kv<VCPP_KV_FP8>(p, stream);
        else err = launch_page_kv<VCPP_KV_F16>(p, stream);
    } else if (p.kv_dtype == VCPP_KV_F16) {
        VCPP_DISPATCH_D(VCPP_KV_F16)
    } else if (p.kv_dtype == VCPP_KV_FP8) {
        VCPP_DISPATCH_D(VCPP_KV_FP8)
    } else {
        VCPP_DISPATCH_D(VCPP_KV_I8)
    }
#undef VCPP_DISPATCH_D
    if (err != hipSuccess) return err;
    if (prof) prof_end(kKernelDecode, stream);
    if (mf) {
        err = hipEventRecord(mf->fork, stream);
        if (err == hipSuccess) err = hipStreamWaitEvent(mf->side, mf->fork, 0);
        if (err != hipSuccess) return err;
        if (forked) *forked = true;
        stream = mf->side;
    }
    if (prof) prof_begin(kKernelMerge, stream);
    dim3 mg(p.num_seqs, (p.pairs + 3) / 4);
    switch (p.head_dim) {
        case 64: hipLaunchKernelGGL(merge_split_kernel<64>, mg, dim3(256), 0, stream, p); break;
        case 80: hipLaunchKernelGGL(merge_split_kernel<80>, mg, dim3(256), 0, stream, p); break;
        default: hipLaunchKernelGGL(merge_split_kernel<128>, mg, dim3(256), 0, stream, p); break;
    }
    err = hipGetLastError();
    if (prof) prof_end(kKernelMerge, stream);
    if (mf) {  // recorded even after a failed merge launch, so the caller can always join
        const hipError_t ej = hipEventRecord(mf->join, stream);
        if (err == hipSuccess) err = ej;
    }
    return err;
}

int decode_page_heads(int kv_dtype, int num_kv_heads, int head_dim) {
    if (kv_dtype != VCPP_KV_F16 && kv_dtype != VCPP_KV_I8 && kv_dtype != VCPP_KV_FP8) return 0;
    if ((head_dim == 64 || head_dim == 80) && num_kv_heads % 8 == 0) return 8;
    if ((head_dim == 64 || head_dim == 80 || head_dim == 128) && num_kv_heads % 4 == 0) return 4;
    return 0;
}

int decode_page_wg_per_cu(int kv_dtype, int num_kv_heads, int head_dim) {
    const int hw = decode_page_heads(kv_dtype, num_kv_heads, head_dim);
#define VCPP_WPC(KVT)                                                                  \
    (hw == 8 ? (head_dim == 64 ? PageCfg<KVT, 64, 8>::WPC : PageCfg<KVT, 80, 8>::WPC) \
     : head_dim == 64 ? PageCfg<KVT, 64, 4>::WPC                                       \
     : head_dim == 80 ? PageCfg<KVT, 80, 4>::WPC : PageCfg<KVT, 128, 4>::WPC)
    if (hw == 0) return 1;
    if (kv_dtype == VCPP_KV_I8) return VCPP_WPC(VCPP_KV_I8);
    if (kv_dtype == VCPP_KV_FP8) return VCPP_WPC(VCPP_KV_FP8);
    return VCPP_WPC(VCPP_KV_F16);
#undef VCPP_WPC
}

bool decode_page_mode_supported(int kv_dtype, int num_kv_heads, int group, int head_dim,
                                int block_size) {
    return decode_page_heads(kv_dtype, num_kv_heads, head_dim) > 0 && group <= 8 &&
           block_size % kTile == 0;
}

bool decode_head_dim_supported(int kv_dtype, int head_dim) {
    if (kv_dtype == VCPP_KV_F32) return head_dim > 0 && head_dim <= 256 && head_dim % 4 == 0;
    return head_dim == 64 || head_dim == 80 || head_dim == 128;
}

int mixed_decode_grid(int kv_dtype, int num_kv_heads, int group, int head_dim, int block_size, int cus) {
    if (kv_dtype != VCPP_KV_F16 && kv_dtype != VCPP_KV_I8 && kv_dtype != VCPP_KV_FP8) return 0;
    if ((head_dim != 64 && head_dim != 80) || num_kv_heads % 4 != 0 || group > 8 || block_size % kTile != 0)
        return 0;
    const int hg = num_kv_heads / 4;
    const int ndec = kMixedWpc - kMixedPrefill;
    if (cus <= 0 || cus % 8 != 0 || (ndec * cus / 8) % hg != 0) return 0;
    return ndec * cus / hg;
}

size_t mixed_lds_bytes(int kv_dtype, int head_dim, int max_blocks) {
#define VCPP_MIXED_LDS(KVT) (head_dim == 64 ? mixed_lds<KVT, 64>(max_blocks) : mixed_lds<KVT, 80>(max_blocks))
    if (kv_dtype == VCPP_KV_I8) return VCPP_MIXED_LDS(VCPP_KV_I8);
    if (kv_dtype == VCPP_KV_FP8) return VCPP_MIXED_LDS(VCPP_KV_FP8);
    return VCPP_MIXED_LDS(VCPP_KV_F16);
#undef VCPP_MIXED_LDS
}

hipError_t launch_mixed(const DecodeParams& dp, const PrefillParams& pp, int cus, hipStream_t stream) {
    hipError_t err;
    const bool prof = prof_enabled();
    if (prof) prof_begin(kKernelMixed, stream);
#define VCPP_MIXED_D(KVT)                                                                          \
    err = dp.head_dim == 64 ? launch_mixed_kd<KVT, 64>(dp, pp, cus, stream) : launch_mixed_kd<KVT, 80>(dp, pp, cus, stream);
    if (dp.kv_dtype == VCPP_KV_I8) {
        VCPP_MIXED_D(VCPP_KV_I8)
    } else if (dp.kv_dtype == VCPP_KV_FP8) {
        VCPP_MIXED_D(VCPP_KV_FP8)
    } else {
        VCPP_MIXED_D(VCPP_KV_F16)
    }
#undef VCPP_MIXED_D
    if (err != hipSuccess) return err;
    if (prof) prof_end(kKernelMixed, stream);
    if (prof) prof_begin(kKernelMerge, stream);
    dim3 mgr(dp.num_seqs, (dp.pairs + 3) / 4);
    if (dp.head_dim == 64) hipLaunchKernelGGL(merge_split_kernel<64>, mgr, dim3(256), 0, stream, dp);
    else hipLaunchKernelGGL(merge_split_kernel<80>, mgr, dim3(256), 0, stream, dp);
    err = hipGetLastError();
    if (prof) prof_end(kKernelMerge, stream);
    return err;
}

}  // namespace vcpp
