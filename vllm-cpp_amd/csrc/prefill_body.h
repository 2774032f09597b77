// prefill_body.h -- the chunked causal prefill workgroup (prefill_tile) for
// gfx950, shared by the prefill kernel (prefill.hip) and the fused mixed-step
// kernel (decode.hip).
//
//
// Reference semantics: the engine prefills one position at a time, writing
// that position's K/V and attending over positions 0..pos
// (src/paged_engine.cpp:348-384, src/model.cpp:1214-1220), i.e. query row i
// of a chunk appended to a prefix of p tokens sees positions 0..p+i, through
// the same paged softmax as src/paged_attention.cpp:11-90 (scale
// 1/sqrt(head_dim), sum + 1e-9, invalid / missing blocks skipped).  The
// reference's GPU slot for dense attention is flash_attention_cuda
// (cuda/attention.cu:58-124); its host loops are not followed.
//
// Work decomposition: a workgroup = (16*RB-token query tile, chunk, kv head,
// group of 4 query heads); one wave per query head holds RB row blocks of 16
// query tokens.  Keys stream in blocks of 32 through a ring of LDS stages that
// the workgroup fills with direct-to-LDS DMA (global_load_lds_dwordx4, one
// page lookup per lane, explicit vmcnt bookkeeping), two blocks per barrier.
// Byte pages (int8, FP8) arrive raw and are widened by the workgroup into an
// fp16 area: FP8 to its values, int8 K to exact integers (its per-key scale
// joins the exp's fma below) and int8 V to fp16(v * scale).  Per row block
// and key block:
//   S^T[32 keys][16 rows] = K_blk x Q^T   (16x16x32 f16; at D = 80 the 16-dim
//                                          remainder reads an LDS zero slot in
//                                          the upper k half)
//   P = exp2(fma(S, scale, -m)) as fp16   (scale = log2(e)/sqrt(D), times the
//                                          key's scale on int8 pages)
//   O[16 rows][D]        += P x V_blk     (16x16x32 f16, P straight from the
//                                          S^T accumulator layout)
// Row sums are v_dot2 sums of exactly the fp16 P that multiplies V.  The
// running max moves lazily: only when a row's max grows by more than 2^8,
// detected after the exp from the lane's block sum of P (so most blocks form
// no max at all).  Causal masks are applied only on key blocks that reach
// past the first query token of the tile.
#pragma once

#include "device_common.h"
#include "prefill.h"

#include <algorithm>
#include <type_traits>

namespace vcpp {

namespace {

constexpr int kKBlk = 32;   // keys per block
constexpr int kHeadsPerGroup = 4;
constexpr float kLazy = 8.0f;  // log2 of the largest P allowed before rescaling
constexpr float kLazyP = 256.0f;  // 2^kLazy

typedef short s4 __attribute__((ext_vector_type(4)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) char lds_char;

// F: the fused mixed-step variant (three workgroups per CU): 32 query rows per
// wave and 4-stage rings, so that its registers and LDS leave room for two
// decode workgroups beside it.
template <int D, bool F = false>
struct PDims {
    static constexpr int NC32 = D / 32;
    static constexpr int REM = (D % 32) / 16;
    static constexpr int NT = D / 16;
#ifdef VCPP_PF_RB
    static constexpr int RB = VCPP_PF_RB;
#else
    static constexpr int RB = D <= 80 && !F ? 4 : 2;  // 16-token row blocks per wave
#endif
    static constexpr int QT = 16 * RB;          // query tokens per workgroup
    static constexpr int CHUNKS = D / 8;        // 16-byte chunks per K/V row
    // LDS row pitch: 16 bytes of padding make the 16-byte K fragment reads of
    // 16 consecutive rows hit 16 distinct 4-bank groups.
    static constexpr int PITCH = D * 2 + 16;
};

__device__ __forceinline__ h4 read_tr(lds_char* a) {
    const s4 x = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        reinterpret_cast<__attribute__((address_space(3))) s4*>(a));
    return __builtin_bit_cast(h4, x);
}

// ---------------------------------------------------------------------------
// fp16 pages: direct-to-LDS gathers through a ring of kStages key blocks.
//
// LDS layout of one stage: K then V, each [chunk][32 keys] of 16-byte chunks
// (chunk = 8 consecutive dims); in odd chunks the key index is XORed with 12.
// That makes the 16 rows of a K fragment read and the 8-byte transposing V
// reads of 32 lanes fall on distinct banks.  Each wave-wide DMA instruction
// fills 64 consecutive chunk slots (1 KiB); a lane picks the page address of
// the slot it fills, or a zero chunk for keys that are past the tile, on a
// missing page or out of the pool.

__device__ __attribute__((aligned(16))) const uint32_t kZeroChunk[4] = {0, 0, 0, 0};

template <int D, bool F = false>
struct DmaDims {
    static constexpr int NCH = D / 8;              // 16-byte chunks per row
    static constexpr int REGION = kKBlk * NCH;     // chunk slots of K (or V) per stage
    static constexpr int NINST = 2 * REGION / 64;  // wave DMA instructions per stage
    static constexpr int PERW = (NINST + 3) / 4;   // per wave (waves < NINST % 4 do one more)
    static constexpr int ZERO = 2 * REGION * 16;   // offset of a 16-byte zero slot
    static constexpr int STAGE = ZERO + 16;        // bytes
#ifdef VCPP_PF_STAGES
    static constexpr int STAGES = VCPP_PF_STAGES;
#else
    static constexpr int STAGES = D <= 80 && !F ? 6 : 4; // ring depth (LDS: <= 64 KiB)
#endif
    static_assert((2 * REGION) % 64 == 0, "stage must be whole DMA instructions");
};

// Key XOR of odd chunks (bits 2 and 3: keys 4 apart land in other banks too).
// 8 and 4 measured the same for fp16 pages; 12 was ~2 % faster for int8 ones.
constexpr int kSwz = 12;
__device__ __forceinline__ int slot_of(int chunk, int key) { return chunk * kKBlk + (key ^ ((chunk & 1) * kSwz)); }

// int8 pages: raw K/V chunks ([chunk of 16 dims][32 keys], 16 bytes per
// slot, K region then V region) and the 32 + 32 fp16 scales of the block (one
// dword per lane), dequantised by the workgroup into fp16 DmaDims stages.
template <int D, bool SCALED, bool F = false>
struct ByteDims {
    static constexpr int NCH = D / 16;             // 16-byte chunks of one byte per value per row
    static constexpr int REGION = kKBlk * NCH;     // slots of K (or V)
    static constexpr int NDATA = 2 * REGION / 64;  // data DMA instructions per block
    static constexpr int NINST = NDATA + (SCALED ? 1 : 0);  // int8: + one for the scales
    static constexpr int PERW = (NINST + 3) / 4;
    static constexpr int SCALES = 2 * REGION * 16; // offset of the scale dwords
    static constexpr int STAGE = SCALES + (SCALED ? 64 * 4 : 0);
    static constexpr int STAGES = D <= 80 && !F ? 8 : 4; // ring depth
    static constexpr int UNITS = 2 * REGION;       // widening units (16 values) per block
    static_assert((2 * REGION) % 64 == 0, "byte stage must be whole DMA instructions");
};


template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// 16 bytes from global memory to LDS (m0 = wave's destination base; lane l
// writes bytes [16 l, 16 l + 16) after it).
// m0 is saved and restored around the load: the compiler does not honour a
// clobber of it.  Default cache policy: a chunk's K/V pages are gathered by
// every query tile and head group, and the re-reads hit L2 (a non-temporal
// load, as decode uses, measured 797 -> 1091 us on config 3).
__device__ __forceinline__ void dma16(const void* src, uint32_t lds_base) {
    uint32_t saved;
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %2, off\n\ts_mov_b32 m0, %0"
                 : "=&s"(saved) : "s"(lds_base), "v"(src) : "memory");
}

// 2 bytes from global memory to LDS, zero-extended into lane l's dword.
__device__ __forceinline__ void dma2(const void* src, uint32_t lds_base) {
    uint32_t saved;
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\tglobal_load_lds_ushort %2, off\n\ts_mov_b32 m0, %0"
                 : "=&s"(saved) : "s"(lds_base), "v"(src) : "memory");
}

// IEEE maximum (NaN-propagating): no operand canonicalisation, and gfx950
// fuses three-input forms into v_maximum3_f32.
__device__ __forceinline__ float vmax(float a, float b) { return __builtin_elementwise_maximum(a, b); }
__device__ __forceinline__ float vmax(float a, float b, float c) { return vmax(vmax(a, b), c); }
__device__ __forceinline__ float vmax3(float a, float b, float c) { return vmax(vmax(a, b), c); }

// Reductions over the four 16-lane groups (lanes l, l ^ 16, l ^ 32, l ^ 48).
// Both run off the hot path (rescales, epilogue), so plain lane shuffles do.
// (hipcc of this ROCm folds the second result of permlane{16,32}_swap with
// identical operands into the first, so those builtins are not used here.)
__device__ __forceinline__ float sum_over_groups(float x) {
    x += shfl_xor(x, 32);
    return x + shfl_xor(x, 16);
}

__device__ __forceinline__ float max_over_groups(float x) {
    x = vmax(x, shfl_xor(x, 32));
    return vmax(x, shfl_xor(x, 16));
}

// One workgroup's work: query tile bx (0 = the chunk's last, heaviest tile)
// of chunk by, kv head / head group bz, key part `part` of p.splits; lds is
// the workgroup's dynamic LDS (prefill_lds_bytes).  Returns with every DMA it
// issued complete.
template <int KV, int D, bool F>
__device__ __forceinline__ void prefill_tile(const PrefillParams& p, int bx, int by, int bz, int part,
                                             lds_char* lds) {
    using DD = DmaDims<D, F>;
    constexpr bool BYTES = KV != VCPP_KV_F16;  // int8 / FP8: byte ring widened to fp16
    constexpr bool SCALED = KV == VCPP_KV_I8;  // per-key fp16 scales
    using ID = ByteDims<D, SCALED, F>;
    // LDS: the DMA ring (fp16 stages, or int8 stages plus an fp16 area of two
    // dequantised blocks), then the tile's block table.
    constexpr int kStages = BYTES ? ID::STAGES : DD::STAGES;
    constexpr int RSTAGE = BYTES ? ID::STAGE : DD::STAGE;
    constexpr int AREA = kStages * RSTAGE;
    constexpr int NF16 = BYTES ? 2 : kStages;       // fp16-format stages
    constexpr int F16BASE = BYTES ? AREA : 0;
    constexpr int SG = SCALED ? 1 : 2;  // row blocks per softmax group (int8: registers)
    constexpr int NC32 = PDims<D>::NC32, NT = PDims<D>::NT;
    constexpr int RB = PDims<D, F>::RB;  // 16-row blocks per wave
    constexpr int kQTile = 16 * RB;
    __attribute__((address_space(3))) int32_t* table_s =
        reinterpret_cast<__attribute__((address_space(3))) int32_t*>(lds + AREA + (BYTES ? 2 * DD::STAGE : 0));
    const uint32_t lds_addr = (uint32_t)(uintptr_t)lds;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, c = lane & 15;
    const int chunk = by;
    const int q0 = p.q_start[chunk], n = p.q_start[chunk + 1] - q0;
    const int ntile = (n + kQTile - 1) / kQTile;
    const int tile = ntile - 1 - bx;  // heaviest (latest) tiles first
    if (tile < 0) return;             // whole workgroup: before any barrier
    const int t0 = tile * kQTile;
    const int prefix = p.prefix_lens[chunk];
    const int kvh = bz / p.head_groups;
    const int hg = bz - kvh * p.head_groups;
    const int hl = hg * kHeadsPerGroup + wave;
    const bool head_ok = hl < p.group;
    const int head = kvh * p.group + (head_ok ? hl : 0);
    const int32_t* table = p.block_tables + (int64_t)chunk * p.max_blocks;
    const int kv_end = prefix + min(t0 + kQTile, n);
    const int nblk = (kv_end + kKBlk - 1) / kKBlk;
    const int nfree = (prefix + t0 + 1) / kKBlk;  // blocks visible to every row
    // This part's key blocks [kb_lo, kb_hi): whole block pairs, the last part
    // up to nblk.
    const int npairs = (nblk + 1) / 2;
    const int kb_lo = 2 * (int)((int64_t)part * npairs / p.splits);
    const int kb_hi = min(2 * (int)((int64_t)(part + 1) * npairs / p.splits), nblk);

    // Q fragments (B operand of S^T = K Q^T).
    h8 qa[RB][NC32 > 0 ? NC32 : 1];
    h8 qr[RB];  // dims 32 NC32 + 8 g.. for g < 2, zero for g >= 2 (16-dim remainder)
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
        const int tok = t0 + 16 * rb + c;
        const bool ok = head_ok && tok < n;
        const _Float16* qrow =
            reinterpret_cast<const _Float16*>(p.q) + ((int64_t)(q0 + (ok ? tok : 0)) * p.num_heads + head) * D;
#pragma unroll
        for (int cc = 0; cc < NC32; ++cc)
            qa[rb][cc] = ok ? *reinterpret_cast<const h8*>(qrow + 32 * cc + 8 * g) : h8{};
        if constexpr (PDims<D>::REM)
            qr[rb] = ok && g < 2 ? *reinterpret_cast<const h8*>(qrow + 32 * NC32 + 8 * g) : h8{};
    }
    if (tid < NF16) {
        *reinterpret_cast<__attribute__((address_space(3))) h8*>(lds + F16BASE + tid * DD::STAGE + DD::ZERO) = h8{};
    }
    // Stage the tile's block ids (validated) in LDS; note any bad entry.
    const int npages = min((kv_end + p.block_size - 1) / p.block_size, p.max_blocks);
    int bad = 0;
    for (int i = tid; i < npages; i += 256) {
        const int bid = table[i];
        const bool ok = bid >= 0 && (int64_t)bid < p.num_blocks;
        table_s[i] = ok ? bid : -1;
        bad |= !ok;
    }
    const bool any_bad = __syncthreads_or(bad) != 0;
    // Q (and table) loads complete here, in a wait the compiler sees: the
    // ring's DMA below is invisible to its counter bookkeeping, which would
    // otherwise wait for everything at the Q fragments' first use in the loop.
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    // Positions covered by the table: keys at or past tab_end are skipped.
    const int tab_end = npages * p.block_size;

    // DMA lanes.  Instruction j = wave + 4 i fills chunk slots 64 j + lane of
    // the stage: region (K or V) and chunk pair are uniform per instruction,
    // and every instruction's lane l carries key (l & 31) ^ 12 (l >> 5) of
    // chunk 2 (j mod 2R/64) + (l >> 5) -- one page lookup per lane serves all.
    constexpr int PERW = DD::PERW;
    const int my_inst = wave < (DD::NINST & 3) || (DD::NINST & 3) == 0 ? PERW : PERW - 1;
    const int dkey = (lane & 31) ^ ((lane >> 5) * kSwz);
    const int64_t row_bytes = (int64_t)p.num_kv_heads * D * 2;
    const int64_t page_bytes = p.block_stride * 2;
    const int64_t lane_off = (int64_t)kvh * D * 2 + (lane >> 5) * 16;
    auto issue = [&](int kb) {  // DMA key block kb into stage kb % kStages
        const uint32_t sbase = lds_addr + (kb % kStages) * DD::STAGE;
        const int pos = kb * kKBlk + dkey;
        int64_t off = -1;
        if (pos < kv_end && pos < tab_end) {
            const int lb = (int)(((uint64_t)(uint32_t)pos * p.bs_magic) >> 40);
            const int bid = table_s[lb];
            if (bid >= 0) off = bid * page_bytes + (pos - lb * p.block_size) * row_bytes + lane_off;
#ifdef VCPP_GATHER_DUMP
            if (bid >= 0 && wave == 0 && kvh == 0 && hg == 0) gather_record(p, chunk, pos, bid, pos - lb * p.block_size);
#endif
        }
#pragma unroll
        for (int i = 0; i < PERW; ++i) {
            if (i < my_inst) {
                const int j = wave + 4 * i;
                const int which = j >= DD::REGION / 64;               // uniform
                const int cp = j - which * (DD::REGION / 64);          // chunk pair
                const char* base = static_cast<const char*>(which ? p.v : p.k) + cp * 32;
                const void* src = off >= 0 ? (const void*)(base + off) : (const void*)kZeroChunk;
                dma16(src, __builtin_amdgcn_readfirstlane(sbase + j * 1024));
            }
        }
    };

    // int8: instruction j = wave + 4 i (j < NDATA) fills slots 64 j + lane,
    // whose key is lane & 31 for every j; the last instruction brings the
    // scales (lanes 0-31 K, 32-63 V).
    constexpr int PERW8 = ID::PERW;
    const int my_inst8 = (ID::NINST & 3) == 0 || wave < (ID::NINST & 3) ? PERW8 : PERW8 - 1;
    auto issue8 = [&](int kb) {
        const uint32_t sbase = lds_addr + (kb % kStages) * RSTAGE;
        const int key = lane & 31;
        const int pos = kb * kKBlk + key;
        int64_t off = -1, soff = 0;
        if (pos < kv_end && pos < tab_end) {
            const int lb = (int)(((uint64_t)(uint32_t)pos * p.bs_magic) >> 40);
            const int bid = table_s[lb];
            if (bid >= 0) {
                const int slot = pos - lb * p.block_size;
                off = bid * p.block_stride + ((int64_t)slot * p.num_kv_heads + kvh) * D;
                soff = ((int64_t)bid * p.scale_block_stride + (int64_t)kvh * p.block_size + slot) * 2;
#ifdef VCPP_GATHER_DUMP
                if (wave == 0 && lane < 32 && kvh == 0 && hg == 0) gather_record(p, chunk, pos, bid, slot);
#endif
            }
        }
#pragma unroll
        for (int i = 0; i < PERW8; ++i) {
            if (i < my_inst8) {
                const int j = wave + 4 * i;
                if (j < ID::NDATA) {
                    const int sl = 64 * j + lane;
                    const int which = sl >= ID::REGION;
                    const int ch = (sl - which * ID::REGION) >> 5;
                    const char* base = static_cast<const char*>(which ? p.v : p.k) + ch * 16;
                    dma16(off >= 0 ? (const void*)(base + off) : (const void*)kZeroChunk,
                          __builtin_amdgcn_readfirstlane(sbase + j * 1024));
                } else {
                    const char* base = reinterpret_cast<const char*>(lane >> 5 ? p.v_scale : p.k_scale);
                    dma2(off >= 0 ? (const void*)(base + soff) : (const void*)kZeroChunk,
                         __builtin_amdgcn_readfirstlane(sbase + ID::SCALES));
                }
            }
        }
    };
    // Block kb (byte ring) -> fp16 block kb & 1 of the fp16 area.  FP8: the
    // values.  int8: K as exact fp16 integers, its per-key scale times
    // log2(e)/sqrt(D) converted in place to fp32 for the exp's fma (at least
    // FLT_MIN, so a masked key's -inf never meets a zero scale); V times its
    // key's scale, one IEEE fp16 rounding of the exact product
    // (v_pk_mul_f16).
    auto widen = [&](int kb) {
        lds_char* st = lds + (kb % kStages) * RSTAGE;
        if constexpr (SCALED) {
            if (tid < 32) {
                lds_char* sw = st + ID::SCALES + tid * 4;
                const float ks = (float)__builtin_bit_cast(
                    _Float16, *reinterpret_cast<__attribute__((address_space(3))) const uint16_t*>(sw));
                *reinterpret_cast<__attribute__((address_space(3))) float*>(sw) =
                    fmaxf(ks * p.scale_log2, 1.17549435e-38f);
            }
        }
        lds_char* dst0 = lds + AREA + (kb & 1) * DD::STAGE;
#pragma unroll
        for (int u0 = 0; u0 < ID::UNITS; u0 += 256) {
            const int v = u0 + tid;
            if (v < ID::UNITS) {
                const int which = v >= ID::REGION;
                const int q = v - which * ID::REGION;
                const int ch = q >> 5, key = q & 31;
                const i4 raw = *reinterpret_cast<__attribute__((address_space(3))) i4*>(st + v * 16);
                h8 lo = bytes8_to_h8<KV>((uint32_t)raw.x, (uint32_t)raw.y);
                h8 hi = bytes8_to_h8<KV>((uint32_t)raw.z, (uint32_t)raw.w);
                if constexpr (SCALED) {
                    if (which) {  // V scale dword of the key: fp16 in the low half
                        const _Float16 sc = __builtin_bit_cast(_Float16, *reinterpret_cast<
                            __attribute__((address_space(3))) const uint16_t*>(st + ID::SCALES + (32 + key) * 4));
                        lo *= sc;
                        hi *= sc;
                    }
                }
                lds_char* dst = dst0 + which * DD::REGION * 16;
                *reinterpret_cast<__attribute__((address_space(3))) h8*>(dst + slot_of(2 * ch, key) * 16) = lo;
                *reinterpret_cast<__attribute__((address_space(3))) h8*>(dst + slot_of(2 * ch + 1, key) * 16) = hi;
            }
        }
    };

    f4 o[RB][NT];
    // Per-lane partial row sums of the fp16 P that weights V (row c, this
    // lane's keys), summed over the four lane groups at the end.
    float lsum[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int t = 0; t < NT; ++t) o[rb][t] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) lsum[rb] = 0.f;
    // Running max per row (log2 units).
    float m_run[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) m_run[rb] = kMaxSeed;

    // LDS byte offsets of this lane's fragment reads: one base each plus
    // compile-time offsets.  K row 16 kt + c of chunk 4 cc + g sits in slot
    // (4 cc + g) 32 + 16 kt + (c ^ 12 (g & 1)); V rows 16 hh + 4 g + c / 4 of
    // chunk 2 t + (c & 3) / 2 likewise.
    const int kbase = (32 * g + (c ^ ((g & 1) * kSwz))) * 16;
    // The 16-dim remainder (D = 80) runs as a 16x16x32 MFMA whose upper half
    // (lanes g >= 2) reads the stage's zero slot (Q side zero too).
    const int rpar = (4 * NC32 + g) & 1;
    const int krb0 = g < 2 ? ((4 * NC32 + g) * 32 + (c ^ (rpar * kSwz))) * 16 : DD::ZERO;
    const int krb1 = g < 2 ? krb0 + 16 * 16 : krb0;
    const int vpar = (c >> 1) & 1;
    const int vbase = DD::REGION * 16 + (((c & 3) >> 1) * 32 + ((4 * g + (c >> 2)) ^ (vpar * kSwz))) * 16 + 8 * (c & 1);

    auto compute = [&](int kb, auto masked_tag) {
        constexpr bool MASKED = decltype(masked_tag)::value;
        lds_char* sb = BYTES ? lds + AREA + (kb & 1) * DD::STAGE : lds + (kb % kStages) * DD::STAGE;
        const int key0 = kb * kKBlk;
        h8 ka[2][NC32 > 0 ? NC32 : 1];
        h8 kr[2];
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
            for (int cc = 0; cc < NC32; ++cc)
                ka[kt][cc] = *reinterpret_cast<__attribute__((address_space(3))) h8*>(sb + kbase + (128 * cc + 16 * kt) * 16);
            if constexpr (PDims<D>::REM)
                kr[kt] = *reinterpret_cast<__attribute__((address_space(3))) h8*>(sb + (kt ? krb1 : krb0));
        }
        h8 vb[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const h4 lo = read_tr(sb + vbase + 64 * t * 16);
            const h4 hi = read_tr(sb + vbase + (64 * t + 16) * 16);
            vb[t] = h8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        }
        bool tile_ok[2] = {true, true};
        if constexpr (MASKED) {
#pragma unroll
            for (int kt = 0; kt < 2; ++kt) {
                const int k16 = key0 + 16 * kt;
                const int lb = k16 / p.block_size;
                tile_ok[kt] = k16 < tab_end && table_s[lb] >= 0;
            }
        }
        // Row blocks go in groups of SG: raw S^T, then exp of the scaled,
        // shifted scores (one fma each) and P V.
        auto s_group = [&](int rb0, float (&sc)[SG][2][4]) {
#pragma unroll
            for (int i = 0; i < SG; ++i) {
                const int rb = rb0 + i;
#pragma unroll
                for (int kt = 0; kt < 2; ++kt) {
                    f4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int cc = 0; cc < NC32; ++cc) acc = mfma32(ka[kt][cc], qa[rb][cc], acc);
                    if constexpr (PDims<D>::REM) acc = mfma32(kr[kt], qr[rb], acc);
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        float x = acc[r];
                        if constexpr (MASKED) {
                            const int key = key0 + 16 * kt + 4 * g + r;
                            const int lim = min(prefix + t0 + 16 * rb + c, kv_end - 1);
                            x = (tile_ok[kt] && key <= lim) ? x : -__builtin_inff();
                        }
                        sc[i][kt][r] = x;
                    }
                }
            }
        };
        // Exp first, check after.  With the running max m, a
        // score past the lazy threshold (m + kLazy in log2 units) has
        // P > 2^kLazy, and one far past it overflows fp16 to inf, so the
        // lane's block sum of P -- which the row sum needs anyway --
        // exceeds 2^kLazy whenever a row of the lane must be rescaled
        // (rarely otherwise).  Only then is the row max formed, and the
        // group's P recomputed if the max moved.  The exp of group j runs
        // under the S^T MFMAs of group j + 1.
        float sc[2][SG][2][4];
        h8 pa[SG];
        float bs[SG];
        // Score scale of this lane's keys 16 kt + 4 g + r: log2(e)/sqrt(D),
        // times the key's scale on int8 pages (read where it is used).
        auto score_scale = [&](float (&ksc)[2][4]) {
#pragma unroll
            for (int kt = 0; kt < 2; ++kt) {
                if constexpr (SCALED) {
                    const f4 w = *reinterpret_cast<__attribute__((address_space(3))) const f4*>(
                        lds + (kb % kStages) * RSTAGE + ID::SCALES + (16 * kt + 4 * g) * 4);
#pragma unroll
                    for (int r = 0; r < 4; ++r) ksc[kt][r] = w[r];
                } else {
#pragma unroll
                    for (int r = 0; r < 4; ++r) ksc[kt][r] = p.scale_log2;
                }
            }
        };
        auto p_sum = [&](int i, int rb, const float (&sci)[2][4]) {
            float ksc[2][4];
            score_scale(ksc);
#pragma unroll
            for (int kt = 0; kt < 2; ++kt)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    pa[i][4 * kt + r] = (_Float16)fast_exp2(fmaf(sci[kt][r], ksc[kt][r], -m_run[rb]));
            float b = 0.f;
#pragma unroll
            for (int e = 0; e < 8; e += 2)
                b = __builtin_amdgcn_fdot2(h2{pa[i][e], pa[i][e + 1]}, h2{1, 1}, b, false);
            bs[i] = b;
        };
        s_group(0, sc[0]);
#pragma unroll
        for (int j = 0; j < RB / SG; ++j) {
            const bool more = j + 1 < RB / SG;
            const int nx = (j + 1) & 1;
#pragma unroll
            for (int i = 0; i < SG; ++i) p_sum(i, j * SG + i, sc[j & 1][i]);
            if (more) s_group((j + 1) * SG, sc[nx]);
            bool cross = false;
#pragma unroll
            for (int i = 0; i < SG; ++i) cross |= !(bs[i] <= kLazyP);  // inf and NaN too
            if (__builtin_expect(__any(cross), 0)) {
#pragma unroll
                for (int i = 0; i < SG; ++i) {
                    const int rb = j * SG + i;
                    const float (&sci)[2][4] = sc[j & 1][i];
                    float ksc[2][4], x[2][4];
                    score_scale(ksc);
#pragma unroll
                    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
                        for (int r = 0; r < 4; ++r) x[kt][r] = sci[kt][r] * ksc[kt][r];
                    const float ml = max_over_groups(vmax(vmax3(x[0][0], x[0][1], x[0][2]),
                                                          vmax3(x[0][3], x[1][0], x[1][1]),
                                                          vmax3(x[1][2], x[1][3], x[1][3])));
                    const bool grow = ml > m_run[rb] + kLazy;  // uniform per row
                    const float m_new = grow ? ml : m_run[rb];
                    const float alpha = fast_exp2(m_run[rb] - m_new);
                    m_run[rb] = m_new;
                    lsum[rb] *= alpha;  // row c: this lane's own
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const float a = shfl(alpha, 4 * g + r);
#pragma unroll
                        for (int t = 0; t < NT; ++t) o[rb][t][r] *= a;
                    }
                    if (__any(grow)) p_sum(i, rb, sci);
                }
            }
#pragma unroll
            for (int i = 0; i < SG; ++i) {
                lsum[j * SG + i] += bs[i];
#pragma unroll
                for (int t = 0; t < NT; ++t) o[j * SG + i][t] = mfma32(pa[i], vb[t], o[j * SG + i][t]);
            }
        }
    };

    // fp16 pages: a ring of kStages 32-key blocks, consumed two per barrier:
    // while blocks kb, kb + 1 are computed, blocks up to kb + kStages - 1 are
    // in flight.  Byte pages: a ring of kStages byte blocks and two fp16
    // blocks, one block per barrier: block kb is computed from its fp16 copy
    // while block kb + 1 is widened into the other one and blocks up to
    // kb + kStages - 2 are in flight.  Blocks past nblk are issued too (as
    // zero chunks) so that every wave's vmcnt arithmetic below stays exact;
    // on fp16 pages an odd tail block is paired with a fully masked one.
    static_assert(kStages >= 4 && kStages % 2 == 0, "ring holds whole pairs");
    const int free_end = any_bad ? 0 : (min(nfree, nblk) & ~1);
    if constexpr (BYTES) {
#pragma unroll
        for (int s = 0; s < kStages - 1; ++s) issue8(kb_lo + s);
        if (my_inst8 == PERW8) wait_vmcnt<(kStages - 2) * PERW8>();
        else wait_vmcnt<(kStages - 2) * (PERW8 - 1)>();
        __syncthreads();  // block kb_lo landed for every wave
        if (kb_lo < kb_hi) widen(kb_lo);
        auto step8 = [&](int kb) {
            if (my_inst8 == PERW8) wait_vmcnt<(kStages - 3) * PERW8>();
            else wait_vmcnt<(kStages - 3) * (PERW8 - 1)>();
            // Block kb + 1 landed for every wave, block kb widened, block
            // kb - 1 computed (its byte stage and fp16 block are free).
            __syncthreads();
            issue8(kb + kStages - 1);
            if (kb + 1 < kb_hi) widen(kb + 1);
        };
        for (int kb = kb_lo; kb < min(free_end, kb_hi); ++kb) {
            step8(kb);
            compute(kb, std::false_type{});
        }
        for (int kb = max(free_end, kb_lo); kb < kb_hi; ++kb) {
            step8(kb);
            compute(kb, std::true_type{});
        }
    } else {
#pragma unroll
        for (int s = 0; s < kStages - 2; ++s) issue(kb_lo + s);
        auto step = [&](int kb) {
            constexpr int kAhead = kStages - 4;  // blocks allowed in flight at the wait
            if (my_inst == PERW) wait_vmcnt<kAhead * PERW>();
            else wait_vmcnt<kAhead * (PERW - 1)>();
            __syncthreads();  // blocks kb, kb + 1 landed for all waves; kb - 2, kb - 1 consumed
            issue(kb + kStages - 2);
            issue(kb + kStages - 1);
        };
        // Two loops, one inlined compute each (one loop with both variants
        // merges their accumulators and spills).
        for (int kb = kb_lo; kb < min(free_end, kb_hi); kb += 2) {
            step(kb);
#pragma unroll 1
            for (int h = 0; h < 2; ++h) compute(kb + h, std::false_type{});
        }
        for (int kb = max(free_end, kb_lo); kb < kb_hi; kb += 2) {
            step(kb);
#pragma unroll 1
            for (int h = 0; h < 2; ++h) compute(kb + h, std::true_type{});
        }
    }
    wait_vmcnt<0>();

    if (!head_ok) return;  // (no barrier follows)
    if (p.splits > 1) {
        // Part outputs: o unnormalised, (m, l) of each row from lanes g == 0.
        const int64_t pbase = (int64_t)part * p.rows_cap;
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            const float rowsum = sum_over_groups(lsum[rb]);  // row c
            const int tc = t0 + 16 * rb + c;
            // (rows past rows_cap -- chunks longer than max_chunk_len, a
            // caller error -- are not stored, and the merge skips the rows
            // of such chunks that no tile covered: their output stays
            // unwritten)
            if (g == 0 && tc < n && q0 + tc < p.rows_cap)
                p.ws_ml[(pbase + q0 + tc) * p.num_heads + head] = make_float2(m_run[rb], rowsum);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int tok = t0 + 16 * rb + 4 * g + r;
                if (tok < n && q0 + tok < p.rows_cap) {
                    float* orow = p.ws_o + ((pbase + q0 + tok) * p.num_heads + head) * D;
#pragma unroll
                    for (int t = 0; t < NT; ++t) orow[16 * t + c] = o[rb][t][r];
                }
            }
        }
        return;
    }
    // Lane (g, c) holds rows 4 g + r, column 16 t + c.  Column pairs: for the
    // row pair (2 k, 2 k + 1) even lanes store row 2 k and odd lanes row 2 k + 1,
    // each the pair (c & ~1, + 1), the other value one DPP swap away.
    const bool odd = (c & 1) != 0;
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
        const float rowsum = sum_over_groups(lsum[rb]);  // row c
#pragma unroll
        for (int k2 = 0; k2 < 2; ++k2) {
            const int r = 2 * k2 + (odd ? 1 : 0);
            const float inv = 1.0f / (shfl(rowsum, 4 * g + r) + 1e-9f);
            const int tok = t0 + 16 * rb + 4 * g + r;
            float* orow = p.out + ((int64_t)(q0 + min(tok, n - 1)) * p.num_heads + head) * D;
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const float x0 = o[rb][t][2 * k2], x1 = o[rb][t][2 * k2 + 1];
                const float y = dpp_swap1(odd ? x0 : x1);  // neighbour's value of my row
                const float2 v = odd ? make_float2(y * inv, x1 * inv) : make_float2(x0 * inv, y * inv);
                if (tok < n) *reinterpret_cast<float2*>(orow + 16 * t + (c & ~1)) = v;
            }
        }
    }
}

}  // namespace

}  // namespace vcpp
