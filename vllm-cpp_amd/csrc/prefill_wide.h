// prefill_wide.h -- the chunked causal prefill workgroup for fp16 pages at
// head_dim 64 and 80 (prefill_wide_run): 128 query rows per wave, one wave
// per SIMD, the output accumulators and Q fragments in the accumulation
// registers (AGPRs), and the matrix-core and vector work of each key block
// interleaved instruction by instruction inside the wave.
//
// Reference semantics are those of prefill_tile (prefill_body.h): query row
// i of a chunk appended to a prefix of p tokens attends positions 0..p+i
// (src/paged_engine.cpp:348-384, src/model.cpp:1214-1220) through the paged
// softmax of src/paged_attention.cpp:11-90 (scale 1/sqrt(head_dim), sum +
// 1e-9, invalid or missing blocks skipped).
//
// Why this shape.  Per 32-key block a wave issues its S^T = K Q^T and
// O += P V MFMAs (16x16x32 f16) and, for every score, an fma, an exp2, half
// a pack to fp16 and half a dot2 for the row sum.  gfx950 overlaps an MFMA
// with vector instructions only inside one wave's instruction stream (about
// half of a 16x16x32's 16 cycles are free for VALU issue), not across
// waves.  So the work is cut into two halves of 64 rows (A: row blocks 0-3,
// B: 4-7) and software-pipelined over key blocks, each phase one stretch of
// code in which every MFMA is followed by its share of the other half's
// softmax:
//   phase 1 (block kb):  MFMA  S_B(kb), then P_B(kb-1) V(kb-1)
//                        VALU  softmax_A(kb); LDS reads of K(kb+1) once
//                              S_B(kb) is issued
//   phase 2 (block kb):  MFMA  S_A(kb+1), then P_A(kb) V(kb)
//                        VALU  softmax_B(kb); LDS reads of V(kb) before
//                              P_A(kb) V(kb) is issued
// Every MFMA result is first read a whole MFMA group later, and every P a
// whole S group later, so neither side waits for the other.  Each K / V
// fragment read from LDS serves 128 rows (twice the two-waves-per-SIMD
// kernel's 64).  The MFMAs are inline assembly so that the accumulators stay
// in AGPRs (C/D operands) and S stays in VGPRs where the softmax reads it;
// sched_barrier fences keep the interleave as written.
//
// Register budget (D = 80): AGPRs O 8x5x4 = 160 + Q 8x2x4 + 4x4 = 80; VGPRs
// S 64, P 32, K fragments 32, V fragments 20, row state 24.  One K and one V
// fragment set suffice: K(kb + 1) is read after the last MFMA that reads
// K(kb) was issued, V(kb) after the last one that reads V(kb - 1).
#pragma once

#include "prefill_body.h"
#include "prefill_wide_regs.h"

#include <utility>

namespace vcpp {

namespace {

template <int D>
struct WDims {
    static constexpr int NC32 = D / 32;
    static constexpr int REM = (D % 32) / 16;
    // K fragments per 16-key half of a block: the full 32-dim ones, then
    // (D = 80) the 16-dim remainder twice, in the low and in the high k half
    // (see qr below).
    static constexpr int NK = NC32 + 2 * REM;
    static constexpr int NT = D / 16;      // 16-column output blocks
    static constexpr int RB = 8;           // 16-row blocks per wave
    static constexpr int QT = 16 * RB;     // query rows per workgroup tile
    static constexpr int STAGES = 8;       // K/V ring depth (32-key blocks)
    // DMA instructions per wave and block: every wave issues the same
    // number (those past a stage's last instruction fill a 1 KiB dummy
    // area from the zero chunk), so each wave's vmcnt arithmetic is one
    // constant and the issue code has no per-wave branch.
    static constexpr int PERW = DmaDims<D>::PERW;
    static constexpr int DMA_GAP = 8;  // MFMA slots between a wave's DMA instructions
    static constexpr int NS = 4 * 2 * (NC32 + REM);  // S MFMAs of one half
    static constexpr int NPV = 4 * NT;     // P V MFMAs of one half
};

#ifdef VCPP_PF_TIMING
// Timing builds only: per-segment shader-clock sums over all waves.
__device__ unsigned long long g_pf_timing[16];
#define VCPP_T(k) do { const uint64_t t_ = __builtin_amdgcn_s_memtime(); tm[k] += t_ - t_last; t_last = t_; } while (0)
#else
#define VCPP_T(k) do { } while (0)
#endif

template <int D>
constexpr bool wide_prefill_ok() { return D == 64 || D == 80; }

__device__ __forceinline__ void fence() { __builtin_amdgcn_sched_barrier(0); }

// f(integral_constant<int, 0>), ..., f(integral_constant<int, N - 1>).
template <class F, int... I>
__device__ __forceinline__ void static_for_impl(F& f, std::integer_sequence<int, I...>) {
    (f(std::integral_constant<int, I>{}), ...);
}
template <int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
    static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// Tile v of a launch of nx tiles per chunk (heaviest first), ny chunks and
// nz (key part, kv head, head group) combinations: as prefill_dma_kernel
// orders its workgroups, each XCD walks a contiguous range of ids.
__device__ __forceinline__ void wide_tile_ids(int v, int nx, int ny, int nz, int& bx, int& by, int& bz) {
    const int total = nx * ny * nz;
    int m = v;
    if ((total & 7) == 0) m = (v & 7) * (total >> 3) + (v >> 3);
    bx = m % nx;
    by = (m / nx) % ny;
    bz = m / (nx * ny);
}

template <int D>
__device__ __forceinline__ void prefill_wide_run(const PrefillParams& p, lds_char* lds) {
    using W = WDims<D>;
    using DD = DmaDims<D>;
    constexpr int NC32 = W::NC32, NK = W::NK, NT = W::NT, RB = W::RB;
    constexpr int kStages = W::STAGES;
    constexpr int kQTile = W::QT;
    // LDS: the ring, a 1 KiB dummy DMA target, then the tile's block table.
    constexpr int kDummy = kStages * DD::STAGE;
    __attribute__((address_space(3))) int32_t* table_s =
        reinterpret_cast<__attribute__((address_space(3))) int32_t*>(lds + kDummy + 1024);
    const uint32_t lds_addr = (uint32_t)(uintptr_t)lds;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, c = lane & 15;
#ifdef VCPP_PF_TIMING
    uint64_t tm[16] = {};
    uint64_t t_last = __builtin_amdgcn_s_memtime();
#endif
    if (tid < kStages) {
        *reinterpret_cast<__attribute__((address_space(3))) h8*>(lds + tid * DD::STAGE + DD::ZERO) = h8{};
    }

    // This workgroup's tile (a 1-D grid of all tiles).
    const int nx = (p.max_chunk_len + kQTile - 1) / kQTile, ny = p.num_chunks;
    const int nz = p.num_kv_heads * p.head_groups * max(p.splits, 1);

    // Per-tile state (set by plan()).
    int chunk = 0, q0 = 0, n = 0, t0 = 0, prefix = 0, kvh = 0, hg = 0, part = 0, head = 0;
    bool head_ok = false;
    int kv_end = 0, nblk = 0, nfree = 0, kb_lo = 0, kb_hi = 0, npages = 0, tab_end = 0;
    bool any_bad = false;
    auto plan = [&](int v) {  // false: no work in tile v (a chunk shorter than max_chunk_len)
        int bx, by, bz;
        wide_tile_ids(v, nx, ny, nz, bx, by, bz);
        const int zh = p.num_kv_heads * p.head_groups;
        part = bz / zh;
        bz -= part * zh;
        chunk = by;
        q0 = p.q_start[chunk];
        n = p.q_start[chunk + 1] - q0;
        const int ntile = (n + kQTile - 1) / kQTile;
        const int tile = ntile - 1 - bx;  // heaviest (latest) tiles first
        if (tile < 0) return false;
        t0 = tile * kQTile;
        prefix = p.prefix_lens[chunk];
        kvh = bz / p.head_groups;
        hg = bz - kvh * p.head_groups;
        const int hl = hg * kHeadsPerGroup + wave;
        head_ok = hl < p.group;
        head = kvh * p.group + (head_ok ? hl : 0);
        kv_end = prefix + min(t0 + kQTile, n);
        nblk = (kv_end + kKBlk - 1) / kKBlk;
        nfree = (prefix + t0 + 1) / kKBlk;  // blocks visible to every row
        const int npairs = (nblk + 1) / 2;
        kb_lo = 2 * (int)((int64_t)part * npairs / p.splits);
        kb_hi = min(2 * (int)((int64_t)(part + 1) * npairs / p.splits), nblk);
        npages = min((kv_end + p.block_size - 1) / p.block_size, p.max_blocks);
        tab_end = npages * p.block_size;
        return true;
    };

    // Q fragments (B operand of S^T = K Q^T), staged in VGPRs and held in
    // AGPRs by the MFMAs.  The 16-dim remainder (D = 80) of row blocks 2 j
    // and 2 j + 1 shares one fragment: k 0-15 (lanes g < 2) hold row block
    // 2 j's dims, k 16-31 (lanes g >= 2) row block 2 j + 1's.  Each
    // remainder MFMA pairs it with a K fragment that is zero in the other
    // row block's k half.
    h8 qa[RB][NC32];
    h8 qr[RB / 2];
    // Block-table entries of the tile, staged in VGPRs (two per thread; a
    // longer table is read in a loop when it is staged).
    int tb[2];
    auto load_tile = [&]() {  // the global loads of the planned tile
        const int32_t* table = p.block_tables + (int64_t)chunk * p.max_blocks;
#pragma unroll
        for (int i = 0; i < 2; ++i) tb[i] = tid + 256 * i < npages ? table[tid + 256 * i] : -1;
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            const int tok = t0 + 16 * rb + c;
            const bool ok = head_ok && tok < n;
            const _Float16* qrow =
                reinterpret_cast<const _Float16*>(p.q) + ((int64_t)(q0 + (ok ? tok : 0)) * p.num_heads + head) * D;
#pragma unroll
            for (int cc = 0; cc < NC32; ++cc)
                qa[rb][cc] = ok ? *reinterpret_cast<const h8*>(qrow + 32 * cc + 8 * g) : h8{};
            if constexpr (W::REM) {
                if ((rb & 1) == (g >> 1))
                    qr[rb >> 1] = ok ? *reinterpret_cast<const h8*>(qrow + 32 * NC32 + 8 * (g & 1)) : h8{};
            } else if ((rb & 1) == 0) {
                qr[rb >> 1] = h8{};
            }
        }
    };
    // The block table into LDS (validated; bad entries noted), after every
    // wave has finished with the previous tile's.
    auto stage_table = [&]() {
        const int32_t* table = p.block_tables + (int64_t)chunk * p.max_blocks;
        __syncthreads();
        int bad = 0;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int e = tid + 256 * i;
            if (e < npages) {
                const bool ok = tb[i] >= 0 && (int64_t)tb[i] < p.num_blocks;
                table_s[e] = ok ? tb[i] : -1;
                bad |= !ok;
            }
        }
        for (int e = tid + 512; e < npages; e += 256) {
            const int bid = table[e];
            const bool ok = bid >= 0 && (int64_t)bid < p.num_blocks;
            table_s[e] = ok ? bid : -1;
            bad |= !ok;
        }
        any_bad = __syncthreads_or(bad) != 0;
    };
    // Q fragments into their AGPRs: fragment (rb, cc) is J = rb * NC32 + cc,
    // remainder pair j is J = RB * NC32 + j (prefill_wide_regs.h); the
    // outputs back to zero.
    auto set_q = [&]() {
        kw_reserve();
        static_for<RB * NC32>([&](auto J) { kw_set_q<J>(qa[J / NC32][J % NC32]); });
        if constexpr (W::REM) static_for<RB / 2>([&](auto j) { kw_set_q<RB * NC32 + j>(qr[j]); });
        static_for<4 * RB * NT>([&](auto N) { kw_zero<N>(); });
    };

    // The ring's DMA: as in prefill_tile (one page lookup per lane; wave w
    // issues instructions w, w + 4, w + 8 of a stage), in three parts so
    // that a step can spread them over its MFMA slots: the block-table
    // lookup, the source address, the DMA instructions.
    constexpr int PERW = W::PERW;
    constexpr int kDmaGap = W::DMA_GAP;
    const int dkey = (lane & 31) ^ ((lane >> 5) * kSwz);
    const int row_bytes = p.num_kv_heads * D * 2;
    const uint64_t page_bytes = (uint64_t)p.block_stride * 2;
    // (lane_off and the table's last entry depend on the tile: formed where used)
    const int bs_shift = __builtin_ctz((unsigned)p.block_size);  // block_size is a power of two here
    // (every expression below is evaluated unconditionally and selected at
    // the end, so the compiler forms no branch inside a step)
    auto dma_lookup = [&](int kb) {  // raw block-table entry of the lane's key
        const int pos = kb * kKBlk + dkey;
        return table_s[min(pos >> bs_shift, max(npages - 1, 0))];
    };
    auto dma_offset = [&](int kb, int bid) -> int64_t {  // byte offset in the pages, or -1
        const int pos = kb * kKBlk + dkey;
        const bool ok = pos < kv_end && pos < tab_end && bid >= 0;
#ifdef VCPP_GATHER_DUMP
        if (ok && wave == 0 && kvh == 0 && hg == 0) gather_record(p, chunk, pos, bid, pos & (p.block_size - 1));
#endif
        const uint64_t off = (uint64_t)(uint32_t)bid * page_bytes +
                             (uint32_t)((pos & (p.block_size - 1)) * row_bytes + kvh * D * 2 + (lane >> 5) * 16);
        return ok ? (int64_t)off : (int64_t)-1;
    };
    const int wave_s = __builtin_amdgcn_readfirstlane(wave);  // (uniform: keeps the issue branch-free)
    auto dma_issue = [&](int kb, int i, int64_t off) {  // this wave's instruction i of block kb
        const int j = wave_s + 4 * i;
        const int which = j >= DD::REGION / 64;
        const int cp = j - which * (DD::REGION / 64);
        const char* base = static_cast<const char*>(which ? p.v : p.k) + cp * 32;
        // Past the stage's last instruction: the dummy area and the zero
        // chunk (selected by masks, not branches).
        const uint32_t real = -(uint32_t)(j < DD::NINST);
        const uint32_t dst = lds_addr + ((((kb % kStages) * DD::STAGE + j * 1024) & real) | (kDummy & ~real));
        const void* src = off >= 0 && real ? (const void*)(base + off) : (const void*)kZeroChunk;
        dma16(src, dst);
    };
    auto issue = [&](int kb) {
        const int64_t off = dma_offset(kb, dma_lookup(kb));
#pragma unroll
        for (int i = 0; i < PERW; ++i) dma_issue(kb, i, off);
    };

    // Fragment offsets (as in prefill_tile).
    const int kbase = (32 * g + (c ^ ((g & 1) * kSwz))) * 16;
    // Remainder K fragments: lane group g reads dims 32 NC32 + 8 (g & 1) of
    // its key in the k half it serves (h = 0: g < 2, h = 1: g >= 2), the
    // stage's zero slot in the other.
    const int rch = 4 * NC32 + (g & 1), rpar = rch & 1;
    const int krem = (rch * 32 + (c ^ (rpar * kSwz))) * 16;
    auto krem_off = [&](int h, int kt) { return (g >> 1) == h ? krem + 256 * kt : DD::ZERO; };
    const int vpar = (c >> 1) & 1;
    const int vbase = DD::REGION * 16 + (((c & 3) >> 1) * 32 + ((4 * g + (c >> 2)) ^ (vpar * kSwz))) * 16 + 8 * (c & 1);

    f4 sacc[RB][2];
    h8 pa[RB];
    h8 ka[2][NK];  // [16-key half][fragment]
    h8 vb[NT];     // [output block]
    float lsum[RB], m_run[RB], bs[RB];

    // K fragment i (16-key half i / NK, fragment i % NK) of block kb.
    auto load_k = [&](int kb, int i) {
        lds_char* sb = lds + (kb % kStages) * DD::STAGE;
        const int kt = i / NK, cc = i - kt * NK;
        if (cc < NC32)
            ka[kt][cc] = *reinterpret_cast<__attribute__((address_space(3))) h8*>(sb + kbase + (128 * cc + 16 * kt) * 16);
        else
            ka[kt][cc] = *reinterpret_cast<__attribute__((address_space(3))) h8*>(sb + krem_off(cc - NC32, kt));
    };
    // V fragment t of block kb (two transposing reads).
    auto load_v = [&](int kb, int t) {
        lds_char* sb = lds + (kb % kStages) * DD::STAGE;
        const h4 lo = read_tr(sb + vbase + 64 * t * 16);
        const h4 hi = read_tr(sb + vbase + (64 * t + 16) * 16);
        vb[t] = h8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    };

    // S MFMA i of half H: fragment j = i / 8 of the 8 independent (row
    // block, key half) chains, so that the MFMAs of one chain are 8 apart.
    auto s_mfma = [&](auto H_, auto i_) {
        constexpr int H = decltype(H_)::value, i = decltype(i_)::value;
        constexpr int j = i >> 3, u = i & 7;
        constexpr int rb = 4 * H + (u >> 1), kt = u & 1;
        if constexpr (j == 0) kw_s0<rb * NC32>(sacc[rb][kt], ka[kt][0]);
        else if constexpr (j < NC32) kw_s<rb * NC32 + j>(sacc[rb][kt], ka[kt][j]);
        else kw_s<RB * NC32 + (rb >> 1)>(sacc[rb][kt], ka[kt][NC32 + (rb & 1)]);  // D = 80's remainder
    };
    auto pv_mfma = [&](auto H_, auto i_) {
        constexpr int H = decltype(H_)::value, i = decltype(i_)::value;
        constexpr int rb = 4 * H + i / NT, t = i % NT;
        kw_pv<rb * NT + t>(pa[rb], vb[t]);
    };

    // The softmax of half H as a software-pipelined stream of "ticks" over
    // its 32 scores per lane (score s = row block 4 H + s / 8, key slot
    // s % 8): tick t forms x_t = fma(s_t, scale, -m) (MASKED: -inf first for
    // keys past the row's last visible position or on a missing page), the
    // exp2 of x_(t-2), the fp16 pack of pair (t - 5) / 2 and the row-sum dot2
    // of pair (t - 7) / 2, so that no instruction waits for the one just
    // before it (one wave per SIMD: nothing else would fill the gap).
    constexpr int NTICK = 32 + 6;
    float xs[32], es[32];
    h2 pk[16];
    auto tick = [&](int H, int t, int kb, bool masked, const bool (&tile_ok)[2]) {
        if (t < 32) {
            const int rb = 4 * H + t / 8, k = t % 8, kt = k >> 2, r = k & 3;
            float x = sacc[rb][kt][r];
            if (masked) {
                const int key = kb * kKBlk + 16 * kt + 4 * g + r;
                const int lim = min(prefix + t0 + 16 * rb + c, kv_end - 1);
                x = (tile_ok[kt] && key <= lim) ? x : -__builtin_inff();
                sacc[rb][kt][r] = x;  // the rescale path re-reads masked scores
            }
            xs[t] = fmaf(x, p.scale_log2, -m_run[rb]);
        }
        if (t >= 2 && t - 2 < 32) es[t - 2] = fast_exp2(xs[t - 2]);
        if (t >= 5 && ((t - 5) & 1) == 0 && (t - 5) / 2 < 16) {
            const int q = (t - 5) / 2;
            pk[q] = h2{(_Float16)es[2 * q], (_Float16)es[2 * q + 1]};
            const int rb = 4 * H + q / 4, k = 2 * (q % 4);
            pa[rb][k] = pk[q][0];
            pa[rb][k + 1] = pk[q][1];
        }
        if (t >= 7 && ((t - 7) & 1) == 0 && (t - 7) / 2 < 16) {
            const int q = (t - 7) / 2, rb = 4 * H + q / 4;
            bs[rb] = __builtin_amdgcn_fdot2(pk[q], h2{1, 1}, (q & 3) == 0 ? 0.f : bs[rb], false);
        }
    };

    // Rare path: a row of half H whose block sum of P passed 2^kLazy (or is
    // inf / NaN) -- form the row max, move the running max if it grew by
    // more than 2^kLazy, rescale the row's sum and outputs, recompute P.
    auto rescale = [&](int H) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int rb = 4 * H + i;
            float x[2][4];
#pragma unroll
            for (int kt = 0; kt < 2; ++kt)
#pragma unroll
                for (int r = 0; r < 4; ++r) x[kt][r] = sacc[rb][kt][r] * p.scale_log2;
            const float ml = max_over_groups(vmax(vmax3(x[0][0], x[0][1], x[0][2]),
                                                  vmax3(x[0][3], x[1][0], x[1][1]),
                                                  vmax3(x[1][2], x[1][3], x[1][3])));
            const bool grow = ml > m_run[rb] + kLazy;
            const float m_new = grow ? ml : m_run[rb];
            const float alpha = fast_exp2(m_run[rb] - m_new);
            m_run[rb] = m_new;
            lsum[rb] *= alpha;
            const float a0 = shfl(alpha, 4 * g), a1 = shfl(alpha, 4 * g + 1);
            const float a2 = shfl(alpha, 4 * g + 2), a3 = shfl(alpha, 4 * g + 3);
            static_for<NT>([&](auto t) {
                switch (rb) {  // (rb is a constant once unrolled)
#define VCPP_W_SCALE(R) case R: kw_scale<R * NT + t>(a0, a1, a2, a3); break;
                    VCPP_W_SCALE(0) VCPP_W_SCALE(1) VCPP_W_SCALE(2) VCPP_W_SCALE(3)
                    VCPP_W_SCALE(4) VCPP_W_SCALE(5) VCPP_W_SCALE(6) VCPP_W_SCALE(7)
#undef VCPP_W_SCALE
                }
            });
            if (__any(grow)) {
                float b = 0.f;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int k0 = 2 * q, k1 = 2 * q + 1;
                    const float e0 = fast_exp2(fmaf(sacc[rb][k0 >> 2][k0 & 3], p.scale_log2, -m_run[rb]));
                    const float e1 = fast_exp2(fmaf(sacc[rb][k1 >> 2][k1 & 3], p.scale_log2, -m_run[rb]));
                    const h2 pp = {(_Float16)e0, (_Float16)e1};
                    pa[rb][k0] = pp[0];
                    pa[rb][k1] = pp[1];
                    b = __builtin_amdgcn_fdot2(pp, h2{1, 1}, b, false);
                }
                bs[rb] = b;
            }
        }
    };
    bool cross = false;  // set by the last slot of each phase
    auto check = [&](int H) {
        if (__builtin_expect(__any(cross), 0)) rescale(H);
#pragma unroll
        for (int i = 0; i < 4; ++i) lsum[4 * H + i] += bs[4 * H + i];
    };

    // Phase PH of block kb: NM MFMAs, each followed by its share of the
    // softmax micro-ops and, phase 1, one K fragment read of block kb + 1
    // in each slot after the S group; phase 2, one V fragment read of
    // block kb in each of the first slots.
    auto phase = [&](int kb, auto ph_tag, auto mask_tag) {
        constexpr int PH = decltype(ph_tag)::value;  // 1 or 2
        constexpr bool MASKED = decltype(mask_tag)::value;
        constexpr int SH = PH == 1 ? 1 : 0;          // half whose S is formed (block kb, or kb + 1)
        constexpr int PH_PV = PH == 1 ? 1 : 0;       // half whose P V is formed (block kb - 1, or kb)
        constexpr int SMH = PH == 1 ? 0 : 1;         // half whose softmax runs
        constexpr int NM = W::NS + W::NPV;
        // Masked blocks: whether each 16-key half lies on a page in the pool.
        bool tile_ok[2] = {true, true};
        if constexpr (MASKED) {
#pragma unroll
            for (int kt = 0; kt < 2; ++kt) {
                const int k16 = kb * kKBlk + 16 * kt;
                tile_ok[kt] = k16 < tab_end && table_s[(int)(((uint64_t)(uint32_t)k16 * p.bs_magic) >> 40)] >= 0;
            }
        }
        int dma_bid = -1;
        int64_t dma_off = -1;
        fence();
        static_for<NM>([&](auto i_) {
            constexpr int i = decltype(i_)::value;
            if constexpr (i < W::NS) s_mfma(std::integral_constant<int, SH>{}, i_);
            else pv_mfma(std::integral_constant<int, PH_PV>{}, std::integral_constant<int, i - W::NS>{});
            if constexpr (PH == 1) {
                // The ring's next block: lookup, address, DMA over slots 0,
                // 8 and 12, 12 + kDmaGap, ... (stage (kb - 1) % kStages is
                // free: every wave passed the step's barrier after its last
                // read).  The DMA instructions are spread out because each
                // holds the wave at issue while the CU's address unit works
                // through the other waves' ones.
                if constexpr (i == 0) dma_bid = dma_lookup(kb + kStages - 1);
                if constexpr (i == 8) dma_off = dma_offset(kb + kStages - 1, dma_bid);
                if constexpr (i >= 12 && (i - 12) % kDmaGap == 0 && (i - 12) / kDmaGap < PERW)
                    dma_issue(kb + kStages - 1, (i - 12) / kDmaGap, dma_off);
                if constexpr (i >= W::NS && i < W::NS + 2 * NK) load_k(kb + 1, i - W::NS);
            } else {
                if constexpr (i < NT) load_v(kb, i);
            }
#pragma unroll
            for (int t = i * NTICK / NM; t < (i + 1) * NTICK / NM; ++t) tick(SMH, t, kb, MASKED, tile_ok);
            if constexpr (i == NM - 1) {
                // The lazy-rescale test of the half, ahead of the branch.
                bool x = false;
#pragma unroll
                for (int k = 0; k < 4; ++k) x |= !(bs[4 * SMH + k] <= kLazyP);  // inf and NaN too
                cross = x;
            }
            fence();
        });
    };

    auto step = [&](int kb, auto mask_tag) {
        // Blocks kb and kb + 1 landed for every wave; stage kb - 1 (last
        // read by phase 2 of block kb - 1) is free for block kb + kStages - 1,
        // whose DMA phase 1 issues.
        VCPP_T(0);
        wait_vmcnt<(kStages - 3) * PERW>();
        VCPP_T(1);
        __syncthreads();
        VCPP_T(2);
        VCPP_T(3);
        phase(kb, std::integral_constant<int, 1>{}, mask_tag);
        VCPP_T(4);
        check(0);
        VCPP_T(5);
        phase(kb, std::integral_constant<int, 2>{}, mask_tag);
        VCPP_T(6);
        check(1);
        VCPP_T(7);
    };

    // The finished tile's outputs (its O still in the AGPRs): normalised rows
    // into out, or for a split the unnormalised rows and each row's (max,
    // sum) into the workspace.  fin_*: the tile's identity and row state.
    int f_q0 = 0, f_n = 0, f_t0 = 0, f_head = 0, f_part = 0;
    bool f_ok = false;
    float f_sum[RB], f_m[RB];
    auto finish = [&]() {  // row sums of the tile just computed
        f_q0 = q0; f_n = n; f_t0 = t0; f_head = head; f_part = part; f_ok = head_ok;
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            f_sum[rb] = sum_over_groups(lsum[rb]);  // row c
            f_m[rb] = m_run[rb];
        }
    };
    auto store = [&]() {
        if (!f_ok) return;
        const bool split = p.splits > 1;
        const int64_t pbase = (int64_t)f_part * p.rows_cap;
        const bool odd_lane = (c & 1) != 0;
        float inv[RB][2];
        if (!split) {
#pragma unroll
            for (int rb = 0; rb < RB; ++rb)
#pragma unroll
                for (int k2 = 0; k2 < 2; ++k2)
                    inv[rb][k2] = 1.0f / (shfl(f_sum[rb], 4 * g + 2 * k2 + (odd_lane ? 1 : 0)) + 1e-9f);
        }
        static_for<RB>([&](auto rb_) {
            constexpr int rb = decltype(rb_)::value;
            f4 ob[NT];
            static_for<NT>([&](auto t) { ob[t] = kw_get<rb * NT + t>(); });
            if (split) {
                const int tc = f_t0 + 16 * rb + c;
                if (g == 0 && tc < f_n && f_q0 + tc < p.rows_cap)
                    p.ws_ml[(pbase + f_q0 + tc) * p.num_heads + f_head] = make_float2(f_m[rb], f_sum[rb]);
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int tok = f_t0 + 16 * rb + 4 * g + r;
                    if (tok < f_n && f_q0 + tok < p.rows_cap) {
                        float* orow = p.ws_o + ((pbase + f_q0 + tok) * p.num_heads + f_head) * D;
#pragma unroll
                        for (int t = 0; t < NT; ++t) orow[16 * t + c] = ob[t][r];
                    }
                }
                return;
            }
            // Lane (g, c) holds rows 4 g + r, column 16 t + c: column pairs
            // as in prefill_tile.
#pragma unroll
            for (int k2 = 0; k2 < 2; ++k2) {
                const int r = 2 * k2 + (odd_lane ? 1 : 0);
                const int tok = f_t0 + 16 * rb + 4 * g + r;
                float* orow = p.out + ((int64_t)(f_q0 + min(tok, f_n - 1)) * p.num_heads + f_head) * D;
#pragma unroll
                for (int t = 0; t < NT; ++t) {
                    const float x0 = ob[t][2 * k2], x1 = ob[t][2 * k2 + 1];
                    const float y = dpp_swap1(odd_lane ? x0 : x1);
                    const float2 v = odd_lane ? make_float2(y * inv[rb][k2], x1 * inv[rb][k2])
                                              : make_float2(x0 * inv[rb][k2], y * inv[rb][k2]);
                    if (tok < f_n) *reinterpret_cast<float2*>(orow + 16 * t + (c & ~1)) = v;
                }
            }
        });
    };

    {
        if (!plan(blockIdx.x)) return;  // whole workgroup, before any barrier
        VCPP_T(11);
        load_tile();
        VCPP_T(12);
        stage_table();
        set_q();
        VCPP_T(8);
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            lsum[rb] = 0.f;
            m_run[rb] = kMaxSeed;
            bs[rb] = 0.f;
            pa[rb] = h8{};
        }
#pragma unroll
        for (int t = 0; t < NT; ++t) vb[t] = h8{};

        // Prologue: the ring's first blocks, K of block kb_lo, S_A(kb_lo).
#pragma unroll
        for (int s = 0; s < kStages - 1; ++s) issue(kb_lo + s);
        wait_vmcnt<(kStages - 2) * PERW>();
        __syncthreads();
#pragma unroll
        for (int i = 0; i < 2 * NK; ++i) load_k(kb_lo, i);
        fence();
        // The Q fragments were just moved into AGPRs by vector instructions
        // the hazard recognizer does not pair with the inline-assembly MFMAs
        // below.
        asm volatile("s_nop 7\n\ts_nop 7" ::: "memory");
        static_for<W::NS>([&](auto i) { s_mfma(std::integral_constant<int, 0>{}, i); });
        fence();
        VCPP_T(9);

        // Blocks visible to every row run unmasked, the rest masked.
        const int free_end = any_bad ? kb_lo : max(min(nfree, kb_hi), kb_lo);
        int kb = kb_lo;
        for (; kb < free_end; ++kb) step(kb, std::false_type{});
        for (; kb < kb_hi; ++kb) step(kb, std::true_type{});
        // Epilogue: P_B V of the last block.
        fence();
        if (kb_hi > kb_lo) static_for<W::NPV>([&](auto i) { pv_mfma(std::integral_constant<int, 1>{}, i); });
        // The outputs are read later by instructions the hazard recognizer
        // does not pair with the inline-assembly MFMAs that wrote them.
        asm volatile("s_nop 15\n\ts_nop 15\n\ts_nop 15" ::: "memory");
        fence();
        wait_vmcnt<0>();
        finish();
        VCPP_T(10);
    }
    store();
#ifdef VCPP_PF_TIMING
    if (lane == 0)
        for (int k = 0; k < 16; ++k) atomicAdd(&g_pf_timing[k], (unsigned long long)tm[k]);
#endif
}

}  // namespace

}  // namespace vcpp
