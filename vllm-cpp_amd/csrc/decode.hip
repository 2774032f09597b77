// decode.hip -- batched paged decode attention for gfx950.
//
// Reference behaviour: src/paged_attention.cpp:11-90 (one query token per
// sequence, GQA map kv_h = h / (H / Hkv), scale 1/sqrt(D), max seeded at
// -1e9, sum + 1e-9, positions past the table or on an invalid block skipped).
// The reference's GPU slot is cuda/attention.cu:11-52; its kernel
// (cuda/attention_kernels.cuh:9-123) is not followed.
//
// Work decomposition: one workgroup per (partition, sequence, kv-head slice);
// one wave per (kv head, chunk of <= 8 query heads of its GQA group), so every
// K/V page is read from HBM once for the whole group.  A 16-token tile is one
// MFMA step:
//   S^T[16 tok][16] = K_tile[16 tok][D] x Qs^T     (16x16x32 f16 steps)
//   O[16][D]       += P[16][16 tok] x V_tile        (16x16x16 f16, D/16 tiles)
// The 16 MFMA rows hold the fp16 "hi" part of the 8 query heads (rows 0-7)
// and the fp16 residual q - hi (rows 8-15); likewise P = p_hi + p_lo.  Summing
// the two halves keeps about 22 significant bits of q and p while K/V stay
// exact fp16, with fp32 accumulation -- the padding rows an 8-head group would
// waste on a 16-row MFMA carry the low halves instead.
// V is needed with tokens along the MFMA k dimension, so each wave stages its
// V tile in LDS (row-major, padded rows) and reads it back transposed.
// Long contexts are split into partitions; each writes (m, l, o) partials and
// the log-sum-exp merge kernel combines them.
#include "decode.h"
#include "device_common.h"

namespace vcpp {

namespace {

constexpr int kTile = 16;          // tokens per MFMA tile
constexpr int kTilesPerIter = 2;   // tiles per softmax update / prefetch step

template <int D>
struct Dims {
    static constexpr int NC32 = D / 32;         // 16x16x32 steps over head_dim
    // A trailing 16-dim remainder runs as one more 16x16x32 step whose lane
    // groups 2-3 carry zeros (padding in registers, not in HBM).  One opcode
    // per accumulation chain: a 16x16x16 step chained straight after a
    // 16x16x32 one on the same accumulator was measured to drop the previous
    // step's contribution on gfx950 with this toolchain.
    static constexpr int REM = (D % 32) / 16;
    static constexpr int NT = D / 16;           // output 16-column tiles
    static constexpr int VROW = D + 8;          // LDS row pitch in halves
    static_assert(D % 16 == 0 && D <= 256, "head_dim must be a multiple of 16");
};

// Registers of one 16-token tile for one lane.
template <int KV, int D>
struct Tile;

template <int D>
struct Tile<VCPP_KV_F16, D> {
    h8 k[Dims<D>::NC32 > 0 ? Dims<D>::NC32 : 1];
    h8 kr;  // dims 32*NC32 + 8g.. for lane groups 0-1, zero for 2-3
    h8 v[Dims<D>::NC32 > 0 ? Dims<D>::NC32 : 1];
    h8 vr;
};

template <int D>
struct Tile<VCPP_KV_I8, D> {
    i2 k[Dims<D>::NC32 > 0 ? Dims<D>::NC32 : 1];
    i2 kr;
    i2 v[Dims<D>::NC32 > 0 ? Dims<D>::NC32 : 1];
    i2 vr;
    i2 ks;  // fp16 K scales of tokens 4g..4g+3
    i2 vs;  // fp16 V scales of tokens 4g..4g+3
};

template <int KV>
struct Elem;
template <>
struct Elem<VCPP_KV_F16> { typedef _Float16 T; };
template <>
struct Elem<VCPP_KV_I8> { typedef int8_t T; };

// Loads the lane's share of one tile: token c of the tile, head_dim chunk g.
// An invalid block yields zeros (its tokens are masked anyway).
template <int KV, int D>
__device__ __forceinline__ void load_tile(Tile<KV, D>& t, const DecodeParams& p, int bid,
                                          int tok_in_block, int kvh, int g, int c) {
    typedef typename Elem<KV>::T E;
    constexpr int NC32 = Dims<D>::NC32;
    if (bid < 0) {
        t = Tile<KV, D>{};
        return;
    }
    const int64_t row = (int64_t)bid * p.block_stride +
                        ((int64_t)(tok_in_block + c) * p.num_kv_heads + kvh) * D;
    const E* kp = reinterpret_cast<const E*>(p.k) + row;
    const E* vp = reinterpret_cast<const E*>(p.v) + row;
    if constexpr (KV == VCPP_KV_F16) {
#pragma unroll
        for (int cc = 0; cc < NC32; ++cc) {
            t.k[cc] = *reinterpret_cast<const h8*>(kp + 32 * cc + 8 * g);
            t.v[cc] = *reinterpret_cast<const h8*>(vp + 32 * cc + 8 * g);
        }
        if constexpr (Dims<D>::REM) {
            t.kr = h8{};
            t.vr = h8{};
            if (g < 2) {
                t.kr = *reinterpret_cast<const h8*>(kp + 32 * NC32 + 8 * g);
                t.vr = *reinterpret_cast<const h8*>(vp + 32 * NC32 + 8 * g);
            }
        }
    } else {
#pragma unroll
        for (int cc = 0; cc < NC32; ++cc) {
            t.k[cc] = *reinterpret_cast<const i2*>(kp + 32 * cc + 8 * g);
            t.v[cc] = *reinterpret_cast<const i2*>(vp + 32 * cc + 8 * g);
        }
        if constexpr (Dims<D>::REM) {
            t.kr = i2{};
            t.vr = i2{};
            if (g < 2) {
                t.kr = *reinterpret_cast<const i2*>(kp + 32 * NC32 + 8 * g);
                t.vr = *reinterpret_cast<const i2*>(vp + 32 * NC32 + 8 * g);
            }
        }
        const int64_t srow = (int64_t)bid * p.scale_block_stride +
                             (int64_t)kvh * p.block_size + tok_in_block + 4 * g;
        t.ks = *reinterpret_cast<const i2*>(p.k_scale + srow);
        t.vs = *reinterpret_cast<const i2*>(p.v_scale + srow);
    }
}

// Decodes a tile's K chunk to fp16 MFMA operands.
template <int KV, int D>
__device__ __forceinline__ h8 k_chunk(const Tile<KV, D>& t, int cc) {
    if constexpr (KV == VCPP_KV_F16) return t.k[cc];
    else return i8x8_to_h8((uint32_t)t.k[cc].x, (uint32_t)t.k[cc].y);
}
template <int KV, int D>
__device__ __forceinline__ h8 k_rem(const Tile<KV, D>& t) {
    if constexpr (KV == VCPP_KV_F16) return t.kr;
    else return i8x8_to_h8((uint32_t)t.kr.x, (uint32_t)t.kr.y);
}

// Writes the lane's V row chunk (token c) into the wave's LDS tile, zeroing
// rows of masked tokens so 0 * garbage cannot produce NaN in P x V.
template <int KV, int D>
__device__ __forceinline__ void stage_v(_Float16* lds, const Tile<KV, D>& t, bool valid, int g,
                                        int c) {
    constexpr int NC32 = Dims<D>::NC32, VROW = Dims<D>::VROW;
    _Float16* row = lds + c * VROW;
#pragma unroll
    for (int cc = 0; cc < NC32; ++cc) {
        h8 x;
        if constexpr (KV == VCPP_KV_F16) x = t.v[cc];
        else x = i8x8_to_h8((uint32_t)t.v[cc].x, (uint32_t)t.v[cc].y);
        if (!valid) x = h8{};
        *reinterpret_cast<h8*>(row + 32 * cc + 8 * g) = x;
    }
    if constexpr (Dims<D>::REM) {
        h8 x;
        if constexpr (KV == VCPP_KV_F16) x = t.vr;
        else x = i8x8_to_h8((uint32_t)t.vr.x, (uint32_t)t.vr.y);
        if (!valid) x = h8{};
        if (g < 2) *reinterpret_cast<h8*>(row + 32 * NC32 + 8 * g) = x;
    }
}

__device__ __forceinline__ float h_to_f(uint32_t bits16) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
}

template <int KV, int D>
__global__ __launch_bounds__(512) void decode_mfma_kernel(DecodeParams p) {
    constexpr int NC32 = Dims<D>::NC32, NT = Dims<D>::NT, VROW = Dims<D>::VROW;
    extern __shared__ _Float16 lds_all[];

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int g = lane >> 4, c = lane & 15;
    const int pair = blockIdx.z * (blockDim.x >> 6) + wave;
    if (pair >= p.pairs) return;
    const int seq = blockIdx.y, part = blockIdx.x;
    const int ctx = min(p.context_lens[seq], p.max_parts * p.partition);
    const int P = p.partition;
    const int np = ctx <= 0 ? 1 : min((ctx + P - 1) / P, p.max_parts);
    if (part >= np) return;

    const int kvh = pair / p.qchunks, qc = pair - kvh * p.qchunks;
    const int head_base = kvh * p.group + qc * 8;
    const int gc = min(8, p.group - qc * 8);
    int tlen = p.max_blocks;
    if (p.table_lens) tlen = min(tlen, p.table_lens[seq]);
    const int start = part * P;
    const int stop = min(start + P, ctx);                          // tokens visited
    const int end = min(stop, (int)min((int64_t)tlen * p.block_size, (int64_t)INT32_MAX));
    const int ntiles = stop > start ? (stop - start + kTile - 1) / kTile : 0;

    // Query fragment (B operand): row c = hi (c < 8) or lo (c >= 8) of head c & 7.
    h8 qa[NC32 > 0 ? NC32 : 1];
    h8 qr = {};
    {
        const bool qv = (c & 7) < gc;
        const float* qrow = p.q + ((int64_t)seq * p.num_heads + head_base + (c & 7)) * D;
#pragma unroll
        for (int cc = 0; cc < NC32; ++cc) {
            f4 x0 = {}, x1 = {};
            if (qv) {
                x0 = *reinterpret_cast<const f4*>(qrow + 32 * cc + 8 * g);
                x1 = *reinterpret_cast<const f4*>(qrow + 32 * cc + 8 * g + 4);
            }
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                float x = i < 4 ? x0[i] : x1[i - 4];
                _Float16 hi = (_Float16)x;
                qa[cc][i] = c < 8 ? hi : (_Float16)(x - (float)hi);
            }
        }
        if constexpr (Dims<D>::REM) {
            f4 x0 = {}, x1 = {};
            if (qv && g < 2) {
                x0 = *reinterpret_cast<const f4*>(qrow + 32 * NC32 + 8 * g);
                x1 = *reinterpret_cast<const f4*>(qrow + 32 * NC32 + 8 * g + 4);
            }
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                float x = i < 4 ? x0[i] : x1[i - 4];
                _Float16 hi = (_Float16)x;
                qr[i] = c < 8 ? hi : (_Float16)(x - (float)hi);
            }
        }
    }

    // Physical block of each tile in the partition (lane j <-> tile j), -1 if
    // the logical block is past the table or the id is out of range.
    int my_bid = -1, my_off = 0;
    if (lane < ntiles) {
        const int pos = start + lane * kTile;
        const int lb = pos / p.block_size;
        my_off = pos - lb * p.block_size;
        if (lb < tlen) {
            const int id = p.block_tables[(int64_t)seq * p.max_blocks + lb];
            if (id >= 0 && (int64_t)id < p.num_blocks) my_bid = id;
        }
    }

    _Float16* lds = lds_all + wave * (kTilesPerIter * kTile * VROW);

    f4 o[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) o[t] = f4{0.f, 0.f, 0.f, 0.f};
    float m_run = kMaxSeed, l_run = 0.f;

    Tile<KV, D> cur[kTilesPerIter], nxt[kTilesPerIter];
    const int niters = (ntiles + kTilesPerIter - 1) / kTilesPerIter;
#pragma unroll
    for (int j = 0; j < kTilesPerIter; ++j) {
        const int bid = j < ntiles ? __builtin_amdgcn_readlane(my_bid, j) : -1;
        const int off = __builtin_amdgcn_readlane(my_off, j & 63);
        load_tile<KV, D>(cur[j], p, bid, off, kvh, g, c);
    }

    for (int it = 0; it < niters; ++it) {
        // Prefetch the next step's tiles while this one computes.
        if (it + 1 < niters) {
#pragma unroll
            for (int j = 0; j < kTilesPerIter; ++j) {
                const int tt = (it + 1) * kTilesPerIter + j;
                const int bid = tt < ntiles ? __builtin_amdgcn_readlane(my_bid, tt) : -1;
                const int off = __builtin_amdgcn_readlane(my_off, tt & 63);
                load_tile<KV, D>(nxt[j], p, bid, off, kvh, g, c);
            }
        }

        float s[kTilesPerIter][4];
        float mx = kMaxSeed;
#pragma unroll
        for (int j = 0; j < kTilesPerIter; ++j) {
            const int tt = it * kTilesPerIter + j;
            const int bid = tt < ntiles ? __builtin_amdgcn_readlane(my_bid, tt & 63) : -1;
            const int pos0 = start + tt * kTile;
            f4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int cc = 0; cc < NC32; ++cc) acc = mfma32(k_chunk<KV, D>(cur[j], cc), qa[cc], acc);
            if constexpr (Dims<D>::REM) acc = mfma32(k_rem<KV, D>(cur[j]), qr, acc);
            stage_v<KV, D>(lds + j * kTile * VROW, cur[j], bid >= 0 && pos0 + c < end, g, c);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                float x = acc[r] + dpp_ror8(acc[r]);
                float f = p.scale_log2;
                if constexpr (KV == VCPP_KV_I8) {
                    const uint32_t w = (uint32_t)(r < 2 ? cur[j].ks.x : cur[j].ks.y);
                    f *= h_to_f((r & 1) ? (w >> 16) : (w & 0xFFFFu));
                }
                x *= f;
                const bool ok = bid >= 0 && pos0 + 4 * g + r < end;
                s[j][r] = ok ? x : -__builtin_inff();
                mx = fmaxf(mx, s[j][r]);
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
                const float a = shfl(alpha, (4 * g + r) & 7);
#pragma unroll
                for (int t = 0; t < NT; ++t) o[t][r] *= a;
            }
        }
        float lsum = 0.f;
#pragma unroll
        for (int j = 0; j < kTilesPerIter; ++j) {
            h4 pa;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                float pr = fast_exp2(s[j][r] - m_new);
                lsum += pr;
                if constexpr (KV == VCPP_KV_I8) {
                    const uint32_t w = (uint32_t)(r < 2 ? cur[j].vs.x : cur[j].vs.y);
                    float sv = h_to_f((r & 1) ? (w >> 16) : (w & 0xFFFFu));
                    const int tt = it * kTilesPerIter + j;
                    const bool ok = start + tt * kTile + 4 * g + r < end;
                    pr *= ok ? sv : 0.f;
                }
                const _Float16 hi = (_Float16)pr;
                pa[r] = c < 8 ? hi : (_Float16)(pr - (float)hi);
            }
            const _Float16* vt = lds + j * kTile * VROW;
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                h4 vb;
#pragma unroll
                for (int r = 0; r < 4; ++r) vb[r] = vt[(4 * g + r) * VROW + 16 * t + c];
                o[t] = mfma16(pa, vb, o[t]);
            }
        }
        l_run = l_run * alpha + lsum;

        if (it + 1 < niters) {
#pragma unroll
            for (int j = 0; j < kTilesPerIter; ++j) cur[j] = nxt[j];
        }
    }

    // Per-head totals: l over the four lane groups; O rows h (hi) + h + 8 (lo).
    l_run += shfl_xor(l_run, 16);
    l_run += shfl_xor(l_run, 32);
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) o[t][r] += shfl_xor(o[t][r], 32);

    float lh[4], mh[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        lh[r] = shfl(l_run, (4 * g + r) & 7);
        mh[r] = shfl(m_run, (4 * g + r) & 7);
    }
    if (g >= 2) return;
    if (np == 1) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int h = 4 * g + r;
            if (h >= gc) continue;
            const float inv = 1.0f / (lh[r] + 1e-9f);
            float* orow = p.out + ((int64_t)seq * p.num_heads + head_base + h) * D;
#pragma unroll
            for (int t = 0; t < NT; ++t) orow[16 * t + c] = o[t][r] * inv;
        }
    } else {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int h = 4 * g + r;
            if (h >= gc) continue;
            const int64_t idx = ((int64_t)seq * p.max_parts + part) * p.num_heads + head_base + h;
            float* orow = p.ws_o + idx * D;
#pragma unroll
            for (int t = 0; t < NT; ++t) orow[16 * t + c] = o[t][r];
            if (c == 0) p.ws_ml[idx] = make_float2(mh[r], lh[r]);
        }
    }
}

// fp32 pages: plain VALU kernel, one wave per (partition, sequence, head).
// Logits of the partition live in LDS; same partial format as the MFMA path.
__global__ __launch_bounds__(64) void decode_f32_kernel(DecodeParams p) {
    __shared__ float sl[1024];
    extern __shared__ float qs_dyn[];
    const int lane = threadIdx.x;
    const int seq = blockIdx.y, part = blockIdx.x, head = blockIdx.z;
    const int D = p.head_dim;
    const int ctx = min(p.context_lens[seq], p.max_parts * p.partition);
    const int P = p.partition;
    const int np = ctx <= 0 ? 1 : min((ctx + P - 1) / P, p.max_parts);
    if (part >= np) return;
    const int kvh = head / p.group;
    int tlen = p.max_blocks;
    if (p.table_lens) tlen = min(tlen, p.table_lens[seq]);
    const int start = part * P;
    const int stop = min(start + P, ctx);
    const int end = (int)min((int64_t)stop, (int64_t)tlen * p.block_size);
    const int n = stop > start ? stop - start : 0;

    const float* qrow = p.q + ((int64_t)seq * p.num_heads + head) * D;
    for (int d = lane; d < D; d += 64) qs_dyn[d] = qrow[d];
    __syncthreads();

    const float* kb = reinterpret_cast<const float*>(p.k);
    const float* vb = reinterpret_cast<const float*>(p.v);
    float mx = kMaxSeed;
    for (int i = lane; i < n; i += 64) {
        const int pos = start + i;
        const int lb = pos / p.block_size;
        int id = -1;
        if (pos < end) {
            id = p.block_tables[(int64_t)seq * p.max_blocks + lb];
            if (id < 0 || (int64_t)id >= p.num_blocks) id = -1;
        }
        float t = -__builtin_inff();
        if (id >= 0) {
            const float* kr = kb + (int64_t)id * p.block_stride +
                              ((int64_t)(pos - lb * p.block_size) * p.num_kv_heads + kvh) * D;
            float acc = 0.f;
            for (int d = 0; d < D; ++d) acc = fmaf(qs_dyn[d], kr[d], acc);
            t = acc * p.scale_log2;
        }
        sl[i] = t;
        mx = fmaxf(mx, t);
    }
    for (int m = 32; m >= 1; m >>= 1) mx = fmaxf(mx, shfl_xor(mx, m));
    float l = 0.f;
    for (int i = lane; i < n; i += 64) {
        const float e = fast_exp2(sl[i] - mx);
        sl[i] = e;
        l += e;
    }
    for (int m = 32; m >= 1; m >>= 1) l += shfl_xor(l, m);
    __syncthreads();
    for (int d = lane; d < D; d += 64) {
        float acc = 0.f;
        for (int i = 0; i < n; ++i) {
            const float w = sl[i];
            if (w == 0.f) continue;
            const int pos = start + i;
            const int lb = pos / p.block_size;
            const int id = p.block_tables[(int64_t)seq * p.max_blocks + lb];
            const float* vr = vb + (int64_t)id * p.block_stride +
                              ((int64_t)(pos - lb * p.block_size) * p.num_kv_heads + kvh) * D;
            acc = fmaf(w, vr[d], acc);
        }
        if (np == 1) {
            p.out[((int64_t)seq * p.num_heads + head) * D + d] = acc / (l + 1e-9f);
        } else {
            const int64_t idx = ((int64_t)seq * p.max_parts + part) * p.num_heads + head;
            p.ws_o[idx * D + d] = acc;
            if (d == lane && lane == 0) p.ws_ml[idx] = make_float2(mx, l);
        }
    }
}

// Log-sum-exp merge of the partitions of one (sequence, head) per wave.
__global__ __launch_bounds__(256) void lse_merge_kernel(DecodeParams p) {
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
    float M = kMaxSeed;
    for (int i = 0; i < np; ++i) M = fmaxf(M, p.ws_ml[base + (int64_t)i * p.num_heads].x);
    float L = 0.f;
    for (int i = 0; i < np; ++i) {
        const float2 ml = p.ws_ml[base + (int64_t)i * p.num_heads];
        L += fast_exp2(ml.x - M) * ml.y;
    }
    const float inv = 1.0f / (L + 1e-9f);
    for (int d = lane; d < D; d += 64) {
        float acc = 0.f;
        for (int i = 0; i < np; ++i) {
            const int64_t idx = base + (int64_t)i * p.num_heads;
            acc += fast_exp2(p.ws_ml[idx].x - M) * p.ws_o[idx * D + d];
        }
        p.out[((int64_t)seq * p.num_heads + head) * D + d] = acc * inv;
    }
}

template <int KV, int D>
hipError_t launch_mfma(const DecodeParams& p, hipStream_t stream) {
    const int wpw = p.pairs < 8 ? p.pairs : 8;
    dim3 grid(p.max_parts, p.num_seqs, (p.pairs + wpw - 1) / wpw);
    const size_t lds = (size_t)wpw * kTilesPerIter * kTile * Dims<D>::VROW * sizeof(_Float16);
    hipLaunchKernelGGL((decode_mfma_kernel<KV, D>), grid, dim3(wpw * 64), lds, stream, p);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_decode(const DecodeParams& p, hipStream_t stream) {
    if (p.num_seqs == 0) return hipSuccess;
    hipError_t err;
    if (p.kv_dtype == VCPP_KV_F32) {
        dim3 grid(p.max_parts, p.num_seqs, p.num_heads);
        hipLaunchKernelGGL(decode_f32_kernel, grid, dim3(64), p.head_dim * sizeof(float), stream,
                           p);
        err = hipGetLastError();
    } else {
#define VCPP_DISPATCH_D(KVT)                                              \
    switch (p.head_dim) {                                                 \
        case 64: err = launch_mfma<KVT, 64>(p, stream); break;            \
        case 80: err = launch_mfma<KVT, 80>(p, stream); break;            \
        case 128: err = launch_mfma<KVT, 128>(p, stream); break;          \
        default: return hipErrorInvalidValue;                             \
    }
        if (p.kv_dtype == VCPP_KV_F16) {
            VCPP_DISPATCH_D(VCPP_KV_F16)
        } else {
            VCPP_DISPATCH_D(VCPP_KV_I8)
        }
#undef VCPP_DISPATCH_D
    }
    if (err != hipSuccess) return err;
    if (p.max_parts > 1) {
        dim3 grid(p.num_seqs, (p.num_heads + 3) / 4);
        hipLaunchKernelGGL(lse_merge_kernel, grid, dim3(256), 0, stream, p);
        err = hipGetLastError();
    }
    return err;
}

bool decode_head_dim_supported(int kv_dtype, int head_dim) {
    if (kv_dtype == VCPP_KV_F32) return head_dim > 0 && head_dim <= 1024 && head_dim % 4 == 0;
    return head_dim == 64 || head_dim == 80 || head_dim == 128;
}

}  // namespace vcpp
