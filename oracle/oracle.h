/*
 * oracle.h -- CPU restatement of the reference paged-attention path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load liboracle.so, and only as the checker
 * (or the timed CPU baseline) -- never as part of the product path.
 *
 * Every function cites the reference file:line whose behaviour it restates
 * (paths relative to the reference repository root).  The code is written
 * independently from the reference's description of the algorithm.
 *
 * Pool layout understood by the oracle (the reference BlockPool per-layer slab,
 * src/kv_cache_manager.cpp:12-34,90-95): for each physical block b the K slab
 * of one layer is [block_size tokens][num_kv_heads][head_dim], contiguous; the
 * distance between consecutive blocks is `block_stride` elements.  V likewise.
 * int8 pages carry one fp16 scale per (token, kv head), laid out per block as
 * [num_kv_heads][block_size] with `scale_block_stride` elements between blocks.
 */
#ifndef VCPP_ORACLE_H
#define VCPP_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { ORC_F32 = 0, ORC_F16 = 1, ORC_I8 = 2, ORC_FP8 = 3 };

typedef struct {
    int32_t kind;              /* ORC_F32 / ORC_F16 / ORC_I8 / ORC_FP8 */
    const void* k;             /* element base of block 0 */
    const void* v;
    const uint16_t* k_scale;   /* ORC_I8 only */
    const uint16_t* v_scale;
    int64_t num_blocks;
    int64_t block_stride;      /* elements between blocks (K and V) */
    int64_t scale_block_stride;/* fp16 elements between blocks (scales) */
    int32_t block_size;
    int32_t num_kv_heads;
    int32_t head_dim;
} orc_pool;

/* fp16 codec of the reference pool (src/kv_cache_manager.cpp:115-184). */
uint16_t orc_f16_encode_trunc(float x);
float orc_f16_decode(uint16_t h);
void orc_f16_encode_trunc_n(const float* x, uint16_t* h, int64_t n);
void orc_f16_decode_n(const uint16_t* h, float* x, int64_t n);

/* FP8 E4M3 codec of the reference KV pool (src/quantization.cpp:25-82,
 * 176-188): bias 7, max finite 240, exponent 15 = inf (mantissa 6) or NaN; the
 * encoder picks the nearest finite code of the value's sign (first, i.e.
 * smaller, on a tie), inf -> 0x7E / 0xFE, NaN -> 0xFF, +0 and -0 -> 0x00. */
float orc_fp8_decode(uint8_t b);
uint8_t orc_fp8_encode(float v);
void orc_fp8_encode_n(const float* x, uint8_t* b, int64_t n);
void orc_fp8_decode_n(const uint8_t* b, float* x, int64_t n);

/* Symmetric int8 quantiser per (token, kv head) vector of `d` values:
 * scale = fp16_rne(max|x| / 127); q = clamp(rne(x / float(scale)), -127, 127);
 * a zero vector gets scale 0 and q = 0.  Build definition (the reference has no
 * INT8 KV; src/config.h:69-73). */
void orc_quant_i8(const float* x, int32_t d, int8_t* q, uint16_t* scale);
/* orc_quant_i8 over `rows` consecutive rows of d values. */
void orc_quant_i8_rows(const float* x, int64_t rows, int32_t d, int8_t* q, uint16_t* scales);
uint16_t orc_f16_encode_rne(float x);

/* Single-query paged attention, reference src/paged_attention.cpp:11-90.
 * q: [num_heads][head_dim] fp32; out: [num_heads][head_dim] fp32. */
void orc_paged_attention(const orc_pool* pool, const float* q,
                         const int32_t* table, int32_t table_len,
                         int32_t seq_len, int32_t num_heads, float* out);

/* Batched decode: seq b uses table row b (row stride `table_stride`), length
 * min(table_lens[b], table_stride) (table_lens may be NULL => table_stride),
 * context ctx[b]; q/out [B][H][D].  Threads over (seq, head) with `nthreads`. */
void orc_decode_batch(const orc_pool* pool, const float* q, const int32_t* tables,
                      int64_t table_stride, const int32_t* table_lens,
                      const int32_t* ctx, int32_t batch, int32_t num_heads,
                      float* out, int32_t nthreads);

/* Chunked causal prefill with the engine's per-position semantics
 * (src/paged_engine.cpp:348-384, src/model.cpp:1214-1220): row i of chunk c
 * attends positions 0 .. prefix[c]+i through table row c.  q/out are
 * [total_rows][H][D]; chunk c owns rows q_start[c] .. q_start[c+1]-1. */
void orc_prefill_batch(const orc_pool* pool, const float* q, const int32_t* tables,
                       int64_t table_stride, const int32_t* q_start,
                       const int32_t* prefix, int32_t num_chunks, int32_t num_heads,
                       float* out, int32_t nthreads);

/* Dense fp64 softmax attention (brute force) over `n` keys for one head:
 * k, v: [n][d] fp64; returns out[d]. */
/* Dense attention of the reference's flash_attention_cuda host loops
 * (cuda/attention.cu:58-124): for each (b, h) only query row 0 of q
 * [B][H][q_len][D] is used; k, v [B][H][kv_len][D]; logits * 1/sqrt(D),
 * attn_mask[s] < 0 -> -1e9; softmax with max from logits[0], sum + 1e-9;
 * w [B*H][kv_len] receives the probabilities, out [B][H][D]. */
void orc_flash_attention(const float* q, const float* k, const float* v, float* out, float* w,
                         int32_t batch, int32_t heads, int32_t head_dim, int32_t q_len,
                         int32_t kv_len, const float* mask);

void orc_dense_f64(const double* q, const double* k, const double* v, int32_t n,
                   int32_t d, double scale, double* out);

/* Split-K partial for positions [p0, p1) of one head, then the log-sum-exp
 * merge of `np` partials (m, l, o[d]).  Used to pin the split-K identity. */
void orc_partial(const orc_pool* pool, const float* q_h, int32_t kv_h,
                 const int32_t* table, int32_t table_len, int32_t p0, int32_t p1,
                 float* m, float* l, float* o);
void orc_lse_merge(const float* m, const float* l, const float* o, int32_t np,
                   int32_t d, float* out);

/* Deterministic N(mean, std) generator: splitmix64 -> two uniforms in (0,1]
 * -> Box-Muller (fp64), stored as fp32.  Stream index i is independent of n. */
void orc_fill_normal(uint64_t seed, float* out, int64_t n, double mean, double std);
/* Uniform integers in [lo, hi] from splitmix64 (modulo reduction). */
void orc_fill_uniform_int(uint64_t seed, int32_t* out, int64_t n, int32_t lo, int32_t hi);
/* Fisher-Yates permutation of 0..n-1 driven by splitmix64. */
void orc_permutation(uint64_t seed, int32_t* out, int32_t n);

/* Per-head RMS norm, src/paged_engine.cpp:14-20 per row of head_dim (in place). */
void orc_head_norm(float* x, const float* w, float eps, int64_t rows, int32_t head_dim);
/* RoPE at per-token positions, src/paged_engine.cpp:47-62; style 0 pairs
 * (2i, 2i+1), style 1 pairs (i, i + head_dim/2) (in place). */
void orc_rope(float* x, int32_t num_tokens, int32_t num_heads, int32_t head_dim,
              const int32_t* positions, const float* inv_freq, int32_t n_freq, int32_t style);
/* apply_rope_cuda semantics, cuda/attention_kernels.cuh:249-287 (in place). */
void orc_rope_table(float* q, float* k, const float* cs, const float* sn, int32_t total_dim,
                    int32_t head_dim, int32_t batch);

#ifdef __cplusplus
}
#endif
#endif
