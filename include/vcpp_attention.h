/*
 * vcpp_attention.h -- C ABI of the MI355X paged-attention library
 * (libvcpp_attn.so, built from vllm-cpp_amd/csrc for gfx950).
 *
 * Two layers:
 *   v1  the reference launcher signatures of cuda/attention.h:19-45, with
 *       C linkage, so code written against that header links unchanged;
 *   v2  descriptor entry points that carry what v1 leaves implicit (separate
 *       K/V bases, strides, KV dtype, device-side lengths, stream, workspace)
 *       and return a status code.  v1 is a thin wrapper over v2.
 *
 * Conventions shared by every entry point:
 *   - all tensor pointers are caller-owned device memory unless stated;
 *   - `half` data is IEEE binary16 passed as uint16_t (ABI-equal to half);
 *   - streams are hipStream_t passed as void* (NULL = the null stream);
 *   - calls are asynchronous on their stream; calls that share a stream are
 *     ordered, calls on different streams that share a workspace race;
 *   - v2 entry points return VCPP_OK (0) or a negative VCPP_E* code and record
 *     a message retrievable with vcpp_last_error() (thread-local).  Nothing
 *     ever calls exit().
 *
 * Attention semantics (reference src/paged_attention.cpp:11-90): for query
 * head h the KV head is h / (num_heads / num_kv_heads); logits are
 * q.k / sqrt(head_dim); out = sum_p exp(s_p - max) v_p / (sum_p exp(s_p - max)
 * + 1e-9).  Positions p < context_len whose logical block p / block_size is at
 * or past the table length, or whose physical block id is outside
 * [0, num_blocks), are skipped.  A sequence with no usable position gets zeros.
 */
#ifndef VCPP_ATTENTION_H
#define VCPP_ATTENTION_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ------------------------------------------------------ */
#define VCPP_OK 0
#define VCPP_E_INVALID (-1)     /* bad argument (shape, dtype, null pointer) */
#define VCPP_E_UNSUPPORTED (-2) /* valid but not implemented for this shape */
#define VCPP_E_WORKSPACE (-3)   /* workspace missing or too small */
#define VCPP_E_HIP (-4)         /* HIP runtime error (message has details) */

/* Message of the last failing call on this thread ("" if none). */
const char* vcpp_last_error(void);
/* Library version string. */
const char* vcpp_version(void);

/* ---- KV page description ----------------------------------------------- */
#define VCPP_KV_F32 0
#define VCPP_KV_F16 1
#define VCPP_KV_I8 2 /* symmetric int8, one fp16 scale per (token, kv head) */
#define VCPP_KV_FP8 3 /* FP8 E4M3 as the reference KV pool stores it (KVDtype::FP8_E4M3,
                         src/quantization.cpp:25-82): bias 7, max finite 240, no scales */

/*
 * One layer of a paged KV pool.  Block b's K page is
 *   k + b * block_stride   (elements of the KV dtype),
 * laid out [block_size tokens][num_kv_heads][head_dim] -- the per-(block,
 * layer) slab of the reference BlockPool (src/kv_cache_manager.cpp:12-34,
 * 90-95).  V likewise.  With the reference's "all layers in one block"
 * allocation, pass k = base + layer * block_size * kv_dim and
 * block_stride = num_layers * block_size * kv_dim.
 * VCPP_KV_I8 adds fp16 scale pages: block b's K scales are
 *   k_scale + b * scale_block_stride,  laid out [num_kv_heads][block_size].
 * VCPP_KV_F16 pages are read as IEEE binary16: a NaN code (which the
 * reference encoder writes for a NaN input as 0x7C01 and its decoder,
 * src/kv_cache_manager.cpp:136-137, reads back as +-inf) is a NaN here, so a
 * non-finite K or V input gives NaN outputs where the reference gives inf or
 * NaN.  Finite codes decode identically.
 * VCPP_KV_FP8 pages hold one byte per value and no scales.  Codes with
 * exponent 15 (the reference's +-inf and NaN, which its encoder produces only
 * from non-finite inputs) are read by the attention kernels as the OCP E4M3
 * values (0x78-0x7E: 256-448, 0x7F: NaN); every other code decodes exactly.
 * Requirements: head_dim % 16 == 0, block_size % 16 == 0, 16-byte aligned
 * bases and row starts (block_stride * elem_size and head_dim * elem_size
 * multiples of 16 for F16/F32, of 8 for I8 and FP8).
 */
typedef struct vcpp_kv_pages {
    int32_t dtype;
    int32_t block_size;
    int32_t num_kv_heads;
    int32_t head_dim;
    int64_t num_blocks;
    int64_t block_stride;
    int64_t scale_block_stride;
    const void* k;
    const void* v;
    const uint16_t* k_scale;
    const uint16_t* v_scale;
} vcpp_kv_pages;

/* ---- v2: batched paged decode ------------------------------------------ */

/*
 * Batched decode attention, one query token per sequence.
 *   q            [num_seqs][num_heads][head_dim] fp32
 *   out          [num_seqs][num_heads][head_dim] fp32 (overwritten)
 *   block_tables [num_seqs][max_blocks_per_seq] int32 physical block ids
 *   table_lens   [num_seqs] int32 usable entries per row, or NULL (= all
 *                max_blocks_per_seq) -- the reference's block_table.size()
 *   context_lens [num_seqs] int32 on the device
 *   max_context_len  host-side upper bound of context_lens (sizes the grid;
 *                a larger context_len is an error the kernel cannot report:
 *                positions past max_context_len are not attended)
 *   partition_size   0 (default): the tiles of all sequences are split
 *                evenly over the workgroups the GPU holds at once (fp16/int8/fp8)
 *                or (fp32) into partitions of 32..256 tokens sized so the
 *                workgroups fill the GPU about twice.  > 0 (a multiple of 16,
 *                <= 1024): fixed partitions -- the tiles are split into
 *                ranges of about that many tokens (fp16/int8/fp8: walked in
 *                runs by the resident workgroups) or partitions of exactly
 *                that many tokens (fp32).  Ranges that end inside a sequence
 *                leave partials, merged by a log-sum-exp kernel.
 *   workspace    device scratch of at least vcpp_decode_workspace_size(...)
 *                bytes (may be NULL when that size is 0); scratch for the
 *                call only, so calls that may overlap need separate ones.
 * Replaces the per-request loop around paged_attention()
 * (src/paged_engine.cpp:505-508, src/paged_attention.cpp:96-121).
 */
int vcpp_paged_decode(const vcpp_kv_pages* kv, const float* q, float* out,
                      const int32_t* block_tables, int32_t max_blocks_per_seq,
                      const int32_t* table_lens, const int32_t* context_lens,
                      int32_t num_seqs, int32_t max_context_len, int32_t num_heads,
                      int32_t partition_size, void* workspace, size_t workspace_bytes,
                      void* stream);

/* Workspace bytes vcpp_paged_decode needs for these arguments on the current
 * device (the split depends on its compute-unit count). */
size_t vcpp_decode_workspace_size(const vcpp_kv_pages* kv, int32_t num_seqs, int32_t num_heads,
                                  int32_t max_context_len, int32_t partition_size);

/*
 * vcpp_paged_decode without a workspace and without allocating: the split-K
 * partials go to a static device array of VCPP_NOALLOC_SCRATCH_BYTES that the
 * library holds on every GPU it runs on until the process ends.  No
 * counterpart in the reference: it is for callers that cannot allocate (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Arguments and results as vcpp_paged_decode.  A call whose
 * partials would need more than the array (vcpp_decode_workspace_size) fails
 * with VCPP_E_UNSUPPORTED and launches nothing; the balanced split
 * (partition_size 0) of a 256-CU GPU needs at most ~21 MB at head_dim 80.
 * Every call on a GPU shares that GPU's array: calls that may overlap on one
 * GPU (different streams) race; calls on one stream are ordered.
 */
#define VCPP_NOALLOC_SCRATCH_BYTES (64u << 20)
int vcpp_paged_decode_noalloc(const vcpp_kv_pages* kv, const float* q, float* out,
                              const int32_t* block_tables, int32_t max_blocks_per_seq,
                              const int32_t* table_lens, const int32_t* context_lens,
                              int32_t num_seqs, int32_t max_context_len, int32_t num_heads,
                              int32_t partition_size, void* stream);

/* ---- v2: chunked causal prefill ---------------------------------------- */

/*
 * Causal attention of chunks of new tokens appended to paged prefixes.  Chunk
 * c owns query rows q_start[c] .. q_start[c+1]-1; row i of the chunk attends
 * positions 0 .. prefix_lens[c] + i of its sequence through table row c --
 * the engine's per-position prefill (src/paged_engine.cpp:348-384,
 * src/model.cpp:1214-1220) done for the whole chunk at once.  The chunk's own
 * K/V must already be in the pages (written before the call, as the engine
 * does).
 *   q            fp16 (binary16 bits) [total_rows][num_heads][head_dim]
 *   out          fp32 [total_rows][num_heads][head_dim] (overwritten)
 *   block_tables [num_chunks][max_blocks_per_seq] int32
 *   q_start      [num_chunks + 1] int32 on the device (q_start[0] == 0)
 *   prefix_lens  [num_chunks] int32 on the device
 *   max_chunk_len host-side upper bound of the chunk lengths (sizes the grid;
 *                 a longer chunk is a caller error: rows the grid does not
 *                 reach -- the chunk's first rows before its last
 *                 max_chunk_len, rounded to whole query tiles, and in
 *                 vcpp_paged_prefill_split also rows past num_chunks *
 *                 max_chunk_len -- are left unwritten, never garbage)
 * KV dtypes: VCPP_KV_F16, VCPP_KV_I8 and VCPP_KV_FP8 (byte pages are widened to fp16 on the
 * way into LDS: FP8 to its values; int8 K to exact integers whose per-key scale multiplies the
 * score in fp32, int8 V to fp16(v * scale), one rounding); head_dim 64, 80 or 128;
 * num_heads / num_kv_heads any.
 * Replaces read_kv_prefill + compute_attention per position
 * (src/paged_attention.cpp:174-201, src/paged_engine.cpp:64-113,381-384).
 */
int vcpp_paged_prefill(const vcpp_kv_pages* kv, const uint16_t* q, float* out,
                       const int32_t* block_tables, int32_t max_blocks_per_seq,
                       const int32_t* q_start, const int32_t* prefix_lens, int32_t num_chunks,
                       int32_t max_chunk_len, int32_t num_heads, void* stream);

/*
 * vcpp_paged_prefill with the keys of each query tile split over several
 * workgroups when the chunks alone would leave the GPU under-filled (few
 * chunks on long prefixes, e.g. chunked prefill of one long request): each
 * part leaves unnormalised outputs and (max, sum) in the workspace and a
 * log-sum-exp merge writes `out`.  Same arguments and results as
 * vcpp_paged_prefill, plus
 *   max_prefix_len  host-side upper bound of prefix_lens (sizes the split)
 *   workspace       device scratch of at least vcpp_prefill_workspace_size(...)
 *                   bytes, 16-byte aligned (none needed when that is 0)
 * Calls on one stream may share a workspace; calls that overlap may not.
 * No reference counterpart: the reference prefills one position at a time
 * (src/paged_engine.cpp:381-384).
 */
int vcpp_paged_prefill_split(const vcpp_kv_pages* kv, const uint16_t* q, float* out,
                             const int32_t* block_tables, int32_t max_blocks_per_seq, const int32_t* q_start,
                             const int32_t* prefix_lens, int32_t num_chunks, int32_t max_chunk_len,
                             int32_t max_prefix_len, int32_t num_heads, void* workspace, size_t workspace_bytes,
                             void* stream);
size_t vcpp_prefill_workspace_size(const vcpp_kv_pages* kv, int32_t num_chunks, int32_t max_chunk_len,
                                   int32_t max_prefix_len, int32_t num_heads);

/* ---- v2: one scheduler step with decodes and prefill chunks ------------- */

/*
 * A step whose ScheduleOutput (src/scheduler.h:14-23) holds both decoding
 * requests and prefill chunks, served together as the engine's step does
 * (src/paged_engine.cpp:254-269): the decode of vcpp_paged_decode (arguments
 * d_* / dq / dout / num_seqs / max_context_len, balanced split) and the
 * prefill of vcpp_paged_prefill (pq / pout / p_* / q_start / prefix_lens /
 * num_chunks / max_chunk_len) over the same pages, with the same results.
 * By default the decode kernel and then the prefill kernel run on `stream`;
 * when both sides are present, the decode's split-K merge runs on a
 * library-owned side stream (default priority, one per device and caller
 * stream, so steps on different streams never share one, also under graph
 * capture) that waits for the decode kernel by an event, so that it overlaps
 * the prefill, and `stream` waits for it by another event before the call
 * returns, also when a later launch fails: all results are ordered on
 * `stream` as with the two separate calls (VCPP_NO_MERGE_FORK=1 keeps the
 * merge on `stream`).  With
 * VCPP_MIXED_FUSED=1, where the shape allows (fp16, int8 or FP8 pages;
 * head_dim 64 or 80; num_kv_heads a multiple of 4; <= 8 query heads per kv
 * head; a CU count that is a multiple of 8), both run in ONE launch that
 * keeps the decode and the prefill on every CU at once, followed by the
 * decode's merge (slower on MI355X; kept for measurement).  Either side may
 * be empty (num_seqs == 0, or num_chunks == 0).
 *   workspace    device scratch of at least vcpp_mixed_workspace_size(...)
 */
int vcpp_paged_mixed_step(const vcpp_kv_pages* kv, const float* dq, float* dout,
                          const int32_t* d_block_tables, int32_t d_max_blocks_per_seq,
                          const int32_t* d_table_lens, const int32_t* d_context_lens, int32_t num_seqs,
                          int32_t max_context_len, const uint16_t* pq, float* pout,
                          const int32_t* p_block_tables, int32_t p_max_blocks_per_seq,
                          const int32_t* q_start, const int32_t* prefix_lens, int32_t num_chunks,
                          int32_t max_chunk_len, int32_t num_heads, void* workspace,
                          size_t workspace_bytes, void* stream);

/* Workspace bytes vcpp_paged_mixed_step needs on the current device
 * (max_blocks_per_chunk = its p_max_blocks_per_seq). */
size_t vcpp_mixed_workspace_size(const vcpp_kv_pages* kv, int32_t num_seqs, int32_t num_heads,
                                 int32_t max_context_len, int32_t max_blocks_per_chunk);

/* ---- v2: writing K/V into the pages ------------------------------------ */

/*
 * Writes num_tokens new K/V rows into the pages described by kv (which must be
 * writable): token t goes to physical slot slots[t] = block_id * block_size +
 * position (slots[t] < 0, or a block id >= num_blocks, skips the token).
 *   k, v   [num_tokens][num_kv_heads][head_dim] fp32 on the device
 *   slots  [num_tokens] int64 on the device
 * Encoding by kv->dtype: F32 copies; F16 uses the reference encoder
 * (src/kv_cache_manager.cpp:157-179: mantissa truncated, values below the
 * normal range flushed to +/-0, overflow to +/-inf) unless fp16_round_nearest
 * is non-zero (IEEE round-to-nearest-even); I8 quantises each (token, kv head)
 * row symmetrically: scale = fp16_rne(max|x| / 127) into the scale page,
 * values rne(x / scale) clamped to +/-127 (0 when the scale is 0).
 * The device side of KVCacheManager::write_kv / write_kv_token /
 * write_kv_prefill (src/kv_cache_manager.cpp:297-314,
 * src/paged_attention.cpp:127-168), batched over tokens.
 */
int vcpp_write_kv(const vcpp_kv_pages* kv, const float* k, const float* v, const int64_t* slots,
                  int32_t num_tokens, int32_t fp16_round_nearest, void* stream);

/* ---- v2: query / key preparation (per-head norm, rotary embedding) ------ */

#define VCPP_ROPE_INTERLEAVED 0 /* pairs (2i, 2i+1): the CPU engine, src/paged_engine.cpp:47-62 */
#define VCPP_ROPE_HALF 1        /* pairs (i, i+head_dim/2): cuda/attention_kernels.cuh:249-287 */

/*
 * Fused in-place preparation of q and k for attention, one HBM pass:
 *   q  [num_tokens][num_heads][head_dim] fp32 on the device
 *   k  [num_tokens][num_kv_heads][head_dim] fp32, or NULL (q only)
 *   q_norm_weight, k_norm_weight  [head_dim] fp32, or NULL (no norm): per-head
 *      RMS norm y = (w * x) / sqrt(sum(x^2) / head_dim + eps), the reference
 *      rms_norm (src/paged_engine.cpp:14-20) applied to each head -- the
 *      Qwen3 q_norm / k_norm (src/model.h:88-89);
 *   positions  [num_tokens] int32, or NULL (no rotation): RoPE with
 *      theta = inv_freq[min(i, inv_freq_size - 1)] * pos for pair i, as
 *      rope_single (src/paged_engine.cpp:47-62) computes it; style selects the
 *      pairing (VCPP_ROPE_INTERLEAVED or VCPP_ROPE_HALF).
 *   inv_freq  [inv_freq_size] fp32 on the device (needed when positions is set)
 * The norm runs before the rotation (the Qwen3 order).  head_dim even and
 * <= 256.  Replaces the per-position rope_single calls of the engine
 * (src/paged_engine.cpp:361-362,377-378,484-485,500-501).
 */
int vcpp_qk_norm_rope(float* q, float* k, int32_t num_tokens, int32_t num_heads,
                      int32_t num_kv_heads, int32_t head_dim, const float* q_norm_weight,
                      const float* k_norm_weight, float eps, const int32_t* positions,
                      const float* inv_freq, int32_t inv_freq_size, int32_t style, void* stream);

/* RoPE alone on one tensor x [num_tokens][num_heads][head_dim] (in place). */
int vcpp_rope(float* x, int32_t num_tokens, int32_t num_heads, int32_t head_dim,
              const int32_t* positions, const float* inv_freq, int32_t inv_freq_size,
              int32_t style, void* stream);

/* Per-head RMS norm alone on x [num_rows][head_dim] (in place), weight [head_dim]. */
int vcpp_head_norm(float* x, const float* weight, float eps, int32_t num_rows, int32_t head_dim,
                   void* stream);

/* ---- v1: reference launcher signatures (cuda/attention.h) -------------- */

/*
 * cuda/attention.h:19-30.  Defined here (the reference leaves these open):
 *   q, out        [batch_size][num_heads][head_dim] fp32
 *   kv_cache      fp16 pages [num_blocks][2 (K, V)][block_size][num_kv_heads][head_dim]
 *                 (K and V behind the one pointer; num_blocks is not passed:
 *                 ids whose block would end past the device allocation that
 *                 holds kv_cache are skipped, hipMemGetAddressRange)
 *   block_tables  [batch_size][max_b ceil(context_lens[b] / block_size)] int32
 *   context_lens  HOST int32 [batch_size] (the reference reads it on the host,
 *                 cuda/attention.cu:25-28); the library stages a device copy.
 *   block_size    16 or 32; anything else launches nothing and records
 *                 VCPP_E_UNSUPPORTED in vcpp_last_error(), as do head counts
 *                 that are not positive multiples (VCPP_E_INVALID).
 * Runs on the null stream, asynchronously; uses a library-owned workspace.
 */
void paged_attention_cuda(const float* q, const uint16_t* kv_cache, const int32_t* block_tables,
                          const int32_t* context_lens, float* out, int32_t num_heads,
                          int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                          int32_t batch_size);

/*
 * cuda/attention.h:32-45 (flash_attention_cuda), contiguous K/V.  As in the
 * reference (cuda/attention.cu:58-124), only query row 0 of each (b, h) is
 * used and one output row per (b, h) is written:
 *   q             [batch_size][num_heads][q_len][head_dim] fp32
 *   k, v          [batch_size][num_heads][kv_len][head_dim] fp32
 *   out           [batch_size][num_heads][head_dim] fp32
 *   attn_weights  [batch_size * num_heads][kv_len] fp32, receives the softmax
 *                 probabilities (logits * 1/sqrt(head_dim), sum + 1e-9)
 *   attn_mask     [kv_len] fp32 or NULL; attn_mask[s] < 0 sets logit s to -1e9
 * All pointers are device memory (the reference dereferences them on the
 * host).  kv_len, q_len and head_dim must be > 0 (else VCPP_E_INVALID is
 * recorded and nothing runs).  Null stream, asynchronous.
 */
void flash_attention_cuda(const float* q, const float* k, const float* v, float* out,
                          float* attn_weights, int32_t batch_size, int32_t num_heads,
                          int32_t head_dim, int32_t q_len, int32_t kv_len, const float* attn_mask);

/*
 * cuda/attention.h:47-56 (apply_rope_cuda), with the reference kernel's
 * semantics (cuda/attention_kernels.cuh:249-287, launched by
 * cuda/attention.cu:130-145):
 *   q, k      [batch_size][total_dim] fp32 on the device, rotated in place
 *   cos, sin  [head_dim / 2] fp32 on the device, one row for every batch row
 * Element d (head d / head_dim, hdim = d % head_dim < head_dim / 2) pairs with
 * d + head_dim / 2, or with itself when that index reaches total_dim (then the
 * second write, x s + x c, is what remains).  Null stream; returns after the
 * kernel finished, as the reference does (cudaDeviceSynchronize).
 */
void apply_rope_cuda(float* q, float* k, const float* cos, const float* sin, int32_t total_dim,
                     int32_t head_dim, int32_t batch_size);

/*
 * cuda/attention.h:58-66 (head_norm_cuda).  The reference launcher defines its
 * kernel but launches nothing (cuda/attention.cu:152-189); this one does what
 * its comment states: x [batch_size][num_heads][head_dim] fp32 on the device,
 * each head scaled in place by weight[d] / sqrt(sum(x^2) / head_dim + eps)
 * (src/paged_engine.cpp:14-20 per head).  Null stream, returns when done.
 */
void head_norm_cuda(float* x, const float* weight, float eps, int32_t num_heads, int32_t head_dim,
                    int32_t batch_size);

/* ---- instrumentation (no reference counterpart) --------------------------- */

/* Kernel ids for vcpp_profile_read. */
#define VCPP_KERNEL_DECODE 0  /* decode attention (fp16/int8/fp8 MFMA or fp32) */
#define VCPP_KERNEL_MERGE 1   /* split-K log-sum-exp merge */
#define VCPP_KERNEL_PREFILL 2 /* chunked causal prefill */
#define VCPP_KERNEL_MIXED 3   /* fused decode + prefill step (vcpp_paged_mixed_step) */

/* Start (on != 0) or stop per-kernel timing and clear the counters.  While on,
 * each launch records a HIP event before and after the kernel on the stream
 * it is launched on. */
int vcpp_profile_enable(int on);
/* Total milliseconds and launch count of one kernel since the last enable;
 * waits for the recorded events. */
int vcpp_profile_read(int kernel_id, double* total_ms, int64_t* launches);

#ifdef __cplusplus
}
#endif
#endif
