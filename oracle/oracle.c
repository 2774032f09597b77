/*
 * oracle.c -- CPU restatement of the reference paged-attention path.
 *
 * TEST INFRASTRUCTURE ONLY (see oracle.h).  Built with -ffp-contract=off so the
 * arithmetic is the plain sequential fp32 the reference source describes.
 *
 * Pins (tests/test_oracle.py): the compiled reference (oracle/_ref), the
 * committed golden vectors in tests/golden/, closed forms (ctx=1, constant
 * keys, dominant logit, ctx=0), fp64 brute force, the split-K LSE identity and
 * fp16/int8 known-answer values.  No function here is "parity unpinned".
 */
#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ---- FP8 E4M3 codec (src/quantization.cpp) ---------------------------- */

/* compute_e4m3_to_float, src/quantization.cpp:25-48. */
float orc_fp8_decode(uint8_t b) {
    const int sign = (b >> 7) & 1, e = (b >> 3) & 0xF, m = b & 7;
    if (e == 0xF) {
        if (m == 6) return sign ? -INFINITY : INFINITY;
        return NAN;
    }
    float v;
    if (e == 0) v = (float)m / 8.0f * ldexpf(1.0f, -6);
    else v = (1.0f + (float)m / 8.0f) * ldexpf(1.0f, e - 7);
    return sign ? -v : v;
}

/* compute_float_to_e4m3, src/quantization.cpp:50-82 -- the encoder of the KV
 * pool's write path (float_to_fp8_e4m3_batch, :183-188): the sign is v < 0
 * (so -0.0 encodes as 0x00); scan every code of that sign and keep the first
 * with the smallest |abs_v - |decode(code)|| (NaN errors never win). */
uint8_t orc_fp8_encode(float v) {
    if (isnan(v)) return 0xFF;
    if (isinf(v)) return v > 0 ? 0x7E : 0xFE;
    const int sign = v < 0 ? 1 : 0;
    const float a = fabsf(v);
    if (a == 0.0f) return (uint8_t)(sign << 7);
    uint8_t best = 0;
    float best_err = INFINITY;
    for (int i = 0; i < 256; i++) {
        if ((i >> 7) != sign) continue;
        const float err = fabsf(a - fabsf(orc_fp8_decode((uint8_t)i)));
        if (err < best_err) {
            best_err = err;
            best = (uint8_t)i;
        }
    }
    return best;
}

void orc_fp8_encode_n(const float* x, uint8_t* b, int64_t n) {
    for (int64_t i = 0; i < n; i++) b[i] = orc_fp8_encode(x[i]);
}

void orc_fp8_decode_n(const uint8_t* b, float* x, int64_t n) {
    for (int64_t i = 0; i < n; i++) x[i] = orc_fp8_decode(b[i]);
}

/* ---- fp16 codec ------------------------------------------------------- */

/* Reference fp32 -> fp16 encoder, src/kv_cache_manager.cpp:157-179:
 * truncates the mantissa (frac >> 13), flushes anything below 2^-14 to a
 * signed zero, saturates overflow to inf, keeps NaN as quiet 0x7C01 class. */
uint16_t orc_f16_encode_trunc(float x) {
    uint32_t b;
    memcpy(&b, &x, 4);
    uint32_t s = b >> 31, e = (b >> 23) & 0xFFu, f = b & 0x7FFFFFu;
    if (e == 0xFFu) return (uint16_t)((s << 15) | (0x1Fu << 10) | (f ? 1u : 0u));
    if (e == 0) return (uint16_t)(s << 15);
    int ee = (int)e - 127 + 15;
    if (ee <= 0) return (uint16_t)(s << 15);
    if (ee >= 31) return (uint16_t)((s << 15) | (0x1Fu << 10));
    return (uint16_t)((s << 15) | ((uint32_t)ee << 10) | ((f >> 13) & 0x3FFu));
}

/* Reference fp16 -> fp32 decoder, src/kv_cache_manager.cpp:120-143: exact for
 * zeros, subnormals and normals; exponent 31 (inf and NaN alike) -> +/-inf. */
float orc_f16_decode(uint16_t h) {
    uint32_t s = (h >> 15) & 1u, e = (h >> 10) & 0x1Fu, f = h & 0x3FFu;
    uint32_t bits;
    if (e == 0) {
        if (f == 0) {
            bits = s << 31;
        } else {
            int ee = 1;
            while ((f & 0x400u) == 0) { f <<= 1; ee--; }
            f &= 0x3FFu;
            bits = (s << 31) | ((uint32_t)(127 - 15 + ee) << 23) | (f << 13);
        }
    } else if (e == 31) {
        return s ? -INFINITY : INFINITY;
    } else {
        bits = (s << 31) | ((127 - 15 + e) << 23) | (f << 13);
    }
    float out;
    memcpy(&out, &bits, 4);
    return out;
}

void orc_f16_encode_trunc_n(const float* x, uint16_t* h, int64_t n) {
    for (int64_t i = 0; i < n; i++) h[i] = orc_f16_encode_trunc(x[i]);
}

void orc_f16_decode_n(const uint16_t* h, float* x, int64_t n) {
    for (int64_t i = 0; i < n; i++) x[i] = orc_f16_decode(h[i]);
}

/* IEEE round-to-nearest-even fp32 -> fp16 (used for int8 scales, which are a
 * build definition, not a reference format). */
uint16_t orc_f16_encode_rne(float x) {
    uint32_t b;
    memcpy(&b, &x, 4);
    uint32_t s = (b >> 16) & 0x8000u;
    uint32_t e = (b >> 23) & 0xFFu;
    uint32_t f = b & 0x7FFFFFu;
    if (e == 0xFFu) return (uint16_t)(s | 0x7C00u | (f ? 0x200u : 0u));
    int32_t ee = (int32_t)e - 127 + 15;
    if (ee >= 31) return (uint16_t)(s | 0x7C00u);
    if (ee <= 0) {
        if (ee < -10) return (uint16_t)s;
        uint32_t m = f | 0x800000u;
        int shift = 14 - ee;               /* 14..24 */
        uint32_t half = 1u << (shift - 1);
        uint32_t r = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        if (rem > half || (rem == half && (r & 1u))) r++;
        return (uint16_t)(s | r);
    }
    uint32_t r = ((uint32_t)ee << 10) | (f >> 13);
    uint32_t rem = f & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) r++;
    return (uint16_t)(s | r);
}

/* ---- int8 quantiser (build definition) -------------------------------- */

void orc_quant_i8(const float* x, int32_t d, int8_t* q, uint16_t* scale) {
    float amax = 0.0f;
    for (int32_t i = 0; i < d; i++) {
        float a = fabsf(x[i]);
        if (a > amax) amax = a;
    }
    uint16_t sh = orc_f16_encode_rne(amax / 127.0f);
    *scale = sh;
    float s = orc_f16_decode(sh);
    for (int32_t i = 0; i < d; i++) {
        float r = (s > 0.0f) ? nearbyintf(x[i] / s) : 0.0f;
        if (r > 127.0f) r = 127.0f;
        if (r < -127.0f) r = -127.0f;
        q[i] = (int8_t)r;
    }
}

void orc_quant_i8_rows(const float* x, int64_t rows, int32_t d, int8_t* q, uint16_t* scales) {
    for (int64_t r = 0; r < rows; r++) orc_quant_i8(x + r * d, d, q + r * d, scales + r);
}

/* ---- pool access ------------------------------------------------------- */

/* Mirrors BlockPool::get_k/get_v returning NULL for an out-of-range block id
 * (src/kv_cache_manager.cpp:90-95) and the float view with conversion at
 * access (src/kv_cache_manager.cpp:186-211).  Returns 0 when the block is
 * invalid; otherwise fills `row` with the head_dim values of (token, kv head). */
static int load_row(const orc_pool* p, int which, int32_t block_id, int32_t tok,
                    int32_t kv_h, float* row) {
    if (block_id < 0 || (int64_t)block_id >= p->num_blocks) return 0;
    const int32_t D = p->head_dim;
    int64_t off = (int64_t)block_id * p->block_stride +
                  ((int64_t)tok * p->num_kv_heads + kv_h) * D;
    const void* base = which ? p->v : p->k;
    if (p->kind == ORC_F32) {
        memcpy(row, (const float*)base + off, sizeof(float) * (size_t)D);
    } else if (p->kind == ORC_F16) {
        const uint16_t* h = (const uint16_t*)base + off;
        for (int32_t d = 0; d < D; d++) row[d] = orc_f16_decode(h[d]);
    } else if (p->kind == ORC_FP8) {
        const uint8_t* c = (const uint8_t*)base + off;
        for (int32_t d = 0; d < D; d++) row[d] = orc_fp8_decode(c[d]);
    } else {
        const int8_t* c = (const int8_t*)base + off;
        const uint16_t* sc = which ? p->v_scale : p->k_scale;
        float s = orc_f16_decode(sc[(int64_t)block_id * p->scale_block_stride +
                                    (int64_t)kv_h * p->block_size + tok]);
        for (int32_t d = 0; d < D; d++) row[d] = (float)c[d] * s;
    }
    return 1;
}

static float dot_f32(const float* a, const float* b, int32_t n) {
    float acc = 0.0f;
    for (int32_t i = 0; i < n; i++) acc += a[i] * b[i];
    return acc;
}

/* ---- single-query paged attention ------------------------------------- */

/* One head of src/paged_attention.cpp:26-89: three passes over the logical
 * positions, each recomputing q.k; max initialised to -1e9f (:34), the sum
 * gets +1e-9f (:67), positions past the table (:38) or on an invalid block
 * (:42) are skipped. */
static void attend_head(const orc_pool* p, const float* q_h, int32_t kv_h,
                        const int32_t* table, int32_t table_len, int32_t seq_len,
                        float* o_h) {
    const int32_t D = p->head_dim, BS = p->block_size;
    const float scale = 1.0f / sqrtf((float)D);
    float krow[512], vrow[512];
    for (int32_t d = 0; d < D; d++) o_h[d] = 0.0f;

    float max_logit = -1e9f;
    for (int32_t pos = 0; pos < seq_len; pos++) {
        int32_t bi = pos / BS, slot = pos % BS;
        if (bi >= table_len) continue;
        if (!load_row(p, 0, table[bi], slot, kv_h, krow)) continue;
        float logit = dot_f32(q_h, krow, D) * scale;
        if (logit > max_logit) max_logit = logit;
    }
    float sum_exp = 0.0f;
    for (int32_t pos = 0; pos < seq_len; pos++) {
        int32_t bi = pos / BS, slot = pos % BS;
        if (bi >= table_len) continue;
        if (!load_row(p, 0, table[bi], slot, kv_h, krow)) continue;
        float logit = dot_f32(q_h, krow, D) * scale;
        sum_exp += expf(logit - max_logit);
    }
    sum_exp += 1e-9f;
    for (int32_t pos = 0; pos < seq_len; pos++) {
        int32_t bi = pos / BS, slot = pos % BS;
        if (bi >= table_len) continue;
        if (!load_row(p, 0, table[bi], slot, kv_h, krow)) continue;
        if (!load_row(p, 1, table[bi], slot, kv_h, vrow)) continue;
        float w = expf(dot_f32(q_h, krow, D) * scale - max_logit) / sum_exp;
        for (int32_t d = 0; d < D; d++) o_h[d] += w * vrow[d];
    }
}

/* src/paged_attention.cpp:11-90 (GQA map kv_h = h / (H/Hkv), :22,27). */
void orc_paged_attention(const orc_pool* pool, const float* q, const int32_t* table,
                         int32_t table_len, int32_t seq_len, int32_t num_heads,
                         float* out) {
    const int32_t D = pool->head_dim;
    const int32_t hpg = num_heads / pool->num_kv_heads;
    for (int32_t h = 0; h < num_heads; h++)
        attend_head(pool, q + (int64_t)h * D, h / hpg, table, table_len, seq_len,
                    out + (int64_t)h * D);
}

/* ---- threaded batch drivers ------------------------------------------- */

typedef struct {
    const orc_pool* pool;
    const float* q;
    float* out;
    const int32_t* tables;
    int64_t table_stride;
    const int32_t* table_lens;  /* decode */
    const int32_t* ctx;         /* decode */
    const int32_t* q_start;     /* prefill */
    const int32_t* prefix;      /* prefill */
    const int32_t* row_chunk;   /* prefill: chunk of each row */
    int64_t num_items;          /* rows * heads */
    int32_t num_heads;
    int32_t mode;               /* 0 decode, 1 prefill */
    int32_t tid, nthreads;
} job_t;

static void* run_job(void* arg) {
    job_t* j = (job_t*)arg;
    const int32_t H = j->num_heads, D = j->pool->head_dim;
    const int32_t hpg = H / j->pool->num_kv_heads;
    for (int64_t it = j->tid; it < j->num_items; it += j->nthreads) {
        int64_t row = it / H;
        int32_t h = (int32_t)(it % H);
        int32_t seq_row, seq_len, tlen;
        if (j->mode == 0) {
            seq_row = (int32_t)row;
            seq_len = j->ctx[row];
            tlen = (int32_t)j->table_stride;
            if (j->table_lens && j->table_lens[row] < tlen) tlen = j->table_lens[row];
        } else {
            seq_row = j->row_chunk[row];
            seq_len = j->prefix[seq_row] + (int32_t)(row - j->q_start[seq_row]) + 1;
            tlen = (int32_t)j->table_stride;
        }
        attend_head(j->pool, j->q + (row * H + h) * D, h / hpg,
                    j->tables + (int64_t)seq_row * j->table_stride, tlen, seq_len,
                    j->out + (row * H + h) * D);
    }
    return NULL;
}

static void run_threads(job_t* proto, int32_t nthreads) {
    if (nthreads < 1) nthreads = 1;
    if (nthreads > 256) nthreads = 256;
    pthread_t th[256];
    job_t jobs[256];
    for (int32_t t = 0; t < nthreads; t++) {
        jobs[t] = *proto;
        jobs[t].tid = t;
        jobs[t].nthreads = nthreads;
    }
    for (int32_t t = 1; t < nthreads; t++) pthread_create(&th[t], NULL, run_job, &jobs[t]);
    run_job(&jobs[0]);
    for (int32_t t = 1; t < nthreads; t++) pthread_join(th[t], NULL);
}

void orc_decode_batch(const orc_pool* pool, const float* q, const int32_t* tables,
                      int64_t table_stride, const int32_t* table_lens,
                      const int32_t* ctx, int32_t batch, int32_t num_heads,
                      float* out, int32_t nthreads) {
    job_t j;
    memset(&j, 0, sizeof(j));
    j.pool = pool; j.q = q; j.out = out; j.tables = tables;
    j.table_stride = table_stride; j.table_lens = table_lens; j.ctx = ctx;
    j.num_items = (int64_t)batch * num_heads; j.num_heads = num_heads; j.mode = 0;
    run_threads(&j, nthreads);
}

void orc_prefill_batch(const orc_pool* pool, const float* q, const int32_t* tables,
                       int64_t table_stride, const int32_t* q_start,
                       const int32_t* prefix, int32_t num_chunks, int32_t num_heads,
                       float* out, int32_t nthreads) {
    int64_t rows = q_start[num_chunks];
    int32_t* row_chunk = (int32_t*)malloc(sizeof(int32_t) * (size_t)(rows > 0 ? rows : 1));
    for (int32_t c = 0; c < num_chunks; c++)
        for (int32_t r = q_start[c]; r < q_start[c + 1]; r++) row_chunk[r] = c;
    job_t j;
    memset(&j, 0, sizeof(j));
    j.pool = pool; j.q = q; j.out = out; j.tables = tables;
    j.table_stride = table_stride; j.q_start = q_start; j.prefix = prefix;
    j.row_chunk = row_chunk; j.num_items = rows * num_heads; j.num_heads = num_heads;
    j.mode = 1;
    run_threads(&j, nthreads);
    free(row_chunk);
}

/* ---- brute force and split-K ------------------------------------------ */

void orc_dense_f64(const double* q, const double* k, const double* v, int32_t n,
                   int32_t d, double scale, double* out) {
    double* s = (double*)malloc(sizeof(double) * (size_t)(n > 0 ? n : 1));
    double m = -INFINITY, l = 0.0;
    for (int32_t i = 0; i < n; i++) {
        double acc = 0.0;
        for (int32_t t = 0; t < d; t++) acc += q[t] * k[(int64_t)i * d + t];
        s[i] = acc * scale;
        if (s[i] > m) m = s[i];
    }
    for (int32_t t = 0; t < d; t++) out[t] = 0.0;
    for (int32_t i = 0; i < n; i++) {
        double w = exp(s[i] - m);
        l += w;
        for (int32_t t = 0; t < d; t++) out[t] += w * v[(int64_t)i * d + t];
    }
    for (int32_t t = 0; t < d; t++) out[t] = (n > 0) ? out[t] / l : 0.0;
    free(s);
}

/* Partial softmax state over positions [p0, p1): m = max logit (or -1e9f if
 * none valid), l = sum exp(s - m), o = sum exp(s - m) v (unnormalised). */
void orc_partial(const orc_pool* p, const float* q_h, int32_t kv_h,
                 const int32_t* table, int32_t table_len, int32_t p0, int32_t p1,
                 float* m, float* l, float* o) {
    const int32_t D = p->head_dim, BS = p->block_size;
    const float scale = 1.0f / sqrtf((float)D);
    float krow[512], vrow[512];
    float mx = -1e9f, sum = 0.0f;
    for (int32_t pos = p0; pos < p1; pos++) {
        int32_t bi = pos / BS;
        if (bi >= table_len || !load_row(p, 0, table[bi], pos % BS, kv_h, krow)) continue;
        float s = dot_f32(q_h, krow, D) * scale;
        if (s > mx) mx = s;
    }
    for (int32_t d = 0; d < D; d++) o[d] = 0.0f;
    for (int32_t pos = p0; pos < p1; pos++) {
        int32_t bi = pos / BS;
        if (bi >= table_len || !load_row(p, 0, table[bi], pos % BS, kv_h, krow)) continue;
        if (!load_row(p, 1, table[bi], pos % BS, kv_h, vrow)) continue;
        float w = expf(dot_f32(q_h, krow, D) * scale - mx);
        sum += w;
        for (int32_t d = 0; d < D; d++) o[d] += w * vrow[d];
    }
    *m = mx;
    *l = sum;
}

/* out = (sum_i e^{m_i - M} o_i) / (sum_i e^{m_i - M} l_i + 1e-9), M = max m_i. */
void orc_lse_merge(const float* m, const float* l, const float* o, int32_t np,
                   int32_t d, float* out) {
    float M = -1e9f;
    for (int32_t i = 0; i < np; i++) if (m[i] > M) M = m[i];
    float L = 0.0f;
    for (int32_t t = 0; t < d; t++) out[t] = 0.0f;
    for (int32_t i = 0; i < np; i++) {
        float w = expf(m[i] - M);
        L += w * l[i];
        for (int32_t t = 0; t < d; t++) out[t] += w * o[(int64_t)i * d + t];
    }
    L += 1e-9f;
    for (int32_t t = 0; t < d; t++) out[t] /= L;
}

/* ---- deterministic inputs --------------------------------------------- */

static uint64_t splitmix64(uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

void orc_fill_normal(uint64_t seed, float* out, int64_t n, double mean, double std) {
    const double two_pi = 6.283185307179586476925286766559;
    uint64_t base = splitmix64(seed);
    for (int64_t i = 0; i < n; i++) {
        uint64_t a = splitmix64(base + 2ull * (uint64_t)i);
        uint64_t b = splitmix64(base + 2ull * (uint64_t)i + 1ull);
        double u1 = ((double)(a >> 11) + 1.0) * (1.0 / 9007199254740992.0);
        double u2 = (double)(b >> 11) * (1.0 / 9007199254740992.0);
        double z = sqrt(-2.0 * log(u1)) * cos(two_pi * u2);
        out[i] = (float)(mean + std * z);
    }
}

void orc_fill_uniform_int(uint64_t seed, int32_t* out, int64_t n, int32_t lo, int32_t hi) {
    uint64_t base = splitmix64(seed ^ 0xA5A5A5A5A5A5A5A5ull);
    uint64_t span = (uint64_t)((int64_t)hi - (int64_t)lo + 1);
    for (int64_t i = 0; i < n; i++)
        out[i] = (int32_t)((int64_t)lo + (int64_t)(splitmix64(base + (uint64_t)i) % span));
}

void orc_permutation(uint64_t seed, int32_t* out, int32_t n) {
    uint64_t base = splitmix64(seed ^ 0x5A5A5A5A5A5A5A5Aull);
    for (int32_t i = 0; i < n; i++) out[i] = i;
    for (int32_t i = n - 1; i > 0; i--) {
        int32_t j = (int32_t)(splitmix64(base + (uint64_t)i) % (uint64_t)(i + 1));
        int32_t t = out[i]; out[i] = out[j]; out[j] = t;
    }
}

/* cuda/attention.cu:58-124 (host loops of flash_attention_cuda). */
void orc_flash_attention(const float* q, const float* k, const float* v, float* out, float* w,
                         int32_t batch, int32_t heads, int32_t head_dim, int32_t q_len,
                         int32_t kv_len, const float* mask) {
    const float scale = 1.0f / sqrtf((float)head_dim);
    for (int32_t b = 0; b < batch; ++b) {
        for (int32_t h = 0; h < heads; ++h) {
            const int64_t bh = (int64_t)b * heads + h;
            const float* qr = q + bh * head_dim * q_len; /* row 0 (:90) */
            const float* kb = k + bh * head_dim * kv_len;
            const float* vb = v + bh * head_dim * kv_len;
            float* lg = w + bh * kv_len;
            for (int32_t s = 0; s < kv_len; ++s) {
                float dot = 0.0f;
                for (int32_t d = 0; d < head_dim; ++d) dot += qr[d] * kb[(int64_t)s * head_dim + d];
                lg[s] = dot * scale;
            }
            if (mask)
                for (int32_t s = 0; s < kv_len; ++s)
                    if (mask[s] < 0) lg[s] = -1e9f;
            float mx = lg[0];
            for (int32_t s = 1; s < kv_len; ++s) mx = fmaxf(mx, lg[s]);
            float sum = 0.0f;
            for (int32_t s = 0; s < kv_len; ++s) {
                lg[s] = expf(lg[s] - mx);
                sum += lg[s];
            }
            for (int32_t s = 0; s < kv_len; ++s) lg[s] /= (sum + 1e-9f);
            float* o = out + bh * head_dim;
            for (int32_t d = 0; d < head_dim; ++d) {
                float acc = 0.0f;
                for (int32_t s = 0; s < kv_len; ++s) acc += lg[s] * vb[(int64_t)s * head_dim + d];
                o[d] = acc;
            }
        }
    }
}

/* ---- query / key preparation ------------------------------------------ */

/* src/paged_engine.cpp:14-20 (rms_norm) applied to each head_dim row: the sum
 * of squares in order, inv = 1 / sqrt(sum / dim + eps), y = (w * x) * inv. */
void orc_head_norm(float* x, const float* w, float eps, int64_t rows, int32_t head_dim) {
    for (int64_t r = 0; r < rows; ++r) {
        float* xr = x + r * head_dim;
        float ss = 0.0f;
        for (int32_t i = 0; i < head_dim; ++i) ss += xr[i] * xr[i];
        const float inv = 1.0f / sqrtf(ss / (float)head_dim + eps);
        for (int32_t i = 0; i < head_dim; ++i) xr[i] = w[i] * xr[i] * inv;
    }
}

/* src/paged_engine.cpp:47-62 (rope_single) for every token at its own
 * position: pair i uses inv_freq[min(i, n_freq - 1)] * (float)pos, cosf/sinf,
 * and the pair (2i, 2i + 1) (style 0) or (i, i + head_dim / 2) (style 1, the
 * pairing of cuda/attention_kernels.cuh:249-287). */
void orc_rope(float* x, int32_t num_tokens, int32_t num_heads, int32_t head_dim,
              const int32_t* positions, const float* inv_freq, int32_t n_freq, int32_t style) {
    const int32_t half = head_dim / 2;
    for (int32_t t = 0; t < num_tokens; ++t) {
        const float pos = (float)positions[t];
        for (int32_t h = 0; h < num_heads; ++h) {
            float* xh = x + ((int64_t)t * num_heads + h) * head_dim;
            for (int32_t i = 0; i < half; ++i) {
                const int32_t fi = i < n_freq - 1 ? i : n_freq - 1;
                const float freq = inv_freq[fi] * pos;
                const float c = cosf(freq), s = sinf(freq);
                const int32_t i0 = style ? i : 2 * i, i1 = style ? i + half : 2 * i + 1;
                const float x0 = xh[i0], x1 = xh[i1];
                xh[i0] = x0 * c - x1 * s;
                xh[i1] = x0 * s + x1 * c;
            }
        }
    }
}

/* cuda/attention_kernels.cuh:249-287 as launched by apply_rope_cuda
 * (cuda/attention.cu:130-145): cos/sin [head_dim / 2] shared by every batch
 * row; element d with d % head_dim < head_dim / 2 pairs with d + head_dim / 2,
 * or with itself past total_dim (the second store then wins). */
void orc_rope_table(float* q, float* k, const float* cs, const float* sn, int32_t total_dim,
                    int32_t head_dim, int32_t batch) {
    for (int32_t b = 0; b < batch; ++b) {
        float* qb = q + (int64_t)b * total_dim;
        float* kb = k + (int64_t)b * total_dim;
        for (int32_t d = 0; d < total_dim; ++d) {
            const int32_t hd = d % head_dim;
            if (hd >= head_dim / 2) continue;
            const float c = cs[hd], s = sn[hd];
            int32_t i1 = d + head_dim / 2;
            if (i1 >= total_dim) i1 = d;
            const float q0 = qb[d], q1 = qb[i1], k0 = kb[d], k1 = kb[i1];
            qb[d] = q0 * c - q1 * s;
            qb[i1] = q0 * s + q1 * c;
            kb[d] = k0 * c - k1 * s;
            kb[i1] = k0 * s + k1 * c;
        }
    }
}
