/*
 * CPU oracle for the grouped-query attention path -- TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load this library, and only to check results / as the CPU baseline.  The HIP
 * product never links it and never falls back to it.
 *
 * It restates, in plain C, the reference engine's scalar ("NAIVE" backend)
 * semantics so that results can be compared element by element:
 *
 *   oracle_rope       <- src/ops.cpp:1223-1281  (rope)
 *   oracle_softmax    <- src/ops.cpp:1072-1091  (softmax)
 *   oracle_attention  <- src/ops.cpp:1317-1371 (append) + the naive branches
 *                        src/ops.cpp:1425-1433 (scores) and 1494-1508 (P.V);
 *                        KV layout src/run_state.h:93-101, GQA map
 *                        src/ops.cpp:1329/1383, scale src/ops.cpp:1335
 *   oracle_prefill    <- the token-by-token prompt loop src/generate.cpp:56-59
 *                        restricted to the attention block src/forward.cpp:192-208
 *   oracle_fp16_to_f32 <- src/ops.cpp:119-156
 *   oracle_matmul     <- matmul() src/ops.cpp:959-983 and the naive branches of
 *                        matmul_f32/f16/q8_0/q4_0/q6_k src/ops.cpp:178-957;
 *                        block layouts src/gguf.h:56-135
 *   oracle_rmsnorm    <- src/ops.cpp:1003-1055 (naive branch)
 *   oracle_vec_add    <- src/ops.cpp:1165-1184 (naive branch)
 *   oracle_silu, oracle_elementwise_mul <- src/ops.cpp:1107-1148 (naive)
 *   oracle_ffn_swiglu <- src/ops.cpp:1535-1564
 *   oracle_embed      <- embed_token() src/forward.cpp:17-134
 *   oracle_forward    <- forward() src/forward.cpp:167-266 (with the ops above;
 *                        weights by pointer instead of by GGUF tensor name)
 *   oracle_argmax     <- sample_argmax() src/ops.cpp:1587-1597
 *
 * Float semantics: every product and sum is rounded separately, as the
 * reference's x86-64 -O2 build does (no FMA in the baseline ISA).  Build with
 * -ffp-contract=off; the libm calls (powf/cosf/sinf/expf/sqrtf) are the ones
 * the reference makes through std::pow/std::cos/std::sin/std::exp/std::sqrt.
 *
 * Pinning (how each function is checked independently of itself):
 *   - golden vectors written in this container from the compiled reference
 *     (tests/golden/), bit-exact;
 *   - live comparison with oracle/_ref (the reference's own ops.cpp) where built;
 *   - closed forms and invariants (rope pair formula, norm preservation,
 *     softmax sums/limits, pos-0 identity, equal-key averaging, GQA map);
 *   - fp64 brute force (oracle_attention_f64) and torch SDPA on the CPU.
 *
 * oracle_fault() plants deliberate mistakes so the tests can show that each
 * pin catches a plausible error (a dropped term, a wrong sign or index).
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <string.h>
#include <stdlib.h>
#include <pthread.h>

/* Planted-mistake switch (tests only). 0 = faithful. */
static int g_fault = 0;
void oracle_fault(int mode) { g_fault = mode; }

enum {
    FAULT_NONE = 0,
    FAULT_ROPE_SIN_SIGN = 1,   /* x0' = x0*c + x1*s                           */
    FAULT_GQA_MODULO = 2,      /* kvh = qh % n_head_kv instead of qh / ratio  */
    FAULT_NO_SCALE = 3,        /* drop 1/sqrt(head_dim)                       */
    FAULT_SKIP_LAST = 4,       /* attend over 0..pos-1 (off by one)           */
    FAULT_ROPE_PAIR_HALF = 5,  /* rotate (i, i+hd/2) halves, not (2i, 2i+1)   */
    FAULT_SOFTMAX_NO_MAX = 6,  /* skip the max subtraction                    */
    FAULT_Q4_NIBBLE_ORDER = 7, /* low nibble -> element 2j, high -> 2j+1      */
    FAULT_Q6K_QH_SHIFT = 8,    /* upper 2 bits taken from the wrong qh pair   */
    FAULT_RMS_NO_MEAN = 9,     /* sum of squares not divided by size          */
    FAULT_SILU_SIGN = 10,      /* sigmoid(+x) instead of sigmoid(-x) flip     */
    FAULT_FFN_SWAP = 11,       /* silu applied to the up projection           */
    FAULT_FWD_NO_RESIDUAL = 12,/* attention output replaces x (no residual)   */
};

/* ---- rope: src/ops.cpp:1223-1281 ------------------------------------- */
static void rope_heads(float* x, int n_heads, int pos, int head_dim, float freq_base)
{
    const int n_pairs = head_dim / 2;
    for (int h = 0; h < n_heads; ++h) {
        float* row = x + (size_t)h * head_dim;
        for (int i = 0; i < n_pairs; ++i) {
            /* same float expression as the reference: 1/powf(base, 2i/hd) */
            float expo = (float)(2 * i) / (float)head_dim;
            float freq = 1.0f / powf(freq_base, expo);
            float angle = (float)pos * freq;
            float c = cosf(angle);
            float s = sinf(angle);
            int a = 2 * i, b = 2 * i + 1;
            if (g_fault == FAULT_ROPE_PAIR_HALF) { a = i; b = i + n_pairs; }
            float x0 = row[a];
            float x1 = row[b];
            float t0 = x0 * c;
            float t1 = x1 * s;
            float t2 = x0 * s;
            float t3 = x1 * c;
            row[a] = (g_fault == FAULT_ROPE_SIN_SIGN) ? t0 + t1 : t0 - t1;
            row[b] = t2 + t3;
        }
    }
}

void oracle_rope(float* q, float* k, int pos, int head_dim, int n_head,
                 int n_head_kv, float freq_base)
{
    rope_heads(q, n_head, pos, head_dim, freq_base);
    rope_heads(k, n_head_kv, pos, head_dim, freq_base);
}

/* One (cos, sin) pair per (position, pair index), same expressions as above.
 * Used by tests to check the device RoPE table bit for bit. */
void oracle_rope_table(float* cs, int n_pos, int head_dim, float freq_base)
{
    const int n_pairs = head_dim / 2;
    for (int p = 0; p < n_pos; ++p)
        for (int i = 0; i < n_pairs; ++i) {
            float expo = (float)(2 * i) / (float)head_dim;
            float freq = 1.0f / powf(freq_base, expo);
            float angle = (float)p * freq;
            cs[((size_t)p * n_pairs + i) * 2 + 0] = cosf(angle);
            cs[((size_t)p * n_pairs + i) * 2 + 1] = sinf(angle);
        }
}

/* ---- softmax: src/ops.cpp:1072-1091 ---------------------------------- */
void oracle_softmax(float* x, int size)
{
    float m = x[0];
    for (int i = 1; i < size; ++i)
        if (x[i] > m) m = x[i];
    if (g_fault == FAULT_SOFTMAX_NO_MAX) m = 0.0f;
    float total = 0.0f;
    for (int i = 0; i < size; ++i) {
        float e = expf(x[i] - m);
        x[i] = e;
        total += e;
    }
    float inv = 1.0f / total;
    for (int i = 0; i < size; ++i) x[i] *= inv;
}

/* ---- attention: src/ops.cpp:1317-1515 (naive branches) --------------- */
static int gqa_kv_head(int qh, int n_head, int n_head_kv)
{
    if (g_fault == FAULT_GQA_MODULO) return qh % n_head_kv;
    return qh / (n_head / n_head_kv);
}

void oracle_attention(float* out, const float* q, const float* k, const float* v,
                      float* key_cache, float* value_cache, float* att,
                      int layer, int pos, int n_head, int n_head_kv, int head_dim,
                      int n_ctx)
{
    const int kv_dim = n_head_kv * head_dim;
    const float scale = (g_fault == FAULT_NO_SCALE)
                            ? 1.0f : 1.0f / sqrtf((float)head_dim);
    /* size_t offsets (the reference uses int, which is equal within its range) */
    const size_t base = (size_t)layer * (size_t)n_ctx * (size_t)kv_dim;

    memcpy(key_cache + base + (size_t)pos * kv_dim, k, sizeof(float) * kv_dim);
    memcpy(value_cache + base + (size_t)pos * kv_dim, v, sizeof(float) * kv_dim);

    const int last = (g_fault == FAULT_SKIP_LAST && pos > 0) ? pos - 1 : pos;
    for (int qh = 0; qh < n_head; ++qh) {
        const float* qrow = q + (size_t)qh * head_dim;
        const int kvh = gqa_kv_head(qh, n_head, n_head_kv);
        for (int p = 0; p <= last; ++p) {
            const float* krow = key_cache + base + (size_t)p * kv_dim + (size_t)kvh * head_dim;
            float dot = 0.0f;
            for (int d = 0; d < head_dim; ++d) dot += qrow[d] * krow[d];
            att[p] = dot * scale;
        }
        oracle_softmax(att, last + 1);
        float* orow = out + (size_t)qh * head_dim;
        for (int d = 0; d < head_dim; ++d) orow[d] = 0.0f;
        for (int p = 0; p <= last; ++p) {
            const float* vrow = value_cache + base + (size_t)p * kv_dim + (size_t)kvh * head_dim;
            const float w = att[p];
            for (int d = 0; d < head_dim; ++d) orow[d] += w * vrow[d];
        }
    }
}

/* ---- fp64 brute force over an already-appended cache ----------------- */
/* out64[n_head*head_dim] = softmax(q.K^T / sqrt(hd)) V in double precision. */
void oracle_attention_f64(double* out64, const float* q, const float* key_cache,
                          const float* value_cache, int layer, int pos, int n_head,
                          int n_head_kv, int head_dim, int n_ctx)
{
    const int kv_dim = n_head_kv * head_dim;
    const size_t base = (size_t)layer * (size_t)n_ctx * (size_t)kv_dim;
    const double scale = 1.0 / sqrt((double)head_dim);
    double* sc = (double*)malloc(sizeof(double) * (size_t)(pos + 1));
    for (int qh = 0; qh < n_head; ++qh) {
        const int kvh = qh / (n_head / n_head_kv);
        double mx = -INFINITY;
        for (int p = 0; p <= pos; ++p) {
            const float* krow = key_cache + base + (size_t)p * kv_dim + (size_t)kvh * head_dim;
            double dot = 0.0;
            for (int d = 0; d < head_dim; ++d)
                dot += (double)q[(size_t)qh * head_dim + d] * (double)krow[d];
            sc[p] = dot * scale;
            if (sc[p] > mx) mx = sc[p];
        }
        double sum = 0.0;
        for (int p = 0; p <= pos; ++p) { sc[p] = exp(sc[p] - mx); sum += sc[p]; }
        for (int d = 0; d < head_dim; ++d) {
            double acc = 0.0;
            for (int p = 0; p <= pos; ++p)
                acc += sc[p] * (double)value_cache[base + (size_t)p * kv_dim + (size_t)kvh * head_dim + d];
            out64[(size_t)qh * head_dim + d] = acc / sum;
        }
    }
    free(sc);
}

/* ---- prompt prefill as the reference runs it: src/generate.cpp:56-59 -- */
/* For t = 0..n_tok-1: rope(q_t, k_t, pos0+t); attention(out_t, ..., pos0+t).
 * q: [n_tok][n_head*hd], k/v: [n_tok][n_head_kv*hd] (raw, not rotated; they
 * are copied so the caller's inputs stay unchanged), out: [n_tok][n_head*hd]. */
void oracle_prefill(float* out, const float* q, const float* k, const float* v,
                    float* key_cache, float* value_cache, int layer, int pos0,
                    int n_tok, int n_head, int n_head_kv, int head_dim, int n_ctx,
                    float freq_base)
{
    const int qd = n_head * head_dim, kd = n_head_kv * head_dim;
    float* qt = (float*)malloc(sizeof(float) * (size_t)qd);
    float* kt = (float*)malloc(sizeof(float) * (size_t)kd);
    float* att = (float*)malloc(sizeof(float) * (size_t)n_ctx);
    for (int t = 0; t < n_tok; ++t) {
        memcpy(qt, q + (size_t)t * qd, sizeof(float) * qd);
        memcpy(kt, k + (size_t)t * kd, sizeof(float) * kd);
        oracle_rope(qt, kt, pos0 + t, head_dim, n_head, n_head_kv, freq_base);
        oracle_attention(out + (size_t)t * qd, qt, kt, v + (size_t)t * kd, key_cache,
                         value_cache, att, layer, pos0 + t, n_head, n_head_kv,
                         head_dim, n_ctx);
    }
    free(att); free(kt); free(qt);
}

/* ---- batched decode on several host threads (CPU baseline) ----------- */
/* A "unit" is one (sequence, layer) decode problem with its own cache
 * slice.  Units are split across threads in contiguous chunks, the pattern
 * of the reference's parallel_for (src/ops.cpp:67-110).  Each unit runs
 * rope + oracle_attention exactly as one forward() layer step does. */
typedef struct {
    int u0, u1;
    float* out; const float* q; const float* k; const float* v;
    float* kc; float* vc;
    const int* pos;          /* per unit */
    size_t unit_cache_stride;/* floats between units' caches */
    int n_head, n_head_kv, head_dim, n_ctx; float freq_base; int rotate;
} decode_job;

static void* decode_worker(void* arg)
{
    decode_job* j = (decode_job*)arg;
    const int qd = j->n_head * j->head_dim, kd = j->n_head_kv * j->head_dim;
    float* qt = (float*)malloc(sizeof(float) * (size_t)qd);
    float* kt = (float*)malloc(sizeof(float) * (size_t)kd);
    float* att = (float*)malloc(sizeof(float) * (size_t)j->n_ctx);
    for (int u = j->u0; u < j->u1; ++u) {
        memcpy(qt, j->q + (size_t)u * qd, sizeof(float) * qd);
        memcpy(kt, j->k + (size_t)u * kd, sizeof(float) * kd);
        if (j->rotate)
            oracle_rope(qt, kt, j->pos[u], j->head_dim, j->n_head, j->n_head_kv, j->freq_base);
        oracle_attention(j->out + (size_t)u * qd, qt, kt, j->v + (size_t)u * kd,
                         j->kc + (size_t)u * j->unit_cache_stride,
                         j->vc + (size_t)u * j->unit_cache_stride, att, 0, j->pos[u],
                         j->n_head, j->n_head_kv, j->head_dim, j->n_ctx);
    }
    free(att); free(kt); free(qt);
    return NULL;
}

int oracle_decode_units_mt(int n_threads, int n_units, float* out, const float* q,
                           const float* k, const float* v, float* key_cache,
                           float* value_cache, size_t unit_cache_stride,
                           const int* pos, int n_head, int n_head_kv, int head_dim,
                           int n_ctx, float freq_base, int rotate)
{
    if (n_threads < 1) n_threads = 1;
    if (n_threads > n_units) n_threads = n_units;
    if (n_threads > 256) n_threads = 256;
    pthread_t tid[256];
    decode_job jobs[256];
    const int chunk = n_units / n_threads;
    for (int t = 0; t < n_threads; ++t) {
        decode_job* j = &jobs[t];
        j->u0 = t * chunk;
        j->u1 = (t == n_threads - 1) ? n_units : (t + 1) * chunk;
        j->out = out; j->q = q; j->k = k; j->v = v; j->kc = key_cache; j->vc = value_cache;
        j->pos = pos; j->unit_cache_stride = unit_cache_stride;
        j->n_head = n_head; j->n_head_kv = n_head_kv; j->head_dim = head_dim;
        j->n_ctx = n_ctx; j->freq_base = freq_base; j->rotate = rotate;
    }
    for (int t = 1; t < n_threads; ++t)
        if (pthread_create(&tid[t], NULL, decode_worker, &jobs[t]) != 0) return -1;
    decode_worker(&jobs[0]);
    for (int t = 1; t < n_threads; ++t) pthread_join(tid[t], NULL);
    return 0;
}


/* ---- weights: src/gguf.h:23-32 (type ids), 56-135 (block layouts) ------ */
enum { T_F32 = 0, T_F16 = 1, T_Q4_0 = 2, T_Q8_0 = 8, T_Q6_K = 14 };

/* src/ops.cpp:119-156: exact widening of an IEEE half (subnormals normalised,
 * NaN made quiet). */
float oracle_fp16_to_f32(uint16_t h)
{
    const uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = ((uint32_t)h >> 10) & 0x1Fu;
    uint32_t m = (uint32_t)h & 0x3FFu;
    uint32_t bits;
    if (e == 0) {
        if (m == 0) {
            bits = sign;
        } else {
            int ex = -14;
            while ((m & 0x400u) == 0) { m <<= 1; --ex; }
            bits = sign | ((uint32_t)(ex + 127) << 23) | ((m & 0x3FFu) << 13);
        }
    } else if (e == 31) {
        bits = sign | 0x7F800000u | (m << 13) | (m ? 0x00400000u : 0u);
    } else {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &bits, sizeof f);
    return f;
}

static uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* One output row of the reference's naive matmul for each type: a single fp32
 * accumulator over the row in the reference's order.  Q8_0 and Q4_0 sum each
 * block of 32 first and add scale * block_sum; Q6_K adds every product
 * d*scale*q*x to the row sum directly. */
static float row_dot(const uint8_t* row, const float* x, int cols, int type)
{
    float sum = 0.0f;
    if (type == T_F32) {
        const float* w = (const float*)row;
        for (int j = 0; j < cols; ++j) sum += w[j] * x[j];
    } else if (type == T_F16) {
        for (int j = 0; j < cols; ++j) sum += oracle_fp16_to_f32(rd16(row + 2 * j)) * x[j];
    } else if (type == T_Q8_0) {
        for (int b = 0; b < cols / 32; ++b) {
            const uint8_t* blk = row + 34 * b;
            const float scale = oracle_fp16_to_f32(rd16(blk));
            const int8_t* qs = (const int8_t*)(blk + 2);
            const float* xb = x + 32 * b;
            float bs = 0.0f;
            for (int j = 0; j < 32; ++j) bs += (float)qs[j] * xb[j];
            sum += scale * bs;
        }
    } else if (type == T_Q4_0) {
        for (int b = 0; b < cols / 32; ++b) {
            const uint8_t* blk = row + 18 * b;
            const float scale = oracle_fp16_to_f32(rd16(blk));
            const uint8_t* qs = blk + 2;
            const float* xb = x + 32 * b;
            float bs = 0.0f;
            for (int j = 0; j < 16; ++j) {
                const int lo = (int)(qs[j] & 0x0F) - 8, hi = (int)(qs[j] >> 4) - 8;
                if (g_fault == FAULT_Q4_NIBBLE_ORDER) {
                    bs += (float)lo * xb[2 * j];
                    bs += (float)hi * xb[2 * j + 1];
                } else {
                    bs += (float)lo * xb[j];
                    bs += (float)hi * xb[j + 16];
                }
            }
            sum += scale * bs;
        }
    } else if (type == T_Q6_K) {
        /* super-block of 256: ql[128] qh[64] scales[16] d (210 bytes) */
        for (int b = 0; b < cols / 256; ++b) {
            const uint8_t* blk = row + 210 * b;
            const uint8_t* ql0 = blk;
            const uint8_t* qh0 = blk + 128;
            const int8_t* sc0 = (const int8_t*)(blk + 192);
            const float d = oracle_fp16_to_f32(rd16(blk + 208));
            const float* xb = x + 256 * b;
            for (int half = 0; half < 2; ++half) {
                const uint8_t* ql = ql0 + 64 * half;
                const uint8_t* qh = qh0 + 32 * half;
                const int8_t* sc = sc0 + 8 * half;
                const float* xh = xb + 128 * half;
                for (int l = 0; l < 32; ++l) {
                    const int is = l / 16;
                    const int s2 = g_fault == FAULT_Q6K_QH_SHIFT ? 4 : 2;
                    const int s4 = g_fault == FAULT_Q6K_QH_SHIFT ? 2 : 4;
                    const int q1 = ((ql[l] & 0x0F) | (((qh[l] >> 0) & 3) << 4)) - 32;
                    const int q2 = ((ql[l + 32] & 0x0F) | (((qh[l] >> s2) & 3) << 4)) - 32;
                    const int q3 = ((ql[l] >> 4) | (((qh[l] >> s4) & 3) << 4)) - 32;
                    const int q4 = ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                    sum += d * (float)sc[is + 0] * (float)q1 * xh[l + 0];
                    sum += d * (float)sc[is + 2] * (float)q2 * xh[l + 32];
                    sum += d * (float)sc[is + 4] * (float)q3 * xh[l + 64];
                    sum += d * (float)sc[is + 6] * (float)q4 * xh[l + 96];
                }
            }
        }
    }
    return sum;
}

/* Bytes of one row of `cols` weights of `type`; 0 for an unknown type. */
long long oracle_row_bytes(int type, int cols)
{
    switch (type) {
    case T_F32: return 4LL * cols;
    case T_F16: return 2LL * cols;
    case T_Q8_0: return 34LL * (cols / 32);
    case T_Q4_0: return 18LL * (cols / 32);
    case T_Q6_K: return 210LL * (cols / 256);
    default: return 0;
    }
}

/* out[rows] = W[rows][cols] . x[cols]; returns -1 for an unknown type. */
int oracle_matmul(float* out, const void* W, const float* x, int rows, int cols, int type)
{
    const long long rb = oracle_row_bytes(type, cols);
    if (rb == 0) return -1;
    for (int i = 0; i < rows; ++i) out[i] = row_dot((const uint8_t*)W + rb * i, x, cols, type);
    return 0;
}

/* src/ops.cpp:1003-1055 naive branch. */
void oracle_rmsnorm(float* out, const float* x, const float* weight, int size, float eps)
{
    float ss = 0.0f;
    for (int i = 0; i < size; ++i) ss += x[i] * x[i];
    const float ms = g_fault == FAULT_RMS_NO_MEAN ? ss : ss / (float)size;
    const float rms = 1.0f / sqrtf(ms + eps);
    for (int i = 0; i < size; ++i) out[i] = x[i] * rms * weight[i];
}

/* src/ops.cpp:1165-1184 naive branch. */
void oracle_vec_add(float* out, const float* x, int size)
{
    for (int i = 0; i < size; ++i) out[i] += x[i];
}

/* ---- FFN: src/ops.cpp:1107-1148 and 1535-1564 ------------------------- */

/* silu(x) = x * (1 / (1 + exp(-x))), in place (src/ops.cpp:1107-1115). */
void oracle_silu(float* x, int size)
{
    for (int i = 0; i < size; ++i) {
        const float val = x[i];
        const float e = g_fault == FAULT_SILU_SIGN ? expf(val) : expf(-val);
        const float sigmoid = 1.0f / (1.0f + e);
        x[i] = val * sigmoid;
    }
}

/* a[i] *= b[i] (src/ops.cpp:1128-1148 naive branch). */
void oracle_elementwise_mul(float* a, const float* b, int size)
{
    for (int i = 0; i < size; ++i) a[i] *= b[i];
}

/* out = W_down . (silu(W_gate . in) * (W_up . in)); hb and hb2 are left as
 * the reference leaves them (gated gate projection, up projection). */
int oracle_ffn_swiglu(float* out, const float* in, float* hb, float* hb2, const void* w_gate,
                      const void* w_up, const void* w_down, int n_ff, int n_embd, int type)
{
    if (oracle_matmul(hb, w_gate, in, n_ff, n_embd, type) ||
        oracle_matmul(hb2, w_up, in, n_ff, n_embd, type))
        return -1;
    if (g_fault == FAULT_FFN_SWAP) {
        oracle_silu(hb2, n_ff);
    } else {
        oracle_silu(hb, n_ff);
    }
    oracle_elementwise_mul(hb, hb2, n_ff);
    return oracle_matmul(out, w_down, hb, n_embd, n_ff, type);
}

/* ---- embed_token: src/forward.cpp:17-134 ------------------------------ */
/* Row `token` of the embedding table, dequantised element by element with
 * the reference's expressions (value * scale; Q6_K d * scale * q). */
int oracle_embed(float* out, const void* table, int token, int n_embd, int type)
{
    const long long rb = oracle_row_bytes(type, n_embd);
    if (rb == 0) return -1;
    const uint8_t* row = (const uint8_t*)table + rb * (long long)token;
    if (type == T_F32) {
        memcpy(out, row, sizeof(float) * (size_t)n_embd);
    } else if (type == T_F16) {
        for (int i = 0; i < n_embd; ++i) out[i] = oracle_fp16_to_f32(rd16(row + 2 * i));
    } else if (type == T_Q8_0) {
        for (int b = 0; b < n_embd / 32; ++b) {
            const uint8_t* blk = row + 34 * b;
            const float scale = oracle_fp16_to_f32(rd16(blk));
            for (int j = 0; j < 32; ++j) out[32 * b + j] = (float)(int8_t)blk[2 + j] * scale;
        }
    } else if (type == T_Q4_0) {
        for (int b = 0; b < n_embd / 32; ++b) {
            const uint8_t* blk = row + 18 * b;
            const float scale = oracle_fp16_to_f32(rd16(blk));
            for (int j = 0; j < 16; ++j) {
                const int v0 = (int)(blk[2 + j] & 0x0F) - 8, v1 = (int)(blk[2 + j] >> 4) - 8;
                out[32 * b + j] = (float)v0 * scale;
                out[32 * b + j + 16] = (float)v1 * scale;
            }
        }
    } else { /* T_Q6_K */
        for (int b = 0; b < n_embd / 256; ++b) {
            const uint8_t* blk = row + 210 * b;
            const float d = oracle_fp16_to_f32(rd16(blk + 208));
            for (int half = 0; half < 2; ++half) {
                const uint8_t* ql = blk + 64 * half;
                const uint8_t* qh = blk + 128 + 32 * half;
                const int8_t* sc = (const int8_t*)(blk + 192) + 8 * half;
                float* o = out + 256 * b + 128 * half;
                for (int l = 0; l < 32; ++l) {
                    const int is = l / 16;
                    const int q1 = ((ql[l] & 0x0F) | (((qh[l] >> 0) & 3) << 4)) - 32;
                    const int q2 = ((ql[l + 32] & 0x0F) | (((qh[l] >> 2) & 3) << 4)) - 32;
                    const int q3 = ((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                    const int q4 = ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                    o[l + 0] = d * (float)sc[is + 0] * (float)q1;
                    o[l + 32] = d * (float)sc[is + 2] * (float)q2;
                    o[l + 64] = d * (float)sc[is + 4] * (float)q3;
                    o[l + 96] = d * (float)sc[is + 6] * (float)q4;
                }
            }
        }
    }
    return 0;
}

/* ---- sample_argmax: src/ops.cpp:1587-1597 ----------------------------- */
int oracle_argmax(const float* logits, int n_vocab)
{
    int best = 0;
    float best_val = logits[0];
    for (int i = 1; i < n_vocab; ++i)
        if (logits[i] > best_val) {
            best_val = logits[i];
            best = i;
        }
    return best;
}

/* ---- forward: src/forward.cpp:167-266 --------------------------------- */
typedef struct oracle_layer {
    const float* attn_norm;
    const void *wq, *wk, *wv, *wo;
    int type_q, type_k, type_v, type_o;
    const float* ffn_norm;
    const void *w_gate, *w_up, *w_down;
    int type_ffn;
} oracle_layer;

typedef struct oracle_model {
    int n_layers, n_embd, n_head, n_head_kv, n_ff, n_vocab, n_ctx;
    float rope_freq_base, rms_norm_eps;
    const void* token_embd;
    int type_embd;
    const float* output_norm;
    const void* output; /* the classifier; token_embd when the file has none */
    int type_output;
    const oracle_layer* layers;
} oracle_model;

/* One token at position pos: state.x ... state.logits as forward() computes
 * them.  key_cache/value_cache: [n_layers][n_ctx][kv_dim]; scratch holds at
 * least 5*n_embd + 2*kv_dim + n_ctx + 2*n_ff floats. */
int oracle_forward(const oracle_model* m, float* key_cache, float* value_cache, float* scratch,
                   int token, int pos, float* logits)
{
    const int n_embd = m->n_embd, kv_dim = m->n_head_kv * (m->n_embd / m->n_head);
    const int head_dim = m->n_embd / m->n_head;
    float* x = scratch;
    float* xb = x + n_embd;
    float* xb2 = xb + n_embd;
    float* q = xb2 + n_embd;
    float* k = q + n_embd;
    float* v = k + kv_dim;
    float* att = v + kv_dim;
    float* hb = att + m->n_ctx;
    float* hb2 = hb + m->n_ff;
    if (oracle_embed(x, m->token_embd, token, n_embd, m->type_embd)) return -1;
    for (int l = 0; l < m->n_layers; ++l) {
        const oracle_layer* L = &m->layers[l];
        oracle_rmsnorm(xb, x, L->attn_norm, n_embd, m->rms_norm_eps);
        if (oracle_matmul(q, L->wq, xb, n_embd, n_embd, L->type_q) ||
            oracle_matmul(k, L->wk, xb, kv_dim, n_embd, L->type_k) ||
            oracle_matmul(v, L->wv, xb, kv_dim, n_embd, L->type_v))
            return -1;
        oracle_rope(q, k, pos, head_dim, m->n_head, m->n_head_kv, m->rope_freq_base);
        oracle_attention(xb2, q, k, v, key_cache, value_cache, att, l, pos, m->n_head,
                         m->n_head_kv, head_dim, m->n_ctx);
        if (oracle_matmul(xb, L->wo, xb2, n_embd, n_embd, L->type_o)) return -1;
        if (g_fault == FAULT_FWD_NO_RESIDUAL)
            memcpy(x, xb, sizeof(float) * (size_t)n_embd);
        else
            oracle_vec_add(x, xb, n_embd);
        oracle_rmsnorm(xb, x, L->ffn_norm, n_embd, m->rms_norm_eps);
        if (oracle_ffn_swiglu(xb2, xb, hb, hb2, L->w_gate, L->w_up, L->w_down, m->n_ff, n_embd,
                              L->type_ffn))
            return -1;
        oracle_vec_add(x, xb2, n_embd);
    }
    oracle_rmsnorm(x, x, m->output_norm, n_embd, m->rms_norm_eps);
    return oracle_matmul(logits, m->output, x, m->n_vocab, n_embd, m->type_output);
}
