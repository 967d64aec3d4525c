/*
 * tla_attention.h -- C ABI of the MI355X (gfx950) grouped-query attention
 * path: RoPE, device-resident KV cache with in-kernel RoPE+append,
 * split-KV decode attention and causal MFMA prefill attention.
 *
 * It replaces the attention block of the reference engine's forward pass
 * (src/forward.cpp:192-208) and the helpers it calls:
 *     rope()      src/ops.h:175-176   (src/ops.cpp:1223-1281)
 *     softmax()   src/ops.h:107       (src/ops.cpp:1072-1091)
 *     attention() src/ops.h:204-206   (src/ops.cpp:1317-1515)
 *     RunState key_cache/value_cache  src/run_state.h:93-101, 134-153
 *
 * Conventions
 *   - Every entry point returns int status, TLA_OK (0) on success.  The ABI
 *     never throws.  tla_last_error() gives a message for the calling
 *     thread's last failure.  (The reference's ops never validate; its
 *     callers throw std::runtime_error -- the C++ wrapper in
 *     tinyllama-engine_amd/host/ turns non-zero codes into exactly that.)
 *   - Pointers named *_dev are device (HBM) pointers; the library never
 *     dereferences them on the host.  All compute entry points are
 *     asynchronous and ordered on the engine's own HIP stream.
 *   - Layout of one KV cache is the reference's: element (layer, pos, kv_head,
 *     j) at ((layer * n_ctx + pos) * n_head_kv + kv_head) * head_dim + j,
 *     fp32.  Several sequences stack with a caller-given seq_stride.
 *   - Kernels implement head_dim == 64 and n_head / n_head_kv <= 16.
 *   - One engine is not re-entrant: calls on one engine from several host
 *     threads must be serialised by the caller.
 */
#ifndef TLA_ATTENTION_H
#define TLA_ATTENTION_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

enum tla_status {
    TLA_OK = 0,
    TLA_ERR_INVALID_ARGUMENT = 1, /* null pointer, bad size, inconsistent shape */
    TLA_ERR_OUT_OF_RANGE = 2,     /* pos >= n_ctx, layer >= n_layers, ...        */
    TLA_ERR_UNSUPPORTED = 3,      /* a shape the kernels do not implement        */
    TLA_ERR_DEVICE = 4,           /* HIP runtime failure                          */
    TLA_ERR_OUT_OF_MEMORY = 5
};

/* Flags for tla_decode / tla_prefill. */
enum tla_flags {
    /* Apply RoPE to q and to the new k (at each token's position) inside the
     * kernel, as forward() does with rope() before attention()
     * (src/forward.cpp:192-206).  Without it q and k are taken as already
     * rotated, which is attention()'s contract (src/ops.h:185-186). */
    TLA_ROTATE = 1,
    /* tla_generate_greedy: run the prompt through the model as one batch
     * (tla_prefill_forward) instead of token by token. */
    TLA_BATCH_PROMPT = 2,
    /* tla_decode: the k and v rows at each token's position are already in
     * the cache (as the step's projection wrote them, rotated); only the
     * attention runs, and k_dev / v_dev are not read (may be NULL).  With
     * TLA_ROTATE, q is still rotated in the kernel. */
    TLA_KV_IN_CACHE = 4
};

/* Shape fields of llama_config_t (src/gguf.h:139-168) that the path uses.
 * head_dim = n_embd / n_head, as llama_config_t::head_dim(). */
typedef struct tla_config {
    int n_layers;
    int n_embd;
    int n_head;
    int n_head_kv;
    int n_ctx;
    float rope_freq_base;
} tla_config;

/* Engine: one device, one HIP stream, the RoPE cos/sin table for
 * positions [0, n_ctx) and a split-KV workspace.  No reference counterpart
 * (the reference keeps no device state); it stands in for the
 * `const llama_config_t& cfg` argument of attention(). */
typedef struct tla_engine tla_engine;

/* Message for the calling thread's last non-zero status ("" if none). */
const char* tla_last_error(void);

/* ABI version: bumped on any signature change. */
int tla_abi_version(void);

int tla_engine_create(const tla_config* cfg, int device, tla_engine** out);
int tla_engine_destroy(tla_engine* e);
/* Wait for all work queued on the engine's stream. */
int tla_synchronize(tla_engine* e);

/* ---- device memory (RunState::allocate / free_buffers,
 *      src/run_state.h:115-170) ---------------------------------------- */
/* Zero-filled device allocation of `bytes` bytes. */
int tla_alloc(tla_engine* e, size_t bytes, void** out_dev);
int tla_free(tla_engine* e, void* dev);
/* KV cache for n_seq sequences, each [n_layers][n_ctx][n_head_kv*head_dim]
 * fp32, zero-filled (src/run_state.h:134-153).  Free with tla_free. */
int tla_kv_cache_alloc(tla_engine* e, int n_seq, float** key_cache_dev,
                       float** value_cache_dev);
/* Blocking copies host<->device and a device copy kernel (device->device,
 * used e.g. to clone a sequence's cache).  Ordered after queued work. */
/* Pinned (page-locked) host memory, zero-filled, for buffers that cross to
 * the device every step (RunState's q|k|v and attention output). */
int tla_host_alloc(tla_engine* e, size_t bytes, void** out_host);
int tla_host_free(tla_engine* e, void* host);
int tla_memcpy_h2d(tla_engine* e, void* dst_dev, const void* src_host, size_t bytes);
int tla_memcpy_d2h(tla_engine* e, void* dst_host, const void* src_dev, size_t bytes);
int tla_memcpy_d2d(tla_engine* e, void* dst_dev, const void* src_dev, size_t bytes);

/* ---- operators ------------------------------------------------------ */

/* rope() src/ops.h:175-176, in place on device q [n_head*head_dim] and
 * k [n_head_kv*head_dim].  Bit-exact with the reference: cos/sin come from
 * the host's libm with the reference's float expressions, and the rotation
 * rounds each product and sum separately.  Any pos >= 0 (no n_ctx limit). */
int tla_rope(tla_engine* e, float* q_dev, float* k_dev, int pos, int head_dim, int n_head,
             int n_head_kv, float freq_base);

/* softmax() src/ops.h:107, in place on device x[size]. */
int tla_softmax(tla_engine* e, float* x_dev, int size);

/* attention() src/ops.h:204-206 for one token of one sequence: appends the
 * (already rotated) k and v at `pos` of `layer`, then writes
 * out[n_head*head_dim] = softmax(q.K^T / sqrt(head_dim)) V over positions
 * 0..pos.  key_cache/value_cache are device caches laid out
 * [n_layers][n_ctx][kv_dim] as RunState's.  `att` is the reference's score
 * scratch; it is not used (pass NULL or anything). */
int tla_attention(tla_engine* e, float* out_dev, const float* q_dev, const float* k_dev,
                  const float* v_dev, float* key_cache_dev, float* value_cache_dev,
                  float* att, int layer, int pos);

/* The whole attention block of forward() (src/forward.cpp:192-208):
 * rope(q, k, pos) then attention(...), fused into one launch sequence.
 * q and k are read unrotated and are left unchanged; the cache receives the
 * rotated k. */
int tla_rope_attention(tla_engine* e, float* out_dev, const float* q_dev, const float* k_dev,
                       const float* v_dev, float* key_cache_dev, float* value_cache_dev,
                       int layer, int pos);

/* The same block for a caller whose q, k, v and output live in host memory,
 * as forward()'s RunState scratch does (src/forward.cpp:192-208 reads
 * state.q/k/v and writes state.xb2): qkv_host holds q [n_head*head_dim],
 * k and v [n_head_kv*head_dim] back to back; they are uploaded to qkv_dev
 * (same layout), the fused RoPE + append + attention runs, the output is
 * downloaded from out_dev to out_host, all queued on the engine's stream
 * with one synchronization at the end.  Pinned host buffers
 * (tla_host_alloc) make the two copies direct transfers. */
int tla_rope_attention_host(tla_engine* e, float* out_host, const float* qkv_host, float* qkv_dev,
                            float* out_dev, float* key_cache_dev, float* value_cache_dev, int layer,
                            int pos);

/* Batched decode: one new token for each of n_seq sequences, for each of the
 * n_step_layers layers layer0 .. layer0+n_step_layers-1.  Equivalent to
 * calling attention() (or rope()+attention() with TLA_ROTATE) once per
 * (sequence, layer) with that sequence's position.
 *   pos_host  [n_seq]                       host array, 0 <= pos < n_ctx
 *   q_dev     [n_seq][n_step_layers][n_head][head_dim]
 *   k/v_dev   [n_seq][n_step_layers][n_head_kv][head_dim]
 *   out_dev   [n_seq][n_step_layers][n_head][head_dim]
 *   caches    sequence s, layer l at key_cache_dev + s*seq_stride
 *             + l*n_ctx*kv_dim (floats); seq_stride >= n_layers*n_ctx*kv_dim
 *             unless n_seq == 1.
 * Ragged lengths are supported.  Up to 256 sequences per call. */
int tla_decode(tla_engine* e, int n_seq, const int* pos_host, int layer0, int n_step_layers,
               int flags, float* out_dev, const float* q_dev, const float* k_dev,
               const float* v_dev, float* key_cache_dev, float* value_cache_dev,
               size_t seq_stride);

/* tla_decode without any allocation: same arguments, same kernels and the
 * same results bit for bit, but the split partials and arrival counters live
 * in a fixed per-device static array (32 MiB of partials, 65,536 counters)
 * instead of the engine's workspace, so the call never allocates device
 * memory (tla_decode grows its workspace with hipMalloc on first use of a
 * larger shape), nor host memory unless profiling is on (below).  No counterpart in the reference: it is for callers that
 * cannot allocate -- code under HIP graph capture, tight serving loops,
 * harnesses that forbid allocation.  A launch whose partials or counters
 * exceed the array returns TLA_ERR_UNSUPPORTED and launches nothing (e.g. 22
 * layers x 2048 positions x 1 sequence needs 2 MB; 8 x 22 x 16384 about 5 MB).
 * The array is shared by every engine on the device and keeps the last
 * call's contents: calls that overlap on one device (other streams, other
 * host threads) race.  The counters are zeroed when the first engine is
 * created on the device, and every launch returns the ones it uses to zero.
 * With profiling on (tla_profile), the call records a pair of HIP events
 * around its launch, and the event pool may grow on the host. */
int tla_decode_noalloc(tla_engine* e, int n_seq, const int* pos_host, int layer0,
                       int n_step_layers, int flags, float* out_dev, const float* q_dev,
                       const float* k_dev, const float* v_dev, float* key_cache_dev,
                       float* value_cache_dev, size_t seq_stride);

/* Causal prefill of n_tok prompt tokens at positions pos0 .. pos0+n_tok-1 of
 * one sequence, for layers layer0 .. layer0+n_step_layers-1.  Equal to the
 * reference's token-by-token prompt loop (src/generate.cpp:56-59) over the
 * attention block: every token's k,v are appended to the cache and token t
 * attends to positions 0 .. pos0+t.  With TLA_ROTATE, q and k are rotated in
 * the kernel at their own positions.
 *   q_dev/out_dev [n_step_layers][n_tok][n_head][head_dim]
 *   k/v_dev       [n_step_layers][n_tok][n_head_kv][head_dim]
 * Engine memory it keeps for later calls: the keys and values of positions
 * 0 .. pos0+n_tok-1 as bf16 planes, n_step_layers x n_head_kv x
 * ceil((pos0 + n_tok) / 32) x 24 KiB, grown (after a stream synchronize) when
 * a call needs more. */
int tla_prefill(tla_engine* e, int pos0, int n_tok, int layer0, int n_step_layers, int flags,
                float* out_dev, const float* q_dev, const float* k_dev, const float* v_dev,
                float* key_cache_dev, float* value_cache_dev);

/* ---- projections either side of the attention block ------------------ */

/* Weight formats: the reference's ggml_type ids (src/gguf.h:23-32) and block
 * layouts (src/gguf.h:56-135).  Weights are row-major [rows][cols] in the
 * GGUF byte layout, on the device, 16-byte aligned. */
enum tla_weight_type {
    TLA_W_F32 = 0,
    TLA_W_F16 = 1,
    TLA_W_Q4_0 = 2,
    TLA_W_Q8_0 = 8,
    TLA_W_Q6_K = 14
};

/* matmul() src/ops.h:64-66: out[rows] = W[rows][cols] . x[cols], device
 * pointers.  cols must be a multiple of 64 (of 256 for Q6_K) and at most
 * 13632 (x is staged in 60 KiB of LDS); other shapes return
 * TLA_ERR_UNSUPPORTED.  fp32 accumulation; equal
 * to the reference to fp32 rounding (the sums are grouped differently). */
int tla_matmul(tla_engine* e, float* out_dev, const void* w_dev, const float* x_dev, int rows,
               int cols, int type);

/* matmul() over a batch of n_tok vectors: out[t][rows] = W . x[t] (x
 * [n_tok][cols]).  3-64 vectors (F32, F16, Q8_0, Q4_0; F16 and F32 from
 * 2) run as one product that dequantises the weights in registers on the
 * fp32 matrix cores; from 65 vectors on (Q6_K from 16) as the split product:
 * x split into three bf16 pieces (an engine workspace of 6 bytes per
 * element, tokens padded to 64), weights dequantised in registers into exact
 * bf16 pieces, every product of pieces exact in the fp32 accumulator of the
 * bf16 matrix cores (K cut into ranges for small grids, their sums added in
 * order from a second workspace); fewer vectors (Q6_K: under 16) run as
 * groups of matrix-vector products.  fp32 accumulation throughout: equal to
 * the reference to fp32 rounding.  Used for the prompt's projections. */
int tla_matmul_batch(tla_engine* e, float* out_dev, const void* w_dev, const float* x_dev, int rows,
                     int cols, int n_tok, int type);

/* rmsnorm() src/ops.h:95-96: out = x / sqrt(mean(x^2) + eps) * weight. */
int tla_rmsnorm(tla_engine* e, float* out_dev, const float* x_dev, const float* weight_dev,
                int size, float eps);

/* vec_add() src/ops.h:143: out[i] += x[i]. */
int tla_vec_add(tla_engine* e, float* out_dev, const float* x_dev, int size);

/* The input half of the attention block for n_seq sequences
 * (src/forward.cpp:180-190): xb = rmsnorm(x, norm_w, eps) (skipped when
 * norm_w is NULL), q = Wq.xb, k = Wk.xb, v = Wv.xb, in one launch per 8
 * sequences (fewer when 8 x n_embd floats exceed 60 KiB).  x, q [n_seq][n_embd];
 * k, v [n_seq][kv_dim]; Wq [n_embd][n_embd],
 * Wk, Wv [kv_dim][n_embd], all of one type.  q and k leave unrotated, ready
 * for tla_decode with TLA_ROTATE (RoPE and the cache append are its
 * prologue). */
int tla_attn_qkv(tla_engine* e, int n_seq, float* q_dev, float* k_dev, float* v_dev,
                 const float* x_dev, const float* norm_w_dev, float eps, const void* wq_dev,
                 const void* wk_dev, const void* wv_dev, int type);

/* The output half (src/forward.cpp:210-213): x += Wo . xb2 for n_seq
 * sequences, x and xb2 [n_seq][n_embd], Wo [n_embd][n_embd]. */
int tla_attn_out(tla_engine* e, int n_seq, float* x_dev, const void* wo_dev,
                 const float* xb2_dev, int type);

/* ---- the rest of a layer, and the whole forward pass ------------------ */

/* silu() src/ops.h:118: x = x * (1 / (1 + exp(-x))) in place. */
int tla_silu(tla_engine* e, float* x_dev, int size);

/* elementwise_mul() src/ops.h:131: a[i] *= b[i]. */
int tla_elementwise_mul(tla_engine* e, float* a_dev, const float* b_dev, int size);

/* ffn_swiglu() src/ops.h:232-235: out = W_down . (silu(W_gate . in) *
 * (W_up . in)).  hb, hb2 [n_ff] are left as the reference leaves them (the
 * gated projection, the up projection).  W_gate, W_up [n_ff][n_embd],
 * W_down [n_embd][n_ff], all of one type (the reference passes one type). */
int tla_ffn_swiglu(tla_engine* e, float* out_dev, const float* in_dev, float* hb_dev,
                   float* hb2_dev, const void* w_gate_dev, const void* w_up_dev,
                   const void* w_down_dev, int n_ff, int n_embd, int type);

/* The FFN half of a layer (src/forward.cpp:215-228) for n_seq sequences:
 * x += ffn_swiglu(rmsnorm(x, norm_w, eps)), in two launches (rmsnorm + gate
 * and up projections; SiLU, gating, down projection and the residual add).
 * x [n_seq][n_embd]; hb_dev scratch [n_seq][2][n_ff] receives the raw gate
 * and up projections, except for one sequence of Q8_0 / Q4_0 / Q6_K weights
 * (n_embd <= 4096, n_ff even): then the gate half receives SiLU(gate) x up,
 * formed in the first launch, and the up half is unspecified. */
int tla_ffn_block(tla_engine* e, int n_seq, float* x_dev, const float* norm_w_dev, float eps,
                  const void* w_gate_dev, const void* w_up_dev, const void* w_down_dev, int n_ff,
                  int type, float* hb_dev);

/* embed_token() src/forward.cpp:17-134: out = row `token` of the embedding
 * table [n_vocab][n_embd] (any of the five types), dequantised with the
 * reference's expressions (bit-exact).  A token outside [0, n_vocab) is
 * TLA_ERR_OUT_OF_RANGE and launches nothing (the reference's embed_token()
 * does not check; its table's row count comes from the GGUF tensor shape). */
int tla_embed(tla_engine* e, float* out_dev, const void* table_dev, int token, int n_embd,
              int n_vocab, int type);

/* sample_argmax() src/ops.h:249: the first index of the largest logit. */
int tla_argmax(tla_engine* e, const float* logits_dev, int n_vocab, int* token_host);

/* matmul() then sample_argmax() (src/ops.cpp:959-983, 1587-1597), the last
 * two steps of a greedy decode step (src/generate.cpp:84-90): out = W . x
 * as tla_matmul (rows of at most 4096 columns), and *token_host = the first
 * index of the largest out, from argmax keys each workgroup of the product
 * posts with one atomic (a NaN never wins, except at index 0; -0 ties with
 * +0), read by a one-wave launch.  tla_generate_greedy takes every token
 * after its first this way. */
int tla_matmul_argmax(tla_engine* e, float* out_dev, const void* w_dev, const float* x_dev, int rows,
                      int cols, int type, int* token_host);

/* The weights forward() reads from the GGUF file (src/forward.cpp:167-266),
 * as device pointers to the tensors' unchanged bytes (16-byte aligned) and
 * their ggml_type ids.  `output` is token_embd when the file has no
 * output.weight (tied embeddings, src/forward.cpp:250-258). */
typedef struct tla_layer_weights {
    const float* attn_norm;            /* [n_embd] F32 */
    const void *wq, *wk, *wv, *wo;
    int type_q, type_k, type_v, type_o;
    const float* ffn_norm;             /* [n_embd] F32 */
    const void *w_gate, *w_up, *w_down;
    int type_ffn;                      /* one type for the three, as ffn_swiglu takes */
} tla_layer_weights;

typedef struct tla_model {
    int n_ff, n_vocab;
    float rms_norm_eps;
    const void* token_embd;
    int type_embd;
    const float* output_norm;          /* [n_embd] F32 */
    const void* output;
    int type_output;
    const tla_layer_weights* layers;   /* host array [cfg.n_layers] */
} tla_model;

/* forward() src/forward.cpp:167-266 for one token at position pos: the
 * embedding, every layer (rmsnorm + Q/K/V, RoPE + append + attention, W_o +
 * residual, rmsnorm + SwiGLU FFN + residual) and the classifier, on the
 * device: logits_dev [n_vocab].  Caches as from tla_kv_cache_alloc (one
 * sequence); the residual stream and scratch are the engine's.  4 launches
 * per layer + 2 where the layer's Q/K/V launch can rotate and append (one
 * weight type for the three, n_embd <= 2048), pos < 192, n_head_kv <= 4,
 * n_head / n_head_kv <= 8 (a multiple of 4 for a Q6_K W_o) and n_ff <=
 * 8192: attention and W_o are then one
 * launch whose workgroups each recompute one kv head's attention and write
 * W_o's partial products for that head's columns, which the FFN launches
 * add to the residual; else 5 per layer + 2. */
int tla_forward(tla_engine* e, const tla_model* m, float* key_cache_dev, float* value_cache_dev,
                int token, int pos, float* logits_dev);

/* The prompt loop of src/generate.cpp:56-59 as one batch: forward() for
 * tokens_host[0..n_tok) at positions pos0..pos0+n_tok-1, each layer over all
 * tokens at once (the projections as tla_matmul_batch products, the causal
 * MFMA prefill attention with RoPE + append in-kernel); logits_dev
 * [n_vocab] receives the last
 * token's logits (the ones generate() samples from).  The KV cache ends as
 * after n_tok forward() calls (to fp32 rounding: the attention sums are
 * grouped differently).  Engine memory it keeps for later calls: the split
 * product's workspaces, for prompts past 64 tokens (or with a Q6_K layer
 * matrix past 15): 6 bytes per token (padded to 64) and column of the
 * widest product input (TinyLlama, 512 tokens: 17 MB), and partial sums of
 * at most a few MB. */
int tla_prefill_forward(tla_engine* e, const tla_model* m, float* key_cache_dev,
                        float* value_cache_dev, const int* tokens_host, int n_tok, int pos0,
                        float* logits_dev);

/* The generation loop with greedy sampling (src/generate.cpp:56-100 at
 * temperature 0, without the tokenizer): forward() over the prompt at
 * positions 0..n_prompt-1 (token by token, or as one batch with
 * TLA_BATCH_PROMPT), then n_gen tokens each from the argmax of the
 * previous logits: the first by an argmax launch, the later ones (n_embd
 * <= 4096) from the argmax keys the classifier's workgroups post, as
 * tla_matmul_argmax, read by the next step's embedding launch (engine
 * memory: 512 bytes per generated token).  The sampled token stays on the
 * device between steps, so every launch is queued without waiting;
 * tokens_host [n_gen] is written at the end.  The caller stops at its EOS token, as the reference
 * does (tokens after it are computed but not used).  Needs n_prompt >= 1
 * and n_prompt + n_gen - 1 <= n_ctx. */
int tla_generate_greedy(tla_engine* e, const tla_model* m, float* key_cache_dev,
                        float* value_cache_dev, const int* prompt_host, int n_prompt, int n_gen,
                        int flags, int* tokens_host);

/* ---- measurement hooks (no reference counterpart) ------------------- */
enum tla_kernel_id {
    TLA_KERNEL_DECODE = 0,  /* split-KV decode attention (and forward()'s
                               short-context attention + W_o): RoPE + append +
                               attention + split merge, one launch           */
    TLA_KERNEL_PREFILL = 1, /* causal MFMA prefill attention                 */
    TLA_KERNEL_APPEND = 2,  /* prefill RoPE + cache append                   */
    TLA_KERNEL_GEMV = 3,    /* projections: matmul / attn_qkv / attn_out /
                               ffn / classifier                              */
    TLA_KERNEL_COUNT = 4
};
/* When enabled, HIP events bracket every launch of each kernel on the
 * engine's stream; tla_profile_read sums their durations (ms) since the
 * last reset.  Enabling or disabling resets the sums. */
int tla_profile_enable(tla_engine* e, int enable);
int tla_profile_read(tla_engine* e, int kernel_id, double* total_ms, long long* launches);

/* Stream-ordered HIP events for timing whole steps: record into one of 64
 * slots, then read the elapsed time between two recorded slots. */
int tla_event_record(tla_engine* e, int slot);
int tla_event_elapsed(tla_engine* e, int slot_begin, int slot_end, float* ms);

/* Streaming-read floor: read `bytes` at src_dev (16-byte aligned, a multiple
 * of 16) with n_workgroups workgroups of 256 threads, each summing one
 * contiguous chunk with `depth` (8, 16 or 32) 16-byte loads in flight per
 * thread, in the load form `load_kind` (below), on the engine's stream;
 * sink_dev [n_workgroups] floats is never written in practice (the sums are
 * kept only so the loads stay).  The buffer forms need chunks under 2 GiB.
 * What one launch can read from HBM in the time it takes -- the bar the
 * decode kernel's byte rate is set against.  No reference counterpart. */
enum tla_read_kind {
    TLA_READ_GLOBAL = 0,       /* global_load_dwordx4 */
    TLA_READ_GLOBAL_NT = 1,    /* the same, non-temporal */
    TLA_READ_BUFFER = 2,       /* buffer_load_dwordx4, loads past the chunk return zeros */
    TLA_READ_BUFFER_NT = 3     /* the same, non-temporal */
};
int tla_read_floor(tla_engine* e, const void* src_dev, size_t bytes, int n_workgroups, int load_kind,
                   int depth, float* sink_dev);

/* MFMA floor: n_workgroups workgroups of 4 waves on the engine's stream,
 * each wave `iters` rounds of 16 v_mfma_f32_32x32x16_bf16 (2 x 32 x 32 x 16
 * flops each) on two independent accumulators with operands that change from
 * lane to lane; sink_dev [n_workgroups] floats is never written in practice.
 * What one launch can execute of bf16 MFMA work in the time it takes -- the
 * bar the prefill attention kernel's products are set against.  No
 * reference counterpart. */
int tla_mfma_floor(tla_engine* e, int n_workgroups, int iters, float* sink_dev);

/* Tuning knobs (0 = automatic). */
enum tla_option {
    TLA_OPT_DECODE_SPLIT = 0, /* positions per decode workgroup (rounded up to 16) */
    TLA_OPT_DECODE_PLAN = 1,  /* 1: one split length per sequence; 2: equal ranges across
                                 sequences and layers */
    TLA_OPT_DECODE_GROUP = 2, /* kv heads per decode workgroup in the plan of one split
                                 length: 1, 2 or 4 (the other plan always takes 4);
                                 results do not depend on it */
    TLA_OPT_STREAM_TILES = 3, /* batched products of 2-64 vectors: vectors per
                                 workgroup in tiles of 16, 1 to 4; results do not
                                 depend on it */
    TLA_OPT_SPLIT_ROWS = 4,   /* batched products past 64 vectors (Q6_K: from 16):
                                 16-row subtiles per wave, 1, 2 or 4 (0: per
                                 shape); results do not depend on it */
    TLA_OPT_SPLIT_K = 5       /* the same products: ranges K is cut into, 1 to 64
                                 (0: per shape; at most one per 32-column block);
                                 results change by fp32 rounding only */
};
enum tla_decode_plan { TLA_PLAN_AUTO = 0, TLA_PLAN_ALIGNED = 1, TLA_PLAN_BALANCED = 2 };
int tla_set_option(tla_engine* e, int option, long long value);

#ifdef __cplusplus
}  /* extern "C" */
#endif

#endif /* TLA_ATTENTION_H */
