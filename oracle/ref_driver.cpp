// extern "C" entry points over the reference engine's own, unmodified ops.cpp
// (compiled where it lies by oracle/Makefile into oracle/_ref/).  TEST
// INFRASTRUCTURE ONLY: used to write golden vectors, to check the C oracle
// live, and as bench.py's "reference" CPU baseline.
//
// Wrapped interfaces:
//   ref_rope       -> rope()       src/ops.h:175-176
//   ref_softmax    -> softmax()    src/ops.h:107
//   ref_attention  -> attention()  src/ops.h:204-206, with a llama_config_t
//                     filled the way src/test_ops.cpp:299-306 fills it
//   ref_decode_units_mt -> rope()+attention() per (sequence, layer) unit, one
//                     std::thread per contiguous chunk of units, the pattern of
//                     parallel_for (src/ops.cpp:67-110).
//   ref_matmul     -> matmul()     src/ops.h:64 (type = ggml_type id)
//   ref_rmsnorm    -> rmsnorm()    src/ops.h:95
//   ref_vec_add    -> vec_add()    src/ops.h:143
//   ref_fp16_to_f32 -> fp16_to_f32() src/ops.h:39
//   ref_silu       -> silu()       src/ops.h:118
//   ref_elementwise_mul -> elementwise_mul() src/ops.h:131
//   ref_ffn_swiglu -> ffn_swiglu() src/ops.h:232-235
//   ref_argmax     -> sample_argmax() src/ops.h:249
#include <cstddef>
#include <cstring>
#include <thread>
#include <vector>

#include "gguf.h"
#include "ops.h"

static llama_config_t make_cfg(int n_layers, int n_head, int n_head_kv, int head_dim, int n_ctx)
{
    llama_config_t cfg;
    cfg.n_layers = static_cast<std::uint32_t>(n_layers);
    cfg.n_head = static_cast<std::uint32_t>(n_head);
    cfg.n_head_kv = static_cast<std::uint32_t>(n_head_kv);
    cfg.n_embd = static_cast<std::uint32_t>(n_head * head_dim);  // head_dim() = n_embd / n_head
    cfg.n_ctx = static_cast<std::uint32_t>(n_ctx);
    return cfg;
}

extern "C" {

void ref_rope(float* q, float* k, int pos, int head_dim, int n_head, int n_head_kv, float freq_base)
{
    rope(q, k, pos, head_dim, n_head, n_head_kv, freq_base);
}

void ref_softmax(float* x, int size) { softmax(x, size); }

void ref_attention(float* out, const float* q, const float* k, const float* v,
                   float* key_cache, float* value_cache, float* att, int layer, int pos,
                   int n_layers, int n_head, int n_head_kv, int head_dim, int n_ctx)
{
    const llama_config_t cfg = make_cfg(n_layers, n_head, n_head_kv, head_dim, n_ctx);
    attention(out, q, k, v, key_cache, value_cache, att, layer, pos, cfg);
}

int ref_decode_units_mt(int n_threads, int n_units, float* out, const float* q,
                        const float* k, const float* v, float* key_cache, float* value_cache,
                        std::size_t unit_cache_stride, const int* pos, int n_head,
                        int n_head_kv, int head_dim, int n_ctx, float freq_base, int rotate)
{
    if (n_threads < 1) n_threads = 1;
    if (n_threads > n_units) n_threads = n_units;
    const llama_config_t cfg = make_cfg(1, n_head, n_head_kv, head_dim, n_ctx);
    const int qd = n_head * head_dim, kd = n_head_kv * head_dim;
    auto work = [&](int u0, int u1) {
        std::vector<float> qt(qd), kt(kd), att(n_ctx);
        for (int u = u0; u < u1; ++u) {
            std::memcpy(qt.data(), q + static_cast<std::size_t>(u) * qd, sizeof(float) * qd);
            std::memcpy(kt.data(), k + static_cast<std::size_t>(u) * kd, sizeof(float) * kd);
            if (rotate) rope(qt.data(), kt.data(), pos[u], head_dim, n_head, n_head_kv, freq_base);
            attention(out + static_cast<std::size_t>(u) * qd, qt.data(), kt.data(),
                      v + static_cast<std::size_t>(u) * kd,
                      key_cache + static_cast<std::size_t>(u) * unit_cache_stride,
                      value_cache + static_cast<std::size_t>(u) * unit_cache_stride, att.data(),
                      0, pos[u], cfg);
        }
    };
    const int chunk = n_units / n_threads;
    std::vector<std::thread> pool;
    for (int t = 0; t + 1 < n_threads; ++t) pool.emplace_back(work, t * chunk, (t + 1) * chunk);
    work((n_threads - 1) * chunk, n_units);
    for (auto& th : pool) th.join();
    return 0;
}

// The prompt fed token by token (src/generate.cpp:56-59) through the
// attention block (src/forward.cpp:192-208): rope() then attention() for
// token t at position pos0 + t, with the same arguments as oracle_prefill.
void ref_prefill(float* out, const float* q, const float* k, const float* v, float* key_cache,
                 float* value_cache, int layer, int pos0, int n_tok, int n_head, int n_head_kv,
                 int head_dim, int n_ctx, float freq_base)
{
    const llama_config_t cfg = make_cfg(layer + 1, n_head, n_head_kv, head_dim, n_ctx);
    const int qd = n_head * head_dim, kd = n_head_kv * head_dim;
    std::vector<float> qt(qd), kt(kd), att(n_ctx);
    for (int t = 0; t < n_tok; ++t) {
        std::memcpy(qt.data(), q + static_cast<std::size_t>(t) * qd, sizeof(float) * qd);
        std::memcpy(kt.data(), k + static_cast<std::size_t>(t) * kd, sizeof(float) * kd);
        rope(qt.data(), kt.data(), pos0 + t, head_dim, n_head, n_head_kv, freq_base);
        attention(out + static_cast<std::size_t>(t) * qd, qt.data(), kt.data(),
                  v + static_cast<std::size_t>(t) * kd, key_cache, value_cache, att.data(), layer,
                  pos0 + t, cfg);
    }
}

void ref_matmul(float* out, const void* W, const float* x, int rows, int cols, int type)
{
    matmul(out, W, x, rows, cols, static_cast<ggml_type>(type));
}

void ref_rmsnorm(float* out, const float* x, const float* weight, int size, float eps)
{
    rmsnorm(out, x, weight, size, eps);
}

void ref_vec_add(float* out, const float* x, int size) { vec_add(out, x, size); }

float ref_fp16_to_f32(unsigned short h) { return fp16_to_f32(h); }


void ref_silu(float* x, int size) { silu(x, size); }

void ref_elementwise_mul(float* a, const float* b, int size) { elementwise_mul(a, b, size); }

void ref_ffn_swiglu(float* out, const float* in, float* hb, float* hb2, const void* w_gate,
                    const void* w_up, const void* w_down, int n_ff, int n_embd, int type)
{
    ffn_swiglu(out, in, hb, hb2, w_gate, w_up, w_down, n_ff, n_embd, static_cast<ggml_type>(type));
}

int ref_argmax(const float* logits, int n_vocab) { return sample_argmax(logits, n_vocab); }

}  // extern "C"
