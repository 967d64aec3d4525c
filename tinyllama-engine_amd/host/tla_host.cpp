// C++20 host side over the C ABI; see tla_host.h for the reference mapping.
#include "tla_host.h"

#include <cstring>
#include <new>

namespace tla_host {

void check(int status, const char* what)
{
    if (status != TLA_OK) throw std::runtime_error(std::string(what) + ": " + tla_last_error());
}

tla_config Config::to_c() const
{
    tla_config c{};
    c.n_layers = static_cast<int>(n_layers);
    c.n_embd = static_cast<int>(n_embd);
    c.n_head = static_cast<int>(n_head);
    c.n_head_kv = static_cast<int>(n_head_kv);
    c.n_ctx = static_cast<int>(n_ctx);
    c.rope_freq_base = rope_freq_base;
    return c;
}

Engine::Engine(const Config& cfg, int device) : cfg_(cfg)
{
    const tla_config c = cfg.to_c();
    check(tla_engine_create(&c, device, &e_), "tla_engine_create");
}

Engine::~Engine()
{
    tla_engine_destroy(e_);
}

void Engine::synchronize()
{
    check(tla_synchronize(e_), "tla_synchronize");
}

void rope(Engine& eng, float* q, float* k, int pos, int head_dim, int n_head, int n_head_kv,
          float freq_base)
{
    check(tla_rope(eng.get(), q, k, pos, head_dim, n_head, n_head_kv, freq_base), "rope");
}

void softmax(Engine& eng, float* x, int size)
{
    check(tla_softmax(eng.get(), x, size), "softmax");
}

void attention(Engine& eng, float* out, const float* q, const float* k, const float* v,
               float* key_cache, float* value_cache, float* att, int layer, int pos)
{
    check(tla_attention(eng.get(), out, q, k, v, key_cache, value_cache, att, layer, pos),
          "attention");
}

void RunState::allocate(const Config& cfg, Engine& eng)
{
    free_buffers();
    engine = &eng;
    n_embd_ = cfg.n_embd;
    kv_dim_ = cfg.n_head_kv * cfg.head_dim();

    x = new float[cfg.n_embd]();
    xb = new float[cfg.n_embd]();
    xb2 = new float[cfg.n_embd]();
    qkv_host_ = new float[cfg.n_embd + 2 * kv_dim_]();
    q = qkv_host_;
    k = q + cfg.n_embd;
    v = k + kv_dim_;
    att = new float[cfg.n_ctx]();
    hb = new float[cfg.n_ff ? cfg.n_ff : 1]();
    hb2 = new float[cfg.n_ff ? cfg.n_ff : 1]();
    logits = new float[cfg.n_vocab ? cfg.n_vocab : 1]();

    check(tla_kv_cache_alloc(eng.get(), 1, &key_cache, &value_cache), "KV cache allocation");
    void* p = nullptr;
    check(tla_alloc(eng.get(), sizeof(float) * (cfg.n_embd + 2 * kv_dim_), &p), "q|k|v staging");
    d_qkv = static_cast<float*>(p);
    check(tla_alloc(eng.get(), sizeof(float) * cfg.n_embd, &p), "output staging");
    d_out = static_cast<float*>(p);
    pos = 0;
}

void RunState::free_buffers()
{
    delete[] x;
    delete[] xb;
    delete[] xb2;
    delete[] qkv_host_;
    delete[] att;
    delete[] hb;
    delete[] hb2;
    delete[] logits;
    x = xb = xb2 = q = k = v = att = hb = hb2 = logits = nullptr;
    qkv_host_ = nullptr;
    if (engine) {
        tla_free(engine->get(), key_cache);
        tla_free(engine->get(), value_cache);
        tla_free(engine->get(), d_qkv);
        tla_free(engine->get(), d_out);
    }
    key_cache = value_cache = d_qkv = d_out = nullptr;
    engine = nullptr;
}

void attention_block(RunState& state, int layer, int pos)
{
    if (!state.engine) throw std::runtime_error("attention_block: RunState not allocated");
    tla_engine* e = state.engine->get();
    const std::size_t n = state.n_embd_ + 2 * static_cast<std::size_t>(state.kv_dim_);
    check(tla_memcpy_h2d(e, state.d_qkv, state.q, sizeof(float) * n), "q|k|v upload");
    const float* dq = state.d_qkv;
    const float* dk = dq + state.n_embd_;
    const float* dv = dk + state.kv_dim_;
    check(tla_rope_attention(e, state.d_out, dq, dk, dv, state.key_cache, state.value_cache, layer,
                             pos),
          "rope+attention");
    check(tla_memcpy_d2h(e, state.xb2, state.d_out, sizeof(float) * state.n_embd_),
          "attention output download");
}

}  // namespace tla_host
