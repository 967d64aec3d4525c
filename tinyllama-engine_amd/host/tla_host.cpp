// C++20 host side over the C ABI; see tla_host.h for the reference mapping.
#include "tla_host.h"

#include <cstring>
#include <memory>
#include <mutex>
#include <new>

#include "run_state.h"

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

namespace {

std::mutex g_engines_mu;
Engine* g_engine = nullptr;          // set by use_engine
std::vector<Engine*> g_own_engines;  // made by engine_for; kept until the process ends

bool same_shape(const Config& a, const Config& b)
{
    return a.n_layers == b.n_layers && a.n_embd == b.n_embd && a.n_head == b.n_head &&
           a.n_head_kv == b.n_head_kv && a.n_ctx == b.n_ctx && a.rope_freq_base == b.rope_freq_base;
}

}  // namespace

void use_engine(Engine* eng)
{
    std::lock_guard<std::mutex> lock(g_engines_mu);
    g_engine = eng;
}

Engine& engine_for(const Config& cfg)
{
    std::lock_guard<std::mutex> lock(g_engines_mu);
    if (g_engine) {
        if (!same_shape(g_engine->config(), cfg))
            throw std::runtime_error("RunState::allocate: the engine set with use_engine has another shape");
        return *g_engine;
    }
    for (Engine* e : g_own_engines)
        if (same_shape(e->config(), cfg)) return *e;
    // Never destroyed: it serves RunStates for the rest of the process.
    g_own_engines.push_back(new Engine(cfg));
    return *g_own_engines.back();
}

namespace detail {

void allocate_state(::RunState& st, const Config& cfg, Engine& eng)
{
    if (!same_shape(eng.config(), cfg))
        throw std::runtime_error("RunState::allocate: engine and config differ in shape");
    st.free_buffers();
    st.engine = &eng;
    st.n_embd = cfg.n_embd;
    st.kv_dim = cfg.n_head_kv * cfg.head_dim();
    st.n_vocab = cfg.n_vocab;
    try {
        st.x = new float[cfg.n_embd]();
        st.xb = new float[cfg.n_embd]();
        void* h = nullptr;  // the two buffers the attention block moves: pinned
        check(tla_host_alloc(eng.get(), sizeof(float) * cfg.n_embd, &h), "output host buffer");
        st.xb2 = static_cast<float*>(h);
        check(tla_host_alloc(eng.get(), sizeof(float) * (cfg.n_embd + 2 * st.kv_dim), &h), "q|k|v host buffer");
        st.qkv_host = static_cast<float*>(h);
        st.q = st.qkv_host;
        st.k = st.q + cfg.n_embd;
        st.v = st.k + st.kv_dim;
        st.att = new float[cfg.n_ctx]();
        st.hb = new float[cfg.n_ff ? cfg.n_ff : 1]();
        st.hb2 = new float[cfg.n_ff ? cfg.n_ff : 1]();
        st.logits = new float[cfg.n_vocab ? cfg.n_vocab : 1]();
        check(tla_kv_cache_alloc(eng.get(), 1, &st.key_cache, &st.value_cache), "KV cache allocation");
        void* p = nullptr;
        check(tla_alloc(eng.get(), sizeof(float) * (cfg.n_embd + 2 * st.kv_dim), &p), "q|k|v staging");
        st.d_qkv = static_cast<float*>(p);
        check(tla_alloc(eng.get(), sizeof(float) * cfg.n_embd, &p), "output staging");
        st.d_out = static_cast<float*>(p);
        if (cfg.n_vocab) {
            check(tla_alloc(eng.get(), sizeof(float) * cfg.n_vocab, &p), "logits");
            st.d_logits = static_cast<float*>(p);
        }
    } catch (...) {
        free_state(st);
        throw;
    }
    st.pos = 0;
}

void free_state(::RunState& st) noexcept
{
    delete[] st.x;
    delete[] st.xb;
    if (st.engine) {
        tla_host_free(st.engine->get(), st.xb2);
        tla_host_free(st.engine->get(), st.qkv_host);
    }
    delete[] st.att;
    delete[] st.hb;
    delete[] st.hb2;
    delete[] st.logits;
    st.x = st.xb = st.xb2 = st.q = st.k = st.v = st.att = st.hb = st.hb2 = st.logits = nullptr;
    st.qkv_host = nullptr;
    if (st.engine) {
        tla_engine* e = st.engine->get();
        if (st.key_cache) tla_free(e, st.key_cache);
        if (st.value_cache) tla_free(e, st.value_cache);
        if (st.d_qkv) tla_free(e, st.d_qkv);
        if (st.d_out) tla_free(e, st.d_out);
        if (st.d_logits) tla_free(e, st.d_logits);
    }
    st.key_cache = st.value_cache = st.d_qkv = st.d_out = st.d_logits = nullptr;
    st.engine = nullptr;
}

}  // namespace detail

void attention_block(::RunState& state, int layer, int pos)
{
    if (!state.engine) throw std::runtime_error("attention_block: RunState not allocated");
    tla_engine* e = state.engine->get();
    // q | k | v (contiguous in qkv_host) up, RoPE + append + attention, the
    // output down into xb2: one queue, one synchronization
    check(tla_rope_attention_host(e, state.xb2, state.qkv_host, state.d_qkv, state.d_out, state.key_cache,
                                  state.value_cache, layer, pos),
          "attention block");
}

void matmul(Engine& eng, float* out, const void* w, const float* x, int rows, int cols, int type)
{
    check(tla_matmul(eng.get(), out, w, x, rows, cols, type), "matmul");
}

void rmsnorm(Engine& eng, float* out, const float* x, const float* weight, int size, float eps)
{
    check(tla_rmsnorm(eng.get(), out, x, weight, size, eps), "rmsnorm");
}

void vec_add(Engine& eng, float* out, const float* x, int size)
{
    check(tla_vec_add(eng.get(), out, x, size), "vec_add");
}

void silu(Engine& eng, float* x, int size)
{
    check(tla_silu(eng.get(), x, size), "silu");
}

void elementwise_mul(Engine& eng, float* a, const float* b, int size)
{
    check(tla_elementwise_mul(eng.get(), a, b, size), "elementwise_mul");
}

void ffn_swiglu(Engine& eng, float* out, const float* input, float* hb, float* hb2,
                const void* w_gate, const void* w_up, const void* w_down, int n_ff, int n_embd,
                int type)
{
    check(tla_ffn_swiglu(eng.get(), out, input, hb, hb2, w_gate, w_up, w_down, n_ff, n_embd, type),
          "ffn_swiglu");
}

const void* DeviceModel::upload(const TensorRef& t)
{
    void* p = nullptr;
    check(tla_alloc(engine.get(), t.bytes, &p), "weight allocation");
    buffers_.push_back(p);
    check(tla_memcpy_h2d(engine.get(), p, t.data, t.bytes), "weight upload");
    weight_bytes += t.bytes;
    return p;
}

DeviceModel::DeviceModel(Engine& eng, float rms_norm_eps, const Lookup& tensor) : engine(eng)
{
    const Config& cfg = eng.config();
    try {
        const TensorRef embd = tensor("token_embd.weight");
        model.token_embd = upload(embd);
        model.type_embd = embd.type;
        model.output_norm = static_cast<const float*>(upload(tensor("output_norm.weight")));
        TensorRef out{};
        bool tied = false;
        try {
            out = tensor("output.weight");
        } catch (const std::exception&) {
            tied = true;  // tied embeddings (src/forward.cpp:250-258)
        }
        model.output = tied ? model.token_embd : upload(out);
        model.type_output = tied ? embd.type : out.type;
        model.n_ff = static_cast<int>(cfg.n_ff);
        model.n_vocab = static_cast<int>(cfg.n_vocab);
        model.rms_norm_eps = rms_norm_eps;
        layers.resize(cfg.n_layers);
        for (std::uint32_t l = 0; l < cfg.n_layers; ++l) {
            const std::string p = "blk." + std::to_string(l) + ".";
            tla_layer_weights& L = layers[l];
            auto w = [&](const char* name, int* type) {
                const TensorRef t = tensor(p + name);
                if (type) *type = t.type;
                return upload(t);
            };
            L.attn_norm = static_cast<const float*>(w("attn_norm.weight", nullptr));
            L.wq = w("attn_q.weight", &L.type_q);
            L.wk = w("attn_k.weight", &L.type_k);
            L.wv = w("attn_v.weight", &L.type_v);
            L.wo = w("attn_output.weight", &L.type_o);
            L.ffn_norm = static_cast<const float*>(w("ffn_norm.weight", nullptr));
            L.w_gate = w("ffn_gate.weight", &L.type_ffn);  // one type for the FFN, as ffn_swiglu takes
            L.w_up = w("ffn_up.weight", nullptr);
            L.w_down = w("ffn_down.weight", nullptr);
        }
        model.layers = layers.data();
    } catch (...) {
        for (void* b : buffers_) tla_free(engine.get(), b);
        throw;
    }
}

DeviceModel::~DeviceModel()
{
    for (void* b : buffers_) tla_free(engine.get(), b);
}

void forward(DeviceModel& model, ::RunState& state, int token, int pos)
{
    if (!state.engine || !state.d_logits) throw std::runtime_error("forward: RunState not allocated with n_vocab");
    tla_engine* e = state.engine->get();
    check(tla_forward(e, &model.model, state.key_cache, state.value_cache, token, pos, state.d_logits),
          "forward");
    check(tla_memcpy_d2h(e, state.logits, state.d_logits, sizeof(float) * state.n_vocab), "logits download");
}

std::vector<int> generate_greedy(DeviceModel& model, ::RunState& state, const std::vector<int>& prompt,
                                 int n_gen, bool batch_prompt)
{
    if (!state.engine) throw std::runtime_error("generate_greedy: RunState not allocated");
    std::vector<int> out(n_gen > 0 ? n_gen : 0);
    check(tla_generate_greedy(state.engine->get(), &model.model, state.key_cache, state.value_cache,
                              prompt.data(), static_cast<int>(prompt.size()), n_gen, batch_prompt ? TLA_BATCH_PROMPT : 0,
                              out.data()),
          "generate_greedy");
    state.pos = static_cast<int>(prompt.size()) + n_gen - 1;
    return out;
}

}  // namespace tla_host
