// C++20 host side of the MI355X attention path, shaped like the reference
// engine's own interfaces so that its forward() can switch with a few edits.
//
//   tla_host::check            -> the reference's error convention: a failed
//                                 operation throws std::runtime_error, caught
//                                 by main (src/main.cpp:180-183)
//   tla_host::Config           -> llama_config_t fields used by the path
//                                 (src/gguf.h:139-168)
//   tla_host::rope / softmax / attention
//                              -> rope() src/ops.h:175-176, softmax()
//                                 src/ops.h:107, attention() src/ops.h:204-206,
//                                 same argument order, device pointers, plus
//                                 the engine that replaces `cfg`
//   ::RunState (run_state.h)   -> struct RunState (src/run_state.h:27-182),
//                                 a drop-in for that header: the same global
//                                 struct, members and lifecycle; key_cache and
//                                 value_cache hold DEVICE pointers; device
//                                 staging for the attention block is appended
//                                 after the reference's members
//   tla_host::attention_block  -> the block of forward() at
//                                 src/forward.cpp:192-208 (rope + attention)
//   tla_host::matmul / rmsnorm / vec_add / silu / elementwise_mul / ffn_swiglu
//                              -> the ops of src/ops.h:64-66, 95-96, 118,
//                                 131, 143, 232-235 (device pointers)
//   tla_host::DeviceModel      -> the weights forward() reads from the GGUF
//                                 file (src/forward.cpp:167-266), copied to
//                                 the device unchanged
//   tla_host::forward          -> forward(GGUFModel&, RunState&, token, pos)
//                                 (src/forward.h): the whole pass on the
//                                 device, logits into state.logits
//   tla_host::generate_greedy  -> the generation loop of src/generate.cpp:56-100
//                                 at temperature 0 (tokens, not text)
#pragma once

#include <cstddef>
#include <cstdint>
#include <functional>
#include <stdexcept>
#include <string>
#include <vector>

#include "tla_attention.h"

// The reference's own forward declaration (src/forward.h:11,
// src/generate.h:6); defined in run_state.h.
struct RunState;

namespace tla_host {

// Throws std::runtime_error("<what>: <library message>") when status != 0.
void check(int status, const char* what);

struct Config {
    std::uint32_t n_layers = 0;
    std::uint32_t n_embd = 0;
    std::uint32_t n_head = 0;
    std::uint32_t n_head_kv = 0;
    std::uint32_t n_ff = 0;
    float rope_freq_base = 10000.0f;
    std::uint32_t n_ctx = 2048;
    std::uint32_t n_vocab = 0;
    std::uint32_t head_dim() const { return n_head > 0 ? n_embd / n_head : 0; }
    tla_config to_c() const;
};

// Owns one tla_engine (device, stream, RoPE table, split workspace).
class Engine {
public:
    explicit Engine(const Config& cfg, int device = 0);
    ~Engine();
    Engine(const Engine&) = delete;
    Engine& operator=(const Engine&) = delete;
    tla_engine* get() const { return e_; }
    const Config& config() const { return cfg_; }
    void synchronize();

private:
    tla_engine* e_ = nullptr;
    Config cfg_;
};

// ---- operators (device pointers) -------------------------------------------
void rope(Engine& eng, float* q, float* k, int pos, int head_dim, int n_head, int n_head_kv,
          float freq_base);
void softmax(Engine& eng, float* x, int size);
void attention(Engine& eng, float* out, const float* q, const float* k, const float* v,
               float* key_cache, float* value_cache, float* att, int layer, int pos);

// ---- engines for RunState ------------------------------------------------------
// The fields of a llama_config_t-like struct that the path reads.
template <class Cfg>
Config config_of(const Cfg& c)
{
    Config t;
    t.n_layers = static_cast<std::uint32_t>(c.n_layers);
    t.n_embd = static_cast<std::uint32_t>(c.n_embd);
    t.n_head = static_cast<std::uint32_t>(c.n_head);
    t.n_head_kv = static_cast<std::uint32_t>(c.n_head_kv);
    t.n_ff = static_cast<std::uint32_t>(c.n_ff);
    t.n_ctx = static_cast<std::uint32_t>(c.n_ctx);
    t.n_vocab = static_cast<std::uint32_t>(c.n_vocab);
    t.rope_freq_base = c.rope_freq_base;
    return t;
}

// The engine RunState::allocate(cfg) uses: the one set here (which must have
// cfg's attention shape; NULL clears), else one made for cfg on device 0 the
// first time (one per distinct shape, kept for the rest of the process).
void use_engine(Engine* eng);
Engine& engine_for(const Config& cfg);

namespace detail {
void allocate_state(::RunState& state, const Config& cfg, Engine& eng);
void free_state(::RunState& state) noexcept;
}  // namespace detail

// rope(state.q, state.k, pos) + attention(state.xb2, ..., layer, pos) on the
// device: one host->device copy of q|k|v, one fused launch sequence, one
// device->host copy of the output into state.xb2.  state.q and state.k are
// left unrotated on the host (forward() does not read them afterwards).
void attention_block(::RunState& state, int layer, int pos);

// ---- the projections and the FFN (device pointers) --------------------------
void matmul(Engine& eng, float* out, const void* w, const float* x, int rows, int cols, int type);
void rmsnorm(Engine& eng, float* out, const float* x, const float* weight, int size, float eps);
void vec_add(Engine& eng, float* out, const float* x, int size);
void silu(Engine& eng, float* x, int size);
void elementwise_mul(Engine& eng, float* a, const float* b, int size);
void ffn_swiglu(Engine& eng, float* out, const float* input, float* hb, float* hb2,
                const void* w_gate, const void* w_up, const void* w_down, int n_ff, int n_embd,
                int type);

// ---- the whole forward pass --------------------------------------------------
// One tensor as the GGUF file holds it: host bytes and ggml_type id.
struct TensorRef {
    const void* data = nullptr;
    std::size_t bytes = 0;
    int type = 0;
};

// The tensors forward() reads, copied to the device.  `tensor(name)` returns
// a tensor by its GGUF name and throws when it is missing (the reference's
// GGUFModel::tensor_info does); "output.weight" may be missing (tied
// embeddings), then token_embd.weight is the classifier.
struct DeviceModel {
    using Lookup = std::function<TensorRef(const std::string&)>;

    DeviceModel(Engine& eng, float rms_norm_eps, const Lookup& tensor);
    ~DeviceModel();
    DeviceModel(const DeviceModel&) = delete;
    DeviceModel& operator=(const DeviceModel&) = delete;

    Engine& engine;
    tla_model model{};
    std::vector<tla_layer_weights> layers;
    std::size_t weight_bytes = 0;

private:
    std::vector<void*> buffers_;
    const void* upload(const TensorRef& t);
};

// forward(model, state, token, pos): state.logits (host) receives the
// n_vocab logits; the KV cache is state's (device).
void forward(DeviceModel& model, ::RunState& state, int token, int pos);

// Greedy generation on the device (prompt at positions 0.., token by token
// or as one batch, then n_gen tokens); returns the generated tokens.
std::vector<int> generate_greedy(DeviceModel& model, ::RunState& state, const std::vector<int>& prompt,
                                 int n_gen, bool batch_prompt = false);

}  // namespace tla_host
