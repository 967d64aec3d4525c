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
//   tla_host::RunState         -> struct RunState (src/run_state.h:27-182):
//                                 same members in the same order; key_cache
//                                 and value_cache hold DEVICE pointers; device
//                                 staging for the attention block is appended
//                                 after the reference's members
//   tla_host::attention_block  -> the block of forward() at
//                                 src/forward.cpp:192-208 (rope + attention)
#pragma once

#include <cstdint>
#include <stdexcept>
#include <string>

#include "tla_attention.h"

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

// ---- RunState ----------------------------------------------------------------
struct RunState {
    // Host scratch, as in the reference (the CPU GEMVs read and write these).
    float* x = nullptr;
    float* xb = nullptr;
    float* xb2 = nullptr;
    float* q = nullptr;
    float* k = nullptr;
    float* v = nullptr;
    float* att = nullptr;
    float* hb = nullptr;
    float* hb2 = nullptr;
    float* logits = nullptr;
    // KV cache [n_layers][n_ctx][n_head_kv*head_dim] fp32 -- DEVICE memory.
    float* key_cache = nullptr;
    float* value_cache = nullptr;
    int pos = 0;

    // ---- appended: device side of the attention block ----
    Engine* engine = nullptr;
    float* d_qkv = nullptr;  // device copy of q | k | v (one transfer)
    float* d_out = nullptr;  // device attention output [n_embd]

    void allocate(const Config& cfg, Engine& eng);
    void free_buffers();

    RunState(const RunState&) = delete;
    RunState& operator=(const RunState&) = delete;
    RunState() = default;
    ~RunState() { free_buffers(); }

private:
    friend void attention_block(RunState& state, int layer, int pos);
    float* qkv_host_ = nullptr;  // q | k | v contiguous, so one H2D copy
    std::uint32_t n_embd_ = 0, kv_dim_ = 0;
};

// rope(state.q, state.k, pos) + attention(state.xb2, ..., layer, pos) on the
// device: one host->device copy of q|k|v, one fused launch sequence, one
// device->host copy of the output into state.xb2.  state.q and state.k are
// left unrotated on the host (forward() does not read them afterwards).
void attention_block(RunState& state, int layer, int pos);

}  // namespace tla_host
