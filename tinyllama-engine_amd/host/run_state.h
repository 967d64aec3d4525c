// Drop-in replacement for the reference engine's src/run_state.h
// (src/run_state.h:27-182): the same global `struct RunState`, with the same
// members in the same order and the same lifecycle (allocate / free_buffers,
// non-copyable, default-constructible), so that the reference's own files
// compile unchanged against it -- the forward declarations `struct RunState;`
// in src/forward.h:11 and src/generate.h:6, `state.allocate(model.config())`
// in src/main.cpp:172 and src/benchmark.cpp:120, and every `state.x`,
// `state.logits`, `state.pos` use.
//
// What changes: key_cache and value_cache hold DEVICE pointers (the KV cache
// lives in HBM, [n_layers][n_ctx][n_head_kv * head_dim] fp32 as before), and
// device staging for the attention block is appended after the reference's
// members.  The host scratch (x, xb, xb2, q, k, v, att, hb, hb2, logits)
// stays in host memory, so the reference's CPU code around the attention
// block runs as it did; the block itself (src/forward.cpp:192-208) becomes
// tla_host::attention_block(state, l, pos).
//
// allocate() takes any config with the fields of llama_config_t
// (src/gguf.h:139-168) that it reads: n_layers, n_embd, n_head, n_head_kv,
// n_ff, n_ctx, n_vocab, rope_freq_base.  The device engine comes from
// tla_host::use_engine() when the caller set one, else one is created for
// the config on device 0 and kept for the rest of the process.
#pragma once

#include <cstddef>
#include <cstdint>
#include <cstring>
#include <stdexcept>

// The reference's run_state.h brings llama_config_t into every file that
// includes it; keep that where the reference's headers are on the path.
#if __has_include("gguf.h")
#include "gguf.h"
#endif

#include "tla_host.h"

struct RunState {
    // ---- the reference's members, in its order ----
    float* x = nullptr;       // [n_embd]
    float* xb = nullptr;      // [n_embd]
    float* xb2 = nullptr;     // [n_embd]; the attention block's output lands here
    float* q = nullptr;       // [n_embd]
    float* k = nullptr;       // [n_head_kv * head_dim]
    float* v = nullptr;       // [n_head_kv * head_dim]
    float* att = nullptr;     // [n_ctx]
    float* hb = nullptr;      // [n_ff]
    float* hb2 = nullptr;     // [n_ff]
    float* logits = nullptr;  // [n_vocab]
    float* key_cache = nullptr;    // DEVICE [n_layers][n_ctx][kv_dim]
    float* value_cache = nullptr;  // DEVICE [n_layers][n_ctx][kv_dim]
    int pos = 0;

    // ---- appended: the device side ----
    tla_host::Engine* engine = nullptr;
    float* d_qkv = nullptr;     // device copy of q | k | v (one transfer per block)
    float* d_out = nullptr;     // device attention output [n_embd]
    float* d_logits = nullptr;  // device logits [n_vocab] (tla_host::forward)
    float* qkv_host = nullptr;  // q, k and v as one host block (q, k, v point into it)
    std::uint32_t n_embd = 0;
    std::uint32_t kv_dim = 0;
    std::uint32_t n_vocab = 0;

    // Allocate every buffer for `cfg` (src/run_state.h:115-154): host scratch
    // zero-filled, device KV cache zero-filled.  Engine: tla_host::use_engine()'s,
    // else one made for the config.
    template <class Cfg>
    void allocate(const Cfg& cfg)
    {
        const tla_host::Config c = tla_host::config_of(cfg);
        tla_host::detail::allocate_state(*this, c, tla_host::engine_for(c));
    }

    // The same on a given engine (whose config must match).
    template <class Cfg>
    void allocate(const Cfg& cfg, tla_host::Engine& eng)
    {
        tla_host::detail::allocate_state(*this, tla_host::config_of(cfg), eng);
    }

    // Free all buffers (src/run_state.h:157-170).
    void free_buffers() { tla_host::detail::free_state(*this); }

    RunState(const RunState&) = delete;
    RunState& operator=(const RunState&) = delete;
    RunState() = default;
    ~RunState() { free_buffers(); }
};
