// extern "C" entry points over the reference engine's own, unmodified
// forward pass: src/forward.cpp, src/gguf_model.cpp, src/tokenizer.cpp and
// src/ops.cpp compiled where they lie by oracle/Makefile into oracle/_ref/.
// TEST INFRASTRUCTURE ONLY: used to write golden vectors and to check the C
// oracle's forward live.  The model is a GGUF file the tests write.
//
// Wrapped interfaces:
//   ref_forward_tokens  -> GGUFModel(path) (src/gguf_model.h:56-58), a
//                          RunState allocated as src/run_state.h:115-154, then
//                          forward() (src/forward.h) once per token at
//                          positions 0..n-1, the prompt loop of
//                          src/generate.cpp:56-59; logits of every step.
//   ref_generate_greedy -> that loop followed by the argmax decode loop of
//                          src/generate.cpp:63-100 (temperature 0), without
//                          the tokenizer and the EOS stop.
//   ref_bench_trial     -> one trial of the reference's benchmark
//                          (run_trial, src/benchmark.cpp:113-165): prompt
//                          forward() calls timed, then n_decode greedy steps
//                          timed, after set_num_threads() (src/ops.h).
#include <chrono>
#include <cstring>
#include <exception>
#include <string>

#include "forward.h"
#include "gguf_model.h"
#include "ops.h"
#include "run_state.h"

static std::string g_error;

extern "C" {

const char* ref_forward_error() { return g_error.c_str(); }

int ref_forward_tokens(const char* path, const int* tokens, int n, float* logits, int* n_vocab)
{
    try {
        GGUFModel model(path);
        RunState state;
        state.allocate(model.config());
        const int nv = static_cast<int>(model.config().n_vocab);
        if (n_vocab) *n_vocab = nv;
        for (int i = 0; i < n; ++i) {
            forward(model, state, tokens[i], i);
            if (logits) std::memcpy(logits + static_cast<std::size_t>(i) * nv, state.logits,
                                    sizeof(float) * static_cast<std::size_t>(nv));
        }
        return 0;
    } catch (const std::exception& ex) {
        g_error = ex.what();
        return -1;
    }
}

int ref_generate_greedy(const char* path, const int* prompt, int n_prompt, int n_gen, int* out)
{
    try {
        GGUFModel model(path);
        RunState state;
        state.allocate(model.config());
        const int nv = static_cast<int>(model.config().n_vocab);
        state.pos = 0;
        for (int i = 0; i < n_prompt; ++i) {
            forward(model, state, prompt[i], state.pos);
            state.pos++;
        }
        int next = sample_argmax(state.logits, nv);
        for (int i = 0; i < n_gen; ++i) {
            out[i] = next;
            if (i + 1 == n_gen) break;
            forward(model, state, next, state.pos);
            state.pos++;
            next = sample_argmax(state.logits, nv);
        }
        return 0;
    } catch (const std::exception& ex) {
        g_error = ex.what();
        return -1;
    }
}

int ref_bench_trial(const char* path, const int* prompt, int n_prompt, int n_decode, int threads,
                    double* prefill_ms, double* decode_ms)
{
    try {
        using Clock = std::chrono::steady_clock;
        set_num_threads(threads);
        GGUFModel model(path);
        RunState state;
        state.allocate(model.config());
        const int nv = static_cast<int>(model.config().n_vocab);
        state.pos = 0;
        const auto t0 = Clock::now();
        for (int i = 0; i < n_prompt; ++i) {
            forward(model, state, prompt[i], state.pos);
            state.pos++;
        }
        const auto t1 = Clock::now();
        int next = sample_argmax(state.logits, nv);
        const auto t2 = Clock::now();
        for (int i = 0; i < n_decode; ++i) {
            forward(model, state, next, state.pos);
            state.pos++;
            next = sample_argmax(state.logits, nv);
        }
        const auto t3 = Clock::now();
        *prefill_ms = std::chrono::duration<double, std::milli>(t1 - t0).count();
        *decode_ms = std::chrono::duration<double, std::milli>(t3 - t2).count();
        set_num_threads(1);
        return 0;
    } catch (const std::exception& ex) {
        g_error = ex.what();
        return -1;
    }
}

}  // extern "C"
