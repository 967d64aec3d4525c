// C++ test of the host side (tinyllama-engine_amd/host) on the GPU, written
// in the style of the reference's src/test_ops.cpp (a check() counter, exit
// code 1 on any failure).  It drives:
//   - tla_host::attention with the cases of src/test_ops.cpp:295-431,
//   - tla_host::rope with the cases of src/test_ops.cpp:433-546,
//   - RunState + attention_block (the forward() block, src/forward.cpp:192-208)
//     over a 64-token sequence on two layers, checked against the CPU oracle
//     (oracle/tl_oracle.c) within 1e-4 and the KV cache bit for bit,
//   - the error convention: an out-of-range position throws std::runtime_error,
//   - DeviceModel + forward (src/forward.cpp:167-266) on a 2-layer model of
//     TinyLlama's widths with seeded Q8_0 weights and a Q6_K-free tied
//     classifier, against the oracle's forward within 1e-4 of the largest
//     logit, and generate_greedy against the oracle's argmax chain.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <map>
#include <random>
#include <string>
#include <stdexcept>
#include <vector>

#include "run_state.h"
#include "tla_host.h"

extern "C" {
struct oracle_layer {
    const float* attn_norm;
    const void *wq, *wk, *wv, *wo;
    int type_q, type_k, type_v, type_o;
    const float* ffn_norm;
    const void *w_gate, *w_up, *w_down;
    int type_ffn;
};
struct oracle_model {
    int n_layers, n_embd, n_head, n_head_kv, n_ff, n_vocab, n_ctx;
    float rope_freq_base, rms_norm_eps;
    const void* token_embd;
    int type_embd;
    const float* output_norm;
    const void* output;
    int type_output;
    const oracle_layer* layers;
};
int oracle_forward(const oracle_model* m, float* key_cache, float* value_cache, float* scratch,
                   int token, int pos, float* logits);
void oracle_rope(float* q, float* k, int pos, int head_dim, int n_head, int n_head_kv,
                 float freq_base);
void oracle_attention(float* out, const float* q, const float* k, const float* v,
                      float* key_cache, float* value_cache, float* att, int layer, int pos,
                      int n_head, int n_head_kv, int head_dim, int n_ctx);
}

static int passed = 0, failed = 0;

static void check(const char* name, bool ok)
{
    std::printf("  %s %s\n", ok ? "ok  " : "FAIL", name);
    (ok ? passed : failed)++;
}

static bool near(float a, float b, float tol = 1e-4f) { return std::fabs(a - b) < tol; }

struct Dev {
    tla_host::Engine& eng;
    float* p = nullptr;
    size_t n = 0;
    Dev(tla_host::Engine& e, size_t count) : eng(e), n(count)
    {
        void* v = nullptr;
        tla_host::check(tla_alloc(e.get(), count * sizeof(float), &v), "alloc");
        p = static_cast<float*>(v);
    }
    ~Dev() { tla_free(eng.get(), p); }
    void put(const std::vector<float>& h) { tla_host::check(tla_memcpy_h2d(eng.get(), p, h.data(), n * 4), "h2d"); }
    std::vector<float> get() const
    {
        std::vector<float> h(n);
        tla_host::check(tla_memcpy_d2h(eng.get(), h.data(), p, n * 4), "d2h");
        return h;
    }
};

static void test_attention(tla_host::Engine& eng)
{
    std::printf("\n=== attention (src/test_ops.cpp cases) ===\n");
    const int n_embd = 2048, kv_dim = 256, hd = 64, n_ctx = 64, n_layers = 2;
    Dev out(eng, n_embd), q(eng, n_embd), k(eng, kv_dim), v(eng, kv_dim);
    Dev kc(eng, size_t(n_layers) * n_ctx * kv_dim), vc(eng, size_t(n_layers) * n_ctx * kv_dim);
    std::vector<float> zeros(kc.n, 0.f), hq(n_embd, 1.f), hk(kv_dim, 1.f), hv(kv_dim);

    for (int i = 0; i < kv_dim; ++i) hv[i] = float(i % hd);
    q.put(hq); k.put(hk); v.put(hv);
    tla_host::attention(eng, out.p, q.p, k.p, v.p, kc.p, vc.p, nullptr, 0, 0);
    auto o = out.get();
    bool ok = true;
    for (int d = 0; d < hd; ++d) ok = ok && near(o[d], float(d), 1e-3f);
    check("single token: output = value", ok);

    kc.put(zeros); vc.put(zeros);
    v.put(std::vector<float>(kv_dim, 1.f));
    tla_host::attention(eng, out.p, q.p, k.p, v.p, kc.p, vc.p, nullptr, 0, 0);
    v.put(std::vector<float>(kv_dim, 3.f));
    tla_host::attention(eng, out.p, q.p, k.p, v.p, kc.p, vc.p, nullptr, 0, 1);
    check("uniform attention: 50/50 blend -> 2.0", near(out.get()[0], 2.f, 0.01f));

    kc.put(zeros); vc.put(zeros);
    std::vector<float> hkc(kc.n, 0.f), hvc(vc.n, 0.f), att(n_ctx), ref(n_embd);
    bool finite = true, match = true;
    for (int p = 0; p < 10; ++p) {
        for (int i = 0; i < n_embd; ++i) hq[i] = float((i + p) % 11) - 5.f;
        for (int i = 0; i < kv_dim; ++i) {
            hk[i] = float((i + p * 3) % 7) - 3.f;
            hv[i] = float((i + p * 5) % 9) - 4.f;
        }
        q.put(hq); k.put(hk); v.put(hv);
        tla_host::attention(eng, out.p, q.p, k.p, v.p, kc.p, vc.p, nullptr, 0, p);
        oracle_attention(ref.data(), hq.data(), hk.data(), hv.data(), hkc.data(), hvc.data(),
                         att.data(), 0, p, 32, 4, 64, n_ctx);
        o = out.get();
        for (int i = 0; i < n_embd; ++i) {
            finite = finite && std::isfinite(o[i]);
            match = match && near(o[i], ref[i]);
        }
    }
    check("10 tokens: no NaN/Inf in output", finite);
    check("10 tokens: matches the oracle within 1e-4", match);
    check("10 tokens: key cache bit-exact", std::memcmp(kc.get().data(), hkc.data(), kc.n * 4) == 0);
    check("10 tokens: value cache bit-exact", std::memcmp(vc.get().data(), hvc.data(), vc.n * 4) == 0);

    kc.put(zeros); vc.put(zeros);
    std::fill(hk.begin(), hk.end(), 1.f);
    std::fill(hq.begin(), hq.end(), 1.f);
    std::fill(hv.begin(), hv.end(), 0.f);
    for (int d = 0; d < hd; ++d) { hv[d] = 10.f; hv[hd + d] = 20.f; }
    q.put(hq); k.put(hk); v.put(hv);
    tla_host::attention(eng, out.p, q.p, k.p, v.p, kc.p, vc.p, nullptr, 0, 0);
    o = out.get();
    check("GQA: head 0 uses KV head 0 (val=10)", near(o[0], 10.f, 0.01f));
    check("GQA: head 8 uses KV head 1 (val=20)", near(o[8 * hd], 20.f, 0.01f));
}

static void test_rope(tla_host::Engine& eng)
{
    std::printf("\n=== rope (src/test_ops.cpp cases) ===\n");
    const int hd = 64, nh = 32, nkv = 4;
    Dev q(eng, nh * hd), k(eng, nkv * hd);
    std::vector<float> hq(nh * hd, 1.f), hk(nkv * hd, 1.f);
    q.put(hq); k.put(hk);
    tla_host::rope(eng, q.p, k.p, 0, hd, nh, nkv, 10000.f);
    check("position 0: Q unchanged", q.get() == hq);
    check("position 0: K unchanged", k.get() == hk);

    for (int i = 0; i < nh * hd; ++i) hq[i] = float(i % 7) - 3.f;
    q.put(hq);
    tla_host::rope(eng, q.p, k.p, 42, hd, nh, nkv, 10000.f);
    auto r = q.get();
    float n0 = 0.f, n1 = 0.f;
    for (int i = 0; i < hd; ++i) { n0 += hq[i] * hq[i]; n1 += r[i] * r[i]; }
    check("rotation preserves vector length", near(std::sqrt(n0), std::sqrt(n1), 1e-3f));

    bool exact = true;
    std::mt19937 gen(3);
    std::normal_distribution<float> nd;
    for (int pos : {1, 5, 17, 100, 2047, 5000, 16383, 70000}) {
        for (auto& x : hq) x = nd(gen);
        for (auto& x : hk) x = nd(gen);
        std::vector<float> eq = hq, ek = hk;
        oracle_rope(eq.data(), ek.data(), pos, hd, nh, nkv, 10000.f);
        q.put(hq); k.put(hk);
        tla_host::rope(eng, q.p, k.p, pos, hd, nh, nkv, 10000.f);
        exact = exact && std::memcmp(q.get().data(), eq.data(), eq.size() * 4) == 0 &&
                std::memcmp(k.get().data(), ek.data(), ek.size() * 4) == 0;
    }
    check("rope bit-exact with the oracle at 8 positions", exact);

    std::fill(hq.begin(), hq.end(), 0.f);
    hq[0] = 3.f; hq[1] = 4.f;
    q.put(hq);
    tla_host::rope(eng, q.p, k.p, 1, hd, nh, nkv, 10000.f);
    r = q.get();
    check("manual rotation q[0]", near(r[0], 3.f * std::cos(1.f) - 4.f * std::sin(1.f)));
    check("manual rotation q[1]", near(r[1], 3.f * std::sin(1.f) + 4.f * std::cos(1.f)));
}

static void test_block(tla_host::Engine& eng, const tla_host::Config& cfg)
{
    std::printf("\n=== RunState + attention_block (forward.cpp:192-208) ===\n");
    RunState st;
    st.allocate(cfg, eng);
    const int kv_dim = 256, n_embd = 2048, n_ctx = int(cfg.n_ctx);
    std::vector<float> hkc(size_t(cfg.n_layers) * n_ctx * kv_dim, 0.f), hvc(hkc.size(), 0.f);
    std::vector<float> qq(n_embd), kk(kv_dim), ref(n_embd), att(n_ctx);
    std::mt19937 gen(7);
    std::normal_distribution<float> nd;
    float worst = 0.f;
    for (int pos = 0; pos < 64; ++pos)
        for (int layer = 0; layer < int(cfg.n_layers); ++layer) {
            for (int i = 0; i < n_embd; ++i) st.q[i] = nd(gen);
            for (int i = 0; i < kv_dim; ++i) { st.k[i] = nd(gen); st.v[i] = nd(gen); }
            std::memcpy(qq.data(), st.q, n_embd * 4);
            std::memcpy(kk.data(), st.k, kv_dim * 4);
            tla_host::attention_block(st, layer, pos);
            oracle_rope(qq.data(), kk.data(), pos, 64, 32, 4, cfg.rope_freq_base);
            oracle_attention(ref.data(), qq.data(), kk.data(), st.v, hkc.data(), hvc.data(),
                             att.data(), layer, pos, 32, 4, 64, n_ctx);
            for (int i = 0; i < n_embd; ++i) worst = std::fmax(worst, std::fabs(st.xb2[i] - ref[i]));
        }
    std::printf("    max-abs error over 64 tokens x %u layers: %.3g\n", cfg.n_layers, worst);
    check("attention_block matches the oracle within 1e-4", worst <= 1e-4f);
    std::vector<float> dk(hkc.size()), dv(hvc.size());
    tla_host::check(tla_memcpy_d2h(eng.get(), dk.data(), st.key_cache, dk.size() * 4), "d2h");
    tla_host::check(tla_memcpy_d2h(eng.get(), dv.data(), st.value_cache, dv.size() * 4), "d2h");
    check("device key cache bit-exact", std::memcmp(dk.data(), hkc.data(), dk.size() * 4) == 0);
    check("device value cache bit-exact", std::memcmp(dv.data(), hvc.data(), dv.size() * 4) == 0);

    bool threw = false;
    try {
        tla_host::attention_block(st, 0, n_ctx);
    } catch (const std::runtime_error& e) {
        threw = std::strstr(e.what(), "outside") != nullptr;
    }
    check("pos == n_ctx throws std::runtime_error", threw);
    threw = false;
    try {
        tla_host::attention_block(st, int(cfg.n_layers), 0);
    } catch (const std::runtime_error&) {
        threw = true;
    }
    check("layer == n_layers throws std::runtime_error", threw);
}

// Half-precision bits of a positive normal float (truncated mantissa).
static std::uint16_t half_bits(float f)
{
    std::uint32_t b;
    std::memcpy(&b, &f, 4);
    const int e = int((b >> 23) & 0xFF) - 127 + 15;
    return static_cast<std::uint16_t>((e << 10) | ((b >> 13) & 0x3FF));
}

// Seeded Q8_0 matrix [rows][cols]: scales in [2e-4, 3e-4), int8 weights.
static std::vector<std::uint8_t> q8_matrix(std::mt19937& gen, int rows, int cols)
{
    std::vector<std::uint8_t> m(size_t(rows) * (cols / 32) * 34);
    std::uniform_real_distribution<float> sd(2e-4f, 3e-4f);
    std::uniform_int_distribution<int> qd(0, 255);
    for (size_t b = 0; b < m.size() / 34; ++b) {
        const std::uint16_t h = half_bits(sd(gen));
        m[34 * b] = h & 0xFF;
        m[34 * b + 1] = h >> 8;
        for (int j = 0; j < 32; ++j) m[34 * b + 2 + j] = static_cast<std::uint8_t>(qd(gen));
    }
    return m;
}

static void test_forward(tla_host::Engine& eng, const tla_host::Config& cfg)
{
    std::printf("\n=== DeviceModel + forward (forward.cpp:167-266) ===\n");
    const int E = int(cfg.n_embd), KV = 256, FF = int(cfg.n_ff), V = int(cfg.n_vocab), L = int(cfg.n_layers);
    std::mt19937 gen(11);
    std::uniform_real_distribution<float> nd(0.5f, 1.5f);
    std::map<std::string, std::vector<std::uint8_t>> bytes;
    auto norm = [&](const std::string& name) {
        std::vector<float> v(E);
        for (float& x : v) x = nd(gen);
        bytes[name].resize(E * 4);
        std::memcpy(bytes[name].data(), v.data(), E * 4);
    };
    bytes["token_embd.weight"] = q8_matrix(gen, V, E);  // tied classifier: no output.weight
    norm("output_norm.weight");
    for (int l = 0; l < L; ++l) {
        const std::string p = "blk." + std::to_string(l) + ".";
        norm(p + "attn_norm.weight");
        norm(p + "ffn_norm.weight");
        bytes[p + "attn_q.weight"] = q8_matrix(gen, E, E);
        bytes[p + "attn_k.weight"] = q8_matrix(gen, KV, E);
        bytes[p + "attn_v.weight"] = q8_matrix(gen, KV, E);
        bytes[p + "attn_output.weight"] = q8_matrix(gen, E, E);
        bytes[p + "ffn_gate.weight"] = q8_matrix(gen, FF, E);
        bytes[p + "ffn_up.weight"] = q8_matrix(gen, FF, E);
        bytes[p + "ffn_down.weight"] = q8_matrix(gen, E, FF);
    }
    auto lookup = [&](const std::string& name) {
        auto it = bytes.find(name);
        if (it == bytes.end()) throw std::runtime_error("Tensor not found: " + name);
        const bool norm_w = name.find("norm") != std::string::npos;
        return tla_host::TensorRef{it->second.data(), it->second.size(), norm_w ? 0 : 8};
    };
    const float eps = 1e-5f;
    tla_host::DeviceModel dm(eng, eps, lookup);
    RunState st;
    st.allocate(cfg, eng);

    std::vector<oracle_layer> ol(L);
    for (int l = 0; l < L; ++l) {
        const std::string p = "blk." + std::to_string(l) + ".";
        auto d = [&](const char* n) { return static_cast<const void*>(bytes[p + n].data()); };
        ol[l] = {static_cast<const float*>(d("attn_norm.weight")), d("attn_q.weight"), d("attn_k.weight"),
                 d("attn_v.weight"), d("attn_output.weight"), 8, 8, 8, 8,
                 static_cast<const float*>(d("ffn_norm.weight")), d("ffn_gate.weight"),
                 d("ffn_up.weight"), d("ffn_down.weight"), 8};
    }
    const oracle_model om = {L, E, int(cfg.n_head), int(cfg.n_head_kv), FF, V, int(cfg.n_ctx),
                             cfg.rope_freq_base, eps, bytes["token_embd.weight"].data(), 8,
                             reinterpret_cast<const float*>(bytes["output_norm.weight"].data()),
                             bytes["token_embd.weight"].data(), 8, ol.data()};
    std::vector<float> okc(size_t(L) * cfg.n_ctx * KV, 0.f), ovc(okc.size(), 0.f);
    std::vector<float> scratch(5 * E + 2 * KV + cfg.n_ctx + 2 * FF), ologits(V);
    const int tokens[6] = {1, 15043, 29871, 31999, 0, 2};
    float worst = 0.f;
    for (int pos = 0; pos < 6; ++pos) {
        tla_host::forward(dm, st, tokens[pos], pos);
        oracle_forward(&om, okc.data(), ovc.data(), scratch.data(), tokens[pos], pos, ologits.data());
        float scale = 0.f, err = 0.f;
        for (int i = 0; i < V; ++i) {
            scale = std::fmax(scale, std::fabs(ologits[i]));
            err = std::fmax(err, std::fabs(st.logits[i] - ologits[i]));
        }
        worst = std::fmax(worst, err / scale);
    }
    std::printf("    max |gpu - oracle| / max|logit| over 6 tokens: %.3g\n", worst);
    check("forward matches the oracle within 1e-4 of the largest logit", worst <= 1e-4f);

    // greedy: the oracle's argmax chain from a fresh cache
    std::fill(okc.begin(), okc.end(), 0.f);
    std::fill(ovc.begin(), ovc.end(), 0.f);
    const std::vector<int> prompt = {1, 450, 4996};
    const int n_gen = 8;
    std::vector<int> want;
    int pos = 0;
    for (int t : prompt) oracle_forward(&om, okc.data(), ovc.data(), scratch.data(), t, pos++, ologits.data());
    bool clear = true;
    for (int i = 0; i < n_gen; ++i) {
        int best = 0, second = -1;
        for (int j = 1; j < V; ++j)
            if (ologits[j] > ologits[best]) best = j;
        for (int j = 0; j < V; ++j)
            if (j != best && (second < 0 || ologits[j] > ologits[second])) second = j;
        clear = clear && ologits[best] - ologits[second] > 2e-4f * std::fabs(ologits[best]);
        want.push_back(best);
        if (i + 1 < n_gen) oracle_forward(&om, okc.data(), ovc.data(), scratch.data(), best, pos++, ologits.data());
    }
    RunState st2;
    st2.allocate(cfg, eng);
    const std::vector<int> got = tla_host::generate_greedy(dm, st2, prompt, n_gen);
    check("greedy path has no near-ties", clear);
    check("generate_greedy equals the oracle's argmax chain", got == want);
    bool threw = false;
    try {
        tla_host::forward(dm, st, V, 0);
    } catch (const std::runtime_error&) {
        threw = true;
    }
    check("token == n_vocab throws std::runtime_error", threw);
}

int main()
{
    try {
        tla_host::Config cfg;
        cfg.n_layers = 2;
        cfg.n_embd = 2048;
        cfg.n_head = 32;
        cfg.n_head_kv = 4;
        cfg.n_ff = 5632;
        cfg.n_vocab = 32000;
        cfg.n_ctx = 64;
        tla_host::Engine eng(cfg);
        test_attention(eng);
        test_rope(eng);
        test_block(eng, cfg);
        test_forward(eng, cfg);
    } catch (const std::exception& e) {
        std::printf("ERROR: %s\n", e.what());
        return 1;
    }
    std::printf("\n%d passed, %d failed\n", passed, failed);
    return failed ? 1 : 0;
}
