// C ABI of libtla.so: engine lifetime, device memory, argument validation
// and launch planning.  Kernels live in decode.hip, prefill.hip and
// small_ops.hip.
#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <deque>
#include <mutex>
#include <string>
#include <utility>
#include <vector>


#include "batch.h"
#include "tla_internal.h"

using namespace tla;

namespace {

// The calling thread's last error message: a fixed buffer, so that no error
// path allocates (the allocation-free entry point shares these paths).
thread_local char g_last_error[512];

int fail(int code, const char* fmt, ...)
{
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(g_last_error, sizeof g_last_error, fmt, ap);
    va_end(ap);
    return code;
}

int ok()
{
    return TLA_OK;
}

#define TLA_HIP(call)                                                                         \
    do {                                                                                      \
        const hipError_t err_ = (call);                                                       \
        if (err_ != hipSuccess)                                                               \
            return fail(err_ == hipErrorOutOfMemory ? TLA_ERR_OUT_OF_MEMORY : TLA_ERR_DEVICE, \
                        "%s failed: %s", #call, hipGetErrorString(err_));                     \
    } while (0)

// cos/sin table with the reference's float expressions (src/ops.cpp:1244-1251):
//   freq  = 1.0f / powf(base, (float)(2i) / (float)head_dim)
//   angle = (float)pos * freq;  c = cosf(angle);  s = sinf(angle)
// Contraction off so that nothing is fused; the libm is the host's, as the
// reference's.
void rope_cos_sin(float2* out, int pos, int head_dim, float freq_base)
{
#pragma clang fp contract(off)
    const int pairs = head_dim / 2;
    for (int i = 0; i < pairs; ++i) {
        const float expo = static_cast<float>(2 * i) / static_cast<float>(head_dim);
        const float freq = 1.0f / std::pow(freq_base, expo);
        const float angle = static_cast<float>(pos) * freq;
        out[i].x = std::cos(angle);
        out[i].y = std::sin(angle);
    }
}

void rope_table_host(std::vector<float2>& tab, int n_pos, int head_dim, float freq_base)
{
#pragma clang fp contract(off)
    const int pairs = head_dim / 2;
    std::vector<float> freq(pairs);
    for (int i = 0; i < pairs; ++i) {
        const float expo = static_cast<float>(2 * i) / static_cast<float>(head_dim);
        freq[i] = 1.0f / std::pow(freq_base, expo);
    }
    tab.resize(static_cast<size_t>(n_pos) * pairs);
    for (int p = 0; p < n_pos; ++p)
        for (int i = 0; i < pairs; ++i) {
            const float angle = static_cast<float>(p) * freq[i];
            tab[static_cast<size_t>(p) * pairs + i] = make_float2(std::cos(angle), std::sin(angle));
        }
}

constexpr int kEventSlots = 64;

}  // namespace

// ---- split scratch of the allocation-free decode entry point ---------------
// tla_decode_noalloc keeps the split partials and arrival counters of a
// launch in this fixed array instead of an engine workspace: 32 MiB of
// partials (66 floats per q head for each (sequence, layer, split, kv head))
// and 64 Ki counters.  Each device holds its own copy until the process ends.
// Host code never names it directly: it uses the per-device address from
// hipGetSymbolAddress, taken once per device when the first engine is created
// there.
namespace {
constexpr size_t kScratchPartBytes = size_t(32) << 20;
constexpr size_t kScratchCounters = size_t(1) << 16;
constexpr size_t kScratchBytes = kScratchPartBytes + kScratchCounters * sizeof(int);
constexpr int kScratchDevices = 64;
}  // namespace

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {
std::mutex g_scratch_mu;
void* g_scratch_ptr[kScratchDevices] = {};  // device address of `scratch`, per device

}  // namespace

struct tla_engine {
    tla_config cfg{};
    int device = 0;
    int head_dim = 0;
    int kv_dim = 0;
    int gqa = 0;
    hipStream_t stream = nullptr;
    float2* rope = nullptr;  // [n_ctx][head_dim/2]
    void* scratch = nullptr; // this device's copy of `scratch` (tla_decode_noalloc), or NULL
    void* ws = nullptr;      // split-KV partials
    size_t ws_bytes = 0;
    int* counters = nullptr; // per-unit split arrival counters, zero between launches
    size_t n_counters = 0;
    void* fwd = nullptr;     // forward(): residual stream, q|k|v, attention out, FFN, tokens
    size_t fwd_bytes = 0;
    unsigned char* xs = nullptr;  // batched products: x split into bf16 planes
    size_t xs_bytes = 0;
    float* part = nullptr;        // and their K splits' partial sums
    size_t part_bytes = 0;
    unsigned char* kvp = nullptr; // prefill: K and V tiles as bf16 planes
    size_t kvp_bytes = 0;
    int* argmax_slot = nullptr;
    unsigned long long* amax_keys = nullptr;  // kAmaxSlots keys (tla_matmul_argmax)
    long long opt_split = 0;
    int opt_plan = TLA_PLAN_AUTO;
    int opt_group = 0;  // kv heads per aligned-plan workgroup, 0 = per launch
    int opt_stream_tiles = 0;  // streamed product: token tiles per workgroup, 0 = per shape
    int opt_split_rows = 0;    // split product: 16-row subtiles per wave, 0 = per shape
    int opt_split_k = 0;       // split product: K ranges, 0 = per shape
    int n_cu = 256;          // compute units: decode workgroups per launch

    bool prof = false;
    std::vector<std::pair<hipEvent_t, hipEvent_t>> prof_pending[TLA_KERNEL_COUNT];
    double prof_ms[TLA_KERNEL_COUNT] = {};
    long long prof_n[TLA_KERNEL_COUNT] = {};
    std::vector<hipEvent_t> event_pool;

    hipEvent_t slots[kEventSlots] = {};
};

namespace {

int set_device(tla_engine* e)
{
    TLA_HIP(hipSetDevice(e->device));
    return TLA_OK;
}

// Once per device, with the device current: the device address of the
// static scratch, and its counters zeroed (every decode launch returns the
// counters it uses to zero, so they stay zero between launches).  Devices past
// kScratchDevices get none (tla_decode_noalloc then returns an error).
int scratch_setup(tla_engine* e)
{
    if (e->device >= kScratchDevices) return TLA_OK;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[e->device]) {
        void* ptr = nullptr;
        TLA_HIP(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
        TLA_HIP(launch_zero(static_cast<char*>(ptr) + kScratchPartBytes, kScratchCounters * sizeof(int),
                            e->stream));
        TLA_HIP(hipStreamSynchronize(e->stream));
        g_scratch_ptr[e->device] = ptr;
    }
    e->scratch = g_scratch_ptr[e->device];
    return TLA_OK;
}

int take_event(tla_engine* e, hipEvent_t* ev)
{
    if (!e->event_pool.empty()) {
        *ev = e->event_pool.back();
        e->event_pool.pop_back();
        return TLA_OK;
    }
    TLA_HIP(hipEventCreate(ev));
    return TLA_OK;
}

// Settle finished profiling events into the per-kernel sums.
int prof_collect(tla_engine* e)
{
    for (int k = 0; k < TLA_KERNEL_COUNT; ++k) {
        for (auto& pr : e->prof_pending[k]) {
            TLA_HIP(hipEventSynchronize(pr.second));
            float ms = 0.f;
            TLA_HIP(hipEventElapsedTime(&ms, pr.first, pr.second));
            e->prof_ms[k] += ms;
            e->prof_n[k] += 1;
            e->event_pool.push_back(pr.first);
            e->event_pool.push_back(pr.second);
        }
        e->prof_pending[k].clear();
    }
    return TLA_OK;
}

// Launch `fn` on the engine stream, bracketed by events when profiling.
template <class Fn>
int launch(tla_engine* e, int kernel_id, const char* what, Fn&& fn)
{
    hipEvent_t a = nullptr, b = nullptr;
    if (e->prof) {
        if (int rc = take_event(e, &a)) return rc;
        if (int rc = take_event(e, &b)) return rc;
        TLA_HIP(hipEventRecord(a, e->stream));
    }
    const hipError_t err = fn();
    if (err != hipSuccess)
        return fail(TLA_ERR_DEVICE, "%s launch failed: %s", what, hipGetErrorString(err));
    if (e->prof) {
        TLA_HIP(hipEventRecord(b, e->stream));
        e->prof_pending[kernel_id].emplace_back(a, b);
        // Keep the pending list bounded for long profiled runs.
        if (e->prof_pending[kernel_id].size() > 4096)
            if (int rc = prof_collect(e)) return rc;
    }
    return TLA_OK;
}

// Split partials for a decode launch (every word is written before it is
// read within one launch, so no clearing is needed).
int ensure_ws(tla_engine* e, size_t bytes)
{
    if (bytes <= e->ws_bytes) return TLA_OK;
    TLA_HIP(hipStreamSynchronize(e->stream));
    if (e->ws) TLA_HIP(hipFree(e->ws));
    e->ws = nullptr;
    e->ws_bytes = 0;
    const size_t rounded = (bytes + (1u << 20) - 1) & ~static_cast<size_t>((1u << 20) - 1);
    TLA_HIP(hipMalloc(&e->ws, rounded));
    e->ws_bytes = rounded;
    return TLA_OK;
}

// Arrival counters for `units` (unit, kv head group) pairs.  Zeroed once
// when (re)allocated (by a kernel: no memset node); the decode kernel returns
// every counter it uses to zero.
int ensure_counters(tla_engine* e, size_t units)
{
    if (units <= e->n_counters) return TLA_OK;
    TLA_HIP(hipStreamSynchronize(e->stream));
    if (e->counters) TLA_HIP(hipFree(e->counters));
    e->counters = nullptr;
    e->n_counters = 0;
    const size_t n = std::max<size_t>(units, 1024);
    TLA_HIP(hipMalloc(&e->counters, n * sizeof(int)));
    TLA_HIP(launch_zero(e->counters, n * sizeof(int), e->stream));
    TLA_HIP(hipStreamSynchronize(e->stream));
    e->n_counters = n;
    return TLA_OK;
}


int check_engine(const tla_engine* e)
{
    if (!e) return fail(TLA_ERR_INVALID_ARGUMENT, "engine is NULL");
    return TLA_OK;
}

float scale_log2(int head_dim)
{
    // scores are q.k / sqrt(head_dim) (src/ops.cpp:1335); softmax runs in base 2.
    return static_cast<float>(1.4426950408889634 / std::sqrt(static_cast<double>(head_dim)));
}

// Decode work plans.  Either has 8 waves per CU: four 2-wave workgroups of
// one kv head, two 4-wave workgroups of 2 or one 8-wave workgroup of 4 (see
// kv_group).
//
// Aligned: every unit (sequence, layer) is cut into splits of one length,
// each a workgroup of its own.  The length gives about 15/16 of the CUs a
// split each when that fills one round of workgroups, and is at least 64
// positions, at most the longest sequence and at most 4096: a bigger batch
// then takes whole sequences per workgroup, longest first, in several
// rounds.  No workgroup pays for more than one split's fixed costs.
//
// Balanced: the tiles of all units laid end to end are cut into one equal
// range per CU; a range that meets a unit boundary continues into the next
// unit.  Every workgroup streams the same number of tiles, but one that
// crosses a boundary starts its pipeline twice (q and the first tiles
// loaded with nothing else in flight) and may merge two units at the end.
//
// Measured on MI355X (22 layers): one sequence at 2048-16384 positions,
// aligned (one round of 242 workgroups) 24.2-129.5 us against balanced
// 30-32 / 133-143 us whatever its workgroup count (217-256): the
// workgroups that cross a boundary end last.  8 sequences at 16384
// (aligned: 2.75 rounds of 4096-position splits) 76.2 % of HBM aligned,
// 77.5 % balanced.  64 ragged sequences (256-2048; ranges span about six
// units) 70.8 % aligned, 66.6 % balanced.  Hence: aligned when it fits one
// round; otherwise balanced when a range is no longer than the shortest
// unit (so it crosses at most one boundary), else aligned.
//
// Below 64 positions per split a launch is latency-bound: one tile costs a
// wave ~1,000 cycles of MFMA (half of it the GQA padding columns), a second
// batch of tiles a memory round trip, and a split merge ~2 us.  Same-box
// A/B, back-to-back launches, 1 / 8 / 22 layers (append path; the
// attention-only path alike): sequences of up to 128 positions as one
// split each, 6.6-6.9 us at 128 positions against 7.3-7.7 us in splits of
// 64; of 129-256 positions in splits of 32, 6.5 / 7.6 / 9.9 us at 256
// against 7.1 / 7.6 / 10.1 us in splits of 64; longer ones in splits of 64
// (1 layer at 1024: 7.8 us, 8.9 us in splits of 32).
long long aligned_wg_tiles(long long total_positions, int max_len, int n_cu)
{
    const long long target = std::max(1, n_cu - n_cu / 16);
    long long s = (total_positions + target - 1) / target;
    if (s < 64) s = max_len <= 128 ? max_len : max_len <= 256 ? 32 : 64;
    s = std::min<long long>(s, max_len);
    s = std::min<long long>(std::max<long long>(s, 16), 4096);
    return (s + kDecodeTile - 1) / kDecodeTile;
}

long long balanced_wg_tiles(long long total_tiles, int n_cu)
{
    return std::max<long long>(4, (total_tiles + n_cu - 1) / n_cu);
}

}  // namespace

extern "C" {

const char* tla_last_error(void)
{
    return g_last_error;
}

int tla_abi_version(void)
{
    return 2;
}

int tla_engine_create(const tla_config* cfg, int device, tla_engine** out)
{
    if (!cfg || !out) return fail(TLA_ERR_INVALID_ARGUMENT, "cfg and out must not be NULL");
    *out = nullptr;
    if (cfg->n_layers < 1 || cfg->n_head < 1 || cfg->n_head_kv < 1 || cfg->n_embd < 1 || cfg->n_ctx < 1)
        return fail(TLA_ERR_INVALID_ARGUMENT,
                    "n_layers, n_head, n_head_kv, n_embd and n_ctx must be >= 1");
    if (cfg->n_embd % cfg->n_head != 0)
        return fail(TLA_ERR_INVALID_ARGUMENT, "n_embd (%d) is not a multiple of n_head (%d)",
                    cfg->n_embd, cfg->n_head);
    if (cfg->n_head % cfg->n_head_kv != 0)
        return fail(TLA_ERR_INVALID_ARGUMENT, "n_head (%d) is not a multiple of n_head_kv (%d)",
                    cfg->n_head, cfg->n_head_kv);
    if (!(cfg->rope_freq_base > 0.0f) || !std::isfinite(cfg->rope_freq_base))
        return fail(TLA_ERR_INVALID_ARGUMENT, "rope_freq_base must be finite and > 0");
    const int head_dim = cfg->n_embd / cfg->n_head;
    const int gqa = cfg->n_head / cfg->n_head_kv;
    if (head_dim != kHeadDim)
        return fail(TLA_ERR_UNSUPPORTED, "head_dim %d: kernels implement head_dim 64", head_dim);
    if (gqa > kMaxGqa)
        return fail(TLA_ERR_UNSUPPORTED, "n_head/n_head_kv = %d > %d", gqa, kMaxGqa);
    if (cfg->n_ctx > (1 << 24)) return fail(TLA_ERR_UNSUPPORTED, "n_ctx %d > 2^24", cfg->n_ctx);
    // The decode kernel addresses one (sequence, layer) cache slice with
    // 32-bit byte offsets below 2^31.
    if (static_cast<long long>(cfg->n_ctx) * cfg->n_head_kv * head_dim * 4 > (1ll << 31) - 256)
        return fail(TLA_ERR_UNSUPPORTED, "one layer's KV cache (n_ctx x kv_dim x 4 = %lld B) > 2 GiB",
                    static_cast<long long>(cfg->n_ctx) * cfg->n_head_kv * head_dim * 4);
    if (device < 0) return fail(TLA_ERR_INVALID_ARGUMENT, "device %d < 0", device);

    int n_dev = 0;
    TLA_HIP(hipGetDeviceCount(&n_dev));
    if (device >= n_dev) return fail(TLA_ERR_INVALID_ARGUMENT, "device %d of %d", device, n_dev);

    tla_engine* e = new tla_engine;
    e->cfg = *cfg;
    e->device = device;
    e->head_dim = head_dim;
    e->kv_dim = cfg->n_head_kv * head_dim;
    e->gqa = gqa;

    auto bail = [&](int rc) {
        tla_engine_destroy(e);
        return rc;
    };
    if (int rc = set_device(e)) return bail(rc);
    {
        hipError_t err = hipDeviceGetAttribute(&e->n_cu, hipDeviceAttributeMultiprocessorCount, device);
        if (err == hipSuccess && e->n_cu < 1) e->n_cu = 1;
        if (err == hipSuccess) err = hipStreamCreateWithFlags(&e->stream, hipStreamNonBlocking);
        if (err != hipSuccess)
            return bail(fail(TLA_ERR_DEVICE, "device query / stream: %s", hipGetErrorString(err)));
    }
    std::vector<float2> tab;
    rope_table_host(tab, cfg->n_ctx, head_dim, cfg->rope_freq_base);
    const size_t tab_bytes = tab.size() * sizeof(float2);
    hipError_t err = hipMalloc(&e->rope, tab_bytes);
    if (err == hipSuccess) err = hipMemcpy(e->rope, tab.data(), tab_bytes, hipMemcpyHostToDevice);
    if (err != hipSuccess)
        return bail(fail(err == hipErrorOutOfMemory ? TLA_ERR_OUT_OF_MEMORY : TLA_ERR_DEVICE,
                         "rope table: %s", hipGetErrorString(err)));
    if (int rc = scratch_setup(e)) return bail(rc);
    // Every kernel's code object is loaded now, not at its first launch (a
    // load allocates device memory: tla_decode_noalloc's first call would).
    for (hipError_t (*load)() : {load_decode_code, load_prefill_code, load_gemv_code, load_batch_code,
                                 load_small_ops_code}) {
        const hipError_t lerr = load();
        if (lerr != hipSuccess)
            return bail(fail(TLA_ERR_DEVICE, "loading kernel code: %s", hipGetErrorString(lerr)));
    }
    *out = e;
    return ok();
}

int tla_engine_destroy(tla_engine* e)
{
    if (!e) return TLA_OK;
    (void)hipSetDevice(e->device);
    if (e->stream) (void)hipStreamSynchronize(e->stream);
    for (auto& v : e->prof_pending)
        for (auto& pr : v) {
            (void)hipEventDestroy(pr.first);
            (void)hipEventDestroy(pr.second);
        }
    for (hipEvent_t ev : e->event_pool) (void)hipEventDestroy(ev);
    for (hipEvent_t ev : e->slots)
        if (ev) (void)hipEventDestroy(ev);
    if (e->ws) (void)hipFree(e->ws);
    if (e->counters) (void)hipFree(e->counters);
    if (e->fwd) (void)hipFree(e->fwd);
    if (e->xs) (void)hipFree(e->xs);
    if (e->part) (void)hipFree(e->part);
    if (e->kvp) (void)hipFree(e->kvp);
    if (e->argmax_slot) (void)hipFree(e->argmax_slot);
    if (e->amax_keys) (void)hipFree(e->amax_keys);
    if (e->rope) (void)hipFree(e->rope);
    if (e->stream) (void)hipStreamDestroy(e->stream);
    delete e;
    return TLA_OK;
}

int tla_synchronize(tla_engine* e)
{
    if (int rc = check_engine(e)) return rc;
    if (int rc = set_device(e)) return rc;
    TLA_HIP(hipStreamSynchronize(e->stream));
    return ok();
}

int tla_alloc(tla_engine* e, size_t bytes, void** out_dev)
{
    if (int rc = check_engine(e)) return rc;
    if (!out_dev) return fail(TLA_ERR_INVALID_ARGUMENT, "out_dev is NULL");
    *out_dev = nullptr;
    if (bytes == 0) return fail(TLA_ERR_INVALID_ARGUMENT, "zero-byte allocation");
    if (int rc = set_device(e)) return rc;
    void* p = nullptr;
    TLA_HIP(hipMalloc(&p, bytes));
    hipError_t err = hipMemsetAsync(p, 0, bytes, e->stream);
    if (err == hipSuccess) err = hipStreamSynchronize(e->stream);
    if (err != hipSuccess) {
        (void)hipFree(p);
        return fail(TLA_ERR_DEVICE, "zero fill: %s", hipGetErrorString(err));
    }
    *out_dev = p;
    return ok();
}

int tla_host_alloc(tla_engine* e, size_t bytes, void** out_host)
{
    if (int rc = check_engine(e)) return rc;
    if (!out_host) return fail(TLA_ERR_INVALID_ARGUMENT, "out_host is NULL");
    *out_host = nullptr;
    if (bytes == 0) return fail(TLA_ERR_INVALID_ARGUMENT, "zero-byte allocation");
    if (int rc = set_device(e)) return rc;
    void* p = nullptr;
    const hipError_t err = hipHostMalloc(&p, bytes, hipHostMallocDefault);
    if (err != hipSuccess)
        return fail(err == hipErrorOutOfMemory ? TLA_ERR_OUT_OF_MEMORY : TLA_ERR_DEVICE,
                    "pinned host allocation of %zu bytes: %s", bytes, hipGetErrorString(err));
    std::memset(p, 0, bytes);
    *out_host = p;
    return ok();
}

int tla_host_free(tla_engine* e, void* host)
{
    if (int rc = check_engine(e)) return rc;
    if (!host) return TLA_OK;
    if (int rc = set_device(e)) return rc;
    TLA_HIP(hipStreamSynchronize(e->stream));
    TLA_HIP(hipHostFree(host));
    return ok();
}

int tla_free(tla_engine* e, void* dev)
{
    if (int rc = check_engine(e)) return rc;
    if (!dev) return TLA_OK;
    if (int rc = set_device(e)) return rc;
    TLA_HIP(hipStreamSynchronize(e->stream));
    TLA_HIP(hipFree(dev));
    return ok();
}

int tla_kv_cache_alloc(tla_engine* e, int n_seq, float** key_cache_dev, float** value_cache_dev)
{
    if (int rc = check_engine(e)) return rc;
    if (!key_cache_dev || !value_cache_dev)
        return fail(TLA_ERR_INVALID_ARGUMENT, "output pointers must not be NULL");
    if (n_seq < 1) return fail(TLA_ERR_INVALID_ARGUMENT, "n_seq %d < 1", n_seq);
    const size_t bytes = static_cast<size_t>(n_seq) * e->cfg.n_layers * e->cfg.n_ctx * e->kv_dim *
                         sizeof(float);
    void* k = nullptr;
    void* v = nullptr;
    if (int rc = tla_alloc(e, bytes, &k)) return rc;
    if (int rc = tla_alloc(e, bytes, &v)) {
        tla_free(e, k);
        return rc;
    }
    *key_cache_dev = static_cast<float*>(k);
    *value_cache_dev = static_cast<float*>(v);
    return ok();
}

int tla_memcpy_h2d(tla_engine* e, void* dst_dev, const void* src_host, size_t bytes)
{
    if (int rc = check_engine(e)) return rc;
    if (bytes == 0) return TLA_OK;
    if (!dst_dev || !src_host) return fail(TLA_ERR_INVALID_ARGUMENT, "NULL pointer");
    if (int rc = set_device(e)) return rc;
    TLA_HIP(hipMemcpyAsync(dst_dev, src_host, bytes, hipMemcpyHostToDevice, e->stream));
    TLA_HIP(hipStreamSynchronize(e->stream));
    return ok();
}

int tla_memcpy_d2h(tla_engine* e, void* dst_host, const void* src_dev, size_t bytes)
{
    if (int rc = check_engine(e)) return rc;
    if (bytes == 0) return TLA_OK;
    if (!dst_host || !src_dev) return fail(TLA_ERR_INVALID_ARGUMENT, "NULL pointer");
    if (int rc = set_device(e)) return rc;
    TLA_HIP(hipMemcpyAsync(dst_host, src_dev, bytes, hipMemcpyDeviceToHost, e->stream));
    TLA_HIP(hipStreamSynchronize(e->stream));
    return ok();
}

int tla_memcpy_d2d(tla_engine* e, void* dst_dev, const void* src_dev, size_t bytes)
{
    if (int rc = check_engine(e)) return rc;
    if (bytes == 0) return TLA_OK;
    if (!dst_dev || !src_dev) return fail(TLA_ERR_INVALID_ARGUMENT, "NULL pointer");
    if (int rc = set_device(e)) return rc;
    const hipError_t err = launch_copy(dst_dev, src_dev, bytes, e->stream);
    if (err != hipSuccess) return fail(TLA_ERR_DEVICE, "copy launch: %s", hipGetErrorString(err));
    return ok();
}

int tla_rope(tla_engine* e, float* q_dev, float* k_dev, int pos, int head_dim, int n_head,
             int n_head_kv, float freq_base)
{
    if (int rc = check_engine(e)) return rc;
    if (!q_dev || !k_dev) return fail(TLA_ERR_INVALID_ARGUMENT, "q and k must not be NULL");
    if (pos < 0) return fail(TLA_ERR_OUT_OF_RANGE, "pos %d < 0", pos);
    if (head_dim < 2 || head_dim % 2 != 0 || head_dim / 2 > kMaxRopePairs)
        return fail(TLA_ERR_UNSUPPORTED, "head_dim %d (even, <= %d)", head_dim, 2 * kMaxRopePairs);
    if (n_head < 0 || n_head_kv < 0 || n_head + n_head_kv < 1)
        return fail(TLA_ERR_INVALID_ARGUMENT, "head counts %d, %d", n_head, n_head_kv);
    if (int rc = set_device(e)) return rc;
    RopeParams p{};
    p.q = q_dev;
    p.k = k_dev;
    p.n_head = n_head;
    p.n_head_kv = n_head_kv;
    p.head_dim = head_dim;
    rope_cos_sin(p.cs, pos, head_dim, freq_base);
    const hipError_t err = launch_rope(p, e->stream);
    if (err != hipSuccess) return fail(TLA_ERR_DEVICE, "rope launch: %s", hipGetErrorString(err));
    return ok();
}

int tla_softmax(tla_engine* e, float* x_dev, int size)
{
    if (int rc = check_engine(e)) return rc;
    if (!x_dev) return fail(TLA_ERR_INVALID_ARGUMENT, "x is NULL");
    if (size < 1) return fail(TLA_ERR_INVALID_ARGUMENT, "size %d < 1", size);
    if (int rc = set_device(e)) return rc;
    const hipError_t err = launch_softmax(x_dev, size, e->stream);
    if (err != hipSuccess) return fail(TLA_ERR_DEVICE, "softmax launch: %s", hipGetErrorString(err));
    return ok();
}

// ---- projections -------------------------------------------------------------

namespace {

// x vectors staged in LDS per launch: at most this many bytes, well inside a
// workgroup's share of the CU's LDS.
constexpr int kGemvLdsBytes = 60 * 1024;

// LDS bytes for one staged x vector: the floats, 4 floats of padding per 64
// and one sum per 16.
int gemv_lds_per_vec(int cols) { return (cols + cols / 8) * 4; }

int gemv_chunk(int n_seq, int cols)
{
    return std::max(1, std::min({n_seq, kGemvMaxVec, kGemvLdsBytes / gemv_lds_per_vec(cols)}));
}

// Shape and pointer checks shared by the matrix-vector entry points (and the
// model check, so that a NULL weight of any layer is an error, not a launch).
int check_gemv(int type, int cols, int n_vec, const void* w)
{
    if (!w) return fail(TLA_ERR_INVALID_ARGUMENT, "weight pointer is NULL");
    if (weight_row_bytes(type, cols) == 0 || (type != kQ6_K && cols % 32 != 0) ||
        (type == kQ6_K && cols % 256 != 0))
        return fail(TLA_ERR_INVALID_ARGUMENT, "weight type %d with %d columns", type, cols);
    if (cols < 64 || cols % 64 != 0 || gemv_lds_per_vec(cols) > kGemvLdsBytes)
        return fail(TLA_ERR_UNSUPPORTED, "cols %d: multiples of 64 up to %d are supported", cols,
                    kGemvLdsBytes / 288 * 64);
    if (static_cast<long long>(n_vec) * gemv_lds_per_vec(cols) > kGemvLdsBytes)
        return fail(TLA_ERR_UNSUPPORTED, "%d vectors of %d floats exceed %d bytes of LDS", n_vec,
                    cols, kGemvLdsBytes);
    if (reinterpret_cast<std::uintptr_t>(w) % 16 != 0)
        return fail(TLA_ERR_INVALID_ARGUMENT, "weights must be 16-byte aligned");
    return TLA_OK;
}

int run_gemv(tla_engine* e, int type, const GemvParams& p)
{
    if (p.rope) return launch(e, TLA_KERNEL_GEMV, "gemv", [&] { return launch_gemv(type, p, e->stream); });
    GemvParams q = p;
    q.rope = e->rope;  // read by every launch; rotates nothing with rope_rows = 0
    return launch(e, TLA_KERNEL_GEMV, "gemv", [&] { return launch_gemv(type, q, e->stream); });
}

}  // namespace

int tla_matmul(tla_engine* e, float* out_dev, const void* w_dev, const float* x_dev, int rows,
               int cols, int type)
{
    if (int rc = check_engine(e)) return rc;
    if (!out_dev || !w_dev || !x_dev) return fail(TLA_ERR_INVALID_ARGUMENT, "NULL device pointer");
    if (rows < 1) return fail(TLA_ERR_INVALID_ARGUMENT, "rows %d < 1", rows);
    if (int rc = check_gemv(type, cols, 1, w_dev)) return rc;
    if (int rc = set_device(e)) return rc;
    GemvParams p{};
    p.seg[0] = {static_cast<const unsigned char*>(w_dev), out_dev, rows, 0};
    p.n_seg = 1;
    p.total_rows = rows;
    p.cols = cols;
    p.row_bytes = static_cast<int>(weight_row_bytes(type, cols));
    p.n_vec = 1;
    p.x = x_dev;
    p.x_stride = cols;
    if (int rc = run_gemv(e, type, p)) return rc;
    return ok();
}

int tla_rmsnorm(tla_engine* e, float* out_dev, const float* x_dev, const float* weight_dev,
                int size, float eps)
{
    if (int rc = check_engine(e)) return rc;
    if (!out_dev || !x_dev || !weight_dev) return fail(TLA_ERR_INVALID_ARGUMENT, "NULL device pointer");
    if (size < 1) return fail(TLA_ERR_INVALID_ARGUMENT, "size %d < 1", size);
    if (int rc = set_device(e)) return rc;
    const hipError_t err = launch_rmsnorm(out_dev, x_dev, weight_dev, size, eps, e->stream);
    if (err != hipSuccess) return fail(TLA_ERR_DEVICE, "rmsnorm launch: %s", hipGetErrorString(err));
    return ok();
}

int tla_vec_add(tla_engine* e, float* out_dev, const float* x_dev, int size)
{
    if (int rc = check_engine(e)) return rc;
    if (!out_dev || !x_dev) return fail(TLA_ERR_INVALID_ARGUMENT, "NULL device pointer");
    if (size < 1) return fail(TLA_ERR_INVALID_ARGUMENT, "size %d < 1", size);
    if (int rc = set_device(e)) return rc;
    const hipError_t err = launch_vec_add(out_dev, x_dev, size, e->stream);
    if (err != hipSuccess) return fail(TLA_ERR_DEVICE, "vec_add launch: %s", hipGetErrorString(err));
    return ok();
}

int tla_attn_qkv(tla_engine* e, int n_seq, float* q_dev, float* k_dev, float* v_dev,
                 const float* x_dev, const float* norm_w_dev, float eps, const void* wq_dev,
                 const void* wk_dev, const void* wv_dev, int type)
{
    if (int rc = check_engine(e)) return rc;
    if (!q_dev || !k_dev || !v_dev || !x_dev || !wq_dev || !wk_dev || !wv_dev)
        return fail(TLA_ERR_INVALID_ARGUMENT, "NULL device pointer");
    if (n_seq < 1) return fail(TLA_ERR_INVALID_ARGUMENT, "n_seq %d < 1", n_seq);
    const int embd = e->cfg.n_embd, kv = e->kv_dim;
    const int chunk = gemv_chunk(n_seq, embd);
    if (int rc = check_gemv(type, embd, chunk, wq_dev)) return rc;
    if (reinterpret_cast<std::uintptr_t>(wk_dev) % 16 || reinterpret_cast<std::uintptr_t>(wv_dev) % 16)
        return fail(TLA_ERR_INVALID_ARGUMENT, "weights must be 16-byte aligned");
    if (int rc = set_device(e)) return rc;
    for (int s0 = 0; s0 < n_seq; s0 += chunk) {
        const int nv = std::min(chunk, n_seq - s0);
        GemvParams p{};
        p.seg[0] = {static_cast<const unsigned char*>(wq_dev), q_dev + static_cast<long long>(s0) * embd, embd, embd};
        p.seg[1] = {static_cast<const unsigned char*>(wk_dev), k_dev + static_cast<long long>(s0) * kv, kv, kv};
        p.seg[2] = {static_cast<const unsigned char*>(wv_dev), v_dev + static_cast<long long>(s0) * kv, kv, kv};
        p.n_seg = 3;
        p.total_rows = embd + 2 * kv;
        p.cols = embd;
        p.row_bytes = static_cast<int>(weight_row_bytes(type, embd));
        p.n_vec = nv;
        p.x = x_dev + static_cast<long long>(s0) * embd;
        p.x_stride = embd;
        p.norm_w = norm_w_dev;
        p.eps = eps;
        if (int rc = run_gemv(e, type, p)) return rc;
    }
    return ok();
}

int tla_attn_out(tla_engine* e, int n_seq, float* x_dev, const void* wo_dev, const float* xb2_dev,
                 int type)
{
    if (int rc = check_engine(e)) return rc;
    if (!x_dev || !wo_dev || !xb2_dev) return fail(TLA_ERR_INVALID_ARGUMENT, "NULL device pointer");
    if (n_seq < 1) return fail(TLA_ERR_INVALID_ARGUMENT, "n_seq %d < 1", n_seq);
    const int embd = e->cfg.n_embd;
    const int chunk = gemv_chunk(n_seq, embd);
    if (int rc = check_gemv(type, embd, chunk, wo_dev)) return rc;
    if (int rc = set_device(e)) return rc;
    for (int s0 = 0; s0 < n_seq; s0 += chunk) {
        const int nv = std::min(chunk, n_seq - s0);
        GemvParams p{};
        p.seg[0] = {static_cast<const unsigned char*>(wo_dev), x_dev + static_cast<long long>(s0) * embd, embd, embd};
        p.n_seg = 1;
        p.total_rows = embd;
        p.cols = embd;
        p.row_bytes = static_cast<int>(weight_row_bytes(type, embd));
        p.n_vec = nv;
        p.x = xb2_dev + static_cast<long long>(s0) * embd;
        p.x_stride = embd;
        p.add = 1;
        if (int rc = run_gemv(e, type, p)) return rc;
    }
    return ok();
}

}  // extern "C"

namespace {

// tla_decode, with the split partials and counters in the engine's workspace
// (grown on demand) or, with fixed_scratch, in the device's static scratch
// (no allocation; launches that need more than it holds are rejected).
int decode_impl(tla_engine* e, bool fixed_scratch, int n_seq, const int* pos_host, int layer0,
                int n_step_layers, int flags, float* out_dev, const float* q_dev, const float* k_dev,
                const float* v_dev, float* key_cache_dev, float* value_cache_dev, size_t seq_stride)
{
    if (int rc = check_engine(e)) return rc;
    const tla_config& c = e->cfg;
    if (n_seq < 1 || n_seq > kMaxSeqPerLaunch)
        return fail(TLA_ERR_INVALID_ARGUMENT, "n_seq %d not in [1, %d]", n_seq, kMaxSeqPerLaunch);
    if (!pos_host) return fail(TLA_ERR_INVALID_ARGUMENT, "pos is NULL");
    const bool in_cache = (flags & TLA_KV_IN_CACHE) != 0;
    if (!out_dev || !q_dev || (!in_cache && (!k_dev || !v_dev)) || !key_cache_dev || !value_cache_dev)
        return fail(TLA_ERR_INVALID_ARGUMENT, "NULL device pointer");
    if (flags & ~(TLA_ROTATE | TLA_KV_IN_CACHE))
        return fail(TLA_ERR_INVALID_ARGUMENT, "unknown flags 0x%x", flags);
    if (n_step_layers < 1) return fail(TLA_ERR_INVALID_ARGUMENT, "n_step_layers %d < 1", n_step_layers);
    if (layer0 < 0 || layer0 + n_step_layers > c.n_layers)
        return fail(TLA_ERR_OUT_OF_RANGE, "layers [%d, %d) outside [0, %d)", layer0,
                    layer0 + n_step_layers, c.n_layers);
    const long long layer_stride = static_cast<long long>(c.n_ctx) * e->kv_dim;
    if (n_seq > 1 && seq_stride < static_cast<size_t>(layer_stride) * c.n_layers)
        return fail(TLA_ERR_INVALID_ARGUMENT, "seq_stride %zu < n_layers*n_ctx*kv_dim", seq_stride);

    DecodeParams p{};
    DecodeSeqs<kMaxSeqPerLaunch> seqs{};
    for (int s = 0; s < n_seq; ++s) {
        const int pos = pos_host[s];
        if (pos < 0 || pos >= c.n_ctx)
            return fail(TLA_ERR_OUT_OF_RANGE, "pos[%d] = %d outside [0, n_ctx=%d)", s, pos, c.n_ctx);
        seqs.seq_id[s] = s;
    }
    // Ranks by length, longest first (ties in caller order); the flat tile
    // space lays out each rank's n_step_layers units in turn.  An insertion
    // sort in place: stable, and no temporary buffer.
    for (int i = 1; i < n_seq; ++i) {
        const int id = seqs.seq_id[i];
        int j = i;
        for (; j > 0 && pos_host[seqs.seq_id[j - 1]] < pos_host[id]; --j) seqs.seq_id[j] = seqs.seq_id[j - 1];
        seqs.seq_id[j] = id;
    }
    long long total_positions = 0, real_tiles = 0;
    for (int r = 0; r < n_seq; ++r) {
        seqs.pos[r] = pos_host[seqs.seq_id[r]];
        total_positions += static_cast<long long>(seqs.pos[r] + 1) * n_step_layers;
        real_tiles += static_cast<long long>(seqs.pos[r] / kDecodeTile + 1) * n_step_layers;
    }
    const long long a_tiles = aligned_wg_tiles(total_positions, seqs.pos[0] + 1, e->n_cu);
    long long a_groups = 0;  // workgroups of the aligned plan
    for (int r = 0; r < n_seq; ++r)
        a_groups += (seqs.pos[r] / kDecodeTile + a_tiles) / a_tiles * n_step_layers;
    const long long b_tiles = balanced_wg_tiles(real_tiles, e->n_cu);
    const long long min_unit = seqs.pos[n_seq - 1] / kDecodeTile + 1;  // shortest rank
    int aligned = e->opt_plan == TLA_PLAN_ALIGNED;
    if (e->opt_plan == TLA_PLAN_AUTO) aligned = a_groups <= e->n_cu || b_tiles > min_unit;
    long long wg = aligned ? a_tiles : b_tiles;
    if (e->opt_split > 0) wg = (e->opt_split + kDecodeTile - 1) / kDecodeTile;
    wg = std::min(wg, real_tiles);
    const int wg_tiles = static_cast<int>(wg);
    // Flat layout; splits of a unit = workgroup ranges it meets.
    long long total_tiles = 0;
    int max_splits = 1;
    for (int r = 0; r < n_seq; ++r) {
        const long long unit_tiles = seqs.pos[r] / kDecodeTile + 1;
        const long long span = aligned ? (unit_tiles + wg - 1) / wg * wg : unit_tiles;
        seqs.tile_prefix[r] = static_cast<int>(total_tiles);
        for (int lb = 0; lb < n_step_layers; ++lb) {
            const long long u0 = total_tiles + lb * span;
            max_splits = std::max(max_splits,
                                  static_cast<int>((u0 + unit_tiles - 1) / wg - u0 / wg + 1));
        }
        total_tiles += span * n_step_layers;
        if (total_tiles > 0x3fffffffLL) return fail(TLA_ERR_UNSUPPORTED, "too many positions");
    }
    seqs.tile_prefix[n_seq] = static_cast<int>(total_tiles);
    if (int rc = set_device(e)) return rc;

    // Kv heads per workgroup (two waves each).  Same-box A/B with 1 / 2 / 4:
    // 1 layer at 128 positions 7.3 / 8.2 / 10.6 us and 22 x 2048 23.05 /
    // 23.4 / 24.2 us (one round of ranges of at most 256 positions: 1);
    // 64 ragged sequences, several rounds, 626 / 600 / 607 us (2); 22 x 4096
    // (376-position ranges) 39.8 / 40.9 / 40.0 us and 22 x 16384 136 /
    // 135.7 / 131.9 us (4, which streams whole 1 KiB position rows; the
    // balanced plan always).
    const long long ranges = (total_tiles + wg - 1) / wg;
    const int kv_group = !aligned                    ? kDecodeKvGroupLarge
                         : e->opt_group > 0           ? e->opt_group
                         : ranges > e->n_cu           ? kDecodeKvGroupMid
                         : wg * kDecodeTile <= 256    ? kDecodeKvGroupSmall
                                                      : kDecodeKvGroupLarge;
    const long long units = static_cast<long long>(n_seq) * n_step_layers;
    const int n_groups = (c.n_head_kv + kv_group - 1) / kv_group;
    if (max_splits > 1) {
        // per (unit, split, kv head): 64 output floats + max + sum for each real head
        const size_t bytes = decode_part_bytes(units, max_splits, c.n_head_kv, e->gqa);
        const size_t n_counters = static_cast<size_t>(units * n_groups);
        if (fixed_scratch) {
            if (!e->scratch)
                return fail(TLA_ERR_UNSUPPORTED, "device %d has no static split scratch", e->device);
            if (bytes > kScratchPartBytes || n_counters > kScratchCounters)
                return fail(TLA_ERR_UNSUPPORTED,
                            "this launch needs %zu bytes of split partials and %zu counters; the static "
                            "scratch holds %zu bytes and %zu counters (use tla_decode, or fewer "
                            "sequences / layers per call)",
                            bytes, n_counters, kScratchPartBytes, kScratchCounters);
            p.part = static_cast<float*>(e->scratch);
            p.counters = reinterpret_cast<int*>(static_cast<char*>(e->scratch) + kScratchPartBytes);
        } else {
            if (int rc = ensure_ws(e, bytes)) return rc;
            if (int rc = ensure_counters(e, n_counters)) return rc;
            p.part = static_cast<float*>(e->ws);
            p.counters = e->counters;
        }
    }
    p.q = q_dev;
    p.k = k_dev;
    p.v = v_dev;
    p.out = out_dev;
    p.kc = key_cache_dev;
    p.vc = value_cache_dev;
    p.rope = e->rope;
    p.seq_stride = static_cast<long long>(seq_stride);
    p.layer_stride = layer_stride;
    p.n_seq = n_seq;
    p.n_lb = n_step_layers;
    p.layer0 = layer0;
    p.n_head = c.n_head;
    p.n_head_kv = c.n_head_kv;
    p.gqa = e->gqa;
    p.wg_tiles = wg_tiles;
    p.max_splits = max_splits;
    p.total_tiles = static_cast<int>(total_tiles);
    p.aligned = aligned;
    p.rotate = (flags & TLA_ROTATE) ? 1 : 0;
    p.in_cache = in_cache ? 1 : 0;
    p.kv_group = kv_group;
    p.scale_log2 = scale_log2(e->head_dim);
    p.n_groups = n_groups;

    if (int rc = launch(e, TLA_KERNEL_DECODE, "decode",
                        [&] { return launch_decode(p, seqs, e->stream); }))
        return rc;
    return ok();
}

}  // namespace

extern "C" {

int tla_decode(tla_engine* e, int n_seq, const int* pos_host, int layer0, int n_step_layers,
               int flags, float* out_dev, const float* q_dev, const float* k_dev,
               const float* v_dev, float* key_cache_dev, float* value_cache_dev,
               size_t seq_stride)
{
    return decode_impl(e, false, n_seq, pos_host, layer0, n_step_layers, flags, out_dev, q_dev, k_dev,
                       v_dev, key_cache_dev, value_cache_dev, seq_stride);
}

int tla_decode_noalloc(tla_engine* e, int n_seq, const int* pos_host, int layer0, int n_step_layers,
                       int flags, float* out_dev, const float* q_dev, const float* k_dev,
                       const float* v_dev, float* key_cache_dev, float* value_cache_dev,
                       size_t seq_stride)
{
    return decode_impl(e, true, n_seq, pos_host, layer0, n_step_layers, flags, out_dev, q_dev, k_dev,
                       v_dev, key_cache_dev, value_cache_dev, seq_stride);
}

int tla_attention(tla_engine* e, float* out_dev, const float* q_dev, const float* k_dev,
                  const float* v_dev, float* key_cache_dev, float* value_cache_dev, float* att,
                  int layer, int pos)
{
    (void)att;
    return tla_decode(e, 1, &pos, layer, 1, 0, out_dev, q_dev, k_dev, v_dev, key_cache_dev,
                      value_cache_dev, 0);
}

int tla_rope_attention(tla_engine* e, float* out_dev, const float* q_dev, const float* k_dev,
                       const float* v_dev, float* key_cache_dev, float* value_cache_dev, int layer,
                       int pos)
{
    return tla_decode(e, 1, &pos, layer, 1, TLA_ROTATE, out_dev, q_dev, k_dev, v_dev,
                      key_cache_dev, value_cache_dev, 0);
}

int tla_rope_attention_host(tla_engine* e, float* out_host, const float* qkv_host, float* qkv_dev,
                            float* out_dev, float* key_cache_dev, float* value_cache_dev, int layer,
                            int pos)
{
    if (int rc = check_engine(e)) return rc;
    if (!out_host || !qkv_host) return fail(TLA_ERR_INVALID_ARGUMENT, "NULL host pointer");
    if (!qkv_dev || !out_dev || !key_cache_dev || !value_cache_dev)
        return fail(TLA_ERR_INVALID_ARGUMENT, "NULL device pointer");
    if (int rc = set_device(e)) return rc;
    const size_t q_floats = static_cast<size_t>(e->cfg.n_head) * e->head_dim;
    const size_t qkv_bytes = (q_floats + 2 * static_cast<size_t>(e->kv_dim)) * sizeof(float);
    TLA_HIP(hipMemcpyAsync(qkv_dev, qkv_host, qkv_bytes, hipMemcpyHostToDevice, e->stream));
    const float* dq = qkv_dev;
    const float* dk = dq + q_floats;
    const float* dv = dk + e->kv_dim;
    if (int rc = tla_decode(e, 1, &pos, layer, 1, TLA_ROTATE, out_dev, dq, dk, dv, key_cache_dev,
                            value_cache_dev, 0)) {
        (void)hipStreamSynchronize(e->stream);  // the upload may still read qkv_host
        return rc;
    }
    TLA_HIP(hipMemcpyAsync(out_host, out_dev, q_floats * sizeof(float), hipMemcpyDeviceToHost, e->stream));
    TLA_HIP(hipStreamSynchronize(e->stream));
    return ok();
}

namespace {

// Grows a workspace to `bytes` (after the stream's queued work, which may
// still read it).
int ensure_buf(tla_engine* e, void** buf, size_t& have, size_t bytes, const char* what)
{
    if (bytes <= have) return TLA_OK;
    TLA_HIP(hipStreamSynchronize(e->stream));
    if (*buf) TLA_HIP(hipFree(*buf));
    *buf = nullptr;
    have = 0;
    const hipError_t err = hipMalloc(buf, bytes);
    if (err != hipSuccess)
        return fail(err == hipErrorOutOfMemory ? TLA_ERR_OUT_OF_MEMORY : TLA_ERR_DEVICE, "%s (%zu bytes): %s",
                    what, bytes, hipGetErrorString(err));
    have = bytes;
    return TLA_OK;
}

}  // namespace

int tla_prefill(tla_engine* e, int pos0, int n_tok, int layer0, int n_step_layers, int flags,
                float* out_dev, const float* q_dev, const float* k_dev, const float* v_dev,
                float* key_cache_dev, float* value_cache_dev)
{
    if (int rc = check_engine(e)) return rc;
    const tla_config& c = e->cfg;
    if (!out_dev || !q_dev || !k_dev || !v_dev || !key_cache_dev || !value_cache_dev)
        return fail(TLA_ERR_INVALID_ARGUMENT, "NULL device pointer");
    if (flags & ~TLA_ROTATE) return fail(TLA_ERR_INVALID_ARGUMENT, "unknown flags 0x%x", flags);
    if (n_tok < 1) return fail(TLA_ERR_INVALID_ARGUMENT, "n_tok %d < 1", n_tok);
    if (pos0 < 0 || static_cast<long long>(pos0) + n_tok > c.n_ctx)
        return fail(TLA_ERR_OUT_OF_RANGE, "positions [%d, %lld) outside [0, n_ctx=%d)", pos0,
                    static_cast<long long>(pos0) + n_tok, c.n_ctx);
    if (n_step_layers < 1) return fail(TLA_ERR_INVALID_ARGUMENT, "n_step_layers %d < 1", n_step_layers);
    if (layer0 < 0 || layer0 + n_step_layers > c.n_layers)
        return fail(TLA_ERR_OUT_OF_RANGE, "layers [%d, %d) outside [0, %d)", layer0,
                    layer0 + n_step_layers, c.n_layers);
    if (int rc = set_device(e)) return rc;
    PrefillParams p{};
    p.q = q_dev;
    p.k = k_dev;
    p.v = v_dev;
    p.out = out_dev;
    p.kc = key_cache_dev;
    p.vc = value_cache_dev;
    p.rope = e->rope;
    p.layer_stride = static_cast<long long>(c.n_ctx) * e->kv_dim;
    p.n_lb = n_step_layers;
    p.layer0 = layer0;
    p.pos0 = pos0;
    p.n_tok = n_tok;
    p.n_head = c.n_head;
    p.n_head_kv = c.n_head_kv;
    p.gqa = e->gqa;
    p.rotate = (flags & TLA_ROTATE) ? 1 : 0;
    p.scale_log2 = scale_log2(e->head_dim);
    p.n_ptiles = (pos0 + n_tok + 31) / 32;
    if (int rc = ensure_buf(e, reinterpret_cast<void**>(&e->kvp), e->kvp_bytes,
                            prefill_planes_bytes(n_step_layers, c.n_head_kv, pos0, n_tok), "prefill K/V planes"))
        return rc;
    p.kvp = e->kvp;
    if (int rc = launch(e, TLA_KERNEL_APPEND, "prefill append",
                        [&] { return launch_prefill_append(p, e->stream); }))
        return rc;
    if (int rc = launch(e, TLA_KERNEL_PREFILL, "prefill attention",
                        [&] { return launch_prefill_attention(p, e->stream); }))
        return rc;
    return ok();
}

// ---- FFN, embedding, sampling, the whole forward pass ------------------------

namespace {

int elementwise_check(tla_engine* e, const void* a, const void* b, int size)
{
    if (int rc = check_engine(e)) return rc;
    if (!a || !b) return fail(TLA_ERR_INVALID_ARGUMENT, "NULL device pointer");
    if (size < 1) return fail(TLA_ERR_INVALID_ARGUMENT, "size %d < 1", size);
    return set_device(e);
}

int check_hip(hipError_t err, const char* what)
{
    if (err != hipSuccess) return fail(TLA_ERR_DEVICE, "%s launch: %s", what, hipGetErrorString(err));
    return TLA_OK;
}

// One GEMV launch over a single matrix: out (+)= W . f(x), f = the SwiGLU
// and / or rmsnorm prologues.
int gemv1(tla_engine* e, int type, const void* w, float* out, int rows, int cols, const float* x,
          const float* x2, const float* norm_w, float eps, int add)
{
    GemvParams p{};
    p.seg[0] = {static_cast<const unsigned char*>(w), out, rows, rows};
    p.n_seg = 1;
    p.total_rows = rows;
    p.cols = cols;
    p.row_bytes = static_cast<int>(weight_row_bytes(type, cols));
    p.n_vec = 1;
    p.x = x;
    p.x_stride = cols;
    p.x2 = x2;
    p.norm_w = norm_w;
    p.eps = eps;
    p.add = add;
    return run_gemv(e, type, p);
}

bool aligned16(const void* p) { return reinterpret_cast<std::uintptr_t>(p) % 16 == 0; }

// Shapes, types and pointers of a model against the engine's config.
int check_model(const tla_engine* e, const tla_model* m)
{
    if (!m || !m->layers) return fail(TLA_ERR_INVALID_ARGUMENT, "model or its layer array is NULL");
    const int embd = e->cfg.n_embd, kv = e->kv_dim;
    if (m->n_ff < 1 || m->n_vocab < 1) return fail(TLA_ERR_INVALID_ARGUMENT, "n_ff, n_vocab must be >= 1");
    if (!m->token_embd || !m->output_norm || !m->output)
        return fail(TLA_ERR_INVALID_ARGUMENT, "NULL embedding, output norm or classifier");
    if (weight_row_bytes(m->type_embd, embd) == 0)
        return fail(TLA_ERR_INVALID_ARGUMENT, "token_embd type %d", m->type_embd);
    if (m->type_embd == kQ6_K ? embd % 256 : embd % 32)
        return fail(TLA_ERR_INVALID_ARGUMENT, "n_embd %d is not whole blocks of type %d", embd,
                    m->type_embd);
    if (int rc = check_gemv(m->type_output, embd, 1, m->output)) return rc;
    for (int l = 0; l < e->cfg.n_layers; ++l) {
        const tla_layer_weights& L = m->layers[l];
        if (!L.attn_norm || !L.ffn_norm)
            return fail(TLA_ERR_INVALID_ARGUMENT, "layer %d: NULL norm weight", l);
        if (int rc = check_gemv(L.type_q, embd, 1, L.wq)) return rc;
        if (int rc = check_gemv(L.type_k, embd, 1, L.wk)) return rc;
        if (int rc = check_gemv(L.type_v, embd, 1, L.wv)) return rc;
        if (int rc = check_gemv(L.type_o, embd, 1, L.wo)) return rc;
        if (int rc = check_gemv(L.type_ffn, embd, 1, L.w_gate)) return rc;
        if (int rc = check_gemv(L.type_ffn, embd, 1, L.w_up)) return rc;
        if (int rc = check_gemv(L.type_ffn, m->n_ff, 1, L.w_down)) return rc;
        (void)kv;
    }
    return TLA_OK;
}

// Engine scratch for forward() over `rows` tokens at once: x | xb | q | att
// [rows][n_embd], k | v [rows][kv_dim], hb [rows][2][n_ff] (gate, up),
// logits [n_vocab] floats, then n_ints ints.
struct FwdBufs {
    float *x, *xb, *q, *k, *v, *att, *hb, *hb2, *logits;
    float* parts;  // [kAttnOutMaxParts][n_embd]: the fused attention + W_o launch's partials
    int* tokens;
    unsigned long long* amax;  // [n_amax rows][kAmaxSlots]: argmax keys of generated tokens
};

int fwd_bufs(tla_engine* e, const tla_model* m, int rows, int n_ints, FwdBufs* b, int n_amax = 0)
{
    const size_t embd = e->cfg.n_embd, kv = e->kv_dim, ff = m->n_ff, nv = m->n_vocab;
    const size_t r = static_cast<size_t>(rows);
    const size_t parts_at = (r * (4 * embd + 2 * kv + 2 * ff) + nv + 63) / 64 * 64;  // 256-byte aligned
    const size_t floats = parts_at + kAttnOutMaxParts * embd;
    const size_t ints_at = (floats * sizeof(float) + 255) / 256 * 256;
    const size_t amax_at = (ints_at + (n_ints + 1) * sizeof(int) + 255) / 256 * 256;
    const size_t bytes = amax_at + static_cast<size_t>(n_amax) * kAmaxSlots * sizeof(unsigned long long);
    if (bytes > e->fwd_bytes) {
        TLA_HIP(hipStreamSynchronize(e->stream));
        if (e->fwd) TLA_HIP(hipFree(e->fwd));
        e->fwd = nullptr;
        e->fwd_bytes = 0;
        const hipError_t err = hipMalloc(&e->fwd, bytes);
        if (err != hipSuccess)
            return fail(TLA_ERR_OUT_OF_MEMORY, "forward scratch: %s", hipGetErrorString(err));
        e->fwd_bytes = bytes;
    }
    float* f = static_cast<float*>(e->fwd);
    b->x = f;
    b->xb = b->x + r * embd;
    b->q = b->xb + r * embd;
    b->att = b->q + r * embd;
    b->k = b->att + r * embd;
    b->v = b->k + r * kv;
    b->hb = b->v + r * kv;
    b->hb2 = b->hb + ff;  // row 0's up projection; row t's gate at hb + 2*n_ff*t
    b->logits = b->hb + r * 2 * ff;
    b->parts = f + parts_at;
    b->tokens = reinterpret_cast<int*>(static_cast<char*>(e->fwd) + ints_at);
    b->amax = reinterpret_cast<unsigned long long*>(static_cast<char*>(e->fwd) + amax_at);
    return TLA_OK;
}

// One forward() step: the token from `token`, from token_dev when that is
// non-null, or from the argmax keys at token_amax when that is non-null
// (then also stored at token_out); logits written when `logits` is
// non-null, with their argmax keys posted to logits_amax (kAmaxSlots keys,
// zero before) when that is non-null.
int forward_step(tla_engine* e, const tla_model* m, const FwdBufs& b, float* kc, float* vc,
                 int token, const int* token_dev, int pos, float* logits,
                 const unsigned long long* token_amax = nullptr, int* token_out = nullptr,
                 unsigned long long* logits_amax = nullptr)
{
    const int embd = e->cfg.n_embd, kv = e->kv_dim, ff = m->n_ff;
    const float eps = m->rms_norm_eps;
    if (int rc = check_hip(launch_embed(m->type_embd, b.x, static_cast<const unsigned char*>(m->token_embd),
                                        token, token_dev, 1, embd, e->stream, token_amax, token_out),
                           "embed"))
        return rc;
    for (int l = 0; l < e->cfg.n_layers; ++l) {
        const tla_layer_weights& L = m->layers[l];
        // rmsnorm + Q/K/V (src/forward.cpp:180-190): one launch when the
        // three share a type.  Where the rows allow it, the launch's epilogue
        // also applies RoPE to q and k and writes k and v straight into the
        // cache row at pos (src/forward.cpp:192-196, src/ops.cpp:1370-1371),
        // so the attention launch only attends.
        const bool fused = L.type_q == L.type_k && L.type_q == L.type_v;
        const bool rope_in_gemv = fused && gemv_can_rope(embd);
        if (fused) {
            const long long row = static_cast<long long>(l) * e->cfg.n_ctx * kv + static_cast<long long>(pos) * kv;
            GemvParams p{};
            p.seg[0] = {static_cast<const unsigned char*>(L.wq), b.q, embd, embd};
            p.seg[1] = {static_cast<const unsigned char*>(L.wk), rope_in_gemv ? kc + row : b.k, kv, kv};
            p.seg[2] = {static_cast<const unsigned char*>(L.wv), rope_in_gemv ? vc + row : b.v, kv, kv};
            if (rope_in_gemv) {
                p.rope = e->rope + static_cast<long long>(pos) * (e->head_dim / 2);
                p.rope_rows = embd + kv;
            }
            p.n_seg = 3;
            p.total_rows = embd + 2 * kv;
            p.cols = embd;
            p.row_bytes = static_cast<int>(weight_row_bytes(L.type_q, embd));
            p.n_vec = 1;
            p.x = b.x;
            p.x_stride = embd;
            p.norm_w = L.attn_norm;
            p.eps = eps;
            if (int rc = run_gemv(e, L.type_q, p)) return rc;
        } else {
            if (int rc = check_hip(launch_rmsnorm(b.xb, b.x, L.attn_norm, embd, eps, e->stream), "rmsnorm"))
                return rc;
            if (int rc = gemv1(e, L.type_q, L.wq, b.q, embd, embd, b.xb, nullptr, nullptr, 0.f, 0)) return rc;
            if (int rc = gemv1(e, L.type_k, L.wk, b.k, kv, embd, b.xb, nullptr, nullptr, 0.f, 0)) return rc;
            if (int rc = gemv1(e, L.type_v, L.wv, b.v, kv, embd, b.xb, nullptr, nullptr, 0.f, 0)) return rc;
        }
        // Attention and x += Wo . att (src/forward.cpp:198-213).  Over a
        // context of at most kAttnOutMaxPos positions, one launch: the
        // partials of W_o per kv head, which the FFN launches add to x (x
        // itself is not written here).
        const int gqa = e->cfg.n_head / e->cfg.n_head_kv;
        const bool fused_out = rope_in_gemv && gemv_can_add_parts(ff) &&
                               attn_out_supported(L.type_o, gqa, e->cfg.n_head_kv, pos + 1);
        if (fused_out) {
            const long long layer = static_cast<long long>(l) * e->cfg.n_ctx * kv;
            AttnOutParams a{};
            a.q = b.q;
            a.kc = kc + layer;
            a.vc = vc + layer;
            a.n_pos = pos + 1;
            a.kv_dim = kv;
            a.gqa = gqa;
            a.n_head_kv = e->cfg.n_head_kv;
            a.w = static_cast<const unsigned char*>(L.wo);
            a.row_bytes = weight_row_bytes(L.type_o, embd);
            a.group_bytes = weight_row_bytes(L.type_o, 64 * gqa);
            a.rows = embd;
            a.parts = b.parts;
            if (int rc = launch(e, TLA_KERNEL_DECODE, "attention + W_o",
                                [&] { return launch_attn_out(L.type_o, a, e->stream); }))
                return rc;
        } else {
            // RoPE + append + attention
            if (int rc = tla_decode(e, 1, &pos, l, 1, rope_in_gemv ? TLA_KV_IN_CACHE : TLA_ROTATE, b.att, b.q,
                                    b.k, b.v, kc, vc, 0))
                return rc;
            if (int rc = gemv1(e, L.type_o, L.wo, b.x, embd, embd, b.att, nullptr, nullptr, 0.f, 1)) return rc;
        }
        // rmsnorm + gate and up projections, then SiLU x up, W_down and the
        // residual (src/forward.cpp:215-228, src/ops.cpp:1535-1564).  SiLU x
        // up is the gate/up launch's epilogue where the format pairs rows
        // (computed once), else the down projection's prologue.
        const bool paired = gemv_can_pair(L.type_ffn, ff, embd);
        {
            GemvParams p{};
            p.seg[0] = {static_cast<const unsigned char*>(L.w_gate), b.hb, ff, ff};
            p.seg[1] = {static_cast<const unsigned char*>(L.w_up), b.hb2, ff, ff};
            p.n_seg = 2;
            p.total_rows = 2 * ff;
            p.cols = embd;
            p.row_bytes = static_cast<int>(weight_row_bytes(L.type_ffn, embd));
            p.n_vec = 1;
            p.x = b.x;
            p.x_stride = embd;
            p.norm_w = L.ffn_norm;
            p.eps = eps;
            p.pair = paired ? 1 : 0;
            if (fused_out) {
                p.xparts = b.parts;
                p.n_parts = e->cfg.n_head_kv;
            }
            if (int rc = run_gemv(e, L.type_ffn, p)) return rc;
        }
        {
            GemvParams p{};
            p.seg[0] = {static_cast<const unsigned char*>(L.w_down), b.x, embd, embd};
            p.n_seg = 1;
            p.total_rows = embd;
            p.cols = ff;
            p.row_bytes = static_cast<int>(weight_row_bytes(L.type_ffn, ff));
            p.n_vec = 1;
            p.x = b.hb;
            p.x_stride = ff;
            p.x2 = paired ? nullptr : b.hb2;
            p.add = 1;
            if (fused_out) {
                p.rparts = b.parts;
                p.n_parts = e->cfg.n_head_kv;
            }
            if (int rc = run_gemv(e, L.type_ffn, p)) return rc;
        }
    }
    // final rmsnorm + classifier (src/forward.cpp:241-265), with the
    // logits' argmax keys where asked (sample_argmax, src/ops.cpp:1587-1597)
    if (logits) {
        GemvParams p{};
        p.seg[0] = {static_cast<const unsigned char*>(m->output), logits, m->n_vocab, m->n_vocab};
        p.n_seg = 1;
        p.total_rows = m->n_vocab;
        p.cols = embd;
        p.row_bytes = static_cast<int>(weight_row_bytes(m->type_output, embd));
        p.n_vec = 1;
        p.x = b.x;
        p.x_stride = embd;
        p.norm_w = m->output_norm;
        p.eps = eps;
        p.amax = logits_amax;
        if (int rc = run_gemv(e, m->type_output, p)) return rc;
    }
    return TLA_OK;
}

// out[t][rows] = W . x[t] for n vectors x [n][cols], in launches of up to
// gemv_chunk vectors.
int gemv_rows(tla_engine* e, int type, const void* w, float* out, int rows, int cols, const float* x, int n)
{
    const int chunk = gemv_chunk(n, cols);
    for (int t0 = 0; t0 < n; t0 += chunk) {
        GemvParams p{};
        p.seg[0] = {static_cast<const unsigned char*>(w), out + static_cast<long long>(t0) * rows, rows, rows};
        p.n_seg = 1;
        p.total_rows = rows;
        p.cols = cols;
        p.row_bytes = static_cast<int>(weight_row_bytes(type, cols));
        p.n_vec = std::min(chunk, n - t0);
        p.x = x + static_cast<long long>(t0) * cols;
        p.x_stride = cols;
        if (int rc = run_gemv(e, type, p)) return rc;
    }
    return TLA_OK;
}

// Token batches at least this long (and past the streamed product's range)
// take the split product below; shorter ones the multi-vector GEMV (weights
// read once per group of up to 8 tokens).
constexpr int kBatchMinTokens = 16;

// out_s[t][row] (+)= W_s[row] . x[t] as the split product (split_product.hip):
// x split into three bf16 planes, then one launch over all segments, the
// weights dequantised in registers.  Two 16-row subtiles per wave where
// that still gives half the CUs a workgroup, else one; then K cut into
// ranges of at least 8 blocks until the grid holds about 2.5 workgroups per
// CU (each a workgroup walking its range, the ranges' sums added in order
// by a second launch).  A workgroup's blocks follow one another at about a
// memory round trip each, so shorter ranges and more resident workgroups
// are what shortens a product.  Same box, TinyLlama's four matrices, Q4_0,
// rows per wave x K ranges swept: at 512 tokens gate | up 129 us (2 x 1)
// against 174 us with 4 rows per wave, W_down 73 us (2 x 4-6) against 107
// (1 x 2); at 128 tokens every matrix within 2 us of its best.
int split_batch(tla_engine* e, int type, const GemvSegment* segs, int n_seg, int total, int cols, const float* x,
                long long x_stride, int n, int add, int* deferred = nullptr)
{
    if (deferred) *deferred = 0;
    if (int rc = ensure_buf(e, reinterpret_cast<void**>(&e->xs), e->xs_bytes, split_x_bytes(n, cols), "split-x workspace")) return rc;
    SplitParams p{};
    for (int i = 0; i < n_seg; ++i) p.seg[i] = segs[i];
    p.n_seg = n_seg;
    p.total_rows = total;
    p.cols = cols;
    p.row_bytes = weight_row_bytes(type, cols);
    p.xs = e->xs;
    p.n = n;
    p.n_sub = split_tokens(n) / 16;
    p.add = add;
    const long long token_tiles = p.n_sub / 4;
    auto groups = [&](int rw) { return (total + 64LL * rw - 1) / (64LL * rw) * token_tiles; };
    p.rows_per_wave = 2 * groups(2) >= e->n_cu ? 2 : 1;
    if (e->opt_split_rows > 0) p.rows_per_wave = e->opt_split_rows;
    const int n_blk = cols / 32;
    const long long g = groups(p.rows_per_wave), target = 5LL * e->n_cu / 2;
    int splits = static_cast<int>(std::min<long long>((target + g - 1) / g, n_blk / 8));
    if (e->opt_split_k > 0) splits = e->opt_split_k;
    splits = std::max(1, std::min(splits, n_blk));
    p.blk_per_split = (n_blk + splits - 1) / splits;
    p.k_splits = (n_blk + p.blk_per_split - 1) / p.blk_per_split;
    if (p.k_splits > 1) {
        if (int rc = ensure_buf(e, reinterpret_cast<void**>(&e->part), e->part_bytes, split_part_bytes(n, total, p.k_splits),
                                "split-product partial sums"))
            return rc;
        p.part = e->part;
        // one segment added to rows of its own width: the caller may add the
        // ranges' sums itself, with the rmsnorm that follows
        // (launch_reduce_rmsnorm_rows), instead of a launch of their own
        if (deferred && n_seg == 1 && add && segs[0].out_stride == total) {
            p.defer_reduce = 1;
            *deferred = p.k_splits;
        }
    }
    if (int rc = launch(e, TLA_KERNEL_GEMV, "split rows",
                        [&]() -> hipError_t { return launch_split_rows(x, x_stride, n, cols, e->xs, e->stream); }))
        return rc;
    return launch(e, TLA_KERNEL_GEMV, "split product",
                  [&]() -> hipError_t { return launch_split_product(type, p, e->stream); });
}

// out_s[t][row] (+)= W_s[row] . x[t] for the n_seg matrices of `segs`, one
// type, over n tokens (x rows x_stride floats apart).
// Batches of stream_min_tokens(type) .. kStreamMaxTokens vectors multiply F32
// / F16 / Q8_0 / Q4_0 weights where they lie, dequantised in registers by
// stream_product_kernel; a library product on an fp32 copy of the weights
// ran far below the MFMA rate at these widths (Q4_0 prompts of 33 / 48 / 64
// tokens 2.79 / 3.22 / 3.60 ms streamed against 3.60 / 3.64 / 3.65 ms), and
// the
// multi-vector GEMVs read the weights once per 2-6 vectors (Q4_0 prompts of
// 3 / 8 / 15 tokens 1.67 / 1.82 / ~2.0 ms streamed against 1.89 / 4.21 /
// 7.25 ms).  At 2 tokens the GEMVs keep the quantised formats (Q4_0 1.53
// against 1.63 ms, Q8_0 1.59 against 1.62) but not F16 / F32 (1.69 / 1.93
// against 1.41 / 1.72 ms).  Past 64 vectors the split product takes over:
// each 16-row workgroup of the streamed product loads all of x itself.
constexpr int kStreamMaxTokens = 64;

int stream_min_tokens(int type) { return type == kF16 || type == kF32 ? 2 : 3; }

bool use_stream(int type, int cols, int n, long long x_stride)
{
    return stream_supported(type) && n >= stream_min_tokens(type) && n <= kStreamMaxTokens && cols % 32 == 0 &&
           x_stride % 4 == 0;
}

int stream_batch(tla_engine* e, int type, const GemvSegment* segs, int n_seg, int total, int cols,
                 const float* x, long long x_stride, int n, int add)
{
    StreamParams p{};
    for (int i = 0; i < n_seg; ++i) p.seg[i] = segs[i];
    p.n_seg = n_seg;
    p.total_rows = total;
    p.cols = cols;
    p.row_bytes = weight_row_bytes(type, cols);
    p.x = x;
    p.x_stride = x_stride;
    p.n = n;
    p.add = add;
    // token tiles of 16 per workgroup: one for matrices of at most 128 row
    // tiles (their workgroups are too few to fill the CUs otherwise; W_o and
    // W_down at TinyLlama's shapes, 32 tokens: 11.6 against 15.2 us and 22.4
    // against 30.1 us), else as many as kStreamMaxTiles allows (W_qkv,
    // gate + up: 15.4 against 19.7 us, 40.6 against 52.7 us)
    const int nt = (n + 15) / 16;
    p.tiles = e->opt_stream_tiles > 0 ? e->opt_stream_tiles
              : (total + 15) / 16 <= 128 ? 1
                                         : std::min(nt, kStreamMaxTiles);
    return launch(e, TLA_KERNEL_GEMV, "streamed product",
                  [&]() -> hipError_t { return launch_stream_product(type, p, e->stream); });
}

// deferred (when non-null): the K ranges whose sums a split product left in
// e->part for the caller to add (launch_reduce_rmsnorm_rows), else 0.
int matrix_batch(tla_engine* e, int type, const GemvSegment* segs, int n_seg, int cols, const float* x,
                 long long x_stride, int n, int add, int* deferred = nullptr)
{
    if (deferred) *deferred = 0;
    int total = 0;
    for (int i = 0; i < n_seg; ++i) total += segs[i].rows;
    if (use_stream(type, cols, n, x_stride)) return stream_batch(e, type, segs, n_seg, total, cols, x, x_stride, n, add);
    if (n >= kBatchMinTokens && cols % 32 == 0 && (type != kQ6_K || cols % 256 == 0) && x_stride % 4 == 0 &&
        reinterpret_cast<std::uintptr_t>(x) % 16 == 0)
        return split_batch(e, type, segs, n_seg, total, cols, x, x_stride, n, add, deferred);
    const int chunk = std::max(1, std::min({n, kGemvMaxVec, kGemvLdsBytes / gemv_lds_per_vec(cols)}));
    for (int t0 = 0; t0 < n; t0 += chunk) {
        GemvParams p{};
        for (int i = 0; i < n_seg; ++i) {
            p.seg[i] = segs[i];
            p.seg[i].out = segs[i].out + static_cast<long long>(t0) * segs[i].out_stride;
        }
        p.n_seg = n_seg;
        p.total_rows = total;
        p.cols = cols;
        p.row_bytes = static_cast<int>(weight_row_bytes(type, cols));
        p.n_vec = std::min(chunk, n - t0);
        p.x = x + static_cast<long long>(t0) * x_stride;
        p.x_stride = x_stride;
        p.add = add;
        if (int rc = run_gemv(e, type, p)) return rc;
    }
    return TLA_OK;
}

// The prompt as one batch (n_tok tokens at positions pos0..): embeddings,
// then per layer rmsnorm + Q/K/V over all tokens, the causal prefill
// attention (RoPE + append in-kernel), W_o + residual and the FFN;
// logits of the last token only (when `logits` is non-null).  Every
// product is a matrix_batch: multi-vector GEMVs, streamed products or
// split products by the prompt's length.
int prompt_step(tla_engine* e, const tla_model* m, const FwdBufs& b, float* kc, float* vc,
                const int* tokens_dev, int n_tok, int pos0, float* logits)
{
    const int embd = e->cfg.n_embd, kv = e->kv_dim, ff = m->n_ff;
    const float eps = m->rms_norm_eps;
    if (int rc = check_hip(launch_embed(m->type_embd, b.x, static_cast<const unsigned char*>(m->token_embd),
                                        0, tokens_dev, n_tok, embd, e->stream),
                           "embed"))
        return rc;
    const auto U = [](const void* w) { return static_cast<const unsigned char*>(w); };
    const int n_layers = e->cfg.n_layers;
    // The W_o and W_down products add to x; where their K ranges' sums are
    // left in e->part (pending), the rmsnorm rows launch after them adds
    // them first (one launch for both), before any other product reuses
    // e->part.  After the last layer x is added to by the product itself.
    int pending = 0;
    auto norm_rows = [&](const float* w) -> int {
        const hipError_t err = pending ? launch_reduce_rmsnorm_rows(b.x, e->part, pending, b.xb, w, n_tok, embd,
                                                                    eps, e->stream)
                                       : launch_rmsnorm_rows(b.xb, b.x, w, n_tok, embd, eps, e->stream);
        pending = 0;
        return check_hip(err, "rmsnorm rows");
    };
    for (int l = 0; l < n_layers; ++l) {
        const tla_layer_weights& L = m->layers[l];
        auto product = [&](int type, const GemvSegment* segs, int n_seg, int cols, const float* x,
                           long long x_stride, int add) -> int {
            return matrix_batch(e, type, segs, n_seg, cols, x, x_stride, n_tok, add);
        };
        // rmsnorm rows, then Q/K/V (src/forward.cpp:180-190)
        if (int rc = norm_rows(L.attn_norm)) return rc;
        if (L.type_q == L.type_k && L.type_q == L.type_v) {
            const GemvSegment segs[3] = {{U(L.wq), b.q, embd, embd}, {U(L.wk), b.k, kv, kv}, {U(L.wv), b.v, kv, kv}};
            if (int rc = product(L.type_q, segs, 3, embd, b.xb, embd, 0)) return rc;
        } else {
            const GemvSegment sq{U(L.wq), b.q, embd, embd}, sk{U(L.wk), b.k, kv, kv}, sv{U(L.wv), b.v, kv, kv};
            if (int rc = matrix_batch(e, L.type_q, &sq, 1, embd, b.xb, embd, n_tok, 0)) return rc;
            if (int rc = matrix_batch(e, L.type_k, &sk, 1, embd, b.xb, embd, n_tok, 0)) return rc;
            if (int rc = matrix_batch(e, L.type_v, &sv, 1, embd, b.xb, embd, n_tok, 0)) return rc;
        }
        // RoPE + append + causal attention (src/forward.cpp:192-208)
        if (int rc = tla_prefill(e, pos0, n_tok, l, 1, TLA_ROTATE, b.att, b.q, b.k, b.v, kc, vc)) return rc;
        // x += Wo . att (src/forward.cpp:210-213)
        {
            const GemvSegment so{U(L.wo), b.x, embd, embd};
            if (int rc = matrix_batch(e, L.type_o, &so, 1, embd, b.att, embd, n_tok, 1, &pending)) return rc;
        }
        // FFN (src/forward.cpp:215-228): rmsnorm rows, gate and up into
        // hb [t][gate | up], SiLU x up in place, x += W_down . h
        if (int rc = norm_rows(L.ffn_norm)) return rc;
        {
            const GemvSegment segs[2] = {{U(L.w_gate), b.hb, ff, 2LL * ff}, {U(L.w_up), b.hb + ff, ff, 2LL * ff}};
            if (int rc = product(L.type_ffn, segs, 2, embd, b.xb, embd, 0)) return rc;
        }
        if (int rc = check_hip(launch_swiglu_rows(b.hb, n_tok, ff, e->stream), "swiglu rows")) return rc;
        {
            const GemvSegment sd{U(L.w_down), b.x, embd, embd};
            if (int rc = matrix_batch(e, L.type_ffn, &sd, 1, ff, b.hb, 2LL * ff, n_tok, 1,
                                      l + 1 < n_layers ? &pending : nullptr))
                return rc;
        }
    }
    if (logits)
        if (int rc = gemv1(e, m->type_output, m->output, logits, m->n_vocab, embd,
                           b.x + static_cast<long long>(n_tok - 1) * embd, nullptr, m->output_norm, eps, 0))
            return rc;
    (void)kv;
    return TLA_OK;
}

}  // namespace

int tla_matmul_batch(tla_engine* e, float* out_dev, const void* w_dev, const float* x_dev, int rows,
                     int cols, int n_tok, int type)
{
    if (int rc = check_engine(e)) return rc;
    if (!out_dev || !w_dev || !x_dev) return fail(TLA_ERR_INVALID_ARGUMENT, "NULL device pointer");
    if (rows < 1 || n_tok < 1) return fail(TLA_ERR_INVALID_ARGUMENT, "rows %d, n_tok %d must be >= 1", rows, n_tok);
    if (int rc = check_gemv(type, cols, 1, w_dev)) return rc;
    if (reinterpret_cast<std::uintptr_t>(x_dev) % 16) return fail(TLA_ERR_INVALID_ARGUMENT, "x must be 16-byte aligned");
    if (int rc = set_device(e)) return rc;
    const GemvSegment seg{static_cast<const unsigned char*>(w_dev), out_dev, rows, rows};
    if (int rc = matrix_batch(e, type, &seg, 1, cols, x_dev, cols, n_tok, 0)) return rc;
    return ok();
}

int tla_silu(tla_engine* e, float* x_dev, int size)
{
    if (int rc = elementwise_check(e, x_dev, x_dev, size)) return rc;
    if (int rc = check_hip(launch_silu(x_dev, size, e->stream), "silu")) return rc;
    return ok();
}

int tla_elementwise_mul(tla_engine* e, float* a_dev, const float* b_dev, int size)
{
    if (int rc = elementwise_check(e, a_dev, b_dev, size)) return rc;
    if (int rc = check_hip(launch_elementwise_mul(a_dev, b_dev, size, e->stream), "elementwise_mul")) return rc;
    return ok();
}

int tla_ffn_swiglu(tla_engine* e, float* out_dev, const float* in_dev, float* hb_dev,
                   float* hb2_dev, const void* w_gate_dev, const void* w_up_dev,
                   const void* w_down_dev, int n_ff, int n_embd, int type)
{
    if (int rc = check_engine(e)) return rc;
    if (!out_dev || !in_dev || !hb_dev || !hb2_dev || !w_gate_dev || !w_up_dev || !w_down_dev)
        return fail(TLA_ERR_INVALID_ARGUMENT, "NULL device pointer");
    if (n_ff < 1) return fail(TLA_ERR_INVALID_ARGUMENT, "n_ff %d < 1", n_ff);
    if (int rc = check_gemv(type, n_embd, 1, w_gate_dev)) return rc;
    if (int rc = check_gemv(type, n_embd, 1, w_up_dev)) return rc;
    if (int rc = check_gemv(type, n_ff, 1, w_down_dev)) return rc;
    if (int rc = set_device(e)) return rc;
    GemvParams p{};
    p.seg[0] = {static_cast<const unsigned char*>(w_gate_dev), hb_dev, n_ff, n_ff};
    p.seg[1] = {static_cast<const unsigned char*>(w_up_dev), hb2_dev, n_ff, n_ff};
    p.n_seg = 2;
    p.total_rows = 2 * n_ff;
    p.cols = n_embd;
    p.row_bytes = static_cast<int>(weight_row_bytes(type, n_embd));
    p.n_vec = 1;
    p.x = in_dev;
    p.x_stride = n_embd;
    if (int rc = run_gemv(e, type, p)) return rc;
    if (int rc = check_hip(launch_silu(hb_dev, n_ff, e->stream), "silu")) return rc;
    if (int rc = check_hip(launch_elementwise_mul(hb_dev, hb2_dev, n_ff, e->stream), "elementwise_mul"))
        return rc;
    if (int rc = gemv1(e, type, w_down_dev, out_dev, n_embd, n_ff, hb_dev, nullptr, nullptr, 0.f, 0))
        return rc;
    return ok();
}

int tla_ffn_block(tla_engine* e, int n_seq, float* x_dev, const float* norm_w_dev, float eps,
                  const void* w_gate_dev, const void* w_up_dev, const void* w_down_dev, int n_ff,
                  int type, float* hb_dev)
{
    if (int rc = check_engine(e)) return rc;
    if (!x_dev || !norm_w_dev || !w_gate_dev || !w_up_dev || !w_down_dev || !hb_dev)
        return fail(TLA_ERR_INVALID_ARGUMENT, "NULL device pointer");
    if (n_seq < 1) return fail(TLA_ERR_INVALID_ARGUMENT, "n_seq %d < 1", n_seq);
    if (n_ff < 1) return fail(TLA_ERR_INVALID_ARGUMENT, "n_ff %d < 1", n_ff);
    const int embd = e->cfg.n_embd;
    const int chunk_up = gemv_chunk(n_seq, embd), chunk_down = gemv_chunk(n_seq, n_ff);
    if (int rc = check_gemv(type, embd, chunk_up, w_gate_dev)) return rc;
    if (int rc = check_gemv(type, embd, chunk_up, w_up_dev)) return rc;
    if (int rc = check_gemv(type, n_ff, chunk_down, w_down_dev)) return rc;
    if (int rc = set_device(e)) return rc;
    // hb_dev: [n_seq][2][n_ff], gate then up; for one sequence in a format
    // that pairs rows, the gate half receives SiLU(gate) x up directly.
    const bool paired = n_seq == 1 && gemv_can_pair(type, n_ff, embd);
    for (int s0 = 0; s0 < n_seq; s0 += chunk_up) {
        const int nv = std::min(chunk_up, n_seq - s0);
        GemvParams p{};
        float* h = hb_dev + static_cast<long long>(s0) * 2 * n_ff;
        p.seg[0] = {static_cast<const unsigned char*>(w_gate_dev), h, n_ff, 2LL * n_ff};
        p.seg[1] = {static_cast<const unsigned char*>(w_up_dev), h + n_ff, n_ff, 2LL * n_ff};
        p.n_seg = 2;
        p.total_rows = 2 * n_ff;
        p.cols = embd;
        p.row_bytes = static_cast<int>(weight_row_bytes(type, embd));
        p.n_vec = nv;
        p.x = x_dev + static_cast<long long>(s0) * embd;
        p.x_stride = embd;
        p.norm_w = norm_w_dev;
        p.eps = eps;
        p.pair = paired ? 1 : 0;
        if (int rc = run_gemv(e, type, p)) return rc;
    }
    for (int s0 = 0; s0 < n_seq; s0 += chunk_down) {
        const int nv = std::min(chunk_down, n_seq - s0);
        GemvParams p{};
        p.seg[0] = {static_cast<const unsigned char*>(w_down_dev), x_dev + static_cast<long long>(s0) * embd,
                    embd, embd};
        p.n_seg = 1;
        p.total_rows = embd;
        p.cols = n_ff;
        p.row_bytes = static_cast<int>(weight_row_bytes(type, n_ff));
        p.n_vec = nv;
        p.x = hb_dev + static_cast<long long>(s0) * 2 * n_ff;
        p.x2 = paired ? nullptr : p.x + n_ff;
        p.x_stride = 2LL * n_ff;
        p.add = 1;
        if (int rc = run_gemv(e, type, p)) return rc;
    }
    return ok();
}

int tla_embed(tla_engine* e, float* out_dev, const void* table_dev, int token, int n_embd,
              int n_vocab, int type)
{
    if (int rc = check_engine(e)) return rc;
    if (!out_dev || !table_dev) return fail(TLA_ERR_INVALID_ARGUMENT, "NULL device pointer");
    if (n_vocab < 1) return fail(TLA_ERR_INVALID_ARGUMENT, "n_vocab %d < 1", n_vocab);
    if (token < 0 || token >= n_vocab)
        return fail(TLA_ERR_OUT_OF_RANGE, "token %d outside [0, n_vocab=%d)", token, n_vocab);
    if (n_embd < 1 || weight_row_bytes(type, n_embd) == 0 || (type == kQ6_K ? n_embd % 256 : n_embd % 32))
        return fail(TLA_ERR_INVALID_ARGUMENT, "type %d with n_embd %d", type, n_embd);
    if (int rc = set_device(e)) return rc;
    if (int rc = check_hip(launch_embed(type, out_dev, static_cast<const unsigned char*>(table_dev), token,
                                        nullptr, 1, n_embd, e->stream),
                           "embed"))
        return rc;
    return ok();
}

int tla_argmax(tla_engine* e, const float* logits_dev, int n_vocab, int* token_host)
{
    if (int rc = check_engine(e)) return rc;
    if (!logits_dev || !token_host) return fail(TLA_ERR_INVALID_ARGUMENT, "NULL pointer");
    if (n_vocab < 1) return fail(TLA_ERR_INVALID_ARGUMENT, "n_vocab %d < 1", n_vocab);
    if (int rc = set_device(e)) return rc;
    if (!e->argmax_slot) TLA_HIP(hipMalloc(reinterpret_cast<void**>(&e->argmax_slot), sizeof(int)));
    hipError_t err = launch_argmax(e->argmax_slot, nullptr, logits_dev, n_vocab, e->stream);
    if (err == hipSuccess)
        err = hipMemcpyAsync(token_host, e->argmax_slot, sizeof(int), hipMemcpyDeviceToHost, e->stream);
    if (err == hipSuccess) err = hipStreamSynchronize(e->stream);
    if (err != hipSuccess) return fail(TLA_ERR_DEVICE, "argmax: %s", hipGetErrorString(err));
    return ok();
}

int tla_matmul_argmax(tla_engine* e, float* out_dev, const void* w_dev, const float* x_dev, int rows,
                      int cols, int type, int* token_host)
{
    if (int rc = check_engine(e)) return rc;
    if (!out_dev || !w_dev || !x_dev || !token_host) return fail(TLA_ERR_INVALID_ARGUMENT, "NULL pointer");
    if (rows < 1) return fail(TLA_ERR_INVALID_ARGUMENT, "rows %d < 1", rows);
    if (int rc = check_gemv(type, cols, 1, w_dev)) return rc;
    if (!gemv_can_amax(cols)) return fail(TLA_ERR_UNSUPPORTED, "argmax keys: rows of %d > 4096 columns", cols);
    if (int rc = set_device(e)) return rc;
    if (!e->argmax_slot) TLA_HIP(hipMalloc(reinterpret_cast<void**>(&e->argmax_slot), sizeof(int)));
    if (!e->amax_keys)
        TLA_HIP(hipMalloc(reinterpret_cast<void**>(&e->amax_keys), kAmaxSlots * sizeof(unsigned long long)));
    TLA_HIP(launch_zero(e->amax_keys, kAmaxSlots * sizeof(unsigned long long), e->stream));
    GemvParams p{};
    p.seg[0] = {static_cast<const unsigned char*>(w_dev), out_dev, rows, 0};
    p.n_seg = 1;
    p.total_rows = rows;
    p.cols = cols;
    p.row_bytes = static_cast<int>(weight_row_bytes(type, cols));
    p.n_vec = 1;
    p.x = x_dev;
    p.x_stride = cols;
    p.amax = e->amax_keys;
    if (int rc = run_gemv(e, type, p)) return rc;
    hipError_t err = launch_amax_token(e->amax_keys, e->argmax_slot, e->stream);
    if (err == hipSuccess)
        err = hipMemcpyAsync(token_host, e->argmax_slot, sizeof(int), hipMemcpyDeviceToHost, e->stream);
    if (err == hipSuccess) err = hipStreamSynchronize(e->stream);
    if (err != hipSuccess) return fail(TLA_ERR_DEVICE, "matmul_argmax: %s", hipGetErrorString(err));
    return ok();
}

int tla_forward(tla_engine* e, const tla_model* m, float* key_cache_dev, float* value_cache_dev,
                int token, int pos, float* logits_dev)
{
    if (int rc = check_engine(e)) return rc;
    if (!key_cache_dev || !value_cache_dev || !logits_dev)
        return fail(TLA_ERR_INVALID_ARGUMENT, "NULL device pointer");
    if (int rc = check_model(e, m)) return rc;
    if (token < 0 || token >= m->n_vocab)
        return fail(TLA_ERR_OUT_OF_RANGE, "token %d outside [0, n_vocab=%d)", token, m->n_vocab);
    if (pos < 0 || pos >= e->cfg.n_ctx)
        return fail(TLA_ERR_OUT_OF_RANGE, "pos %d outside [0, n_ctx=%d)", pos, e->cfg.n_ctx);
    if (int rc = set_device(e)) return rc;
    FwdBufs b{};
    if (int rc = fwd_bufs(e, m, 1, 0, &b)) return rc;
    if (int rc = forward_step(e, m, b, key_cache_dev, value_cache_dev, token, nullptr, pos, logits_dev))
        return rc;
    return ok();
}

int tla_prefill_forward(tla_engine* e, const tla_model* m, float* key_cache_dev, float* value_cache_dev,
                        const int* tokens_host, int n_tok, int pos0, float* logits_dev)
{
    if (int rc = check_engine(e)) return rc;
    if (!key_cache_dev || !value_cache_dev || !tokens_host)
        return fail(TLA_ERR_INVALID_ARGUMENT, "NULL pointer");
    if (int rc = check_model(e, m)) return rc;
    if (n_tok < 1) return fail(TLA_ERR_INVALID_ARGUMENT, "n_tok %d < 1", n_tok);
    if (pos0 < 0 || static_cast<long long>(pos0) + n_tok > e->cfg.n_ctx)
        return fail(TLA_ERR_OUT_OF_RANGE, "positions [%d, %lld) outside [0, n_ctx=%d)", pos0,
                    static_cast<long long>(pos0) + n_tok, e->cfg.n_ctx);
    for (int i = 0; i < n_tok; ++i)
        if (tokens_host[i] < 0 || tokens_host[i] >= m->n_vocab)
            return fail(TLA_ERR_OUT_OF_RANGE, "tokens[%d] = %d outside [0, n_vocab)", i, tokens_host[i]);
    if (int rc = set_device(e)) return rc;
    FwdBufs b{};
    if (int rc = fwd_bufs(e, m, n_tok, n_tok, &b)) return rc;
    TLA_HIP(hipMemcpyWithStream(b.tokens, tokens_host, sizeof(int) * n_tok, hipMemcpyHostToDevice, e->stream));
    if (int rc = prompt_step(e, m, b, key_cache_dev, value_cache_dev, b.tokens, n_tok, pos0, logits_dev))
        return rc;
    return ok();
}

int tla_generate_greedy(tla_engine* e, const tla_model* m, float* key_cache_dev,
                        float* value_cache_dev, const int* prompt_host, int n_prompt, int n_gen,
                        int flags, int* tokens_host)
{
    if (flags & ~TLA_BATCH_PROMPT) return fail(TLA_ERR_INVALID_ARGUMENT, "unknown flags 0x%x", flags);
    if (int rc = check_engine(e)) return rc;
    if (!key_cache_dev || !value_cache_dev || !prompt_host || !tokens_host)
        return fail(TLA_ERR_INVALID_ARGUMENT, "NULL pointer");
    if (int rc = check_model(e, m)) return rc;
    if (n_prompt < 1 || n_gen < 1) return fail(TLA_ERR_INVALID_ARGUMENT, "n_prompt, n_gen must be >= 1");
    if (static_cast<long long>(n_prompt) + n_gen - 1 > e->cfg.n_ctx)
        return fail(TLA_ERR_OUT_OF_RANGE, "n_prompt + n_gen - 1 = %lld > n_ctx %d",
                    static_cast<long long>(n_prompt) + n_gen - 1, e->cfg.n_ctx);
    for (int i = 0; i < n_prompt; ++i)
        if (prompt_host[i] < 0 || prompt_host[i] >= m->n_vocab)
            return fail(TLA_ERR_OUT_OF_RANGE, "prompt[%d] = %d outside [0, n_vocab)", i, prompt_host[i]);
    if (int rc = set_device(e)) return rc;
    const bool batch = (flags & TLA_BATCH_PROMPT) != 0;
    // argmax keys by the classifier launch: rows of generated tokens 1 ..
    // n_gen - 1 (n_gen rows, row 0 unused), zeroed by a fill kernel
    const bool keys = gemv_can_amax(e->cfg.n_embd);
    FwdBufs b{};
    if (int rc = fwd_bufs(e, m, batch ? n_prompt : 1, n_gen + n_prompt, &b, keys ? n_gen : 0)) return rc;
    if (keys && n_gen > 1)
        TLA_HIP(launch_zero(b.amax, static_cast<size_t>(n_gen) * kAmaxSlots * sizeof(unsigned long long), e->stream));
    int pos = 0;
    if (batch) {
        int* prompt_dev = b.tokens + 1 + n_gen;
        TLA_HIP(hipMemcpyWithStream(prompt_dev, prompt_host, sizeof(int) * n_prompt, hipMemcpyHostToDevice,
                                    e->stream));
        if (int rc = prompt_step(e, m, b, key_cache_dev, value_cache_dev, prompt_dev, n_prompt, 0, b.logits))
            return rc;
        pos = n_prompt;
    } else {
        // token by token; only the last token's logits are needed (the
        // reference computes and overwrites the others)
        for (int i = 0; i < n_prompt; ++i, ++pos)
            if (int rc = forward_step(e, m, b, key_cache_dev, value_cache_dev, prompt_host[i], nullptr, pos,
                                      i + 1 == n_prompt ? b.logits : nullptr))
                return rc;
    }
    // b.tokens[0]: the current token; b.tokens[1 + i]: generated token i.
    // Token 0 from the prompt's logits by the argmax launch; with keys, each
    // later token i from the keys its step's classifier posted to row i,
    // read by the next step's embedding launch (which stores it) or, for
    // the last, by a one-wave launch.
    if (int rc = check_hip(launch_argmax(b.tokens, b.tokens + 1, b.logits, m->n_vocab, e->stream), "argmax"))
        return rc;
    for (int i = 1; i < n_gen; ++i) {
        unsigned long long* row = b.amax + static_cast<size_t>(i) * kAmaxSlots;
        if (keys) {
            const bool from_keys = i >= 2;  // token i - 1
            if (int rc = forward_step(e, m, b, key_cache_dev, value_cache_dev, 0, from_keys ? nullptr : b.tokens,
                                      pos++, b.logits, from_keys ? row - kAmaxSlots : nullptr,
                                      from_keys ? b.tokens + i : nullptr, row))
                return rc;
        } else {
            if (int rc = forward_step(e, m, b, key_cache_dev, value_cache_dev, 0, b.tokens, pos++, b.logits))
                return rc;
            if (int rc = check_hip(launch_argmax(b.tokens, b.tokens + 1 + i, b.logits, m->n_vocab, e->stream),
                                   "argmax"))
                return rc;
        }
    }
    if (keys && n_gen > 1)
        if (int rc = check_hip(launch_amax_token(b.amax + static_cast<size_t>(n_gen - 1) * kAmaxSlots,
                                                 b.tokens + n_gen, e->stream),
                               "argmax keys"))
            return rc;
    TLA_HIP(hipMemcpyAsync(tokens_host, b.tokens + 1, sizeof(int) * n_gen, hipMemcpyDeviceToHost, e->stream));
    TLA_HIP(hipStreamSynchronize(e->stream));
    return ok();
}

int tla_profile_enable(tla_engine* e, int enable)
{
    if (int rc = check_engine(e)) return rc;
    if (int rc = set_device(e)) return rc;
    if (int rc = prof_collect(e)) return rc;
    for (int k = 0; k < TLA_KERNEL_COUNT; ++k) {
        e->prof_ms[k] = 0.0;
        e->prof_n[k] = 0;
    }
    e->prof = enable != 0;
    return ok();
}

int tla_profile_read(tla_engine* e, int kernel_id, double* total_ms, long long* launches)
{
    if (int rc = check_engine(e)) return rc;
    if (kernel_id < 0 || kernel_id >= TLA_KERNEL_COUNT)
        return fail(TLA_ERR_INVALID_ARGUMENT, "kernel id %d", kernel_id);
    if (!total_ms || !launches) return fail(TLA_ERR_INVALID_ARGUMENT, "NULL output");
    if (int rc = set_device(e)) return rc;
    if (int rc = prof_collect(e)) return rc;
    *total_ms = e->prof_ms[kernel_id];
    *launches = e->prof_n[kernel_id];
    return ok();
}

int tla_event_record(tla_engine* e, int slot)
{
    if (int rc = check_engine(e)) return rc;
    if (slot < 0 || slot >= kEventSlots) return fail(TLA_ERR_INVALID_ARGUMENT, "slot %d", slot);
    if (int rc = set_device(e)) return rc;
    if (!e->slots[slot]) TLA_HIP(hipEventCreate(&e->slots[slot]));
    TLA_HIP(hipEventRecord(e->slots[slot], e->stream));
    return ok();
}

int tla_event_elapsed(tla_engine* e, int slot_begin, int slot_end, float* ms)
{
    if (int rc = check_engine(e)) return rc;
    if (!ms) return fail(TLA_ERR_INVALID_ARGUMENT, "ms is NULL");
    if (slot_begin < 0 || slot_begin >= kEventSlots || slot_end < 0 || slot_end >= kEventSlots ||
        !e->slots[slot_begin] || !e->slots[slot_end])
        return fail(TLA_ERR_INVALID_ARGUMENT, "slots %d, %d not recorded", slot_begin, slot_end);
    if (int rc = set_device(e)) return rc;
    TLA_HIP(hipEventSynchronize(e->slots[slot_end]));
    TLA_HIP(hipEventElapsedTime(ms, e->slots[slot_begin], e->slots[slot_end]));
    return ok();
}

int tla_read_floor(tla_engine* e, const void* src_dev, size_t bytes, int n_workgroups, int load_kind,
                   int depth, float* sink_dev)
{
    if (int rc = check_engine(e)) return rc;
    if (!src_dev || !sink_dev) return fail(TLA_ERR_INVALID_ARGUMENT, "NULL device pointer");
    if (bytes < 16 || bytes % 16 != 0 || reinterpret_cast<std::uintptr_t>(src_dev) % 16 != 0)
        return fail(TLA_ERR_INVALID_ARGUMENT, "bytes %zu: a positive multiple of 16 at a 16-byte aligned address",
                    bytes);
    if (n_workgroups < 1 || n_workgroups > (1 << 20))
        return fail(TLA_ERR_INVALID_ARGUMENT, "n_workgroups %d not in [1, 2^20]", n_workgroups);
    if (load_kind < TLA_READ_GLOBAL || load_kind > TLA_READ_BUFFER_NT)
        return fail(TLA_ERR_INVALID_ARGUMENT, "load_kind %d not in [0, 3]", load_kind);
    if (depth != 8 && depth != 16 && depth != 32)
        return fail(TLA_ERR_INVALID_ARGUMENT, "depth %d not 8, 16 or 32", depth);
    if (load_kind >= TLA_READ_BUFFER &&
        (bytes / 16 / n_workgroups + 1 + 32 * 256) * 16 >= (1ull << 31))
        return fail(TLA_ERR_INVALID_ARGUMENT, "buffer loads: %zu bytes over %d workgroups is 2 GiB or more each",
                    bytes, n_workgroups);
    if (int rc = set_device(e)) return rc;
    const hipError_t err = launch_read_floor(src_dev, bytes, n_workgroups, load_kind, depth, sink_dev, e->stream);
    if (err != hipSuccess) return fail(TLA_ERR_DEVICE, "read floor launch: %s", hipGetErrorString(err));
    return ok();
}

int tla_mfma_floor(tla_engine* e, int n_workgroups, int iters, float* sink_dev)
{
    if (int rc = check_engine(e)) return rc;
    if (!sink_dev) return fail(TLA_ERR_INVALID_ARGUMENT, "NULL device pointer");
    if (n_workgroups < 1 || n_workgroups > (1 << 20))
        return fail(TLA_ERR_INVALID_ARGUMENT, "n_workgroups %d not in [1, 2^20]", n_workgroups);
    if (iters < 1 || iters > (1 << 20))
        return fail(TLA_ERR_INVALID_ARGUMENT, "iters %d not in [1, 2^20]", iters);
    if (int rc = set_device(e)) return rc;
    const hipError_t err = launch_mfma_floor(n_workgroups, iters, sink_dev, e->stream);
    if (err != hipSuccess) return fail(TLA_ERR_DEVICE, "mfma floor launch: %s", hipGetErrorString(err));
    return ok();
}

int tla_set_option(tla_engine* e, int option, long long value)
{
    if (int rc = check_engine(e)) return rc;
    switch (option) {
    case TLA_OPT_DECODE_SPLIT:
        if (value < 0) return fail(TLA_ERR_INVALID_ARGUMENT, "split %lld < 0", value);
        e->opt_split = value;
        return ok();
    case TLA_OPT_DECODE_PLAN:
        if (value < TLA_PLAN_AUTO || value > TLA_PLAN_BALANCED)
            return fail(TLA_ERR_INVALID_ARGUMENT, "decode plan %lld not in [0, 2]", value);
        e->opt_plan = static_cast<int>(value);
        return ok();
    case TLA_OPT_DECODE_GROUP:
        if (value != 0 && value != kDecodeKvGroupSmall && value != kDecodeKvGroupMid &&
            value != kDecodeKvGroupLarge)
            return fail(TLA_ERR_INVALID_ARGUMENT, "decode kv group %lld not 0, 1, 2 or 4", value);
        e->opt_group = static_cast<int>(value);
        return ok();
    case TLA_OPT_STREAM_TILES:
        if (value < 0 || value > kStreamMaxTiles)
            return fail(TLA_ERR_INVALID_ARGUMENT, "stream tiles %lld not in [0, %d]", value, kStreamMaxTiles);
        e->opt_stream_tiles = static_cast<int>(value);
        return ok();
    case TLA_OPT_SPLIT_ROWS:
        if (value != 0 && value != 1 && value != 2 && value != 4)
            return fail(TLA_ERR_INVALID_ARGUMENT, "split rows %lld not 0, 1, 2 or 4", value);
        e->opt_split_rows = static_cast<int>(value);
        return ok();
    case TLA_OPT_SPLIT_K:
        if (value < 0 || value > 64) return fail(TLA_ERR_INVALID_ARGUMENT, "split K %lld not in [0, 64]", value);
        e->opt_split_k = static_cast<int>(value);
        return ok();
    default:
        return fail(TLA_ERR_INVALID_ARGUMENT, "unknown option %d", option);
    }
}

}  // extern "C"
