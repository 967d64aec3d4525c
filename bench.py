#!/usr/bin/env python3
"""Throughput of the MI355X attention path on one GPU.

Default (no flags): the full-model decode-attention step -- 22 layers, KV
cache [2048 positions][4 kv heads][64] fp32 per layer, one new token per
layer (RoPE + append + split-KV attention) -- timed over K steps after W
warmup steps, with inputs resident in HBM.  To keep the 92.7 MB step out of
the 256 MB Infinity Cache, steps rotate over 5 copies of the whole cache
(461 MB).  Prints ONE JSON line:

  value      decode KV GB/s = algorithmic bytes per step / step time, with
             algorithmic bytes 2048*L + 20480 per (sequence, layer), L = 2048
  roofline   the decode kernel against HBM 8 TB/s: a step is one launch, so
             HIP events around the K timed steps on the engine's stream give
             its average duration; `traffic` is the HBM bytes per launch
             measured with rocprofv3 and recorded under profiles/
  prefill    the causal prefill workload (512 tokens, 22 layers): exact causal
             TFLOP/s against fp32 MFMA 157.3 TFLOP/s, after at least 200
             untimed steps (the clocks' ramp under sustained MFMA work)
  cpu_baseline  the reference's own scalar attention() (oracle/_ref) -- or the
             C restatement when that is not built -- on the host's cores, over
             a bounded sample of the same workload
  extra      the other decode configurations, measured the same way:
             decode_long and decode_ragged (GB/s, with roofline) and
             decode_single (latency, us); --no-extra skips them

Other workloads (--workload): decode_long (16384 context, batch 8, 22 layers),
decode_ragged (64 sequences, L in [256, 2048], 22 layers), prefill,
decode_single (one layer, position 127: reported as latency), decode_sweep
(batch 1, 22 layers, contexts 2K-16K), prefill_sweep (one prompt of 512 to
4096 tokens, 22 layers), prefill_layer_sweep (one layer per launch, 128 to
2048 tokens: the launches a batched prompt makes), proj (the
attention block's projections for a 22-layer decode step, and the GEMV kernel
on a 32000 x 2048 matrix in every weight format), matmul (that GEMV alone in
one format, --wtype), copy (the
device copy kernel, used to calibrate rocprofv3 byte counters), read (a
plain library reduction over 6 GiB) and read_floor (this package's streaming
read over exactly the bytes of a batch-1 decode step at 2K-16K context: what
one launch can move in that time, the ceiling the decode step sits under;
also in the default line's extra) and mfma_floor (this package's bf16 MFMA
loop over the prefill kernel's executed flops: the ceiling the prefill
kernel sits under; also in the default line's prefill entry).
"""
from __future__ import annotations

import argparse
import importlib
import json
import os
import re
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
tla = importlib.import_module("tinyllama-engine_amd")
W = importlib.import_module("tinyllama-engine_amd.workloads")

HBM_PEAK_GBS = 8000.0
FP32_MFMA_PEAK_TFLOPS = 157.3
BF16_MFMA_PEAK_TFLOPS = 2500.0  # dense
# bf16 matrix-core products per fp32-accurate multiply-add in tla_matmul_batch
SPLIT_PRODUCTS = {W.W_F32: 6, W.W_F16: 5, W.W_Q8_0: 3, W.W_Q4_0: 3, W.W_Q6_K: 5}
# The prefill attention kernel's products run on the bf16 matrix cores with
# both operands split into three bf16 pieces, six piece products per
# fp32-accurate multiply-add: its ceiling is the bf16 peak over six.
PREFILL_SPLIT_PRODUCTS = 6
PREFILL_PEAK_TFLOPS = BF16_MFMA_PEAK_TFLOPS / PREFILL_SPLIT_PRODUCTS
MALL_BYTES = 256 << 20


def log(msg):
    print(msg, file=sys.stderr, flush=True)


# The sources each profiled kernel is built from: a profile records their
# digest, and its byte count is used only while the sources are unchanged.
KERNEL_SOURCES = {
    "decode_split_kernel": ("decode.hip", "tla_internal.h", "rope_math.h", "lane_math.h"),
    "prefill_attention_kernel": ("prefill.hip", "tla_internal.h", "rope_math.h", "lane_math.h", "bf16_split.h"),
    "gemv_kernel": ("gemv.hip", "tla_internal.h", "row_math.h", "rope_math.h"),
}


def kernel_source_digest(kernel):
    """sha256 (first 16 hex digits) over the kernel's source files."""
    import hashlib
    h = hashlib.sha256()
    for name in KERNEL_SOURCES[kernel]:
        with open(os.path.join(ROOT, "tinyllama-engine_amd", "csrc", name), "rb") as f:
            h.update(f.read())
    return h.hexdigest()[:16]


def profiled_traffic(kernel, workload):
    """HBM bytes per launch measured with rocprofv3 (FETCH_SIZE x2.0 +
    WRITE_SIZE x1.0, scaled by the copy-kernel calibration) and recorded in
    profiles/<kernel>__<workload>.md -- or None when not profiled, or when the
    profile records a digest of the kernel's sources other than the current
    one (the bytes would belong to another build)."""
    path = os.path.join(ROOT, "profiles", f"{kernel}__{workload}.md")
    if not os.path.exists(path):
        return None
    text = open(path).read()
    m = re.search(r"^traffic_bytes_per_launch:\s*(\d+)\s*$", text, re.M)
    d = re.search(r"^source_digest:\s*([0-9a-f]+)\s*$", text, re.M)
    if not m or not d or d.group(1) != kernel_source_digest(kernel):
        return None
    return int(m.group(1))


def median(xs):
    xs = sorted(xs)
    n = len(xs)
    return xs[n // 2] if n % 2 else 0.5 * (xs[n // 2 - 1] + xs[n // 2])


# ------------------------------------------------------------------ decode --

class DecodeBench:
    """Inputs for one decode workload resident on the device, with enough
    rotated copies of the whole KV cache to exceed the Infinity Cache."""

    def __init__(self, eng, case, copies):
        self.eng, self.case, self.copies = eng, case, copies
        cfg = eng.cfg
        self.n_seq = case.n_seq
        self.seq_stride = cfg.n_layers * cfg.n_ctx * cfg.kv_dim
        self.kc, self.vc = eng.kv_cache(case.n_seq * copies)
        self.kc_host_shape = case.kc.shape
        one = case.kc.nbytes
        # upload copy 0, replicate on the device
        tla.lib().tla_memcpy_h2d(eng.h, self.kc.ptr, case.kc.ctypes.data, one)
        tla.lib().tla_memcpy_h2d(eng.h, self.vc.ptr, case.vc.ctypes.data, one)
        for c in range(1, copies):
            eng.copy(self.kc.ptr + c * one, self.kc.ptr, one)
            eng.copy(self.vc.ptr + c * one, self.vc.ptr, one)
        self.q, self.k, self.v = eng.array(case.q), eng.array(case.k), eng.array(case.v)
        self.out = eng.array(case.q.shape)
        self.bytes_per_copy = one
        eng.synchronize()

    def step(self, i):
        c = i % self.copies
        off = c * self.bytes_per_copy
        self.eng.decode(self.case.pos, 0, self.case.n_layers, self.out.ptr, self.q.ptr, self.k.ptr,
                        self.v.ptr, self.kc.ptr + off, self.vc.ptr + off, self.seq_stride)

    def free(self):
        for a in (self.kc, self.vc, self.q, self.k, self.v, self.out):
            a.free()


def time_steps(eng, step, steps, warmup):
    for i in range(warmup):
        step(i)
    eng.synchronize()
    eng.event(0)
    for i in range(steps):
        step(warmup + i)
    eng.event(1)
    eng.synchronize()
    return eng.elapsed(0, 1) / steps


def kernel_avg_ms(eng, step, steps, kernel_id, start=0):
    eng.profile(True)
    for i in range(steps):
        step(start + i)
    eng.synchronize()
    total, n = eng.profile_read(kernel_id)
    eng.profile(False)
    return total / max(n, 1), n


def back_to_back_ms(eng, launch, steps, blocker_ms=1.0):
    """Average GPU time of `steps` launches queued back to back: a blocker
    (large F32 matrix-vector products, about blocker_ms of GPU work) is
    queued first, so that the host has queued every timed launch before the
    GPU reaches them and the timed region holds no host gaps.  The events
    bracket only the timed launches."""
    rows, cols = 8192, 8192  # 256 MiB of F32 weights, ~45 us per launch
    wb = eng.array((rows * cols * 4,), np.uint8)
    xb = eng.array(np.zeros(cols, np.float32))
    ob = eng.array((rows,))
    n_block = max(1, int(blocker_ms / 0.045))
    eng.synchronize()
    for _ in range(n_block):
        eng.matmul(ob.ptr, wb.ptr, xb.ptr, rows, cols, W.W_F32)
    eng.event(0)
    for i in range(steps):
        launch(i)
    eng.event(1)
    eng.synchronize()
    for a in (wb, xb, ob):
        a.free()
    return eng.elapsed(0, 1) / steps


def make_decode_case(workload, n_layers=22):
    if workload == "decode_model":
        return W.decode_model(n_layers=n_layers, n_ctx=2048), 2048
    if workload == "decode_ragged":
        return W.decode_ragged(n_seq=64, n_layers=n_layers, n_ctx=2048), 2048
    if workload == "decode_long":
        # one layer's data from the generator (16384 ctx x 8 seqs, peaked
        # keys), repeated for every layer: the byte stream per layer is the
        # same, and host generation stays a few seconds
        return W.replicate_layers(W.decode_long_layer(n_seq=8, n_ctx=16384), n_layers), 16384
    if workload == "decode_single":
        return W.decode_single(), 128
    raise ValueError(workload)


def run_decode(workload, steps, warmup, cpu, split=0, plan=0):
    n_layers = 1 if workload == "decode_single" else 22
    case, n_ctx = make_decode_case(workload, n_layers)
    one_copy = case.kc.nbytes * 2
    copies = 1 if workload == "decode_single" else max(1, -(-3 * MALL_BYTES // 2 // one_copy))
    copies = max(copies, 2 if one_copy < MALL_BYTES else 1)
    log(f"[bench] {workload}: {case.n_seq} seq x {n_layers} layers, ctx {n_ctx}, "
        f"{copies} rotated cache copies ({copies * one_copy / 1e6:.0f} MB)")
    eng = tla.Engine(tla.Config.tinyllama(n_layers=n_layers, n_ctx=n_ctx))
    if split:
        eng.set_option(tla.OPT_DECODE_SPLIT, split)
    eng.set_option(tla.OPT_DECODE_PLAN, plan)
    b = DecodeBench(eng, case, copies)
    # A decode step is exactly one launch of the decode kernel, so the HIP
    # events around the K timed steps (engine stream) give its average
    # duration; per-launch event pairs are kept as a cross-check (they add
    # ~2 us of event overhead to each launch).
    ms = time_steps(eng, b.step, steps, warmup)
    ev_ms, k_n = kernel_avg_ms(eng, b.step, steps, tla.KERNEL_DECODE, start=warmup + steps)
    algo = case.algorithmic_bytes
    res = {
        "workload": workload, "ms_per_step": ms, "algorithmic_bytes": algo,
        "value": algo / (ms * 1e-3) / 1e9,
        "decode_kernel_ms": ms, "decode_kernel_ms_per_launch_events": ev_ms,
        "cache_copies": copies, "mall_resident": copies * one_copy <= MALL_BYTES,
    }
    achieved = algo / (ms * 1e-3) / 1e9
    res["roofline"] = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                       "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                       "traffic": profiled_traffic("decode_split_kernel", workload),
                       "algorithmic_bytes": algo, "kernel": "decode_split_kernel",
                       "launches": steps}
    log(f"[bench] {workload}: {ms * 1e3:.1f} us/step = decode kernel -> {achieved:.0f} GB/s "
        f"({achieved / HBM_PEAK_GBS:.1%}); per-launch events {ev_ms * 1e3:.1f} us")
    b.free()
    eng.close()
    if cpu:
        res["cpu_baseline"] = cpu_decode_baseline(case, n_ctx, workload)
    return res


def run_decode_sweep(steps, warmup, contexts=(2048, 4096, 8192, 16384), n_layers=22, plan=0):
    """Batch-1 decode steps (22 layers, one sequence, new token at the last
    position) over a range of contexts: where the fixed costs of one launch
    stop mattering.  One layer's K/V (N(0,1), seeded) repeated for every
    layer, as decode_long does; cache copies rotated past the Infinity
    Cache."""
    out = []
    for ctx in contexts:
        case = W.replicate_layers(W.decode_sweep_layer(ctx), n_layers)
        one_copy = case.kc.nbytes * 2
        copies = max(1, -(-3 * MALL_BYTES // 2 // one_copy))
        copies = max(copies, 2 if one_copy < MALL_BYTES else 1)
        eng = tla.Engine(tla.Config.tinyllama(n_layers=n_layers, n_ctx=ctx))
        eng.set_option(tla.OPT_DECODE_PLAN, plan)
        b = DecodeBench(eng, case, copies)
        ms = time_steps(eng, b.step, steps, warmup)
        algo = case.algorithmic_bytes
        gbs = algo / (ms * 1e-3) / 1e9
        log(f"[bench] decode batch 1, ctx {ctx}, {n_layers} layers: {ms * 1e3:.1f} us/step, "
            f"{algo / 1e6:.0f} MB -> {gbs:.0f} GB/s ({gbs / HBM_PEAK_GBS:.1%}), {copies} copies")
        out.append({"ctx": ctx, "us": round(ms * 1e3, 2), "bytes": algo, "GB_s": round(gbs, 1),
                    "frac": round(gbs / HBM_PEAK_GBS, 4)})
        b.free()
        eng.close()
    return out


def cpu_threads():
    return max(1, min(16, os.cpu_count() or 1))


def cpu_host():
    """The host the CPU baseline ran on: its CPU model and hardware threads."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"cpu_model": model, "hardware_threads": os.cpu_count()}


def cpu_decode_baseline(case, n_ctx, workload, budget_s=10.0):
    """Time the reference's attention() (oracle/_ref) or the C restatement on
    the host over whole steps of the same workload for about budget_s."""
    import oracle as O
    kind = "reference" if O.ref_available() else "port"
    lib = O.ref() if kind == "reference" else None
    units = case.n_seq * case.n_layers
    s = O.Shape(n_ctx=n_ctx)
    q = case.q.reshape(units, -1)
    k = case.k.reshape(units, -1)
    v = case.v.reshape(units, -1)
    kc = case.kc.reshape(units, n_ctx, -1).copy()
    vc = case.vc.reshape(units, n_ctx, -1).copy()
    pos = np.repeat(case.pos, case.n_layers).astype(np.int32)

    def measure(threads, budget):
        times = []
        t_end = time.perf_counter() + budget
        while True:
            t0 = time.perf_counter()
            O.decode_units_mt(threads, q, k, v, kc, vc, pos, s, rotate=True, lib=lib)
            times.append(time.perf_counter() - t0)
            if time.perf_counter() > t_end and len(times) >= 2:
                break
        return median(times), len(times)

    threads = cpu_threads()
    t1, n1 = measure(1, budget_s * 0.25)
    tn, nn = measure(threads, budget_s * 0.75)
    algo = case.algorithmic_bytes
    log(f"[bench] cpu {kind}: 1 thread {t1 * 1e3:.1f} ms/step, {threads} threads "
        f"{tn * 1e3:.1f} ms/step")
    return {"value": round(algo / tn / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": kind,
            "sample": f"{nn} full steps of {workload} ({case.n_seq} seq x {case.n_layers} layers), "
                      f"median, {threads} threads; 1 thread: {n1} steps",
            "single_thread_value": round(algo / t1 / 1e9, 3),
            "ms_per_step": round(tn * 1e3, 3), "single_thread_ms_per_step": round(t1 * 1e3, 3),
            **cpu_host()}


# ----------------------------------------------------------------- prefill --

# Untimed prefill steps before timing: the GPU's clocks ramp over the first
# tens of milliseconds of sustained MFMA work (512 tokens x 22 layers: 247
# us/step after 10 warmup steps, 212 us/step after 200 or 2000).  Decode
# steps are HBM-bound and measure the same after 10 or 2000.
PREFILL_MIN_WARMUP = 200


def run_prefill(steps, warmup, cpu, n_layers=22, n_tok=512, label="prefill"):
    warmup = max(warmup, PREFILL_MIN_WARMUP)
    case = W.make_prefill(n_layers=n_layers, n_tok=n_tok)
    eng = tla.Engine(tla.Config.tinyllama(n_layers=n_layers, n_ctx=n_tok))
    kc, vc = eng.kv_cache(1)
    q, k, v = eng.array(case.q), eng.array(case.k), eng.array(case.v)
    out = eng.array(case.q.shape)

    def step(i):
        eng.prefill(0, n_tok, 0, n_layers, out.ptr, q.ptr, k.ptr, v.ptr, kc.ptr, vc.ptr)

    ms = time_steps(eng, step, steps, warmup)
    k_ms, k_n = kernel_avg_ms(eng, step, steps, tla.KERNEL_PREFILL)
    a_ms, _ = kernel_avg_ms(eng, step, steps, tla.KERNEL_APPEND)
    flops = case.algorithmic_flops
    achieved = flops / (k_ms * 1e-3) / 1e12
    res = {"workload": "prefill", "metric": "prefill-attn TFLOP/s (% MFMA peak)",
           "value": flops / (ms * 1e-3) / 1e12, "unit": "TFLOP/s", "ms_per_step": ms,
           "warmup": warmup,
           "algorithmic_flops": flops, "prefill_kernel_ms": k_ms, "append_kernel_ms": a_ms,
           "roofline": {"bound": "mfma", "achieved": round(achieved, 2),
                        "peak": round(PREFILL_PEAK_TFLOPS, 1), "unit": "TFLOP/s",
                        "frac": round(achieved / PREFILL_PEAK_TFLOPS, 4),
                        "peak_basis": f"bf16 dense {BF16_MFMA_PEAK_TFLOPS:.0f} TFLOP/s over "
                                      f"{PREFILL_SPLIT_PRODUCTS} bf16 products per fp32-accurate "
                                      "multiply-add",
                        "frac_of_fp32_mfma_peak": round(achieved / FP32_MFMA_PEAK_TFLOPS, 4),
                        "traffic": profiled_traffic("prefill_attention_kernel", "prefill"),
                        "algorithmic_flops": flops,
                        "kernel": "prefill_attention_kernel", "launches": k_n}}
    log(f"[bench] {label}: {ms * 1e3:.1f} us/step ({res['value']:.1f} TFLOP/s), attention kernel "
        f"{k_ms * 1e3:.1f} us -> {achieved:.1f} TFLOP/s fp32-accurate ({achieved / PREFILL_PEAK_TFLOPS:.1%} "
        f"of the split-bf16 ceiling {PREFILL_PEAK_TFLOPS:.0f}; {achieved / FP32_MFMA_PEAK_TFLOPS:.1%} of "
        f"the fp32 MFMA peak), append {a_ms * 1e3:.1f} us")
    for a in (kc, vc, q, k, v, out):
        a.free()
    eng.close()
    if cpu:
        res["cpu_baseline"] = cpu_prefill_baseline(case, n_tok)
    return res


def run_prefill_sweep(steps, warmup, lengths=(512, 1024, 2048, 4096), n_layers=22):
    """Causal prefill of one prompt of each length over n_layers layers in
    one launch (Q/K/V N(0,1), seeded): the attention kernel's TFLOP/s as the
    prompt grows."""
    out = []
    for n_tok in lengths:
        r = run_prefill(steps, warmup, False, n_layers, n_tok,
                        label=f"prefill {n_tok} tokens" + ("" if n_layers == 22 else f", {n_layers} layer(s)"))
        out.append({"n_tok": n_tok, "us": round(r["prefill_kernel_ms"] * 1e3, 2),
                    "flops": r["algorithmic_flops"], "TFLOP_s": r["roofline"]["achieved"],
                    "frac": r["roofline"]["frac"]})
    return out


def cpu_prefill_baseline(case, n_tok, budget_s=8.0):
    """The reference's own token-by-token prompt loop -- its rope() and
    attention() compiled from src/ops.cpp (oracle/_ref), or the C restatement
    when that is not built -- one layer per host thread (the reference's
    attention() has no threading)."""
    from concurrent.futures import ThreadPoolExecutor

    import oracle as O
    kind = "reference" if O.ref_available() else "port"
    lib = O.ref() if kind == "reference" else None
    s = O.Shape(n_ctx=n_tok, n_layers=1)
    threads = cpu_threads()
    times = []
    t_end = time.perf_counter() + budget_s
    with ThreadPoolExecutor(threads) as ex:
        while True:
            t0 = time.perf_counter()

            def one(layer):
                kc = np.zeros(n_tok * 256, np.float32)
                vc = np.zeros_like(kc)
                O.prefill(case.q[layer], case.k[layer], case.v[layer], kc, vc, 0, 0, s, lib=lib)

            list(ex.map(one, range(case.n_layers)))
            times.append(time.perf_counter() - t0)
            if time.perf_counter() > t_end:
                break
    t = median(times)
    log(f"[bench] cpu prefill {kind}: {t * 1e3:.0f} ms/step on {threads} threads")
    return {"value": round(case.algorithmic_flops / t / 1e12, 5), "unit": "TFLOP/s",
            "cores": threads, "kind": kind,
            "sample": f"{len(times)} full prefill steps (512 tokens x {case.n_layers} layers, one "
                      f"layer per thread), median", **cpu_host()}


# -------------------------------------------------------------------- copy --

def run_copy(steps, warmup, nbytes=1 << 30):
    """Device copy kernel over nbytes: the known-size reference for scaling
    rocprofv3 FETCH_SIZE / WRITE_SIZE."""
    eng = tla.Engine(tla.Config.tinyllama(n_layers=1, n_ctx=16))
    a = tla.DeviceArray(eng, (nbytes,), np.uint8)
    b = tla.DeviceArray(eng, (nbytes,), np.uint8)
    ms = time_steps(eng, lambda i: eng.copy(b.ptr, a.ptr, nbytes), steps, warmup)
    log(f"[bench] copy {nbytes >> 20} MiB: {ms * 1e3:.1f} us, {2 * nbytes / ms / 1e6:.0f} GB/s")
    a.free()
    b.free()
    eng.close()
    return {"workload": "copy", "bytes_read": nbytes, "bytes_written": nbytes, "ms": ms,
            "value": 2 * nbytes / (ms * 1e-3) / 1e9}


def run_proj(steps, warmup, n_layers=22, wtype=W.W_F16):
    """The attention block's projections for one decode step of every layer,
    issued as a forward pass issues them: per layer, one fused
    rmsnorm + Wq/Wk/Wv launch (tla_attn_qkv) and one Wo + residual launch
    (tla_attn_out), batch 1.  Weights are distinct per layer (F16: 415 MB,
    beyond the 256 MB Infinity Cache).  Also the GEMV kernel alone on a
    vocabulary-sized matrix (32000 x 2048, the output projection's shape) in
    every weight format."""
    embd, kv = 2048, 256
    eng = tla.Engine(tla.Config.tinyllama(n_layers=n_layers, n_ctx=16))
    arrays = []

    def dev(a):
        d = eng.array(a)
        arrays.append(d)
        return d

    layers = []
    for layer in range(n_layers):
        layers.append({"wq": dev(W.make_weights(wtype, embd, embd, salt=4 * layer)),
                       "wk": dev(W.make_weights(wtype, kv, embd, salt=4 * layer + 1)),
                       "wv": dev(W.make_weights(wtype, kv, embd, salt=4 * layer + 2)),
                       "wo": dev(W.make_weights(wtype, embd, embd, salt=4 * layer + 3)),
                       "nw": dev(np.ones(embd, np.float32))})
    rg = np.random.default_rng(0)
    x = dev(rg.standard_normal(embd).astype(np.float32))
    xb2 = dev(rg.standard_normal(embd).astype(np.float32))
    q, k, v = dev(np.zeros(embd, np.float32)), dev(np.zeros(kv, np.float32)), dev(np.zeros(kv, np.float32))
    step_bytes = n_layers * (2 * W.weight_row_bytes(wtype, embd) * embd
                             + 2 * W.weight_row_bytes(wtype, embd) * kv)

    def step(i):
        for L in layers:
            eng.attn_qkv(1, q.ptr, k.ptr, v.ptr, x.ptr, L["nw"].ptr, 1e-5, L["wq"].ptr, L["wk"].ptr,
                         L["wv"].ptr, wtype)
            eng.attn_out(1, x.ptr, L["wo"].ptr, xb2.ptr, wtype)

    ms = time_steps(eng, step, steps, warmup)
    # the same steps queued behind a blocker: the GPU's own time per step
    # (a step is 44 Python calls, about 5 us of host time each)
    dev_ms = back_to_back_ms(eng, step, steps, blocker_ms=steps * 2 * n_layers * 0.008)
    k_ms, k_n = kernel_avg_ms(eng, step, max(2, steps // 5), tla.KERNEL_GEMV)
    log(f"[bench] proj {W.W_NAMES[wtype]} x {n_layers} layers, batch 1: {ms * 1e3:.1f} us/step "
        f"as issued from Python, {dev_ms * 1e3:.1f} us/step queued back to back; "
        f"{step_bytes / 1e6:.0f} MB of weights -> {step_bytes / dev_ms / 1e6:.0f} GB/s; "
        f"per-launch events {k_ms * 1e3:.2f} us")
    for a in arrays:
        a.free()
    # the GEMV kernel alone on one large matrix, each format
    big = {}
    for t in (W.W_F32, W.W_F16, W.W_Q8_0, W.W_Q4_0, W.W_Q6_K):
        big[W.W_NAMES[t]] = matmul_kernel(eng, t, steps, warmup)
    eng.close()
    value = step_bytes / (dev_ms * 1e-3) / 1e9
    return {"workload": "proj", "metric": "attention-block projection weight GB/s (% HBM peak)",
            "value": value, "unit": "GB/s", "ms_per_step": dev_ms, "end_to_end_ms": ms,
            "weight_bytes": step_bytes, "launch_us": round(k_ms * 1e3, 2), "launches": k_n,
            "roofline": {"bound": "hbm", "achieved": big["q8_0"]["GB_s"], "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": big["q8_0"]["frac"],
                         "traffic": profiled_traffic("gemv_kernel", "matmul_q8_0"),
                         "kernel": "gemv_kernel", "config": "matmul q8_0 32000x2048"},
            "matmul_32000x2048": big}


def matmul_kernel(eng, t, steps, warmup, rows=32000, cols=2048):
    """The GEMV kernel alone on a vocabulary-sized matrix (rows x cols, the
    output projection's shape) in weight format t, with enough rotated
    copies of the weights to exceed the Infinity Cache; timed per launch."""
    rg = np.random.default_rng(1)
    wd = eng.array(W.make_weights(t, rows, cols, salt=99))
    xd = eng.array(rg.standard_normal(cols).astype(np.float32))
    od = eng.array((rows,))
    nbytes = W.weight_row_bytes(t, cols) * rows
    copies = 1
    extra = []
    if nbytes < 300e6:
        copies = int(np.ceil(300e6 / nbytes))
        extra = [eng.array(W.make_weights(t, rows, cols, salt=100 + c)) for c in range(copies - 1)]
    ws = [wd] + extra

    def one(i):
        eng.matmul(od.ptr, ws[i % copies].ptr, xd.ptr, rows, cols, t)

    # A Python call per launch costs about as much as the kernel, so the
    # launches are queued behind a blocker and timed back to back; the HIP
    # event pair around each launch (which adds the events' own cost) is
    # reported beside.
    for i in range(warmup):
        one(i)
    t_ms = back_to_back_ms(eng, one, steps)
    ev_ms, _ = kernel_avg_ms(eng, one, steps, tla.KERNEL_GEMV)
    out = {"us": round(t_ms * 1e3, 2), "bytes": nbytes, "GB_s": round(nbytes / t_ms / 1e6, 1),
           "frac": round(nbytes / t_ms / 1e6 / HBM_PEAK_GBS, 4), "ms": t_ms,
           "per_launch_event_us": round(ev_ms * 1e3, 2)}
    log(f"[bench] matmul {W.W_NAMES[t]} {rows}x{cols}: {t_ms * 1e3:.1f} us back to back, "
        f"{nbytes / t_ms / 1e6:.0f} GB/s ({nbytes / t_ms / 1e6 / HBM_PEAK_GBS:.1%}), "
        f"{copies} rotated copies; per-launch events {ev_ms * 1e3:.1f} us")
    for a in [wd, xd, od] + extra:
        a.free()
    return out


def batch_product_tflops(eng, t, steps, rows=5632, cols=2048, n_tok=512):
    """tla_matmul_batch on one matrix (the FFN gate shape by default) for a
    token batch, back to back: fp32-accurate TFLOP/s (2 n rows cols over
    the time).  The product runs on the bf16 matrix cores, 3 bf16 products
    per multiply-add for Q4_0 / Q8_0, 5 for F16 / Q6_K, 6 for F32; the share
    of the bf16 peak those execute is printed beside it."""
    rg = np.random.default_rng(2)
    wd = eng.array(W.make_weights(t, rows, cols, salt=7))
    xd = eng.array(rg.standard_normal((n_tok, cols)).astype(np.float32))
    od = eng.array((n_tok, rows))

    def one(i):
        eng.matmul_batch(od.ptr, wd.ptr, xd.ptr, rows, cols, n_tok, t)

    for i in range(3):
        one(i)
    ms = back_to_back_ms(eng, one, steps)
    flops = 2 * n_tok * rows * cols
    bf16 = SPLIT_PRODUCTS[t] * flops / ms / 1e9
    log(f"[bench] matmul_batch {W.W_NAMES[t]} {rows}x{cols} x {n_tok} tokens: {ms * 1e3:.1f} us, "
        f"{flops / ms / 1e9:.1f} TFLOP/s fp32-accurate ({SPLIT_PRODUCTS[t]} bf16 products each: "
        f"{bf16:.0f} TFLOP/s, {bf16 / BF16_MFMA_PEAK_TFLOPS:.1%} of the bf16 MFMA peak)")
    for a in (wd, xd, od):
        a.free()
    return {"us": round(ms * 1e3, 2), "TFLOP_s": round(flops / ms / 1e9, 2),
            "bf16_TFLOP_s": round(bf16, 1)}


def run_matmul(steps, warmup, name):
    t = {v: k for k, v in W.W_NAMES.items()}[name]
    eng = tla.Engine(tla.Config.tinyllama(n_layers=1, n_ctx=16))
    r = matmul_kernel(eng, t, steps, warmup)
    if t != W.W_Q6_K:
        r["batch512"] = batch_product_tflops(eng, t, steps)
    eng.close()
    return r


GEN_FORMATS = {"q4_0": (W.W_Q4_0, W.W_Q6_K), "q8_0": (W.W_Q8_0, W.W_Q8_0), "f16": (W.W_F16, W.W_F16)}


def run_generate(steps, warmup, cpu, wname="q4_0", n_prompt=32, n_gen=20):
    """The reference's own benchmark (run_trial, src/benchmark.cpp:113-165)
    on TinyLlama's shapes with seeded random weights in the layout of the
    TinyLlama GGUF files (Q4_0 weights with a Q6_K classifier, or Q8_0 / F16
    throughout): a 32-token prompt through forward(), then 20 greedy decode
    steps, as one tla_generate_greedy call on the device.  Prefill time =
    the call with one generated token; decode ms/token = (the call with 21)
    minus that, over 20.  HIP events on the engine's stream bracket each
    call, which returns after its last copy, so host time between launches
    is inside the figure."""
    wt, ot = GEN_FORMATS[wname]
    spec = W.tinyllama_spec(n_ctx=2048)
    t = W.make_model(spec, wt, salt=5, output_type=ot)
    eng = tla.Engine(tla.Config.tinyllama(n_ctx=spec.n_ctx))
    dm = tla.DeviceModel(eng, t, spec.n_ff, spec.n_vocab, spec.rms_norm_eps)
    kc, vc = eng.kv_cache(1)
    prompt = [1] + W.rng("block", 3).integers(2, spec.n_vocab, n_prompt - 1).tolist()

    def call(n, batch=False):
        eng.synchronize()
        eng.event(0)
        toks = eng.generate_greedy(dm, kc.ptr, vc.ptr, prompt, n, batch_prompt=batch)
        eng.event(1)
        return eng.elapsed(0, 1), toks

    for _ in range(max(1, warmup)):
        call(n_gen + 1)
        call(1, True)
    trials = max(3, steps // 5)
    pre = median([call(1)[0] for _ in range(trials)])
    pre_batch = median([call(1, True)[0] for _ in range(trials)])
    full = median([call(n_gen + 1)[0] for _ in range(trials)])
    dec = (full - pre) / n_gen
    _, toks = call(n_gen + 1)
    _, toks_b = call(n_gen + 1, True)
    log(f"[bench] generate {wname}: prompt as one batch {pre_batch:.2f} ms "
        f"({pre_batch / n_prompt * 1e3:.0f} us/token); same tokens: {toks_b == toks}")
    # a long prompt as one batch (tla_prefill_forward): the projections as
    # batched products; flops = 2 x tokens x (every matrix's rows x cols)
    # over the layers
    n_long = 512
    long_prompt = [1] + W.rng("block", 4).integers(2, spec.n_vocab, n_long - 1).tolist()
    lg = eng.array((spec.n_vocab,))
    for _ in range(2):
        eng.prefill_forward(dm, kc.ptr, vc.ptr, long_prompt, 0, lg.ptr)
    eng.synchronize()
    eng.event(0)
    reps = 3
    for _ in range(reps):
        eng.prefill_forward(dm, kc.ptr, vc.ptr, long_prompt, 0, lg.ptr)
    eng.event(1)
    long_ms = eng.elapsed(0, 1) / reps
    lg.free()
    e_, kvd, ff = spec.n_embd, spec.kv_dim, spec.n_ff
    gemm_flops = 2 * n_long * spec.n_layers * e_ * (e_ + 2 * kvd + e_ + 2 * ff + ff)
    log(f"[bench] generate {wname}: {n_long}-token prompt as one batch {long_ms:.2f} ms "
        f"= {n_long / long_ms * 1e3:.0f} tokens/s; projections {gemm_flops / 1e9:.0f} GFLOP "
        f"-> {gemm_flops / long_ms / 1e9:.1f} TFLOP/s overall")
    # HBM bytes a decode token must move: every weight once (one embedding
    # row), the KV cache up to its position (mean position of the 20 steps)
    weight_bytes = sum(len(r) for name, (d, ty, r) in t.items() if name != "token_embd.weight")
    weight_bytes += W.weight_row_bytes(t["token_embd.weight"][1], spec.n_embd)
    mean_pos = n_prompt + (n_gen - 1) / 2
    kv_bytes = spec.n_layers * 2 * spec.kv_dim * 4 * (mean_pos + 1)
    tok_bytes = weight_bytes + kv_bytes
    gbs = tok_bytes / dec / 1e6
    log(f"[bench] generate {wname}: prefill {n_prompt} tokens {pre:.2f} ms ({pre / n_prompt * 1e3:.0f} "
        f"us/token), decode {dec * 1e3:.0f} us/token = {1e3 / dec:.0f} tok/s; {tok_bytes / 1e6:.0f} MB "
        f"per token -> {gbs:.0f} GB/s ({gbs / HBM_PEAK_GBS:.1%}); tokens {toks[:8]}...")
    res = {"decode_ms_per_token": dec, "prefill_ms": pre, "prefill_batched_ms": pre_batch,
           "prompt512_ms": long_ms,
           "tok_per_s": 1e3 / dec,
           "bytes_per_token": tok_bytes, "GB_s": gbs, "frac": gbs / HBM_PEAK_GBS,
           "n_prompt": n_prompt, "n_gen": n_gen}
    dm.free()
    kc.free()
    vc.free()
    eng.close()
    if cpu:
        res["cpu_baseline"] = cpu_generate_baseline(spec, t, prompt, wname)
    return res


def cpu_generate_baseline(spec, tensors, prompt, wname, n_prompt=8, n_decode=8):
    """The reference's own forward pass and benchmark loop (oracle/_ref,
    built from src/forward.cpp, gguf_model.cpp, tokenizer.cpp, ops.cpp) over
    a GGUF file of the same model, on the host: a bounded sample (8 prompt
    tokens, 8 decode tokens) with its thread pool at the host's cores, and 4
    decode tokens on one thread."""
    import tempfile

    import oracle as O
    if not O.ref_forward_available():
        return None
    write_gguf = importlib.import_module("tinyllama-engine_amd.gguf_writer").write_gguf
    threads = cpu_threads()
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "model.gguf")
        write_gguf(path, spec, tensors)
        _, dn = O.ref_bench_trial(path, prompt[:n_prompt], n_decode, threads)
        _, d1 = O.ref_bench_trial(path, prompt[:2], 4, 1)
    ms_n, ms_1 = dn / n_decode, d1 / 4
    log(f"[bench] cpu reference forward {wname}: {threads} threads {ms_n:.0f} ms/token, "
        f"1 thread {ms_1:.0f} ms/token")
    return {"value": round(1e3 / ms_n, 3), "unit": "tok/s", "cores": threads, "kind": "reference",
            "sample": f"reference forward(), {n_prompt} prompt + {n_decode} decode tokens, "
                      f"{threads} threads; 1 thread: 4 decode tokens",
            "ms_per_token": round(ms_n, 2), "single_thread_ms_per_token": round(ms_1, 2),
            **cpu_host()}


DROPIN_DIR = os.path.join(ROOT, "tinyllama-engine_amd", "_dropin")
# one token per byte with the model's byte vocabulary (no spaces: each would
# be three bytes of U+2581)
DROPIN_PROMPT = "attentionblocksonthedevice" * 15


def run_benchmark_program(prog, model, threads, trials, warmup, decode_tokens, prompt):
    """One run of the reference's benchmark program (src/benchmark.cpp:265-401)
    in its CSV mode; returns its row as a dict."""
    import subprocess
    cmd = [prog, model, "--threads", str(threads), "--trials", str(trials), "--warmup", str(warmup),
           "--decode-tokens", str(decode_tokens), "--prompt", prompt, "--csv"]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=900)
    if r.returncode != 0:
        raise RuntimeError(f"{os.path.basename(prog)} failed ({r.returncode}): {r.stderr[-2000:]}")
    row = r.stdout.strip().splitlines()[-1].split(",")
    # label, backend, threads, quant, prompt tokens, decode tokens, prefill ms,
    # prefill tok/s, decode ms/token, decode tok/s (src/benchmark.cpp:188-203)
    return {"threads": int(row[2]), "prompt_tokens": int(row[4]), "decode_tokens": int(row[5]),
            "prefill_ms": float(row[6]), "prefill_tok_s": float(row[7]), "decode_ms_per_token": float(row[8]),
            "decode_tok_s": float(row[9])}


def attention_block_cost(n_ctx, pos, reps=2000):
    """What one attention block of the drop-in costs the reference's
    forward() at position `pos`, as tla_host::attention_block makes it:
    tla_rope_attention_host from RunState's pinned host buffers (the 10 KiB
    upload of q|k|v, the fused RoPE + append + attention launch, the 8 KiB
    download of the output, one synchronization), called here through the
    C ABI from Python, against the launch alone queued back to back."""
    import ctypes as C
    eng = tla.Engine(tla.Config.tinyllama(n_layers=1, n_ctx=n_ctx))
    cfg = eng.cfg
    kc, vc = eng.kv_cache(1)
    n_qkv = cfg.n_embd + 2 * cfg.kv_dim
    qkv_host = eng.host_alloc(4 * n_qkv)
    out_host = eng.host_alloc(4 * cfg.n_embd)
    vals = np.random.default_rng(9).standard_normal(n_qkv).astype(np.float32)
    C.memmove(qkv_host, vals.ctypes.data, vals.nbytes)
    qkv = eng.array((n_qkv,))
    out = eng.array((cfg.n_embd,))
    dq, dk, dv = qkv.ptr, qkv.ptr + 4 * cfg.n_embd, qkv.ptr + 4 * (cfg.n_embd + cfg.kv_dim)
    lib = tla.lib()

    def block():
        lib.tla_rope_attention_host(eng.h, out_host, qkv_host, qkv.ptr, out.ptr, kc.ptr, vc.ptr, 0, pos)

    for _ in range(50):
        block()
    t0 = time.perf_counter()
    for _ in range(reps):
        block()
    block_us = (time.perf_counter() - t0) / reps * 1e6
    kernel_us = back_to_back_ms(eng, lambda i: eng.rope_attention(out.ptr, dq, dk, dv, kc.ptr, vc.ptr, 0, pos),
                                reps) * 1e3
    for a in (kc, vc, qkv, out):
        a.free()
    eng.host_free(qkv_host)
    eng.host_free(out_host)
    eng.close()
    return {"block_us": round(block_us, 2), "kernel_us": round(kernel_us, 2),
            "staging_us": round(block_us - kernel_us, 2)}


def run_dropin(trials=1, warmup=0, decode_tokens=16, cpu=True):
    """The reference's own benchmark program (run_trial,
    src/benchmark.cpp:113-165: the prompt token by token through forward(),
    then greedy decode steps) built on the drop-in attention path
    (tinyllama-engine_amd/_dropin/benchmark_dropin: run_state.h and the block
    of src/forward.cpp:192-208 replaced, every token's RoPE, cache append
    and attention on the GPU, everything else the reference's on the host
    cores), on TinyLlama's shapes with seeded random weights in the
    TinyLlama Q4_0 file's layout; the reference's unmodified build
    (benchmark_ref) on the same file and host threads is the CPU baseline."""
    import tempfile
    gw = importlib.import_module("tinyllama-engine_amd.gguf_writer")
    prog = os.path.join(DROPIN_DIR, "benchmark_dropin")
    if not os.access(prog, os.X_OK):
        raise RuntimeError("benchmark_dropin is not built (build() builds it where the reference's "
                           "sources are)")
    threads = cpu_threads()
    wt, ot = GEN_FORMATS["q4_0"]
    spec = W.tinyllama_spec(n_ctx=2048)
    t = W.make_model(spec, wt, salt=5, output_type=ot)
    res = {}
    with tempfile.TemporaryDirectory() as d:
        model = os.path.join(d, "model.gguf")
        gw.write_gguf(model, spec, t, vocab=gw.byte_vocab(spec.n_vocab))
        del t
        r = run_benchmark_program(prog, model, threads, trials, warmup, decode_tokens, DROPIN_PROMPT)
        log(f"[bench] dropin: reference benchmark on the drop-in, {threads} threads, Q4_0 TinyLlama shapes: "
            f"prompt {r['prompt_tokens']} tokens {r['prefill_ms']:.0f} ms ({r['prefill_tok_s']:.1f} tok/s), "
            f"decode {r['decode_ms_per_token']:.2f} ms/token ({r['decode_tok_s']:.1f} tok/s)")
        res.update(r)
        if cpu:
            import oracle as O
            ref = os.path.join(O.HERE, "_ref", "benchmark_ref")
            if os.access(ref, os.X_OK):
                c = run_benchmark_program(ref, model, threads, trials, warmup, decode_tokens, DROPIN_PROMPT)
                log(f"[bench] dropin cpu reference: prompt {c['prefill_ms']:.0f} ms "
                    f"({c['prefill_tok_s']:.1f} tok/s), decode {c['decode_ms_per_token']:.2f} ms/token "
                    f"({c['decode_tok_s']:.1f} tok/s)")
                res["cpu_baseline"] = {"value": c["decode_tok_s"], "unit": "tok/s", "cores": threads,
                                       "kind": "reference",
                                       "sample": f"the reference's benchmark program unmodified, same model and "
                                                 f"prompt, {trials} trial(s), {decode_tokens} decode tokens",
                                       **c, **cpu_host()}
    pos = res["prompt_tokens"] + decode_tokens // 2
    res["attention_block"] = {"pos": pos, **attention_block_cost(2048, pos)}
    b = res["attention_block"]
    log(f"[bench] dropin: one attention block at position {pos}: {b['block_us']:.1f} us with its host "
        f"copies, {b['kernel_us']:.1f} us for the launch alone -> {b['staging_us']:.1f} us of staging per "
        f"layer, {b['staging_us'] * spec.n_layers / 1e3:.2f} ms per token over {spec.n_layers} layers")
    return res


READ_FLOOR_GRIDS = (256, 512, 1024, 2048, 4096, 8192, 16384)
READ_FLOOR_KINDS = {"global": 0, "global_nt": 1, "buffer": 2, "buffer_nt": 3}
READ_FLOOR_DEPTHS = (8, 16, 32)
# the 8-sequence x 16384-position x 22-layer step (decode_long)'s algorithmic bytes
DECODE_LONG_BYTES = 8 * 22 * (2048 * 16384 + 20480)


def read_floor_sizes(contexts=(2048, 4096, 8192, 16384), n_layers=22, long=True):
    sizes = [(f"ctx {ctx}", ctx, W.decode_bytes(ctx) * n_layers) for ctx in contexts]
    if long:
        sizes.append(("decode_long", 16384, DECODE_LONG_BYTES))
    return sizes


def run_read_floor(steps, warmup, sizes=None, kinds=None, depths=READ_FLOOR_DEPTHS,
                   grids=READ_FLOOR_GRIDS):
    """The hand-written streaming read (tla_read_floor) over exactly the bytes
    a decode step moves: batch 1 x 22 layers at each context (2048*L + 20480
    per layer) and the 8 x 16384 x 22 step, launches rotating over copies past
    the Infinity Cache and queued back to back; the best of every load form,
    depth and grid size.  What one launch can read in the time it takes: the
    bar for the decode kernel at that size."""
    sizes = read_floor_sizes() if sizes is None else sizes
    kinds = READ_FLOOR_KINDS if kinds is None else kinds
    eng = tla.Engine(tla.Config.tinyllama(n_layers=1, n_ctx=16))
    sink = eng.array((max(grids),))
    out = []
    for label, ctx, nbytes in sizes:
        span = (nbytes + 255) // 256 * 256
        copies = max(1 if nbytes > 4 * MALL_BYTES else 2, -(-3 * MALL_BYTES // 2 // nbytes))
        buf = tla.DeviceArray(eng, (span * copies,), np.uint8)
        best, by_kind = None, {}
        for kname, kind in kinds.items():
            for depth in depths:
                for grid in grids:
                    def one(i, grid=grid, kind=kind, depth=depth):
                        eng.read_floor(buf.ptr + (i % copies) * span, nbytes, grid, sink.ptr, kind, depth)
                    for i in range(warmup):
                        one(i)
                    ms = back_to_back_ms(eng, one, steps)
                    cand = (ms, kname, depth, grid)
                    if best is None or ms < best[0]:
                        best = cand
                    if kname not in by_kind or ms < by_kind[kname][0]:
                        by_kind[kname] = cand
        ms, kname, depth, grid = best
        gbs = nbytes / (ms * 1e-3) / 1e9
        log(f"[bench] read floor {nbytes / 1e6:.1f} MB ({label}): {ms * 1e3:.2f} us with {grid} workgroups, "
            f"{kname} loads, {depth} per thread in flight -> {gbs:.0f} GB/s ({gbs / HBM_PEAK_GBS:.1%}), "
            f"{copies} rotated copies; best per load form: "
            + ", ".join(f"{k} {v[0] * 1e3:.2f} us ({v[2]} deep, {v[3]} wg)" for k, v in by_kind.items()))
        out.append({"size": label, "ctx": ctx, "bytes": nbytes, "us": round(ms * 1e3, 2),
                    "GB_s": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4), "workgroups": grid,
                    "load": kname, "depth": depth, "copies": copies,
                    "best_by_load": {k: {"us": round(v[0] * 1e3, 2), "depth": v[2], "workgroups": v[3]}
                                     for k, v in by_kind.items()}})
        buf.free()
    sink.free()
    eng.close()
    return out


MFMA_FLOOR_GRIDS = (768, 1024, 2048)
MFMA_FLOOR_WG_FLOPS = 4 * 16 * 2 * 32 * 32 * 16  # per workgroup and round: 4 waves x 16 MFMAs


def prefill_executed_flops(n_tok=512, n_layers=22, n_head=32, tile=32, head_dim=64):
    """bf16 MFMA flops the prefill kernel executes (diagonal tiles whole):
    per (layer, head), n_qt (n_qt + 1) / 2 tile pairs of 32 queries x 32 keys,
    two products of 2 x 32 x 32 x head_dim flops each, each product as six
    products of bf16 pieces."""
    n_qt = -(-n_tok // tile)
    return (n_layers * n_head * n_qt * (n_qt + 1) // 2 * 2 * (2 * tile * tile * head_dim)
            * PREFILL_SPLIT_PRODUCTS)


def run_mfma_floor(steps, warmup, flops=None):
    """The hand-written MFMA loop (tla_mfma_floor) executing as many
    v_mfma_f32_32x32x16_bf16 flops as the 512-token, 22-layer prefill kernel
    (its diagonal tiles counted whole), launches back to back; the best of a
    few grid sizes, each after the prefill workload's warmup.  What one
    launch can execute in the time it takes: the bar for the prefill
    kernel."""
    flops = flops or prefill_executed_flops()
    warmup = max(warmup, PREFILL_MIN_WARMUP)  # the clocks ramp under sustained MFMA work
    eng = tla.Engine(tla.Config.tinyllama(n_layers=1, n_ctx=16))
    sink = eng.array((max(MFMA_FLOOR_GRIDS),))
    best = None
    for grid in MFMA_FLOOR_GRIDS:
        iters = max(1, round(flops / (grid * MFMA_FLOOR_WG_FLOPS)))

        def one(i, grid=grid, iters=iters):
            eng.mfma_floor(grid, iters, sink.ptr)
        for i in range(warmup):
            one(i)
        ms = back_to_back_ms(eng, one, steps)
        done = grid * iters * MFMA_FLOOR_WG_FLOPS
        tf = done / (ms * 1e-3) / 1e12
        if best is None or tf > best["TFLOP_s"]:
            best = {"flops": done, "us": round(ms * 1e3, 2), "TFLOP_s": round(tf, 2),
                    "frac": round(tf / BF16_MFMA_PEAK_TFLOPS, 4), "workgroups": grid, "iters": iters}
    log(f"[bench] mfma floor {best['flops'] / 1e9:.2f} GFLOP (the 512-token prefill kernel's executed "
        f"bf16 MFMA work): {best['us']:.1f} us with {best['workgroups']} workgroups -> "
        f"{best['TFLOP_s']:.1f} TFLOP/s ({best['frac']:.1%} of {BF16_MFMA_PEAK_TFLOPS:.0f})")
    sink.free()
    eng.close()
    return best


def run_read(steps, warmup, nbytes=6 << 30):
    """HBM read ceiling: torch's sum over an nbytes float32 tensor (a library
    streaming reduction, none of this package's kernels), timed with events on torch's
    current stream, which is where it runs."""
    import torch
    x = torch.ones(nbytes // 4, dtype=torch.float32, device="cuda")
    for _ in range(warmup):
        x.sum()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(steps):
        x.sum()
    b.record()
    b.synchronize()
    ms = a.elapsed_time(b) / steps
    log(f"[bench] read {nbytes >> 20} MiB (torch sum): {ms * 1e3:.1f} us, {nbytes / ms / 1e6:.0f} GB/s")
    del x
    return {"workload": "read", "bytes_read": nbytes, "ms": ms, "value": nbytes / (ms * 1e-3) / 1e9}


# -------------------------------------------------------------------- main --

PLANS = {"auto": tla.PLAN_AUTO, "aligned": tla.PLAN_ALIGNED, "balanced": tla.PLAN_BALANCED}


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", default="decode_model",
                    choices=["decode_model", "decode_long", "decode_ragged", "decode_single",
                             "prefill", "proj", "matmul", "generate", "decode_sweep",
                             "prefill_sweep", "prefill_layer_sweep", "copy", "read", "read_floor", "mfma_floor",
                             "dropin"])
    ap.add_argument("--wtype", default=None, choices=["f32", "f16", "q8_0", "q4_0", "q6_k"],
                    help="weight format of the matmul (default q8_0) or generate (q4_0) workload")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-prefill", action="store_true", help="skip the prefill half")
    ap.add_argument("--split", type=int, default=0, help="decode positions per workgroup (0 = auto)")
    ap.add_argument("--plan", default="auto", choices=["auto", "aligned", "balanced"],
                    help="decode work plan (default: the engine's choice)")
    ap.add_argument("--extra", action="store_true",
                    help="(default) also measure decode_long, decode_ragged and decode_single")
    ap.add_argument("--no-extra", action="store_true",
                    help="skip the other decode workloads in the default line")
    ap.add_argument("--source-digest", metavar="KERNEL", choices=sorted(KERNEL_SOURCES),
                    help="print the digest of a kernel's sources (recorded in its profiles) and exit")
    args = ap.parse_args()
    if args.source_digest:
        print(kernel_source_digest(args.source_digest))
        return

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the library has no multi-GPU path "
              "(run with --gpus 1)", file=sys.stderr)
        sys.exit(2)
    cpu = not args.no_cpu

    if args.workload == "copy":
        print(json.dumps(run_copy(args.steps, args.warmup)))
        return
    if args.workload == "read":
        print(json.dumps(run_read(args.steps, args.warmup)))
        return
    if args.workload == "dropin":
        r = run_dropin(cpu=cpu)
        print(json.dumps({"metric": "decode tok/s of the reference's benchmark program on the drop-in",
                          "value": r["decode_tok_s"], "unit": "tok/s", "n_gpus": 1, "steps": r["decode_tokens"],
                          "warmup": 0, "ms_per_step": r["decode_ms_per_token"], "higher_is_better": True,
                          "scaling": "weak", "vs_baseline": None, "dtype": "q4_0 weights, f32 compute",
                          "data": "synthetic (seeded random weights)",
                          "config": {"workload": "dropin", "model": "TinyLlama-1.1B shapes", "weights": "q4_0",
                                     "prompt_tokens": r["prompt_tokens"], "threads": r["threads"],
                                     "parallelism": "none"},
                          "prefill_ms": r["prefill_ms"], "prefill_tok_s": r["prefill_tok_s"],
                          "attention_block": r["attention_block"],
                          "cpu_baseline": r.get("cpu_baseline")}))
        return
    if args.workload == "read_floor":
        r = run_read_floor(args.steps, args.warmup)
        print(json.dumps({"metric": "streaming-read floor GB/s (% HBM peak)", "value": r[0]["GB_s"],
                          "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
                          "ms_per_step": r[0]["us"] / 1e3, "higher_is_better": True, "scaling": "weak",
                          "vs_baseline": None, "dtype": "f32", "data": "synthetic",
                          "config": {"workload": "read_floor",
                                     "bytes": "decode batch 1 x 22 layers; decode_long",
                                     "sizes": [x["size"] for x in r], "parallelism": "none"},
                          "sweep": r}))
        return
    if args.workload == "mfma_floor":
        r = run_mfma_floor(args.steps, args.warmup)
        print(json.dumps({"metric": "bf16 MFMA floor TFLOP/s (% MFMA peak)", "value": r["TFLOP_s"],
                          "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
                          "ms_per_step": r["us"] / 1e3, "higher_is_better": True, "scaling": "weak",
                          "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
                          "config": {"workload": "mfma_floor",
                                     "flops": "the 512-token x 22-layer prefill kernel's executed MFMA work",
                                     "parallelism": "none"},
                          "roofline": {"bound": "mfma", "achieved": r["TFLOP_s"],
                                       "peak": BF16_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                                       "frac": r["frac"], "traffic": None},
                          "floor": r}))
        return
    if args.workload == "decode_sweep":
        r = run_decode_sweep(args.steps, args.warmup, plan=PLANS[args.plan])
        last = r[-1]
        print(json.dumps({"metric": HEADLINE_METRIC, "value": last["GB_s"], "unit": "GB/s",
                          "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
                          "ms_per_step": last["us"] / 1e3, "higher_is_better": True,
                          "scaling": "weak", "vs_baseline": None, "dtype": "f32",
                          "data": "synthetic",
                          "config": {"workload": "decode_sweep", "batch": 1, "n_layers": 22,
                                     "contexts": [x["ctx"] for x in r], "parallelism": "none"},
                          "sweep": r}))
        return
    if args.workload in ("prefill_sweep", "prefill_layer_sweep"):
        one = args.workload == "prefill_layer_sweep"
        n_layers = 1 if one else 22
        r = run_prefill_sweep(args.steps, args.warmup, (128, 256, 512, 1024, 2048) if one else
                              (512, 1024, 2048, 4096), n_layers)
        last = r[-1]
        print(json.dumps({"metric": HEADLINE_METRIC, "value": last["TFLOP_s"], "unit": "TFLOP/s",
                          "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
                          "ms_per_step": last["us"] / 1e3, "higher_is_better": True,
                          "scaling": "weak", "vs_baseline": None, "dtype": "f32",
                          "data": "synthetic",
                          "config": {"workload": args.workload, "batch": 1, "n_layers": n_layers,
                                     "lengths": [x["n_tok"] for x in r], "parallelism": "none"},
                          "sweep": r}))
        return
    if args.workload == "generate":
        wname = args.wtype or "q4_0"
        r = run_generate(args.steps, args.warmup, cpu, wname)
        line = {"metric": "decode tok/s (greedy, TinyLlama shapes)", "value": round(r["tok_per_s"], 1),
                "unit": "tok/s", "n_gpus": 1, "steps": r["n_gen"], "warmup": args.warmup,
                "ms_per_step": round(r["decode_ms_per_token"], 4), "higher_is_better": True,
                "scaling": "weak", "vs_baseline": None, "dtype": f"{wname} weights, f32 compute",
                "data": "synthetic (seeded random weights)",
                "config": {"workload": "generate", "model": "TinyLlama-1.1B shapes", "weights": wname,
                           "prompt_tokens": r["n_prompt"], "decode_tokens": r["n_gen"], "batch": 1,
                           "parallelism": "none"},
                "prefill_ms": round(r["prefill_ms"], 3),
                "prefill_batched_ms": round(r["prefill_batched_ms"], 3),
                "prompt512_ms": round(r["prompt512_ms"], 3),
                "roofline": {"bound": "hbm", "achieved": round(r["GB_s"], 1), "peak": HBM_PEAK_GBS,
                             "unit": "GB/s", "frac": round(r["frac"], 4), "traffic": None,
                             "kernel": "whole decode step (113 launches)",
                             "bytes_per_token": int(r["bytes_per_token"])}}
        if r.get("cpu_baseline"):
            line["cpu_baseline"] = r["cpu_baseline"]
        print(json.dumps(line))
        return
    if args.workload == "matmul":
        args.wtype = args.wtype or "q8_0"
        r = run_matmul(args.steps, args.warmup, args.wtype)
        line = {"metric": "GEMV weight GB/s", "value": r["GB_s"], "unit": "GB/s", "n_gpus": 1,
                "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(r["ms"], 5),
                "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
                "dtype": args.wtype, "data": "synthetic",
                "config": {"workload": "matmul", "rows": 32000, "cols": 2048, "weights": args.wtype,
                           "batch": 1, "parallelism": "none"},
                "roofline": {"bound": "hbm", "achieved": r["GB_s"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                             "frac": r["frac"],
                             "traffic": profiled_traffic("gemv_kernel", f"matmul_{args.wtype}")}}
        print(json.dumps(line))
        return
    if args.workload == "proj":
        p = run_proj(args.steps, args.warmup)
        line = {"metric": p["metric"], "value": round(p["value"], 1), "unit": "GB/s", "n_gpus": 1,
                "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(p["ms_per_step"], 4),
                "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f16",
                "data": "synthetic",
                "config": {"workload": "proj", "n_layers": 22, "n_embd": 2048, "kv_dim": 256,
                           "weights": "f16", "batch": 1, "parallelism": "none"},
                "roofline": p["roofline"], "launch_us": p["launch_us"],
                "end_to_end_ms": round(p["end_to_end_ms"], 4),
                "matmul_32000x2048": p["matmul_32000x2048"]}
        print(json.dumps(line))
        return
    if args.workload == "prefill":
        p = run_prefill(args.steps, args.warmup, cpu)
        line = {"metric": HEADLINE_METRIC, "value": round(p["value"], 3), "unit": "TFLOP/s",
                "n_gpus": 1, "steps": args.steps, "warmup": p["warmup"],
                "ms_per_step": round(p["ms_per_step"], 4), "higher_is_better": True,
                "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
                "config": {"workload": "prefill", "n_tok": 512, "n_layers": 22, "n_head": 32,
                           "n_head_kv": 4, "head_dim": 64, "parallelism": "none"},
                "roofline": p["roofline"]}
        if cpu:
            line["cpu_baseline"] = p["cpu_baseline"]
        print(json.dumps(line))
        return

    d = run_decode(args.workload, args.steps, args.warmup, cpu, args.split, PLANS[args.plan])
    cfg = {"decode_model": {"n_seq": 1, "n_layers": 22, "context": 2048},
           "decode_long": {"n_seq": 8, "n_layers": 22, "context": 16384},
           "decode_ragged": {"n_seq": 64, "n_layers": 22, "context": "U[256,2048]"},
           "decode_single": {"n_seq": 1, "n_layers": 1, "context": 128}}[args.workload]
    line = {"metric": HEADLINE_METRIC, "value": round(d["value"], 1), "unit": "GB/s",
            "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "ms_per_step": round(d["ms_per_step"], 5), "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
            "config": dict({"workload": args.workload, "n_head": 32, "n_head_kv": 4,
                            "head_dim": 64, "parallelism": "none",
                            "cache_copies": d["cache_copies"],
                            "mall_resident": d["mall_resident"]}, **cfg),
            "roofline": d["roofline"],
            "kernels_us": {"decode": round(d["decode_kernel_ms"] * 1e3, 2),
                           "decode_per_launch_events": round(
                               d["decode_kernel_ms_per_launch_events"] * 1e3, 2)}}
    if cpu:
        line["cpu_baseline"] = d["cpu_baseline"]
    if not args.no_prefill and args.workload == "decode_model":
        p = run_prefill(args.steps, args.warmup, cpu)
        line["prefill"] = {k: p[k] for k in ("value", "unit", "ms_per_step", "warmup", "roofline")}
        line["prefill"]["value"] = round(p["value"], 3)
        line["prefill"]["config"] = {"workload": "prefill", "n_tok": 512, "n_layers": 22}
        if cpu:
            line["prefill"]["cpu_baseline"] = p["cpu_baseline"]
        # what one launch can execute of the same fp32 MFMA work, and the
        # prefill kernel's time over it
        mf = run_mfma_floor(args.steps, args.warmup)
        line["prefill"]["mfma_floor"] = mf
        line["prefill"]["kernel_over_mfma_floor"] = round(
            mf["us"] * (prefill_executed_flops() / mf["flops"]) / (p["prefill_kernel_ms"] * 1e3), 4)
    if not args.no_extra and args.workload == "decode_model":
        # the other decode configurations, measured the same way (no CPU
        # baseline): long context x 8 and the ragged batch as HBM
        # throughput, one layer at position 127 as latency
        line["extra"] = {}
        for wl in ("decode_long", "decode_ragged"):
            e = run_decode(wl, args.steps, args.warmup, False)
            line["extra"][wl] = {"value": round(e["value"], 1), "unit": "GB/s",
                                 "ms_per_step": round(e["ms_per_step"], 4),
                                 "roofline": e["roofline"]}
        e = run_decode("decode_single", args.steps, args.warmup, False)
        line["extra"]["decode_single"] = {"value": round(e["ms_per_step"] * 1e3, 2), "unit": "us",
                                          "higher_is_better": False,
                                          "note": "1 layer, position 127: latency-bound"}
        # what one launch can read of the same byte counts (the decode step's
        # ceiling at batch 1), and the decode kernel's rate over it at 2048
        floor = run_read_floor(args.steps, args.warmup)
        line["extra"]["read_floor"] = floor
        f2k = next(x for x in floor if x["size"] == "ctx 2048")
        line["extra"]["decode_model_over_read_floor"] = round(f2k["us"] / (d["ms_per_step"] * 1e3), 4)
        flong = next(x for x in floor if x["size"] == "decode_long")
        line["extra"]["decode_long_over_read_floor"] = round(
            flong["us"] / (line["extra"]["decode_long"]["ms_per_step"] * 1e3), 4)
    print(json.dumps(line))


HEADLINE_METRIC = "decode-attn KV GB/s (% HBM peak); prefill-attn TFLOP/s (% MFMA peak)"

if __name__ == "__main__":
    main()
