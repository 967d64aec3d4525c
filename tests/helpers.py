"""Shared drivers for the GPU parity tests: run a workload through the C ABI
and through the oracle on the same inputs."""
import contextlib
import importlib
import os
import sys

import numpy as np

tla = importlib.import_module("tinyllama-engine_amd")

ORACLE_THREADS = min(16, os.cpu_count() or 4)

# Tolerances.  Decode: the path's stated bound, max-abs 1e-4 against the
# reference's fp32 attention.  Prefill: fp32 MFMA products with fp32
# accumulation in a different order than the reference's sequential loops;
# measured error is ~1e-6 on N(0,1) inputs, bound stated at 1e-4.
DECODE_TOL = 1e-4
PREFILL_TOL = 1e-4


def log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@contextlib.contextmanager
def device_arrays():
    made = []

    def track(a):
        made.append(a)
        return a

    try:
        yield track
    finally:
        for a in made:
            a.free()


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def max_err(a, b):
    return float(np.abs(np.asarray(a, np.float64) - np.asarray(b, np.float64)).max())


def gpu_decode(eng, case, rotate=True, split=0, keep_cache=False, plan=0):
    """tla_decode over every (sequence, layer) of `case` in one call, with
    the given positions per workgroup and work plan (0 = the engine's choice).
    Returns (out [n_seq, n_layers, q_dim], key rows at pos, value rows at pos,
    [full caches if keep_cache])."""
    cfg = eng.cfg
    assert cfg.n_layers == case.n_layers and cfg.n_ctx == case.n_ctx
    eng.set_option(tla.OPT_DECODE_SPLIT, split)
    eng.set_option(tla.OPT_DECODE_PLAN, plan)
    with device_arrays() as track:
        kc, vc = eng.kv_cache(case.n_seq)
        track(kc), track(vc)
        kc.upload(case.kc)
        vc.upload(case.vc)
        q, k, v = track(eng.array(case.q)), track(eng.array(case.k)), track(eng.array(case.v))
        out = track(eng.array(case.q.shape))
        stride = case.n_layers * case.n_ctx * cfg.kv_dim
        log(f"  tla_decode n_seq={case.n_seq} layers={case.n_layers} ctx={case.n_ctx} "
            f"pos[0]={int(case.pos[0])} rotate={rotate} split={split} plan={plan}")
        eng.decode(case.pos, 0, case.n_layers, out.ptr, q.ptr, k.ptr, v.ptr, kc.ptr, vc.ptr,
                   stride, rotate)
        res = out.download()
        if keep_cache:
            return res, kc.download(), vc.download()
        krow = np.empty((case.n_seq, case.n_layers, cfg.kv_dim), np.float32)
        vrow = np.empty_like(krow)
        row_bytes = cfg.kv_dim * 4
        for s in range(case.n_seq):
            for layer in range(case.n_layers):
                off = ((s * case.n_layers + layer) * case.n_ctx + int(case.pos[s])) * row_bytes
                for dst, arr in ((krow, kc), (vrow, vc)):
                    host = np.empty(cfg.kv_dim, np.float32)
                    rc = tla.lib().tla_memcpy_d2h(eng.h, host.ctypes.data, arr.ptr + off, row_bytes)
                    assert rc == 0, tla.last_error()
                    dst[s, layer] = host
        return res, krow, vrow


def oracle_decode(O, case, rotate=True, keep_cache=False):
    """Oracle for every (sequence, layer) unit.  Returns (out, key rows, value
    rows[, full caches])."""
    units = case.n_seq * case.n_layers
    kv_dim = case.kc.shape[-1]
    kc = case.kc.reshape(units, case.n_ctx, kv_dim).copy()
    vc = case.vc.reshape(units, case.n_ctx, kv_dim).copy()
    pos = np.repeat(case.pos, case.n_layers).astype(np.int32)
    shape = O.Shape(n_head=case.n_head, n_head_kv=case.n_head_kv, n_ctx=case.n_ctx)
    out = O.decode_units_mt(ORACLE_THREADS, case.q.reshape(units, -1), case.k.reshape(units, -1),
                            case.v.reshape(units, -1), kc, vc, pos, shape, rotate=rotate)
    out = out.reshape(case.n_seq, case.n_layers, -1)
    if keep_cache:
        return out, kc.reshape(case.kc.shape), vc.reshape(case.vc.shape)
    idx = np.arange(units)
    krow = kc[idx, pos].reshape(case.n_seq, case.n_layers, kv_dim)
    vrow = vc[idx, pos].reshape(case.n_seq, case.n_layers, kv_dim)
    return out, krow, vrow


def check_decode(O, eng, case, rotate=True, split=0, tol=DECODE_TOL, plan=0):
    got, gk, gv = gpu_decode(eng, case, rotate=rotate, split=split, plan=plan)
    ref, rk, rv = oracle_decode(O, case, rotate=rotate)
    err = max_err(got, ref)
    log(f"    max-abs error {err:.3e}")
    assert err <= tol, f"decode max-abs error {err} > {tol}"
    assert np.array_equal(bits(gk), bits(rk)), "appended key rows differ"
    assert np.array_equal(bits(gv), bits(rv)), "appended value rows differ"
    return err
