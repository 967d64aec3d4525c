"""The allocation-free decode entry point, tla_decode_noalloc, through the C
ABI: the same launch as tla_decode on the same inputs, its split partials and
counters in the device's static scratch instead of the engine's workspace.
Outputs and appended cache rows must equal tla_decode's bit for bit (same
kernels, same plan, same summation order) and lie within the decode bound of
the oracle, on two calls in a row, the second with a smaller input; a launch
needing more scratch than the array holds is refused before any launch."""
import ctypes as C

import numpy as np
import pytest

from helpers import DECODE_TOL, bits, device_arrays, log, max_err, oracle_decode

pytestmark = pytest.mark.gpu


def device_free_bytes():
    """Free device memory as the HIP runtime reports it (hipMemGetInfo)."""
    for name in ("libamdhip64.so", "libamdhip64.so.7", "/opt/rocm/lib/libamdhip64.so"):
        try:
            hip = C.CDLL(name)
            break
        except OSError:
            continue
    else:
        pytest.fail("the HIP runtime library is not loadable")
    free, total = C.c_size_t(), C.c_size_t()
    assert hip.hipMemGetInfo(C.byref(free), C.byref(total)) == 0
    return free.value


def run_entry(tla, eng, case, entry, check_free=False):
    """One call of `entry` (tla_decode or tla_decode_noalloc) over every
    (sequence, layer) of `case`, on fresh copies of its caches; returns the
    output and both whole caches.  With check_free, the device's free memory
    must be the same before and after the call (inputs allocated before)."""
    cfg = eng.cfg
    with device_arrays() as track:
        kc, vc = eng.kv_cache(case.n_seq)
        track(kc), track(vc)
        kc.upload(case.kc)
        vc.upload(case.vc)
        q, k, v = track(eng.array(case.q)), track(eng.array(case.k)), track(eng.array(case.v))
        out = track(eng.array(case.q.shape))
        pos = np.ascontiguousarray(case.pos, np.int32)
        stride = cfg.n_layers * cfg.n_ctx * cfg.kv_dim
        log(f"  {entry}: n_seq={case.n_seq} layers={case.n_layers} pos={pos.tolist()[:4]}")
        eng.synchronize()
        before = device_free_bytes()
        rc = getattr(tla.lib(), entry)(eng.h, int(pos.size), pos.ctypes.data_as(C.POINTER(C.c_int)),
                                       0, case.n_layers, tla.TLA_ROTATE, out.ptr, q.ptr, k.ptr, v.ptr,
                                       kc.ptr, vc.ptr, stride)
        assert rc == tla.TLA_OK, tla.last_error()
        eng.synchronize()
        after = device_free_bytes()
        log(f"    device free memory {before} -> {after} bytes")
        if check_free:
            assert after == before, f"{entry} changed free device memory by {before - after} bytes"
        return out.download(), kc.download(), vc.download()


def test_noalloc_equals_decode_on_two_calls(tla, O, W):
    """On an engine of its own that has never decoded (no workspace yet),
    tla_decode_noalloc runs first with the device's free memory unchanged,
    then tla_decode (which allocates its workspace: the free memory drops)
    on the same inputs.  Run alone in a fresh process, this is also the
    process's first decode launch: the decode kernels' code object must
    already be loaded (at engine creation), since its load allocates."""
    eng = tla.Engine(tla.Config.tinyllama(n_layers=22, n_ctx=2048))
    cases = [
        # 22 layers x 2048 positions, one sequence: 11 splits per unit merged
        W.decode_model(n_layers=22, n_ctx=2048),
        # smaller: two ragged sequences, fewer splits, fewer units
        W.make_decode(41, 2, 22, 2048, [700, 64], salt=3),
    ]
    try:
        results = []
        for case in cases:
            got, gk, gv = run_entry(tla, eng, case, "tla_decode_noalloc", check_free=True)
            want, wk, wv = run_entry(tla, eng, case, "tla_decode")
            results.append((case, got, gk, gv, want, wk, wv))
    finally:
        eng.close()
    for case, got, gk, gv, want, wk, wv in results:
        assert np.array_equal(bits(got), bits(want)), "outputs differ from tla_decode"
        assert np.array_equal(bits(gk), bits(wk)) and np.array_equal(bits(gv), bits(wv)), "caches differ"
        ref, _, _ = oracle_decode(O, case)
        err = max_err(got, ref)
        log(f"    bit-identical to tla_decode; max-abs vs oracle {err:.3e}")
        assert err <= DECODE_TOL


def test_noalloc_refuses_launches_beyond_the_scratch(tla, engines):
    """64 sequences at position 2047 in splits of 16 positions need about
    69 MB of partials: refused with TLA_ERR_UNSUPPORTED, nothing launched
    (the output keeps its contents), while tla_decode would grow its
    workspace."""
    eng = engines(1, 2048)
    n_seq = 64
    eng.set_option(tla.OPT_DECODE_SPLIT, 16)
    eng.set_option(tla.OPT_DECODE_PLAN, tla.PLAN_ALIGNED)
    try:
        with device_arrays() as track:
            kc, vc = eng.kv_cache(n_seq)
            track(kc), track(vc)
            q = track(eng.array(np.zeros((n_seq, 2048), np.float32)))
            kv = track(eng.array(np.zeros((n_seq, 256), np.float32)))
            out = track(eng.array(np.full((n_seq, 2048), 7.0, np.float32)))
            pos = np.full(n_seq, 2047, np.int32)
            rc = tla.lib().tla_decode_noalloc(eng.h, n_seq, pos.ctypes.data_as(C.POINTER(C.c_int)), 0, 1,
                                              tla.TLA_ROTATE, out.ptr, q.ptr, kv.ptr, kv.ptr, kc.ptr, vc.ptr,
                                              2048 * 256)
            assert rc == tla.TLA_ERR_UNSUPPORTED, tla.last_error()
            assert "static" in tla.last_error()
            eng.synchronize()
            assert np.all(out.download() == 7.0)
    finally:
        eng.set_option(tla.OPT_DECODE_SPLIT, 0)
        eng.set_option(tla.OPT_DECODE_PLAN, 0)
