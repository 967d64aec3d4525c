"""GPU parity of causal prefill (RoPE in-kernel, KV append, fp32 MFMA
attention) through the C ABI against the reference's token-by-token prompt
loop (src/generate.cpp:56-59): golden vectors and the oracle.  Bar: max-abs
1e-4 on outputs (fp32 accumulate), KV cache bit-exact."""
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest

from conftest import golden
from helpers import PREFILL_TOL, ORACLE_THREADS, bits, device_arrays, log, max_err

pytestmark = pytest.mark.gpu


def gpu_prefill(eng, case, layer0=0, chunks=None, kc_init=None, vc_init=None, rotate=True):
    """Run `case` (n_layers x n_tok) at positions pos0.. in the given chunks;
    returns (out [n_layers, n_tok, q_dim], key cache, value cache)."""
    nl, nt = case.n_layers, case.n_tok
    q_dim = case.q.shape[-1]
    chunks = chunks or [nt]
    outs = np.zeros((nl, nt, q_dim), np.float32)
    with device_arrays() as track:
        kc, vc = eng.kv_cache(1)
        track(kc), track(vc)
        if kc_init is not None:
            kc.upload(kc_init)
            vc.upload(vc_init)
        t0 = 0
        for c in chunks:
            q = track(eng.array(np.ascontiguousarray(case.q[:, t0:t0 + c])))
            k = track(eng.array(np.ascontiguousarray(case.k[:, t0:t0 + c])))
            v = track(eng.array(np.ascontiguousarray(case.v[:, t0:t0 + c])))
            out = track(eng.array((nl, c, q_dim)))
            log(f"  tla_prefill pos0={case.pos0 + t0} n_tok={c} layers={layer0}..{layer0 + nl - 1}")
            eng.prefill(case.pos0 + t0, c, layer0, nl, out.ptr, q.ptr, k.ptr, v.ptr, kc.ptr, vc.ptr,
                        rotate=rotate)
            outs[:, t0:t0 + c] = out.download()
            t0 += c
        return outs, kc.download(), vc.download()


def oracle_prefill(O, case, n_layers_total, n_ctx, layer0=0, kc=None, vc=None):
    s = O.Shape(n_head=case.n_head, n_head_kv=case.n_head_kv, n_ctx=n_ctx,
                n_layers=n_layers_total)
    if kc is None:
        kc = np.zeros(n_layers_total * n_ctx * s.kv_dim, np.float32)
        vc = np.zeros_like(kc)
    outs = [None] * case.n_layers

    def one(layer):
        outs[layer] = O.prefill(case.q[layer], case.k[layer], case.v[layer], kc, vc,
                                layer0 + layer, case.pos0, s)

    with ThreadPoolExecutor(ORACLE_THREADS) as ex:  # layers touch disjoint cache slices
        list(ex.map(one, range(case.n_layers)))
    return np.stack(outs), kc, vc


def test_prefill_golden_in_two_chunks(W, engines):
    g = golden("prefill.npz")
    case = W.make_prefill(n_layers=1, n_tok=40, salt=7)
    assert W.digest(case.q, case.k, case.v) == str(g["digest"])
    out, kc, vc = gpu_prefill(engines(2, 64), case, layer0=1, chunks=[32, 8])
    err = max_err(out[0], g["out"])
    log(f"    vs reference: max-abs {err:.3e}")
    assert err <= PREFILL_TOL
    assert np.array_equal(bits(kc[0, 1, :40]), bits(g["kc"]))
    assert np.array_equal(bits(vc[0, 1, :40]), bits(g["vc"]))
    assert not kc[0, 0].any() and not kc[0, 1, 40:].any()


def test_prefill_512_tokens_22_layers(O, W, engines):
    """The prefill workload at full size against the oracle loop."""
    case = W.make_prefill(n_layers=22, n_tok=512)
    out, kc, vc = gpu_prefill(engines(22, 512), case)
    ref, rkc, rvc = oracle_prefill(O, case, 22, 512)
    err = max_err(out, ref)
    log(f"    max-abs {err:.3e}")
    assert err <= PREFILL_TOL
    assert np.array_equal(bits(kc.reshape(-1)), bits(rkc))
    assert np.array_equal(bits(vc.reshape(-1)), bits(rvc))


def test_prefill_2048_tokens(O, W, engines):
    """A long prompt (2048 tokens, one of the measured prefill sizes) over 8
    layers against the oracle loop: every query row sees up to 2048 keys."""
    case = W.make_prefill(n_layers=8, n_tok=2048, salt=11)
    out, kc, vc = gpu_prefill(engines(8, 2048), case)
    ref, rkc, rvc = oracle_prefill(O, case, 8, 2048)
    err = max_err(out, ref)
    log(f"    max-abs {err:.3e}")
    assert err <= PREFILL_TOL
    assert np.array_equal(bits(kc.reshape(-1)), bits(rkc))
    assert np.array_equal(bits(vc.reshape(-1)), bits(rvc))


@pytest.mark.parametrize("pos0,n_tok", [(0, 1), (0, 31), (0, 33), (7, 100), (64, 64), (100, 5),
                                        (130, 126)])
def test_prefill_odd_sizes_and_offsets(O, W, engines, pos0, n_tok):
    """Prompts continuing an existing cache (pos0 > 0) and ragged tile edges."""
    n_ctx = 256
    hist = W.make_prefill(n_layers=2, n_tok=max(pos0, 1), salt=11)
    case = W.make_prefill(n_layers=2, n_tok=n_tok, pos0=pos0, salt=12)
    s = O.Shape(n_ctx=n_ctx, n_layers=2)
    kc = np.zeros(2 * n_ctx * 256, np.float32)
    vc = np.zeros_like(kc)
    if pos0:
        for layer in range(2):
            O.prefill(hist.q[layer, :pos0], hist.k[layer, :pos0], hist.v[layer, :pos0], kc, vc,
                      layer, 0, s)
    kc0, vc0 = kc.copy(), vc.copy()
    ref, rkc, rvc = oracle_prefill(O, case, 2, n_ctx, kc=kc, vc=vc)
    out, gkc, gvc = gpu_prefill(engines(2, n_ctx), case, kc_init=kc0.reshape(1, 2, n_ctx, 256),
                                vc_init=vc0.reshape(1, 2, n_ctx, 256))
    err = max_err(out, ref)
    log(f"    max-abs {err:.3e}")
    assert err <= PREFILL_TOL
    assert np.array_equal(bits(gkc.reshape(-1)), bits(rkc))
    assert np.array_equal(bits(gvc.reshape(-1)), bits(rvc))


def test_prefill_then_decode(O, W, engines, tla):
    """A 300-token prompt by prefill, then token 300 by decode, equals the
    oracle's 301 token-by-token steps."""
    eng = engines(1, 512)
    case = W.make_prefill(n_layers=1, n_tok=301, salt=13)
    s = O.Shape(n_ctx=512, n_layers=1)
    kc_ref = np.zeros(512 * 256, np.float32)
    vc_ref = np.zeros_like(kc_ref)
    ref = O.prefill(case.q[0], case.k[0], case.v[0], kc_ref, vc_ref, 0, 0, s)
    with device_arrays() as track:
        kc, vc = eng.kv_cache(1)
        track(kc), track(vc)
        q = track(eng.array(np.ascontiguousarray(case.q[:, :300])))
        k = track(eng.array(np.ascontiguousarray(case.k[:, :300])))
        v = track(eng.array(np.ascontiguousarray(case.v[:, :300])))
        out = track(eng.array((1, 300, 2048)))
        eng.prefill(0, 300, 0, 1, out.ptr, q.ptr, k.ptr, v.ptr, kc.ptr, vc.ptr)
        assert max_err(out.download()[0], ref[:300]) <= PREFILL_TOL
        q1, k1, v1 = track(eng.array(case.q[0, 300])), track(eng.array(case.k[0, 300])), \
            track(eng.array(case.v[0, 300]))
        o1 = track(eng.array((2048,)))
        eng.rope_attention(o1.ptr, q1.ptr, k1.ptr, v1.ptr, kc.ptr, vc.ptr, 0, 300)
        assert max_err(o1.download(), ref[300]) <= PREFILL_TOL
        assert np.array_equal(bits(kc.download().reshape(-1)), bits(kc_ref))


def test_prefill_without_rotation(O, W, engines):
    """Without TLA_ROTATE, q and k are taken as already rotated."""
    case = W.make_prefill(n_layers=1, n_tok=70, salt=14)
    s = O.Shape(n_ctx=128, n_layers=1)
    qr = np.empty_like(case.q)
    kr = np.empty_like(case.k)
    for t in range(70):
        qr[0, t], kr[0, t] = O.rope(case.q[0, t], case.k[0, t], t, s)
    ref, _, _ = oracle_prefill(O, case, 1, 128)
    pre = W.PrefillCase(1, 70, 0, qr, kr, case.v)
    out, _, _ = gpu_prefill(engines(1, 128), pre, rotate=False)
    assert max_err(out, ref) <= PREFILL_TOL


def test_prefill_range_errors(tla, W, engines):
    eng = engines(2, 64)
    with device_arrays() as track:
        kc, vc = eng.kv_cache(1)
        track(kc), track(vc)
        buf = track(eng.array((64 * 2048,)))
        for pos0, n, l0, nl, code in ((60, 5, 0, 1, tla.TLA_ERR_OUT_OF_RANGE),
                                      (-1, 5, 0, 1, tla.TLA_ERR_OUT_OF_RANGE),
                                      (0, 0, 0, 1, tla.TLA_ERR_INVALID_ARGUMENT),
                                      (0, 5, 1, 2, tla.TLA_ERR_OUT_OF_RANGE)):
            with pytest.raises(tla.TlaError) as ei:
                eng.prefill(pos0, n, l0, nl, buf.ptr, buf.ptr, buf.ptr, buf.ptr, kc.ptr, vc.ptr)
            assert ei.value.code == code


@pytest.mark.parametrize("n_head,n_head_kv", [(32, 8), (32, 2), (16, 1), (24, 6), (64, 4), (12, 12)])
def test_prefill_other_head_shapes(O, W, engines, n_head, n_head_kv):
    """GQA ratios 1..16 and kv head counts that leave workgroup waves idle."""
    n_ctx = 256
    case = W.make_prefill(n_layers=2, n_tok=77, pos0=0, salt=n_head * 100 + n_head_kv,
                          n_head=n_head, n_head_kv=n_head_kv)
    eng = engines(2, n_ctx, n_head, n_head_kv)
    got, gkc, gvc = gpu_prefill(eng, case)
    ref, rkc, rvc = oracle_prefill(O, case, 2, n_ctx)
    err = max_err(got, ref)
    log(f"    heads {n_head}/{n_head_kv}: max-abs error {err:.3e}")
    assert err <= PREFILL_TOL
    assert np.array_equal(bits(gkc.reshape(-1)), bits(rkc.reshape(-1)))
    assert np.array_equal(bits(gvc.reshape(-1)), bits(rvc.reshape(-1)))
