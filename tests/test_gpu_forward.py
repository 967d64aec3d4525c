"""GPU parity of the whole forward pass through the C ABI: embed_token
(src/forward.cpp:17-134), silu / elementwise_mul / ffn_swiglu
(src/ops.cpp:1107-1148, 1535-1564), the FFN half of a layer
(src/forward.cpp:215-228), sample_argmax (src/ops.cpp:1587-1597), forward()
(src/forward.cpp:167-266) and the greedy generation loop
(src/generate.cpp:56-100).

Tolerances: embed, elementwise_mul, argmax bit-exact; silu within 2 ulp
(the device expf against glibc's); GEMV-based results per output row within
2e-5 * sum_j |w_ij x_j| of the oracle; forward() logits within 1e-4 of
the largest |logit| of the step against the reference's own logits (golden)
and the oracle's, and the same argmax wherever the top two logits are
further apart than twice that bound; greedy generation token for token."""
import ast

import numpy as np
import pytest

import quant_ref as Q
from conftest import golden
from forward_ref import model_from_golden
from helpers import bits, device_arrays, log

pytestmark = pytest.mark.gpu

CASES = ["q8_0", "f16_tied", "q4_0", "f32", "mixed"]
TYPES = [(Q.F32, "f32"), (Q.F16, "f16"), (Q.Q4_0, "q4_0"), (Q.Q8_0, "q8_0"), (Q.Q6_K, "q6_k")]
ORACLE_TOL = 2e-5
LOGIT_TOL = 1e-4


def spec_engine(engines, spec):
    assert spec.head_dim == 64
    return engines(spec.n_layers, spec.n_ctx, spec.n_head, spec.n_head_kv)


@pytest.mark.parametrize("t,name", TYPES)
def test_embed_bit_exact(tla, O, W, engines, t, name):
    eng = engines(1, 64)
    n_vocab, n_embd = 40, 2048
    raw = W.make_weights(t, n_vocab, n_embd, salt=9)
    with device_arrays() as track:
        tab = track(eng.array(raw))
        out = track(eng.array((n_embd,)))
        for tok in (0, 1, 23, 39):
            eng.embed(out.ptr, tab.ptr, tok, n_embd, n_vocab, t)
            assert np.array_equal(bits(out.download()), bits(O.embed(raw, tok, n_embd, t))), (name, tok)
        for tok in (-1, n_vocab):  # past either end of the table: an error, nothing launched
            with pytest.raises(tla.TlaError) as e:
                eng.embed(out.ptr, tab.ptr, tok, n_embd, n_vocab, t)
            assert e.value.code == tla.TLA_ERR_OUT_OF_RANGE


def test_silu_and_elementwise_mul(O, engines):
    eng = engines(1, 64)
    g = golden("forward.npz")
    x = g["silu_x"]
    rg = np.random.default_rng(4)
    b = rg.standard_normal(x.size).astype(np.float32)
    with device_arrays() as track:
        d = track(eng.array(x))
        eng.silu(d.ptr, x.size)
        got = d.download()
        want = g["silu_out"]  # the reference's silu()
        ulp = np.spacing(np.abs(want).astype(np.float32))
        err = np.abs(got.astype(np.float64) - want)
        log(f"  silu: max error {float((err / np.maximum(ulp, 1e-45)).max()):.1f} ulp")
        assert np.all(err <= 2 * ulp + 1e-38)
        bd = track(eng.array(b))
        eng.elementwise_mul(d.ptr, bd.ptr, x.size)
        assert np.array_equal(bits(d.download()), bits(got * b))


def row_scale(raw, x, t, rows, cols):
    return Q.matmul_f64(raw, x, t, rows, cols)[1] + 1e-30


@pytest.mark.parametrize("t", [Q.Q8_0, Q.F16, Q.Q4_0, Q.Q6_K])
def test_ffn_swiglu(O, W, engines, t):
    eng = engines(1, 64, 4, 2)  # n_embd 256
    n_ff, n_embd = 512, 256
    wg, wu = W.make_weights(t, n_ff, n_embd, salt=31), W.make_weights(t, n_ff, n_embd, salt=32)
    wd = W.make_weights(t, n_embd, n_ff, salt=33)
    xin = np.random.default_rng(t).standard_normal(n_embd).astype(np.float32)
    out_o, hb_o, hb2_o = O.ffn_swiglu(xin, wg, wu, wd, n_ff, n_embd, t)
    with device_arrays() as track:
        dg, du, dd = (track(eng.array(w)) for w in (wg, wu, wd))
        dx = track(eng.array(xin))
        out, hb, hb2 = track(eng.array((n_embd,))), track(eng.array((n_ff,))), track(eng.array((n_ff,)))
        eng.ffn_swiglu(out.ptr, dx.ptr, hb.ptr, hb2.ptr, dg.ptr, du.ptr, dd.ptr, n_ff, n_embd, t)
        got_out, got_hb, got_hb2 = out.download(), hb.download(), hb2.download()
    s_up = row_scale(wu, xin, t, n_ff, n_embd)
    s_gate = row_scale(wg, xin, t, n_ff, n_embd)
    assert np.max(np.abs(got_hb2 - hb2_o) / s_up) <= ORACLE_TOL
    # gated: silu(gate) * up, errors of both factors carried through
    bound = ORACLE_TOL * (s_gate * np.abs(hb2_o) + s_up * np.abs(hb_o / np.where(hb2_o == 0, 1, hb2_o)))
    assert np.all(np.abs(got_hb - hb_o) <= bound + 1e-6 * np.abs(hb_o) + 1e-30)
    s_down = row_scale(wd, hb_o, t, n_embd, n_ff)
    assert np.max(np.abs(got_out - out_o) / s_down) <= 2 * ORACLE_TOL


@pytest.mark.parametrize("n_seq", [1, 3, 9])
def test_ffn_block(O, W, engines, n_seq):
    """x += ffn_swiglu(rmsnorm(x)) for n_seq vectors (n_ff 5632 columns for
    the down projection: 64 lanes per row)."""
    eng = engines(1, 64, 4, 2)
    t, n_ff, n_embd = Q.Q8_0, 5632, 256
    wg, wu = W.make_weights(t, n_ff, n_embd, salt=51), W.make_weights(t, n_ff, n_embd, salt=52)
    wd = W.make_weights(t, n_embd, n_ff, salt=53)
    rg = np.random.default_rng(n_seq)
    x = rg.standard_normal((n_seq, n_embd)).astype(np.float32)
    nw = rg.uniform(0.5, 1.5, n_embd).astype(np.float32)
    with device_arrays() as track:
        dg, du, dd = (track(eng.array(w)) for w in (wg, wu, wd))
        dx, dn = track(eng.array(x)), track(eng.array(nw))
        hb = track(eng.array((n_seq, 2, n_ff)))
        eng.ffn_block(n_seq, dx.ptr, dn.ptr, 1e-5, dg.ptr, du.ptr, dd.ptr, n_ff, t, hb.ptr)
        got = dx.download()
    for s in range(n_seq):
        xn = O.rmsnorm(x[s], nw, 1e-5)
        out, hbo, _ = O.ffn_swiglu(xn, wg, wu, wd, n_ff, n_embd, t)
        want = x[s] + out
        scale = row_scale(wd, hbo, t, n_embd, n_ff) + np.abs(x[s])
        err = float(np.max(np.abs(got[s] - want) / scale))
        log(f"  ffn_block seq {s}: {err:.2e}")
        assert err <= 4 * ORACLE_TOL


@pytest.mark.parametrize("t", [Q.Q8_0, Q.Q4_0, Q.Q6_K, Q.F16])
@pytest.mark.parametrize("n_head", [4, 48])
def test_ffn_block_one_sequence_formats(O, W, engines, t, n_head):
    """One sequence: block formats form SiLU(gate) x up in the gate/up
    launch's epilogue (gate and up rows paired in one lane group), with rows
    of 32 lanes (n_embd 256) and of 64 lanes (n_embd 3072); F16 keeps SwiGLU
    in the down projection's prologue."""
    eng = engines(1, 64, n_head, 2 if n_head == 4 else 4)
    n_ff, n_embd = 1024, 64 * n_head
    wg, wu = W.make_weights(t, n_ff, n_embd, salt=61), W.make_weights(t, n_ff, n_embd, salt=62)
    wd = W.make_weights(t, n_embd, n_ff, salt=63)
    rg = np.random.default_rng(n_head + t)
    x = rg.standard_normal((1, n_embd)).astype(np.float32)
    nw = rg.uniform(0.5, 1.5, n_embd).astype(np.float32)
    with device_arrays() as track:
        dg, du, dd = (track(eng.array(w)) for w in (wg, wu, wd))
        dx, dn = track(eng.array(x)), track(eng.array(nw))
        hb = track(eng.array((1, 2, n_ff)))
        eng.ffn_block(1, dx.ptr, dn.ptr, 1e-5, dg.ptr, du.ptr, dd.ptr, n_ff, t, hb.ptr)
        got = dx.download()
    xn = O.rmsnorm(x[0], nw, 1e-5)
    out, hbo, _ = O.ffn_swiglu(xn, wg, wu, wd, n_ff, n_embd, t)
    scale = row_scale(wd, hbo, t, n_embd, n_ff) + np.abs(x[0])
    err = float(np.max(np.abs(got[0] - (x[0] + out)) / scale))
    log(f"  ffn_block type {t} n_embd {n_embd}: {err:.2e}")
    assert err <= 4 * ORACLE_TOL


def test_argmax(O, engines):
    eng = engines(1, 64)
    rg = np.random.default_rng(8)
    cases = []
    x = rg.standard_normal(32000).astype(np.float32)
    cases.append(x)
    y = x.copy()
    y[[5, 900, 31999]] = y.max() + 1  # ties: the first wins
    cases.append(y)
    z = x.copy()
    z[[3, 77]] = np.nan  # NaN never wins
    cases.append(z)
    n0 = x.copy()
    n0[0] = np.nan  # the reference's scan never leaves index 0
    cases.append(n0)
    cases.append(np.full(100, -np.inf, np.float32))
    cases.append(np.array([2.5], np.float32))
    cases.append(np.concatenate([np.zeros(1025, np.float32), [1.0]]).astype(np.float32))
    # past one batch of loads per thread (32768 entries): the maximum in the
    # last batch, then at the first entry of the second
    big = rg.standard_normal(70001).astype(np.float32)
    big[70000] = 9.0
    cases.append(big)
    edge = rg.standard_normal(32769).astype(np.float32)
    edge[32768] = 9.0
    cases.append(edge)
    lib = O.oracle()
    from oracle import fptr
    for c in cases:
        with device_arrays() as track:
            d = track(eng.array(c))
            got = eng.argmax(d.ptr, c.size)
        want = lib.oracle_argmax(fptr(np.ascontiguousarray(c)), c.size)
        assert got == want, (got, want)


def test_matmul_argmax(tla, O, W, engines):
    """matmul then sample_argmax with the argmax keys that the product's
    workgroups post (the path tla_generate_greedy takes for every token
    after its first): against the oracle's argmax of the same launch's
    logits, over ties (identical rows: the first wins), NaN rows (never
    win), a NaN at row 0 (index 0), +0 ties with everything else negative,
    and random Q8_0 / Q6_K / F16 / Q4_0 products with 512 workgroups (8 per
    key slot)."""
    eng = engines(1, 64)
    lib = O.oracle()
    from oracle import fptr
    rg = np.random.default_rng(12)
    rows, cols = 32000, 256
    x = np.abs(rg.standard_normal(cols)).astype(np.float32) + 0.1  # positive
    base = rg.standard_normal((rows, cols)).astype(np.float32)
    cases = []
    w = base.copy()
    w[[5, 900, 31999]] = 1.0  # the largest logit, three times, bit-equal
    cases.append(("ties", w, 5))
    w = base.copy()
    w[[3, 77]] = np.nan
    cases.append(("nan rows", w, None))
    w = base.copy()
    w[0, 17] = np.nan
    cases.append(("nan at 0", w, 0))
    w = -np.abs(base) - 0.01  # every logit negative ...
    w[[7, 10]] = 0.0          # ... but two exact zeros
    cases.append(("zero ties", w, 7))
    cases.append(("random f32", base, None))
    with device_arrays() as track:
        dx = track(eng.array(x))
        out = track(eng.array((rows,)))
        for name, wf, want_idx in cases:
            dw = track(eng.array(np.ascontiguousarray(wf, np.float32)))
            got = eng.matmul_argmax(out.ptr, dw.ptr, dx.ptr, rows, cols, Q.F32)
            lg = out.download()
            want = lib.oracle_argmax(fptr(lg), rows)
            assert got == want, (name, got, want)
            if want_idx is not None:
                assert got == want_idx, (name, got, want_idx)
        for t in (Q.Q8_0, Q.Q6_K, Q.F16, Q.Q4_0):
            raw = W.make_weights(t, rows, cols, salt=40 + t)
            dw = track(eng.array(raw))
            got = eng.matmul_argmax(out.ptr, dw.ptr, dx.ptr, rows, cols, t)
            lg = out.download()
            assert got == lib.oracle_argmax(fptr(lg), rows), t
        # rows past 64 units (4096 columns) take no argmax keys: refused
        wide = track(eng.array(np.zeros((8, 4160), np.float32)))
        xw = track(eng.array(np.zeros(4160, np.float32)))
        with pytest.raises(tla.TlaError) as e:
            eng.matmul_argmax(out.ptr, wide.ptr, xw.ptr, 8, 4160, Q.F32)
        assert e.value.code == tla.TLA_ERR_UNSUPPORTED


def run_forward(tla, eng, spec, t, tokens):
    dm = tla.DeviceModel(eng, t, spec.n_ff, spec.n_vocab, spec.rms_norm_eps)
    try:
        with device_arrays() as track:
            kc, vc = eng.kv_cache(1)
            track(kc), track(vc)
            lg = track(eng.array((spec.n_vocab,)))
            out = []
            for i, tok in enumerate(tokens):
                eng.forward(dm, kc.ptr, vc.ptr, int(tok), i, lg.ptr)
                out.append(lg.download())
        return np.stack(out)
    finally:
        dm.free()


def check_logits(got, want, what):
    for i in range(got.shape[0]):
        scale = float(np.abs(want[i]).max())
        err = float(np.abs(got[i] - want[i]).max())
        assert err <= LOGIT_TOL * scale, (what, i, err, scale)
        top2 = np.sort(want[i])[-2:]
        if top2[1] - top2[0] > 2 * LOGIT_TOL * scale:
            assert int(np.argmax(got[i])) == int(np.argmax(want[i])), (what, i)
    log(f"  {what}: max |gpu - ref| / max|logit| = "
        f"{float((np.abs(got - want).max(axis=1) / np.abs(want).max(axis=1)).max()):.2e}")


@pytest.mark.parametrize("name", CASES)
def test_forward_matches_reference_logits(tla, O, W, engines, name):
    g = golden("forward.npz")
    spec, t = model_from_golden(W, g, name)
    eng = spec_engine(engines, spec)
    log(f"  tla_forward {name}: {spec.n_layers} layers, n_embd {spec.n_embd}, "
        f"{len(g['tokens'])} tokens")
    got = run_forward(tla, eng, spec, t, g["tokens"])
    check_logits(got, g[f"{name}_logits"], f"{name} vs reference")


@pytest.mark.parametrize("name", CASES)
def test_generate_greedy_matches_reference(tla, O, W, engines, name):
    g = golden("forward.npz")
    spec, t = model_from_golden(W, g, name)
    eng = spec_engine(engines, spec)
    # the path must not pass near-ties, or token equality would test noise
    om = O.Model(spec, t)
    prompt, n = g["prompt"].tolist(), len(g[f"{name}_greedy"])
    seq = prompt + g[f"{name}_greedy"].tolist()
    for i in range(len(prompt) - 1 + n - 1):
        lg = om.forward(seq[i], i)
        if i >= len(prompt) - 1:
            top2 = np.sort(lg)[-2:]
            assert top2[1] - top2[0] > 2 * LOGIT_TOL * np.abs(lg).max(), "near-tie on the path"
    dm = tla.DeviceModel(eng, t, spec.n_ff, spec.n_vocab, spec.rms_norm_eps)
    try:
        with device_arrays() as track:
            kc, vc = eng.kv_cache(1)
            track(kc), track(vc)
            got = eng.generate_greedy(dm, kc.ptr, vc.ptr, prompt, n)
    finally:
        dm.free()
    log(f"  greedy {name}: {got}")
    assert got == g[f"{name}_greedy"].tolist()


@pytest.mark.parametrize("name", ["q8_0", "f32"])
def test_generate_greedy_short_runs(tla, O, W, engines, name):
    """1, 2 and 3 generated tokens are the first tokens of the golden run:
    the first comes from the argmax launch alone, the second from the keys
    the classifier posts read by the one-wave launch at the end, the third
    also through the embedding launch's read of the keys."""
    g = golden("forward.npz")
    spec, t = model_from_golden(W, g, name)
    eng = spec_engine(engines, spec)
    prompt, want = g["prompt"].tolist(), g[f"{name}_greedy"].tolist()
    assert len(want) >= 3
    dm = tla.DeviceModel(eng, t, spec.n_ff, spec.n_vocab, spec.rms_norm_eps)
    try:
        with device_arrays() as track:
            kc, vc = eng.kv_cache(1)
            track(kc), track(vc)
            for n in (1, 2, 3):
                for batch in (False, True):
                    got = eng.generate_greedy(dm, kc.ptr, vc.ptr, prompt, n, batch_prompt=batch)
                    assert got == want[:n], (n, batch, got)
    finally:
        dm.free()


def test_forward_tinyllama_shape(tla, O, W, engines):
    """TinyLlama's shapes (22 layers, n_embd 2048, 32/4 heads, n_ff 5632,
    vocabulary 32000), Q8_0 weights with a Q6_K classifier, against the
    oracle for 3 tokens."""
    spec = W.ModelSpec(22, 2048, 32, 4, 5632, 32000, 64)
    t = W.make_model(spec, W.W_Q8_0, salt=77, output_type=W.W_Q6_K)
    toks = [1, 15043, 29871]
    om = O.Model(spec, t)
    want = np.stack([om.forward(tk, i) for i, tk in enumerate(toks)])
    eng = spec_engine(engines, spec)
    got = run_forward(tla, eng, spec, t, toks)
    check_logits(got, want, "tinyllama-shaped q8_0 vs oracle")


def test_forward_wide_embedding(tla, O, W, engines):
    """n_embd 3072 (48 q heads on 4 kv heads, rows of 48 units): the Q/K/V
    launch cannot rotate in its epilogue (rows of more than 32 units), so
    RoPE and the append run in the attention launch; the gate/up launch
    pairs rows with 64 lanes each.  Q4_0 weights, 2 layers, 3 tokens
    against the oracle."""
    spec = W.ModelSpec(2, 3072, 48, 4, 1024, 512, 64)
    t = W.make_model(spec, W.W_Q4_0, salt=81)
    toks = [1, 300, 77]
    om = O.Model(spec, t)
    want = np.stack([om.forward(tk, i) for i, tk in enumerate(toks)])
    eng = spec_engine(engines, spec)
    got = run_forward(tla, eng, spec, t, toks)
    check_logits(got, want, "n_embd 3072 q4_0 vs oracle")


@pytest.mark.parametrize("n_embd,n_head,n_head_kv,wtype,wo_type", [
    (256, 4, 4, "W_Q8_0", "W_F32"),   # gqa 1
    (512, 8, 2, "W_Q4_0", "W_Q6_K"),  # gqa 4: W_o column groups of one Q6_K super-block
    (1024, 16, 2, "W_F16", "W_Q4_0"),  # gqa 8
    (512, 8, 1, "W_Q8_0", "W_F16"),   # gqa 8, one kv head
    (512, 8, 8, "W_Q4_0", "W_Q8_0"),  # 8 kv heads: no fused launch at any position
    (768, 12, 4, "W_Q4_0", "W_Q8_0"),  # gqa 3: column groups of 192 (6 blocks, 108 / 204 B)
    (384, 6, 3, "W_F16", "W_F16"),     # 3 kv heads: three partials
])
def test_forward_short_context_fusion(tla, O, W, engines, n_embd, n_head, n_head_kv, wtype, wo_type):
    """A decode step over at most 192 positions runs attention and W_o as
    one launch (each workgroup recomputes one kv head's attention, waves
    taking 1-3 tiles of 16 positions; the W_o partials per kv head reach x
    through the FFN launches); from position 192 on, the attention launch
    and the W_o GEMV.  200 tokens one at a time against the oracle, every
    step's logits (the last 8 past the switch)."""
    spec = W.ModelSpec(2, n_embd, n_head, n_head_kv, 512, 384, 208)
    t = W.make_model(spec, getattr(W, wtype), salt=91 + n_head,
                     output_type=W.W_Q6_K if n_embd % 256 == 0 else W.W_Q8_0,
                     overrides={"attn_output.weight": getattr(W, wo_type)})
    toks = [(37 * i + 11) % spec.n_vocab for i in range(200)]
    om = O.Model(spec, t)
    want = np.stack([om.forward(tk, i) for i, tk in enumerate(toks)])
    eng = spec_engine(engines, spec)
    got = run_forward(tla, eng, spec, t, toks)
    check_logits(got, want, f"gqa {n_head // n_head_kv} x {n_head_kv} kv heads, W_o {wo_type} vs oracle")


def test_forward_errors(tla, W, engines):
    spec = W.ModelSpec(2, 256, 4, 2, 512, 384, 64)
    t = W.make_model(spec, W.W_Q8_0, salt=3)
    eng = spec_engine(engines, spec)
    dm = tla.DeviceModel(eng, t, spec.n_ff, spec.n_vocab, spec.rms_norm_eps)
    try:
        with device_arrays() as track:
            kc, vc = eng.kv_cache(1)
            track(kc), track(vc)
            lg = track(eng.array((spec.n_vocab,)))
            for tok, pos, code in ((384, 0, 2), (-1, 0, 2), (0, 64, 2)):
                with pytest.raises(tla.TlaError) as e:
                    eng.forward(dm, kc.ptr, vc.ptr, tok, pos, lg.ptr)
                assert e.value.code == code
            dm.c.n_ff = 544  # whole Q8_0 blocks, not a multiple of 64: unsupported GEMV columns
            with pytest.raises(tla.TlaError) as e:
                eng.forward(dm, kc.ptr, vc.ptr, 0, 0, lg.ptr)
            assert e.value.code == 3
            dm.c.n_ff = 512
            with pytest.raises(tla.TlaError) as e:
                eng.generate_greedy(dm, kc.ptr, vc.ptr, [1, 2], 64)  # 2 + 64 - 1 > n_ctx
            assert e.value.code == 2
            # a NULL projection weight in any layer is rejected before any launch
            for field in ("wq", "wo", "w_down"):
                saved = getattr(dm.layers[1], field)
                setattr(dm.layers[1], field, None)
                try:
                    for call in (lambda: eng.forward(dm, kc.ptr, vc.ptr, 0, 0, lg.ptr),
                                 lambda: eng.prefill_forward(dm, kc.ptr, vc.ptr, [1, 2, 3], 0, lg.ptr),
                                 lambda: eng.generate_greedy(dm, kc.ptr, vc.ptr, [1, 2], 4)):
                        with pytest.raises(tla.TlaError) as e:
                            call()
                        assert e.value.code == tla.TLA_ERR_INVALID_ARGUMENT, (field, tla.last_error())
                finally:
                    setattr(dm.layers[1], field, saved)
            eng.forward(dm, kc.ptr, vc.ptr, 0, 0, lg.ptr)  # restored: runs
            eng.synchronize()
    finally:
        dm.free()


@pytest.mark.parametrize("name", CASES)
def test_prefill_forward_matches_token_loop(tla, O, W, engines, name):
    """tla_prefill_forward: the prompt as one batch (src/generate.cpp:56-59
    batched).  The last token's logits against the reference's (golden),
    in one call and in two calls (pos0 > 0); the KV cache against the
    token-by-token device path within 1e-4 of the largest entry (the
    streamed products sum in another order), and the layer 0 of a prompt
    short enough for the multi-vector GEMVs (2 tokens of Q8_0 / Q4_0, else
    1) bit for bit (their sums are the token path's; the inputs are the
    embeddings in both)."""
    g = golden("forward.npz")
    spec, t = model_from_golden(W, g, name)
    eng = spec_engine(engines, spec)
    toks = g["tokens"].tolist()
    want = g[f"{name}_logits"][-1]
    dm = tla.DeviceModel(eng, t, spec.n_ff, spec.n_vocab, spec.rms_norm_eps)
    try:
        with device_arrays() as track:
            kc, vc = eng.kv_cache(1)
            track(kc), track(vc)
            kc2, vc2 = eng.kv_cache(1)
            track(kc2), track(vc2)
            lg = track(eng.array((spec.n_vocab,)))
            eng.prefill_forward(dm, kc.ptr, vc.ptr, toks, 0, lg.ptr)
            check_logits(lg.download()[None], want[None], f"{name} prefill_forward, one batch")
            eng.prefill_forward(dm, kc2.ptr, vc2.ptr, toks[:7], 0, lg.ptr)
            eng.prefill_forward(dm, kc2.ptr, vc2.ptr, toks[7:], 7, lg.ptr)
            check_logits(lg.download()[None], want[None], f"{name} prefill_forward, two batches")
            batch_k, batch_v = kc.download(), vc.download()
            kc4, vc4 = eng.kv_cache(1)
            track(kc4), track(vc4)
            n_short = 2 if name in ("q8_0", "q4_0") else 1
            eng.prefill_forward(dm, kc4.ptr, vc4.ptr, toks[:n_short], 0, lg.ptr)
            short_k, short_v = kc4.download(), vc4.download()
            # token-by-token device path into fresh caches
            kc3, vc3 = eng.kv_cache(1)
            track(kc3), track(vc3)
            for i, tk in enumerate(toks):
                eng.forward(dm, kc3.ptr, vc3.ptr, int(tk), i, lg.ptr)
            loop_k, loop_v = kc3.download(), vc3.download()
    finally:
        dm.free()
    n = len(toks)
    assert np.array_equal(bits(short_k[0, 0, :n_short]), bits(loop_k[0, 0, :n_short])), "layer 0 keys"
    assert np.array_equal(bits(short_v[0, 0, :n_short]), bits(loop_v[0, 0, :n_short])), "layer 0 values"
    for a, b in ((batch_k, loop_k), (batch_v, loop_v)):
        assert np.abs(a - b).max() <= 1e-4 * np.abs(b).max()


@pytest.mark.parametrize("name", ["q8_0", "mixed"])
def test_generate_greedy_batched_prompt(tla, O, W, engines, name):
    g = golden("forward.npz")
    spec, t = model_from_golden(W, g, name)
    eng = spec_engine(engines, spec)
    dm = tla.DeviceModel(eng, t, spec.n_ff, spec.n_vocab, spec.rms_norm_eps)
    try:
        with device_arrays() as track:
            kc, vc = eng.kv_cache(1)
            track(kc), track(vc)
            got = eng.generate_greedy(dm, kc.ptr, vc.ptr, g["prompt"].tolist(),
                                      len(g[f"{name}_greedy"]), batch_prompt=True)
    finally:
        dm.free()
    assert got == g[f"{name}_greedy"].tolist()


def test_prefill_forward_errors(tla, W, engines):
    spec = W.ModelSpec(2, 256, 4, 2, 512, 384, 64)
    t = W.make_model(spec, W.W_Q8_0, salt=3)
    eng = spec_engine(engines, spec)
    dm = tla.DeviceModel(eng, t, spec.n_ff, spec.n_vocab, spec.rms_norm_eps)
    try:
        with device_arrays() as track:
            kc, vc = eng.kv_cache(1)
            track(kc), track(vc)
            lg = track(eng.array((spec.n_vocab,)))
            for toks, pos0 in (([1, 2, 384], 0), ([1] * 10, 60), ([1], -1)):
                with pytest.raises(tla.TlaError) as e:
                    eng.prefill_forward(dm, kc.ptr, vc.ptr, toks, pos0, lg.ptr)
                assert e.value.code == 2
    finally:
        dm.free()


@pytest.mark.parametrize("name", ["q8_0", "f16_tied", "q4_0", "mixed"])
def test_prefill_forward_long_prompt(tla, O, W, engines, name):
    """A 48-token prompt: the batched projections as streamed products with
    three token tiles (Q6_K matrices as split products).
    Last token's logits against the oracle's token loop."""
    g = golden("forward.npz")
    spec, t = model_from_golden(W, g, name)
    eng = spec_engine(engines, spec)
    toks = np.random.default_rng(48).integers(0, spec.n_vocab, 48).tolist()
    om = O.Model(spec, t)
    want = om.tokens(toks)[-1]
    dm = tla.DeviceModel(eng, t, spec.n_ff, spec.n_vocab, spec.rms_norm_eps)
    try:
        with device_arrays() as track:
            kc, vc = eng.kv_cache(1)
            track(kc), track(vc)
            lg = track(eng.array((spec.n_vocab,)))
            eng.prefill_forward(dm, kc.ptr, vc.ptr, toks, 0, lg.ptr)
            got = lg.download()
            k_dev = kc.download()
    finally:
        dm.free()
    check_logits(got[None], want[None], f"{name} 48-token batched prompt vs oracle")
    kv = spec.kv_dim
    ok = om.kc.reshape(spec.n_layers, spec.n_ctx, kv)
    assert np.abs(k_dev[0, :, :48] - ok[:, :48]).max() <= 1e-4 * np.abs(ok[:, :48]).max()


@pytest.mark.parametrize("name", ["q8_0", "f16_tied", "q4_0", "f32", "mixed"])
def test_prefill_forward_streamed_prompt(tla, O, W, engines, name):
    """A 32-token prompt, in one call and as two calls of 16 (the second at
    pos0 = 16): every batched projection as the streamed product (weights
    dequantised in registers; Q/K/V as one product of three segments where
    their formats agree).  Last token's logits and the K cache against the
    oracle's token loop."""
    g = golden("forward.npz")
    spec, t = model_from_golden(W, g, name)
    eng = spec_engine(engines, spec)
    n = 32
    toks = np.random.default_rng(32).integers(0, spec.n_vocab, n).tolist()
    om = O.Model(spec, t)
    want = om.tokens(toks)[-1]
    dm = tla.DeviceModel(eng, t, spec.n_ff, spec.n_vocab, spec.rms_norm_eps)
    try:
        with device_arrays() as track:
            kc, vc = eng.kv_cache(1)
            track(kc), track(vc)
            lg = track(eng.array((spec.n_vocab,)))
            eng.prefill_forward(dm, kc.ptr, vc.ptr, toks, 0, lg.ptr)
            got = lg.download()
            k_dev = kc.download()
            kc2, vc2 = eng.kv_cache(1)
            track(kc2), track(vc2)
            eng.prefill_forward(dm, kc2.ptr, vc2.ptr, toks[:16], 0, lg.ptr)
            eng.prefill_forward(dm, kc2.ptr, vc2.ptr, toks[16:], 16, lg.ptr)
            got2 = lg.download()
            k_dev2 = kc2.download()
    finally:
        dm.free()
    check_logits(got[None], want[None], f"{name} {n}-token streamed prompt vs oracle")
    check_logits(got2[None], want[None], f"{name} {n}-token prompt as 16 + 16 vs oracle")
    ok = om.kc.reshape(spec.n_layers, spec.n_ctx, spec.kv_dim)
    for kd in (k_dev, k_dev2):
        assert np.abs(kd[0, :, :n] - ok[:, :n]).max() <= 1e-4 * np.abs(ok[:, :n]).max()


@pytest.mark.parametrize("name", ["q8_0", "f16_tied", "q4_0", "f32", "mixed"])
def test_prefill_forward_split_prompt(tla, O, W, engines, name):
    """A 300-token prompt: every batched projection as the split product (bf16
    pieces on the matrix cores, fp32 sums), Q/K/V as one launch of three
    segments where their formats agree and gate | up as one of two.  The
    golden case's weights on a 320-position context, in one call and as two
    calls of 150 tokens (the second at pos0 = 150); last token's logits and
    the whole K cache against the oracle's token loop."""
    g = golden("forward.npz")
    base = W.ModelSpec(*[int(v) for v in g["spec"]])
    spec = W.ModelSpec(base.n_layers, base.n_embd, base.n_head, base.n_head_kv, base.n_ff, base.n_vocab,
                       320)
    salt, wt, et, ot = [int(v) for v in g[f"{name}_case"]]
    ov = dict(ast.literal_eval(str(g[f"{name}_overrides"])))
    t = W.make_model(spec, wt, salt=salt, embd_type=None if et < 0 else et,
                     output_type=None if ot < 0 else ot, overrides=ov)
    eng = spec_engine(engines, spec)
    n = 300
    toks = np.random.default_rng(300).integers(0, spec.n_vocab, n).tolist()
    om = O.Model(spec, t)
    want = om.tokens(toks)[-1]
    log(f"  {name}: {n}-token prompt through the split products")
    dm = tla.DeviceModel(eng, t, spec.n_ff, spec.n_vocab, spec.rms_norm_eps)
    try:
        with device_arrays() as track:
            kc, vc = eng.kv_cache(1)
            track(kc), track(vc)
            lg = track(eng.array((spec.n_vocab,)))
            eng.prefill_forward(dm, kc.ptr, vc.ptr, toks, 0, lg.ptr)
            got = lg.download()
            k_dev = kc.download()
            # the same prompt as two batches of 150 (the second at pos0 = 150)
            kc2, vc2 = eng.kv_cache(1)
            track(kc2), track(vc2)
            eng.prefill_forward(dm, kc2.ptr, vc2.ptr, toks[:150], 0, lg.ptr)
            eng.prefill_forward(dm, kc2.ptr, vc2.ptr, toks[150:], 150, lg.ptr)
            got2 = lg.download()
            k_dev2 = kc2.download()
    finally:
        dm.free()
    check_logits(got[None], want[None], f"{name} {n}-token batched prompt vs oracle")
    check_logits(got2[None], want[None], f"{name} {n}-token prompt in two batches vs oracle")
    ok = om.kc.reshape(spec.n_layers, spec.n_ctx, spec.kv_dim)
    for kd in (k_dev, k_dev2):
        assert np.abs(kd[0, :, :n] - ok[:, :n]).max() <= 1e-4 * np.abs(ok[:, :n]).max()


def test_prefill_forward_after_queued_weight_writes(tla, O, W, engines):
    """Weights written on the engine's stream and not yet synchronized when a
    prompt starts: every product of the prompt must see them.  Layers 0 and
    1 are overwritten with garbage, then restored with tla_memcpy_d2d, and a
    100-token prompt follows at once; its last logits against the oracle's
    token loop."""
    g = golden("forward.npz")
    base = W.ModelSpec(*[int(v) for v in g["spec"]])
    spec = W.ModelSpec(base.n_layers, base.n_embd, base.n_head, base.n_head_kv, base.n_ff, base.n_vocab,
                       128)
    salt, wt, et, ot = [int(v) for v in g["q8_0_case"]]
    ov = dict(ast.literal_eval(str(g["q8_0_overrides"])))
    t = W.make_model(spec, wt, salt=salt, embd_type=None if et < 0 else et,
                     output_type=None if ot < 0 else ot, overrides=ov)
    eng = spec_engine(engines, spec)
    toks = np.random.default_rng(100).integers(0, spec.n_vocab, 100).tolist()
    want = O.Model(spec, t).tokens(toks)[-1]
    names = [f"blk.{l}.{w}.weight" for l in (0, 1)
             for w in ("attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down")]
    dm = tla.DeviceModel(eng, t, spec.n_ff, spec.n_vocab, spec.rms_norm_eps)
    try:
        with device_arrays() as track:
            saved = {n: track(eng.array(np.ascontiguousarray(t[n][2], np.uint8))) for n in names}
            junk = np.random.default_rng(7).integers(0, 256, max(a.nbytes for a in saved.values()), np.uint8)
            for n in names:
                dm.arrays[n].upload(junk[:dm.arrays[n].nbytes])
            eng.synchronize()
            kc, vc = eng.kv_cache(1)
            track(kc), track(vc)
            lg = track(eng.array((spec.n_vocab,)))
            for n in names:
                eng.copy(dm.arrays[n].ptr, saved[n].ptr, saved[n].nbytes)
            eng.prefill_forward(dm, kc.ptr, vc.ptr, toks, 0, lg.ptr)
            got = lg.download()
    finally:
        dm.free()
    check_logits(got[None], want[None], "100-token prompt after queued weight writes vs oracle")
