"""GPU parity of the projections either side of the attention block, through
the C ABI: matmul() in the five weight formats (src/ops.cpp:959-983),
rmsnorm() (src/ops.cpp:1003-1055), vec_add() (src/ops.cpp:1165-1184), the
fused input half (rmsnorm + Wq/Wk/Wv, src/forward.cpp:180-190) and output half
(Wo + residual, src/forward.cpp:210-213), and the whole attention block of a
layer on the device, token by token, against the oracle.

Tolerance (fp32 accumulation in a different order than the reference's
sequential loops): per output row, |gpu - fp64| <= 1e-5 * sum_j |w_ij x_j| and
|gpu - oracle| <= 2e-5 * the same sum; rmsnorm within 1e-6 relative; vec_add
bit-exact; the chained block within max(1e-4, 5e-6 * max|x|) of the oracle's
chain, x being the residual stream."""
import numpy as np
import pytest

import quant_ref as Q
from helpers import bits, device_arrays, log

pytestmark = pytest.mark.gpu

TYPES = [(Q.F32, "f32"), (Q.F16, "f16"), (Q.Q4_0, "q4_0"), (Q.Q8_0, "q8_0"), (Q.Q6_K, "q6_k")]
ROW_TOL, ORACLE_TOL = 1e-5, 2e-5
# The residual stream of the chained block grows to |x| ~ 1e3 under random
# weights; its error is bounded relative to that magnitude.
CHAIN_REL_TOL = 5e-6


def gpu_matmul(eng, raw, x, rows, cols, t):
    with device_arrays() as track:
        w = track(eng.array(np.ascontiguousarray(raw, np.uint8)))
        xd = track(eng.array(np.ascontiguousarray(x, np.float32)))
        out = track(eng.array((rows,)))
        eng.matmul(out.ptr, w.ptr, xd.ptr, rows, cols, t)
        return out.download()


def check_rows(got, ora, raw, x, t, rows, cols, what):
    ref, scale = Q.matmul_f64(raw, x, t, rows, cols)
    scale = scale + 1e-30
    e64 = float(np.max(np.abs(got - ref) / scale))
    eor = float(np.max(np.abs(got - ora) / scale))
    log(f"    {what}: |gpu-fp64|/sum|wx| {e64:.2e}, |gpu-oracle|/sum|wx| {eor:.2e}")
    assert e64 <= ROW_TOL, what
    assert eor <= ORACLE_TOL, what


# The last two have enough rows for the launches that give each lane group
# several rows (32 lanes per row at 1024 columns, 64 at 2560).
SHAPES = [(1, 64), (3, 128), (64, 512), (256, 2048), (2048, 2048), (300, 5632), (37, 4096),
          (20000, 1024), (8200, 2560)]


@pytest.mark.parametrize("t,name", TYPES)
@pytest.mark.parametrize("rows,cols", SHAPES)
def test_matmul_parity(O, W, engines, t, name, rows, cols):
    if t == Q.Q6_K and cols % 256:
        pytest.skip("Q6_K rows are whole 256-weight super-blocks")
    raw = W.make_weights(t, rows, cols, salt=rows + cols)
    x = np.random.default_rng(rows * cols).standard_normal(cols).astype(np.float32)
    log(f"  tla_matmul {name} {rows}x{cols}")
    got = gpu_matmul(engines(1, 64), raw, x, rows, cols, t)
    check_rows(got, O.matmul(raw, x, rows, cols, t), raw, x, t, rows, cols, f"{name} {rows}x{cols}")


def pad64(raw, x, rows, cols, t):
    """A reference known-answer case widened to a multiple of 64 columns with
    zero weights (zero scale for the block formats) and zero inputs."""
    if cols % 64 == 0:
        return raw, x, cols
    c2 = (cols + 63) // 64 * 64
    rb, rb2 = Q_row_bytes(t, cols), Q_row_bytes(t, c2)
    out = np.zeros((rows, rb2), np.uint8)
    out[:, :rb] = np.asarray(raw, np.uint8).reshape(rows, rb)
    xp = np.zeros(c2, np.float32)
    xp[:cols] = x
    return out.reshape(-1), xp, c2


def Q_row_bytes(t, cols):
    return {Q.F32: 4 * cols, Q.F16: 2 * cols, Q.Q8_0: 34 * (cols // 32), Q.Q4_0: 18 * (cols // 32),
            Q.Q6_K: 210 * (cols // 256)}[t]


def test_reference_known_answers_on_gpu(engines):
    """src/test_ops.cpp:42-90 and 638-853, on the device."""
    from test_oracle_proj import reference_matmul_cases
    eng = engines(1, 64)
    for name, raw, x, rows, cols, t, expect, tol in reference_matmul_cases():
        raw2, x2, c2 = pad64(raw, x, rows, cols, t)
        got = gpu_matmul(eng, raw2, x2, rows, c2, t)
        log(f"  {name}: {got}")
        assert np.abs(got - np.asarray(expect, np.float32)).max() <= tol, name


def test_rmsnorm_and_vec_add(O, engines):
    eng = engines(1, 64)
    rg = np.random.default_rng(4)
    for n in (1, 7, 256, 2048, 5632):
        x = (rg.standard_normal(n) * 3).astype(np.float32)
        w = rg.uniform(0.5, 1.5, n).astype(np.float32)
        with device_arrays() as track:
            xd, wd, od = track(eng.array(x)), track(eng.array(w)), track(eng.array((n,)))
            eng.rmsnorm(od.ptr, xd.ptr, wd.ptr, n, 1e-5)
            got = od.download()
            ref = O.rmsnorm(x, w, 1e-5)
            assert np.max(np.abs(got - ref) / (np.abs(ref) + 1e-30)) <= 1e-6, n
            y = rg.standard_normal(n).astype(np.float32)
            yd = track(eng.array(y))
            eng.vec_add(yd.ptr, xd.ptr, n)
            assert np.array_equal(bits(yd.download()), bits(O.vec_add(y, x))), n


def tiny_block_weights(W, t, embd, kv, salt):
    return (W.make_weights(t, embd, embd, salt=salt), W.make_weights(t, kv, embd, salt=salt + 1),
            W.make_weights(t, kv, embd, salt=salt + 2), W.make_weights(t, embd, embd, salt=salt + 3))


@pytest.mark.parametrize("t,name", TYPES)
@pytest.mark.parametrize("n_seq", [1, 3, 8, 11])
def test_attn_qkv_and_out(O, W, engines, t, name, n_seq):
    """The fused input half (rmsnorm, Wq, Wk, Wv) and output half (x += Wo.xb2)
    for n_seq sequences, against the oracle's rmsnorm and matmul."""
    eng = engines(1, 64)
    embd, kv = 2048, 256
    wq, wk, wv, wo = tiny_block_weights(W, t, embd, kv, 100 + n_seq)
    rg = np.random.default_rng(n_seq)
    x = rg.standard_normal((n_seq, embd)).astype(np.float32)
    nw = rg.uniform(0.5, 1.5, embd).astype(np.float32)
    xb2 = rg.standard_normal((n_seq, embd)).astype(np.float32)
    with device_arrays() as track:
        d = {k: track(eng.array(v)) for k, v in
             (("wq", wq), ("wk", wk), ("wv", wv), ("wo", wo), ("x", x), ("nw", nw), ("xb2", xb2))}
        q, k, v = track(eng.array((n_seq, embd))), track(eng.array((n_seq, kv))), track(eng.array((n_seq, kv)))
        for norm in (True, False):
            log(f"  tla_attn_qkv {name} n_seq={n_seq} norm={norm}")
            eng.attn_qkv(n_seq, q.ptr, k.ptr, v.ptr, d["x"].ptr, d["nw"].ptr if norm else None,
                         1e-5, d["wq"].ptr, d["wk"].ptr, d["wv"].ptr, t)
            gq, gk, gv = q.download(), k.download(), v.download()
            for s in range(n_seq):
                xb = O.rmsnorm(x[s], nw, 1e-5) if norm else x[s]
                for got, raw, rows in ((gq[s], wq, embd), (gk[s], wk, kv), (gv[s], wv, kv)):
                    check_rows(got, O.matmul(raw, xb, rows, embd, t), raw, xb, t, rows, embd,
                               f"{name} seq {s} rows {rows}")
        log(f"  tla_attn_out {name} n_seq={n_seq}")
        eng.attn_out(n_seq, d["x"].ptr, d["wo"].ptr, d["xb2"].ptr, t)
        gx = d["x"].download()
        for s in range(n_seq):
            want = O.vec_add(x[s], O.matmul(wo, xb2[s], embd, embd, t))
            _, scale = Q.matmul_f64(wo, xb2[s], t, embd, embd)
            assert np.max(np.abs(gx[s] - want) / (scale + np.abs(x[s]) + 1e-30)) <= ORACLE_TOL, s


@pytest.mark.parametrize("t,name", [(Q.Q8_0, "q8_0"), (Q.F16, "f16"), (Q.Q4_0, "q4_0")])
def test_attention_block_on_device_token_by_token(O, W, engines, t, name):
    """One layer's attention block entirely on the device for 40 tokens
    (src/forward.cpp:180-213): rmsnorm + QKV (tla_attn_qkv), RoPE + append +
    attention (tla_decode), Wo + residual (tla_attn_out); the residual stream
    x carries over between tokens.  The oracle runs the reference's sequence
    of ops on the host."""
    n_ctx, embd, kv = 128, 2048, 256
    eng = engines(1, n_ctx)
    wq, wk, wv, wo = tiny_block_weights(W, t, embd, kv, 900)
    rg = np.random.default_rng(77)
    nw = rg.uniform(0.5, 1.5, embd).astype(np.float32)
    s = O.Shape(n_ctx=n_ctx, n_layers=1)
    kc_ref = np.zeros(n_ctx * kv, np.float32)
    vc_ref = np.zeros_like(kc_ref)
    x_ref = rg.standard_normal(embd).astype(np.float32)
    worst = 0.0
    with device_arrays() as track:
        d = {k: track(eng.array(v)) for k, v in
             (("wq", wq), ("wk", wk), ("wv", wv), ("wo", wo), ("nw", nw), ("x", x_ref))}
        kc, vc = eng.kv_cache(1)
        track(kc), track(vc)
        q, k, v = track(eng.array((embd,))), track(eng.array((kv,))), track(eng.array((kv,)))
        att = track(eng.array((embd,)))
        for pos in range(40):
            eng.attn_qkv(1, q.ptr, k.ptr, v.ptr, d["x"].ptr, d["nw"].ptr, 1e-5, d["wq"].ptr,
                         d["wk"].ptr, d["wv"].ptr, t)
            eng.decode(np.array([pos], np.int32), 0, 1, att.ptr, q.ptr, k.ptr, v.ptr, kc.ptr,
                       vc.ptr, 0, True)
            eng.attn_out(1, d["x"].ptr, d["wo"].ptr, att.ptr, t)
            # oracle: the reference's forward() attention half, op by op
            xb = O.rmsnorm(x_ref, nw, 1e-5)
            qh = O.matmul(wq, xb, embd, embd, t)
            kh = O.matmul(wk, xb, kv, embd, t)
            vh = O.matmul(wv, xb, kv, embd, t)
            qh, kh = O.rope(qh, kh, pos, s)
            out = O.attention(qh, kh, vh, kc_ref, vc_ref, 0, pos, s)
            x_ref = O.vec_add(x_ref, O.matmul(wo, out, embd, embd, t))
            err = float(np.abs(d["x"].download() - x_ref).max())
            bound = max(1e-4, CHAIN_REL_TOL * float(np.abs(x_ref).max()))
            worst = max(worst, err / bound)
            assert err <= bound, (pos, err, bound)
    log(f"    {name}: worst error / bound over 40 tokens {worst:.2f}")


def test_projection_errors(tla, W, engines):
    eng = engines(1, 64)
    raw = W.make_weights(Q.Q8_0, 4, 96, salt=1)  # 96 columns: 3 blocks per row
    with device_arrays() as track:
        w = track(eng.array(raw))
        x = track(eng.array(np.ones(96, np.float32)))
        out = track(eng.array((4,)))
        with pytest.raises(tla.TlaError) as e:
            eng.matmul(out.ptr, w.ptr, x.ptr, 4, 96, Q.Q8_0)
        assert e.value.code == 3  # unsupported shape
        with pytest.raises(tla.TlaError) as e:
            eng.matmul(out.ptr, w.ptr, x.ptr, 4, 64, 5)  # Q5_0: not a format of the reference
        assert e.value.code == 1
        with pytest.raises(tla.TlaError) as e:
            eng.matmul(out.ptr, w.ptr + 2, x.ptr, 1, 64, Q.Q8_0)
        assert e.value.code == 1


BATCH_SHAPES = [(32, 256, 16), (2560, 2048, 33), (64, 5632, 128), (5632, 2048, 130), (96, 512, 300),
                (2048, 2048, 256), (40, 5632, 257), (48, 256, 7), (40, 512, 20), (48, 256, 2)]
# (48, 256, 2): GEMV groups (streamed for F16 / F32); (48, 256, 7), (32, 256, 16), (40, 512, 20):
# streamed products


@pytest.mark.parametrize("t,name", TYPES)
@pytest.mark.parametrize("rows,cols,n_tok", BATCH_SHAPES)
def test_matmul_batch(O, W, engines, t, name, rows, cols, n_tok):
    """tla_matmul_batch: groups of GEMVs (under 3 tokens, F16 / F32 under 2,
    Q6_K under 16), the streamed product (up to 64 tokens, weights
    dequantised in registers) or the split product (bf16 pieces of x and of
    the weights on the matrix cores, fp32 sums), per token against the
    oracle's matmul."""
    if t == Q.Q6_K and cols % 256:
        pytest.skip("Q6_K rows are whole 256-weight super-blocks")
    eng = engines(1, 64)
    raw = W.make_weights(t, rows, cols, salt=rows + 3 * cols)
    x = np.random.default_rng(n_tok).standard_normal((n_tok, cols)).astype(np.float32)
    log(f"  tla_matmul_batch {name} {rows}x{cols}, {n_tok} tokens")
    with device_arrays() as track:
        w = track(eng.array(raw))
        xd = track(eng.array(x))
        out = track(eng.array((n_tok, rows)))
        eng.matmul_batch(out.ptr, w.ptr, xd.ptr, rows, cols, n_tok, t)
        got = out.download()
    for i in sorted({0, n_tok // 2, n_tok - 1}):
        check_rows(got[i], O.matmul(raw, x[i], rows, cols, t), raw, x[i], t, rows, cols,
                   f"{name} {rows}x{cols} token {i}")


STREAM_SHAPES = [(2560, 2048, 16), (2048, 5632, 32), (40, 64, 17), (200, 128, 31), (96, 256, 40), (72, 512, 4),
                 (2048, 2048, 9), (64, 256, 3), (48, 512, 2), (300, 256, 64), (32, 128, 65), (2048, 2048, 57)]


@pytest.mark.parametrize("t,name", TYPES)
@pytest.mark.parametrize("rows,cols,n_tok", STREAM_SHAPES)
def test_matmul_batch_streamed(tla, O, W, engines, t, name, rows, cols, n_tok):
    """The streamed product (2 or 3 to 64 tokens): rows not a multiple of its
    16-row tiles, rows of 2 blocks (two of its four waves idle), token counts
    not a multiple of 16, 57 and 64 tokens (four token tiles) and 65 tokens
    (the split product past the bound); every token against the oracle's
    matmul, and the same bits with one to four token tiles per workgroup
    (Q6_K takes the GEMVs under 16 tokens, the split product from 16)."""
    if t == Q.Q6_K and cols % 256:
        pytest.skip("Q6_K rows are whole 256-weight super-blocks")
    eng = engines(1, 64)
    raw = W.make_weights(t, rows, cols, salt=rows + 5 * cols)
    x = np.random.default_rng(n_tok + 1).standard_normal((n_tok, cols)).astype(np.float32)
    log(f"  streamed product {name} {rows}x{cols}, {n_tok} tokens")
    outs = []
    with device_arrays() as track:
        w = track(eng.array(raw))
        xd = track(eng.array(x))
        out = track(eng.array((n_tok, rows)))
        try:
            for tiles in (0, 1, 2, 3, 4):
                eng.set_option(tla.OPT_STREAM_TILES, tiles)
                eng.matmul_batch(out.ptr, w.ptr, xd.ptr, rows, cols, n_tok, t)
                outs.append(out.download())
        finally:
            eng.set_option(tla.OPT_STREAM_TILES, 0)
    for i in range(n_tok):
        check_rows(outs[0][i], O.matmul(raw, x[i], rows, cols, t), raw, x[i], t, rows, cols,
                   f"{name} {rows}x{cols} token {i}")
    for o in outs[1:]:
        assert np.array_equal(o.view(np.uint32), outs[0].view(np.uint32))


def test_stream_tiles_option(tla, engines):
    """TLA_OPT_STREAM_TILES takes 0 (per shape) to 4."""
    eng = engines(1, 64)
    for bad in (-1, 5):
        with pytest.raises(tla.TlaError) as e:
            eng.set_option(tla.OPT_STREAM_TILES, bad)
        assert e.value.code == tla.TLA_ERR_INVALID_ARGUMENT
    eng.set_option(tla.OPT_STREAM_TILES, 2)
    eng.set_option(tla.OPT_STREAM_TILES, 0)


def test_matmul_batch_many_shapes(O, W, engines):
    """Q6_K products of every batch size from 16 to 275 in a row on an engine
    of its own (the split product from 16 vectors), so that the split-x and
    partial-sum workspaces grow while products are queued; products at
    several sizes against the oracle's matmul."""
    eng = engines(1, 96)  # a key no other test uses: the workspaces start empty
    rows, cols, t = 32, 256, Q.Q6_K
    raw = W.make_weights(t, rows, cols, salt=11)
    x = np.random.default_rng(260).standard_normal((300, cols)).astype(np.float32)
    with device_arrays() as track:
        w = track(eng.array(raw))
        xd = track(eng.array(x))
        out = track(eng.array((300, rows)))
        for n_tok in range(16, 276):
            eng.matmul_batch(out.ptr, w.ptr, xd.ptr, rows, cols, n_tok, t)
            if n_tok in (16, 65, 200, 275):
                got = out.download()
                for i in (0, n_tok - 1):
                    check_rows(got[i], O.matmul(raw, x[i], rows, cols, t), raw, x[i], t, rows, cols,
                               f"{n_tok} tokens, token {i}")


SPLIT_SHAPES = [(2048, 5632, 130), (2560, 2048, 65), (11264, 2048, 100), (40, 512, 70), (300, 256, 128)]


@pytest.mark.parametrize("t,name", TYPES)
@pytest.mark.parametrize("rows,cols,n_tok", SPLIT_SHAPES)
def test_split_product_tilings(tla, O, W, engines, t, name, rows, cols, n_tok):
    """The split product with 1, 2 and 4 row subtiles per wave (K in 3
    ranges) gives the same bits: every output is one wave's sums in the same
    order.  K cut into 1, 3 and 7 ranges (sums added in range order by the
    second launch), and the per-shape choice, each within the oracle bound
    for every token checked."""
    if t == Q.Q6_K and cols % 256:
        pytest.skip("Q6_K rows are whole 256-weight super-blocks")
    eng = engines(1, 64)
    raw = W.make_weights(t, rows, cols, salt=rows + 7 * cols)
    x = np.random.default_rng(n_tok + 3).standard_normal((n_tok, cols)).astype(np.float32)
    outs = {}
    with device_arrays() as track:
        w = track(eng.array(raw))
        xd = track(eng.array(x))
        out = track(eng.array((n_tok, rows)))
        try:
            # row tilings with K fixed (the per-shape K split follows the tiling)
            eng.set_option(tla.OPT_SPLIT_K, 3)
            for v in (1, 2, 4):
                eng.set_option(tla.OPT_SPLIT_ROWS, v)
                eng.matmul_batch(out.ptr, w.ptr, xd.ptr, rows, cols, n_tok, t)
                outs[(tla.OPT_SPLIT_ROWS, v)] = out.download()
            eng.set_option(tla.OPT_SPLIT_ROWS, 0)
            for v in (0, 1, 3, 7):
                eng.set_option(tla.OPT_SPLIT_K, v)
                eng.matmul_batch(out.ptr, w.ptr, xd.ptr, rows, cols, n_tok, t)
                outs[(tla.OPT_SPLIT_K, v)] = out.download()
        finally:
            eng.set_option(tla.OPT_SPLIT_ROWS, 0)
            eng.set_option(tla.OPT_SPLIT_K, 0)
    base = outs[(tla.OPT_SPLIT_ROWS, 1)]
    for v in (2, 4):
        assert np.array_equal(outs[(tla.OPT_SPLIT_ROWS, v)].view(np.uint32), base.view(np.uint32)), v
    for (opt, v), got in outs.items():
        for i in sorted({0, n_tok // 3, n_tok - 1}):
            check_rows(got[i], O.matmul(raw, x[i], rows, cols, t), raw, x[i], t, rows, cols,
                       f"{name} {rows}x{cols} opt {opt}={v} token {i}")


def test_split_options(tla, engines):
    """TLA_OPT_SPLIT_ROWS takes 0, 1, 2, 4; TLA_OPT_SPLIT_K 0 to 64."""
    eng = engines(1, 64)
    for opt, bad in ((tla.OPT_SPLIT_ROWS, (-1, 3, 8)), (tla.OPT_SPLIT_K, (-1, 65))):
        for b in bad:
            with pytest.raises(tla.TlaError) as e:
                eng.set_option(opt, b)
            assert e.value.code == tla.TLA_ERR_INVALID_ARGUMENT
        eng.set_option(opt, 0)


@pytest.mark.parametrize("rows,cols,n_tok", [(2048, 5632, 16), (256, 2048, 300), (11264, 2048, 512)])
def test_matmul_batch_is_reproducible(W, engines, rows, cols, n_tok):
    """The split product gives the same bits when repeated (fixed tiling and
    K ranges per shape, the ranges' sums added in a fixed order)."""
    eng = engines(1, 64)
    raw = W.make_weights(Q.Q4_0, rows, cols, salt=5)
    x = np.random.default_rng(7).standard_normal((n_tok, cols)).astype(np.float32)
    with device_arrays() as track:
        w = track(eng.array(raw))
        xd = track(eng.array(x))
        out = track(eng.array((n_tok, rows)))
        first = None
        for _ in range(5):
            eng.matmul_batch(out.ptr, w.ptr, xd.ptr, rows, cols, n_tok, Q.Q4_0)
            got = out.download()
            if first is None:
                first = got
            else:
                assert np.array_equal(got.view(np.uint32), first.view(np.uint32))
