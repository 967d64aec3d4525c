"""CPU tests that pin the oracle (oracle/tl_oracle.c) before anything is
compared with it:

  1. golden vectors written from the compiled reference (tests/golden/),
     bit for bit;
  2. the compiled reference itself, live, where oracle/_ref was built;
  3. mathematics that fixes the answer independently: closed forms,
     invariants, fp64 brute force, torch's SDPA;
  4. planted mistakes (oracle_fault) -- each must trip at least one pin.
"""
import math

import numpy as np
import pytest

from conftest import golden

S = None


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def assert_bitexact(a, b, what=""):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    assert a.shape == b.shape, (what, a.shape, b.shape)
    diff = np.flatnonzero(bits(a).reshape(-1) != bits(b).reshape(-1))
    assert diff.size == 0, f"{what}: {diff.size} elements differ, first at {diff[:5]}"


# ---------------------------------------------------------------- golden ----

def test_softmax_golden(O):
    g = golden("softmax.npz")
    names = [n[3:] for n in g.files if n.startswith("in_")]
    assert len(names) >= 18
    for n in names:
        assert_bitexact(O.softmax(g["in_" + n]), g["out_" + n], n)


def test_rope_golden(O):
    g = golden("rope.npz")
    s = O.Shape()
    for i, p in enumerate(g["positions"]):
        q, k = O.rope(g["q"], g["k"], int(p), s)
        assert_bitexact(q, g["q_out"][i], f"q pos {p}")
        assert_bitexact(k, g["k_out"][i], f"k pos {p}")
    q, k = O.rope(g["manual_q"], np.zeros(s.kv_dim, np.float32), 1, s)
    assert_bitexact(q, g["manual_q_out"], "manual pair")


def test_attention_testops_golden(O):
    """src/test_ops.cpp:295-431 cases, replayed: bit-exact, plus the
    reference's own assertions."""
    g = golden("attention_testops.npz")
    s = O.Shape(n_ctx=64, n_layers=2)
    n = s.n_layers * s.n_ctx * s.kv_dim
    ones_q, ones_k = np.ones(s.q_dim, np.float32), np.ones(s.kv_dim, np.float32)

    kc, vc = np.zeros(n, np.float32), np.zeros(n, np.float32)
    v1 = (np.arange(s.kv_dim) % 64).astype(np.float32)
    out = O.attention(ones_q, ones_k, v1, kc, vc, 0, 0, s)
    assert_bitexact(out, g["t1_out"], "T1")
    assert np.all(np.abs(out[:64] - np.arange(64)) < 1e-3)

    kc, vc = np.zeros(n, np.float32), np.zeros(n, np.float32)
    O.attention(ones_q, ones_k, np.ones(s.kv_dim, np.float32), kc, vc, 0, 0, s)
    out = O.attention(ones_q, ones_k, np.full(s.kv_dim, 3, np.float32), kc, vc, 0, 1, s)
    assert_bitexact(out, g["t2_out"], "T2")
    assert abs(out[0] - 2.0) < 0.01

    kc, vc = np.zeros(n, np.float32), np.zeros(n, np.float32)
    for p in range(10):
        out = O.attention(g["t3_q"][p], g["t3_k"][p], g["t3_v"][p], kc, vc, 0, p, s)
        assert_bitexact(out, g["t3_out"][p], f"T3 token {p}")
    assert np.all(np.isfinite(out))
    assert_bitexact(kc, g["t3_kc"], "T3 key cache")
    assert_bitexact(vc, g["t3_vc"], "T3 value cache")

    kc, vc = np.zeros(n, np.float32), np.zeros(n, np.float32)
    out = O.attention(ones_q, ones_k, g["t4_v"], kc, vc, 0, 0, s)
    assert_bitexact(out, g["t4_out"], "T4")
    assert abs(out[0] - 10) < 0.01 and abs(out[8 * 64] - 20) < 0.01


def test_decode_single_golden(O, W):
    g = golden("decode_single.npz")
    s = O.Shape(n_ctx=128, n_layers=1)
    rg = W.rng("decode_single", 7)
    q, k, v = W.normal(rg, (128, s.q_dim)), W.normal(rg, (128, s.kv_dim)), W.normal(rg, (128, s.kv_dim))
    assert W.digest(q, k, v) == str(g["digest"]), "input generator drifted on this host"
    kc = np.zeros(s.n_ctx * s.kv_dim, np.float32)
    vc = np.zeros_like(kc)
    for p in range(128):
        qr, kr = O.rope(q[p], k[p], p, s)
        out = O.attention(qr, kr, v[p], kc, vc, 0, p, s)
    assert_bitexact(out, g["out"], "out")
    assert_bitexact(kc, g["kc"], "key cache")
    assert_bitexact(vc, g["vc"], "value cache")


def test_decode_peaked_golden(O, W):
    g = golden("decode_peaked.npz")
    s = O.Shape(n_ctx=1024, n_layers=1)
    case = W.make_decode("decode_long", 1, 1, 1024, 1023, kv_std=0.5, peaked_frac=0.01, salt=7)
    assert W.digest(case.q, case.k, case.v, case.kc, case.vc) == str(g["digest"])
    kc, vc = case.kc.reshape(-1).copy(), case.vc.reshape(-1).copy()
    qr, kr = O.rope(case.q[0, 0], case.k[0, 0], 1023, s)
    out = O.attention(qr, kr, case.v[0, 0], kc, vc, 0, 1023, s)
    assert_bitexact(out, g["out"], "out")
    assert_bitexact(kc.reshape(1024, -1)[1023], g["k_row"], "appended k")


def test_decode_ragged_golden(O, W):
    g = golden("decode_ragged.npz")
    s = O.Shape(n_ctx=64, n_layers=2)
    pos = [int(p) for p in g["pos"]]
    case = W.make_decode("decode_ragged", 3, 2, 64, pos, salt=7)
    assert W.digest(case.q, case.k, case.v, case.kc, case.vc) == str(g["digest"])
    for si in range(3):
        kc, vc = case.kc[si].reshape(-1).copy(), case.vc[si].reshape(-1).copy()
        for layer in range(2):
            qr, kr = O.rope(case.q[si, layer], case.k[si, layer], pos[si], s)
            out = O.attention(qr, kr, case.v[si, layer], kc, vc, layer, pos[si], s)
            assert_bitexact(out, g["out"][si, layer], f"seq {si} layer {layer}")


def test_prefill_golden(O, W):
    g = golden("prefill.npz")
    s = O.Shape(n_ctx=64, n_layers=2)
    case = W.make_prefill(n_layers=1, n_tok=40, salt=7)
    assert W.digest(case.q, case.k, case.v) == str(g["digest"])
    kc = np.zeros(2 * 64 * s.kv_dim, np.float32)
    vc = np.zeros_like(kc)
    out = O.prefill(case.q[0], case.k[0], case.v[0], kc, vc, 1, 0, s)
    assert_bitexact(out, g["out"], "prefill out")
    assert_bitexact(kc.reshape(2, 64, -1)[1, :40], g["kc"], "key cache")
    assert_bitexact(vc.reshape(2, 64, -1)[1, :40], g["vc"], "value cache")


# ------------------------------------------------------- live reference ----

needs_ref = pytest.mark.skipif(not __import__("oracle").ref_available(),
                               reason="oracle/_ref not built (no /root/reference here)")


@needs_ref
def test_live_reference_rope_and_softmax(O):
    R, s = O.ref(), O.Shape()
    rg = np.random.default_rng(11)
    for pos in list(range(0, 70)) + [int(x) for x in rg.integers(0, 1 << 17, 60)]:
        q = rg.standard_normal(s.q_dim).astype(np.float32) * 3
        k = rg.standard_normal(s.kv_dim).astype(np.float32) * 3
        a, b = O.rope(q, k, pos, s), O.rope(q, k, pos, s, lib=R)
        assert_bitexact(a[0], b[0], f"q {pos}")
        assert_bitexact(a[1], b[1], f"k {pos}")
    for n in (1, 3, 100, 4097):
        x = (rg.standard_normal(n) * 20).astype(np.float32)
        assert_bitexact(O.softmax(x), O.softmax(x, lib=R), f"softmax {n}")


@needs_ref
def test_live_reference_attention(O):
    R = O.ref()
    s = O.Shape(n_ctx=300, n_layers=3)
    rg = np.random.default_rng(12)
    n = s.n_layers * s.n_ctx * s.kv_dim
    kc1, vc1 = np.zeros(n, np.float32), np.zeros(n, np.float32)
    kc2, vc2 = kc1.copy(), vc1.copy()
    for pos in range(300):
        layer = pos % 3
        q = rg.standard_normal(s.q_dim).astype(np.float32)
        k = rg.standard_normal(s.kv_dim).astype(np.float32)
        v = rg.standard_normal(s.kv_dim).astype(np.float32)
        a = O.attention(q, k, v, kc1, vc1, layer, pos, s)
        b = O.attention(q, k, v, kc2, vc2, layer, pos, s, lib=R)
        assert_bitexact(a, b, f"pos {pos}")
    assert_bitexact(kc1, kc2, "key caches")
    assert_bitexact(vc1, vc2, "value caches")


@needs_ref
def test_live_reference_prefill_loop(O, W):
    """The prompt loop through the reference's own rope() + attention() (the
    prefill CPU baseline) equals the restatement bit for bit, outputs and
    caches, at layer 1 of 2 from a nonzero start position."""
    case = W.make_prefill(n_layers=1, n_tok=70, salt=13)
    s = O.Shape(n_ctx=96, n_layers=2)
    outs = []
    for lib in (None, O.ref()):
        kc = np.zeros(2 * 96 * s.kv_dim, np.float32)
        vc = np.zeros_like(kc)
        outs.append((O.prefill(case.q[0], case.k[0], case.v[0], kc, vc, 1, 9, s, lib=lib), kc, vc))
    for a, b in zip(outs[0], outs[1]):
        assert_bitexact(a, b, "prefill loop")


@needs_ref
def test_live_reference_threaded_units(O, W):
    case = W.make_decode(9, 6, 1, 96, [0, 5, 31, 32, 64, 95])
    s = O.Shape(n_ctx=96)
    outs = []
    for lib in (None, O.ref()):
        kc, vc = case.kc.copy(), case.vc.copy()
        outs.append(O.decode_units_mt(3, case.q.reshape(6, -1), case.k.reshape(6, -1),
                                      case.v.reshape(6, -1), kc, vc, case.pos, s, lib=lib))
    assert_bitexact(outs[0], outs[1], "threaded units")


# ---------------------------------------------------------- mathematics ----

def rope_f64(x, pos, head_dim=64, base=10000.0):
    """Adjacent-pair rotation in float64 (independent closed form)."""
    x = np.asarray(x, np.float64).reshape(-1, head_dim)
    i = np.arange(head_dim // 2)
    ang = pos * base ** (-2.0 * i / head_dim)
    c, s = np.cos(ang), np.sin(ang)
    out = x.copy()
    out[:, 0::2] = x[:, 0::2] * c - x[:, 1::2] * s
    out[:, 1::2] = x[:, 0::2] * s + x[:, 1::2] * c
    return out.reshape(-1)


def pin_failures(O, W):
    """Run every mathematical pin on the oracle; return names of those that fail."""
    fails = []
    s = O.Shape(n_ctx=96, n_layers=2)
    rg = np.random.default_rng(5)
    # rope: identity at 0, closed form, norm
    q = rg.standard_normal(s.q_dim).astype(np.float32)
    k = rg.standard_normal(s.kv_dim).astype(np.float32)
    q0, k0 = O.rope(q, k, 0, s)
    if not (np.array_equal(q0, q) and np.array_equal(k0, k)):
        fails.append("rope identity")
    for pos in (1, 7, 50, 300):
        qp, kp = O.rope(q, k, pos, s)
        if np.abs(qp - rope_f64(q, pos)).max() > 2e-4 or np.abs(kp - rope_f64(k, pos)).max() > 2e-4:
            fails.append(f"rope closed form {pos}")
        pairs_in = np.hypot(q[0::2].astype(np.float64), q[1::2])
        pairs_out = np.hypot(qp[0::2].astype(np.float64), qp[1::2])
        if np.abs(pairs_in - pairs_out).max() > 1e-5 * max(1.0, pairs_in.max()):
            fails.append(f"rope pair norm {pos}")
    # softmax
    x = np.array([1000, 1000, 999], np.float32)
    y = O.softmax(x)
    if not np.all(np.isfinite(y)):
        fails.append("softmax large logits")
    x = (rg.standard_normal(777) * 4).astype(np.float32)
    ref = np.exp(x.astype(np.float64) - x.max())
    ref /= ref.sum()
    if np.abs(O.softmax(x) - ref).max() > 1e-6:
        fails.append("softmax fp64")
    # attention against fp64 brute force, several positions and both layers
    n = s.n_layers * s.n_ctx * s.kv_dim
    kc, vc = np.zeros(n, np.float32), np.zeros(n, np.float32)
    for pos in range(60):
        layer = pos % 2
        q = rg.standard_normal(s.q_dim).astype(np.float32)
        k = rg.standard_normal(s.kv_dim).astype(np.float32)
        v = rg.standard_normal(s.kv_dim).astype(np.float32)
        out = O.attention(q, k, v, kc, vc, layer, pos, s)
        ref = O.attention_f64(q, kc, vc, layer, pos, s)
        if np.abs(out - ref).max() > 1e-5:
            fails.append(f"attention fp64 pos {pos}")
            break
    # pos 0 -> out = v of the head's kv head; GQA map with distinct V per kv head
    kc, vc = np.zeros(n, np.float32), np.zeros(n, np.float32)
    v = np.repeat(np.arange(1, 5, dtype=np.float32) * 10, 64)
    out = O.attention(q, k, v, kc, vc, 1, 0, s).reshape(32, 64)
    if not np.array_equal(out, np.repeat(np.arange(1, 5, dtype=np.float32) * 10, 8)[:, None]
                          * np.ones((1, 64), np.float32)):
        fails.append("gqa map / pos 0")
    # equal keys average V
    kc, vc = np.zeros(n, np.float32), np.zeros(n, np.float32)
    kk = rg.standard_normal(s.kv_dim).astype(np.float32)
    vs = rg.standard_normal((5, s.kv_dim)).astype(np.float32)
    for pos in range(5):
        out = O.attention(q, kk, vs[pos], kc, vc, 0, pos, s)
    expect = np.repeat(vs.mean(0).reshape(4, 64), 8, axis=0).reshape(-1)
    if np.abs(out - expect).max() > 1e-5:
        fails.append("equal keys mean")
    return fails


def test_math_pins_pass_on_faithful_oracle(O, W):
    assert pin_failures(O, W) == []


@pytest.mark.parametrize("mode,name", [(1, "rope sin sign"), (2, "gqa modulo"), (3, "no scale"),
                                       (4, "skip last position"), (5, "half-split pairs"),
                                       (6, "softmax without max")])
def test_planted_mistakes_are_caught(O, W, faulty_oracle, mode, name):
    faulty_oracle(mode)
    assert pin_failures(O, W), f"planted mistake '{name}' passed every pin"


def test_prefill_matches_torch_sdpa(O, W):
    """The oracle's token-by-token prompt loop equals causal SDPA (fp64, CPU)
    over independently rotated q/k with kv heads repeated per GQA group."""
    torch = pytest.importorskip("torch")
    s = O.Shape(n_ctx=80, n_layers=1)
    case = W.make_prefill(n_layers=1, n_tok=70, salt=3)
    kc = np.zeros(s.n_ctx * s.kv_dim, np.float32)
    vc = np.zeros_like(kc)
    out = O.prefill(case.q[0], case.k[0], case.v[0], kc, vc, 0, 0, s)
    qr = np.stack([rope_f64(case.q[0, t], t) for t in range(70)]).reshape(70, 32, 64)
    kr = np.stack([rope_f64(case.k[0, t], t) for t in range(70)]).reshape(70, 4, 64)
    vv = case.v[0].astype(np.float64).reshape(70, 4, 64)
    Q = torch.from_numpy(qr).permute(1, 0, 2)                               # [32, T, 64]
    K = torch.from_numpy(np.repeat(kr, 8, axis=1)).permute(1, 0, 2)        # qh -> qh // 8
    V = torch.from_numpy(np.repeat(vv, 8, axis=1)).permute(1, 0, 2)
    ref = torch.nn.functional.scaled_dot_product_attention(Q, K, V, is_causal=True)
    ref = ref.permute(1, 0, 2).reshape(70, -1).numpy()
    assert np.abs(out - ref).max() < 2e-5


def test_threaded_oracle_equals_single_thread(O, W):
    case = W.make_decode(9, 5, 1, 64, [0, 1, 17, 40, 63], salt=2)
    s = O.Shape(n_ctx=64)
    a_kc, a_vc = case.kc.copy(), case.vc.copy()
    a = O.decode_units_mt(1, case.q.reshape(5, -1), case.k.reshape(5, -1), case.v.reshape(5, -1),
                          a_kc, a_vc, case.pos, s)
    b_kc, b_vc = case.kc.copy(), case.vc.copy()
    b = O.decode_units_mt(4, case.q.reshape(5, -1), case.k.reshape(5, -1), case.v.reshape(5, -1),
                          b_kc, b_vc, case.pos, s)
    assert_bitexact(a, b)
    assert_bitexact(a_kc, b_kc)
