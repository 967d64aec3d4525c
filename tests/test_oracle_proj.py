"""CPU tests that pin the oracle's projections (matmul in the five weight
formats, rmsnorm, vec_add, fp16_to_f32) before the GPU is compared with it:

  1. golden vectors from the compiled reference (tests/golden/projections.npz),
     bit for bit;
  2. the compiled reference itself, live, where oracle/_ref was built;
  3. the reference's own known-answer cases (src/test_ops.cpp:42-128,
     638-853), with its assertions;
  4. fp64 dequantisation written from the format descriptions
     (tests/quant_ref.py) and fp64 rmsnorm;
  5. planted mistakes (oracle_fault 7-9) -- each must trip a pin.
"""
import numpy as np
import pytest

import quant_ref as Q
from conftest import golden

TYPES = [(Q.F32, "f32"), (Q.F16, "f16"), (Q.Q4_0, "q4_0"), (Q.Q8_0, "q8_0"), (Q.Q6_K, "q6_k")]
needs_ref = pytest.mark.skipif(not __import__("oracle").ref_available(),
                               reason="oracle/_ref not built (no reference tree)")


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def f16(v):
    return int(np.float16(v).view(np.uint16))


# ------------------------------------------------------------------ golden --

def test_projections_golden(O):
    g = golden("projections.npz")
    for t, name in TYPES:
        raw, x = g[f"{name}_w"], g[f"{name}_x"]
        rows = g[f"{name}_out"].size
        out = O.matmul(raw, x, rows, 512, t)
        assert np.array_equal(bits(out), bits(g[f"{name}_out"])), name
    for i in range(3):
        out = O.rmsnorm(g[f"rms{i}_x"], g[f"rms{i}_w"], float(g[f"rms{i}_eps"]))
        assert np.array_equal(bits(out), bits(g[f"rms{i}_out"])), f"rmsnorm {i}"


def test_fp16_every_pattern(O):
    """All 65536 halves: the reference's conversion (golden) and numpy's."""
    g = golden("projections.npz")["fp16_bits"]
    lib = O.oracle()
    mine = np.array([np.float32(lib.oracle_fp16_to_f32(h)) for h in range(65536)],
                    np.float32).view(np.uint32)
    assert np.array_equal(mine, g)
    npv = np.arange(65536, dtype=np.uint16).view(np.float16).astype(np.float32)
    finite = np.isfinite(npv) | np.isinf(npv)
    assert np.array_equal(mine[finite], npv[finite].view(np.uint32))
    assert np.all(np.isnan(mine.view(np.float32)[~finite]))


# ------------------------------------------------------ reference test cases --

def pack_q8(d, qs):
    return np.concatenate([np.frombuffer(np.uint16(d).tobytes(), np.uint8),
                           np.asarray(qs, np.int8).view(np.uint8)])


def pack_q4(d, qs):
    return np.concatenate([np.frombuffer(np.uint16(d).tobytes(), np.uint8),
                           np.asarray(qs, np.uint8)])


def pack_q6k(d, ql, qh, sc):
    return np.concatenate([np.asarray(ql, np.uint8), np.asarray(qh, np.uint8),
                           np.asarray(sc, np.int8).view(np.uint8),
                           np.frombuffer(np.uint16(d).tobytes(), np.uint8)])


def reference_matmul_cases():
    """(name, raw bytes, x, rows, cols, type, expected, tolerance) from
    src/test_ops.cpp:42-90 and 638-853."""
    c = []
    W = np.array([1, 2, 3, 4, 5, 6], np.float32)
    c.append(("f32 2x3", W.view(np.uint8), np.ones(3, np.float32), 2, 3, Q.F32, [6, 15], 1e-5))
    x4 = np.array([3.14, 2.71, 1.41, 1.73], np.float32)
    c.append(("f32 identity", np.eye(4, dtype=np.float32).view(np.uint8).reshape(-1), x4, 4, 4,
              Q.F32, x4, 1e-5))
    wf16 = np.array([0x4000, 0x0000, 0x0000, 0x4200], np.uint16).view(np.uint8)
    c.append(("f16 2x2", wf16, np.array([5, 7], np.float32), 2, 2, Q.F16, [10, 21], 1e-5))
    ones32 = np.ones(32, np.float32)
    c.append(("q8 simple", pack_q8(f16(1.0), [2] * 32), ones32, 1, 32, Q.Q8_0, [64], 0.1))
    c.append(("q8 sequential", pack_q8(f16(0.5), np.arange(32)), ones32, 1, 32, Q.Q8_0, [248], 0.5))
    two = np.concatenate([pack_q8(f16(1.0), [1] * 32), pack_q8(f16(1.0), [1] * 32),
                          pack_q8(f16(2.0), [1] * 32), pack_q8(f16(2.0), [1] * 32)])
    c.append(("q8 two rows", two, np.ones(64, np.float32), 2, 64, Q.Q8_0, [64, 128], 0.5))
    c.append(("q8 dispatch", pack_q8(f16(1.0), [3] * 32), ones32, 1, 32, Q.Q8_0, [96], 0.5))
    c.append(("q4 nibbles 9", pack_q4(f16(1.0), [0x99] * 16), ones32, 1, 32, Q.Q4_0, [32], 0.5))
    c.append(("q4 nibbles 8", pack_q4(f16(1.0), [0x88] * 16), ones32, 1, 32, Q.Q4_0, [0], 0.5))
    c.append(("q4 dispatch", pack_q4(f16(2.0), [0x99] * 16), ones32, 1, 32, Q.Q4_0, [64], 0.5))
    ones256 = np.ones(256, np.float32)
    q6 = pack_q6k(0x3C00, np.zeros(128), np.zeros(64), np.ones(16))
    c.append(("q6k all -32", q6, ones256, 1, 256, Q.Q6_K, [-8192], 1.0))
    c.append(("q6k all 0", pack_q6k(0x3C00, np.zeros(128), np.full(64, 0xAA), np.ones(16)),
              ones256, 1, 256, Q.Q6_K, [0], 1.0))
    q6d2 = pack_q6k(0x4000, np.zeros(128), np.zeros(64), np.ones(16))
    c.append(("q6k two rows d=2", np.concatenate([q6d2, q6d2]), ones256, 2, 256, Q.Q6_K,
              [-16384, -16384], 1.0))
    return c


@pytest.mark.parametrize("case", reference_matmul_cases(), ids=lambda c: c[0])
def test_matmul_reference_known_answers(O, case):
    name, raw, x, rows, cols, t, expect, tol = case
    out = O.matmul(raw, x, rows, cols, t)
    assert np.abs(out - np.asarray(expect, np.float32)).max() <= tol, (name, out)
    if O.ref_available():
        assert np.array_equal(bits(out), bits(O.matmul(raw, x, rows, cols, t, lib=O.ref())))


def test_rmsnorm_reference_known_answers(O):
    """src/test_ops.cpp:92-128."""
    out = O.rmsnorm(np.ones(4, np.float32), np.ones(4, np.float32), 1e-5)
    assert abs(out[0] - 1.0) < 1e-3
    r = 1.0 / np.sqrt(12.5)
    x2 = np.array([3, 4], np.float32)
    out = O.rmsnorm(x2, np.ones(2, np.float32), 0.0)
    assert np.allclose(out, [3 * r, 4 * r], atol=1e-5)
    out = O.rmsnorm(x2, np.array([2, 0.5], np.float32), 0.0)
    assert np.allclose(out, [3 * r * 2, 4 * r * 0.5], atol=1e-5)


def test_vec_add(O):
    rg = np.random.default_rng(1)
    a, b = rg.standard_normal(1000).astype(np.float32), rg.standard_normal(1000).astype(np.float32)
    assert np.array_equal(O.vec_add(a, b), a + b)
    if O.ref_available():
        assert np.array_equal(O.vec_add(a, b, lib=O.ref()), a + b)


# ------------------------------------------------------------ live reference --

@needs_ref
@pytest.mark.parametrize("t,name", TYPES)
def test_matmul_live_reference(O, W, t, name):
    R = O.ref()
    rg = np.random.default_rng(t)
    for rows, cols in ((1, 256), (33, 1024), (64, 2048), (5, 5632)):
        raw = W.make_weights(t, rows, cols, salt=rows)
        x = rg.standard_normal(cols).astype(np.float32)
        assert np.array_equal(bits(O.matmul(raw, x, rows, cols, t)),
                              bits(O.matmul(raw, x, rows, cols, t, lib=R))), (name, rows, cols)


@needs_ref
def test_rmsnorm_live_reference(O):
    rg = np.random.default_rng(2)
    for n in (1, 2, 100, 2048, 5632):
        x = (rg.standard_normal(n) * 3).astype(np.float32)
        w = rg.standard_normal(n).astype(np.float32)
        assert np.array_equal(bits(O.rmsnorm(x, w, 1e-5)), bits(O.rmsnorm(x, w, 1e-5, lib=O.ref())))


# ----------------------------------------------------------- math pins ------

def proj_pin_failures(O, W):
    fails = []
    rg = np.random.default_rng(9)
    for t, name in TYPES:
        for rows, cols in ((9, 512), (4, 2048)):
            raw = W.make_weights(t, rows, cols, salt=3)
            x = rg.standard_normal(cols).astype(np.float32)
            ref, scale = Q.matmul_f64(raw, x, t, rows, cols)
            if np.max(np.abs(O.matmul(raw, x, rows, cols, t) - ref) / scale) > 1e-6:
                fails.append(f"matmul fp64 {name} {rows}x{cols}")
    for n in (64, 2048):
        x = (rg.standard_normal(n) * 2).astype(np.float32)
        w = rg.uniform(0.5, 2, n).astype(np.float32)
        x64 = x.astype(np.float64)
        ref = x64 / np.sqrt(np.mean(x64 * x64) + 1e-5) * w
        if np.max(np.abs(O.rmsnorm(x, w, 1e-5) - ref)) > 1e-5:
            fails.append(f"rmsnorm fp64 {n}")
    return fails


def test_projection_pins_pass_on_faithful_oracle(O, W):
    assert proj_pin_failures(O, W) == []


@pytest.mark.parametrize("mode,name", [(7, "q4_0 nibble order"), (8, "q6_k high-bit pairs"),
                                       (9, "rmsnorm without mean")])
def test_projection_planted_mistakes_are_caught(O, W, faulty_oracle, mode, name):
    faulty_oracle(mode)
    assert proj_pin_failures(O, W), f"planted mistake '{name}' passed every pin"
