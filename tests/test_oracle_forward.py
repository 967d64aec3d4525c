"""CPU tests that pin the oracle's forward pass (embed_token, the layers,
SwiGLU FFN, classifier; src/forward.cpp:167-266) and the greedy generation
loop (src/generate.cpp:56-100) before the GPU is compared with it:

  1. golden logits and greedy tokens from the reference's own forward() and
     GGUF loader (tests/golden/forward.npz, written from GGUF files that
     tinyllama-engine_amd/gguf_writer.py produced), bit for bit, five weight layouts
     including tied embeddings and mixed per-tensor types;
  2. the compiled reference itself, live, where oracle/_ref was built;
  3. an fp64 forward written from the model's definition
     (tests/forward_ref.py), and exact dequantisation for embed_token;
  4. planted mistakes (oracle_fault 10-12) -- each must trip a pin.
"""
import importlib
import os
import tempfile

import numpy as np
import pytest

import quant_ref as Q
from conftest import golden
from forward_ref import Forward64, model_from_golden

CASES = ["q8_0", "f16_tied", "q4_0", "f32", "mixed"]
needs_ref_fwd = pytest.mark.skipif(not __import__("oracle").ref_forward_available(),
                                   reason="oracle/_ref not built (no reference tree)")


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


@pytest.mark.parametrize("name", CASES)
def test_forward_golden(O, W, name):
    g = golden("forward.npz")
    spec, t = model_from_golden(W, g, name)
    logits = O.Model(spec, t).tokens(g["tokens"])
    assert np.array_equal(bits(logits), bits(g[f"{name}_logits"])), name
    greedy = O.Model(spec, t).greedy(g["prompt"], len(g[f"{name}_greedy"]))
    assert greedy == g[f"{name}_greedy"].tolist()


def test_gguf_bytes_match_golden(W):
    """The writer reproduces the exact files the golden vectors came from."""
    import hashlib

    write_gguf = importlib.import_module("tinyllama-engine_amd.gguf_writer").write_gguf
    g = golden("forward.npz")
    for name in CASES:
        spec, t = model_from_golden(W, g, name)
        with tempfile.TemporaryDirectory() as d:
            path = os.path.join(d, "m.gguf")
            write_gguf(path, spec, t)
            assert hashlib.sha256(open(path, "rb").read()).hexdigest() == str(g[f"{name}_gguf_sha256"])


def test_silu_and_ffn_golden(O, W):
    g = golden("forward.npz")
    assert np.array_equal(bits(O.silu(g["silu_x"])), bits(g["silu_out"]))
    for t, nm in ((W.W_Q8_0, "q8_0"), (W.W_F16, "f16")):
        wg, wu = W.make_weights(t, 512, 256, salt=31), W.make_weights(t, 512, 256, salt=32)
        wd = W.make_weights(t, 256, 512, salt=33)
        assert W.digest(wg, wu, wd) == str(g[f"ffn_{nm}_w_sha256"])
        out, hb, hb2 = O.ffn_swiglu(g[f"ffn_{nm}_x"], wg, wu, wd, 512, 256, t)
        for a, key in ((out, "out"), (hb, "hb"), (hb2, "hb2")):
            assert np.array_equal(bits(a), bits(g[f"ffn_{nm}_{key}"])), (nm, key)


@needs_ref_fwd
@pytest.mark.parametrize("wtype", [8, 1, 2, 0, 14])
def test_forward_live_reference(O, W, wtype):
    """40 positions of a fresh model (different salt), every format."""
    write_gguf = importlib.import_module("tinyllama-engine_amd.gguf_writer").write_gguf
    spec = W.ModelSpec(2, 256, 4, 1, 768, 300, 48)
    t = W.make_model(spec, wtype, salt=50 + wtype, output_type=None)
    toks = np.random.default_rng(wtype).integers(0, spec.n_vocab, 40)
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "m.gguf")
        write_gguf(path, spec, t)
        ref = O.ref_forward_tokens(path, toks, spec.n_vocab)
        ref_greedy = O.ref_generate_greedy(path, toks[:5], 20)
    assert np.array_equal(bits(O.Model(spec, t).tokens(toks)), bits(ref))
    assert O.Model(spec, t).greedy(toks[:5], 20) == ref_greedy


@needs_ref_fwd
def test_ffn_and_silu_live_reference(O, W):
    R = O.ref()
    rg = np.random.default_rng(3)
    x = (rg.standard_normal(5000) * 6).astype(np.float32)
    assert np.array_equal(bits(O.silu(x)), bits(O.silu(x, lib=R)))
    for t in (W.W_Q4_0, W.W_Q6_K, W.W_F32):
        wg, wu = W.make_weights(t, 768, 512, salt=41), W.make_weights(t, 768, 512, salt=42)
        wd = W.make_weights(t, 512, 768, salt=43)
        xin = rg.standard_normal(512).astype(np.float32)
        mine = O.ffn_swiglu(xin, wg, wu, wd, 768, 512, t)
        ref = O.ffn_swiglu(xin, wg, wu, wd, 768, 512, t, lib=R)
        for a, b in zip(mine, ref):
            assert np.array_equal(bits(a), bits(b)), t


@pytest.mark.parametrize("wtype", [0, 1, 2, 8, 14])
def test_embed_is_exact_dequantisation(O, W, wtype):
    """Every dequantised value is exact in fp32 (at most 23 significant bits),
    so embed_token equals the fp64 dequantisation bit for bit."""
    n_vocab, n_embd = 37, 512
    raw = W.make_weights(wtype, n_vocab, n_embd, salt=7)
    table = Q.dequant(raw, wtype, n_vocab, n_embd)
    for tok in (0, 1, 17, 36):
        got = O.embed(raw, tok, n_embd, wtype)
        assert np.array_equal(got.astype(np.float64), table[tok]), (wtype, tok)


def forward_pin_failures(O, W):
    g = golden("forward.npz")
    fails = []
    for name in ("q8_0", "mixed"):
        spec, t = model_from_golden(W, g, name)
        mine = O.Model(spec, t).tokens(g["tokens"][:6])
        f = Forward64(spec, t)
        ref = np.stack([f.forward(int(tk), i) for i, tk in enumerate(g["tokens"][:6])])
        if np.abs(mine - ref).max() > 1e-5 * np.abs(ref).max():
            fails.append(f"fp64 forward {name}")
    rg = np.random.default_rng(5)
    x = (rg.standard_normal(512) * 5).astype(np.float32)
    if np.abs(O.silu(x) - x / (1 + np.exp(-x.astype(np.float64)))).max() > 1e-5:
        fails.append("silu fp64")
    return fails


def test_forward_pins_pass_on_faithful_oracle(O, W):
    assert forward_pin_failures(O, W) == []


@pytest.mark.parametrize("mode,name", [(10, "silu sign"), (11, "silu on the up projection"),
                                       (12, "no attention residual")])
def test_forward_planted_mistakes_are_caught(O, W, faulty_oracle, mode, name):
    faulty_oracle(mode)
    assert forward_pin_failures(O, W), f"planted mistake '{name}' passed every pin"
