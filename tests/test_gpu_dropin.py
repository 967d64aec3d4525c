"""The reference's own programs running on the drop-in.  These are its
`engine` (main.cpp: prompt, greedy generation, text out) and its `benchmark`
(benchmark.cpp: run_trial's prefill and decode loops), built from its
sources: as they are by oracle/dropin.py (*_ref, in oracle/_ref), and on
the drop-in by tinyllama-engine_amd/host/dropin.py (*_dropin, in
tinyllama-engine_amd/_dropin).  In the *_dropin builds, run_state.h is
this repository's, the block of src/forward.cpp:192-208 is
tla_host::attention_block, and the RoPE, KV-cache append and attention of
every token and layer run on the GPU.  In the *_ref builds everything is the
reference's, on the CPU.  Both read one seeded GGUF model (2 layers, 4 / 2
heads, Q8_0, a byte-level vocabulary) written by the package's gguf_writer.

Greedy generation must print the same text, token for token (the default
prompt is 115 tokens, then 24 are generated): attention on the GPU is within
1e-6 of the CPU's, and no generated token may flip.  The benchmark must
count the same prompt and decode tokens."""
import os
import subprocess

import pytest

from conftest import ROOT
from helpers import log

pytestmark = pytest.mark.gpu

REF_DIR = os.path.join(ROOT, "oracle", "_ref")
DROPIN_DIR = os.path.join(ROOT, "tinyllama-engine_amd", "_dropin")
PROGS = {n: os.path.join(DROPIN_DIR if n.endswith("_dropin") else REF_DIR, n)
         for n in ("engine_ref", "engine_dropin", "benchmark_ref", "benchmark_dropin")}
needs_programs = pytest.mark.skipif(
    not all(os.access(p, os.X_OK) for p in PROGS.values()),
    reason="oracle/_ref programs not built (building them needs the reference's sources)")


@pytest.fixture(scope="module")
def model_path(tmp_path_factory, W):
    from importlib import import_module
    gw = import_module("tinyllama-engine_amd.gguf_writer")
    byte_vocab, write_gguf = gw.byte_vocab, gw.write_gguf
    spec = W.ModelSpec(2, 256, 4, 2, 512, 384, 256)
    path = str(tmp_path_factory.mktemp("dropin") / "model.gguf")
    write_gguf(path, spec, W.make_model(spec, W.W_Q8_0, salt=44), vocab=byte_vocab(spec.n_vocab))
    return path


def run(prog, args):
    cmd = [PROGS[prog]] + args
    log(f"  running {prog} {' '.join(args[1:])}")
    r = subprocess.run(cmd, capture_output=True, timeout=120)
    assert r.returncode == 0, (prog, r.returncode, r.stderr[-2000:])
    return r.stdout


@needs_programs
@pytest.mark.parametrize("prompt", [None, "Tell me about GPUs and their memory."])
def test_reference_engine_generates_the_same_text_on_the_dropin(model_path, prompt):
    args = [model_path, "--temperature", "0", "--max_tokens", "24"]
    if prompt:
        args += ["--prompt", prompt]
    want = run("engine_ref", args)
    got = run("engine_dropin", args)
    text = want.split(b"Generating...\n\n", 1)[1]
    log(f"    generated: {text[:80]!r}")
    assert len(text.strip()) > 0
    assert got == want


@needs_programs
def test_reference_benchmark_runs_on_the_dropin(model_path):
    args = [model_path, "--trials", "2", "--warmup", "1", "--decode-tokens", "8", "--csv"]
    want = run("benchmark_ref", args).decode().strip().split(",")
    got = run("benchmark_dropin", args).decode().strip().split(",")
    log(f"    reference: {want}")
    log(f"    drop-in:   {got}")
    # label, backend, threads, quant, prompt tokens, decode tokens, then timings
    assert got[:6] == want[:6]
    assert int(got[4]) > 100 and int(got[5]) == 8
