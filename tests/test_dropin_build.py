"""The C++ drop-in, shown against the reference's own call sites: the
reference's unmodified main.cpp, benchmark.cpp, generate.cpp, gguf_model.cpp,
tokenizer.cpp and ops.cpp, plus forward.cpp with the one documented edit
(src/forward.cpp:192-208: rope() + attention() -> tla_host::attention_block),
compile and link against this repository's run_state.h (in place of
src/run_state.h), libtla_host.so and libtla.so, into the two binaries of the
reference's Makefile (Makefile:4-14).  A compile-and-link check only: the
sources are copied from /root/reference into a temporary directory at test
time (nothing of the reference is kept), and the test is skipped where the
reference is absent."""
import os
import re
import shutil
import subprocess

import pytest

from conftest import ROOT

REF_SRC = "/root/reference/src"
PKG = os.path.join(ROOT, "tinyllama-engine_amd")

pytestmark = pytest.mark.skipif(not os.path.isdir(REF_SRC), reason="no reference sources here")

# Makefile:4-8
ENGINE = ["main.cpp", "gguf_model.cpp", "forward.cpp", "generate.cpp", "tokenizer.cpp", "ops.cpp"]
BENCHMARK = ["benchmark.cpp", "gguf_model.cpp", "forward.cpp", "tokenizer.cpp", "ops.cpp"]

BLOCK = re.compile(r"rope\(state\.q, state\.k, pos,.*?l, pos, cfg\);", re.S)


def dropin_tree(dst):
    src = os.path.join(dst, "src")
    os.makedirs(src)
    for name in os.listdir(REF_SRC):
        if name.endswith((".cpp", ".h")):
            shutil.copy(os.path.join(REF_SRC, name), src)
    shutil.copy(os.path.join(PKG, "host", "run_state.h"), os.path.join(src, "run_state.h"))
    fwd = os.path.join(src, "forward.cpp")
    text = open(fwd).read()
    text, n = BLOCK.subn("tla_host::attention_block(state, l, pos);", text)
    assert n == 1, "the rope() + attention() block of forward() was not found"
    open(fwd, "w").write(text)
    return src


def build(src, sources, out):
    cmd = (["g++", "-std=c++20", "-O2", "-Wall", "-Wextra", "-pthread"]
           + [os.path.join(src, s) for s in sources]
           + [f"-I{src}", f"-I{os.path.join(ROOT, 'include')}", f"-I{os.path.join(PKG, 'host')}",
              f"-L{PKG}", "-ltla_host", "-ltla", f"-Wl,-rpath,{PKG}",
              "-Wl,-rpath-link,/opt/rocm/lib", "-o", out])
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-4000:]
    return r


def test_reference_engine_and_benchmark_build_against_the_dropin(tmp_path):
    src = dropin_tree(str(tmp_path))
    for sources, name in ((ENGINE, "engine"), (BENCHMARK, "benchmark")):
        out = os.path.join(str(tmp_path), name)
        build(src, sources, out)
        syms = subprocess.run(["nm", "-C", "--undefined-only", out], capture_output=True,
                              text=True).stdout
        # the block runs through the drop-in, and RunState comes from it
        assert "tla_host::attention_block(RunState&, int, int)" in syms
        assert "tla_host::detail::allocate_state(RunState&" in syms


def test_dropin_changes_only_run_state_and_forward(tmp_path):
    """The drop-in needs no other change to the reference: the built tree
    differs from the reference's sources in run_state.h (replaced) and
    forward.cpp (the one block) alone."""
    src = dropin_tree(str(tmp_path))
    changed = []
    for name in sorted(os.listdir(src)):
        a = open(os.path.join(src, name), "rb").read()
        b = open(os.path.join(REF_SRC, name), "rb").read()
        if a != b:
            changed.append(name)
    assert changed == ["forward.cpp", "run_state.h"]
