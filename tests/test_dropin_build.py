"""The C++ drop-in, shown against the reference's own call sites: the
reference's unmodified main.cpp, benchmark.cpp, generate.cpp, gguf_model.cpp,
tokenizer.cpp and ops.cpp, plus forward.cpp with the one documented edit
(src/forward.cpp:192-208: rope() + attention() -> tla_host::attention_block),
compile and link against this repository's run_state.h (in place of
src/run_state.h), libtla_host.so and libtla.so, into the two binaries of the
reference's Makefile (Makefile:4-14).  A compile-and-link check only (the GPU
test test_gpu_dropin.py runs them): the sources are copied from
/root/reference into a temporary directory at test time (nothing of the
reference is kept), and the test is skipped where the reference is absent."""
import os
import subprocess

import pytest

from oracle import dropin as ref_programs

dropin = ref_programs.PACKAGE_DROPIN  # tinyllama-engine_amd/host/dropin.py
REF_SRC = ref_programs.REF_SRC
pytestmark = pytest.mark.skipif(not os.path.isdir(REF_SRC), reason="no reference sources here")


def test_reference_engine_and_benchmark_build_against_the_dropin(tmp_path):
    src = dropin.dropin_tree(REF_SRC, str(tmp_path))
    for sources, name in dropin.PROGRAMS:
        out = os.path.join(str(tmp_path), name)
        dropin.build_dropin(src, sources, out)
        syms = subprocess.run(["nm", "-C", "--undefined-only", out], capture_output=True,
                              text=True).stdout
        # the block runs through the drop-in, and RunState comes from it
        assert "tla_host::attention_block(RunState&, int, int)" in syms
        assert "tla_host::detail::allocate_state(RunState&" in syms


def test_dropin_changes_only_run_state_and_forward(tmp_path):
    """The drop-in needs no other change to the reference: the built tree
    differs from the reference's sources in run_state.h (replaced) and
    forward.cpp (the one block) alone."""
    src = dropin.dropin_tree(REF_SRC, str(tmp_path))
    changed = []
    for name in sorted(os.listdir(src)):
        a = open(os.path.join(src, name), "rb").read()
        b = open(os.path.join(REF_SRC, name), "rb").read()
        if a != b:
            changed.append(name)
    assert changed == ["forward.cpp", "run_state.h"]
