"""The reference engine with this repository's drop-in attention path.

TEST INFRASTRUCTURE ONLY (with the rest of oracle/): it builds, from the
reference's own sources, the programs the tests run to show the drop-in at
work, and nothing under tinyllama-engine_amd/ uses it.

The drop-in is two changes to the reference's src/ tree and a link line:
  * src/run_state.h is replaced by tinyllama-engine_amd/host/run_state.h
    (the same global RunState, KV cache on the device);
  * the rope() + attention() block of forward() (src/forward.cpp:192-208)
    becomes tla_host::attention_block(state, l, pos);
  * the programs link libtla_host.so and libtla.so (Makefile:1-14 plus the
    libraries).

`python3 oracle/dropin.py OUT_DIR` builds into OUT_DIR (oracle/_ref):
  engine_ref, benchmark_ref          the reference's `engine` and `benchmark`
                                     targets (Makefile:4-14) compiled from
                                     its sources where they lie;
  engine_dropin, benchmark_dropin    the same targets with the two changes,
                                     compiled in a temporary copy of src/
                                     outside the repository, deleted after.
Only the programs land in OUT_DIR (git-ignored)."""
import os
import re
import shutil
import subprocess
import sys
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
PKG = os.path.join(ROOT, "tinyllama-engine_amd")
REF_SRC = "/root/reference/src"

# the reference's Makefile:4-8
ENGINE = ["main.cpp", "gguf_model.cpp", "forward.cpp", "generate.cpp", "tokenizer.cpp", "ops.cpp"]
BENCHMARK = ["benchmark.cpp", "gguf_model.cpp", "forward.cpp", "tokenizer.cpp", "ops.cpp"]

# the block of forward() that the drop-in replaces (src/forward.cpp:192-208)
BLOCK = re.compile(r"rope\(state\.q, state\.k, pos,.*?l, pos, cfg\);", re.S)
CALL = "tla_host::attention_block(state, l, pos);"

CXX = os.environ.get("DROPIN_CXX", "g++")
CXXFLAGS = ["-std=c++20", "-O2", "-Wall", "-Wextra", "-pthread"]


def dropin_tree(dst: str) -> str:
    """Copy the reference's src/*.cpp, *.h into dst/src with the two
    changes; returns that directory."""
    src = os.path.join(dst, "src")
    os.makedirs(src)
    for name in os.listdir(REF_SRC):
        if name.endswith((".cpp", ".h")):
            shutil.copy(os.path.join(REF_SRC, name), src)
    shutil.copy(os.path.join(PKG, "host", "run_state.h"), os.path.join(src, "run_state.h"))
    fwd = os.path.join(src, "forward.cpp")
    with open(fwd) as f:
        text = f.read()
    text, n = BLOCK.subn(CALL, text)
    if n != 1:
        raise RuntimeError("the rope() + attention() block of forward() was not found")
    with open(fwd, "w") as f:
        f.write(text)
    return src


def build_dropin(src: str, sources, out: str, rpath: str = None) -> None:
    """Compile and link one program of the drop-in tree against the libraries."""
    cmd = ([CXX] + CXXFLAGS + [os.path.join(src, s) for s in sources]
           + [f"-I{src}", f"-I{os.path.join(ROOT, 'include')}", f"-I{os.path.join(PKG, 'host')}",
              f"-L{PKG}", "-ltla_host", "-ltla", f"-Wl,-rpath,{rpath or PKG}",
              "-Wl,-rpath-link,/opt/rocm/lib", "-o", out])
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"building {os.path.basename(out)} failed:\n{r.stderr[-4000:]}")


def build_reference(sources, out: str) -> None:
    """Compile one of the reference's programs from its sources where they lie."""
    cmd = [CXX] + CXXFLAGS + [os.path.join(REF_SRC, s) for s in sources] + [f"-I{REF_SRC}", "-o", out]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"building {os.path.basename(out)} failed:\n{r.stderr[-4000:]}")


def main(out_dir: str) -> None:
    os.makedirs(out_dir, exist_ok=True)
    for sources, name in ((ENGINE, "engine"), (BENCHMARK, "benchmark")):
        build_reference(sources, os.path.join(out_dir, name + "_ref"))
    # the libraries sit at ../../tinyllama-engine_amd from OUT_DIR = oracle/_ref
    rel = os.path.relpath(PKG, os.path.abspath(out_dir))
    with tempfile.TemporaryDirectory(prefix="tla_dropin_") as tmp:
        src = dropin_tree(tmp)
        for sources, name in ((ENGINE, "engine"), (BENCHMARK, "benchmark")):
            build_dropin(src, sources, os.path.join(out_dir, name + "_dropin"),
                         rpath=f"$ORIGIN/{rel}")


if __name__ == "__main__":
    if len(sys.argv) != 2:
        sys.exit("usage: dropin.py OUT_DIR")
    main(sys.argv[1])
