"""The reference's own programs built on the drop-in attention path.

The drop-in is two changes to the reference's src/ tree and a link line
(INTEGRATION.md shows them as a maintainer would apply them):
  * src/run_state.h is replaced by this directory's run_state.h (the same
    global RunState, KV cache on the device);
  * the rope() + attention() block of forward() (src/forward.cpp:192-208)
    becomes tla_host::attention_block(state, l, pos);
  * the programs link libtla_host.so and libtla.so (Makefile:1-14 plus the
    libraries).

`python3 dropin.py SRC OUT_DIR` copies the reference's src/*.cpp, *.h from
SRC into a temporary directory outside the repository, applies the two
changes there, compiles the reference's `engine` and `benchmark` targets
(Makefile:4-14) into OUT_DIR as engine_dropin and benchmark_dropin, and
deletes the copy: only the two programs are kept (git-ignored)."""
import os
import re
import shutil
import subprocess
import sys
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.dirname(HERE)
ROOT = os.path.dirname(PKG)

# the reference's Makefile:4-8
ENGINE = ["main.cpp", "gguf_model.cpp", "forward.cpp", "generate.cpp", "tokenizer.cpp", "ops.cpp"]
BENCHMARK = ["benchmark.cpp", "gguf_model.cpp", "forward.cpp", "tokenizer.cpp", "ops.cpp"]
PROGRAMS = ((ENGINE, "engine"), (BENCHMARK, "benchmark"))

# the block of forward() that the drop-in replaces (src/forward.cpp:192-208)
BLOCK = re.compile(r"rope\(state\.q, state\.k, pos,.*?l, pos, cfg\);", re.S)
CALL = "tla_host::attention_block(state, l, pos);"

CXX = os.environ.get("DROPIN_CXX", "g++")
CXXFLAGS = ["-std=c++20", "-O2", "-Wall", "-Wextra", "-pthread"]


def dropin_tree(ref_src: str, dst: str) -> str:
    """Copy the reference's src/*.cpp, *.h from ref_src into dst/src with the
    two changes; returns that directory."""
    src = os.path.join(dst, "src")
    os.makedirs(src)
    for name in os.listdir(ref_src):
        if name.endswith((".cpp", ".h")):
            shutil.copy(os.path.join(ref_src, name), src)
    shutil.copy(os.path.join(HERE, "run_state.h"), os.path.join(src, "run_state.h"))
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
           + [f"-I{src}", f"-I{os.path.join(ROOT, 'include')}", f"-I{HERE}",
              f"-L{PKG}", "-ltla_host", "-ltla", f"-Wl,-rpath,{rpath or PKG}",
              "-Wl,-rpath-link,/opt/rocm/lib", "-o", out])
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"building {os.path.basename(out)} failed:\n{r.stderr[-4000:]}")


def main(ref_src: str, out_dir: str) -> None:
    os.makedirs(out_dir, exist_ok=True)
    # the libraries sit in the package directory; found relative to the programs
    rel = os.path.relpath(PKG, os.path.abspath(out_dir))
    with tempfile.TemporaryDirectory(prefix="tla_dropin_") as tmp:
        src = dropin_tree(ref_src, tmp)
        for sources, name in PROGRAMS:
            build_dropin(src, sources, os.path.join(out_dir, name + "_dropin"), rpath=f"$ORIGIN/{rel}")


if __name__ == "__main__":
    if len(sys.argv) != 3:
        sys.exit("usage: dropin.py REFERENCE_SRC OUT_DIR")
    main(sys.argv[1], sys.argv[2])
