"""The committed rocprofv3 summaries that bench.py reads its measured HBM
traffic from: each names the build it measured (a digest of the kernel's
sources) and the commands that produced it, and bench.py uses the bytes only
for that build."""
import glob
import os
import re

import bench
from conftest import ROOT

PROFILES = sorted(glob.glob(os.path.join(ROOT, "profiles", "*__*.md")))


def test_traffic_profiles_record_their_build():
    seen = 0
    for path in PROFILES:
        text = open(path).read()
        if not re.search(r"^traffic_bytes_per_launch:", text, re.M):
            continue
        seen += 1
        kernel = os.path.basename(path).split("__")[0]
        assert kernel in bench.KERNEL_SOURCES, path
        assert re.search(r"^source_digest:\s*[0-9a-f]{16}\s*$", text, re.M), path
        assert "rocprofv3 --pmc FETCH_SIZE" in text and "rocprofv3 --pmc WRITE_SIZE" in text, path
    assert seen >= 4


def test_profiled_traffic_is_dropped_for_another_build(tmp_path, monkeypatch):
    kernel = "decode_split_kernel"
    prof = tmp_path / "profiles"
    prof.mkdir()
    good = bench.kernel_source_digest(kernel)
    (prof / f"{kernel}__w_ok.md").write_text(f"traffic_bytes_per_launch: 123\nsource_digest: {good}\n")
    (prof / f"{kernel}__w_old.md").write_text("traffic_bytes_per_launch: 123\nsource_digest: 0123456789abcdef\n")
    (prof / f"{kernel}__w_none.md").write_text("traffic_bytes_per_launch: 123\n")
    real = os.path.join(ROOT, "tinyllama-engine_amd")
    (tmp_path / "tinyllama-engine_amd").symlink_to(real)
    monkeypatch.setattr(bench, "ROOT", str(tmp_path))
    assert bench.profiled_traffic(kernel, "w_ok") == 123
    assert bench.profiled_traffic(kernel, "w_old") is None
    assert bench.profiled_traffic(kernel, "w_none") is None
    assert bench.profiled_traffic(kernel, "w_missing") is None
