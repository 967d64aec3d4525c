"""GPU parity of the stand-alone ops through the C ABI: rope (bit-exact),
softmax, device copy, and the C++ host side (its own test program)."""
import os
import subprocess

import numpy as np
import pytest

from conftest import ROOT, golden
from helpers import bits, device_arrays, log, max_err

pytestmark = pytest.mark.gpu


def test_rope_bitexact_against_reference_golden(engines):
    g = golden("rope.npz")
    eng = engines(1, 64)
    with device_arrays() as track:
        q, k = track(eng.array((2048,))), track(eng.array((256,)))
        for i, p in enumerate(g["positions"]):
            q.upload(g["q"])
            k.upload(g["k"])
            eng.rope(q.ptr, k.ptr, int(p))
            assert np.array_equal(bits(q.download()), bits(g["q_out"][i])), f"q at {p}"
            assert np.array_equal(bits(k.download()), bits(g["k_out"][i])), f"k at {p}"
        q.upload(g["manual_q"])
        k.upload(np.zeros(256, np.float32))
        eng.rope(q.ptr, k.ptr, 1)
        assert np.array_equal(bits(q.download()), bits(g["manual_q_out"]))


def test_rope_bitexact_against_oracle_random(O, engines):
    eng = engines(1, 64)
    rg = np.random.default_rng(21)
    s = O.Shape()
    with device_arrays() as track:
        q, k = track(eng.array((2048,))), track(eng.array((256,)))
        for p in [int(x) for x in rg.integers(0, 1 << 20, 40)] + [65535, 1 << 24]:
            hq = (rg.standard_normal(2048) * 5).astype(np.float32)
            hk = (rg.standard_normal(256) * 5).astype(np.float32)
            q.upload(hq)
            k.upload(hk)
            eng.rope(q.ptr, k.ptr, p)
            eq, ek = O.rope(hq, hk, p, s)
            assert np.array_equal(bits(q.download()), bits(eq)), p
            assert np.array_equal(bits(k.download()), bits(ek)), p


def test_rope_other_shapes(O, engines):
    """rope() takes its shape per call (src/ops.h:175-176): other head_dim,
    head counts and base."""
    eng = engines(1, 64)
    rg = np.random.default_rng(22)
    for hd, nh, nkv, base in ((128, 8, 2, 500000.0), (32, 4, 4, 10000.0), (2, 1, 0, 10.0)):
        s = O.Shape(n_head=nh, n_head_kv=max(nkv, 1), head_dim=hd, freq_base=base)
        hq = rg.standard_normal(nh * hd).astype(np.float32)
        hk = rg.standard_normal(max(nkv, 1) * hd).astype(np.float32)
        eq, ek = O.rope(hq, hk, 777, O.Shape(n_head=nh, n_head_kv=nkv, head_dim=hd,
                                             freq_base=base))
        with device_arrays() as track:
            q, k = track(eng.array(hq)), track(eng.array(hk))
            eng.rope(q.ptr, k.ptr, 777, hd, nh, nkv, base)
            assert np.array_equal(bits(q.download()), bits(eq))
            assert np.array_equal(bits(k.download()), bits(ek))
        del s


def test_softmax_against_reference_golden(engines):
    g = golden("softmax.npz")
    eng = engines(1, 64)
    for name in [n[3:] for n in g.files if n.startswith("in_")]:
        x = g["in_" + name]
        with device_arrays() as track:
            d = track(eng.array(x))
            eng.softmax(d.ptr, x.size)
            y = d.download()
        assert max_err(y, g["out_" + name]) <= 1e-6, name
        assert abs(float(y.astype(np.float64).sum()) - 1.0) < 1e-5, name
    with device_arrays() as track:  # src/test_ops.cpp:152-160
        d = track(eng.array(np.array([1000, 1000, 999], np.float32)))
        eng.softmax(d.ptr, 3)
        assert np.all(np.isfinite(d.download()))


def test_softmax_long_vectors(O, engines):
    """Long vectors (vocabulary-sized): the reference sums exp() sequentially
    in fp32 (src/ops.cpp:1080-1084), whose own error grows with n, so the GPU
    is held to 1e-6 of fp64 and to 1e-6 plus the reference's error of it."""
    eng = engines(1, 64)
    rg = np.random.default_rng(23)
    for n in (1, 1023, 1024, 1025, 32000, 100003):
        x = (rg.standard_normal(n) * 6).astype(np.float32)
        with device_arrays() as track:
            d = track(eng.array(x))
            eng.softmax(d.ptr, n)
            y = d.download()
        f64 = np.exp(x.astype(np.float64) - x.max())
        f64 /= f64.sum()
        ref = O.softmax(x)
        e_gpu, e_ref = np.abs(y - f64), np.abs(ref - f64)
        log(f"  softmax n={n}: GPU vs fp64 {e_gpu.max():.2e}, reference vs fp64 {e_ref.max():.2e}")
        assert e_gpu.max() <= 1e-6
        assert np.all(np.abs(y.astype(np.float64) - ref) <= 1e-6 + e_ref)


def test_device_copy_any_size_and_alignment(tla, engines):
    eng = engines(1, 64)
    rg = np.random.default_rng(24)
    src_host = rg.integers(0, 256, 1 << 20, dtype=np.uint8)
    with device_arrays() as track:
        src = track(tla.DeviceArray(eng, (1 << 20,), np.uint8)).upload(src_host)
        dst = track(tla.DeviceArray(eng, (1 << 20,), np.uint8))
        for off_s, off_d, n in ((0, 0, 1 << 20), (0, 0, 1000), (3, 5, 777), (16, 32, 65536 + 7),
                                (1, 0, 0)):
            dst.upload(np.zeros(1 << 20, np.uint8))
            eng.copy(dst.at(off_d), src.at(off_s), n)
            got = dst.download()
            assert np.array_equal(got[off_d:off_d + n], src_host[off_s:off_s + n])
            assert not got[:off_d].any() and not got[off_d + n:].any()


def test_cpp_host_side_program():
    """tests/cpp/test_host_block (built by build()): the reference's attention
    and rope test cases, RunState + attention_block vs the oracle, and the
    std::runtime_error convention."""
    exe = os.path.join(ROOT, "tests", "cpp", "test_host_block")
    assert os.path.exists(exe), "build() did not produce tests/cpp/test_host_block"
    r = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    log(r.stdout[-3000:])
    assert r.returncode == 0, r.stdout + r.stderr
    assert " 0 failed" in r.stdout


def test_mfma_floor_runs_and_leaves_the_sink(tla, engines):
    """The fp32 MFMA floor hook: runs a few grids and round counts, never
    writes its sink for its own operands, and validates its arguments before
    launching."""
    eng = engines(1, 64)
    with device_arrays() as track:
        sink = track(eng.array(np.full(1024, 7.0, np.float32)))
        for grid, iters in ((1, 1), (768, 3), (1024, 1)):
            eng.mfma_floor(grid, iters, sink.ptr)
        eng.synchronize()
        assert np.all(sink.download() == 7.0)
        for grid, iters, ptr in ((0, 1, sink.ptr), (4, 0, sink.ptr), (4, 1, 0)):
            with pytest.raises(tla.TlaError) as e:
                eng.mfma_floor(grid, iters, ptr)
            assert e.value.code == tla.TLA_ERR_INVALID_ARGUMENT


def test_read_floor_reads_and_leaves_the_sink(tla, engines):
    """The streaming-read hook: every load form and depth runs over an odd
    byte count with grids whose chunks end mid-round (777 workgroups: 1.3
    rounds of 256 loads per thread; 3: many full rounds and a remainder),
    never writes its sink for ordinary data, and validates its arguments
    before launching."""
    eng = engines(1, 64)
    with device_arrays() as track:
        src = track(eng.array(np.arange(1 << 20, dtype=np.float32)))
        sink = track(eng.array(np.full(777, 7.0, np.float32)))
        for kind in (tla.READ_GLOBAL, tla.READ_GLOBAL_NT, tla.READ_BUFFER, tla.READ_BUFFER_NT):
            for depth in (8, 16, 32):
                for grid in (777, 3):
                    eng.read_floor(src.ptr, (1 << 22) - 48, grid, sink.ptr, kind, depth)
        eng.synchronize()
        assert np.all(sink.download() == 7.0)
        for nbytes, grid, kind, depth in ((15, 4, 0, 8), (1 << 22, 0, 0, 8), (40, 4, 0, 8),
                                          (1 << 22, 4, 4, 8), (1 << 22, 4, -1, 8), (1 << 22, 4, 2, 12)):
            with pytest.raises(tla.TlaError) as e:
                eng.read_floor(src.ptr, nbytes, grid, sink.ptr, kind, depth)
            assert e.value.code == tla.TLA_ERR_INVALID_ARGUMENT
