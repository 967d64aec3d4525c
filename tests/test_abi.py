"""CPU tests of the C ABI: the library loads, exports every symbol
include/*.h declares, and rejects bad arguments with a status code and a
message before touching the device (the reference's ops never validate;
callers got undefined behaviour for pos >= n_ctx, src/ops.cpp:1350-1353)."""
import ctypes as C
import glob
import os
import re

import numpy as np
import pytest

from conftest import ROOT


def declared_functions():
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names |= set(re.findall(r"\b(tla_[a-z0-9_]+)\s*\(", text))
    return names


def test_header_declares_the_reference_interfaces():
    names = declared_functions()
    for required in ("tla_rope", "tla_softmax", "tla_attention", "tla_rope_attention",
                     "tla_decode", "tla_prefill", "tla_kv_cache_alloc", "tla_engine_create",
                     "tla_last_error"):
        assert required in names


def test_library_exports_every_declared_symbol(tla):
    lib = tla.lib()
    missing = [n for n in sorted(declared_functions()) if not hasattr(lib, n)]
    assert not missing, missing
    assert set(tla.SIGNATURES) == declared_functions()
    assert lib.tla_abi_version() == 2


def test_host_library_loads(tla):
    assert os.path.exists(tla.HOST_LIB_PATH)
    C.CDLL(tla.HOST_LIB_PATH)


def test_engine_create_validates_before_device(tla):
    lib = tla.lib()
    out = C.c_void_p()
    assert lib.tla_engine_create(None, 0, C.byref(out)) == tla.TLA_ERR_INVALID_ARGUMENT
    assert "NULL" in tla.last_error()
    bad = [
        (tla.Config(22, 2048, 32, 3, 2048, 1e4), tla.TLA_ERR_INVALID_ARGUMENT),  # 32 % 3
        (tla.Config(22, 2000, 32, 4, 2048, 1e4), tla.TLA_ERR_INVALID_ARGUMENT),  # n_embd % n_head
        (tla.Config(22, 1024, 32, 4, 2048, 1e4), tla.TLA_ERR_UNSUPPORTED),       # head_dim 32
        (tla.Config(22, 2048, 32, 1, 2048, 1e4), tla.TLA_ERR_UNSUPPORTED),       # gqa 32 > 16
        (tla.Config(0, 2048, 32, 4, 2048, 1e4), tla.TLA_ERR_INVALID_ARGUMENT),
        (tla.Config(22, 2048, 32, 4, 0, 1e4), tla.TLA_ERR_INVALID_ARGUMENT),
        (tla.Config(22, 2048, 32, 4, 2048, 0.0), tla.TLA_ERR_INVALID_ARGUMENT),
        (tla.Config(22, 2048, 32, 4, 2048, float("inf")), tla.TLA_ERR_INVALID_ARGUMENT),
    ]
    for cfg, code in bad:
        assert lib.tla_engine_create(C.byref(cfg), 0, C.byref(out)) == code, tla.last_error()
        assert out.value is None
    assert lib.tla_engine_create(C.byref(tla.Config.tinyllama()), -1, C.byref(out)) == \
        tla.TLA_ERR_INVALID_ARGUMENT


def test_null_engine_is_rejected_everywhere(tla):
    lib = tla.lib()
    one = (C.c_int * 1)(0)
    calls = {
        "tla_synchronize": (None,),
        "tla_alloc": (None, 16, C.byref(C.c_void_p())),
        "tla_rope": (None, None, None, 0, 64, 32, 4, 1e4),
        "tla_softmax": (None, None, 4),
        "tla_attention": (None,) + (None,) * 7 + (0, 0),
        "tla_rope_attention": (None,) + (None,) * 6 + (0, 0),
        "tla_decode": (None, 1, one, 0, 1, 0) + (None,) * 6 + (0,),
        "tla_prefill": (None, 0, 1, 0, 1, 0) + (None,) * 6,
        "tla_set_option": (None, 0, 0),
        "tla_event_record": (None, 0),
        "tla_profile_enable": (None, 1),
    }
    for name, args in calls.items():
        assert getattr(lib, name)(*args) == tla.TLA_ERR_INVALID_ARGUMENT, name
        assert tla.last_error() == "engine is NULL"
    assert lib.tla_engine_destroy(None) == tla.TLA_OK


def test_python_binding_fails_loudly_without_library(tla, tmp_path, monkeypatch):
    monkeypatch.setattr(tla, "LIB_PATH", str(tmp_path / "missing.so"))
    monkeypatch.setattr(tla, "_lib", None)
    with pytest.raises(FileNotFoundError):
        tla.lib()


def test_work_counts_match_the_stated_definitions(W):
    # 2*L*Hkv*d*4 + 2*H*d*4 + 4*Hkv*d*4 = 2048 L + 20480
    assert W.decode_bytes(128) == 282_624
    assert W.decode_bytes(2048) * 22 == 92_725_248
    assert W.decode_bytes(16384) * 8 * 22 == 5_909_184_512
    # 2*H*d*S(S+1)
    assert W.prefill_flops(512) == 1_075_838_976
    assert W.prefill_flops(512) * 22 == 23_668_457_472
    # a continued prompt sees pos0 more keys per token
    assert W.prefill_flops(10, pos0=5) == W.prefill_flops(15) - W.prefill_flops(5)


def test_workload_generator_is_deterministic(W):
    a = W.decode_ragged(n_seq=4, n_layers=1, n_ctx=2048)
    b = W.decode_ragged(n_seq=4, n_layers=1, n_ctx=2048)
    assert W.digest(a.q, a.kc) == W.digest(b.q, b.kc)
    pos = W.ragged_positions(64)
    assert pos.min() >= 255 and pos.max() <= 2047
    c = W.decode_long(n_seq=1, n_layers=1, n_ctx=512)
    rows = c.kc[0, 0, :511].reshape(511, 4, 64)
    peaked = np.abs(rows).max(-1) > 4.0 * 0.5 * 2  # an x8 row of N(0, 0.25) stands out
    assert 0 < peaked.mean() < 0.05

