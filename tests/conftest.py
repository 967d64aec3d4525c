import importlib
import os
import sys

import numpy as np
import pytest

ROOT = os.path.abspath(os.path.join(os.path.dirname(__file__), ".."))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP path through the C ABI)")


def tla_module():
    return importlib.import_module("tinyllama-engine_amd")


def workloads_module():
    return importlib.import_module("tinyllama-engine_amd.workloads")


def golden(name):
    return np.load(os.path.join(GOLDEN, name), allow_pickle=False)


@pytest.fixture(scope="session")
def tla():
    return tla_module()


@pytest.fixture(scope="session")
def W():
    return workloads_module()


@pytest.fixture(scope="session")
def O():
    import oracle
    oracle.oracle()  # builds liboracle.so if needed
    return oracle


@pytest.fixture
def faulty_oracle(O):
    """Yields a setter for the oracle's planted-mistake mode; always resets."""
    lib = O.oracle()
    yield lib.oracle_fault
    lib.oracle_fault(0)


@pytest.fixture(scope="session")
def engines(tla):
    """Cache of GPU engines keyed by (n_layers, n_ctx, n_head, n_head_kv);
    closed at session end.  Heads default to TinyLlama's 32 / 4 (head_dim 64)."""
    made = {}

    def get(n_layers, n_ctx, n_head=32, n_head_kv=4):
        key = (n_layers, n_ctx, n_head, n_head_kv)
        if key not in made:
            cfg = tla.Config(n_layers, n_head * 64, n_head, n_head_kv, n_ctx, 10000.0)
            made[key] = tla.Engine(cfg)
        return made[key]

    yield get
    for e in made.values():
        e.close()
