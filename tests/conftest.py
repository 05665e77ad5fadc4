"""Shared pytest fixtures.

`-m "not gpu"` tests run anywhere (oracle vs golden vectors, host logic, the
C ABI's exports); `-m gpu` tests drive the HIP library on an MI355X and check
it against the CPU oracle.
"""
from __future__ import annotations

import importlib.util
import pathlib
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
TESTS = ROOT / "tests"
if str(TESTS) not in sys.path:
    sys.path.insert(0, str(TESTS))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def load_package():
    """Imports the package directory llama.rs_amd/ as module `llama_rs_amd`."""
    if "llama_rs_amd" in sys.modules:
        return sys.modules["llama_rs_amd"]
    pkg = ROOT / "llama.rs_amd"
    spec = importlib.util.spec_from_file_location(
        "llama_rs_amd", pkg / "__init__.py", submodule_search_locations=[str(pkg)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["llama_rs_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


@pytest.fixture(scope="session")
def llrs():
    return load_package()


@pytest.fixture(scope="session")
def oracle():
    from oracle_ffi import Oracle
    return Oracle()


@pytest.fixture(scope="session")
def backend(llrs):
    b = llrs.HipBackend(0)
    print(f"[backend] {b.name()} with {b.threads()} CUs", flush=True)
    return b
