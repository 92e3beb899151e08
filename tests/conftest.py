"""Shared fixtures.  Tests marked ``gpu`` need a visible MI355X and fail (not
skip) without one; everything else runs on the CPU."""
import importlib
import importlib.util
import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if REPO not in sys.path:
    sys.path.insert(0, REPO)
TESTS = os.path.dirname(os.path.abspath(__file__))
if TESTS not in sys.path:
    sys.path.insert(0, TESTS)

PKG_NAME = "qwen3-runtime-byyourself_amd"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a real MI355X (gfx950) GPU")


def pytest_sessionfinish(session, exitstatus):
    """Write the GPU parity statistics when Q3K_PARITY_REPORT names a file."""
    try:
        import gpu_util
    except ImportError:
        return
    gpu_util.write_report()


def _load_oracle():
    path = os.path.join(REPO, "oracle", "q3k_oracle.py")
    spec = importlib.util.spec_from_file_location("q3k_oracle", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


@pytest.fixture(scope="session")
def q3k():
    return importlib.import_module(PKG_NAME)


@pytest.fixture(scope="session")
def synth():
    return importlib.import_module(PKG_NAME + ".synth")


@pytest.fixture(scope="session")
def configs():
    return importlib.import_module(PKG_NAME + ".configs")


@pytest.fixture(scope="session")
def oracle():
    return _load_oracle()


@pytest.fixture(scope="session")
def hip(q3k):
    mod = importlib.import_module(PKG_NAME + ".hip")
    if not mod.available():
        pytest.fail("no visible GPU: tests marked gpu need an MI355X")
    return mod
