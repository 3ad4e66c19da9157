import os
import sys
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "tests"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (MI355X / gfx950)")
    config.addinivalue_line("markers", "slow: long-running parity case")


def model_root() -> str:
    d = os.environ.get("TMG_MODEL_DIR") or os.path.join(tempfile.gettempdir(), "tmg_models")
    os.makedirs(d, exist_ok=True)
    return d


@pytest.fixture(scope="session")
def tiny_path():
    from tinyminigo_amd import workloads as W
    return W.ensure_model(W.TINY, model_root())


@pytest.fixture(scope="session")
def oracle_mod():
    from oracle import oracle as O
    return O

