import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP C ABI)")
    config.addinivalue_line("markers", "slow: long CPU-side work")


@pytest.fixture(scope="session")
def oracle():
    from oracle.oracle import Oracle
    return Oracle()


@pytest.fixture(scope="session")
def reference():
    from oracle.oracle import Reference
    return Reference()


@pytest.fixture(scope="session")
def ctx():
    from fortai_amd import backend
    c = backend.Context(0)
    yield c
    c.close()


@pytest.fixture(scope="session")
def tiny_model_path(tmp_path_factory):
    from fortai_amd import synth
    path = str(tmp_path_factory.mktemp("models") / "tiny.gguf")
    synth.write_model(path, synth.CONFIGS["qwen35-tiny"])
    return path
