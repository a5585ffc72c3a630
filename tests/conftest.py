import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "exact-integer-inference_amd")
for p in (PKG, ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")
    config.addinivalue_line("markers", "slow: long CPU check")


@pytest.fixture(scope="session")
def model_path():
    from eii import synth
    return synth.ensure_model("base")


@pytest.fixture(scope="session")
def stress_model_path():
    from eii import synth
    return synth.ensure_model("stress")


@pytest.fixture(scope="session")
def oracle(model_path):
    from oracle.intref_np import OracleModel
    return OracleModel(model_path)


@pytest.fixture(scope="session")
def engine(model_path):
    from eii.engine import Engine
    e = Engine(model_path)
    yield e
    e.close()
