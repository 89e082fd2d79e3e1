import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

FIXTURES = ROOT / "tests" / "golden" / "fixtures"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP C ABI)")


@pytest.fixture(scope="session")
def tensors():
    from hikoboshi_amd import weights

    return weights.load_tensors()


@pytest.fixture(scope="session")
def oracle(tensors):
    from oracle import Oracle

    return Oracle(tensors)


@pytest.fixture(scope="session")
def reference(tensors):
    from oracle import Reference

    if not Reference.available():
        pytest.skip("reference build oracle/_ref not present")
    return Reference(tensors)


@pytest.fixture(scope="session")
def gpu_ctx():
    from hikoboshi_amd import _lib, weights

    ctx = _lib.Context(weights.read_package_bytes(), device=0)
    yield ctx
    ctx.close()


def golden_cases():
    import json

    return [json.loads(p.read_text()) for p in sorted(FIXTURES.glob("*.golden.json"))]


def rng(seed=0):
    return np.random.default_rng(seed)
