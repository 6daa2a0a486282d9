import os
import sys

import numpy as np
import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(REPO, "nemo-c_amd"), os.path.join(REPO, "oracle")):
    if p not in sys.path:
        sys.path.insert(0, p)

MODEL_CACHE = os.environ.get("NEMO_MODEL_CACHE", "/tmp/nemo_models")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")
    config.addinivalue_line("markers", "slow: full-size model on the CPU oracle")


def model_dir(kind: str, seed: int = 0, blank_bias: float = 0.0) -> str:
    import synth

    dims = synth.TINY_DIMS if kind == "tiny" else synth.FULL_DIMS
    d = os.path.join(MODEL_CACHE, f"{kind}_s{seed}_b{blank_bias:g}")
    synth.write_model(d, dims, seed, blank_bias)
    return d


@pytest.fixture(scope="session")
def tiny_model_dir():
    return model_dir("tiny")


@pytest.fixture(scope="session")
def full_model_dir():
    return model_dir("full")


@pytest.fixture(scope="session")
def tiny_oracle(tiny_model_dir):
    import oracle

    return oracle.Model(tiny_model_dir, "en-US")


@pytest.fixture(scope="session")
def gpu():
    import nemoasr

    g = nemoasr.Gpu()
    yield g
    g.close()


def rel_err(a: np.ndarray, b: np.ndarray) -> float:
    """max |a - b| / max |b| (the reference's encoder gate, tools/compare.py:30-32)."""
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    den = max(float(np.max(np.abs(b))) if b.size else 0.0, 1e-30)
    return float(np.max(np.abs(a - b))) / den if b.size else 0.0
