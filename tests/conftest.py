"""Shared fixtures.  GPU tests are marked `gpu` and call the HIP library through its C ABI; the
oracle (oracle/, CPU) is only ever the checker."""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "kokoro-rust_amd"))
sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built HIP library")


@pytest.fixture(scope="session")
def weights():
    from kokoro_hip import model_spec
    return model_spec.random_weights(seed=0)


@pytest.fixture(scope="session")
def oracle_model(weights):
    from oracle import oracle as O
    return O.Model(weights)


@pytest.fixture(scope="session")
def gpu_ctx(weights):
    from kokoro_hip import api
    ctx = api.Context(0)
    ctx.upload_model(weights)
    yield ctx
    ctx.close()


def snr_db(ref, x):
    ref = np.asarray(ref, np.float64)
    e = ref - np.asarray(x, np.float64)
    return float(10 * np.log10((ref ** 2).sum() / max((e ** 2).sum(), 1e-300)))
