import os
import sys

import numpy as np
import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (REPO, os.path.join(REPO, "cube-awq_amd"), os.path.join(REPO, "oracle")):
    if p not in sys.path:
        sys.path.insert(0, p)

GOLDEN = os.path.join(REPO, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a real MI355X (gfx950) GPU")


def load_golden(name):
    with np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.fixture(scope="session")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a GPU (deselect with -m 'not gpu')")
    import cube_awq
    cube_awq.lib()  # fail loudly if the HIP library is not built
    return torch.device("cuda:0")


@pytest.fixture(autouse=True)
def _tuning_overrides(monkeypatch):
    """The library reads its AWQ_* tuning overrides once per process
    (awq_tuning_reload() re-reads them): re-read them whenever a test sets
    one, and again once the test's environment has been restored."""
    real_setenv, real_delenv = monkeypatch.setenv, monkeypatch.delenv
    touched = []

    def reload():
        import cube_awq
        cube_awq.lib().awq_tuning_reload()

    def setenv(name, value, prepend=None):
        real_setenv(name, value, prepend)
        if name.startswith("AWQ_"):
            touched.append(name)
            reload()

    def delenv(name, raising=True):
        real_delenv(name, raising)
        if name.startswith("AWQ_"):
            touched.append(name)
            reload()

    monkeypatch.setenv, monkeypatch.delenv = setenv, delenv
    yield
    if touched:
        monkeypatch.undo()
        reload()
