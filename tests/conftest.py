"""Shared fixtures.  `gpu`-marked tests need a MI355X (run with -m gpu)."""
import importlib.util
import os
import sys

import numpy as np
import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(REPO, "oracle"))
GOLDEN = os.path.join(REPO, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD MI355X GPU (gfx950) and the built libmiq.so")


def load_miq():
    """Import the package directory `sycl-infer_amd` (not a valid module name) as `sycl_infer_amd`."""
    name = "sycl_infer_amd"
    if name in sys.modules:
        return sys.modules[name]
    spec = importlib.util.spec_from_file_location(name, os.path.join(REPO, "sycl-infer_amd", "__init__.py"))
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


@pytest.fixture(scope="session")
def miq():
    return load_miq()


@pytest.fixture(scope="session")
def oracle():
    from oracle import Oracle
    return Oracle()


@pytest.fixture(scope="session")
def ref():
    from oracle import Ref, REF_LIB
    if not os.path.exists(REF_LIB):
        pytest.skip("oracle/_ref/libsiref.so not built (needs the reference sources)")
    return Ref()


@pytest.fixture(scope="session")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


@pytest.fixture
def switch(miq):
    """switch(name, value): set a library tuning switch (miq_set_switch) for
    one test; every switch it set returns to its default afterwards."""
    names = []

    def set_(name, value):
        miq.set_switch(name, int(value))
        names.append(name)

    yield set_
    for n in names:
        miq.set_switch(n, miq.SWITCH_DEFAULT)


def golden(name):
    path = os.path.join(GOLDEN, name)
    return np.load(path, allow_pickle=False)


def max_rel(got, exp):
    """max|got-exp| / max|exp| -- the normalisation of the reference's own
    check_f32 (tests/backend/cpu/kernels/test_cpu_gemv_units.cpp:26-37)."""
    got = np.asarray(got, np.float64)
    exp = np.asarray(exp, np.float64)
    den = max(np.abs(exp).max(), 1e-30)
    return float(np.abs(got - exp).max() / den)
