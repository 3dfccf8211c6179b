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


# code bytes of one block per type (zeroed, the block dequantizes to its offset
# term alone: -dmin*m for Q4_K/Q5_K, -32*d*sc for Q6_K, 0 for Q8_0)
_CODE_BYTES = {12: (144, 16, 144), 13: (176, 16, 176), 14: (210, 0, 192), 8: (34, 2, 34)}


def elem_bound(oracle, qt, wq, K, act, alpha=1.0):
    """Per-output bound on a summation-order difference: with x = x8*sx the
    dequantized activation, W the dequantized weights and W0 the same blocks
    with their codes zeroed (the block's offset term), every fp32 product and
    partial sum on either side is at most S = |x| (|W| + 2|W0|)^T in magnitude
    (|d*sc*q| <= |w| + |w0| per weight), so two evaluations of the same
    exact group dots in different fp32 orders differ by at most
    (K/32 + 32) * 2^-24 * |alpha| * S.  Returns that bound [TB, n_rows]."""
    bb, c0, c1 = _CODE_BYTES[qt]
    w = np.ascontiguousarray(wq, np.uint8)
    z = w.reshape(w.shape[0], -1, bb).copy()
    z[:, :, c0:c1] = 0
    W = np.abs(oracle.dequantize(qt, w, K)).astype(np.float32)
    W += 2 * np.abs(oracle.dequantize(qt, z.reshape(w.shape), K))
    x8, xm, _ = act
    x = np.abs(x8.astype(np.float32) * xm[..., :1]).transpose(1, 0, 2).reshape(x8.shape[1], K)
    S = (x @ W.T).astype(np.float64) * abs(alpha)
    return (K // 32 + 32) * 2.0 ** -24 * S


def assert_elem(got, exp, bound, residual=None):
    """|got - exp| <= bound + one rounding of the output itself, element by element."""
    got = np.asarray(got, np.float64)
    exp = np.asarray(exp, np.float64)
    slack = bound + 2.0 ** -23 * (np.abs(exp) + (0 if residual is None else np.abs(residual)))
    err = np.abs(got - exp)
    bad = err > slack
    assert not bad.any(), (f"{int(bad.sum())} outputs beyond the per-output bound; worst err/bound "
                           f"{float((err / np.maximum(slack, 1e-38)).max()):.3g}")
    return float((err / np.maximum(slack, 1e-38)).max())


def max_rel(got, exp):
    """max|got-exp| / max|exp| -- the normalisation of the reference's own
    check_f32 (tests/backend/cpu/kernels/test_cpu_gemv_units.cpp:26-37)."""
    got = np.asarray(got, np.float64)
    exp = np.asarray(exp, np.float64)
    den = max(np.abs(exp).max(), 1e-30)
    return float(np.abs(got - exp).max() / den)
