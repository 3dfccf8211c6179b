"""CPU: the C-ABI library loads, exports every symbol include/miq.h declares,
and its host-side pieces (row sizes, argument checks, the encoder) behave.
No GPU compute is launched here."""
import ctypes
import os
import re

import numpy as np

from conftest import REPO

Q8_0, Q4_K, Q5_K, Q6_K = 8, 12, 13, 14


def header_symbols():
    txt = open(os.path.join(REPO, "include", "miq.h")).read()
    return sorted(set(re.findall(r"\b(miq_[a-z0-9_]+)\s*\(", txt)))


def test_exports_match_header(miq):
    lib = miq.lib()
    syms = header_symbols()
    assert len(syms) >= 14
    for s in syms:
        assert hasattr(lib, s), s
    assert sorted(miq.EXPORTS) == syms


def test_version_and_row_bytes(miq):
    lib = miq.lib()
    assert b"gfx950" in lib.miq_version()
    assert miq.row_bytes(Q4_K, 5120) == 20 * 144
    assert miq.row_bytes(Q5_K, 5120) == 20 * 176
    assert miq.row_bytes(Q6_K, 5120) == 20 * 210
    assert miq.row_bytes(Q8_0, 5120) == 160 * 34
    assert miq.row_bytes(Q4_K, 100) == 0 and miq.row_bytes(99, 256) == 0


def test_argument_errors_need_no_gpu(miq):
    lib = miq.lib()
    rc = lib.miq_xq(None, None, None, 0, 0, None, None, None, 1, 32)
    assert rc == -1 and b"bad arguments" in lib.miq_last_error()
    s = miq.Seg()
    assert lib.miq_i8_gemv(None, ctypes.byref(s)) == -1
    # a type the integer path does not serve is "unsupported" (caller falls back)
    buf = (ctypes.c_uint8 * 64)()
    s.w = s.out = s.x8 = s.xmeta = s.xsumq = ctypes.addressof(buf)
    s.type, s.K, s.n_rows = 2, 256, 1
    assert lib.miq_i8_gemm(None, ctypes.byref(s), 1) == 1
    s.type, s.K = Q4_K, 300
    assert lib.miq_i8_gemm(None, ctypes.byref(s), 1) == 1 and b"multiple" in lib.miq_last_error()


def test_encoder_roundtrip(miq, oracle):
    """Encoded blocks dequantize (oracle) back to the input within the format's step."""
    rng = np.random.default_rng(7)
    for qt, tol in ((Q4_K, 0.09), (Q5_K, 0.045), (Q6_K, 0.02), (Q8_0, 0.005)):
        W = (rng.standard_normal((16, 512)) * 0.02).astype(np.float32)
        wq = miq.quantize_rows(qt, W)
        assert wq.shape == (16, miq.row_bytes(qt, 512))
        y = oracle.dequantize(qt, wq, 512)
        rel = np.abs(y - W).max() / np.abs(W).max()
        assert rel < tol, (qt, rel)
    # threaded and serial encodes are identical
    W = rng.standard_normal((4096, 256)).astype(np.float32)
    assert np.array_equal(miq.quantize_rows(Q4_K, W, 1), miq.quantize_rows(Q4_K, W, 8))
