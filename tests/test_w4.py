"""CPU: pins the oracle's u4 native-width store functions (w4_pack, the per-group
activation quantizer, the u4 GEMV) before the GPU tests trust them.

* w4_pack: bit-exact against the compiled reference's fixtures (random blocks,
  subnormal d / dmin, the reference GPU test's pattern) and, live, against
  oracle/_ref where it is built; the reference test_w4.cpp round trip against
  dequantize_row (relative L2 < 0.002).
* float->half rounding to nearest even: numpy's float16 conversion over random
  values and every f16 rounding boundary.
* activation quantizer: per-group invariants (max code 127, |q| <= 127, error
  <= half a step, code sums, split planes).
* u4 GEMV: the dequantize x activation double sum (the reference GPU test's
  expected value and its 2e-3 bound) and the pack identity in double.
"""
import numpy as np
import pytest

from conftest import golden, max_rel

Q4_K, Q5_K = 12, 13


def unpack(vals, scale, off, K, N):
    """w = off + step*q per element, from the store planes (test_w4.cpp:71-78)."""
    q = np.empty((N, K), np.float32)
    q[:, 0::2] = vals & 0xF
    q[:, 1::2] = vals >> 4
    st = scale.view(np.float16).astype(np.float32).T  # [N, K/32]
    of = off.view(np.float16).astype(np.float32).T
    return np.repeat(of, 32, axis=1) + np.repeat(st, 32, axis=1) * q


def test_w4_pack_golden(oracle):
    g = golden("w4_pack.npz")
    K, N = int(g["K"]), int(g["N"])
    v, s, o = oracle.w4_pack(g["w"], K, N)
    assert np.array_equal(v, g["vals"]) and np.array_equal(s, g["scale"]) and np.array_equal(o, g["off"])
    v, s, o = oracle.w4_pack(g["pat_w"], 512, 3)
    assert np.array_equal(v, g["pat_vals"]) and np.array_equal(s, g["pat_scale"]) and np.array_equal(o, g["pat_off"])
    # the subnormal-d row keeps a nonzero step plane (quant.h:112-133's subnormal branch)
    assert np.count_nonzero(g["scale"][:, 3]) > 0


def test_w4_pack_vs_compiled_reference(oracle, ref, miq):
    rng = np.random.default_rng(5)
    for N, K in ((7, 256), (33, 1024), (5, 2816)):
        w = miq.quantize_rows(Q4_K, (rng.standard_normal((N, K)) * 0.05).astype(np.float32))
        a, b = oracle.w4_pack(w, K, N), ref.w4_pack(w, K, N)
        for x, y in zip(a, b):
            assert np.array_equal(x, y), (N, K)


def test_w4_pack_round_trip(oracle, miq):
    """test_w4.cpp:61-90: the unpacked store equals dequantize_row up to the f16
    rounding of the two per-group constants (worst relative L2 < 0.002)."""
    rng = np.random.default_rng(6)
    N, K = 16, 2048
    w = miq.quantize_rows(Q4_K, (rng.standard_normal((N, K)) * 0.02).astype(np.float32))
    v, s, o = oracle.w4_pack(w, K, N)
    got = unpack(v, s, o, K, N).astype(np.float64)
    deq = oracle.dequantize(Q4_K, w, K).astype(np.float64)
    rel = np.sqrt(((got - deq) ** 2).sum(1) / (deq ** 2).sum(1))
    assert rel.max() < 0.002, rel.max()
    g = golden("w4_pack.npz")
    z = unpack(g["vals"], g["scale"], g["off"], 512, 24)[5]  # d = dmin = 0 row
    assert np.all(z == 0)


def test_w4_pack_rejects_ragged_k(oracle):
    with pytest.raises(ValueError):
        oracle.w4_pack(np.zeros((1, 144), np.uint8), 255, 1)


def test_float_to_half_rne_vs_numpy(oracle):
    rng = np.random.default_rng(7)
    f = np.concatenate([
        (rng.standard_normal(20000) * 10.0 ** rng.integers(-10, 6, 20000)).astype(np.float32),
        np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, -65520.0, 1e9, np.inf, -np.inf,
                  2.0 ** -24, 2.0 ** -25, 2.0 ** -25 * 1.0000001, 3 * 2.0 ** -26, 2.0 ** -14, 1e-30], np.float32)])
    # every f16 rounding boundary: the midpoints between consecutive f16 values, and one f32 ulp either side
    h = np.arange(0, 0x7C00, dtype=np.uint16).view(np.float16).astype(np.float64)
    mid = ((h[:-1] + h[1:]) / 2).astype(np.float32)
    f = np.concatenate([f, mid, np.nextafter(mid, np.float32(0)), np.nextafter(mid, np.float32(np.inf)), -mid])
    got = np.array([oracle.float_to_half_rne(float(x)) for x in f], np.uint16)
    with np.errstate(over="ignore"):
        exp = f.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, exp)


def test_w4_act_invariants(oracle):
    rng = np.random.default_rng(8)
    M, K = 3, 1024
    x = (rng.standard_normal((M, K)) * 10.0 ** rng.integers(-3, 3, (M, K // 32)).repeat(32, 1)).astype(np.float32)
    x[1, 64:96] = 0.0
    xq, asa, xs, axe, axo = oracle.w4_act(x)
    q = xq.reshape(M, -1, 32).astype(np.int32)
    sc = asa.view(np.float16).astype(np.float64)
    mx = np.abs(x.reshape(M, -1, 32)).max(2)
    nz = mx > 0
    assert np.all(np.abs(q).max(2)[nz] == 127)          # the group max maps to +-127
    assert np.all(q[~nz] == 0) and np.all(sc[~nz] == 1.0)  # an all-zero group: scale 1, codes 0
    # within half a step of the value (the step being max/127 before the f16 store)
    step = (mx / 127.0)[..., None]
    err = np.abs(q * step - x.reshape(M, -1, 32))
    assert np.all(err <= step * 0.5 * (1 + 1e-5) + 1e-30)
    # the stored scale is max/127 to f16 precision (half an ulp; 2^-25 absolute in the subnormal range)
    assert np.all(np.abs(sc[nz] - mx[nz] / 127.0) <= np.maximum(mx[nz] / 127.0 * 2.0 ** -11, 2.0 ** -25))
    assert np.array_equal(xs, q.sum(2).astype(np.float32))
    assert np.array_equal(axe, xq[:, 0::2]) and np.array_equal(axo, xq[:, 1::2])


def test_w4_act_up(oracle):
    """with up: the quantized value is silu(x)*up"""
    rng = np.random.default_rng(9)
    x = rng.standard_normal((2, 256)).astype(np.float32)
    up = rng.standard_normal((2, 256)).astype(np.float32)
    a = oracle.w4_act(x, up)
    b = oracle.w4_act((x / (1 + np.exp(-x.astype(np.float64)))).astype(np.float32) * up)
    assert np.abs(a[0].astype(int) - b[0].astype(int)).max() <= 1


@pytest.mark.parametrize("N,K", [(3, 512), (40, 2048)])
def test_w4_gemv_vs_dequant(oracle, miq, N, K):
    """w4_gemv against the reference GPU test's expected value
    (test_kernel_units_native.cpp:137-145): sum_k deq[n][k]*asa[k/32]*xq[k] in
    double, bound 2e-3 (the f16 rounding of step/off)."""
    rng = np.random.default_rng(N)
    if N == 3:
        w = golden("w4_pack.npz")["pat_w"]
    else:
        w = miq.quantize_rows(Q4_K, (rng.standard_normal((N, K)) * 0.02).astype(np.float32))
    st = oracle.w4_pack(w, K, N)
    x = rng.standard_normal((1, K)).astype(np.float32)
    act = oracle.w4_act(x)
    got = oracle.w4_gemv(st, act)
    xa = act[0][0].astype(np.float64) * np.repeat(act[1][0].view(np.float16).astype(np.float64), 32)
    exp = oracle.dequantize(Q4_K, w, K).astype(np.float64) @ xa
    assert max_rel(got, exp) < 2e-3
    # and the pack identity with the stored constants, in double (no f16 slack)
    exp2 = unpack(*st, K, N).astype(np.float64) @ xa
    assert max_rel(got, exp2) < 1e-5
    # alpha / residual
    res = rng.standard_normal(N).astype(np.float32)
    got2 = oracle.w4_gemv(st, act, residual=res, alpha=0.5)
    assert np.allclose(got2, 0.5 * got + res, rtol=1e-6, atol=1e-6)


def test_k5_pack_golden(oracle):
    g = golden("k5_pack.npz")
    K, N = int(g["K"]), int(g["N"])
    got = oracle.k5_pack(g["w"], K, N)
    for x, nm in zip(got, ("vals", "hi", "scale", "off")):
        assert np.array_equal(x, g[nm]), nm
    assert np.all(g["hi"][6] == 0xFF)  # an all-ones qh row sets every fifth bit


def test_k5_pack_vs_compiled_reference(oracle, ref, miq):
    rng = np.random.default_rng(15)
    for N, K in ((9, 256), (40, 1536)):
        w = miq.quantize_rows(Q5_K, (rng.standard_normal((N, K)) * 0.05).astype(np.float32))
        for x, y in zip(oracle.k5_pack(w, K, N), ref.k5_pack(w, K, N)):
            assert np.array_equal(x, y), (N, K)


def test_k5_gemv_vs_dequant(oracle, miq):
    """k5: the Q5_K dequantize x activation double sum (2e-3, the f16 metadata)
    and the unpacked-store identity in double"""
    rng = np.random.default_rng(16)
    N, K = 24, 2048
    w = miq.quantize_rows(Q5_K, (rng.standard_normal((N, K)) * 0.02).astype(np.float32))
    vals, hi, sc, of = oracle.k5_pack(w, K, N)
    x = rng.standard_normal((1, K)).astype(np.float32)
    act = oracle.w4_act(x)
    got = oracle.k5_gemv((vals, hi, sc, of), act)
    xa = act[0][0].astype(np.float64) * np.repeat(act[1][0].view(np.float16).astype(np.float64), 32)
    assert max_rel(got, oracle.dequantize(Q5_K, w, K).astype(np.float64) @ xa) < 2e-3
    # q5 = lo4 | bit << 4 with the hi plane's bit order
    hw = hi.view(np.uint32).reshape(N, K // 32)
    bits = np.empty((N, K), np.float32)
    for i in range(16):
        bits[:, 2 * i::32] = (hw >> i) & 1
        bits[:, 2 * i + 1::32] = (hw >> (16 + i)) & 1
    q = np.empty((N, K), np.float32)
    q[:, 0::2], q[:, 1::2] = vals & 0xF, vals >> 4
    q += 16 * bits
    st = np.repeat(sc.view(np.float16).astype(np.float64).T, 32, 1)
    ofs = np.repeat(of.view(np.float16).astype(np.float64).T, 32, 1)
    assert max_rel(got, (ofs + st * q) @ xa) < 1e-5
