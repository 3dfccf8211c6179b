"""CPU: pin the oracle (oracle/miq_oracle.c) before trusting it.

Each check is chosen so that a plausible mistake in the restatement (a wrong
nibble, plane or sign, a dropped min term, a transposed index) fails:
  * golden fixtures written by sycl-infer's own compiled CPU kernels
    (tests/golden/make_golden.py) -- bit-exact;
  * closed forms and invariants (IEEE half conversion over all 2^16 patterns,
    truncation bracketing, scale pack/unpack, rank top-k, renormalisation);
  * brute force: integer dots from independently decoded codes, and the
    reference's own test tolerance against a dequantize + double-dot.
"""
import numpy as np
import pytest

from conftest import golden, max_rel

Q8_0, Q4_K, Q5_K, Q6_K = 8, 12, 13, 14
NAMES = {Q4_K: "q4k", Q5_K: "q5k", Q6_K: "q6k", Q8_0: "q80"}


# ------------------------------------------------------------------ f16
def test_half_to_float_exhaustive(oracle):
    """quant.h:67-92 is the exact IEEE binary16 -> binary32 map: all 2^16 patterns."""
    bits = np.arange(1 << 16, dtype=np.uint16)
    exp = bits.view(np.float16).astype(np.float32)
    got = np.array([oracle.half_to_float(int(b)) for b in bits], np.float32)
    fin = np.isfinite(exp)
    assert np.array_equal(got[fin].view(np.uint32), exp[fin].view(np.uint32))
    assert np.all(np.isnan(got[np.isnan(exp)])) and np.array_equal(got[np.isinf(exp)], exp[np.isinf(exp)])


def test_float_to_half_truncates(oracle):
    """quant.h:112-133 truncates toward zero: |h| <= |f| < next(|h|) on the finite range."""
    rng = np.random.default_rng(3)
    f = (rng.standard_normal(20000) * 10.0 ** rng.integers(-9, 5, 20000)).astype(np.float32)
    for v in f:
        h = oracle.float_to_half(float(v))
        a = abs(float(np.float32(v)))
        lo = abs(oracle.half_to_float(h))
        hi = abs(oracle.half_to_float((h & 0x7FFF) + 1)) if (h & 0x7FFF) < 0x7BFF else np.inf
        if a >= 65520.0:
            assert (h & 0x7FFF) == 0x7C00
        else:
            assert lo <= a < hi, (v, h)
            assert (h >> 15) == (np.float32(v).view(np.uint32) >> 31)


def test_float_to_half_golden(oracle):
    g = golden("f16.npz")
    got = np.array([oracle.float_to_half(float(v)) for v in g["f"]], np.uint16)
    assert np.array_equal(got, g["h"])


# ------------------------------------------------------------------ scales
def test_get_scale_min_k4_roundtrip(oracle):
    """Pack 8 arbitrary 6-bit (sc, m) with the ggml layout, unpack with the oracle."""
    rng = np.random.default_rng(4)
    for _ in range(300):
        sc = rng.integers(0, 64, 8)
        m = rng.integers(0, 64, 8)
        s = np.zeros(12, np.uint8)
        for j in range(4):
            s[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
            s[j + 4] = (m[j] & 63) | ((m[j + 4] >> 4) << 6)
            s[j + 8] = (sc[j + 4] & 15) | ((m[j + 4] & 15) << 4)
        for j in range(8):
            assert oracle.get_scale_min_k4(j, s) == (sc[j], m[j])


# ------------------------------------------------------------------ dequant
@pytest.mark.parametrize("qt", [Q4_K, Q5_K, Q6_K, Q8_0])
def test_dequant_golden(oracle, qt):
    g = golden(f"gemm_{NAMES[qt]}.npz")
    got = oracle.dequantize(qt, g["w"], int(g["K"]))
    assert np.array_equal(got.view(np.uint32), g["deq"].view(np.uint32))


def test_dequant_q8_0_hand_built(oracle):
    """Q8_0 is d*q (the hand-built patterns of tests/model/test_quant_synth.cpp)."""
    blk = np.zeros(34, np.uint8)
    blk[0:2] = np.array([0x3800], np.uint16).view(np.uint8)  # d = 0.5
    blk[2:] = np.arange(-16, 16, dtype=np.int8).view(np.uint8)
    got = oracle.dequantize(Q8_0, blk, 32)[0]
    assert np.array_equal(got, 0.5 * np.arange(-16, 16, dtype=np.float32))


def test_dequant_q4_k_hand_built(oracle):
    """One Q4_K block with known fields: y = d*sc*q - dmin*m."""
    blk = np.zeros(144, np.uint8)
    blk[0:2] = np.array([np.float16(0.5).view(np.uint16)], np.uint16).view(np.uint8)
    blk[2:4] = np.array([np.float16(0.25).view(np.uint16)], np.uint16).view(np.uint8)
    sc = [1, 2, 3, 4, 5, 6, 7, 63]
    m = [0, 1, 2, 3, 40, 50, 60, 33]
    for j in range(4):
        blk[4 + j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        blk[8 + j] = (m[j] & 63) | ((m[j + 4] >> 4) << 6)
        blk[12 + j] = (sc[j + 4] & 15) | ((m[j + 4] & 15) << 4)
    q = np.arange(256) % 16
    for g in range(8):
        for l in range(32):
            blk[16 + (g // 2) * 32 + l] |= q[g * 32 + l] << (4 * (g & 1))
    got = oracle.dequantize(Q4_K, blk, 256)[0]
    exp = np.array([0.5 * sc[i // 32] * q[i] - 0.25 * m[i // 32] for i in range(256)], np.float32)
    assert np.array_equal(got, exp)


# ------------------------------------------------------------------ xq
@pytest.mark.parametrize("case", ["ut", "ut_up", "rand", "ties"])
def test_xq_golden(oracle, case):
    g = golden("xq.npz")
    up = g[f"{case}_up"] if f"{case}_up" in g else None
    x8, xm, xs = oracle.xq(g[f"{case}_x"], up)
    assert np.array_equal(x8, g[f"{case}_x8"])
    assert np.array_equal(xm.view(np.uint32), g[f"{case}_xmeta"].view(np.uint32))
    assert np.array_equal(xs, g[f"{case}_xsumq"])


def test_xq_closed_form(oracle):
    """The reference unit test's closed form (test_cpu_elementwise_units.cpp:221-266)
    restated in numpy: round half away from zero, clamp, f16-truncated scale."""
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((4, 256)) * 2).astype(np.float32)
    x[2, 64:96] = 0
    x8, xm, xs = oracle.xq(x)
    for t in range(4):
        for g in range(8):
            v = x[t, g * 32:(g + 1) * 32]
            mx = np.float32(np.abs(v).max())
            inv = np.float32(127.0) / mx if mx > 0 else np.float32(0)
            r = v * inv
            q = np.clip(np.sign(r) * np.floor(np.abs(r) + np.float32(0.5)), -127, 127).astype(np.int32)
            assert np.array_equal(x8[g, t], q.astype(np.int8))
            assert xs[g, t, 0] == q[:16].sum() and xs[g, t, 1] == q[16:].sum()
            sc = np.float32(mx / np.float32(127.0)) if mx > 0 else np.float32(0)
            h = oracle.float_to_half(float(sc))
            assert xm[g, t, 0] == np.float32(oracle.half_to_float(h)) and xm[g, t, 1] == 0
    assert np.all(x8[2:3, 2] == 0) and xm[2, 2, 0] == 0 and xs[2, 2, 0] == 0


# ------------------------------------------------------------------ integer dots
def _codes(oracle, qt, w, K):
    """Unsigned integer codes recovered from the dequantized values: q = (y + dmin*m)/(d*sc)
    would need the scales; instead decode with an independent numpy bit parser."""
    w = np.asarray(w, np.uint8)
    n = w.shape[0]
    out = np.zeros((n, K), np.int32)
    if qt == Q8_0:
        b = w.reshape(n, -1, 34)
        return b[:, :, 2:].view(np.int8).reshape(n, K).astype(np.int32)
    bb = {Q4_K: 144, Q5_K: 176, Q6_K: 210}[qt]
    b = w.reshape(n, -1, bb)
    for bi in range(K // 256):
        blk = b[:, bi].astype(np.int32)
        for i in range(256):
            if qt in (Q4_K, Q5_K):
                g, l = divmod(i, 32)
                qs = blk[:, (16 if qt == Q4_K else 48) + (g // 2) * 32 + l]
                q = (qs >> (4 * (g & 1))) & 15
                if qt == Q5_K:
                    q |= ((blk[:, 16 + l] >> g) & 1) << 4
            else:
                n128, r = divmod(i, 128)
                plane, l = divmod(r, 32)
                ql = blk[:, n128 * 64 + (32 if plane & 1 else 0) + l]
                lo = (ql >> 4) if plane >= 2 else (ql & 15)
                q = lo | (((blk[:, 128 + n128 * 32 + l] >> (2 * plane)) & 3) << 4)
            out[:, bi * 256 + i] = q
    return out


@pytest.mark.parametrize("qt", [Q4_K, Q5_K, Q6_K, Q8_0])
def test_group_dots_brute_force(oracle, qt):
    g = golden(f"gemm_{NAMES[qt]}.npz")
    K, N = int(g["K"]), int(g["N"])
    x = g["x3"]
    x8, _, _ = oracle.xq(x)
    got = oracle.group_dots(qt, g["w"], K, N, x8)
    q = _codes(oracle, qt, g["w"], K)
    xv = x8.transpose(1, 0, 2).reshape(3, K).astype(np.int64)  # [t][k]
    L = 16 if qt == Q6_K else 32
    exp = (q[None, :, :].astype(np.int64) * xv[:, None, :]).reshape(3, N, K // L, L).sum(-1)
    assert np.array_equal(got, exp)


@pytest.mark.parametrize("qt", [Q4_K, Q5_K, Q6_K])
def test_codes_match_dequant(oracle, qt):
    """The independently parsed codes reproduce the golden dequant through the
    published scale formulas (pins the bit parser used above)."""
    g = golden(f"gemm_{NAMES[qt]}.npz")
    K = int(g["K"])
    q = _codes(oracle, qt, g["w"], K)
    w = g["w"].reshape(g["w"].shape[0], -1, {Q4_K: 144, Q5_K: 176, Q6_K: 210}[qt])
    deq = np.zeros(q.shape, np.float32)
    for bi in range(K // 256):
        blk = w[:, bi]
        if qt == Q6_K:
            d = blk[:, 208:210].copy().view(np.float16)[:, 0].astype(np.float32)
            sc = blk[:, 192:208].view(np.int8).astype(np.float32)
            for i in range(256):
                n128, r = divmod(i, 128)
                plane, l = divmod(r, 32)
                s = n128 * 8 + plane * 2 + l // 16
                deq[:, bi * 256 + i] = d * sc[:, s] * (q[:, bi * 256 + i] - 32).astype(np.float32)
        else:
            d = blk[:, 0:2].copy().view(np.float16)[:, 0].astype(np.float32)
            dm = blk[:, 2:4].copy().view(np.float16)[:, 0].astype(np.float32)
            for r in range(blk.shape[0]):
                for gi in range(8):
                    sc, m = oracle.get_scale_min_k4(gi, blk[r, 4:16])
                    sl = slice(bi * 256 + gi * 32, bi * 256 + gi * 32 + 32)
                    deq[r, sl] = np.float32(d[r] * np.float32(sc)) * q[r, sl].astype(np.float32) - np.float32(dm[r] * np.float32(m))
    assert np.array_equal(deq, g["deq"])


# ------------------------------------------------------------------ GEMV / GEMM
@pytest.mark.parametrize("qt", [Q4_K, Q5_K, Q6_K, Q8_0])
@pytest.mark.parametrize("TB", [1, 3, 16, 32])
def test_gemm_golden(oracle, qt, TB):
    """cpu_i8_gemv (TB=1) / cpu_i8_gemm (tiled, TB>=2) of the compiled reference: bit-exact."""
    g = golden(f"gemm_{NAMES[qt]}.npz")
    K, N = int(g["K"]), int(g["N"])
    act = oracle.xq(g[f"x{TB}"])
    out = oracle.gemm(qt, g["w"], K, N, act)
    assert np.array_equal(out.view(np.uint32), g[f"out{TB}"].view(np.uint32)), max_rel(out, g[f"out{TB}"])
    if qt != Q8_0:
        out = oracle.gemm(qt, g["w"], K, N, act, residual=g[f"res{TB}"], alpha=0.75)
        assert np.array_equal(out.view(np.uint32), g[f"outra{TB}"].view(np.uint32))


def test_q80_odd_groups_golden(oracle):
    """Q8_0 rows with an odd number of 32-value groups (K = 96, 160, 352, 5152): the
    oracle equals the compiled reference's native Q8_0 down (cpu_q8_0_down_grouped,
    q4exp.cpp:442-484, which loops G = K/32 groups) bit for bit, and its group dots
    equal the brute-force dots of the independently parsed codes."""
    g = golden("gemm_q80_odd.npz")
    for k in g.files:
        if not k.startswith("out"):
            continue
        K, TB = (int(v) for v in k[3:].split("_"))
        w = g[f"w{K}"]
        act = oracle.xq(g[f"x{K}_{TB}"])
        out = oracle.gemm(Q8_0, w, K, w.shape[0], act)
        assert np.array_equal(out.view(np.uint32), g[k].view(np.uint32)), k
        got = oracle.group_dots(Q8_0, w, K, w.shape[0], act[0])
        q = _codes(oracle, Q8_0, w, K).astype(np.int64)
        xv = act[0].transpose(1, 0, 2).reshape(TB, K).astype(np.int64)
        exp = (q[None, :, :] * xv[:, None, :]).reshape(TB, w.shape[0], K // 32, 32).sum(-1)
        assert np.array_equal(got, exp), k


def test_gemm_reference_pattern(oracle):
    """The reference unit test's hand-built Q4_K tensor (test_cpu_gemv_units.cpp:91-150)."""
    g = golden("gemm_q4k_pattern.npz")
    for TB in (1, 3):
        out = oracle.gemm(Q4_K, g["w"], 256, 3, oracle.xq(g[f"x{TB}"]))
        assert np.array_equal(out, g[f"out{TB}"])
        exp = (g[f"x{TB}"].astype(np.float64) @ g["deq"].T.astype(np.float64))
        # the reference test's own tolerance: 3e-2 * max(1e-2, |exp|)
        assert np.abs(out - exp).max() <= 3e-2 * max(1e-2, np.abs(exp).max())


@pytest.mark.parametrize("qt", [Q4_K, Q5_K, Q6_K, Q8_0])
def test_gemm_vs_double_dequant(oracle, qt):
    """Independent of the fixtures: the integer GEMM approximates the fp64 product of
    the dequantized weights with the fp32 activations within the int8 activation error."""
    g = golden(f"gemm_{NAMES[qt]}.npz")
    K, N = int(g["K"]), int(g["N"])
    x = g["x16"]
    out = oracle.gemm(qt, g["w"], K, N, oracle.xq(x))
    exp = x.astype(np.float64) @ g["deq"].T.astype(np.float64)
    assert max_rel(out, exp) < 3e-2
    # and it is exactly the fp64 product with the dequantized *activations*, up to fp32 rounding
    x8, xm, _ = oracle.xq(x)
    xd = (x8.astype(np.float64) * xm[:, :, :1].astype(np.float64)).transpose(1, 0, 2).reshape(16, K)
    assert max_rel(out, xd @ g["deq"].T.astype(np.float64)) < 2e-5


# ------------------------------------------------------------------ MoE
def test_moe_route_golden(oracle):
    g = golden("moe.npz")
    top_k = int(g["dims"][2])
    ids, wts, probs = oracle.moe_route(g["logits"], top_k)
    assert np.array_equal(ids, g["ids"])
    assert np.array_equal(wts, g["wts"])
    assert np.array_equal(probs, g["probs"])
    r = golden("moe_router.npz")
    ids, wts, probs = oracle.moe_route(np.zeros((5, 16), np.float32), 4, x=r["x"], gate_inp=r["gate_inp"])
    assert np.array_equal(ids, r["ids"]) and np.array_equal(wts, r["wts"]) and np.array_equal(probs, r["probs"])


def test_moe_route_invariants(oracle):
    """Top-k by rank with ties to the lower index; weights renormalised to sum 1."""
    rng = np.random.default_rng(6)
    lg = rng.standard_normal((50, 64)).astype(np.float32)
    lg[3] = 0.25
    ids, wts, _ = oracle.moe_route(lg, 8)
    for t in range(50):
        order = np.lexsort((np.arange(64), -lg[t].astype(np.float64)))[:8]
        assert np.array_equal(ids[t], order)
        assert abs(wts[t].sum() - 1.0) < 1e-6 and np.all(np.diff(wts[t]) <= 0)
    assert np.array_equal(ids[3], np.arange(8))


def test_moe_experts_golden(oracle):
    g = golden("moe.npz")
    n_tok, n_expert, top_k, n_embd, n_ff = (int(v) for v in g["dims"])
    acc = oracle.moe_experts(Q4_K, g["gate"], g["up"], g["down"], n_embd, n_ff, n_expert, g["x"], top_k, g["ids"])
    assert np.array_equal(acc.view(np.uint32), g["acc"].view(np.uint32)), max_rel(acc, g["acc"])
    out = oracle.moe_reduce(g["acc"], g["wts"], top_k, g["out0"])
    assert np.array_equal(out, g["out"])


def test_moe_experts_composition(oracle):
    """The expert output is the composition of the pinned pieces: gate/up GEMV,
    silu*up, requantisation, down GEMV (cpu_moe_experts_i8, moe.cpp:476-559)."""
    g = golden("moe.npz")
    n_tok, n_expert, top_k, n_embd, n_ff = (int(v) for v in g["dims"])
    acc, h = oracle.moe_experts(Q4_K, g["gate"], g["up"], g["down"], n_embd, n_ff, n_expert, g["x"], top_k,
                                g["ids"], want_h=True)
    rb_g = n_embd // 256 * 144
    rb_d = n_ff // 256 * 144
    for p in (0, 7, 17):
        t, e = p // top_k, int(g["ids"].reshape(-1)[p])
        a = oracle.xq(g["x"][t:t + 1])
        gw = g["gate"].reshape(n_expert, n_ff, rb_g)[e]
        uw = g["up"].reshape(n_expert, n_ff, rb_g)[e]
        gg = oracle.gemm(Q4_K, gw, n_embd, n_ff, a)[0]
        uu = oracle.gemm(Q4_K, uw, n_embd, n_ff, a)[0]
        hh = np.array([oracle.silu(float(v)) for v in gg], np.float32) * uu
        assert np.array_equal(hh, h[p])
        dw = g["down"].reshape(n_expert, n_embd, rb_d)[e]
        assert np.array_equal(oracle.gemm(Q4_K, dw, n_ff, n_embd, oracle.xq(hh[None]))[0], acc[p])


def test_moe_grouped_flow(ref, oracle, miq):
    """The reference's grouped expert flow (moe_experts_grouped_i8, moe.cpp:147-334:
    pairs bucketed per expert, the row-tiled integer GEMM on each expert's gathered
    rows padded to 32 tokens) against the oracle's grouped composition, bit for bit,
    on the golden case and on a routed 16-token case with several pairs per expert.
    Its per-pair flow (cpu_moe_experts_i8) sums each block before the row, so with
    more than one block per row the two flows differ in the last bits; both stay
    well inside the 1e-4 bound the GPU kernels are held to."""
    g = golden("moe.npz")
    n_tok, n_expert, top_k, n_embd, n_ff = (int(v) for v in g["dims"])
    a_grp = ref.moe_experts_grouped(Q4_K, g["gate"], g["up"], g["down"], n_embd, n_ff, n_expert, g["x"], top_k,
                                    g["ids"])
    a_orc = oracle.moe_experts_grouped(Q4_K, g["gate"], g["up"], g["down"], n_embd, n_ff, n_expert, g["x"], top_k,
                                       g["ids"])
    assert np.array_equal(a_orc.view(np.uint32), a_grp.view(np.uint32))
    assert np.array_equal(a_grp.view(np.uint32), g["acc"].view(np.uint32))  # one block per row: flows agree
    rng = np.random.default_rng(11)
    n_tok, n_expert, top_k, n_embd, n_ff = 16, 12, 4, 1024, 512
    gate = miq.quantize_rows(Q4_K, (rng.standard_normal((n_expert * n_ff, n_embd)) * 0.02).astype(np.float32))
    up = miq.quantize_rows(Q4_K, (rng.standard_normal((n_expert * n_ff, n_embd)) * 0.02).astype(np.float32))
    down = miq.quantize_rows(Q4_K, (rng.standard_normal((n_expert * n_embd, n_ff)) * 0.02).astype(np.float32))
    x = rng.standard_normal((n_tok, n_embd)).astype(np.float32)
    ids, _, _ = ref.moe_route(rng.standard_normal((n_tok, n_expert)).astype(np.float32), top_k)
    ids[3, 1] = n_expert + 2  # an out-of-range id: a zero row in both flows
    assert np.bincount(ids[ids < n_expert], minlength=n_expert).max() >= 6  # experts with many pairs
    a_grp = ref.moe_experts_grouped(Q4_K, gate, up, down, n_embd, n_ff, n_expert, x, top_k, ids)
    a_orc = oracle.moe_experts_grouped(Q4_K, gate, up, down, n_embd, n_ff, n_expert, x, top_k, ids)
    assert np.array_equal(a_orc.view(np.uint32), a_grp.view(np.uint32))
    a_pair = ref.moe_experts(Q4_K, gate, up, down, n_embd, n_ff, n_expert, x, top_k, ids)
    assert not np.array_equal(a_pair, a_grp)
    assert max_rel(a_grp, a_pair) < 1e-5


def test_expf_method_exhaustive(oracle):
    """The device expf's method (glibc expf, Arm optimized-routines e_expf.c,
    FMA build) restated in C equals the host libm's expf -- what the
    reference's cpu_silu and router softmax call -- on all 2^32 inputs."""
    from concurrent.futures import ThreadPoolExecutor
    part = 1 << 29
    with ThreadPoolExecutor(8) as ex:
        res = list(ex.map(lambda i: oracle.expf_method_mismatches(i * part, part), range(8)))
    assert all(n == 0 for n, _ in res), res


def test_expf_method_known_values(oracle):
    """Closed-form points: exp(0) = 1, the overflow and underflow thresholds,
    infinities and NaN, exp(1) to the nearest float."""
    import math
    f = oracle.L.miqo_expf_method
    assert f(0.0) == 1.0 and f(-0.0) == 1.0
    assert f(float("inf")) == float("inf") and f(float("-inf")) == 0.0
    assert math.isnan(f(float("nan")))
    assert f(89.0) == float("inf") and f(-104.0) == 0.0
    assert f(1.0) == np.float32(math.e)
    assert f(-1.0) == np.float32(1 / math.e)
