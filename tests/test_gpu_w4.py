"""GPU: the u4 native-width store (miq_w4_pack / miq_w4_act / miq_w4_gemv)
against the oracle on the same inputs.

Bit-exact: the repacked planes and the quantized activation (without `up`).
fp32 GEMV outputs: max|got-exp|/max|exp| < 1e-4 against the oracle's double
sum over the same store and activation.  Covers the 16-byte staging path
(N % 8 == 0) and the element path (ragged N), every tile shape, one-group K,
the bench shapes, alpha/residual, and K split across workgroups."""
import numpy as np
import pytest

from conftest import golden, max_rel

pytestmark = pytest.mark.gpu
Q4_K = 12


def _np(t):
    return t.cpu().numpy()


def _store(miq, oracle, w, K, N, dev):
    import torch
    wd = torch.from_numpy(np.ascontiguousarray(w)).to(dev)
    st = miq.w4_pack(wd, K, N)
    torch.cuda.synchronize()
    exp = oracle.w4_pack(w, K, N)
    got = (_np(st.vals), _np(st.scale).view(np.uint16), _np(st.off).view(np.uint16))
    for g, e, nm in zip(got, exp, ("vals", "scale", "off")):
        assert np.array_equal(g, e), nm
    return st, exp


def test_w4_pack_golden(miq, oracle, dev):
    g = golden("w4_pack.npz")
    print("w4 pack golden", flush=True)
    _store(miq, oracle, g["w"], int(g["K"]), int(g["N"]), dev)
    _store(miq, oracle, g["pat_w"], 512, 3, dev)


@pytest.mark.parametrize("M,K", [(1, 32), (3, 1024), (2, 17408)])
def test_w4_act_bit_exact(miq, oracle, dev, M, K):
    import torch
    print(f"w4 act M={M} K={K}", flush=True)
    rng = np.random.default_rng(K)
    x = (rng.standard_normal((M, K)) * 10.0 ** rng.integers(-4, 3, (M, K // 32)).repeat(32, 1)).astype(np.float32)
    x[0, :32] = 0.0  # an all-zero group
    if K >= 64:
        x[-1, 32:40] = [2.5, -2.5, 0.5, -0.5, 126.5, -126.5, 127.0, 1e-3]  # exact .5 ties at inv == 1
    a = miq.w4_act(torch.from_numpy(x).to(dev))
    torch.cuda.synchronize()
    e = oracle.w4_act(x)
    for g, ex, nm in zip((_np(a.xq), _np(a.asa).view(np.uint16), _np(a.xs), _np(a.axe), _np(a.axo)), e,
                         ("xq", "asa", "xs", "axe", "axo")):
        assert np.array_equal(g, ex), nm


def test_w4_act_up(miq, oracle, dev):
    """silu(x)*up: the device expf restates the host libm's, so every plane is bit-exact"""
    import torch
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((2, 512)) * 8).astype(np.float32)
    up = rng.standard_normal((2, 512)).astype(np.float32)
    x[0, :64] = np.linspace(-110, 110, 64, dtype=np.float32)
    a = miq.w4_act(torch.from_numpy(x).to(dev), torch.from_numpy(up).to(dev))
    torch.cuda.synchronize()
    e = oracle.w4_act(x, up)
    for g, ex, nm in zip((_np(a.xq), _np(a.asa).view(np.uint16), _np(a.xs), _np(a.axe), _np(a.axo)), e,
                         ("xq", "asa", "xs", "axe", "axo")):
        assert np.array_equal(g, ex), nm


# tiles: 32 rows for K/32 <= 192 groups (first six), 16 rows with 2 or 4 K-parts beyond
# (the 16-row tile with one K-part serves the quantizing form at long K)
@pytest.mark.parametrize("N,K", [(3, 512), (37, 256), (64, 1024), (200, 4096), (1000, 2816), (17408, 5120),
                                 (16384, 7168), (8192, 12288), (5120, 17408), (77, 17408)])
def test_w4_gemv_vs_oracle(miq, oracle, dev, N, K):
    import torch
    print(f"w4 gemv N={N} K={K}", flush=True)
    rng = np.random.default_rng(N + K)
    if N == 3:
        w = golden("w4_pack.npz")["pat_w"]
    else:
        w = miq.quantize_rows(Q4_K, (rng.standard_normal((N, K)) * 0.02).astype(np.float32))
    st, est = _store(miq, oracle, w, K, N, dev)
    x = rng.standard_normal((1, K)).astype(np.float32)
    act = miq.w4_act(torch.from_numpy(x).to(dev))
    out = torch.full((N,), float("nan"), dtype=torch.float32, device=dev)
    miq.w4_gemv(st, act, out)
    torch.cuda.synchronize()
    eact = oracle.w4_act(x)
    exp = oracle.w4_gemv(est, eact)
    assert max_rel(_np(out), exp) < 1e-4
    res = rng.standard_normal(N).astype(np.float32)
    miq.w4_gemv(st, act, out, residual=torch.from_numpy(res).to(dev), alpha=0.75)
    torch.cuda.synchronize()
    assert max_rel(_np(out), oracle.w4_gemv(est, eact, residual=res, alpha=0.75)) < 1e-4


def test_w4_gemv_one_group_k(miq, oracle, dev):
    """K = 32: one group per row (the store does not need whole Q4_K blocks)."""
    import torch
    rng = np.random.default_rng(1)
    N, K = 24, 32
    vals = rng.integers(0, 256, (N, K // 2), dtype=np.uint8)
    sc = np.abs(rng.standard_normal((1, N))).astype(np.float16).view(np.uint16)
    of = (-np.abs(rng.standard_normal((1, N)))).astype(np.float16).view(np.uint16)
    st = miq.W4Store(torch.from_numpy(vals).to(dev), torch.from_numpy(sc.view(np.int16)).to(dev),
                     torch.from_numpy(of.view(np.int16)).to(dev), K, N)
    x = rng.standard_normal((1, K)).astype(np.float32)
    act = miq.w4_act(torch.from_numpy(x).to(dev))
    out = torch.empty(N, dtype=torch.float32, device=dev)
    miq.w4_gemv(st, act, out)
    torch.cuda.synchronize()
    assert max_rel(_np(out), oracle.w4_gemv((vals, sc, of), oracle.w4_act(x))) < 1e-4


def test_w4_gemv_long_k(miq, oracle, dev):
    """K = 32768 (1024 groups): K split over seven workgroup parts, sums added in part order"""
    import torch
    rng = np.random.default_rng(32768)
    N, K = 40, 32768
    w = miq.quantize_rows(Q4_K, (rng.standard_normal((N, K)) * 0.02).astype(np.float32))
    st, est = _store(miq, oracle, w, K, N, dev)
    x = rng.standard_normal((1, K)).astype(np.float32)
    act = miq.w4_act(torch.from_numpy(x).to(dev))
    out = torch.empty(N, dtype=torch.float32, device=dev)
    res = rng.standard_normal(N).astype(np.float32)
    miq.w4_gemv(st, act, out, residual=torch.from_numpy(res).to(dev), alpha=2.0)
    torch.cuda.synchronize()
    assert max_rel(_np(out), oracle.w4_gemv(est, oracle.w4_act(x), residual=res, alpha=2.0)) < 1e-4


@pytest.mark.parametrize("N,K", [(24, 512), (37, 2048), (7168, 5120), (5120, 17408)])
def test_k5_pack_and_gemv_vs_oracle(miq, oracle, dev, N, K):
    """k5: the repacked planes bit-exact, the GEMV within 1e-4 of the oracle"""
    import torch
    print(f"k5 N={N} K={K}", flush=True)
    rng = np.random.default_rng(N * 3 + K)
    if N == 24:
        w = golden("k5_pack.npz")["w"]
    else:
        w = miq.quantize_rows(13, (rng.standard_normal((N, K)) * 0.02).astype(np.float32))
    st = miq.k5_pack(torch.from_numpy(np.ascontiguousarray(w)).to(dev), K, N)
    torch.cuda.synchronize()
    exp = oracle.k5_pack(w, K, N)
    got = (_np(st.vals), _np(st.hi), _np(st.scale).view(np.uint16), _np(st.off).view(np.uint16))
    for g, e, nm in zip(got, exp, ("vals", "hi", "scale", "off")):
        assert np.array_equal(g, e), nm
    x = rng.standard_normal((1, K)).astype(np.float32)
    act = miq.w4_act(torch.from_numpy(x).to(dev))
    out = torch.full((N,), float("nan"), dtype=torch.float32, device=dev)
    res = rng.standard_normal(N).astype(np.float32)
    miq.k5_gemv(st, act, out, residual=torch.from_numpy(res).to(dev), alpha=0.5)
    torch.cuda.synchronize()
    assert max_rel(_np(out), oracle.k5_gemv(exp, oracle.w4_act(x), residual=res, alpha=0.5)) < 1e-4


@pytest.mark.parametrize("K,Ns,with_up", [(5120, (17408,), False), (2816, (37, 1000, 64), True),
                                          (8192, (256, 8), False), (7168, (96,), True),
                                          # 193..256 groups whose half is not whole 16-group units: the
                                          # plain GEMV splits K across workgroups, the fused form inside one
                                          (7680, (512,), False), (6912, (300,), True), (7936, (64,), False),
                                          # N >= 16384 with more than one segment (the tile choice by max N)
                                          (4096, (16384, 200), True)])
def test_w4_quant_gemv_matches_two_launches(miq, dev, K, Ns, with_up):
    """the fused quantizer + segments launch is bit-identical to miq_w4_act + one miq_w4_gemv per segment"""
    import torch
    print(f"w4 quant gemv K={K} segs={Ns} up={with_up}", flush=True)
    rng = np.random.default_rng(K + len(Ns))
    x = torch.from_numpy(rng.standard_normal(K).astype(np.float32)).to(dev)
    up = torch.from_numpy(rng.standard_normal(K).astype(np.float32)).to(dev) if with_up else None
    segs, ref = [], []
    for i, N in enumerate(Ns):
        w = miq.quantize_rows(Q4_K, (rng.standard_normal((N, K)) * 0.02).astype(np.float32))
        st = miq.w4_pack(torch.from_numpy(w).to(dev), K, N)
        res = torch.from_numpy(rng.standard_normal(N).astype(np.float32)).to(dev) if i % 2 else None
        out = torch.full((N,), float("nan"), dtype=torch.float32, device=dev)
        segs.append((st, out, 0.5 + i, res))
        ref.append(torch.empty(N, dtype=torch.float32, device=dev))
    miq.w4_quant_gemv(segs, x, up)
    act = miq.w4_act(x.view(1, K), None if up is None else up.view(1, K))
    for (st, out, alpha, res), r in zip(segs, ref):
        miq.w4_gemv(st, act, r, residual=res, alpha=alpha)
    torch.cuda.synchronize()
    for (_, out, _, _), r in zip(segs, ref):
        assert np.array_equal(_np(out), _np(r))


def test_w4_quant_gemv_declines_long_k(miq, dev):
    """beyond what one workgroup quantizes: MIQ_UNSUPPORTED and nothing launched (the caller falls back)"""
    import torch
    K, N = 8224, 16
    st = miq.W4Store(torch.zeros((N, K // 2), dtype=torch.uint8, device=dev),
                     torch.zeros((K // 32, N), dtype=torch.int16, device=dev),
                     torch.zeros((K // 32, N), dtype=torch.int16, device=dev), K, N)
    out = torch.full((N,), 7.0, dtype=torch.float32, device=dev)
    with pytest.raises(miq.MiqError, match="quantizer"):
        miq.w4_quant_gemv([(st, out, 1.0, None)], torch.zeros(K, dtype=torch.float32, device=dev))
    torch.cuda.synchronize()
    assert np.all(_np(out) == 7.0)


@pytest.mark.parametrize("M,N,K", [(2, 1000, 5120), (4, 64, 2816), (7, 17408, 5120), (3, 37, 1024), (5, 5120, 17408)])
def test_w4_gemm_vs_oracle(miq, oracle, dev, M, N, K):
    """several tokens: each output row m against the oracle's one-row GEMV on activation row m"""
    import torch
    print(f"w4 gemm M={M} N={N} K={K}", flush=True)
    rng = np.random.default_rng(M * 7 + N)
    w = miq.quantize_rows(Q4_K, (rng.standard_normal((N, K)) * 0.02).astype(np.float32))
    st, est = _store(miq, oracle, w, K, N, dev)
    x = rng.standard_normal((M, K)).astype(np.float32)
    act = miq.w4_act(torch.from_numpy(x).to(dev))
    stride = N + 3
    out = torch.full((M, stride), float("nan"), dtype=torch.float32, device=dev)
    res = rng.standard_normal((M, stride)).astype(np.float32)
    miq.w4_gemm(st, act, out, residual=torch.from_numpy(res).to(dev), alpha=0.25)
    torch.cuda.synchronize()
    got = _np(out)
    eact = oracle.w4_act(x)
    for m in range(M):
        row = tuple(a[m:m + 1] for a in eact)
        exp = oracle.w4_gemv(est, row, residual=res[m, :N], alpha=0.25)
        assert max_rel(got[m, :N], exp) < 1e-4, m
    assert np.all(np.isnan(got[:, N:]))  # the stride gap is not written


@pytest.mark.parametrize("fmt,M,N,K", [(0, 2, 1000, 5120), (0, 8, 64, 2816), (0, 13, 17408, 5120), (0, 32, 512, 4096),
                                       (0, 20, 5120, 17408), (0, 9, 37, 1024), (1, 2, 24, 512), (1, 5, 7168, 5120),
                                       (1, 8, 5120, 17408), (1, 13, 1000, 2048), (1, 6, 37, 1024)])
def test_nat_gemm_vs_oracle(miq, oracle, dev, fmt, M, N, K):
    """nat_gemm over the u4 / k5 store: each output row m against the oracle's one-row GEMV
    on activation row m (chunks of eight tokens, K split for the LDS budget, ragged N token by token)"""
    import torch
    print(f"nat gemm fmt={fmt} M={M} N={N} K={K}", flush=True)
    rng = np.random.default_rng(fmt * 1000 + M * 7 + N)
    w = miq.quantize_rows(13 if fmt else Q4_K, (rng.standard_normal((N, K)) * 0.02).astype(np.float32))
    if fmt:
        st = miq.k5_pack(torch.from_numpy(np.ascontiguousarray(w)).to(dev), K, N)
        est = oracle.k5_pack(w, K, N)
    else:
        st, est = _store(miq, oracle, w, K, N, dev)
    x = rng.standard_normal((M, K)).astype(np.float32)
    act = miq.w4_act(torch.from_numpy(x).to(dev))
    stride = N + 5
    out = torch.full((M, stride), float("nan"), dtype=torch.float32, device=dev)
    res = rng.standard_normal((M, stride)).astype(np.float32)
    miq.nat_gemm(st, act, out, residual=torch.from_numpy(res).to(dev), alpha=0.75)
    torch.cuda.synchronize()
    got = _np(out)
    eact = oracle.w4_act(x)
    gemv = oracle.k5_gemv if fmt else oracle.w4_gemv
    for m in range(M):
        row = tuple(a[m:m + 1] for a in eact)
        exp = gemv(est, row, residual=res[m, :N], alpha=0.75)
        assert max_rel(got[m, :N], exp) < 1e-4, m
    assert np.all(np.isnan(got[:, N:]))


@pytest.mark.parametrize("fmt,M", [(0, 1), (0, 33), (1, 14), (2, 4), (3, 4)])
def test_nat_gemm_declines(miq, dev, fmt, M):
    """the shapes and formats the reference's launcher declines: MIQ_UNSUPPORTED, nothing written"""
    import torch
    K, N = 512, 64
    st = miq.W4Store(torch.zeros((N, K // 2), dtype=torch.uint8, device=dev),
                     torch.zeros((K // 32, N), dtype=torch.int16, device=dev),
                     torch.zeros((K // 32, N), dtype=torch.int16, device=dev), K, N)
    act = miq.w4_act(torch.zeros((M, K), dtype=torch.float32, device=dev))
    out = torch.full((M, N), 7.0, dtype=torch.float32, device=dev)
    if fmt >= 2:
        rc = miq.lib().miq_nat_gemm(None, fmt, st.vals.data_ptr(), None, None, st.scale.data_ptr(), None, None, None,
                                    act.axe.data_ptr(), act.axo.data_ptr(), None, act.asa.data_ptr(),
                                    act.xs.data_ptr(), out.data_ptr(), N, None, 1.0, M, K, N)
        assert rc == miq.MIQ_UNSUPPORTED and "not built" in miq.lib().miq_last_error().decode()
    else:
        if fmt == 1:
            st = miq.K5Store(st.vals, torch.zeros((N, K // 8), dtype=torch.uint8, device=dev), st.scale, st.off, K, N)
        with pytest.raises(miq.MiqError, match="outside M"):
            miq.nat_gemm(st, act, out)
    torch.cuda.synchronize()
    assert np.all(_np(out) == 7.0)
