"""GPU parity: activation quantizer, per-group integer dots and the GEMV/GEMM
family through the C ABI, against the oracle (bit-exact for integers, 1e-4 max
relative error for fp32 outputs, normalised like the reference's check_f32)."""
import numpy as np
import pytest

from conftest import assert_elem, elem_bound, golden, max_rel

pytestmark = pytest.mark.gpu

Q8_0, Q4_K, Q5_K, Q6_K = 8, 12, 13, 14
NAMES = {Q4_K: "q4k", Q5_K: "q5k", Q6_K: "q6k", Q8_0: "q80"}
TOL = 1e-4  # north-star fp32 bound


def to_dev(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def weights(miq, qt, N, K, seed, scale=0.02):
    rng = np.random.default_rng(seed)
    W = (rng.standard_normal((N, K)) * scale).astype(np.float32)
    return miq.quantize_rows(qt, W)


def run_gemm(miq, dev, qt, wq, K, N, x, residual=None, alpha=1.0, fused=False):
    import torch
    TB = x.shape[0]
    xd = to_dev(x, dev)
    wd = to_dev(wq, dev)
    out = torch.full((TB, N), float("nan"), dtype=torch.float32, device=dev)
    act = miq.alloc_act(TB, K, dev)
    res = to_dev(residual, dev) if residual is not None else None
    seg = miq.make_seg(wd, qt, K, N, act, out, N, residual=res, alpha=alpha, x=xd)
    if fused:
        miq.quant_gemm(seg, TB)
    else:
        miq.xq(xd, out=act)
        if TB == 1:
            miq.i8_gemv(seg)
        else:
            miq.i8_gemm(seg, TB)
    torch.cuda.synchronize()
    return out.cpu().numpy(), act


# ------------------------------------------------------------------ xq
@pytest.mark.parametrize("case", ["ut", "rand", "ties"])
def test_xq_golden(miq, dev, case):
    import torch
    g = golden("xq.npz")
    x = g[f"{case}_x"]
    a = miq.xq(to_dev(x, dev))
    torch.cuda.synchronize()
    assert np.array_equal(a.x8.cpu().numpy(), g[f"{case}_x8"])
    assert np.array_equal(a.xmeta.cpu().numpy().view(np.uint32), g[f"{case}_xmeta"].view(np.uint32))
    assert np.array_equal(a.xsumq.cpu().numpy(), g[f"{case}_xsumq"])


def test_xq_up_golden(miq, dev):
    """silu(x)*up: the device expf restates the host libm's, so codes, scales
    and sums equal cpu_xq's golden output bit for bit."""
    import torch
    g = golden("xq.npz")
    a = miq.xq(to_dev(g["ut_up_x"], dev), up=to_dev(g["ut_up_up"], dev))
    torch.cuda.synchronize()
    assert np.array_equal(a.x8.cpu().numpy(), g["ut_up_x8"])
    assert np.array_equal(a.xmeta.cpu().numpy().view(np.uint32), g["ut_up_xmeta"].view(np.uint32))
    assert np.array_equal(a.xsumq.cpu().numpy(), g["ut_up_xsumq"])


@pytest.mark.parametrize("TB,K,scale", [(1, 17408, 1.0), (16, 17408, 4.0), (64, 2048, 30.0), (3, 512, 100.0)])
def test_xq_up_random_bitexact(miq, oracle, dev, TB, K, scale):
    """silu(x)*up against the oracle's (host libm) on wide ranges of x, including
    |x| past 88 where expf overflows or underflows and rounding edges of codes."""
    import torch
    rng = np.random.default_rng(TB * 7 + K)
    x = (rng.standard_normal((TB, K)) * scale).astype(np.float32)
    up = rng.standard_normal((TB, K)).astype(np.float32)
    x[0, :64] = np.linspace(-110, 110, 64, dtype=np.float32)
    a = miq.xq(to_dev(x, dev), up=to_dev(up, dev))
    torch.cuda.synchronize()
    x8, xm, xs = oracle.xq(x, up)
    assert np.array_equal(a.x8.cpu().numpy(), x8)
    assert np.array_equal(a.xmeta.cpu().numpy().view(np.uint32), xm.view(np.uint32))
    assert np.array_equal(a.xsumq.cpu().numpy(), xs)


def test_expf_exhaustive(miq, oracle, dev):
    """The device expf against the host libm expf on every one of the 2^32 float
    bit patterns, in 2^28-input slices."""
    import torch
    from concurrent.futures import ThreadPoolExecutor
    chunk = 1 << 28
    y = torch.empty(chunk, dtype=torch.float32, device=dev)
    host = torch.empty(chunk, dtype=torch.float32, pin_memory=True)
    bad = []
    with ThreadPoolExecutor(8) as ex:
        for c in range(16):
            miq.expf_range(c * chunk, chunk, y)
            host.copy_(y)
            torch.cuda.synchronize()
            h = host.numpy()
            part = chunk // 8
            res = ex.map(lambda i: oracle.expf_mismatches(c * chunk + i * part, h[i * part:(i + 1) * part]), range(8))
            bad += [r for r in res if r[0]]
    assert not bad, f"device expf differs from the host's: {bad[:4]}"


@pytest.mark.parametrize("TB,K", [(1, 5120), (16, 17408), (512, 5120), (7, 96)])
def test_xq_random_bitexact(miq, oracle, dev, TB, K):
    import torch
    rng = np.random.default_rng(TB * 1000 + K)
    x = rng.standard_normal((TB, K)).astype(np.float32) * np.float32(rng.uniform(0.01, 100))
    x[0, :32] = 0
    a = miq.xq(to_dev(x, dev))
    torch.cuda.synchronize()
    x8, xm, xs = oracle.xq(x)
    assert np.array_equal(a.x8.cpu().numpy(), x8)
    assert np.array_equal(a.xmeta.cpu().numpy().view(np.uint32), xm.view(np.uint32))
    assert np.array_equal(a.xsumq.cpu().numpy(), xs)


# ------------------------------------------------------------------ integer dots
@pytest.mark.parametrize("qt", [Q4_K, Q5_K, Q6_K, Q8_0])
@pytest.mark.parametrize("path", [0, 1, 4])
@pytest.mark.parametrize("TB", [1, 3, 17, 64, 130])
def test_group_dots_bitexact(miq, oracle, dev, qt, path, TB):
    import torch
    g = golden(f"gemm_{NAMES[qt]}.npz")
    K, N = int(g["K"]), int(g["N"])
    rng = np.random.default_rng(TB)
    x = rng.standard_normal((TB, K)).astype(np.float32)
    a = miq.xq(to_dev(x, dev))
    got = miq.group_dots(to_dev(g["w"], dev), qt, K, N, a, path=path)
    torch.cuda.synchronize()
    exp = oracle.group_dots(qt, g["w"], K, N, oracle.xq(x)[0])
    assert np.array_equal(got.cpu().numpy(), exp)


@pytest.mark.parametrize("TB", [1, 2, 3, 17])
@pytest.mark.parametrize("N,K", [("golden", 0), (37, 2304), (5, 4096)])
def test_group_dots_q4k_pieces(miq, oracle, dev, TB, N, K):
    """Path 5, the decode GEMV's Q4_K piece decoder (two lanes per 32-value
    group, half-group dots added by a DPP swap): the int32 group dots equal the
    oracle's, also where a row's blocks end inside a run of eight (K = 2304)."""
    import torch
    if N == "golden":
        g = golden("gemm_q4k.npz")
        K, N, wq = int(g["K"]), int(g["N"]), g["w"]
    else:
        wq = weights(miq, Q4_K, N, K, seed=N + K)
    x = np.random.default_rng(TB + K).standard_normal((TB, K)).astype(np.float32)
    a = miq.xq(to_dev(x, dev))
    got = miq.group_dots(to_dev(wq, dev), Q4_K, K, N, a, path=5)
    torch.cuda.synchronize()
    assert np.array_equal(got.cpu().numpy(), oracle.group_dots(Q4_K, wq, K, N, oracle.xq(x)[0]))


def test_group_dots_pieces_rejects_other_types(miq, dev):
    g = golden("gemm_q6k.npz")
    K, N = int(g["K"]), int(g["N"])
    a = miq.xq(to_dev(np.ones((1, K), np.float32), dev))
    with pytest.raises(miq.MiqError, match="path 5"):
        miq.group_dots(to_dev(g["w"], dev), Q6_K, K, N, a, path=5)


def group_scales(oracle, qt, wq, K, N):
    """The 6-bit group scale sc of every (row, group) of Q4_K/Q5_K rows: the
    block's scales[12] field follows d and dmin (4 bytes in)."""
    rb = wq.reshape(N, -1)
    bb = 144 if qt == Q4_K else 176
    sc = np.zeros((N, K // 32), dtype=np.int64)
    for n in range(N):
        for b in range(K // 256):
            scales = rb[n, b * bb + 4:b * bb + 16]
            for j in range(8):
                sc[n, 8 * b + j] = oracle.get_scale_min_k4(j, scales)[0]
    return sc


def q6k_subgroup_scales(wq, K, N):
    """The signed 8-bit scale of every (row, 16-value sub-group) of Q6_K rows:
    scales[16] at byte 192 of each 210-byte block (quant.h block_q6_K)."""
    blk = wq.reshape(N, K // 256, 210)
    return blk[:, :, 192:208].view(np.int8).astype(np.int64).reshape(N, K // 16)


@pytest.mark.parametrize("TB", [1, 3, 17, 64, 130, 512])
@pytest.mark.parametrize("N,K", [(40, 512), (200, 768)])
def test_group_dots_prefill_q6k_fp16(miq, oracle, dev, TB, N, K):
    """Path 2 for Q6_K: the fp16 prefill GEMM's two-plane decoder (hi = (q-32)*2*(sc>>1),
    lo = (q-32)*(sc&1)) makes one MFMA sum per 32-group, sc0*I0 + sc1*I1 with
    I = dot - 32*xsum over each 16-value sub-group (i8.cpp:125-155), bit-exact against
    the oracle's sub-group dots, the activation's half-group code sums and the block scales."""
    import torch
    if N == 40:
        g = golden("gemm_q6k.npz")
        assert int(g["K"]) == K and int(g["N"]) == N
        wq = g["w"]
    else:
        wq = weights(miq, Q6_K, N, K, seed=N + K + 6)
    rng = np.random.default_rng(TB + 11 * N)
    x = rng.standard_normal((TB, K)).astype(np.float32)
    a = miq.xq(to_dev(x, dev))
    got = miq.group_dots(to_dev(wq, dev), Q6_K, K, N, a, path=2)
    torch.cuda.synchronize()
    _, _, xs = oracle.xq(x)
    dots = oracle.group_dots(Q6_K, wq, K, N, oracle.xq(x)[0]).astype(np.int64)  # [TB][N][K/16]
    xs = np.asarray(xs, np.int64).reshape(K // 32, TB, 2).transpose(1, 0, 2).reshape(TB, 1, K // 16)
    terms = q6k_subgroup_scales(wq, K, N)[None] * (dots - 32 * xs)
    exp = terms.reshape(TB, N, K // 32, 2).sum(axis=3)
    assert got.shape == (TB, N, K // 32)
    assert np.array_equal(got.cpu().numpy().astype(np.int64), exp)


@pytest.mark.parametrize("qt,path", [(Q4_K, 2), (Q5_K, 2), (Q4_K, 3), (Q5_K, 3), (Q6_K, 3), (Q8_0, 3)])
@pytest.mark.parametrize("TB", [1, 3, 17, 64, 130])
@pytest.mark.parametrize("N,K", [(40, 512), (200, 768)])
def test_group_dots_prefill_decoders(miq, oracle, dev, qt, path, TB, N, K):
    """The prefill GEMMs' integer cores: path 3 (int8 MFMA) returns the group
    dot itself, path 2 (fp16 MFMA on q*sc operands) returns sc * dot, which is
    exact in fp32; both bit-exact against the oracle's group dots."""
    import torch
    if N == 40:
        g = golden(f"gemm_{NAMES[qt]}.npz")
        assert int(g["K"]) == K and int(g["N"]) == N
        wq = g["w"]
    else:
        wq = weights(miq, qt, N, K, seed=N + K)
    rng = np.random.default_rng(TB + 7 * N)
    x = rng.standard_normal((TB, K)).astype(np.float32)
    a = miq.xq(to_dev(x, dev))
    got = miq.group_dots(to_dev(wq, dev), qt, K, N, a, path=path)
    torch.cuda.synchronize()
    exp = oracle.group_dots(qt, wq, K, N, oracle.xq(x)[0]).astype(np.int64)
    if path == 2:
        exp = exp * group_scales(oracle, qt, wq, K, N)[None, :, :]
    assert np.array_equal(got.cpu().numpy().astype(np.int64), exp)


def test_group_dots_path_errors(miq, dev):
    """Path 2 serves Q4_K/Q5_K/Q6_K only; unknown paths fail."""
    import torch
    K, N = 512, 40
    a = miq.xq(torch.zeros((1, K), dtype=torch.float32, device=dev))
    for qt, path in [(Q8_0, 2), (Q4_K, 9)]:
        w = torch.zeros(N * (K // 256) * 256, dtype=torch.uint8, device=dev)
        with pytest.raises(RuntimeError):
            miq.group_dots(w, qt, K, N, a, path=path)


# ------------------------------------------------------------------ GEMV / GEMM vs golden
@pytest.mark.parametrize("qt", [Q4_K, Q5_K, Q6_K, Q8_0])
@pytest.mark.parametrize("TB", [1, 3, 16, 32])
def test_gemm_golden(miq, dev, qt, TB):
    g = golden(f"gemm_{NAMES[qt]}.npz")
    K, N = int(g["K"]), int(g["N"])
    out, _ = run_gemm(miq, dev, qt, g["w"], K, N, g[f"x{TB}"])
    assert max_rel(out, g[f"out{TB}"]) <= TOL
    if qt != Q8_0:
        out, _ = run_gemm(miq, dev, qt, g["w"], K, N, g[f"x{TB}"], residual=g[f"res{TB}"], alpha=0.75)
        assert max_rel(out, g[f"outra{TB}"]) <= TOL


# ------------------------------------------------------------------ shapes and batch sizes
@pytest.mark.parametrize("qt", [Q4_K, Q5_K, Q6_K, Q8_0])
@pytest.mark.parametrize("TB", [1, 2, 4, 5, 16, 33])
@pytest.mark.parametrize("N,K", [(1000, 1024), (77, 2560)])
def test_gemm_vs_oracle(miq, oracle, dev, qt, TB, N, K):
    wq = weights(miq, qt, N, K, seed=N + K + qt)
    rng = np.random.default_rng(TB)
    x = rng.standard_normal((TB, K)).astype(np.float32)
    out, _ = run_gemm(miq, dev, qt, wq, K, N, x)
    act = oracle.xq(x)
    exp = oracle.gemm(qt, wq, K, N, act)
    assert max_rel(out, exp) <= TOL
    assert_elem(out, exp, elem_bound(oracle, qt, wq, K, act, 1.0), residual=None)


@pytest.mark.parametrize("qt", [Q4_K, Q5_K, Q6_K, Q8_0])
@pytest.mark.parametrize("TB", [48, 77, 130])
@pytest.mark.parametrize("fp16", ["2", "1", "0"])
def test_gemm_prefill_tiles_vs_oracle(miq, oracle, dev, qt, TB, fp16, switch):
    """Prefill-sized batches, with partial token and row tiles: Q4_K/Q5_K on the
    fp16-MFMA kernel (PREFILL_FP16=2 forces it; 1, the default, lets the cost
    model pick it or the 16-token kernel) and on the 64x128 LDS-tiled
    int8 kernel (0); Q8_0 on the int8 kernel either way."""
    switch("PREFILL_FP16", fp16)
    N, K = 1000, 1024
    wq = weights(miq, qt, N, K, seed=TB + qt)
    x = np.random.default_rng(TB).standard_normal((TB, K)).astype(np.float32)
    res = np.random.default_rng(TB + 1).standard_normal((TB, N)).astype(np.float32)
    out, _ = run_gemm(miq, dev, qt, wq, K, N, x, residual=res, alpha=0.5)
    act = oracle.xq(x)
    exp = oracle.gemm(qt, wq, K, N, act, residual=res, alpha=0.5)
    assert max_rel(out, exp) <= TOL
    assert_elem(out, exp, elem_bound(oracle, qt, wq, K, act, 0.5), residual=res)


@pytest.mark.parametrize("TB,N,K", [(48, 1000, 1024), (130, 300, 2560), (512, 640, 2560), (512, 4352, 256)])
@pytest.mark.parametrize("form", ["fp16", "int8", "int8_fill"])
def test_gemm_prefill_q6k_vs_oracle(miq, oracle, dev, TB, N, K, form, switch):
    """Q6_K prefill.  fp16 (the default): the stream-K fp16-MFMA kernel with the
    sub-group scale folded into two exact fp16 weight planes (v*2*floor(sc/2)
    and v*(sc&1), v = code - 32) whose MFMAs chain into one accumulator, so
    each 32-value group's result is sc0*I0 + sc1*I1 exactly.  int8
    (PREFILL_FP16=0, M32_FILL=0): the LDS-tiled int8-MFMA kernel at every size,
    one MFMA per 16-value sub-group (the other lane half's weights zeroed);
    int8_fill: the same with M32_FILL=1, where grids that leave CUs idle take
    the split-K 16-token kernel.  Partial row and token tiles, residual and
    alpha."""
    print(f"q6k prefill TB={TB} N={N} K={K} form={form}", flush=True)
    # fp16: PREFILL_FP16=2 takes the fp16 GEMM at every prefill size
    switch("PREFILL_FP16", "2" if form == "fp16" else "0")
    switch("M32_FILL", "1" if form == "int8_fill" else "0")
    wq = weights(miq, Q6_K, N, K, seed=TB + N)
    x = np.random.default_rng(TB + 5).standard_normal((TB, K)).astype(np.float32)
    res = np.random.default_rng(TB + 6).standard_normal((TB, N)).astype(np.float32)
    out, _ = run_gemm(miq, dev, Q6_K, wq, K, N, x, residual=res, alpha=0.5)
    act = oracle.xq(x)
    exp = oracle.gemm(Q6_K, wq, K, N, act, residual=res, alpha=0.5)
    assert max_rel(out, exp) <= TOL
    assert_elem(out, exp, elem_bound(oracle, Q6_K, wq, K, act, 0.5), residual=res)


@pytest.mark.parametrize("qt", [Q4_K, Q5_K])
@pytest.mark.parametrize("TB,N,K", [(48, 1000, 1024), (77, 1000, 1024), (130, 1000, 1024), (200, 300, 2560),
                                    (384, 21888, 512), (256, 4352, 2304)])
def test_gemm_prefill_fp16_vs_oracle(miq, oracle, dev, qt, TB, N, K, switch):
    """The exact fp16-MFMA prefill GEMM (q*sc against x8, sx per group in fp32,
    128 x 128 tiles; the dmin term on bf16 MFMA with a three-term split):
    partial row / token tiles, residual and alpha.  Small shapes run as K-split
    parts of a few tiles (stream-K)."""
    print(f"prefill qt={qt} TB={TB} N={N} K={K}", flush=True)
    switch("PREFILL_FP16", "2")
    wq = weights(miq, qt, N, K, seed=TB + qt + 7)
    x = np.random.default_rng(TB + 3).standard_normal((TB, K)).astype(np.float32)
    res = np.random.default_rng(TB + 4).standard_normal((TB, N)).astype(np.float32)
    out, _ = run_gemm(miq, dev, qt, wq, K, N, x, residual=res, alpha=0.5)
    act = oracle.xq(x)
    exp = oracle.gemm(qt, wq, K, N, act, residual=res, alpha=0.5)
    assert max_rel(out, exp) <= TOL
    assert_elem(out, exp, elem_bound(oracle, qt, wq, K, act, 0.5), residual=res)


@pytest.mark.parametrize("qt", [Q4_K, Q5_K, Q6_K, Q8_0])
@pytest.mark.parametrize("TB,N,K", [(4, 1000, 1024), (16, 300, 5632), (11, 77, 2560)])
def test_gemm_cu_form_vs_oracle(miq, oracle, dev, qt, TB, N, K, switch):
    """The CU-resident 16-token form (MIQ_M16_FORM=3): activation staged per CU,
    tiles shared by waves reduced in LDS; K = 5632 needs two K parts (their
    partials meet through the global buffer); N = 77 leaves most CUs idle."""
    switch("M16_FORM", "3")
    wq = weights(miq, qt, N, K, seed=N + TB + qt)
    x = np.random.default_rng(TB + 9).standard_normal((TB, K)).astype(np.float32)
    res = np.random.default_rng(TB + 10).standard_normal((TB, N)).astype(np.float32)
    out, _ = run_gemm(miq, dev, qt, wq, K, N, x, residual=res, alpha=0.5)
    act = oracle.xq(x)
    exp = oracle.gemm(qt, wq, K, N, act, residual=res, alpha=0.5)
    assert max_rel(out, exp) <= TOL
    assert_elem(out, exp, elem_bound(oracle, qt, wq, K, act, 0.5), residual=res)


@pytest.mark.parametrize("waves", ["4", "8"])
@pytest.mark.parametrize("qt", [Q4_K, Q5_K, Q6_K, Q8_0])
@pytest.mark.parametrize("TB,N,K", [(16, 200, 5120), (33, 129, 2816)])
def test_gemm_split_k_waves_vs_oracle(miq, oracle, dev, qt, TB, N, K, waves, switch):
    """The split-K 16-token form with 4- and 8-wave workgroups (MIQ_M16_WAVES):
    64- or 128-row tiles, N not a multiple of either, 1..3 token tiles."""
    switch("M16_FORM", "2")
    switch("M16_WAVES", waves)
    wq = weights(miq, qt, N, K, seed=N + TB + qt + 7)
    x = np.random.default_rng(TB + 19).standard_normal((TB, K)).astype(np.float32)
    res = np.random.default_rng(TB + 20).standard_normal((TB, N)).astype(np.float32)
    out, _ = run_gemm(miq, dev, qt, wq, K, N, x, residual=res, alpha=0.5)
    act = oracle.xq(x)
    exp = oracle.gemm(qt, wq, K, N, act, residual=res, alpha=0.5)
    assert max_rel(out, exp) <= TOL
    assert_elem(out, exp, elem_bound(oracle, qt, wq, K, act, 0.5), residual=res)


@pytest.mark.parametrize("form", ["0", "2", "3"])
@pytest.mark.parametrize("TB", [1, 2, 5, 16, 33, 64])
def test_q6k_tensor_size_2_mod_4(miq, oracle, dev, TB, form, switch):
    """129 rows x 11 Q6_K blocks = 297990 bytes: the tensor ends in the middle
    of a dword, and the last block's scale bytes share that dword.  Every form
    must read it (regression: a straddling dword read as zero)."""
    switch("M16_FORM", form)
    N, K = 129, 2816
    wq = weights(miq, Q6_K, N, K, seed=TB + 555)
    assert wq.nbytes % 4 == 2
    x = np.random.default_rng(TB + 556).standard_normal((TB, K)).astype(np.float32)
    out, _ = run_gemm(miq, dev, Q6_K, wq, K, N, x)
    act = oracle.xq(x)
    exp = oracle.gemm(Q6_K, wq, K, N, act)
    assert max_rel(out, exp) <= TOL
    assert_elem(out, exp, elem_bound(oracle, Q6_K, wq, K, act, 1.0), residual=None)


def test_gemm_cu_form_default_many_tiles(miq, oracle, dev):
    """32768 rows give every CU at least 8 tiles: the default route takes the
    CU-resident form."""
    N, K, TB = 32768, 512, 16
    wq = weights(miq, Q6_K, N, K, seed=32768)
    x = np.random.default_rng(3).standard_normal((TB, K)).astype(np.float32)
    out, _ = run_gemm(miq, dev, Q6_K, wq, K, N, x)
    act = oracle.xq(x)
    exp = oracle.gemm(Q6_K, wq, K, N, act)
    assert max_rel(out, exp) <= TOL
    assert_elem(out, exp, elem_bound(oracle, Q6_K, wq, K, act, 1.0), residual=None)


def test_gemm_prefill_fp16_stream_k(miq, oracle, dev, switch):
    """512 x 16640: 520 tiles of 128 x 128 on 512 resident workgroups, so every
    tile's K blocks are dealt out as contiguous ranges (stream-K), partial sums
    met in the XCD's L2 and added in range order."""
    print("prefill stream-K", flush=True)
    switch("PREFILL_FP16", "2")
    TB, N, K = 512, 16640, 1024
    wq = weights(miq, Q4_K, N, K, seed=520)
    x = np.random.default_rng(520).standard_normal((TB, K)).astype(np.float32)
    out, _ = run_gemm(miq, dev, Q4_K, wq, K, N, x)
    act = oracle.xq(x)
    exp = oracle.gemm(Q4_K, wq, K, N, act)
    assert max_rel(out, exp) <= TOL
    assert_elem(out, exp, elem_bound(oracle, Q4_K, wq, K, act, 1.0), residual=None)


@pytest.mark.parametrize("qt", [Q4_K, Q5_K, Q6_K])
def test_gemm_prefill_wide_activation_range(miq, oracle, dev, qt, switch):
    """The fp16 prefill GEMM on activations whose token and group magnitudes span
    1e-6 .. 1e4 (inside the f16 range of the activation scales), all-zero groups
    and blocks, one token of zeros; checked over the whole output and per token."""
    switch("PREFILL_FP16", "2")
    TB, N, K = 130, 300, 2048
    rng = np.random.default_rng(77)
    wq = weights(miq, qt, N, K, seed=78)
    x = rng.standard_normal((TB, K)).astype(np.float32)
    x *= (10.0 ** rng.uniform(-4, 2, (TB, 1))).astype(np.float32)       # per token
    x *= (10.0 ** rng.uniform(-2, 2, (1, K // 32))).repeat(32, 1).astype(np.float32)  # per group
    x[5] = 0
    x[7, 256:512] = 0
    x[9, 64:96] = 0
    out, _ = run_gemm(miq, dev, qt, wq, K, N, x)
    act = oracle.xq(x)
    exp = oracle.gemm(qt, wq, K, N, act)
    assert max_rel(out, exp) <= TOL
    assert_elem(out, exp, elem_bound(oracle, qt, wq, K, act, 1.0), residual=None)
    # every token against its own magnitude as well (the tolerance applied per row)
    for t in range(TB):
        if np.abs(exp[t]).max() > 0:
            assert max_rel(out[t], exp[t]) <= TOL, t
        else:
            assert np.all(out[t] == 0), t


@pytest.mark.parametrize("TB", [1, 3, 5, 16, 33, 64])
def test_q80_partial_step(miq, oracle, dev, TB):
    """Q8_0 only needs K % 64 == 0: K = 320 leaves a partial 256-value step whose
    missing groups must contribute nothing (the next row's bytes sit there)."""
    N, K = 150, 320
    wq = weights(miq, Q8_0, N, K, seed=320 + TB)
    x = np.random.default_rng(TB).standard_normal((TB, K)).astype(np.float32)
    out, _ = run_gemm(miq, dev, Q8_0, wq, K, N, x)
    assert max_rel(out, oracle.gemm(Q8_0, wq, K, N, oracle.xq(x))) <= TOL


def test_split_k_repeatable(miq, dev):
    """The down shape at 16 tokens splits K over workgroups; the partials are
    summed in a fixed order, so repeated calls agree bit for bit."""
    N, K = 5120, 17408
    wq = weights(miq, Q4_K, N, K, seed=9)
    x = np.random.default_rng(9).standard_normal((16, K)).astype(np.float32)
    a, _ = run_gemm(miq, dev, Q4_K, wq, K, N, x)
    for _ in range(3):
        b, _ = run_gemm(miq, dev, Q4_K, wq, K, N, x)
        assert np.array_equal(a, b)


def test_fused_quant_gemm_equals_two_calls(miq, dev):
    wq = weights(miq, Q4_K, 512, 2048, seed=11)
    x = np.random.default_rng(2).standard_normal((16, 2048)).astype(np.float32)
    a, _ = run_gemm(miq, dev, Q4_K, wq, 2048, 512, x)
    b, _ = run_gemm(miq, dev, Q4_K, wq, 2048, 512, x, fused=True)
    assert np.array_equal(a, b)


@pytest.mark.parametrize("N,K,TB,up", [(17408, 5120, 16, False), (5120, 17408, 16, False), (17408, 5120, 8, True),
                                        (17408, 5120, 33, False), (2048, 5120, 5, False), (4096, 5120, 33, True)])
def test_quant_gemm_sixteen_token_routes(miq, oracle, dev, N, K, TB, up):
    """miq_quant_gemm on the 16-token routes (the bounded split-K form for the first
    four shapes, the all-at-entry form for the last two): the output equals miq_xq +
    miq_i8_gemm bit for bit and x8 / xmeta / xsumq equal miq_xq's, over three calls
    in a row on the same buffers."""
    import torch
    print(f"quant gemm 16-token route N={N} K={K} TB={TB} up={up}", flush=True)
    wq = weights(miq, Q4_K, N, K, seed=N + K + TB)
    rng = np.random.default_rng(TB + K)
    x = to_dev(rng.standard_normal((TB, K)).astype(np.float32), dev)
    u = to_dev(rng.standard_normal((TB, K)).astype(np.float32), dev) if up else None
    wd = to_dev(wq, dev)
    ref = torch.full((TB, N), float("nan"), dtype=torch.float32, device=dev)
    act_r = miq.alloc_act(TB, K, dev)
    miq.xq(x, u, out=act_r)
    miq.i8_gemm(miq.make_seg(wd, Q4_K, K, N, act_r, ref, N), TB)
    for it in range(3):
        out = torch.full((TB, N), float("nan"), dtype=torch.float32, device=dev)
        act = miq.alloc_act(TB, K, dev)
        miq.quant_gemm(miq.make_seg(wd, Q4_K, K, N, act, out, N, x=x, act_up=u), TB)
        torch.cuda.synchronize()
        assert torch.equal(out.cpu().view(torch.int32), ref.cpu().view(torch.int32)), it
        for fa, fb in zip((act.x8, act.xmeta, act.xsumq), (act_r.x8, act_r.xmeta, act_r.xsumq)):
            assert torch.equal(fa.cpu(), fb.cpu()), it
    exp = oracle.gemm(Q4_K, wq, K, N, oracle.xq(x.cpu().numpy(), None if u is None else u.cpu().numpy()))
    assert max_rel(ref.cpu().numpy(), exp) <= TOL


def test_quant_gemm_multi_sixteen_tokens(miq, dev):
    """gate and up at 16 tokens in one miq_quant_gemm_multi call (one split-K launch
    over both): each segment equals miq_xq + its own miq_i8_gemm bit for bit, over
    two calls."""
    import torch
    N, K, TB = 17408, 5120, 16
    print("quant gemm multi 16 tokens", flush=True)
    ws = [to_dev(weights(miq, Q4_K, N, K, seed=s), dev) for s in (1, 2)]
    x = to_dev(np.random.default_rng(3).standard_normal((TB, K)).astype(np.float32), dev)
    act_r = miq.alloc_act(TB, K, dev)
    miq.xq(x, out=act_r)
    refs = []
    for w in ws:
        r = torch.empty((TB, N), dtype=torch.float32, device=dev)
        miq.i8_gemm(miq.make_seg(w, Q4_K, K, N, act_r, r, N), TB)
        refs.append(r)
    for it in range(2):
        act = miq.alloc_act(TB, K, dev)
        outs = [torch.full((TB, N), float("nan"), dtype=torch.float32, device=dev) for _ in ws]
        miq.quant_gemm_multi([miq.make_seg(w, Q4_K, K, N, act, o, N, x=x) for w, o in zip(ws, outs)], TB)
        torch.cuda.synchronize()
        for o, r in zip(outs, refs):
            assert torch.equal(o.cpu().view(torch.int32), r.cpu().view(torch.int32)), it
        assert torch.equal(act.x8.cpu(), act_r.x8.cpu())


@pytest.mark.parametrize("qt", [Q4_K, Q5_K, Q6_K, Q8_0])
@pytest.mark.parametrize("N,K", [(300, 1024), (1000, 5120), (77, 8192)])
def test_fused_one_token_quant_gemv(miq, oracle, dev, qt, N, K, switch):
    """miq_quant_gemm at one token quantizes inside the GEMV launch: the output
    equals the two-launch form (miq_xq, then the GEMV) bit for bit, the x8 /
    xmeta / xsumq it leaves equal miq_xq's, and the output meets the oracle.
    K = 5120 and 8192 take two rounds of 128 groups per workgroup."""
    import torch
    wq = weights(miq, qt, N, K, seed=K + N + qt)
    x = np.random.default_rng(K).standard_normal((1, K)).astype(np.float32)
    x[0, :32] = 0.0  # an all-zero group
    a, act_a = run_gemm(miq, dev, qt, wq, K, N, x, fused=True)
    switch("FUSED_QUANT", "0")
    b, act_b = run_gemm(miq, dev, qt, wq, K, N, x, fused=True)
    assert np.array_equal(a, b)
    for fa, fb in zip((act_a.x8, act_a.xmeta, act_a.xsumq), (act_b.x8, act_b.xmeta, act_b.xsumq)):
        assert torch.equal(fa.cpu(), fb.cpu())
    assert max_rel(a, oracle.gemm(qt, wq, K, N, oracle.xq(x))) <= TOL


# ------------------------------------------------------------------ the benchmark configurations
@pytest.mark.parametrize("N,K,TB", [(3584, 1024, 1), (17408, 5120, 1), (17408, 5120, 16), (5120, 17408, 1),
                                    (5120, 17408, 16)])
def test_config_shapes_q4k(miq, oracle, dev, N, K, TB):
    """configs 1 and 2 (FFN up/gate and down) at full size, every output checked."""
    wq = weights(miq, Q4_K, N, K, seed=N ^ K)
    x = np.random.default_rng(K).standard_normal((TB, K)).astype(np.float32)
    out, _ = run_gemm(miq, dev, Q4_K, wq, K, N, x)
    act = oracle.xq(x)
    exp = oracle.gemm(Q4_K, wq, K, N, act)
    assert max_rel(out, exp) <= TOL
    r = assert_elem(out, exp, elem_bound(oracle, Q4_K, wq, K, act))
    print(f"worst err / per-output bound {r:.3g}", flush=True)


@pytest.mark.parametrize("TB", [1, 16])
def test_config_shapes_q5k_qkv(miq, oracle, dev, TB):
    N, K = 7168, 5120
    wq = weights(miq, Q5_K, N, K, seed=55)
    x = np.random.default_rng(TB).standard_normal((TB, K)).astype(np.float32)
    out, _ = run_gemm(miq, dev, Q5_K, wq, K, N, x)
    act = oracle.xq(x)
    exp = oracle.gemm(Q5_K, wq, K, N, act)
    assert max_rel(out, exp) <= TOL
    assert_elem(out, exp, elem_bound(oracle, Q5_K, wq, K, act))


@pytest.mark.parametrize("TB", [1, 16])
def test_config_shapes_q6k_head(miq, oracle, dev, TB):
    """Q6_K output head 151936 x 5120: 8192 distinct rows tiled to full height, so
    row r must equal row r % 8192 (size-independent property) and the distinct
    rows match the oracle.  At 16 tokens the stream-K split points (and so the
    fp32 summation order) depend on a row's position: equal to the bound, not
    bit for bit."""
    N, K, D = 151936, 5120, 8192
    base = weights(miq, Q6_K, D, K, seed=66)
    wq = np.tile(base, (N // D + 1, 1))[:N]
    x = np.random.default_rng(TB + 6).standard_normal((TB, K)).astype(np.float32)
    out, _ = run_gemm(miq, dev, Q6_K, wq, K, N, x)
    act = oracle.xq(x)
    exp = oracle.gemm(Q6_K, base, K, D, act)
    assert max_rel(out[:, :D], exp) <= TOL
    assert_elem(out[:, :D], exp, elem_bound(oracle, Q6_K, base, K, act))
    tiled = np.tile(out[:, :D], (1, N // D + 1))[:, :N]
    if TB == 1:
        assert np.array_equal(out, tiled)
    else:
        assert max_rel(out, tiled) <= TOL


def test_config_prefill_rows_subset(miq, oracle, dev):
    """config 4 (Q4_K 17408 x 5120, 512-token chunk): all outputs computed, 384
    rows spread over the tensor checked against the oracle."""
    N, K, TB = 17408, 5120, 512
    wq = weights(miq, Q4_K, N, K, seed=4)
    x = np.random.default_rng(44).standard_normal((TB, K)).astype(np.float32)
    out, _ = run_gemm(miq, dev, Q4_K, wq, K, N, x)
    assert np.isfinite(out).all()
    rows = np.concatenate([np.arange(128), np.arange(8640, 8768), np.arange(N - 128, N)])
    act = oracle.xq(x)
    exp = oracle.gemm(Q4_K, wq[rows], K, len(rows), act)
    assert max_rel(out[:, rows], exp) <= TOL
    r = assert_elem(out[:, rows], exp, elem_bound(oracle, Q4_K, wq[rows], K, act))
    print(f"worst err / per-output bound {r:.3g}", flush=True)


# ------------------------------------------------------------------ Q8_0, any group count
def test_q80_odd_groups_golden(miq, dev):
    """Q8_0 rows of an odd number of 32-value groups (K % 64 == 32) against the
    compiled reference's native Q8_0 down (fixture gemm_q80_odd.npz)."""
    g = golden("gemm_q80_odd.npz")
    for k in g.files:
        if not k.startswith("out"):
            continue
        K, TB = (int(v) for v in k[3:].split("_"))
        w = g[f"w{K}"]
        print(f"q80 odd golden K={K} TB={TB}", flush=True)
        out, _ = run_gemm(miq, dev, Q8_0, w, K, w.shape[0], g[f"x{K}_{TB}"])
        assert max_rel(out, g[k]) <= TOL, k


@pytest.mark.parametrize("K", [96, 160, 352, 5152])
@pytest.mark.parametrize("TB", [1, 5, 16, 64])
def test_q80_odd_groups_vs_oracle(miq, oracle, dev, K, TB):
    """Any whole number of groups: every batch size (the decode and batched paths
    all route there), residual and alpha, the fused quantize call, and the int32
    group dots of the kernel's decoder (path 6) bit-exact."""
    import torch
    N = 300 if K < 1000 else 77
    print(f"q80 odd K={K} TB={TB}", flush=True)
    wq = weights(miq, Q8_0, N, K, seed=K + TB)
    rng = np.random.default_rng(K * 7 + TB)
    x = rng.standard_normal((TB, K)).astype(np.float32)
    res = rng.standard_normal((TB, N)).astype(np.float32)
    act = oracle.xq(x)
    out, a = run_gemm(miq, dev, Q8_0, wq, K, N, x, residual=res, alpha=0.5)
    assert max_rel(out, oracle.gemm(Q8_0, wq, K, N, act, residual=res, alpha=0.5)) <= TOL
    outf, _ = run_gemm(miq, dev, Q8_0, wq, K, N, x, fused=True)
    assert max_rel(outf, oracle.gemm(Q8_0, wq, K, N, act)) <= TOL
    d = miq.group_dots(to_dev(wq, dev), Q8_0, K, N, a, path=6)
    torch.cuda.synchronize()
    assert np.array_equal(d.cpu().numpy(), oracle.group_dots(Q8_0, wq, K, N, act[0]))


def test_q80_odd_groups_multi_and_refusals(miq, oracle, dev):
    """Two Q8_0 segments of K = 352 on one activation (each runs the any-group
    kernel), and the unit-walking decoders' dots paths refuse an odd group count."""
    import torch
    K, TB = 352, 3
    rng = np.random.default_rng(352)
    ws = [weights(miq, Q8_0, n, K, seed=n) for n in (100, 37)]
    x = rng.standard_normal((TB, K)).astype(np.float32)
    xd = to_dev(x, dev)
    act = miq.alloc_act(TB, K, dev)
    outs = [torch.empty((TB, n), dtype=torch.float32, device=dev) for n in (100, 37)]
    wds = [to_dev(w, dev) for w in ws]  # alive until the stream has run
    segs = [miq.make_seg(wd, Q8_0, K, n, act, o, n, x=xd) for wd, n, o in zip(wds, (100, 37), outs)]
    miq.quant_gemm_multi(segs, TB)
    torch.cuda.synchronize()
    for w, n, o in zip(ws, (100, 37), outs):
        assert max_rel(o.cpu().numpy(), oracle.gemm(Q8_0, w, K, n, oracle.xq(x))) <= TOL
    for path in (0, 1, 3, 4):
        with pytest.raises(miq.MiqError, match="path 6"):
            miq.group_dots(wds[0], Q8_0, K, 100, act, path=path)
