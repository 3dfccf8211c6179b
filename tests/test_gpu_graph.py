"""GPU: the GEMV/GEMM entry points captured in a HIP graph.

The library never allocates while the caller's stream captures: a warm-up call
of the same shape before capture sizes its buffers (the split-K scratch, the
prefill workspace, the u4 K-part sums), as the reference's engine runs a step
eagerly before recording its decode graph (src/engine/engine.cpp:4528-4583).
Each graph is replayed on new inputs copied in between, with the eager call
run between replays, and every replay must equal the eager result bit for bit;
the first also matches the oracle within the fp32 bound."""
import numpy as np
import pytest

from conftest import max_rel

pytestmark = pytest.mark.gpu
Q4_K, Q6_K = 12, 14
TOL = 1e-4


def _capture(step):
    import torch
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()  # warm-up: sizes every library buffer this shape needs
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    return g


@pytest.mark.parametrize("qt,N,K,TB,pf", [(Q4_K, 4096, 5120, 1, "1"), (Q4_K, 17408, 5120, 16, "1"),
                                          (Q4_K, 5120, 17408, 16, "1"), (Q6_K, 3000, 2048, 9, "1"),
                                          (Q4_K, 2048, 5120, 128, "1"), (Q4_K, 2048, 5120, 128, "2"),
                                          (Q6_K, 1000, 2048, 130, "2")])
def test_quant_gemm_graph_replay(miq, oracle, dev, qt, N, K, TB, pf, switch):
    """pf "2" forces the fp16 prefill GEMM (pre-pass, stream-K partials and
    counters) into the graph; "1" is the default dispatch."""
    import torch
    print(f"graph quant_gemm qt={qt} N={N} K={K} TB={TB} pf={pf}", flush=True)
    switch("PREFILL_FP16", pf)
    rng = np.random.default_rng(N + K + TB)
    wq = miq.quantize_rows(qt, (rng.standard_normal((N, K)) * 0.02).astype(np.float32))
    wd = torch.from_numpy(wq).to(dev)
    xs = [rng.standard_normal((TB, K)).astype(np.float32) for _ in range(3)]
    x = torch.from_numpy(xs[0]).to(dev)
    out = torch.empty((TB, N), dtype=torch.float32, device=dev)
    act = miq.alloc_act(TB, K, dev)
    seg = miq.make_seg(wd, qt, K, N, act, out, N, x=x)
    g = _capture(lambda: miq.quant_gemm(seg, TB))
    for i in range(3):
        x.copy_(torch.from_numpy(xs[i]))
        out.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        got = out.cpu().numpy().copy()
        miq.quant_gemm(seg, TB)
        torch.cuda.synchronize()
        assert np.array_equal(got, out.cpu().numpy()), f"replay {i} differs from the eager call"
        if i == 0:
            exp = oracle.gemm(qt, wq, K, N, oracle.xq(xs[0]))
            assert max_rel(got, exp) <= TOL


@pytest.mark.parametrize("N0,N1,K,TB", [(17408, 17408, 5120, 16), (700, 3000, 2048, 9), (64, 2048, 2048, 1)])
def test_quant_gemm_multi_graph_replay(miq, oracle, dev, N0, N1, K, TB):
    """two matrices on one activation (gate and up) captured as one
    miq_quant_gemm_multi: at 9 and 16 tokens one split-K launch with each
    segment's own slices and partials, at one token the fused GEMV"""
    import torch
    print(f"graph quant_gemm_multi N={N0},{N1} K={K} TB={TB}", flush=True)
    rng = np.random.default_rng(N0 + N1 + K + TB)
    wqs = [miq.quantize_rows(Q4_K, (rng.standard_normal((n, K)) * 0.02).astype(np.float32)) for n in (N0, N1)]
    wds = [torch.from_numpy(w).to(dev) for w in wqs]
    xs = [rng.standard_normal((TB, K)).astype(np.float32) for _ in range(3)]
    x = torch.from_numpy(xs[0]).to(dev)
    act = miq.alloc_act(TB, K, dev)
    outs = [torch.empty((TB, n), dtype=torch.float32, device=dev) for n in (N0, N1)]
    segs = [miq.make_seg(wd, Q4_K, K, n, act, o, n, x=x) for wd, n, o in zip(wds, (N0, N1), outs)]
    g = _capture(lambda: miq.quant_gemm_multi(segs, TB))
    for i in range(3):
        x.copy_(torch.from_numpy(xs[i]))
        for o in outs:
            o.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        got = [o.cpu().numpy().copy() for o in outs]
        miq.quant_gemm_multi(segs, TB)
        torch.cuda.synchronize()
        for gt, o in zip(got, outs):
            assert np.array_equal(gt, o.cpu().numpy()), f"replay {i} differs from the eager call"
        if i == 0:
            ax = oracle.xq(xs[0])
            for gt, wq, n in zip(got, wqs, (N0, N1)):
                assert max_rel(gt, oracle.gemm(Q4_K, wq, K, n, ax)) <= TOL


def test_w4_gemv_graph_replay(miq, oracle, dev):
    """the u4 GEMV at K = 17408 splits K across workgroups into a K-part buffer"""
    import torch
    N, K = 1024, 17408
    print(f"graph w4_gemv N={N} K={K}", flush=True)
    rng = np.random.default_rng(4)
    w = miq.quantize_rows(Q4_K, (rng.standard_normal((N, K)) * 0.02).astype(np.float32))
    st = miq.w4_pack(torch.from_numpy(w).to(dev), K, N)
    xs = [rng.standard_normal((1, K)).astype(np.float32) for _ in range(3)]
    x = torch.from_numpy(xs[0]).to(dev)
    act = miq.w4_act(x)
    out = torch.empty((N,), dtype=torch.float32, device=dev)

    def step():
        miq.w4_act(x, out=act)
        miq.w4_gemv(st, act, out)

    g = _capture(step)
    for i in range(3):
        x.copy_(torch.from_numpy(xs[i]))
        g.replay()
        torch.cuda.synchronize()
        got = out.cpu().numpy().copy()
        step()
        torch.cuda.synchronize()
        assert np.array_equal(got, out.cpu().numpy()), f"replay {i} differs from the eager call"
        if i == 0:
            exp = oracle.w4_gemv(oracle.w4_pack(w, K, N), oracle.w4_act(xs[0]))
            assert max_rel(got, exp) <= TOL


def test_graph_survives_workspace_growth(miq, oracle, dev, switch):
    """A graph of the fp16 prefill GEMM captured at 128 tokens keeps working after
    an eager call at 2048 tokens x K = 16384 has grown the library's prefill
    workspace (its fp16 activation alone is 64 MiB, more than any other shape in
    the suite): the buffer growth replaces is kept, not freed, so the replay
    reads and writes live memory and still equals the eager result."""
    import torch
    print("graph replay after workspace growth", flush=True)
    switch("PREFILL_FP16", "2")
    rng = np.random.default_rng(4242)
    K, TB, N = 2048, 128, 2048
    wq = miq.quantize_rows(Q4_K, (rng.standard_normal((N, K)) * 0.02).astype(np.float32))
    wd = torch.from_numpy(wq).to(dev)
    x = torch.from_numpy(rng.standard_normal((TB, K)).astype(np.float32)).to(dev)
    out = torch.empty((TB, N), dtype=torch.float32, device=dev)
    act = miq.alloc_act(TB, K, dev)
    seg = miq.make_seg(wd, Q4_K, K, N, act, out, N, x=x)
    g = _capture(lambda: miq.quant_gemm(seg, TB))
    KB, TBB, NB = 16384, 2048, 256
    wb = torch.from_numpy(miq.quantize_rows(Q4_K, (rng.standard_normal((NB, KB)) * 0.02).astype(np.float32))).to(dev)
    xb = torch.randn((TBB, KB), dtype=torch.float32, device=dev)
    out_b = torch.empty((TBB, NB), dtype=torch.float32, device=dev)
    seg_b = miq.make_seg(wb, Q4_K, KB, NB, miq.alloc_act(TBB, KB, dev), out_b, NB, x=xb)
    miq.quant_gemm(seg_b, TBB)  # eager, grows the workspace
    torch.cuda.synchronize()
    miq.quant_gemm(seg, TB)
    torch.cuda.synchronize()
    want = out.cpu().numpy().copy()
    for _ in range(2):
        out.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy(), want)
    assert max_rel(want, oracle.gemm(Q4_K, wq, K, N, oracle.xq(x.cpu().numpy()))) <= TOL
