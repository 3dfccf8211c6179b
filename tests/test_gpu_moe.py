"""GPU parity for the MoE path: router, CSR, grouped experts, weighted reduce."""
import numpy as np
import pytest

from conftest import golden, max_rel

pytestmark = pytest.mark.gpu

Q8_0, Q4_K, Q5_K, Q6_K = 8, 12, 13, 14
TOL = 1e-4


def to_dev(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def test_route_golden(miq, dev):
    import torch
    g = golden("moe.npz")
    top_k = int(g["dims"][2])
    lg = to_dev(g["logits"], dev)
    ids, wts = miq.moe_route(lg, top_k)
    torch.cuda.synchronize()
    assert np.array_equal(ids.cpu().numpy(), g["ids"])
    assert bits_equal(wts.cpu().numpy(), g["wts"])
    assert bits_equal(lg.cpu().numpy(), g["probs"])
    r = golden("moe_router.npz")
    lg = torch.zeros((5, 16), dtype=torch.float32, device=dev)
    ids, wts = miq.moe_route(lg, 4, x=to_dev(r["x"], dev), gate_inp=to_dev(r["gate_inp"], dev))
    torch.cuda.synchronize()
    assert np.array_equal(ids.cpu().numpy(), r["ids"])
    # logits from the router matrix: the serial double sum of the reference's
    # F32 router (moe.cpp:84-88), so probabilities and weights are its bits
    assert bits_equal(wts.cpu().numpy(), r["wts"])
    assert bits_equal(lg.cpu().numpy(), r["probs"])


def test_route_gate_inp_near_ties(miq, oracle, dev):
    """Router logits from a router matrix at config 5's size (16 tokens, 256 experts,
    n_embd 2048), with pairs of experts whose rows differ only in the last bits of
    one weight, so their logits tie or differ by one double rounding: ids, weights
    and probabilities equal the oracle's serial double sum bit for bit."""
    import torch
    rng = np.random.default_rng(2048)
    n_tok, n_expert, n_embd, top_k = 16, 256, 2048, 8
    gi = (rng.standard_normal((n_expert, n_embd)) * 0.02).astype(np.float32)
    for e in range(0, n_expert, 2):  # expert e+1: e's row with one weight nudged by an ulp
        gi[e + 1] = gi[e]
        k = rng.integers(n_embd)
        gi[e + 1, k] = np.nextafter(gi[e, k], np.float32(np.inf))
    x = rng.standard_normal((n_tok, n_embd)).astype(np.float32)
    lg = torch.zeros((n_tok, n_expert), dtype=torch.float32, device=dev)
    ids, wts = miq.moe_route(lg, top_k, x=to_dev(x, dev), gate_inp=to_dev(gi, dev))
    torch.cuda.synchronize()
    eids, ewts, eprobs = oracle.moe_route(np.zeros((n_tok, n_expert), np.float32), top_k, x=x, gate_inp=gi)
    assert np.array_equal(ids.cpu().numpy(), eids)
    assert bits_equal(wts.cpu().numpy(), ewts)
    assert bits_equal(lg.cpu().numpy(), eprobs)


def test_route_config5(miq, oracle, dev):
    """16 tokens, 256 experts, top-8 from N(0,1) logits (config 5)."""
    import torch
    lg = np.random.default_rng(5).standard_normal((16, 256)).astype(np.float32)
    ids, wts = miq.moe_route(to_dev(lg, dev), 8)
    torch.cuda.synchronize()
    eids, ewts, _ = oracle.moe_route(lg, 8)
    assert np.array_equal(ids.cpu().numpy(), eids)
    assert bits_equal(wts.cpu().numpy(), ewts)


@pytest.mark.parametrize("n_tok,n_expert,top_k", [
    (5, 8, 2), (9, 64, 8), (3, 100, 7), (6, 128, 4), (7, 200, 64), (16, 512, 8), (4, 600, 10)])
@pytest.mark.parametrize("ties", [False, True])
def test_route_sizes(miq, oracle, dev, n_tok, n_expert, top_k, ties):
    """Router on given logits across expert counts (the one-wave-per-token
    kernel up to 512 experts, the workgroup kernel above), with logits drawn
    from four values when `ties` so equal probabilities meet and the lower
    index must win."""
    import torch
    rng = np.random.default_rng(n_expert * 10 + top_k)
    lg = rng.standard_normal((n_tok, n_expert)).astype(np.float32)
    if ties:
        lg = np.round(lg).clip(-1, 2).astype(np.float32)
    d = to_dev(lg, dev)
    ids, wts = miq.moe_route(d, top_k)
    torch.cuda.synchronize()
    eids, ewts, eprobs = oracle.moe_route(lg, top_k)
    assert np.array_equal(ids.cpu().numpy(), eids)
    assert bits_equal(wts.cpu().numpy(), ewts)
    assert bits_equal(d.cpu().numpy(), eprobs)


def bits_equal(a, b):
    """fp32 arrays equal bit for bit (the router's softmax, sums and division
    follow the reference's order and its libm expf exactly)."""
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("n_pairs,n_expert", [(300, 40), (128, 256), (2000, 1500), (5000, 3000), (7, 2)])
def test_csr(miq, dev, n_pairs, n_expert):
    """CSR by expert: pairs of one expert in ascending pair order, offsets,
    the active list in id order; out-of-range ids skipped.  The shapes cover
    several lanes per pair for the ranks (128 pairs: 8), one lane (2000, 5000)
    and more experts than one scan pass takes (1500, 3000)."""
    import torch
    rng = np.random.default_rng(9 + n_pairs)
    ids = rng.integers(0, n_expert, n_pairs).astype(np.int32)
    ids[min(7, n_pairs - 1)] = -1  # out of range pairs are skipped
    if n_pairs > 20:
        ids[13] = n_expert
    off, pair, active, n_active = miq.moe_csr(to_dev(ids, dev), n_expert)
    torch.cuda.synchronize()
    off, pair, active, n_active = (t.cpu().numpy() for t in (off, pair, active, n_active))
    valid = np.nonzero((ids >= 0) & (ids < n_expert))[0]
    order = valid[np.argsort(ids[valid], kind="stable")]
    assert np.array_equal(pair[:len(order)], order)
    assert np.array_equal(off, np.concatenate([[0], np.cumsum(np.bincount(ids[valid], minlength=n_expert))]))
    act = np.unique(ids[valid])
    assert n_active[0] == len(act) and np.array_equal(active[:len(act)], act)


def run_experts(miq, dev, qt, gate, up, down, n_embd, n_ff, n_expert, x, top_k, ids, down_type=None):
    import torch
    bufs = (to_dev(gate, dev), to_dev(up, dev), to_dev(down, dev))  # alive until the stream has run
    m = miq.make_moe(*bufs, qt, n_embd, n_ff, n_expert, down_type=down_type)
    n_tok = x.shape[0]
    ws = miq.moe_workspace(m, n_tok, top_k, dev)
    acc = torch.full((n_tok * top_k, n_embd), float("nan"), dtype=torch.float32, device=dev)
    miq.moe_experts(m, to_dev(x, dev), top_k, to_dev(ids, dev), acc, ws)
    torch.cuda.synchronize()
    return acc.cpu().numpy()


def test_experts_golden(miq, dev):
    g = golden("moe.npz")
    n_tok, n_expert, top_k, n_embd, n_ff = (int(v) for v in g["dims"])
    acc = run_experts(miq, dev, Q4_K, g["gate"], g["up"], g["down"], n_embd, n_ff, n_expert, g["x"], top_k, g["ids"])
    assert max_rel(acc, g["acc"]) <= TOL


def test_reduce_golden(miq, dev):
    import torch
    g = golden("moe.npz")
    top_k = int(g["dims"][2])
    out = to_dev(g["out0"], dev)
    miq.moe_reduce(to_dev(g["acc"], dev), to_dev(g["wts"], dev), top_k, out)
    torch.cuda.synchronize()
    assert max_rel(out.cpu().numpy(), g["out"]) < 1e-6


@pytest.mark.parametrize("n_tok,top_k,n_embd", [(16, 8, 2048), (3, 9, 100), (5, 17, 33), (1, 1, 4)])
def test_reduce_exact(miq, oracle, dev, n_tok, top_k, n_embd):
    """The weighted reduce sums in double in pair order and adds once in fp32, so
    it equals the oracle's restatement of cpu_moe_reduce bit for bit: the
    four-wide form (n_embd % 4 == 0), the scalar form, and top_k past one batch
    of eight loads."""
    import torch
    rng = np.random.default_rng(n_tok * 100 + top_k)
    acc = rng.standard_normal((n_tok * top_k, n_embd)).astype(np.float32)
    wts = rng.random((n_tok, top_k)).astype(np.float32)
    out0 = rng.standard_normal((n_tok, n_embd)).astype(np.float32)
    out = to_dev(out0, dev)
    miq.moe_reduce(to_dev(acc, dev), to_dev(wts, dev), top_k, out)
    torch.cuda.synchronize()
    exp = oracle.moe_reduce(acc, wts, top_k, out0.copy())
    assert np.array_equal(out.cpu().numpy().view(np.uint32), exp.view(np.uint32))


@pytest.mark.parametrize("qt", [Q4_K, Q6_K])
def test_experts_config5(miq, oracle, dev, qt):
    """config 5: 256 experts, gate/up 512 x 2048, down 2048 x 512, 16 tokens, top-8."""
    n_tok, n_expert, top_k, n_embd, n_ff = 16, 256, 8, 2048, 512
    rng = np.random.default_rng(55)
    ids, wts, _ = oracle.moe_route(rng.standard_normal((n_tok, n_expert)).astype(np.float32), top_k)
    used = np.unique(ids)
    # only the routed experts' weights matter; the rest stay random bytes-free zeros
    gate = np.zeros((n_expert * n_ff, miq.row_bytes(qt, n_embd)), np.uint8)
    up = np.zeros_like(gate)
    down = np.zeros((n_expert * n_embd, miq.row_bytes(qt, n_ff)), np.uint8)
    for e in used:
        gate[e * n_ff:(e + 1) * n_ff] = miq.quantize_rows(qt, (rng.standard_normal((n_ff, n_embd)) * 0.02).astype(np.float32))
        up[e * n_ff:(e + 1) * n_ff] = miq.quantize_rows(qt, (rng.standard_normal((n_ff, n_embd)) * 0.02).astype(np.float32))
        down[e * n_embd:(e + 1) * n_embd] = miq.quantize_rows(qt, (rng.standard_normal((n_embd, n_ff)) * 0.02).astype(np.float32))
    x = rng.standard_normal((n_tok, n_embd)).astype(np.float32)
    acc = run_experts(miq, dev, qt, gate, up, down, n_embd, n_ff, n_expert, x, top_k, ids)
    exp = oracle.moe_experts(qt, gate, up, down, n_embd, n_ff, n_expert, x, top_k, ids)
    assert max_rel(acc, exp) <= TOL
    # The reference's grouped flow (moe.cpp:147-334) accumulates gate/up across blocks, the per-pair flow
    # block by block; a last-bit difference can move a requantised h code by one, so the two reference
    # flows themselves differ (about 6e-4 here).  The kernels are no farther from the grouped flow than
    # the per-pair flow is, to within the 1e-4 bound.
    grp = oracle.moe_experts_grouped(qt, gate, up, down, n_embd, n_ff, n_expert, x, top_k, ids)
    assert max_rel(acc, grp) <= max_rel(exp, grp) + TOL


@pytest.mark.parametrize("form", ["pipelined", "per_expert"])
@pytest.mark.parametrize("qt,dt,n_tok,n_expert,top_k,n_embd,n_ff", [
    (Q5_K, Q5_K, 7, 8, 3, 1536, 768),   # several pairs per expert, K = 24 units (not a power of two)
    (Q4_K, Q8_0, 5, 6, 2, 768, 192),    # Q8_0 down (q8_0_down_row): 3-unit down rows
    (Q4_K, Q8_0, 6, 10, 3, 768, 512),   # Q8_0 down rows of 8 units over 768 rows: two row sets per item
    (Q4_K, Q8_0, 5, 9, 2, 512, 352),    # Q8_0 down rows of 11 groups (n_ff % 64 == 32): the any-group kernel
    (Q4_K, Q4_K, 33, 4, 2, 256, 256),   # 66 pairs over 4 experts: long pair lists, 4-unit rows
    (Q6_K, Q6_K, 3, 300, 4, 4096, 256), # 64 units per gate row (the largest pipelined K)
    (Q4_K, Q4_K, 2, 5, 2, 8192, 256),   # gate K beyond the pipelined kernel: per-expert form either way
    (Q5_K, Q5_K, 5, 12, 2, 1024, 512),  # 8-unit down rows over 1024 rows: two row sets per work item
    (Q4_K, Q4_K, 2, 4, 1, 256, 256),    # top-1 over two tokens, the first unrouted: one pair, one active expert
])
def test_experts_shapes(miq, oracle, dev, switch, form, qt, dt, n_tok, n_expert, top_k, n_embd, n_ff):
    """Both grouped-GEMV forms against the reference per-pair path and its grouped
    path, with an out-of-range expert id (its acc rows are zero) and a duplicated one.
    The down bank may be Q8_0, the reference's native Q8_0 down (q4exp.cpp:442-467)."""
    if form == "per_expert":
        switch("MOE_GRP", "0")
    rng = np.random.default_rng(n_tok * 1000 + n_expert)
    ids = rng.integers(0, n_expert, size=(n_tok, top_k)).astype(np.int32)
    ids[0, 0] = n_expert        # unrouted pair
    ids[-1, -1] = ids[-1, 0]    # the same expert twice for one token
    used = np.unique(ids[(ids >= 0) & (ids < n_expert)])
    gate = np.zeros((n_expert * n_ff, miq.row_bytes(qt, n_embd)), np.uint8)
    up = np.zeros_like(gate)
    down = np.zeros((n_expert * n_embd, miq.row_bytes(dt, n_ff)), np.uint8)
    for e in used:
        gate[e * n_ff:(e + 1) * n_ff] = miq.quantize_rows(qt, (rng.standard_normal((n_ff, n_embd)) * 0.02).astype(np.float32))
        up[e * n_ff:(e + 1) * n_ff] = miq.quantize_rows(qt, (rng.standard_normal((n_ff, n_embd)) * 0.02).astype(np.float32))
        down[e * n_embd:(e + 1) * n_embd] = miq.quantize_rows(dt, (rng.standard_normal((n_embd, n_ff)) * 0.02).astype(np.float32))
    x = rng.standard_normal((n_tok, n_embd)).astype(np.float32)
    acc = run_experts(miq, dev, qt, gate, up, down, n_embd, n_ff, n_expert, x, top_k, ids.reshape(-1), down_type=dt)
    exp = oracle.moe_experts(qt, gate, up, down, n_embd, n_ff, n_expert, x, top_k, ids.reshape(-1), down_type=dt)
    assert not np.any(acc[0]), "unrouted pair must give zeros"
    assert max_rel(acc, exp) <= TOL
    grp = oracle.moe_experts_grouped(qt, gate, up, down, n_embd, n_ff, n_expert, x, top_k, ids.reshape(-1),
                                     down_type=dt)
    assert max_rel(acc, grp) <= max_rel(exp, grp) + TOL


@pytest.mark.parametrize("form", ["pipelined", "per_expert"])
def test_experts_no_active_expert(miq, dev, switch, form):
    """Every pair unrouted (ids past the expert count): no expert is active, both
    grouped kernels find no work item, and every acc row is zero."""
    import torch
    if form == "per_expert":
        switch("MOE_GRP", "0")
    n_tok, n_expert, top_k, n_embd, n_ff = 3, 4, 2, 256, 256
    gate = np.zeros((n_expert * n_ff, miq.row_bytes(Q4_K, n_embd)), np.uint8)
    down = np.zeros((n_expert * n_embd, miq.row_bytes(Q4_K, n_ff)), np.uint8)
    ids = np.full(n_tok * top_k, n_expert, np.int32)
    x = np.random.default_rng(5).standard_normal((n_tok, n_embd)).astype(np.float32)
    acc = run_experts(miq, dev, Q4_K, gate, gate, down, n_embd, n_ff, n_expert, x, top_k, ids)
    assert not np.any(acc)


def ws_h(ws, n_tok, top_k, n_embd, n_ff, n_expert):
    """The fp32 h = silu(g)*u rows [pairs][n_ff] inside the experts workspace (the
    region order of moe_ws_layout in csrc/miq_moe.hip: x8, xmeta, xsumq, off, pair,
    active, n_active, then h; each region 256-byte aligned)."""
    a = lambda b: (b + 255) // 256 * 256
    np_ = n_tok * top_k
    o = (a(n_embd * n_tok) + a(n_embd // 32 * n_tok * 16) + a(n_embd // 32 * n_tok * 8) + a(4 * (n_expert + 1))
         + a(4 * np_) + a(4 * n_expert) + a(4))
    return ws[o:o + 4 * n_ff * np_].view(dtype=__import__("torch").float32).reshape(np_, n_ff)


@pytest.mark.parametrize("form", ["pipelined", "per_expert"])
@pytest.mark.parametrize("qt,n_tok,n_expert,top_k,n_embd,n_ff", [
    (Q4_K, 16, 64, 8, 2048, 512),
    (Q5_K, 9, 24, 4, 1024, 256),
    (Q6_K, 7, 16, 4, 2048, 512),
    (Q4_K, 4, 8, 2, 8192, 256),   # K beyond the pipelined kernel: per-expert form either way
])
def test_experts_h_bit_exact(miq, oracle, dev, switch, form, qt, n_tok, n_expert, top_k, n_embd, n_ff):
    """gate/up run in the reference's fp32 order (i8_row: per group
    fma(d*sc, wd, -(dmin*m)*xsum), block partials fma(xm, T, acc) over the groups
    in order, then the blocks in order), so h = silu(g)*u -- the value that is
    requantised for the down projection -- is the reference per-pair flow's
    (cpu_moe_experts_i8) bit for bit, and the expert outputs differ from it only
    by the down projection's fp32 association."""
    import torch
    if form == "per_expert":
        switch("MOE_GRP", "0")
    rng = np.random.default_rng(n_embd * 7 + n_expert)
    ids, _, _ = oracle.moe_route(rng.standard_normal((n_tok, n_expert)).astype(np.float32), top_k)
    used = np.unique(ids)
    gate = np.zeros((n_expert * n_ff, miq.row_bytes(qt, n_embd)), np.uint8)
    up = np.zeros_like(gate)
    down = np.zeros((n_expert * n_embd, miq.row_bytes(qt, n_ff)), np.uint8)
    for e in used:
        gate[e * n_ff:(e + 1) * n_ff] = miq.quantize_rows(qt, (rng.standard_normal((n_ff, n_embd)) * 0.02).astype(np.float32))
        up[e * n_ff:(e + 1) * n_ff] = miq.quantize_rows(qt, (rng.standard_normal((n_ff, n_embd)) * 0.02).astype(np.float32))
        down[e * n_embd:(e + 1) * n_embd] = miq.quantize_rows(qt, (rng.standard_normal((n_embd, n_ff)) * 0.02).astype(np.float32))
    x = rng.standard_normal((n_tok, n_embd)).astype(np.float32)
    bufs = (to_dev(gate, dev), to_dev(up, dev), to_dev(down, dev))
    m = miq.make_moe(*bufs, qt, n_embd, n_ff, n_expert)
    ws = miq.moe_workspace(m, n_tok, top_k, dev)
    acc = torch.empty((n_tok * top_k, n_embd), dtype=torch.float32, device=dev)
    miq.moe_experts(m, to_dev(x, dev), top_k, to_dev(ids.reshape(-1), dev), acc, ws)
    torch.cuda.synchronize()
    exp, h_exp = oracle.moe_experts(qt, gate, up, down, n_embd, n_ff, n_expert, x, top_k, ids.reshape(-1), want_h=True)
    h = ws_h(ws, n_tok, top_k, n_embd, n_ff, n_expert).cpu().numpy()
    assert np.array_equal(h.view(np.uint32), h_exp.view(np.uint32)), f"h differs in {(h != h_exp).sum()} values"
    assert max_rel(acc.cpu().numpy(), exp) <= 1e-5


def test_experts_q8_0_gate_up_refused(miq, dev):
    """The reference's integer expert path (i8_row, i8.cpp:157-190) serves no Q8_0
    gate/up banks: the call returns MIQ_UNSUPPORTED before any launch and leaves acc alone."""
    import torch
    n_tok, n_expert, top_k, n_embd, n_ff = 6, 10, 3, 640, 512
    gate = torch.zeros(n_expert * n_ff * miq.row_bytes(Q8_0, n_embd), dtype=torch.uint8, device=dev)
    down = torch.zeros(n_expert * n_embd * miq.row_bytes(Q8_0, n_ff), dtype=torch.uint8, device=dev)
    m = miq.make_moe(gate, gate, down, Q8_0, n_embd, n_ff, n_expert)
    ws = miq.moe_workspace(m, n_tok, top_k, dev)
    acc = torch.full((n_tok * top_k, n_embd), 7.0, dtype=torch.float32, device=dev)
    x = torch.zeros((n_tok, n_embd), dtype=torch.float32, device=dev)
    ids = torch.zeros(n_tok * top_k, dtype=torch.int32, device=dev)
    with pytest.raises(miq.MiqError) as ei:
        miq.moe_experts(m, x, top_k, ids, acc, ws)
    assert "-> 1:" in str(ei.value) and "Q8_0 gate/up" in str(ei.value)  # MIQ_UNSUPPORTED
    torch.cuda.synchronize()
    assert bool((acc == 7.0).all())


def test_moe_step_graph_replay(miq, oracle, dev):
    """route + experts + reduce captured once in a HIP graph: every replay, on
    new activations copied in between, equals the eager step bit for bit
    (the eager step runs between replays), and the first equals the oracle."""
    import torch
    qt, n_tok, n_expert, top_k, n_embd, n_ff = Q4_K, 4, 16, 2, 512, 256
    rng = np.random.default_rng(77)
    gate = miq.quantize_rows(qt, (rng.standard_normal((n_expert * n_ff, n_embd)) * 0.02).astype(np.float32))
    up = miq.quantize_rows(qt, (rng.standard_normal((n_expert * n_ff, n_embd)) * 0.02).astype(np.float32))
    down = miq.quantize_rows(qt, (rng.standard_normal((n_expert * n_embd, n_ff)) * 0.02).astype(np.float32))
    bufs = (to_dev(gate, dev), to_dev(up, dev), to_dev(down, dev))
    m = miq.make_moe(*bufs, qt, n_embd, n_ff, n_expert)
    ws = miq.moe_workspace(m, n_tok, top_k, dev)
    xs = [rng.standard_normal((n_tok, n_embd)).astype(np.float32) for _ in range(3)]
    lgs = [rng.standard_normal((n_tok, n_expert)).astype(np.float32) for _ in range(3)]
    x = to_dev(xs[0], dev)
    logits0 = to_dev(lgs[0], dev)
    logits = torch.empty_like(logits0)
    acc = torch.empty((n_tok * top_k, n_embd), dtype=torch.float32, device=dev)
    out = torch.empty((n_tok, n_embd), dtype=torch.float32, device=dev)

    def step():
        logits.copy_(logits0)
        ids, w = miq.moe_route(logits, top_k)
        miq.moe_experts(m, x, top_k, ids, acc, ws)
        out.zero_()
        miq.moe_reduce(acc, w, top_k, out)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    for i in range(3):
        x.copy_(torch.from_numpy(xs[i]))
        logits0.copy_(torch.from_numpy(lgs[i]))
        g.replay()
        torch.cuda.synchronize()
        got = out.cpu().numpy().copy()
        step()
        torch.cuda.synchronize()
        assert np.array_equal(got, out.cpu().numpy()), f"replay {i} differs from the eager step"
        if i == 0:
            ids, wts, _ = oracle.moe_route(lgs[0], top_k)
            a = oracle.moe_experts(qt, gate, up, down, n_embd, n_ff, n_expert, xs[0], top_k, ids)
            exp = oracle.moe_reduce(a, wts, top_k, np.zeros((n_tok, n_embd), np.float32))
            assert max_rel(got, exp) <= TOL
