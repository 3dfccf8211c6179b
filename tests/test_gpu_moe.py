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
    assert max_rel(wts.cpu().numpy(), g["wts"]) < 1e-6
    assert max_rel(lg.cpu().numpy(), g["probs"]) < 1e-6
    r = golden("moe_router.npz")
    lg = torch.zeros((5, 16), dtype=torch.float32, device=dev)
    ids, wts = miq.moe_route(lg, 4, x=to_dev(r["x"], dev), gate_inp=to_dev(r["gate_inp"], dev))
    torch.cuda.synchronize()
    assert np.array_equal(ids.cpu().numpy(), r["ids"])
    assert max_rel(wts.cpu().numpy(), r["wts"]) < 1e-6


def test_route_config5(miq, oracle, dev):
    """16 tokens, 256 experts, top-8 from N(0,1) logits (config 5)."""
    import torch
    lg = np.random.default_rng(5).standard_normal((16, 256)).astype(np.float32)
    ids, wts = miq.moe_route(to_dev(lg, dev), 8)
    torch.cuda.synchronize()
    eids, ewts, _ = oracle.moe_route(lg, 8)
    assert np.array_equal(ids.cpu().numpy(), eids)
    assert max_rel(wts.cpu().numpy(), ewts) < 1e-6


def test_csr(miq, dev):
    import torch
    rng = np.random.default_rng(9)
    ids = rng.integers(0, 40, 300).astype(np.int32)
    ids[7] = -1  # out of range pairs are skipped
    off, pair, active, n_active = miq.moe_csr(to_dev(ids, dev), 40)
    torch.cuda.synchronize()
    off, pair, active, n_active = (t.cpu().numpy() for t in (off, pair, active, n_active))
    valid = np.nonzero(ids >= 0)[0]
    order = valid[np.argsort(ids[valid], kind="stable")]
    assert np.array_equal(pair[:len(order)], order)
    assert np.array_equal(off, np.concatenate([[0], np.cumsum(np.bincount(ids[valid], minlength=40))]))
    act = np.unique(ids[valid])
    assert n_active[0] == len(act) and np.array_equal(active[:len(act)], act)


def run_experts(miq, dev, qt, gate, up, down, n_embd, n_ff, n_expert, x, top_k, ids):
    import torch
    bufs = (to_dev(gate, dev), to_dev(up, dev), to_dev(down, dev))  # alive until the stream has run
    m = miq.make_moe(*bufs, qt, n_embd, n_ff, n_expert)
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
