"""GPU: several output segments of one activation in one call
(miq_i8_gemv_multi / miq_quant_gemm_multi, the reference's
i8_row_gemv_multi and i8_grp_quant_gemv_launch).  Every segment must equal
the single-segment call bit for bit (one launch or several) and the oracle
within the fp32 bound."""
import numpy as np
import pytest

from conftest import max_rel

pytestmark = pytest.mark.gpu
Q8_0, Q4_K, Q5_K, Q6_K = 8, 12, 13, 14
TOL = 1e-4


def _segs(miq, dev, specs, K, TB, seed):
    """specs: [(qtype, N, with_residual, alpha)]"""
    import torch
    rng = np.random.default_rng(seed)
    x = torch.from_numpy(rng.standard_normal((TB, K)).astype(np.float32)).to(dev)
    act = miq.alloc_act(TB, K, dev)
    out = []
    for qt, N, with_res, alpha in specs:
        wq = miq.quantize_rows(qt, (rng.standard_normal((N, K)) * 0.02).astype(np.float32))
        w = torch.from_numpy(wq).to(dev)
        res = torch.from_numpy(rng.standard_normal((TB, N)).astype(np.float32)).to(dev) if with_res else None
        o = torch.full((TB, N), float("nan"), dtype=torch.float32, device=dev)
        out.append(dict(qt=qt, N=N, wq=wq, w=w, res=res, alpha=alpha, out=o,
                        seg=miq.make_seg(w, qt, K, N, act, o, N, residual=res, alpha=alpha, x=x)))
    return x, act, out


@pytest.mark.parametrize("fused", [True, False])
@pytest.mark.parametrize("specs,K,TB", [
    ([(Q4_K, 17408, False, 1.0), (Q4_K, 17408, False, 1.0)], 5120, 1),   # gate + up of configs[1]
    ([(Q4_K, 37, True, 0.5), (Q4_K, 1000, False, 1.0), (Q4_K, 4096, True, 2.0)], 2048, 1),
    ([(Q5_K, 300, False, 1.0), (Q5_K, 64, True, 1.0)], 1024, 2),
    ([(Q6_K, 129, False, 1.0), (Q6_K, 77, False, 0.25)], 2816, 3),
    ([(Q8_0, 200, True, 1.0), (Q8_0, 33, False, 1.0)], 640, 1),
    ([(Q4_K, 500, False, 1.0), (Q6_K, 300, True, 1.0)], 2048, 1),       # mixed types: one launch each
    # past the GEMV: one split-K launch with each segment's own tiles and slices
    ([(Q4_K, 700, True, 1.0), (Q4_K, 900, False, 1.0)], 2048, 16),
    ([(Q4_K, 17408, False, 1.0), (Q4_K, 17408, False, 1.0)], 5120, 16),  # gate + up of configs[1]
    ([(Q4_K, 300, False, 1.0), (Q4_K, 5000, True, 0.5), (Q4_K, 129, False, 1.0)], 3072, 20),
    ([(Q5_K, 1000, True, 1.0), (Q5_K, 64, False, 2.0)], 1280, 9),
    ([(Q6_K, 2000, False, 1.0), (Q6_K, 333, True, 1.0)], 2816, 16),
    ([(Q8_0, 500, False, 1.0), (Q8_0, 77, True, 1.0), (Q8_0, 4000, False, 1.0)], 1600, 33),
    ([(Q4_K, 500, False, 1.0), (Q5_K, 300, True, 1.0)], 2048, 16),      # mixed types: one launch each
    ([(Q4_K, 640, False, 1.0), (Q4_K, 129, True, 1.0)], 1024, 4),       # the split-K kernel's smallest batch
    ([(Q6_K, 333, False, 1.0), (Q6_K, 1024, False, 1.0)], 2048, 47),    # its largest (three token tiles)
    ([(Q4_K, 2048, False, 1.0), (Q4_K, 512, False, 1.0)], 2048, 64),    # prefill sizes: one GEMM per segment
])
def test_multi_matches_single(miq, oracle, dev, specs, K, TB, fused):
    import torch
    print(f"multi fused={fused} K={K} TB={TB} segs={[(s[0], s[1]) for s in specs]}", flush=True)
    x, act, segs = _segs(miq, dev, specs, K, TB, seed=K + TB + len(specs))
    if fused:
        miq.quant_gemm_multi([s["seg"] for s in segs], TB)
    else:
        miq.xq(x, out=act)
        miq.i8_gemv_multi([s["seg"] for s in segs], TB)
    torch.cuda.synchronize()
    got = [s["out"].cpu().numpy().copy() for s in segs]
    ax = oracle.xq(x.cpu().numpy())
    for s, g in zip(segs, got):
        s["out"].fill_(float("nan"))
        if fused:
            miq.quant_gemm(s["seg"], TB)
        else:
            miq.i8_gemm(s["seg"], TB)
        torch.cuda.synchronize()
        assert np.array_equal(g.view(np.uint32), s["out"].cpu().numpy().view(np.uint32)), (s["qt"], s["N"])
        res = None if s["res"] is None else s["res"].cpu().numpy()
        exp = oracle.gemm(s["qt"], s["wq"], K, s["N"], ax, residual=res, alpha=s["alpha"])
        assert max_rel(g, exp) <= TOL
    # the shared activation the fused call wrote equals cpu_xq's
    if fused:
        assert np.array_equal(act.x8.cpu().numpy(), ax[0])
        assert np.array_equal(act.xsumq.cpu().numpy(), ax[2])


def test_multi_rejects_mismatched_k(miq, dev):
    import torch
    x, act, segs = _segs(miq, dev, [(Q4_K, 64, False, 1.0)], 512, 1, seed=1)
    _, _, segs2 = _segs(miq, dev, [(Q4_K, 64, False, 1.0)], 1024, 1, seed=2)
    with pytest.raises(miq.MiqError, match="K="):
        miq.i8_gemv_multi([segs[0]["seg"], segs2[0]["seg"]], 1)
