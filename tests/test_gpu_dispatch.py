"""GPU parity across the batch-size dispatch: every type at token counts on both
sides of each cut-off the library routes by -- the GEMV (1..3 tokens), the
16-token int8-MFMA GEMM (4..47), the prefill GEMMs (48 and up, where the
cost model picks between the fp16 GEMM and the 16-token kernel) -- on a shape
whose rows leave partial tiles everywhere (N = 260) and K = 2304 (nine blocks:
odd slice counts).  Each output is checked against the oracle (the normwise
1e-4 bound and the per-output summation-order bound), and the fused entry point
(miq_quant_gemm) must equal miq_xq + miq_i8_gemm bit for bit."""
import numpy as np
import pytest

from conftest import assert_elem, elem_bound, max_rel

pytestmark = pytest.mark.gpu

Q8_0, Q4_K, Q5_K, Q6_K = 8, 12, 13, 14
TOL = 1e-4
N, K = 260, 2304
TBS = [1, 2, 3, 4, 5, 15, 16, 17, 31, 32, 33, 46, 47, 48, 49, 63, 64, 65, 127, 128, 129, 200]


@pytest.fixture(scope="module")
def banks(miq):
    out = {}
    for qt in (Q4_K, Q5_K, Q6_K, Q8_0):
        rng = np.random.default_rng(1000 + qt)
        out[qt] = miq.quantize_rows(qt, (rng.standard_normal((N, K)) * 0.02).astype(np.float32))
    return out


@pytest.mark.parametrize("qt", [Q4_K, Q5_K, Q6_K, Q8_0])
@pytest.mark.parametrize("TB", TBS)
def test_dispatch_sweep_vs_oracle(miq, oracle, dev, banks, qt, TB):
    import torch
    print(f"dispatch sweep type={qt} TB={TB} N={N} K={K}", flush=True)
    wq = banks[qt]
    wd = torch.from_numpy(wq).to(dev)
    x = np.random.default_rng(TB * 31 + qt).standard_normal((TB, K)).astype(np.float32)
    xd = torch.from_numpy(x).to(dev)
    plain = torch.full((TB, N), float("nan"), dtype=torch.float32, device=dev)
    act = miq.alloc_act(TB, K, dev)
    miq.xq(xd, out=act)
    seg = miq.make_seg(wd, qt, K, N, act, plain, N)
    if TB == 1:
        miq.i8_gemv(seg)
    else:
        miq.i8_gemm(seg, TB)
    fused = torch.full((TB, N), float("nan"), dtype=torch.float32, device=dev)
    act2 = miq.alloc_act(TB, K, dev)
    miq.quant_gemm(miq.make_seg(wd, qt, K, N, act2, fused, N, x=xd), TB)
    torch.cuda.synchronize()
    assert torch.equal(plain.cpu().view(torch.int32), fused.cpu().view(torch.int32))
    a = oracle.xq(x)
    exp = oracle.gemm(qt, wq, K, N, a)
    got = plain.cpu().numpy()
    assert max_rel(got, exp) <= TOL
    assert_elem(got, exp, elem_bound(oracle, qt, wq, K, a, 1.0), residual=None)
