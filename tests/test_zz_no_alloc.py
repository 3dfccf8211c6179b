"""GPU: miq_i8_gemm_noalloc (the split-K scratch in the library's static
device array) against miq_i8_gemm on the same inputs: bit-identical outputs,
on consecutive calls of shrinking size, and a clean refusal for shapes that
need more than the static scratch or a workspace."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu
Q4_K, Q5_K, Q6_K = 12, 13, 14


def _case(miq, dev, qt, N, K, TB, seed):
    import torch
    rng = np.random.default_rng(seed)
    wq = miq.quantize_rows(qt, (rng.standard_normal((N, K)) * 0.02).astype(np.float32))
    w = torch.from_numpy(wq).to(dev)
    x = torch.from_numpy(rng.standard_normal((TB, K)).astype(np.float32)).to(dev)
    act = miq.xq(x)
    outs = []
    for fn in (miq.i8_gemm, miq.i8_gemm_noalloc):
        out = torch.full((TB, N), float("nan"), dtype=torch.float32, device=dev)
        fn(miq.make_seg(w, qt, K, N, act, out, N), TB)
        torch.cuda.synchronize()
        outs.append(out.cpu().numpy())
    return outs


def test_noalloc_matches_i8_gemm_twice(miq, dev):
    """two calls in a row, the second smaller: each equals miq_i8_gemm bit for bit
    (the split-K 16-token kernel, partials and counters in the static array)"""
    for qt, N, K, TB, seed in ((Q4_K, 17408, 5120, 16, 1), (Q5_K, 2048, 5120, 7, 2)):
        print(f"noalloc qt={qt} N={N} K={K} TB={TB}", flush=True)
        ref, got = _case(miq, dev, qt, N, K, TB, seed)
        assert not np.isnan(ref).any()
        assert np.array_equal(ref.view(np.uint32), got.view(np.uint32)), (qt, N, K, TB)


def test_noalloc_cu_resident_k_parts(miq, dev, switch):
    """the CU-resident form with K parts meeting in the static scratch, then a smaller call"""
    switch("M16_FORM", 3)
    for qt, N, K, TB, seed in ((Q4_K, 2048, 17408, 16, 3), (Q6_K, 512, 12288, 3 + 2, 4)):
        print(f"noalloc cu-form qt={qt} N={N} K={K} TB={TB}", flush=True)
        ref, got = _case(miq, dev, qt, N, K, TB, seed)
        assert np.array_equal(ref.view(np.uint32), got.view(np.uint32)), (qt, N, K, TB)


def test_noalloc_refuses_prefill(miq, dev, switch):
    """a prefill-sized Q4_K batch on the fp16 prefill GEMM (PREFILL_FP16=2 takes
    it at this size) needs a workspace: MIQ_UNSUPPORTED with a message, nothing
    launched"""
    import torch
    switch("PREFILL_FP16", "2")
    N, K, TB = 256, 1024, 64
    w = torch.zeros((N, miq.row_bytes(Q4_K, K)), dtype=torch.uint8, device=dev)
    act = miq.alloc_act(TB, K, dev)
    out = torch.full((TB, N), 7.0, dtype=torch.float32, device=dev)
    with pytest.raises(miq.MiqError, match="workspace"):
        miq.i8_gemm_noalloc(miq.make_seg(w, Q4_K, K, N, act, out, N), TB)
    torch.cuda.synchronize()
    assert (out.cpu().numpy() == 7.0).all()
