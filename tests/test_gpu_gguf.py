"""GPU: GGUF tensors read by miq_gguf_open, uploaded to HBM by miq_gguf_upload
and fed to the GEMV/GEMM kernels.  The uploaded bytes must equal the mapping's
(bit-exact), padding between split shards arrives as zeros, and the kernels'
outputs on the uploaded tensors match the oracle on the file's bytes."""
import numpy as np
import pytest

import gguf_synth as gs
from conftest import max_rel

pytestmark = pytest.mark.gpu

F32_T, Q4_K, Q6_K = 0, 12, 14


def make_split(miq, tmp_path, N=256, K=1024):
    rng = np.random.default_rng(11)
    stem = str(tmp_path / "m")
    Wa = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    Wb = (rng.standard_normal((N // 2, K)) * 0.02).astype(np.float32)
    qa, qb = miq.quantize_rows(Q4_K, Wa), miq.quantize_rows(Q6_K, Wb)
    shard = [
        [("split.no", gs.U16, 0), ("split.count", gs.U16, 2)],
        [("split.no", gs.U16, 1), ("split.count", gs.U16, 2)],
    ]
    raw0, _ = gs.build(shard[0], [("ffn_up", (K, N), Q4_K, qa.tobytes())])
    raw1, _ = gs.build(shard[1], [("ffn_down", (K, N // 2), Q6_K, qb.tobytes()),
                                  ("norm", (K,), F32_T, np.ones(K, np.float32).tobytes())])
    for i, raw in enumerate((raw0, raw1)):
        with open(gs.shard_name(stem, i + 1, 2), "wb") as fh:
            fh.write(raw)
    return gs.shard_name(stem, 1, 2), {"ffn_up": (qa, Q4_K, N), "ffn_down": (qb, Q6_K, N // 2)}, K


@pytest.mark.parametrize("TB", [1, 16, 64])
def test_uploaded_tensors_feed_the_kernels(miq, oracle, dev, tmp_path, TB):
    import torch
    path, expect, K = make_split(miq, tmp_path)
    print(f"gguf upload+gemm TB={TB}", flush=True)
    with miq.GgufFile(path) as f:
        for name, (q, qt, N) in expect.items():
            t = f.find(name)
            assert t is not None and t.type == qt and t.n_rows == N
            wd = f.upload_tensor(t, dev)
            torch.cuda.synchronize()
            assert np.array_equal(wd.cpu().numpy(), q), name
            rng = np.random.default_rng(TB)
            x = rng.standard_normal((TB, K)).astype(np.float32)
            xd = torch.from_numpy(x).to(dev)
            out = torch.full((TB, N), float("nan"), dtype=torch.float32, device=dev)
            act = miq.alloc_act(TB, K, dev)
            seg = miq.make_seg(wd, qt, K, N, act, out, N, x=xd)
            miq.quant_gemm(seg, TB)
            torch.cuda.synchronize()
            exp = oracle.gemm(qt, f.tensor_bytes(t).reshape(N, -1), K, N, oracle.xq(x))
            assert max_rel(out.cpu().numpy(), exp) < 1e-4, name


def test_upload_whole_mapping_with_padding(miq, dev, tmp_path):
    import torch
    path, _, _ = make_split(miq, tmp_path)
    with miq.GgufFile(path) as f:
        buf = torch.full((f.map_size,), 0x5A, dtype=torch.uint8, device=dev)
        f.upload(buf, 0, f.map_size)
        got = buf.cpu().numpy()
        pos = 0
        for i, (base, size, _) in enumerate(f.shards):
            off = base - f.map_base
            assert np.all(got[pos:off] == 0)  # padding between shards
            with open(gs.shard_name(path[: -len("-00001-of-00002.gguf")], i + 1, 2), "rb") as fh:
                assert got[off:off + size].tobytes() == fh.read()
            pos = off + size
        assert np.all(got[pos:] == 0)
        # an unaligned sub-range that crosses the gap
        a, b = f.shards[0][1] - 37, f.shards[1][0] - f.map_base + 91
        sub = torch.zeros(b - a, dtype=torch.uint8, device=dev)
        f.upload(sub, a, b - a)
        assert np.array_equal(sub.cpu().numpy(), got[a:b])


def test_upload_larger_than_staging(miq, dev, tmp_path):
    """More than two 32 MiB staging chunks: the double buffer is reused."""
    import torch
    n = (32 << 20) * 2 + 12345
    data = np.random.default_rng(2).integers(0, 256, n, dtype=np.uint8)
    raw, _ = gs.build([], [("blob", (n // 4,), F32_T, data[: n // 4 * 4].tobytes())])
    p = str(tmp_path / "big.gguf")
    with open(p, "wb") as fh:
        fh.write(raw)
    with miq.GgufFile(p) as f:
        t = f.find("blob")
        d = torch.empty(t.nbytes, dtype=torch.uint8, device=dev)
        f.upload(d, t.map_offset, t.nbytes)
        assert np.array_equal(d.cpu().numpy(), data[: n // 4 * 4])
