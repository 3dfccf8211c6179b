"""Write the golden fixtures under tests/golden/ from sycl-infer's own CPU kernels.

Runs in the build container only (it needs oracle/_ref/libsiref.so, compiled
from the reference sources by `make -C oracle ref`).  The fixtures are data:
seeded inputs and the reference's outputs.  Weight blocks are random bytes with
a bounded f16 scale (every byte pattern is a valid block), so the fixtures do
not depend on this repository's encoder.

    python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "..", "..", "oracle"))
from oracle import Q4_K, Q5_K, Q6_K, Q8_0, Ref, row_bytes  # noqa: E402

NAMES = {Q4_K: "q4k", Q5_K: "q5k", Q6_K: "q6k", Q8_0: "q80"}


def f16_bits(rng, n, lo, hi):
    """random normal f16 values in [lo, hi) as bit patterns"""
    v = rng.uniform(lo, hi, n).astype(np.float16)
    return v.view(np.uint16)


def random_blocks(rng, qtype, n_rows, K):
    """random bytes with sane f16 super-scales (d, dmin for Q4_K/Q5_K; d for Q6_K/Q8_0)"""
    rb = row_bytes(qtype, K)
    w = rng.integers(0, 256, (n_rows, rb), dtype=np.uint8)
    if qtype == Q8_0:
        blk = w.reshape(n_rows, -1, 34)
        blk[:, :, 0:2] = f16_bits(rng, blk.shape[0] * blk.shape[1], 1e-4, 4e-3).reshape(n_rows, -1, 1).view(np.uint8)
    elif qtype == Q6_K:
        blk = w.reshape(n_rows, -1, 210)
        blk[:, :, 208:210] = f16_bits(rng, blk.shape[0] * blk.shape[1], 1e-5, 2e-4).reshape(n_rows, -1, 1).view(np.uint8)
    else:
        bb = 144 if qtype == Q4_K else 176
        blk = w.reshape(n_rows, -1, bb)
        nb = blk.shape[0] * blk.shape[1]
        blk[:, :, 0:2] = f16_bits(rng, nb, 1e-5, 3e-4).reshape(n_rows, -1, 1).view(np.uint8)
        blk[:, :, 2:4] = f16_bits(rng, nb, 1e-5, 6e-4).reshape(n_rows, -1, 1).view(np.uint8)
    return w


def rnd_hash(i, scale=2.0):
    """the reference unit tests' deterministic input (test_cpu_gemv_units.cpp:40-43)"""
    h = (np.asarray(i, np.uint64) * np.uint64(2654435761) + np.uint64(1013904223)) & np.uint64(0xFFFFFFFF)
    return ((((h >> np.uint64(8)) & np.uint64(0xFFFF)).astype(np.float32) / np.float32(32768.0)) - np.float32(1.0)) * np.float32(scale)


def make_q4k_pattern(N):
    """the reference test's hand-built Q4_K tensor (test_cpu_gemv_units.cpp:46-55), bytes only"""
    ref = Ref()
    out = np.zeros((N, 144), np.uint8)
    for n in range(N):
        d = ref.float_to_half(0.004 * (n + 1))
        dm = ref.float_to_half(0.001 * (n + 1))
        out[n, 0:2] = np.array([d], np.uint16).view(np.uint8)
        out[n, 2:4] = np.array([dm], np.uint16).view(np.uint8)
        out[n, 4:16] = [(0x11 + 7 * i) & 0xFF for i in range(12)]
        out[n, 16:144] = [(n * 37 + i * 11) & 0xFF for i in range(128)]
    return out


def make_q4k_native_pattern(N, K):
    """the reference GPU unit test's Q4_K tensor (test_kernel_units_native.cpp:91-100), bytes only:
    block b of the flattened tensor has d = 0.004*(b%5+1), dmin = 0.001*(b%3+1),
    scales[i] = 0x11+7i+b, qs[i] = (37b+11i) & 0xFF"""
    ref = Ref()
    nb = N * (K // 256)
    out = np.zeros((nb, 144), np.uint8)
    for b in range(nb):
        out[b, 0:2] = np.array([ref.float_to_half(0.004 * ((b % 5) + 1))], np.uint16).view(np.uint8)
        out[b, 2:4] = np.array([ref.float_to_half(0.001 * ((b % 3) + 1))], np.uint16).view(np.uint8)
        out[b, 4:16] = [(0x11 + 7 * i + b) & 0xFF for i in range(12)]
        out[b, 16:144] = [(b * 37 + i * 11) & 0xFF for i in range(128)]
    return out.reshape(N, -1)


def write_w4():
    """w4_pack (src/common/w4.cpp:416) of random Q4_K rows, rows with a subnormal
    super-block d (the case w4.h's f16 note describes: d = 4.47e-6, f16 0x004b,
    so d*sc falls below 2^-14), and the reference GPU test's pattern."""
    ref = Ref()
    rng = np.random.default_rng(4242)
    N, K = 24, 512
    w = random_blocks(rng, Q4_K, N, K)
    blk = w.reshape(N, -1, 144)
    blk[3, :, 0:2] = np.array([0x004B], np.uint16).view(np.uint8)   # subnormal d
    blk[4, :, 2:4] = np.array([0x0013], np.uint16).view(np.uint8)   # subnormal dmin
    blk[5, :, 0:4] = 0                                             # d = dmin = 0
    vals, sc, of = ref.w4_pack(w, K, N)
    wp = make_q4k_native_pattern(3, 512)
    pv, ps, po = ref.w4_pack(wp, 512, 3)
    np.savez_compressed(os.path.join(HERE, "w4_pack.npz"), w=w, K=np.int32(K), N=np.int32(N), vals=vals, scale=sc,
                        off=of, pat_w=wp, pat_vals=pv, pat_scale=ps, pat_off=po)
    # k5_pack (src/common/w4.cpp:409) of random Q5_K rows, with a subnormal d row and an all-ones qh row
    w5 = random_blocks(rng, Q5_K, N, K)
    b5 = w5.reshape(N, -1, 176)
    b5[3, :, 0:2] = np.array([0x004B], np.uint16).view(np.uint8)
    b5[6, :, 16:48] = 0xFF
    v5, h5, s5, o5 = ref.k5_pack(w5, K, N)
    np.savez_compressed(os.path.join(HERE, "k5_pack.npz"), w=w5, K=np.int32(K), N=np.int32(N), vals=v5, hi=h5,
                        scale=s5, off=o5)


def write_q80_odd():
    """Q8_0 rows with an odd number of 32-value groups (K % 64 == 32) through the
    reference's native Q8_0 down (cpu_q8_0_down_grouped, q4exp.cpp:442-484)."""
    ref = Ref()
    rng = np.random.default_rng(20261202)
    d = {}
    for K, N, tbs in ((96, 24, (1, 5, 16)), (160, 20, (1, 5, 16)), (352, 12, (1, 5, 16)), (5152, 6, (1, 5))):
        w = random_blocks(rng, Q8_0, N, K)
        d[f"w{K}"] = w
        for TB in tbs:
            x = rng.standard_normal((TB, K)).astype(np.float32)
            d[f"x{K}_{TB}"] = x
            d[f"out{K}_{TB}"] = ref.gemm(Q8_0, w, K, N, ref.xq(x))
    np.savez_compressed(os.path.join(HERE, "gemm_q80_odd.npz"), **d)


def main():
    ref = Ref()
    rng = np.random.default_rng(20261201)

    # --- f16 conversions (quant.h:67-133) on a spread of values incl. subnormals / overflow
    fl = np.concatenate([
        rng.standard_normal(2000).astype(np.float32) * np.float32(10.0) ** rng.integers(-9, 6, 2000).astype(np.float32),
        np.array([0.0, -0.0, 65504.0, 65519.0, 65520.0, 1e6, -1e6, 6.1035e-5, 6.0e-5, 5.96e-8, 3e-8, 1e-10,
                  np.float32(2.0) ** -24, np.float32(2.0) ** -25, np.float32(2.0) ** -14], np.float32)])
    f2h = np.array([ref.float_to_half(float(v)) for v in fl], np.uint16)
    np.savez_compressed(os.path.join(HERE, "f16.npz"), f=fl, h=f2h)

    # --- cpu_xq: the reference unit test's case (TB=3, K=64, rnd hash, with and without up),
    #     a random case, a zero group and round-half ties
    x_ut = rnd_hash(np.arange(3 * 64)).reshape(3, 64)
    up_ut = rnd_hash(np.arange(3 * 64) + 9000).reshape(3, 64)
    xr = rng.standard_normal((5, 512)).astype(np.float32) * np.float32(3.0)
    xr[1, 32:64] = 0.0                                # a zero group
    ties = np.zeros((1, 64), np.float32)
    ties[0, 0] = 127.0                                # mx = 127 -> inv = 1: exact .5 values round away from 0
    ties[0, 1:9] = [2.5, -2.5, 3.5, -3.5, 0.5, -0.5, 126.5, -126.5]
    ties[0, 32:64] = rng.standard_normal(32).astype(np.float32) * np.float32(1e-3)
    xq = {}
    for nm, x, up in (("ut", x_ut, None), ("ut_up", x_ut, up_ut), ("rand", xr, None), ("ties", ties, None)):
        x8, xm, xs = ref.xq(x, up)
        xq[f"{nm}_x"] = x
        if up is not None:
            xq[f"{nm}_up"] = up
        xq[f"{nm}_x8"], xq[f"{nm}_xmeta"], xq[f"{nm}_xsumq"] = x8, xm, xs
    np.savez_compressed(os.path.join(HERE, "xq.npz"), **xq)

    # --- integer GEMV / GEMM per type (cpu_i8_gemv / cpu_i8_gemm; Q8_0: cpu_q8_0_down_grouped)
    for qt in (Q4_K, Q5_K, Q6_K, Q8_0):
        N, K = 40, 512
        w = random_blocks(rng, qt, N, K)
        d = {"w": w, "K": np.int32(K), "N": np.int32(N), "deq": ref.dequantize(qt, w, K)}
        for TB in (1, 3, 16, 32):
            x = rng.standard_normal((TB, K)).astype(np.float32)
            act = ref.xq(x)
            d[f"x{TB}"] = x
            d[f"out{TB}"] = ref.gemm(qt, w, K, N, act)
            if qt != Q8_0:
                res = rng.standard_normal((TB, N)).astype(np.float32)
                d[f"res{TB}"] = res
                d[f"outra{TB}"] = ref.gemm(qt, w, K, N, act, residual=res, alpha=0.75)
        np.savez_compressed(os.path.join(HERE, f"gemm_{NAMES[qt]}.npz"), **d)

    # --- the reference unit test's Q4_K pattern (N=3, K=256, rnd inputs)
    wp = make_q4k_pattern(3)
    xp = rnd_hash(np.arange(256) + 100).reshape(1, 256)
    xm3 = rnd_hash(np.arange(3 * 256) + 700).reshape(3, 256)
    np.savez_compressed(os.path.join(HERE, "gemm_q4k_pattern.npz"), w=wp, x1=xp, out1=ref.gemm(Q4_K, wp, 256, 3, ref.xq(xp)),
                        x3=xm3, out3=ref.gemm(Q4_K, wp, 256, 3, ref.xq(xm3)), deq=ref.dequantize(Q4_K, wp, 256))

    # --- MoE: route, experts (Q4_K gate/up/down), reduce; plus a tie case for the router
    n_tok, n_expert, top_k, n_embd, n_ff = 6, 6, 3, 256, 256
    logits = rng.standard_normal((n_tok, n_expert)).astype(np.float32)
    logits[5, :] = logits[5, 0]  # all equal: ties go to the lower index
    logits[4, 2] = logits[4, 5] = logits[4].max() + 0.5
    ids, wts, probs = ref.moe_route(logits, top_k)
    gate = random_blocks(rng, Q4_K, n_expert * n_ff, n_embd)
    up = random_blocks(rng, Q4_K, n_expert * n_ff, n_embd)
    down = random_blocks(rng, Q4_K, n_expert * n_embd, n_ff)
    x = rng.standard_normal((n_tok, n_embd)).astype(np.float32)
    acc = ref.moe_experts(Q4_K, gate, up, down, n_embd, n_ff, n_expert, x, top_k, ids)
    out0 = rng.standard_normal((n_tok, n_embd)).astype(np.float32)
    out = ref.moe_reduce(acc, wts, top_k, out0)
    np.savez_compressed(os.path.join(HERE, "moe.npz"), logits=logits, ids=ids, wts=wts, probs=probs, gate=gate, up=up,
                        down=down, x=x, acc=acc, out0=out0, out=out,
                        dims=np.array([n_tok, n_expert, top_k, n_embd, n_ff], np.int32))
    # router with a real gate_inp (double-precision logits)
    gi = rng.standard_normal((16, 64)).astype(np.float32)
    xr = rng.standard_normal((5, 64)).astype(np.float32)
    ids2, wts2, lg = ref.moe_route(np.zeros((5, 16), np.float32), 4, x=xr, gate_inp=gi)
    np.savez_compressed(os.path.join(HERE, "moe_router.npz"), gate_inp=gi, x=xr, ids=ids2, wts=wts2, probs=lg)
    print("golden fixtures written to", HERE)


if __name__ == "__main__":
    if sys.argv[1:] == ["w4"]:
        write_w4()
    elif sys.argv[1:] == ["q80odd"]:
        write_q80_odd()
    else:
        main()
        write_w4()
        write_q80_odd()
