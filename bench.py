"""Benchmark of the quantized-matmul hot path on one MI355X.

Workload ("dense decode batch"): an FFN's Q4_K
gate and up projections N=17408 x K=5120 and its down projection N=5120 x
K=17408, weights N(0, 0.02) encoded to GGUF Q4_K, activations N(0, 1).  One
step = the FFN's decode at 1 token and at 16 tokens: gate and up in one call
on one activation (miq_quant_gemm_multi: the quantizer and both matrices in a
single launch at one token, as the reference's i8_grp_quant_gemv_launch,
kernels.h:216-219), then down (miq_quant_gemm).  Weights rotate over enough
copies (> 512 MB) that the 256 MB Infinity Cache cannot serve them: every
figure is cold-HBM.

value = whole-step algorithmic bytes / step time (GB/s): weights once, plus
fp32 activations in, int8 codes/scales/sums, fp32 outputs.  The roofline
object is for the dominant kernel, timed per launch with HIP events on the
stream the kernels run on (torch's current stream).  The second half of the
metric, prefill int8 GEMM TOPS (configs[3]: Q4_K 17408 x 5120 x 512 tokens),
is reported as `prefill`.

    python bench.py [--steps K] [--warmup W] [--no-cpu] [--no-prefill]
"""
import argparse
import json
import os
import sys
import time

import numpy as np

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "tests"))
sys.path.insert(0, os.path.join(REPO, "oracle"))

HBM_PEAK_GBS = 8000.0      # MI355X HBM3E
F16_PEAK_TFLOPS = 2500.0
INT8_PEAK_TOPS = 5000.0    # MI355X dense int8 MFMA
ROT_BYTES = 600e6          # rotating weight working set, > 2x the MALL


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU-baseline leg")
    ap.add_argument("--no-prefill", action="store_true", help="skip the prefill GEMM figure")
    ap.add_argument("--no-configs", action="store_true", help="skip configs 1, 3 and 5")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--only", choices=["up1", "up16", "down1", "down16", "prefill", "moe"],
                    help="time one call only (for rocprofv3 --pmc passes over a single kernel); "
                         "prefill: the configs[3] prefill GEMM alone; moe: the configs[4] step alone")
    ap.add_argument("--calib", action="store_true",
                    help="first run a plain copy of 256 MiB (torch.neg) whose HBM counters calibrate --pmc")
    ap.add_argument("--pmc-summary", nargs=3, metavar=("KEY", "FETCH_CSV", "WRITE_CSV"),
                    help="fold two rocprofv3 --pmc counter_collection.csv files (FETCH_SIZE, WRITE_SIZE) "
                         "of a `--calib --only KEY` run into profiles/hbm_traffic.json and exit")
    return ap.parse_args()


def gemv_bytes(N, K, TB, row_bytes):
    """algorithmic bytes of one GEMV/GEMM launch: weights + int8 act + scales/sums + fp32 out"""
    return N * row_bytes + TB * K + TB * (K // 32) * 16 + TB * N * 4


def xq_bytes(K, TB):
    return TB * K * 4 + TB * K + TB * (K // 32) * 16


def main():
    a = parse()
    if a.pmc_summary:
        pmc_summary(*a.pmc_summary)
        return
    if a.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU: every GPU box here has one MI355X and the "
                                   "hot path shards by output rows with no collective; "
                                   "run with --gpus 1"}))
        sys.exit(2)
    import torch
    from conftest import load_miq
    miq = load_miq()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    Q4_K = miq.Q4_K
    rng = np.random.default_rng(20261201)
    shapes = [("gate", 17408, 5120), ("up", 17408, 5120), ("down", 5120, 17408)]

    # ---- weights: encode once, replicate on the device for the rotation
    host_w = {}
    for name, N, K in shapes:
        W = (rng.standard_normal((N, K), dtype=np.float32) * np.float32(0.02))
        host_w[name] = miq.quantize_rows(Q4_K, W)
        del W
    set_bytes = sum(w.nbytes for w in host_w.values())
    n_sets = max(4, int(np.ceil(ROT_BYTES / set_bytes)))
    dw = {name: [torch.from_numpy(host_w[name]).to(dev) for _ in range(n_sets)] for name, _, _ in shapes}
    geo = {name: (N, K) for name, N, K in shapes}

    # ---- activations and outputs.  `mats`: one matrix per launch (the per-launch
    # figures and the roofline); `calls`: the step, an FFN's decode at 1 and 16
    # tokens -- gate and up of one activation in one call (miq_quant_gemm_multi,
    # one launch at one token), then down (miq_quant_gemm)
    mats, calls = [], []
    for TB in (1, 16):
        xs = {K: torch.from_numpy(rng.standard_normal((TB, K), dtype=np.float32)).to(dev) for K in (5120, 17408)}
        acts = {K: miq.alloc_act(TB, K, dev) for K in (5120, 17408)}
        outs = {name: torch.empty((TB, N), dtype=torch.float32, device=dev) for name, N, _ in shapes}
        segs = {name: [miq.make_seg(dw[name][s], Q4_K, K, N, acts[K], outs[name], N, x=xs[K]) for s in range(n_sets)]
                for name, N, K in shapes}
        for name in ("up", "down"):
            N, K = geo[name]
            mats.append(dict(key=f"{name}{TB}", name=name, N=N, K=K, TB=TB, x=xs[K], act=acts[K], segs=segs[name],
                             gemv_bytes=gemv_bytes(N, K, TB, miq.row_bytes(Q4_K, K))))
        N, K = geo["up"]
        rb = miq.row_bytes(Q4_K, K)
        calls.append(dict(key=f"gate_up{TB}", TB=TB, K=K, multi=[[segs["gate"][s], segs["up"][s]] for s in range(n_sets)],
                          bytes=2 * N * rb + TB * K * 4 + TB * K + TB * (K // 32) * 16 + 2 * TB * N * 4))
        N, K = geo["down"]
        calls.append(dict(key=f"down{TB}", TB=TB, K=K, segs=segs["down"],
                          bytes=gemv_bytes(N, K, TB, miq.row_bytes(Q4_K, K)) + xq_bytes(K, TB)))
    if a.only:
        mats = [c for c in mats if c["key"] == a.only]
        calls = []
    step_bytes = sum(c["bytes"] for c in calls)

    if a.calib:  # the copy kernel whose counters convert FETCH_SIZE/WRITE_SIZE into bytes
        src = torch.ones(CALIB_BYTES // 4, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            torch.neg(src, out=dst)
        torch.cuda.synchronize()
        del src, dst
    if a.only == "prefill":
        prefill_only(miq, torch, dev, rng, dw["up"], n_sets)
        return
    if a.only == "moe":
        del dw
        moe_only(miq, torch, dev, rng, a.steps)
        return

    def step(i):
        # a distinct weight set per call (no call finds its weights in the 256 MB
        # Infinity Cache: the sets rotate through > 2x its size)
        for ci, c in enumerate(calls):
            si = (i * len(calls) + ci) % n_sets
            if "multi" in c:
                miq.quant_gemm_multi(c["multi"][si], c["TB"])
            else:
                miq.quant_gemm(c["segs"][si], c["TB"])

    value, ms_per_step = None, None
    if calls:
        for i in range(a.warmup):
            step(i)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(a.steps):
            step(a.warmup + i)
        torch.cuda.synchronize()
        dt = time.perf_counter() - t0
        ms_per_step = dt * 1e3 / a.steps
        value = step_bytes / (dt / a.steps) / 1e9

    # ---- per-launch kernel times (GEMV/GEMM only, activations already quantized): HIP events on
    # the launch stream around chunks of back-to-back launches over the rotating weight sets
    stream = torch.cuda.current_stream()
    per_call = []
    reps = max(50, a.steps)
    for c in mats:
        miq.xq(c["x"], out=c["act"])
        st = {}
        us = timed(torch, lambda r: miq.i8_gemm(c["segs"][r % n_sets], c["TB"]), reps, st)
        gbs = c["gemv_bytes"] / (us * 1e-6) / 1e9
        per_call.append(dict(key=c["key"], shape=f"Q4_K {c['N']}x{c['K']} TB={c['TB']}", us_mean=round(us, 2), **st,
                             GBps=round(gbs, 1), frac_hbm=round(gbs / HBM_PEAK_GBS, 4),
                             kernel="dot4 GEMV" if c["TB"] <= 4 else "int8 MFMA 16-token GEMM"))
    # gate + up of one activation in a single launch (miq_i8_gemv_multi, one token)
    if calls:
        c = calls[0]
        miq.xq(mats[0]["x"], out=mats[0]["act"])  # up1: the activation gate_up1 shares
        st = {}
        us = timed(torch, lambda r: miq.i8_gemv_multi(c["multi"][r % n_sets], 1), reps, st)
        b = c["bytes"] - xq_bytes(c["K"], 1) + c["K"] + (c["K"] // 32) * 16
        per_call.append(dict(key="gate_up1", shape="Q4_K 2 x 17408x5120 TB=1 (one launch)", us_mean=round(us, 2), **st,
                             GBps=round(b / (us * 1e-6) / 1e9, 1), frac_hbm=round(b / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                             kernel="dot4 GEMV, two segments"))
        # gate + up at 16 tokens: one split-K launch over both matrices
        c = calls[2]
        miq.xq(mats[2]["x"], out=mats[2]["act"])  # up16: the activation gate_up16 shares
        st = {}
        us = timed(torch, lambda r: miq.i8_gemv_multi(c["multi"][r % n_sets], 16), reps, st)
        b = c["bytes"] - xq_bytes(c["K"], 16) + 16 * (c["K"] + (c["K"] // 32) * 16)
        per_call.append(dict(key="gate_up16", shape="Q4_K 2 x 17408x5120 TB=16 (one launch)", us_mean=round(us, 2), **st,
                             GBps=round(b / (us * 1e-6) / 1e9, 1), frac_hbm=round(b / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                             kernel="int8 MFMA 16-token GEMM, two segments"))
    dom = max(per_call[:len(mats)], key=lambda p: p["us_mean"])
    dom_c = mats[per_call.index(dom)]
    roofline = {"bound": "hbm", "achieved": dom["GBps"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(dom["GBps"] / HBM_PEAK_GBS, 4), "traffic": measured_traffic(dom["key"]),
                "kernel": dom["shape"], "algorithmic_bytes_per_launch": dom_c["gemv_bytes"],
                "us_per_launch": dom["us_mean"]}

    # ---- prefill GEMM: TOPS = 2*M*N*K / t, on weights rotated past the
    # Infinity Cache; `us_mean` times the GEMM launch(es) on a quantized activation,
    # `us_with_xq` the whole miq_quant_gemm call (activation quantizer included)
    prefill = None
    if not a.no_prefill:
        N, K, M = 17408, 5120, 512
        x = torch.from_numpy(rng.standard_normal((M, K), dtype=np.float32)).to(dev)
        act = miq.alloc_act(M, K, dev)
        out = torch.empty((M, N), dtype=torch.float32, device=dev)
        miq.xq(x, out=act)
        psegs = [miq.make_seg(dw["up"][s], Q4_K, K, N, act, out, N, x=x) for s in range(n_sets)]
        st = {}
        us = timed(torch, lambda r: miq.i8_gemm(psegs[r % n_sets], M), 20, st)
        us_q = timed(torch, lambda r: miq.quant_gemm(psegs[r % n_sets], M), 20)
        tops = 2.0 * M * N * K / (us * 1e-6) / 1e12
        prefill = {"shape": f"Q4_K {N}x{K} M={M}", "us_mean": round(us, 1), **st,
                   "TOPS": round(tops, 2), "peak_TOPS": INT8_PEAK_TOPS, "frac": round(tops / INT8_PEAK_TOPS, 4),
                   "bound": "mfma", "kernel": prefill_kernel_name(),
                   "frac_of_f16_peak": round(tops / F16_PEAK_TFLOPS, 4),
                   "us_with_xq": round(us_q, 1),
                   "TOPS_with_xq": round(2.0 * M * N * K / (us_q * 1e-6) / 1e12, 2),
                   "weights": f"rotated over {n_sets} sets (cold HBM)"}
        del x, act, out, psegs
        # side lines at the down projection's shape (5120 x 17408 x 512): Q4_K, and
        # Q6_K (ffn_down of Q4_K_M models), each on its own rotated weight sets
        N, K = 5120, 17408
        x = torch.from_numpy(rng.standard_normal((M, K), dtype=np.float32)).to(dev)
        act = miq.alloc_act(M, K, dev)
        out = torch.empty((M, N), dtype=torch.float32, device=dev)
        miq.xq(x, out=act)
        for key, qt in (("down_q4k", Q4_K), ("down_q6k", miq.Q6_K)):
            if qt == Q4_K:
                wsets = dw["down"]
            else:
                wq6 = miq.quantize_rows(qt, (rng.standard_normal((N, K), dtype=np.float32) * np.float32(0.02)))
                n6 = max(4, int(np.ceil(ROT_BYTES / wq6.nbytes)))
                wsets = [torch.from_numpy(wq6).to(dev) for _ in range(n6)]
            nw = len(wsets)
            segs = [miq.make_seg(wsets[s], qt, K, N, act, out, N, x=x) for s in range(nw)]
            st = {}
            us = timed(torch, lambda r: miq.i8_gemm(segs[r % nw], M), 20, st)
            tops = 2.0 * M * N * K / (us * 1e-6) / 1e12
            prefill[key] = {"shape": f"{'Q4_K' if qt == Q4_K else 'Q6_K'} {N}x{K} M={M}", "us_mean": round(us, 1), **st,
                            "TOPS": round(tops, 2), "frac": round(tops / INT8_PEAK_TOPS, 4),
                            "weights": f"rotated over {nw} sets (cold HBM)"}
            del segs, wsets
        del x, act, out

    # ---- the other configurations (parity is covered by the tests; here, time and bytes)
    host = {"c2_up": (Q4_K, host_w["up"], 17408, 5120), "c2_down": (Q4_K, host_w["down"], 5120, 17408)}
    configs = None if a.no_configs else other_configs(miq, torch, dev, rng, host)

    # ---- CPU baseline: sycl-infer's own CPU kernels (oracle/_ref) on the host cores
    cpu = None
    if not a.no_cpu:
        cpu = cpu_baseline(host, a.cpu_seconds)

    line = {
        "metric": "Q4_K GEMV achieved HBM GB/s (% of peak) + prefill int8 GEMM TOPS",
        "value": None if value is None else round(value, 1), "unit": "GB/s", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "ms_per_step": None if ms_per_step is None else round(ms_per_step, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "int8 x Q4_K (int32 group dots, fp32 epilogue)", "data": "synthetic (seeded N(0,0.02) weights, N(0,1) activations)",
        "config": {"workload": "configs[1] dense decode batch: an FFN's Q4_K gate + up 17408x5120 (one call on "
                               "one activation) and down 5120x17408, at 1 and 16 tokens",
                   "weight_sets_rotated": n_sets, "rotating_bytes": n_sets * set_bytes,
                   "frac_of_hbm_peak": None if value is None else round(value / HBM_PEAK_GBS, 4)},
        "roofline": roofline,
        "per_launch": per_call,
        "prefill": prefill,
        "configs": configs,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line))


def prefill_only(miq, torch, dev, rng, wsets, n_sets):
    """configs[3] alone (Q4_K 17408 x 5120, 512 tokens, rotated weights): 3 warm-up and
    10 timed GEMM launches, for counter passes over the prefill kernel"""
    N, K, M = 17408, 5120, 512
    x = torch.from_numpy(rng.standard_normal((M, K), dtype=np.float32)).to(dev)
    act = miq.alloc_act(M, K, dev)
    out = torch.empty((M, N), dtype=torch.float32, device=dev)
    miq.xq(x, out=act)
    segs = [miq.make_seg(wsets[s], miq.Q4_K, K, N, act, out, N) for s in range(n_sets)]
    us = timed(torch, lambda r: miq.i8_gemm(segs[r % n_sets], M), 10)
    print(json.dumps({"prefill_only": f"Q4_K {N}x{K} M={M}", "us_mean": round(us, 1),
                      "TOPS": round(2.0 * M * N * K / (us * 1e-6) / 1e12, 2)}))


def prefill_kernel_name():
    return "pf16: fp16 MFMA on integer-valued operands (exact), stream-K"


def timed(torch, fn, reps, stats=None):
    """mean microseconds of fn() per call: HIP events on the current stream around
    back-to-back calls (the device time per call; an event pair around every single
    call would add the dispatch gap, about 2 us, to each).  The calls run in chunks
    of 5, each chunk between its own pair of events; `stats` (a dict) also gets the
    median and the minimum of the chunks' per-call times"""
    stream = torch.cuda.current_stream()
    for _ in range(3):
        fn(0)
    chunk = 5
    n = max(1, reps // chunk)
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(n + 1)]
    evs[0].record(stream)
    for c in range(n):
        for r in range(chunk):
            fn(c * chunk + r)
        evs[c + 1].record(stream)
    torch.cuda.synchronize()
    t = [evs[c].elapsed_time(evs[c + 1]) * 1e3 / chunk for c in range(n)]
    if stats is not None:
        stats["us_median"] = round(float(np.median(t)), 2)
        stats["us_min"] = round(float(np.min(t)), 2)
    return float(np.mean(t))


def other_configs(miq, torch, dev, rng, host):
    """configs[0] (Q4_K 3584x1024, one token), configs[2] (Q6_K head 151936x5120 and
    Q5_K QKV 7168x5120 at 1 and 16 tokens) and configs[4] (MoE: route, grouped
    experts and weighted reduce over 16 tokens, 256 Q4_K experts, top-8), and
    the configs[1] shapes on the repacked u4 store and configs[2]'s QKV on the k5
    store at one token, each on weights rotated past the 256 MB Infinity Cache.  GB/s counts each weight
    byte the call needs once (MoE: the routed experts only), plus activations
    and outputs."""
    res = {}
    for key, qt, N, K, tbs in (("c1_q4k_3584x1024", miq.Q4_K, 3584, 1024, (1,)),
                               ("c3_q6k_head_151936x5120", miq.Q6_K, 151936, 5120, (1, 16)),
                               ("c3_q5k_qkv_7168x5120", miq.Q5_K, 7168, 5120, (1, 16))):
        W = (rng.standard_normal((N, K), dtype=np.float32) * np.float32(0.02))
        wq = miq.quantize_rows(qt, W)
        del W
        host[key.split("_")[0] + "_" + key.split("_")[1]] = (qt, wq, N, K)
        n_sets = max(2, int(np.ceil(ROT_BYTES / wq.nbytes)))
        ws = [torch.from_numpy(wq).to(dev) for _ in range(n_sets)]
        rb = miq.row_bytes(qt, K)
        for TB in tbs:
            x = torch.from_numpy(rng.standard_normal((TB, K), dtype=np.float32)).to(dev)
            act = miq.alloc_act(TB, K, dev)
            out = torch.empty((TB, N), dtype=torch.float32, device=dev)
            miq.xq(x, out=act)
            segs = [miq.make_seg(w, qt, K, N, act, out, N) for w in ws]
            st = {}
            us = timed(torch, lambda r: miq.i8_gemm(segs[r % n_sets], TB), 50, st)
            b = gemv_bytes(N, K, TB, rb)
            res[f"{key}_tb{TB}"] = {"us": round(us, 2), **st, "GBps": round(b / (us * 1e-6) / 1e9, 1),
                                    "frac_hbm": round(b / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
        del ws, segs
    # the u4 native-width store (repacked Q4_K, 0.625 B/weight) at one token: the
    # GEMV alone on a pre-quantized activation, and the activation quantizer + GEMV
    for key, N, K in (("f4_u4_up_17408x5120", 17408, 5120), ("f4_u4_down_5120x17408", 5120, 17408)):
        wq = miq.quantize_rows(miq.Q4_K, rng.standard_normal((N, K), dtype=np.float32) * np.float32(0.02))
        st_bytes = N * K // 2 + (K // 32) * N * 4
        n_sets = max(2, int(np.ceil(ROT_BYTES / st_bytes)))
        wd = torch.from_numpy(wq).to(dev)
        sts = [miq.w4_pack(wd, K, N) for _ in range(n_sets)]
        del wd, wq
        x = torch.from_numpy(rng.standard_normal((1, K), dtype=np.float32)).to(dev)
        act = miq.w4_act(x)
        out = torch.empty(N, dtype=torch.float32, device=dev)
        us = timed(torch, lambda r: miq.w4_gemv(sts[r % n_sets], act, out), 50)
        us2 = timed(torch, lambda r: (miq.w4_act(x, out=act), miq.w4_gemv(sts[r % n_sets], act, out)), 50)
        b = st_bytes + K + (K // 32) * 6 + N * 4
        res[key + "_tb1"] = {"us": round(us, 2), "GBps": round(b / (us * 1e-6) / 1e9, 1),
                             "frac_hbm": round(b / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                             "us_with_act_quant": round(us2, 2), "store_bytes": st_bytes}
        x4 = torch.from_numpy(rng.standard_normal((4, K), dtype=np.float32)).to(dev)
        act4 = miq.w4_act(x4)
        out4 = torch.empty((4, N), dtype=torch.float32, device=dev)
        res[key + "_tb1"]["us_4_tokens"] = round(timed(torch, lambda r: miq.w4_gemm(sts[r % n_sets], act4, out4), 50), 2)
        # the reference's batched verify GEMM (nat_gemm_launch) at its quoted M = 7
        x7 = torch.from_numpy(rng.standard_normal((7, K), dtype=np.float32)).to(dev)
        act7 = miq.w4_act(x7)
        out7 = torch.empty((7, N), dtype=torch.float32, device=dev)
        us7 = timed(torch, lambda r: miq.nat_gemm(sts[r % n_sets], act7, out7), 50)
        res[key + "_tb1"]["us_nat_7_tokens"] = round(us7, 2)
        res[key + "_tb1"]["GBps_nat_7_tokens"] = round(st_bytes / (us7 * 1e-6) / 1e9, 1)
        if K // 32 <= 256:  # the fused quantizer + GEMV launch (f1 on the u4 store)
            xv = x.view(K)
            res[key + "_tb1"]["us_fused_quant"] = round(
                timed(torch, lambda r: miq.w4_quant_gemv([(sts[r % n_sets], out, 1.0, None)], xv), 50), 2)
        del sts
    # the k5 native 5-bit store (repacked Q5_K, 0.75 B/weight): configs[2]'s QKV at one token
    N, K = 7168, 5120
    wq = miq.quantize_rows(miq.Q5_K, rng.standard_normal((N, K), dtype=np.float32) * np.float32(0.02))
    st_bytes = N * K // 2 + N * K // 8 + (K // 32) * N * 4
    n_sets = max(2, int(np.ceil(ROT_BYTES / st_bytes)))
    wd = torch.from_numpy(wq).to(dev)
    sts = [miq.k5_pack(wd, K, N) for _ in range(n_sets)]
    del wd, wq
    x = torch.from_numpy(rng.standard_normal((1, K), dtype=np.float32)).to(dev)
    act = miq.w4_act(x)
    out = torch.empty(N, dtype=torch.float32, device=dev)
    us = timed(torch, lambda r: miq.k5_gemv(sts[r % n_sets], act, out), 50)
    b = st_bytes + K + (K // 32) * 6 + N * 4
    res["f4_k5_qkv_7168x5120_tb1"] = {"us": round(us, 2), "GBps": round(b / (us * 1e-6) / 1e9, 1),
                                      "frac_hbm": round(b / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                                      "store_bytes": st_bytes}
    x7 = torch.from_numpy(rng.standard_normal((7, K), dtype=np.float32)).to(dev)
    act7 = miq.w4_act(x7)
    out7 = torch.empty((7, N), dtype=torch.float32, device=dev)
    us7 = timed(torch, lambda r: miq.nat_gemm(sts[r % n_sets], act7, out7), 50)
    res["f4_k5_qkv_7168x5120_tb1"]["us_nat_7_tokens"] = round(us7, 2)
    res["f4_k5_qkv_7168x5120_tb1"]["GBps_nat_7_tokens"] = round(st_bytes / (us7 * 1e-6) / 1e9, 1)
    del sts
    # MoE: expert banks tiled from one quantized expert (only bytes matter for time)
    M = moe_setup(miq, torch, dev, rng)
    host["c5_moe"] = M["host"]
    moe_step, n_banks, n_act = M["step"], M["n_banks"], M["n_act"]
    qt, g1, d1, n_tok, n_expert, top_k, n_embd, n_ff = M["host"]
    us_eager = timed(torch, moe_step, 50)
    # the same step captured once per bank in a HIP graph (how a serving loop
    # issues a layer): GPU time without the per-call host launch cost
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for r in range(n_banks):
            moe_step(r)
    torch.cuda.current_stream().wait_stream(side)
    graphs = []
    for r in range(n_banks):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            moe_step(r)
        graphs.append(g)
    us = timed(torch, lambda r: graphs[r % n_banks].replay(), 50)
    b = n_act * (2 * g1.nbytes + d1.nbytes) + n_tok * n_embd * 4 * 2 + n_tok * top_k * n_embd * 4
    res["c5_moe_q4k_256x_top8_16tok"] = {"us": round(us_eager, 2), "GBps": round(b / (us_eager * 1e-6) / 1e9, 1),
                                         "frac_hbm": round(b / (us_eager * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                                         "us_graph_replay": round(us, 2), "active_experts": n_act, "bytes": b}
    del graphs
    del M
    return res


def moe_setup(miq, torch, dev, rng):
    """256 Q4_K experts (gate/up 512x2048, down 2048x512), 16 tokens, top-8; banks
    tiled from one quantized expert (only bytes matter for time) and rotated past the MALL.
    Returns the step (route over fresh logits, experts, weighted reduce) and its sizes."""
    n_tok, n_expert, top_k, n_embd, n_ff = 16, 256, 8, 2048, 512
    qt = miq.Q4_K
    g1 = miq.quantize_rows(qt, (rng.standard_normal((n_ff, n_embd), dtype=np.float32) * np.float32(0.02)))
    d1 = miq.quantize_rows(qt, (rng.standard_normal((n_embd, n_ff), dtype=np.float32) * np.float32(0.02)))
    bank_bytes = n_expert * (2 * g1.nbytes + d1.nbytes)
    n_banks = max(2, int(np.ceil(ROT_BYTES / bank_bytes)))
    banks = []
    for _ in range(n_banks):
        gate = torch.from_numpy(np.tile(g1, (n_expert, 1))).to(dev)
        up = torch.from_numpy(np.tile(g1, (n_expert, 1))).to(dev)
        down = torch.from_numpy(np.tile(d1, (n_expert, 1))).to(dev)
        banks.append((gate, up, down, miq.make_moe(gate, up, down, qt, n_embd, n_ff, n_expert)))
    x = torch.from_numpy(rng.standard_normal((n_tok, n_embd), dtype=np.float32)).to(dev)
    logits0 = torch.from_numpy(rng.standard_normal((n_tok, n_expert), dtype=np.float32)).to(dev)
    logits = logits0.clone()
    ws = miq.moe_workspace(banks[0][3], n_tok, top_k, dev)
    acc = torch.empty((n_tok * top_k, n_embd), dtype=torch.float32, device=dev)
    out = torch.zeros((n_tok, n_embd), dtype=torch.float32, device=dev)
    ids, wts = miq.moe_route(logits, top_k)
    n_act = int(torch.unique(ids).numel())

    def step(r):
        logits.copy_(logits0)  # the router's fresh logits (it softmaxes them in place)
        i, w = miq.moe_route(logits, top_k)
        miq.moe_experts(banks[r % n_banks][3], x, top_k, i, acc, ws)
        miq.moe_reduce(acc, w, top_k, out)

    return dict(step=step, n_banks=n_banks, n_act=n_act, banks=banks,
                host=(qt, g1, d1, n_tok, n_expert, top_k, n_embd, n_ff))


def moe_only(miq, torch, dev, rng, steps):
    """`--only moe`: the configs[4] step alone (for rocprofv3 passes over the MoE kernels)."""
    M = moe_setup(miq, torch, dev, rng)
    us = timed(torch, M["step"], steps)
    print(json.dumps({"moe_only": "configs[4] route + experts + reduce", "us": round(us, 2),
                      "active_experts": M["n_act"]}), flush=True)


CALIB_BYTES = 256 << 20
TRAFFIC_FILE = os.path.join(REPO, "profiles", "hbm_traffic.json")


def measured_traffic(key):
    """HBM bytes per launch of call `key`, from the committed --pmc summary (None if absent)."""
    try:
        with open(TRAFFIC_FILE) as f:
            t = json.load(f)
    except (OSError, ValueError):
        return None
    e = t.get(key)
    return None if e is None else e["hbm_bytes_per_launch"]


def pmc_summary(key, fetch_csv, write_csv):
    """FETCH_SIZE / WRITE_SIZE (KiB per dispatch) of the measured kernel, scaled by what the
    same counters read for the calibration copy (CALIB_BYTES read + CALIB_BYTES written)."""
    import csv

    def per_kernel(path, counter):
        vals = {}
        for r in csv.DictReader(open(path)):
            if r["Counter_Name"] != counter:
                continue
            vals.setdefault(r["Kernel_Name"], []).append(float(r["Counter_Value"]) * 1024)
        return vals

    out = {}
    try:
        with open(TRAFFIC_FILE) as f:
            out = json.load(f)
    except (OSError, ValueError):
        pass
    fetch, write = per_kernel(fetch_csv, "FETCH_SIZE"), per_kernel(write_csv, "WRITE_SIZE")
    calib = [k for k in fetch if "neg" in k.lower()]
    main_k = [k for k in fetch if k.startswith("void miq::") and "xq_kernel" not in k]
    if len(calib) != 1 or len(main_k) != 1:
        sys.exit(f"expected one calibration and one miq GEMV/GEMM kernel, found {calib} / {main_k}")
    cf = CALIB_BYTES / np.median(fetch[calib[0]])
    cw = CALIB_BYTES / np.median(write[calib[0]])
    f = float(np.median(fetch[main_k[0]])) * cf
    w = float(np.median(write[main_k[0]])) * cw
    out[key] = {"kernel": main_k[0], "dispatches": len(fetch[main_k[0]]),
                "fetch_bytes_per_launch": round(f), "write_bytes_per_launch": round(w),
                "hbm_bytes_per_launch": round(f + w), "calib_fetch_factor": round(float(cf), 4),
                "calib_write_factor": round(float(cw), 4)}
    with open(TRAFFIC_FILE, "w") as fh:
        json.dump(out, fh, indent=1, sort_keys=True)
    print(json.dumps(out[key]))


def physical_cores():
    """Distinct (physical id, core id) pairs of /proc/cpuinfo: the reference's
    detect_physical_cores (src/backend/cpu/kernels/common.cpp:39-66); 0 when
    the platform does not list them."""
    cores, phys, core = set(), -1, -1
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if not line.strip():
                    if phys >= 0 and core >= 0:
                        cores.add((phys, core))
                    phys = core = -1
                elif line.startswith("physical id"):
                    phys = int(line.split(":")[1])
                elif line.startswith("core id"):
                    core = int(line.split(":")[1])
    except OSError:
        return 0
    if phys >= 0 and core >= 0:
        cores.add((phys, core))
    return len(cores)


def cpu_threads():
    """The reference's default pool size (physical cores, else the hardware
    threads: detect_threads, common.cpp:68-87), capped at the CPUs this process
    may run on and the box's CPU share (OMP_NUM_THREADS where the pool sets it)."""
    hw = os.cpu_count() or 1
    phys = physical_cores()
    n = phys if 1 <= phys <= hw else hw
    allowed = len(os.sched_getaffinity(0))
    share = int(os.environ.get("OMP_NUM_THREADS") or 0)
    used = min(n, allowed, share) if share > 0 else min(n, allowed)
    return used, {"physical_cores": phys, "hw_threads": hw, "affinity": allowed, "share": share or None}


def cpu_items(host):
    """(key, callable) pairs: sycl-infer's CPU path on every BASELINE config
    (cpu_i8_gemv at one token, cpu_i8_gemm at several, the MoE route + expert
    composition + reduce), each on activations quantized by cpu_xq beforehand,
    as the reference's gemv_at quantizes once per call group."""
    from oracle import Ref
    ref = Ref()
    rng = np.random.default_rng(3)
    items = []

    def gemm(qt, wq, N, K, TB):
        act = ref.xq(rng.standard_normal((TB, K), dtype=np.float32))
        return lambda: ref.gemm(qt, wq, K, N, act), 2.0 * N * K * TB, wq.nbytes

    # keys: c1 .. c5 = BASELINE configs[0] .. configs[4]
    for key, TBs in (("c1_q4k", (1,)), ("c2_up", (1, 16)), ("c2_down", (1, 16)), ("c3_q6k", (1,)),
                     ("c3_q5k", (1, 16))):
        if key not in host:
            continue
        qt, wq, N, K = host[key]
        for TB in TBs:
            items.append((f"{key}_{N}x{K}_tb{TB}",) + gemm(qt, wq, N, K, TB))
    qt, wq, N, K = host["c2_up"]
    items.append(("c4_prefill_q4k_17408x5120_m512",) + gemm(qt, wq, N, K, 512))
    if "c5_moe" in host:
        qt, g1, d1, n_tok, n_expert, top_k, n_embd, n_ff = host["c5_moe"]
        gate = np.tile(g1, (n_expert, 1))
        down = np.tile(d1, (n_expert, 1))
        x = rng.standard_normal((n_tok, n_embd), dtype=np.float32)
        lg = rng.standard_normal((n_tok, n_expert), dtype=np.float32)

        def moe():
            ids, wts, _ = ref.moe_route(lg, top_k)
            acc = ref.moe_experts(qt, gate, gate, down, n_embd, n_ff, n_expert, x, top_k, ids)
            return ref.moe_reduce(acc, wts, top_k, np.zeros((n_tok, n_embd), np.float32))
        ids, _, _ = ref.moe_route(lg, top_k)
        n_act = len(np.unique(ids))
        items.append(("c5_moe_q4k_256x_top8_16tok", moe, 2.0 * n_tok * top_k * 3 * n_embd * n_ff,
                      n_act * (2 * g1.nbytes + d1.nbytes)))
    return ref, items


def run_items(items, seconds):
    res = {}
    for key, fn, ops, wbytes in items:
        fn()  # warm the pool and the pages
        n, t0 = 0, time.perf_counter()
        while n == 0 or time.perf_counter() - t0 < seconds:
            fn()
            n += 1
        dt = (time.perf_counter() - t0) / n
        res[key] = {"us": round(dt * 1e6, 1), "GBps": round(wbytes / dt / 1e9, 2), "GOPS": round(ops / dt / 1e9, 2),
                    "calls": n}
    return res


def cpu_baseline(host, seconds):
    """sycl-infer's own CPU kernels (oracle/_ref, built from the reference
    sources) on the GPU box's host: every config at the reference's default
    thread count (physical cores, capped at this process's CPU share), then the
    one-token up projection and the prefill on one core in a child process.
    `value` is the configs[1] up projection at one token, in the metric's GB/s."""
    from oracle import REF_LIB
    if not os.path.exists(REF_LIB):
        return None
    n, topo = cpu_threads()
    os.environ["PF_CPU_THREADS"] = str(n)  # read when the reference's pool starts
    per_item = max(0.5, seconds / 12)
    ref, items = cpu_items(host)
    res = run_items(items, per_item)
    one = None
    try:  # one core: a child process (the pool is sized once per process)
        import subprocess
        import tempfile
        with tempfile.TemporaryDirectory() as td:
            qt, wq, N, K = host["c2_up"]
            np.save(os.path.join(td, "up.npy"), wq)
            env = dict(os.environ, PF_CPU_THREADS="1")
            r = subprocess.run([sys.executable, os.path.abspath(__file__), "--cpu-one-core", td, str(per_item)],
                               env=env, capture_output=True, text=True, timeout=600)
            one = json.loads(r.stdout.strip().splitlines()[-1]) if r.returncode == 0 else {"error": r.stderr[-300:]}
    except Exception as e:  # the 1-core figure is informative; never fail the bench on it
        one = {"error": repr(e)}
    head = res["c2_up_17408x5120_tb1"]
    return {"value": head["GBps"], "unit": "GB/s", "cores": ref.thread_count(), "kind": "reference",
            "isa": ref.isa_spec(), "topology": topo,
            "sample": f"cpu_i8_gemv Q4_K 17408x5120, 1 token: {head['calls']} calls in ~{per_item:.1f}s; every "
                      f"other config for ~{per_item:.1f}s each (warm page cache, activations pre-quantized)",
            "configs": res, "one_core": one}


def cpu_one_core(td, seconds):
    """child of cpu_baseline: the one-token up projection and the 512-token prefill on one thread"""
    sys.path.insert(0, os.path.join(REPO, "oracle"))
    from oracle import Ref
    ref = Ref()
    wq = np.load(os.path.join(td, "up.npy"))
    rng = np.random.default_rng(3)
    out = {"cores": ref.thread_count(), "isa": ref.isa_spec()}
    for TB in (1, 512):
        act = ref.xq(rng.standard_normal((TB, 5120), dtype=np.float32))
        res = run_items([(f"tb{TB}", lambda: ref.gemm(12, wq, 5120, 17408, act), 2.0 * 17408 * 5120 * TB,
                          wq.nbytes)], seconds)
        out[f"c2_up_17408x5120_tb{TB}"] = res[f"tb{TB}"]
    print(json.dumps(out))


if __name__ == "__main__":
    if len(sys.argv) == 4 and sys.argv[1] == "--cpu-one-core":
        cpu_one_core(sys.argv[2], float(sys.argv[3]))
    else:
        main()
