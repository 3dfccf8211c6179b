// GPU unit tests of the C++ host layer (sycl-infer_amd/cpp/miq_backend.hpp),
// written the way the reference's kernel unit tests are
// (tests/backend/cpu/kernels/test_cpu_gemv_units.cpp: named checks, max|diff|
// against max|exp|, a failure count as the exit status).  The checker is the
// oracle's C restatement of the reference CPU path (oracle/miq_oracle.h);
// weights are seeded N(0, 0.02) rows encoded by the library's host encoder.
// Needs a GPU; `--list` prints the test names and exits without one.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <random>
#include <string>
#include <vector>

#include "miq_backend.hpp"
#include "miq_oracle.h"

static int g_fail = 0;

static void fail(const char *name, const char *what) {
    std::printf("%-36s FAIL (%s)\n", name, what);
    g_fail++;
}

static void check_f32(const char *name, const std::vector<float> &got, const std::vector<float> &exp, double tol) {
    if (got.size() != exp.size()) return fail(name, "size");
    double maxd = 0, maxv = 0;
    for (size_t i = 0; i < got.size(); i++) {
        maxd = std::max(maxd, (double)std::fabs(got[i] - exp[i]));
        maxv = std::max(maxv, (double)std::fabs(exp[i]));
    }
    const bool ok = maxd <= tol * std::max(1e-30, maxv);
    std::printf("%-36s n=%-7zu max|exp|=%.5f max|diff|=%.3e %s\n", name, got.size(), maxv, maxd, ok ? "OK" : "FAIL");
    if (!ok) g_fail++;
}

template <class T> static void check_exact(const char *name, const std::vector<T> &got, const std::vector<T> &exp) {
    const bool ok = got.size() == exp.size() && std::memcmp(got.data(), exp.data(), got.size() * sizeof(T)) == 0;
    std::printf("%-36s n=%-7zu %s\n", name, got.size(), ok ? "bit-exact OK" : "FAIL");
    if (!ok) g_fail++;
}

#define HIP_OK(x)                                                                       \
    do {                                                                                \
        if ((x) != hipSuccess) {                                                        \
            std::printf("HIP error at %s:%d: %s\n", __FILE__, __LINE__, #x);            \
            std::exit(2);                                                               \
        }                                                                               \
    } while (0)

template <class T> struct dbuf {  // a device copy of a host vector
    T *p = nullptr;
    size_t n = 0;
    explicit dbuf(size_t count) : n(count) { HIP_OK(hipMalloc(&p, std::max<size_t>(1, n) * sizeof(T))); }
    explicit dbuf(const std::vector<T> &h) : dbuf(h.size()) { put(h); }
    ~dbuf() { (void)hipFree(p); }
    dbuf(const dbuf &) = delete;
    void put(const std::vector<T> &h) { HIP_OK(hipMemcpy(p, h.data(), h.size() * sizeof(T), hipMemcpyHostToDevice)); }
    std::vector<T> get() const {
        std::vector<T> h(n);
        HIP_OK(hipMemcpy(h.data(), p, n * sizeof(T), hipMemcpyDeviceToHost));
        return h;
    }
};

static std::mt19937_64 g_rng(20260101);
static std::vector<float> normal(size_t n, float sd) {
    std::normal_distribution<float> d(0.0f, sd);
    std::vector<float> v(n);
    for (auto &e : v) e = d(g_rng);
    return v;
}

static std::vector<uint8_t> encode(uint32_t type, int n_rows, int K) {
    const std::vector<float> w = normal((size_t)n_rows * K, 0.02f);
    std::vector<uint8_t> q(miq_row_bytes(type, K) * n_rows);
    if (miq_quantize_rows(type, w.data(), q.data(), n_rows, K, 0) != MIQ_OK) {
        std::printf("encode failed: %s\n", miq_last_error());
        std::exit(2);
    }
    return q;
}

struct host_act {  // the oracle's quantized activation
    std::vector<int8_t> x8;
    std::vector<float> meta;
    std::vector<int32_t> sum;
};
static host_act oracle_xq(const std::vector<float> &x, const float *up, int TB, int K) {
    host_act a;
    a.x8.resize((size_t)TB * K);
    a.meta.resize((size_t)TB * (K / 32) * 2);
    a.sum.resize((size_t)TB * (K / 32) * 2);
    miqo_xq(x.data(), up, K, K, a.x8.data(), a.meta.data(), a.sum.data(), TB, K);
    return a;
}

static const char *tname(uint32_t t) { return t == 12 ? "Q4_K" : t == 13 ? "Q5_K" : t == 14 ? "Q6_K" : "Q8_0"; }

static void test_xq(miq::compute_backend &be) {
    const int TB = 5, K = 1024;
    const std::vector<float> x = normal((size_t)TB * K, 1.0f), up = normal((size_t)TB * K, 1.0f);
    for (int with_up = 0; with_up < 2; with_up++) {
        const host_act e = oracle_xq(x, with_up ? up.data() : nullptr, TB, K);
        dbuf<float> dx(x), du(up);
        dbuf<int8_t> x8(e.x8.size());
        dbuf<float> meta(e.meta.size());
        dbuf<int32_t> sum(e.sum.size());
        be.xq(dx.p, with_up ? du.p : nullptr, K, K, x8.p, reinterpret_cast<miq::float2 *>(meta.p), sum.p, nullptr, TB, K);
        be.synchronize();
        check_exact(with_up ? "xq silu(x)*up: codes" : "xq: codes", x8.get(), e.x8);
        check_exact(with_up ? "xq silu(x)*up: scales" : "xq: scales", meta.get(), e.meta);
        check_exact(with_up ? "xq silu(x)*up: sums" : "xq: sums", sum.get(), e.sum);
    }
}

// i8_gemv / i8_gemm through the backend against the oracle's cpu_i8_gemv /
// cpu_i8_gemm, with a residual and alpha; every batch size picks its kernel.
static void test_i8(miq::compute_backend &be, uint32_t type, int N, int K, int TB) {
    const std::vector<uint8_t> wq = encode(type, N, K);
    const std::vector<float> x = normal((size_t)TB * K, 1.0f), res = normal((size_t)TB * N, 0.1f);
    const host_act a = oracle_xq(x, nullptr, TB, K);
    std::vector<float> exp((size_t)TB * N);
    miqo_seg os{};
    os.w = wq.data();
    os.type = type;
    os.K = K;
    os.n_rows = N;
    os.out = exp.data();
    os.out_stride = N;
    os.residual = res.data();
    os.alpha = 0.75f;
    os.x8 = a.x8.data();
    os.xmeta = a.meta.data();
    os.xsumq = a.sum.data();
    if (TB == 1) miqo_i8_gemv(&os);
    else miqo_i8_gemm(&os, TB);
    dbuf<uint8_t> dw(wq);
    dbuf<int8_t> x8(a.x8);
    dbuf<float> meta(a.meta), dres(res), out((size_t)TB * N);
    dbuf<int32_t> sum(a.sum);
    miq::gemv_seg s;
    s.w = dw.p;
    s.type = type;
    s.K = K;
    s.n_rows = N;
    s.out = out.p;
    s.out_stride = N;
    s.residual = dres.p;
    s.alpha = 0.75f;
    s.x8 = x8.p;
    s.xmeta = reinterpret_cast<const miq::float2 *>(meta.p);
    s.xsumq = sum.p;
    if (TB == 1) be.i8_gemv(s);
    else be.i8_gemm(s, TB);
    be.synchronize();
    char name[96];
    std::snprintf(name, sizeof(name), "i8_%s %s %dx%d TB=%d", TB == 1 ? "gemv" : "gemm", tname(type), N, K, TB);
    check_f32(name, out.get(), exp, 1e-4);
}

// two segments on one activation in one call == one call per segment, bit for
// bit: one GEMV launch at one token, one split-K GEMM launch at 16
static void test_multi(miq::compute_backend &be, int TB) {
    const int K = 2048, N0 = 1536, N1 = 512;
    const std::vector<uint8_t> w0 = encode(12, N0, K), w1 = encode(12, N1, K);
    const host_act a = oracle_xq(normal((size_t)TB * K, 1.0f), nullptr, TB, K);
    dbuf<uint8_t> d0(w0), d1(w1);
    dbuf<int8_t> x8(a.x8);
    dbuf<float> meta(a.meta), o0((size_t)TB * N0), o1((size_t)TB * N1), r0((size_t)TB * N0), r1((size_t)TB * N1);
    dbuf<int32_t> sum(a.sum);
    miq::gemv_seg s[2];
    for (int i = 0; i < 2; i++) {
        s[i].type = 12;
        s[i].K = K;
        s[i].x8 = x8.p;
        s[i].xmeta = reinterpret_cast<const miq::float2 *>(meta.p);
        s[i].xsumq = sum.p;
    }
    s[0].w = d0.p, s[0].n_rows = N0, s[0].out = o0.p, s[0].out_stride = N0;
    s[1].w = d1.p, s[1].n_rows = N1, s[1].out = o1.p, s[1].out_stride = N1;
    be.i8_gemv_multi(s, 2, TB);
    miq::gemv_seg t0 = s[0], t1 = s[1];
    t0.out = r0.p;
    t1.out = r1.p;
    if (TB == 1) {
        be.i8_gemv(t0);
        be.i8_gemv(t1);
    } else {
        be.i8_gemm(t0, TB);
        be.i8_gemm(t1, TB);
    }
    be.synchronize();
    check_exact(TB == 1 ? "i8_gemv_multi seg 0 == i8_gemv" : "i8_gemv_multi TB=16 seg 0 == i8_gemm", o0.get(), r0.get());
    check_exact(TB == 1 ? "i8_gemv_multi seg 1 == i8_gemv" : "i8_gemv_multi TB=16 seg 1 == i8_gemm", o1.get(), r1.get());
}

// the fused quantizer + GEMV == xq then GEMV, bit for bit, and its activation outputs == xq's
static void test_quant_gemm(miq::compute_backend &be) {
    const int K = 4096, N = 2048;
    const std::vector<uint8_t> wq = encode(12, N, K);
    const std::vector<float> x = normal(K, 1.0f);
    dbuf<uint8_t> dw(wq);
    dbuf<float> dx(x), meta(K / 16), meta2(K / 16), out(N), out2(N);
    dbuf<int8_t> x8(K), x82(K);
    dbuf<int32_t> sum(K / 16), sum2(K / 16);
    miq::gemv_seg s;
    s.w = dw.p, s.type = 12, s.K = K, s.n_rows = N, s.x = dx.p, s.x_stride = K, s.out = out.p, s.out_stride = N;
    s.x8 = x8.p, s.xmeta = reinterpret_cast<const miq::float2 *>(meta.p), s.xsumq = sum.p;
    be.quant_gemm(s, 1);
    be.xq(dx.p, nullptr, K, K, x82.p, reinterpret_cast<miq::float2 *>(meta2.p), sum2.p, nullptr, 1, K);
    miq::gemv_seg t = s;
    t.out = out2.p, t.x8 = x82.p, t.xmeta = reinterpret_cast<const miq::float2 *>(meta2.p), t.xsumq = sum2.p;
    be.i8_gemv(t);
    be.synchronize();
    check_exact("quant_gemm == xq + i8_gemv", out.get(), out2.get());
    check_exact("quant_gemm writes xq's codes", x8.get(), x82.get());
}

// unsupported shapes: the launcher form returns false, the method throws miq::unsupported
static void test_unsupported(miq::compute_backend &be) {
    dbuf<uint8_t> w(64);
    dbuf<float> o(16), meta(16);
    dbuf<int8_t> x8(256);
    dbuf<int32_t> sum(16);
    miq::gemv_seg s;
    s.w = w.p, s.type = 1 /* F16: not on the integer path */, s.K = 256, s.n_rows = 1, s.out = o.p, s.out_stride = 1;
    s.x8 = x8.p, s.xmeta = reinterpret_cast<const miq::float2 *>(meta.p), s.xsumq = sum.p;
    const bool launched = miq::i8_gemm_launch(nullptr, s, 2);
    std::printf("%-36s %s\n", "i8_gemm_launch(F16) returns false", launched ? "FAIL" : "OK");
    if (launched) g_fail++;
    bool threw = false;
    try {
        be.i8_gemv(s);
    } catch (const miq::unsupported &) {
        threw = true;
    }
    std::printf("%-36s %s\n", "i8_gemv(F16) throws unsupported", threw ? "OK" : "FAIL");
    if (!threw) g_fail++;
}

// route + routed experts + weighted reduce against the oracle (cpu_moe_route,
// cpu_moe_experts_i8's composition, cpu_moe_reduce)
static void test_moe(miq::compute_backend &be) {
    const int n_tok = 6, n_expert = 16, top_k = 4, n_embd = 1024, n_ff = 512;
    const std::vector<uint8_t> gate = encode(12, n_expert * n_ff, n_embd), up = encode(12, n_expert * n_ff, n_embd),
                               down = encode(12, n_expert * n_embd, n_ff);
    const std::vector<float> x = normal((size_t)n_tok * n_embd, 1.0f), lg = normal((size_t)n_tok * n_expert, 1.0f);
    const std::vector<float> out0 = normal((size_t)n_tok * n_embd, 0.1f);
    std::vector<float> elg = lg, ewts((size_t)n_tok * top_k), eacc((size_t)n_tok * top_k * n_embd), eout = out0;
    std::vector<int32_t> eids((size_t)n_tok * top_k);
    miqo_moe_route(nullptr, 0, nullptr, n_tok, n_embd, n_expert, top_k, elg.data(), eids.data(), ewts.data());
    miqo_moe M{};
    M.gate = gate.data(), M.up = up.data(), M.down = down.data();
    M.gate_type = M.up_type = M.down_type = 12;
    M.gate_plane = M.up_plane = miq_row_bytes(12, n_embd) * n_ff;
    M.down_plane = miq_row_bytes(12, n_ff) * n_embd;
    M.n_embd = n_embd, M.n_ff = n_ff, M.n_expert = n_expert;
    miqo_moe_experts(&M, x.data(), n_embd, n_tok, top_k, eids.data(), eacc.data(), n_embd, nullptr);
    miqo_moe_reduce(eacc.data(), ewts.data(), top_k, n_tok, n_embd, n_embd, eout.data(), n_embd);

    dbuf<uint8_t> dg(gate), du(up), dd(down);
    dbuf<float> dx(x), dlg(lg), wts(ewts.size()), acc(eacc.size()), out(out0);
    dbuf<int32_t> ids(eids.size());
    miq::moe_banks B;
    B.gate = dg.p, B.up = du.p, B.down = dd.p;
    B.gate_plane = B.up_plane = M.gate_plane, B.down_plane = M.down_plane;
    B.n_embd = n_embd, B.n_ff_exp = n_ff, B.n_expert = n_expert;
    be.moe_route(nullptr, 0, nullptr, n_tok, n_embd, n_expert, top_k, dlg.p, ids.p, wts.p);
    be.moe_experts(B, dx.p, n_embd, n_tok, top_k, ids.p, acc.p, n_embd);
    be.moe_reduce(acc.p, wts.p, top_k, n_tok, n_embd, n_embd, out.p, n_embd);
    be.synchronize();
    check_exact("moe_route ids", ids.get(), eids);
    check_exact("moe_route weights", wts.get(), ewts);
    check_exact("moe_route probabilities", dlg.get(), elg);
    // gate/up are formed in the reference's fp32 order, so h and its codes are
    // the oracle's and only the down projection's association differs
    check_f32("moe_experts acc", acc.get(), eacc, 1e-5);
    check_f32("moe_reduce out", out.get(), eout, 1e-5);
}

// moe_experts under stream capture: a backend whose workspace would have to
// grow throws unsupported instead of allocating; after an eager warm-up the
// call is captured, and every replay (the eager call, at a larger shape that
// grows the workspace, between replays) equals the eager result bit for bit.
static void test_moe_graph() {
    const int n_expert = 8, top_k = 2, n_embd = 512, n_ff = 256, n_tok = 4, n_big = 12;
    const std::vector<uint8_t> gate = encode(12, n_expert * n_ff, n_embd), up = encode(12, n_expert * n_ff, n_embd),
                               down = encode(12, n_expert * n_embd, n_ff);
    const std::vector<float> x = normal((size_t)n_big * n_embd, 1.0f);
    std::vector<int32_t> hid((size_t)n_big * top_k);
    for (size_t i = 0; i < hid.size(); i++) hid[i] = (int32_t)((i * 5 + i / top_k) % n_expert);
    dbuf<uint8_t> dg(gate), du(up), dd(down);
    dbuf<float> dx(x), acc((size_t)n_big * top_k * n_embd), ref((size_t)n_tok * top_k * n_embd);
    dbuf<int32_t> ids(hid);
    miq::moe_banks B;
    B.gate = dg.p, B.up = du.p, B.down = dd.p;
    B.gate_type = B.up_type = B.down_type = 12;
    B.gate_plane = B.up_plane = miq_row_bytes(12, n_embd) * n_ff;
    B.down_plane = miq_row_bytes(12, n_ff) * n_embd;
    B.n_embd = n_embd, B.n_ff_exp = n_ff, B.n_expert = n_expert;
    hipStream_t st;
    HIP_OK(hipStreamCreateWithFlags(&st, hipStreamNonBlocking));
    auto be = miq::make_gpu_backend(st);
    hipGraph_t g = nullptr;
    bool threw = false;
    HIP_OK(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
    try {
        be->moe_experts(B, dx.p, n_embd, n_tok, top_k, ids.p, acc.p, n_embd);
    } catch (const miq::unsupported &) {
        threw = true;
    }
    HIP_OK(hipStreamEndCapture(st, &g));
    if (g) HIP_OK(hipGraphDestroy(g));
    std::printf("%-36s %s\n", "moe_experts grow under capture", threw ? "unsupported OK" : "FAIL");
    if (!threw) g_fail++;
    be->moe_experts(B, dx.p, n_embd, n_tok, top_k, ids.p, ref.p, n_embd);  // warm-up: sizes the workspace
    HIP_OK(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
    be->moe_experts(B, dx.p, n_embd, n_tok, top_k, ids.p, acc.p, n_embd);
    HIP_OK(hipStreamEndCapture(st, &g));
    hipGraphExec_t ge;
    HIP_OK(hipGraphInstantiate(&ge, g, nullptr, nullptr, 0));
    const size_t nref = (size_t)n_tok * top_k * n_embd;
    be->synchronize();
    const std::vector<float> want = ref.get();
    bool ok = true;
    for (int r = 0; r < 3; r++) {
        HIP_OK(hipMemsetAsync(acc.p, 0, acc.n * sizeof(float), st));
        HIP_OK(hipGraphLaunch(ge, st));
        be->synchronize();
        std::vector<float> got = acc.get();
        got.resize(nref);
        ok = ok && std::memcmp(got.data(), want.data(), nref * sizeof(float)) == 0;
        // eager, at a larger batch: the workspace grows; the graph's old one stays valid
        be->moe_experts(B, dx.p, n_embd, r == 0 ? n_big : n_tok, top_k, ids.p, acc.p, n_embd);
        be->synchronize();
    }
    std::printf("%-36s %s\n", "moe_experts graph replays", ok ? "bit-exact OK" : "FAIL");
    if (!ok) g_fail++;
    HIP_OK(hipGraphExecDestroy(ge));
    HIP_OK(hipGraphDestroy(g));
    be.reset();
    HIP_OK(hipStreamDestroy(st));
}

int main(int argc, char **argv) {
    if (argc > 1 && !std::strcmp(argv[1], "--list")) {
        std::printf("xq i8_gemv i8_gemm i8_gemv_multi quant_gemm unsupported moe moe_graph\n%s\n", miq_version());
        return 0;
    }
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n < 1) {
        std::printf("no GPU\n");
        return 2;
    }
    hipStream_t st;
    HIP_OK(hipStreamCreateWithFlags(&st, hipStreamNonBlocking));
    auto be = miq::make_gpu_backend(st);
    std::printf("backend: %s, %s\n", be->name(), miq_version());
    test_xq(*be);
    for (uint32_t type : {12u, 13u, 14u, 8u})
        for (int TB : {1, 3, 16, 64}) test_i8(*be, type, 1536, 2048, TB);
    test_i8(*be, 12, 17408, 5120, 16);
    test_multi(*be, 1);
    test_multi(*be, 16);
    test_quant_gemm(*be);
    test_unsupported(*be);
    test_moe(*be);
    test_moe_graph();
    be.reset();
    HIP_OK(hipStreamDestroy(st));
    std::printf("%s: %d failure(s)\n", g_fail ? "FAILED" : "PASSED", g_fail);
    return g_fail ? 1 : 0;
}
