// TEST INFRASTRUCTURE ONLY.  C-linkage wrappers over sycl-infer's own CPU
// kernels, compiled from the reference sources where they lie (see
// oracle/Makefile, target `ref`).  The resulting oracle/_ref/libsiref.so is
// used to write the golden fixtures under tests/golden/ and as the timed CPU
// baseline in bench.py; the product library never links it.
//
// Wrapped reference entry points (paths relative to the sycl-infer root):
//   si::cpu_xq                 src/backend/cpu/kernels/xq.cpp:10
//   si::cpu_i8_gemv            src/backend/cpu/kernels/i8.cpp:498
//   si::cpu_i8_gemm            src/backend/cpu/kernels/i8.cpp:518
//   si::cpu_i8_gemv1_chunked   src/backend/cpu/kernels/i8.cpp:461
//   si::cpu_q8_0_down_grouped  src/backend/cpu/kernels/q4exp.cpp:472
//   si::cpu_moe_route          src/backend/cpu/kernels/moe.cpp:72
//   si::cpu_moe_reduce         src/backend/cpu/kernels/moe.cpp:562
//   dequantize_row / f16       src/common/quant.h:67-133,1074
//   gguf_file::load            src/model/gguf.cpp:345 (dumped as text by ref_gguf_dump)
//   si::w4_pack                src/common/w4.cpp:416 (the u4 native-width store)
//   si::k5_pack                src/common/w4.cpp:409 (the k5 native 5-bit store)
#include <cstdint>
#include <algorithm>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "cpu_types.h"
#include "gguf.h"
#include "kernels/common.h"
#include "w4.h"
#include "cpu_isa.h"

using namespace si;

extern "C" {

float ref_half_to_float(uint16_t h) { return ggml_half_to_float(h); }
uint16_t ref_float_to_half(float f) { return ggml_float_to_half(f); }
float ref_silu(float x) { return cpu_silu(x); }
int ref_thread_count() { return cpu_thread_count(); }
int ref_i8_supported() { return isa().qgemv_sb != nullptr; }
const char * ref_isa_spec() { return cpu_isa_spec(); }

void ref_dequantize_row(uint32_t type, const void * data, float * y, int K) { dequantize_row(type, data, y, K); }

void ref_xq(const float * x, const float * up, int x_stride, int up_stride, int8_t * x8, float * xmeta,
            int32_t * xsumq, int TB, int K) {
    cpu_xq(x, up, x_stride, up_stride, x8, xmeta, xsumq, nullptr, TB, K);
}

static cpu_gemv_seg make_seg(const void * w, uint32_t type, int K, int n_rows, const int8_t * x8, const float * xmeta,
                             const int32_t * xsumq, float * out, int out_stride, const float * residual, float alpha) {
    cpu_gemv_seg s{};
    s.w = w;
    s.type = type;
    s.K = K;
    s.n_rows = n_rows;
    s.out = out;
    s.out_stride = out_stride;
    s.residual = residual;
    s.alpha = alpha;
    s.x8 = x8;
    s.xmeta = xmeta;
    s.xsumq = xsumq;
    s.i8 = true;
    return s;
}

void ref_i8_gemv(const void * w, uint32_t type, int K, int n_rows, const int8_t * x8, const float * xmeta,
                 const int32_t * xsumq, float * out, const float * residual, float alpha) {
    cpu_gemv_seg s = make_seg(w, type, K, n_rows, x8, xmeta, xsumq, out, n_rows, residual, alpha);
    cpu_i8_gemv(s, 0);
}

void ref_i8_gemm(const void * w, uint32_t type, int K, int n_rows, const int8_t * x8, const float * xmeta,
                 const int32_t * xsumq, float * out, int out_stride, const float * residual, float alpha, int TB) {
    cpu_gemv_seg s = make_seg(w, type, K, n_rows, x8, xmeta, xsumq, out, out_stride, residual, alpha);
    cpu_i8_gemm(s, TB, 0);
}

void ref_q8_0_gemm(const void * w, int K, int n_rows, const int8_t * x8, const float * xmeta, const int32_t * xsumq,
                   int TB, float * out, int out_stride) {
    cpu_q8_0_down_grouped(w, (size_t)(K / 32) * 34, x8, xmeta, xsumq, TB, TB, n_rows, K, out, out_stride, nullptr);
}

void ref_moe_route(const float * x, int x_stride, const float * gate_inp, int n_tok, int n_embd, int n_expert,
                   int top_k, float * logits, int32_t * ids, float * wts) {
    cpu_moe_route(x, x_stride, gate_inp, 0 /* GGML_TYPE_F32 */, n_tok, n_embd, n_expert, top_k, logits, ids, wts,
                  false);
}

void ref_moe_reduce(const float * acc, const float * wts, int top_k, int n_tok, int n_embd, int acc_stride,
                    float * out, int out_stride) {
    cpu_moe_reduce(acc, wts, top_k, n_tok, n_embd, acc_stride, out, out_stride);
}

// The integer expert composition of cpu_moe_experts_i8 (moe.cpp:476-559) for
// K-quant gate/up/down banks: gate/up through cpu_i8_gemv1_chunked, h =
// cpu_silu(g)*u, h requantised with cpu_xq (== quant_row_1), down through
// cpu_i8_gemv (the reference CPU has no Q4_K integer down store, so a K-quant
// down is the ordinary integer GEMV on K = n_ff).
void ref_moe_experts(const void * gate, const void * up, const void * down, uint32_t gtype, uint32_t utype,
                     uint32_t dtype, size_t gplane, size_t uplane, size_t dplane, int n_embd, int n_ff, int n_expert,
                     const float * x, int x_stride, int n_tok, int top_k, const int32_t * ids, float * acc,
                     int acc_stride) {
    const int K = n_embd, F = n_ff;
    std::vector<int8_t> x8(K), h8(F);
    std::vector<float> xm(K / 16), hm(F / 16), g(F), u(F), h(F);
    std::vector<int32_t> xs(K / 16), hs(F / 16);
    const int nch = std::max(1, cpu_thread_count() * 4);
    for (int p = 0; p < n_tok * top_k; p++) {
        const int t = p / top_k, e = ids[p];
        float * out = acc + (size_t)p * acc_stride;
        if (e < 0 || e >= n_expert) {
            std::memset(out, 0, sizeof(float) * K);
            continue;
        }
        cpu_xq(x + (size_t)t * x_stride, nullptr, K, 0, x8.data(), xm.data(), xs.data(), nullptr, 1, K);
        cpu_gemv_seg s = make_seg((const char *)gate + (size_t)e * gplane, gtype, K, F, x8.data(), xm.data(),
                                  xs.data(), g.data(), 1, nullptr, 1.0f);
        cpu_i8_gemv1_chunked(s, nch);
        s.w = (const char *)up + (size_t)e * uplane;
        s.type = utype;
        s.out = u.data();
        cpu_i8_gemv1_chunked(s, nch);
        for (int i = 0; i < F; i++) h[i] = cpu_silu(g[i]) * u[i];
        cpu_xq(h.data(), nullptr, F, 0, h8.data(), hm.data(), hs.data(), nullptr, 1, F);
        cpu_gemv_seg d = make_seg((const char *)down + (size_t)e * dplane, dtype, F, K, h8.data(), hm.data(),
                                  hs.data(), out, K, nullptr, 1.0f);
        cpu_i8_gemv(d, 0);
    }
}

// The grouped expert flow of moe_experts_grouped_i8 (moe.cpp:147-334): pairs
// bucketed by expert in ascending pair order; the tokens quantized once with
// cpu_xq; per expert the pairs' activation rows gathered into a block padded
// to 32 tokens with zero rows (moe.cpp:233-262) and gate/up run through
// cpu_i8_gemm_batch_serial, the row-tiled integer GEMM the reference uses
// there (its fp32 accumulation runs across blocks, i8.cpp:316-349, where the
// per-pair GEMV sums each block first); h = cpu_silu(g)*u; all pairs' h
// quantized by one cpu_xq.  The reference's grouped down reads a symmetric
// int8 store it builds at load (or Q5_1); for a K-quant down bank the same
// tiled GEMM runs on each expert's gathered h rows.  Pairs with an expert id
// out of range get zero rows.
void ref_moe_experts_grouped(const void * gate, const void * up, const void * down, uint32_t gtype, uint32_t utype,
                             uint32_t dtype, size_t gplane, size_t uplane, size_t dplane, int n_embd, int n_ff,
                             int n_expert, const float * x, int x_stride, int n_tok, int top_k, const int32_t * ids,
                             float * acc, int acc_stride) {
    const int K = n_embd, F = n_ff, E = n_expert, np_ = n_tok * top_k;
    const int G = K / 32, Gd = F / 32;
    std::vector<int> off(E + 1, 0), cur, pairs(np_);
    for (int p = 0; p < np_; p++)
        if (ids[p] >= 0 && ids[p] < E) off[ids[p] + 1]++;
    for (int e = 0; e < E; e++) off[e + 1] += off[e];
    cur = off;
    for (int p = 0; p < np_; p++) {
        if (ids[p] >= 0 && ids[p] < E) pairs[cur[ids[p]]++] = p;
        else std::memset(acc + (size_t)p * acc_stride, 0, sizeof(float) * K);
    }
    std::vector<int8_t> x8((size_t)K * n_tok);
    std::vector<float> xm((size_t)G * n_tok * 2);
    std::vector<int32_t> xs((size_t)G * n_tok * 2);
    cpu_xq(x, nullptr, x_stride, 0, x8.data(), xm.data(), xs.data(), nullptr, n_tok, K);
    std::vector<float> hbuf((size_t)np_ * F, 0.0f);
    auto gather = [](const int8_t * s8, const float * sm, const int32_t * ss, int S, int Gn, const int * rows, int P,
                     int PP, std::vector<int8_t> & d8, std::vector<float> & dm, std::vector<int32_t> & ds) {
        d8.assign((size_t)Gn * PP * 32, 0);
        dm.assign((size_t)Gn * PP * 2, 0.0f);
        ds.assign((size_t)Gn * PP * 2, 0);
        for (int v = 0; v < P; v++)
            for (int g = 0; g < Gn; g++) {
                const size_t dst = (size_t)g * PP + v, src = (size_t)g * S + rows[v];
                std::memcpy(d8.data() + dst * 32, s8 + src * 32, 32);
                dm[dst * 2] = sm[src * 2];
                dm[dst * 2 + 1] = sm[src * 2 + 1];
                ds[dst * 2] = ss[src * 2];
                ds[dst * 2 + 1] = ss[src * 2 + 1];
            }
    };
    std::vector<int8_t> e8;
    std::vector<float> em, gb, ub, ob;
    std::vector<int32_t> es;
    std::vector<int> toks;
    for (int e = 0; e < E; e++) {
        const int b = off[e], P = off[e + 1] - b;
        if (P <= 0) continue;
        const int PP = (P + 31) & ~31;
        toks.resize(P);
        for (int v = 0; v < P; v++) toks[v] = pairs[b + v] / top_k;
        gather(x8.data(), xm.data(), xs.data(), n_tok, G, toks.data(), P, PP, e8, em, es);
        gb.assign((size_t)F * PP, 0.0f);
        ub.assign((size_t)F * PP, 0.0f);
        cpu_i8_gemm_batch_serial(gtype, (const char *)gate + (size_t)e * gplane, e8.data(), em.data(), es.data(), K, F,
                                 PP, gb.data(), F);
        cpu_i8_gemm_batch_serial(utype, (const char *)up + (size_t)e * uplane, e8.data(), em.data(), es.data(), K, F,
                                 PP, ub.data(), F);
        for (int v = 0; v < P; v++)
            for (int i = 0; i < F; i++)
                hbuf[(size_t)pairs[b + v] * F + i] = cpu_silu(gb[(size_t)v * F + i]) * ub[(size_t)v * F + i];
    }
    std::vector<int8_t> h8((size_t)F * np_);
    std::vector<float> hm((size_t)Gd * np_ * 2);
    std::vector<int32_t> hs((size_t)Gd * np_ * 2);
    cpu_xq(hbuf.data(), nullptr, F, 0, h8.data(), hm.data(), hs.data(), nullptr, np_, F);
    for (int e = 0; e < E; e++) {
        const int b = off[e], P = off[e + 1] - b;
        if (P <= 0) continue;
        const int PP = (P + 31) & ~31;
        gather(h8.data(), hm.data(), hs.data(), np_, Gd, pairs.data() + b, P, PP, e8, em, es);
        ob.assign((size_t)K * PP, 0.0f);
        cpu_i8_gemm_batch_serial(dtype, (const char *)down + (size_t)e * dplane, e8.data(), em.data(), es.data(), F, K,
                                 PP, ob.data(), K);
        for (int v = 0; v < P; v++)
            std::memcpy(acc + (size_t)pairs[b + v] * acc_stride, ob.data() + (size_t)v * K, sizeof(float) * K);
    }
}

// One text line per fact of a loaded gguf_file, in the form the tests build
// from miq's C ABI:  "version V", "split COUNT NO SHARDS", "kv KEY VALUE",
// "t NAME TYPE D0,D1.. OFFSET MAPOFF SHARD"; "ERR message" when load throws.
// VALUE: "T:U64:I64:F64:HEXSTR" for a scalar or string, "9[N](V;V;..)" for
// an array (F64 printed with %.17g).
static void dump_val(std::string & o, const gguf_kv & v) {
    char buf[128];
    if (v.type == 9) {
        snprintf(buf, sizeof(buf), "9[%zu](", v.arr.size());
        o += buf;
        for (size_t i = 0; i < v.arr.size(); i++) {
            if (i) o += ";";
            dump_val(o, v.arr[i]);
        }
        o += ")";
        return;
    }
    snprintf(buf, sizeof(buf), "%u:%llu:%lld:%.17g:", v.type, (unsigned long long)v.u64, (long long)v.i64, v.f64);
    o += buf;
    for (unsigned char c : v.str) {
        snprintf(buf, sizeof(buf), "%02x", c);
        o += buf;
    }
}

size_t ref_gguf_dump(const char * path, char * out, size_t cap) {
    std::string o;
    try {
        gguf_file f;
        f.load(path);
        char buf[256];
        snprintf(buf, sizeof(buf), "version %u\nsplit %d %d %zu\n", f.version, f.split_count, f.split_no, f.shards.size());
        o += buf;
        for (auto & e : f.kv) {
            o += "kv " + e.first + " ";
            dump_val(o, e.second);
            o += "\n";
        }
        for (auto & t : f.tensors) {
            o += "t " + t.name + " " + std::to_string(t.type) + " ";
            for (size_t d = 0; d < t.dims.size(); d++) {
                if (d) o += ",";
                o += std::to_string(t.dims[d]);
            }
            int shard = 0;
            for (size_t s = 0; s < f.shards.size(); s++) {
                if ((const uint8_t *)t.data >= (const uint8_t *)f.shards[s].base) shard = (int)s;
            }
            snprintf(buf, sizeof(buf), " %llu %llu %d\n", (unsigned long long)t.offset,
                     (unsigned long long)((const uint8_t *)t.data - (const uint8_t *)f.map_base), shard);
            o += buf;
        }
    } catch (const std::exception & e) {
        o = std::string("ERR ") + e.what() + "\n";
    }
    if (out && cap) {
        size_t n = std::min(cap - 1, o.size());
        memcpy(out, o.data(), n);
        out[n] = 0;
    }
    return o.size();
}

// ggml_type_name / ggml_blck_size / ggml_type_size (src/model/gguf.cpp:13-90);
// returns -1 where the reference throws.
int ref_ggml_geom(uint32_t t, size_t * blck, size_t * size, const char ** name) {
    *name = ggml_type_name(t);
    try {
        *blck = ggml_blck_size(t);
        *size = ggml_type_size(t);
    } catch (const std::exception &) {
        return -1;
    }
    return 0;
}

// si::w4_pack into caller buffers of N*K/2, (K/32)*N and (K/32)*N entries;
// returns 0, or -1 where the reference declines the type/shape.
int ref_w4_pack(uint32_t type, const void * src, int K, int N, uint8_t * vals, uint16_t * scale, uint16_t * off) {
    w4t w;
    if (!w4_pack(type, src, K, N, w) || w.G != 32) {
        return -1;
    }
    memcpy(vals, w.vals.data(), w.vals.size());
    memcpy(scale, w.scale.data(), w.scale.size() * 2);
    memcpy(off, w.off.data(), w.off.size() * 2);
    return 0;
}

// si::k5_pack into caller buffers (vals N*K/2, hi N*K/8, scale/off (K/32)*N)
int ref_k5_pack(uint32_t type, const void * src, int K, int N, uint8_t * vals, uint8_t * hi, uint16_t * scale,
                uint16_t * off) {
    k5t w;
    if (!k5_pack(type, src, K, N, w)) {
        return -1;
    }
    memcpy(vals, w.vals.data(), w.vals.size());
    memcpy(hi, w.hi.data(), w.hi.size());
    memcpy(scale, w.scale.data(), w.scale.size() * 2);
    memcpy(off, w.off.data(), w.off.size() * 2);
    return 0;
}

} // extern "C"
