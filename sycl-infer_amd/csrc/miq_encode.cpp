// Host encoder fp32 -> GGUF blocks (Q4_K, Q5_K, Q6_K, Q8_0) for synthetic
// weights.  sycl-infer ships no K-quant encoder (it only dequantizes), so this
// is written from the published ggml block layout (quant.h:12-41 documents the
// bytes): a min/max fit per 32-group (Q4_K/Q5_K) or an absmax fit per
// 16-sub-group (Q6_K), 6-/8-bit sub-scales relative to an f16 super-scale.
// Any valid block is acceptable: the kernels' parity is defined on the bytes.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <thread>
#include <vector>

#include "../../include/miq.h"

namespace {

// f32 -> f16 bits, round to nearest even (normal and subnormal range)
uint16_t f2h_rne(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    x &= 0x7FFFFFFFu;
    if (x >= 0x47800000u) return (uint16_t)(sign | 0x7C00u);  // overflow / inf / nan -> inf
    if (x < 0x38800000u) {                                      // subnormal half
        float a;
        std::memcpy(&a, &x, 4);
        const float scaled = a * 16777216.0f;  // / 2^-24
        return (uint16_t)(sign | (uint32_t)std::nearbyint(scaled));
    }
    const uint32_t mant = x & 0x7FFFFFu;
    uint32_t h = ((x >> 23) - 112) << 10 | (mant >> 13);
    const uint32_t rem = mant & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1))) h++;
    return (uint16_t)(sign | h);
}
float h2f(uint16_t h) {
    const uint32_t s = (uint32_t)(h >> 15) << 31;
    const int e = (h >> 10) & 31;
    const uint32_t m = h & 0x3FF;
    float v;
    if (e == 0) v = std::ldexp((float)m, -24);
    else if (e == 31) v = m ? NAN : INFINITY;
    else v = std::ldexp((float)(m | 0x400), e - 25);
    uint32_t b;
    std::memcpy(&b, &v, 4);
    b |= s;
    std::memcpy(&v, &b, 4);
    return v;
}
void put16(uint8_t *p, uint16_t v) {
    p[0] = (uint8_t)(v & 0xFF);
    p[1] = (uint8_t)(v >> 8);
}

// 6-bit (scale, min) of 8 groups into scales[12], the inverse of get_scale_min_k4
void pack_scales_k4(const int *sc, const int *m, uint8_t *s) {
    for (int j = 0; j < 4; j++) {
        s[j] = (uint8_t)((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
        s[j + 4] = (uint8_t)((m[j] & 63) | ((m[j + 4] >> 4) << 6));
        s[j + 8] = (uint8_t)((sc[j + 4] & 15) | ((m[j + 4] & 15) << 4));
    }
}

// Q4_K (levels = 15) or Q5_K (levels = 31): y = d*sc*q - dmin*m per 32-group
void encode_kq45(const float *x, uint8_t *blk, int levels) {
    float gscale[8], gmin[8];
    for (int g = 0; g < 8; g++) {
        float lo = 0.0f, hi = 0.0f;  // the fitted range always contains 0: min stays >= 0
        for (int i = 0; i < 32; i++) {
            lo = std::min(lo, x[g * 32 + i]);
            hi = std::max(hi, x[g * 32 + i]);
        }
        gscale[g] = (hi - lo) / (float)levels;
        gmin[g] = -lo;
    }
    const float ms = *std::max_element(gscale, gscale + 8), mm = *std::max_element(gmin, gmin + 8);
    const uint16_t dh = f2h_rne(ms > 0 ? ms / 63.0f : 0.0f), mh = f2h_rne(mm > 0 ? mm / 63.0f : 0.0f);
    const float d = h2f(dh), dmin = h2f(mh);
    int sc[8], m[8];
    for (int g = 0; g < 8; g++) {
        sc[g] = d > 0 ? std::min(63, (int)std::lround(gscale[g] / d)) : 0;
        m[g] = dmin > 0 ? std::min(63, (int)std::lround(gmin[g] / dmin)) : 0;
    }
    put16(blk, dh);
    put16(blk + 2, mh);
    pack_scales_k4(sc, m, blk + 4);
    const bool q5 = levels == 31;
    uint8_t *qh = blk + 16;
    uint8_t *qs = blk + (q5 ? 48 : 16);
    if (q5) std::memset(qh, 0, 32);
    std::memset(qs, 0, 128);
    for (int g = 0; g < 8; g++) {
        const float step = d * sc[g], off = dmin * m[g];
        for (int l = 0; l < 32; l++) {
            int q = step > 0 ? (int)std::lround((x[g * 32 + l] + off) / step) : 0;
            q = std::max(0, std::min(levels, q));
            qs[(g / 2) * 32 + l] |= (uint8_t)((q & 15) << ((g & 1) * 4));
            if (q5 && (q & 16)) qh[l] |= (uint8_t)(1u << g);
        }
    }
}

// Q6_K: y = d*scales[s]*(code-32), 16 sub-groups of 16
void encode_q6k(const float *x, uint8_t *blk) {
    float ssc[16];
    for (int s = 0; s < 16; s++) {
        float amax = 0.0f;
        for (int i = 0; i < 16; i++) amax = std::max(amax, std::fabs(x[s * 16 + i]));
        ssc[s] = amax / 31.0f;
    }
    const float ms = *std::max_element(ssc, ssc + 16);
    const uint16_t dh = f2h_rne(ms > 0 ? ms / 127.0f : 0.0f);
    const float d = h2f(dh);
    std::memset(blk, 0, 210);
    for (int s = 0; s < 16; s++) {
        const int sc = d > 0 ? std::min(127, (int)std::lround(ssc[s] / d)) : 0;
        blk[192 + s] = (uint8_t)(int8_t)sc;
        const float step = d * sc;
        // element position i of sub-group s: blk2 = s>>3, plane = (s&7)>>1, l = (s&1)*16 + i
        const int blk2 = s >> 3, plane = (s & 7) >> 1;
        for (int i = 0; i < 16; i++) {
            int q = step > 0 ? (int)std::lround(x[s * 16 + i] / step) : 0;
            q = std::max(-32, std::min(31, q)) + 32;
            const int l = (s & 1) * 16 + i;
            uint8_t &ql = blk[blk2 * 64 + ((plane & 1) ? 32 : 0) + l];
            ql |= (uint8_t)((q & 15) << (plane >= 2 ? 4 : 0));
            blk[128 + blk2 * 32 + l] |= (uint8_t)(((q >> 4) & 3) << (2 * plane));
        }
    }
    put16(blk + 208, dh);
}

// Q8_0: y = d*q, 32 values
void encode_q80(const float *x, uint8_t *blk) {
    float amax = 0.0f;
    for (int i = 0; i < 32; i++) amax = std::max(amax, std::fabs(x[i]));
    const uint16_t dh = f2h_rne(amax / 127.0f);
    const float d = h2f(dh);
    put16(blk, dh);
    for (int i = 0; i < 32; i++) {
        const int q = d > 0 ? (int)std::lround(x[i] / d) : 0;
        blk[2 + i] = (uint8_t)(int8_t)std::max(-127, std::min(127, q));
    }
}

}  // namespace

extern "C" int miq_quantize_rows(uint32_t type, const float *x, void *out, int64_t n_rows, int K, int n_threads) {
    const size_t rb = miq_row_bytes(type, K);
    if (!x || !out || n_rows < 0 || rb == 0) return MIQ_EINVAL;
    const int vb = type == MIQ_TYPE_Q8_0 ? 32 : 256;
    const int bb = (int)(rb / (size_t)(K / vb));
    const int64_t nblk = n_rows * (K / vb);
    auto work = [&](int64_t b0, int64_t b1) {
        for (int64_t b = b0; b < b1; b++) {
            const float *src = x + b * vb;
            uint8_t *dst = (uint8_t *)out + b * bb;
            switch (type) {
            case MIQ_TYPE_Q4_K: encode_kq45(src, dst, 15); break;
            case MIQ_TYPE_Q5_K: encode_kq45(src, dst, 31); break;
            case MIQ_TYPE_Q6_K: encode_q6k(src, dst); break;
            default: encode_q80(src, dst); break;
            }
        }
    };
    int nt = n_threads > 0 ? n_threads : (int)std::max(1u, std::thread::hardware_concurrency());
    nt = (int)std::min<int64_t>(nt, std::max<int64_t>(1, nblk / 1024));
    if (nt <= 1) {
        work(0, nblk);
        return MIQ_OK;
    }
    std::vector<std::thread> th;
    for (int i = 0; i < nt; i++) th.emplace_back(work, nblk * i / nt, nblk * (i + 1) / nt);
    for (auto &t : th) t.join();
    return MIQ_OK;
}
