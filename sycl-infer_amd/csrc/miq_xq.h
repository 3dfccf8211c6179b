// Activation quantizer: xq_one, one (token, group) per thread (the fused MoE
// set-up kernel), and xq_lanes, eight lanes per (token, group) (the xq kernel).
//
// Semantics of cpu_xq (src/backend/cpu/kernels/xq.cpp:10-50), bit for bit:
//   mx = max|v|; inv = 127/mx (IEEE division); q = clamp(roundf(v*inv), +-127)
//   (round half away from zero); scale = f16trunc(mx/127) as fp32, 0 for an
//   all-zero group; s0 = sum q[0..15], s1 = sum q[16..31].
// With `up` the value is silu(x)*up, silu(x) = x/(1+expf(-x)) with expf_libm,
// so that form is bit-exact too.
#pragma once

#include "miq_common.h"

namespace miq {

__device__ __forceinline__ float silu(float x) { return x / (1.0f + expf_libm(-x)); }

// One thread per (token, group): 128 contiguous input bytes, 32 output bytes.
// LAYOUT 0: group-major x8[(g*TB + t)*32], xmeta float2 {scale, 0} and xsumq
//   int2 {s0, s1} per (g, t) -- what the GEMV/GEMM kernels read.
// LAYOUT 1/2: token-major "unit" layout for one-token gathers (the grouped
//   MoE GEMV), U = K/64 units per token, unit chunk k (16 codes) of unit u at
//   x8[t*K + (k*U + u)*16], so lanes reading consecutive units read
//   consecutive 16-byte words:
//   1: unit u = values [64u, 64u+64) (Q4_K/Q5_K/Q8_0 units), chunk k = values
//      64u+16k..; meta per unit float4 {sx(2u), sx(2u+1), s(2u), s(2u+1)}
//      (s = s0+s1 as int bits) at xmeta[(t*U + u)*4]
//   2: Q6_K units u = 4b + 2*blk2 + half: chunk k = half `half` of group
//      8b + 4*blk2 + k; meta per unit {sx[4]} then {s_half[4]} (int bits) at
//      xmeta[(t*U + u)*8]
template <int LAYOUT>
__device__ __forceinline__ void xq_one(const float *__restrict__ x, const float *__restrict__ up, int x_stride,
                                       int up_stride, int8_t *__restrict__ x8, float *__restrict__ xmeta,
                                       int32_t *__restrict__ xsumq, int TB, int G, int gid) {
    const int t = gid / G;
    const int g = gid - t * G;
    const float4 *src = reinterpret_cast<const float4 *>(x + (size_t)t * x_stride + g * 32);
    float v[32];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const float4 a = src[i];
        v[4 * i + 0] = a.x;
        v[4 * i + 1] = a.y;
        v[4 * i + 2] = a.z;
        v[4 * i + 3] = a.w;
    }
    if (up) {
        const float4 *u = reinterpret_cast<const float4 *>(up + (size_t)t * up_stride + g * 32);
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float4 b = u[i];
            v[4 * i + 0] = silu(v[4 * i + 0]) * b.x;
            v[4 * i + 1] = silu(v[4 * i + 1]) * b.y;
            v[4 * i + 2] = silu(v[4 * i + 2]) * b.z;
            v[4 * i + 3] = silu(v[4 * i + 3]) * b.w;
        }
    }
    float mx = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; i++) {
        const float a = fabsf(v[i]);
        mx = mx < a ? a : mx;
    }
    const float inv = mx > 0.0f ? 127.0f / mx : 0.0f;
    int s0 = 0, s1 = 0;
    uint32_t packed[8];
#pragma unroll
    for (int w = 0; w < 8; w++) {
        uint32_t word = 0;
#pragma unroll
        for (int b = 0; b < 4; b++) {
            float r = roundf(v[4 * w + b] * inv);
            r = r < 127.0f ? r : 127.0f;
            r = -127.0f > r ? -127.0f : r;
            const int q = (int)r;
            if (4 * w + b < 16) s0 += q; else s1 += q;
            word |= ((uint32_t)q & 0xFFu) << (8 * b);
        }
        packed[w] = word;
    }
    const float scale = mx > 0.0f ? mx / 127.0f : 0.0f;
    const float sc = h2f(f2h_trunc(scale));
    const uint4 lo = make_uint4(packed[0], packed[1], packed[2], packed[3]);
    const uint4 hi = make_uint4(packed[4], packed[5], packed[6], packed[7]);
    if constexpr (LAYOUT == 0) {
        const size_t gi = (size_t)g * TB + t;
        uint4 *dst = reinterpret_cast<uint4 *>(x8 + gi * 32);
        dst[0] = lo;
        dst[1] = hi;
        reinterpret_cast<float2 *>(xmeta)[gi] = make_float2(sc, 0.0f);
        reinterpret_cast<int2 *>(xsumq)[gi] = make_int2(s0, s1);
    } else {
        const int U = G / 2;
        uint4 *row = reinterpret_cast<uint4 *>(x8 + (size_t)t * G * 32);
        if constexpr (LAYOUT == 1) {
            const int u = g >> 1, k0 = 2 * (g & 1);
            row[k0 * U + u] = lo;
            row[(k0 + 1) * U + u] = hi;
            float *m = xmeta + ((size_t)t * U + u) * 4;
            m[g & 1] = sc;
            m[2 + (g & 1)] = __int_as_float(s0 + s1);
        } else {
            const int k = g & 3, u0 = (g >> 3) * 4 + ((g >> 2) & 1) * 2;
            row[k * U + u0] = lo;
            row[k * U + u0 + 1] = hi;
            float *m = xmeta + ((size_t)t * U + u0) * 8;
            m[k] = sc;
            m[4 + k] = __int_as_float(s0);
            m[8 + k] = sc;
            m[12 + k] = __int_as_float(s1);
        }
    }
}

// The same quantizer with eight lanes per (token, group): lane l = gid8 & 7
// holds values 4l..4l+3 (one 16-byte load of x, and of up), the group's max
// and the two code sums meet across the eight lanes, and each lane stores its
// four codes as one dword.  Max and integer sums do not depend on the order,
// and every per-value step is xq_one's, so the bytes equal xq_one's.  The
// eight lanes of a group are consecutive lanes of one wave (gid8 = 8*group + l).
template <int LAYOUT>
__device__ __forceinline__ void xq_lanes(const float *__restrict__ x, const float *__restrict__ up, int x_stride,
                                         int up_stride, int8_t *__restrict__ x8, float *__restrict__ xmeta,
                                         int32_t *__restrict__ xsumq, int TB, int G, int gid8, bool live) {
    const int l = gid8 & 7, gid = gid8 >> 3;
    const int t = live ? gid / G : 0;
    const int g = live ? gid - t * G : 0;
    float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (live) {
        const float4 a = *reinterpret_cast<const float4 *>(x + (size_t)t * x_stride + g * 32 + 4 * l);
        v[0] = a.x;
        v[1] = a.y;
        v[2] = a.z;
        v[3] = a.w;
        if (up) {
            const float4 b = *reinterpret_cast<const float4 *>(up + (size_t)t * up_stride + g * 32 + 4 * l);
            v[0] = silu(v[0]) * b.x;
            v[1] = silu(v[1]) * b.y;
            v[2] = silu(v[2]) * b.z;
            v[3] = silu(v[3]) * b.w;
        }
    }
    float mx = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float a = fabsf(v[i]);
        mx = mx < a ? a : mx;
    }
#pragma unroll
    for (int o = 1; o < 8; o <<= 1) {
        const float b = __shfl_xor(mx, o, 64);
        mx = mx < b ? b : mx;
    }
    const float inv = mx > 0.0f ? 127.0f / mx : 0.0f;
    int sq = 0;
    uint32_t word = 0;
#pragma unroll
    for (int b = 0; b < 4; b++) {
        float r = roundf(v[b] * inv);
        r = r < 127.0f ? r : 127.0f;
        r = -127.0f > r ? -127.0f : r;
        const int q = (int)r;
        sq += q;
        word |= ((uint32_t)q & 0xFFu) << (8 * b);
    }
    sq += __shfl_xor(sq, 1, 64);
    sq += __shfl_xor(sq, 2, 64);            // lanes 0..3: s0, lanes 4..7: s1
    const int s1 = __shfl_xor(sq, 4, 64);  // lane 0: s1
    if (!live) return;
    const float scale = mx > 0.0f ? mx / 127.0f : 0.0f;
    const float sc = h2f(f2h_trunc(scale));
    if constexpr (LAYOUT == 0) {
        const size_t gi = (size_t)g * TB + t;
        reinterpret_cast<uint32_t *>(x8 + gi * 32)[l] = word;
        if (l == 0) {
            reinterpret_cast<float2 *>(xmeta)[gi] = make_float2(sc, 0.0f);
            reinterpret_cast<int2 *>(xsumq)[gi] = make_int2(sq, s1);
        }
    } else {
        const int U = G / 2;
        uint32_t *row = reinterpret_cast<uint32_t *>(x8 + (size_t)t * G * 32);
        if constexpr (LAYOUT == 1) {
            const int u = g >> 1, k0 = 2 * (g & 1) + (l >> 2);
            row[(k0 * U + u) * 4 + (l & 3)] = word;
            if (l == 0) {
                float *m = xmeta + ((size_t)t * U + u) * 4;
                m[g & 1] = sc;
                m[2 + (g & 1)] = __int_as_float(sq + s1);
            }
        } else {
            const int k = g & 3, u0 = (g >> 3) * 4 + ((g >> 2) & 1) * 2;
            row[(k * U + u0) * 4 + l] = word;
            if (l == 0) {
                float *m = xmeta + ((size_t)t * U + u0) * 8;
                m[k] = sc;
                m[4 + k] = __int_as_float(sq);
                m[8 + k] = sc;
                m[12 + k] = __int_as_float(s1);
            }
        }
    }
}

}  // namespace miq
