// Per-lane decoders for one 64-weight "unit" of a GGUF row and its exact int8
// dot products against a quantized activation.
//
// A unit is a quarter of a 256-value K-quant block (two 32-groups for
// Q4_K/Q5_K; one (half, 4 planes) slice of 4 16-sub-groups for Q6_K) or two
// consecutive Q8_0 blocks.  The decode GEMV, the grouped MoE GEMV and the
// parity hook all go through these functions, so one set of integer code
// extraction rules serves every kernel:
//   Q4_K  code = nibble of qs[(g/2)*32 + l], low nibble for even g    (i8.cpp:49-52)
//   Q5_K  code |= 16 when bit g of qh[l] is set                       (i8.cpp:110-113)
//   Q6_K  code = lo4 | (2-bit plane << 4), sub-group s -> (blk2 = s>>3,
//         plane = (s&7)>>1, half = s&1), wd - 32*xsum_half epilogue   (i8.cpp:129-152)
//   Q8_0  signed bytes, sum q*x8                                      (q4exp.cpp:442-470)
// The activation of group G for token t is X = x8 + (G*TB + t)*32 (8 dwords).
#pragma once

#include "miq_common.h"

namespace miq {

// ------------------------------------------------------------------ Q4_K
struct RawQ4K {
    uint4 hdr;
    uint4 q0, q1;
};
__device__ __forceinline__ RawQ4K load_q4k(__amdgpu_buffer_rsrc_t r, uint32_t blk_off, int c) {
    RawQ4K u;
    u.hdr = bload16(r, blk_off);
    u.q0 = bload16(r, blk_off + 16 + 32 * c);
    u.q1 = bload16(r, blk_off + 16 + 32 * c + 16);
    return u;
}
// exact dots of the unit's two groups against X0 (group 2c) and X1 (group 2c+1)
__device__ __forceinline__ void dots_q4k(const RawQ4K &u, const uint32_t *X0, const uint32_t *X1, int &wd0,
                                         int &wd1) {
    const uint32_t q[8] = {u.q0.x, u.q0.y, u.q0.z, u.q0.w, u.q1.x, u.q1.y, u.q1.z, u.q1.w};
    int a = 0, b = 0;
#pragma unroll
    for (int k = 0; k < 8; k++) {
        a = dot4(q[k] & 0x0F0F0F0Fu, X0[k], a);
        b = dot4((q[k] >> 4) & 0x0F0F0F0Fu, X1[k], b);
    }
    wd0 = a;
    wd1 = b;
}

// ------------------------------------------------------------------ Q5_K
struct RawQ5K {
    uint4 hdr;
    uint4 h0, h1;  // qh[32]
    uint4 q0, q1;
};
__device__ __forceinline__ RawQ5K load_q5k(__amdgpu_buffer_rsrc_t r, uint32_t blk_off, int c) {
    RawQ5K u;
    u.hdr = bload16(r, blk_off);
    u.h0 = bload16(r, blk_off + 16);
    u.h1 = bload16(r, blk_off + 32);
    u.q0 = bload16(r, blk_off + 48 + 32 * c);
    u.q1 = bload16(r, blk_off + 48 + 32 * c + 16);
    return u;
}
__device__ __forceinline__ void dots_q5k(const RawQ5K &u, int c, const uint32_t *X0, const uint32_t *X1, int &wd0,
                                         int &wd1) {
    const uint32_t q[8] = {u.q0.x, u.q0.y, u.q0.z, u.q0.w, u.q1.x, u.q1.y, u.q1.z, u.q1.w};
    const uint32_t h[8] = {u.h0.x, u.h0.y, u.h0.z, u.h0.w, u.h1.x, u.h1.y, u.h1.z, u.h1.w};
    const int g0 = 2 * c;
    int a = 0, b = 0;
#pragma unroll
    for (int k = 0; k < 8; k++) {
        const uint32_t lo = (q[k] & 0x0F0F0F0Fu) | (((h[k] >> g0) & 0x01010101u) << 4);
        const uint32_t hi = ((q[k] >> 4) & 0x0F0F0F0Fu) | (((h[k] >> (g0 + 1)) & 0x01010101u) << 4);
        a = dot4(lo, X0[k], a);
        b = dot4(hi, X1[k], b);
    }
    wd0 = a;
    wd1 = b;
}

// Q4_K/Q5_K epilogue for the unit's two groups (i8.cpp:60 / :120):
//   acc += sx * (d*sc*wd - dmin*m*xsum)
__device__ __forceinline__ float epi_kq45(uint4 hdr, int c, int wd0, int wd1, float sx0, float sx1, int xs0,
                                          int xs1) {
    const float d = h2f(hdr.x);
    const float dm = h2f(hdr.x >> 16);
    int sc0, m0, sc1, m1;
    scale_min_k4(2 * c, hdr.y, hdr.z, hdr.w, sc0, m0);
    scale_min_k4(2 * c + 1, hdr.y, hdr.z, hdr.w, sc1, m1);
    const float a0 = sx0 * (d * (float)sc0 * (float)wd0 - dm * (float)m0 * (float)xs0);
    const float a1 = sx1 * (d * (float)sc1 * (float)wd1 - dm * (float)m1 * (float)xs1);
    return a0 + a1;
}

// ------------------------------------------------------------------ Q6_K
// 6-bit code -> signed (code - 32) per byte, without inter-byte borrows
__device__ __forceinline__ uint32_t q6_signed(uint32_t code) {
    // code ^ 32 per byte, then its bit 5 (set where code < 32: the sign of
    // code - 32) copied into bits 6 and 7.  One three-input OR of the shifted
    // copies (the compiler would fold (s << 1) | (s << 2) into a multiply by 6,
    // a quarter-rate instruction)
    const uint32_t y = code ^ 0x20202020u;
    const uint32_t s = y & 0x20202020u;
    return __builtin_amdgcn_bitop3_b32(y, s << 1, s << 2, 0xFE);
}

struct RawQ6K {
    uint4 l0, l1, h;  // ql[half*16 ..], ql[32 + half*16 ..], qh[half*16 ..] of the 128-half blk2
    uint4 t;          // bytes 192..207 (scales[16])
    uint32_t dbits;   // f16 d
};
// Raw dwords of a Q6_K unit as loaded (four 16-byte pieces at dword-aligned
// offsets, each followed by the dword that completes it), so a caller can hold
// a unit in flight and decode it later with dec_q6k.
struct FetchQ6K {
    uint4 v[4];
    uint32_t e[4];
};
// blk_off is 2-byte aligned; c = blk2*2 + half
__device__ __forceinline__ FetchQ6K fetch_q6k(__amdgpu_buffer_rsrc_t r, uint32_t blk_off, int c) {
    const int blk2 = c >> 1, half = c & 1;
    const uint32_t o[4] = {blk_off + blk2 * 64 + half * 16, blk_off + blk2 * 64 + 32 + half * 16,
                           blk_off + 128 + blk2 * 32 + half * 16, blk_off + 192};
    FetchQ6K f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        f.v[i] = bload16(r, o[i] & ~3u);
        f.e[i] = bload4(r, (o[i] & ~3u) + 16);
    }
    return f;
}
// every piece of a unit shares the byte shift blk_off & 3 (all piece offsets
// differ from blk_off by multiples of 16)
__device__ __forceinline__ RawQ6K dec_q6k(const FetchQ6K &f, uint32_t blk_off) {
    const uint32_t sh = blk_off & 3u;
    uint4 o[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        o[i].x = __builtin_amdgcn_alignbyte(f.v[i].y, f.v[i].x, sh);
        o[i].y = __builtin_amdgcn_alignbyte(f.v[i].z, f.v[i].y, sh);
        o[i].z = __builtin_amdgcn_alignbyte(f.v[i].w, f.v[i].z, sh);
        o[i].w = __builtin_amdgcn_alignbyte(f.e[i], f.v[i].w, sh);
    }
    RawQ6K u;
    u.l0 = o[0];
    u.l1 = o[1];
    u.h = o[2];
    u.t = o[3];
    u.dbits = __builtin_amdgcn_alignbyte(0u, f.e[3], sh) & 0xFFFFu;
    return u;
}
__device__ __forceinline__ RawQ6K load_q6k(__amdgpu_buffer_rsrc_t r, uint32_t blk_off, int c) {
    return dec_q6k(fetch_q6k(r, blk_off, c), blk_off);
}
// exact dots of the unit's four 16-sub-groups (planes p = 0..3) against the
// half-group activations Xp (4 dwords each): wd[p] = sum code*x8
__device__ __forceinline__ void dots_q6k(const RawQ6K &u, const uint32_t *X[4], int wd[4]) {
    const uint32_t l0[4] = {u.l0.x, u.l0.y, u.l0.z, u.l0.w};
    const uint32_t l1[4] = {u.l1.x, u.l1.y, u.l1.z, u.l1.w};
    const uint32_t hh[4] = {u.h.x, u.h.y, u.h.z, u.h.w};
#pragma unroll
    for (int p = 0; p < 4; p++) {
        int a = 0;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const uint32_t src = (p & 1) ? l1[k] : l0[k];
            const uint32_t lo = (p >= 2 ? (src >> 4) : src) & 0x0F0F0F0Fu;
            const uint32_t code = lo | (((hh[k] >> (2 * p)) & 0x03030303u) << 4);
            a = dot4(code, X[p][k], a);
        }
        wd[p] = a;
    }
}
// signed 8-bit scale of plane p for this unit (scales[blk2*8 + 2p + half])
__device__ __forceinline__ int q6k_scale(const RawQ6K &u, int c, int p) {
    const int blk2 = c >> 1, half = c & 1;
    const uint32_t w = blk2 ? ((p < 2) ? u.t.z : u.t.w) : ((p < 2) ? u.t.x : u.t.y);
    return (int)(int8_t)((w >> (8 * ((2 * p + half) & 3))) & 0xFF);
}

// ------------------------------------------------------------------ Q8_0
struct RawQ80 {
    uint32_t a[8], b[8];  // the two blocks' 32 signed codes
    uint32_t da, db;      // f16 bits
};
// Raw dwords of a Q8_0 unit (68 bytes, 4-byte aligned) as loaded.
struct FetchQ80 {
    uint4 v[4];
    uint32_t e;
};
__device__ __forceinline__ FetchQ80 fetch_q80(__amdgpu_buffer_rsrc_t r, uint32_t unit_off) {
    FetchQ80 f;
#pragma unroll
    for (int i = 0; i < 4; i++) f.v[i] = bload16(r, unit_off + 16 * i);
    f.e = bload4(r, unit_off + 64);
    return f;
}
__device__ __forceinline__ RawQ80 dec_q80(const FetchQ80 &f) {
    const uint32_t d[17] = {f.v[0].x, f.v[0].y, f.v[0].z, f.v[0].w, f.v[1].x, f.v[1].y, f.v[1].z, f.v[1].w, f.v[2].x,
                            f.v[2].y, f.v[2].z, f.v[2].w, f.v[3].x, f.v[3].y, f.v[3].z, f.v[3].w, f.e};
    RawQ80 u;
    u.da = d[0] & 0xFFFFu;
#pragma unroll
    for (int k = 0; k < 8; k++) u.a[k] = __builtin_amdgcn_alignbyte(d[k + 1], d[k], 2);
    u.db = d[8] >> 16;
#pragma unroll
    for (int k = 0; k < 8; k++) u.b[k] = d[9 + k];
    return u;
}
// unit_off is 4-byte aligned (68 bytes per unit)
__device__ __forceinline__ RawQ80 load_q80(__amdgpu_buffer_rsrc_t r, uint32_t unit_off) {
    return dec_q80(fetch_q80(r, unit_off));
}
__device__ __forceinline__ void dots_q80(const RawQ80 &u, const uint32_t *X0, const uint32_t *X1, int &wd0,
                                         int &wd1) {
    int a = 0, b = 0;
#pragma unroll
    for (int k = 0; k < 8; k++) {
        a = dot4(u.a[k], X0[k], a);
        b = dot4(u.b[k], X1[k], b);
    }
    wd0 = a;
    wd1 = b;
}

}  // namespace miq
