// Shared device/host definitions for the miq HIP kernels (gfx950).
//
// GGUF block layouts follow src/common/quant.h:12-41 of sycl-infer:
//   Q4_K 144 B  {f16 d @0, f16 dmin @2, u8 scales[12] @4, u8 qs[128] @16}
//   Q5_K 176 B  {d @0, dmin @2, scales @4, u8 qh[32] @16, u8 qs[128] @48}
//   Q6_K 210 B  {u8 ql[128] @0, u8 qh[64] @128, i8 scales[16] @192, f16 d @208}
//   Q8_0  34 B  {f16 d @0, i8 qs[32] @2}
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/miq.h"

namespace miq {

constexpr int kQ4KBytes = 144;
constexpr int kQ5KBytes = 176;
constexpr int kQ6KBytes = 210;
constexpr int kQ80Bytes = 34;

__host__ __device__ constexpr int block_bytes(uint32_t type) {
    return type == MIQ_TYPE_Q4_K ? kQ4KBytes
         : type == MIQ_TYPE_Q5_K ? kQ5KBytes
         : type == MIQ_TYPE_Q6_K ? kQ6KBytes
         : type == MIQ_TYPE_Q8_0 ? kQ80Bytes : 0;
}
// values per block
__host__ __device__ constexpr int block_values(uint32_t type) { return type == MIQ_TYPE_Q8_0 ? 32 : 256; }

// Error plumbing shared by the entry points (miq_capi.hip).
void set_error(const char *fmt, ...);
int check_launch(const char *what);

// ------------------------------------------------------------ device helpers

// f16 bits -> f32: exact IEEE conversion (quant.h:67-92 is the same mapping).
__device__ __forceinline__ float h2f(uint32_t bits16) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(bits16 & 0xFFFFu));
}

// f32 -> f16 bits, truncating toward zero with truncated subnormals and
// overflow to infinity (the closed form of quant.h:112-133).
__device__ __forceinline__ uint32_t f2h_trunc(float f) {
    const uint32_t bits = __builtin_bit_cast(uint32_t, f);
    const uint32_t sign = (bits >> 16) & 0x8000u;
    const int e32 = (int)((bits >> 23) & 0xFFu);
    const int e16 = e32 - 127 + 15;
    const uint32_t mant = bits & 0x7FFFFFu;
    if (e16 >= 31) return sign | 0x7C00u;
    if (e16 <= 0) {
        const int shift = 126 - e32;
        if (shift >= 32) return sign;
        return sign | ((mant | 0x800000u) >> shift);
    }
    return sign | ((uint32_t)e16 << 10) | (mant >> 13);
}

// Buffer resource over a whole tensor: loads beyond num_bytes return zero
// instead of faulting, which is what makes the 2-byte-aligned Q6_K / Q8_0
// blocks safe to fetch as aligned dwords.
// Range check is per dword: a dword that straddles num_bytes reads as zero.
// A tensor's byte size is therefore rounded up to whole dwords (the dword that
// holds its last byte is read whole), else the last 2-byte-aligned Q6_K block
// of a tensor whose size is 2 mod 4 would lose its final bytes.  Callers keep
// tensors below 4 GiB - 4 KiB, so the rounding cannot wrap.
__host__ __device__ inline uint32_t dword_span(size_t bytes) { return (uint32_t)((bytes + 3) & ~(size_t)3); }
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, uint32_t num_bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)num_bytes, 0x00020000);
}
__device__ __forceinline__ uint4 bload16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}
__device__ __forceinline__ uint32_t bload4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
}
// 16 bytes at a 2-byte-aligned offset from aligned dword loads.
__device__ __forceinline__ uint4 bload16_u2(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    const uint32_t a = off & ~3u;
    const uint32_t sh = off & 3u;
    const uint4 v = bload16(r, a);
    const uint32_t e = bload4(r, a + 16);
    uint4 o;
    o.x = __builtin_amdgcn_alignbyte(v.y, v.x, sh);
    o.y = __builtin_amdgcn_alignbyte(v.z, v.y, sh);
    o.z = __builtin_amdgcn_alignbyte(v.w, v.z, sh);
    o.w = __builtin_amdgcn_alignbyte(e, v.w, sh);
    return o;
}

__device__ __forceinline__ int dot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// get_scale_min_k4 (quant.h:136-144) for group j of a Q4_K/Q5_K block whose
// 12 scale bytes are s0 (bytes 0-3), s1 (4-7), s2 (8-11).
__device__ __forceinline__ void scale_min_k4(int j, uint32_t s0, uint32_t s1, uint32_t s2, int &sc, int &m) {
    if (j < 4) {
        sc = (s0 >> (8 * j)) & 63;
        m = (s1 >> (8 * j)) & 63;
    } else {
        const int k = j - 4;
        const uint32_t hi = (s2 >> (8 * k)) & 0xFF;  // scales[j+4]
        sc = (int)((hi & 0xF) | (((s0 >> (8 * k + 6)) & 3) << 4));
        m = (int)((hi >> 4) | (((s1 >> (8 * k + 6)) & 3) << 4));
    }
}

// expf with the host libm's exact results.  The reference's silu and softmax
// call std::exp on a float (src/backend/cpu/kernels/common.h:31-33,
// moe.cpp:107), which is glibc's expf: the method of Arm's optimized-routines
// e_expf.c (Szabolcs Nagy, 2017; glibc >= 2.27).  x*32/ln2 = k + r with k
// rounded to nearest by the 1.5*2^52 shift; exp(x) = 2^(k/32) * p(r) with a
// 32-entry table of 2^(i/32) and a cubic in double; glibc's x86-64 build runs
// its FMA variant, which fuses both products of x (k and r) and the Horner
// steps.  Exhaustively equal to the host expf over all 2^32 inputs.
__device__ __forceinline__ float expf_libm(float x) {
    // tab[i] = bits(2^(i/32)) - (i << 47), so that tab[k%32] + (k << 47) is 2^(k/32)
    constexpr uint64_t tab[32] = {
        0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
        0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
        0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
        0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
        0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
        0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
        0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
        0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull};
    constexpr double inv_ln2_n = 0x1.71547652b82fep+0 * 32.0;
    constexpr double shift = 0x1.8p+52;
    constexpr double c0 = 0x1.c6af84b912394p-5 / 32.0 / 32.0 / 32.0;
    constexpr double c1 = 0x1.ebfce50fac4f3p-3 / 32.0 / 32.0;
    constexpr double c2 = 0x1.62e42ff0c52d6p-1 / 32.0;
    const uint32_t ux = __builtin_bit_cast(uint32_t, x);
    const uint32_t abstop = (ux >> 20) & 0x7ffu;
    if (abstop >= 0x42bu) {  // |x| >= 88, inf or nan
        if (ux == 0xff800000u) return 0.0f;
        if (abstop >= 0x7f8u) return x + x;
        if (x > 0x1.62e42ep6f) return __builtin_inff();
        if (x < -0x1.9fe368p6f) return 0.0f;
    }
    const double xd = (double)x;
    double kd = __builtin_fma(inv_ln2_n, xd, shift);
    const uint64_t ki = __builtin_bit_cast(uint64_t, kd);
    kd -= shift;
    const double r = __builtin_fma(inv_ln2_n, xd, -kd);
    const double s = __builtin_bit_cast(double, tab[ki & 31] + (ki << 47));
    const double z = __builtin_fma(c0, r, c1);
    double y = __builtin_fma(c2, r, 1.0);
    y = __builtin_fma(z, r * r, y);
    return (float)(y * s);
}

// s_waitcnt immediate that waits for vmcnt <= n only (gfx9 encoding, n clamped
// to the counter's 63; expcnt and lgkmcnt left at their maximum)
__host__ __device__ constexpr int vmcnt_imm(int n) {
    return ((n > 63 ? 63 : n) & 15) | (((n > 63 ? 63 : n) >> 4) << 14) | (7 << 4) | (15 << 8);
}

// wave64 sum over aligned lane segments of width W (power of two <= 64)
template <int W> __device__ __forceinline__ float seg_sum(float v) {
#pragma unroll
    for (int o = W / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

}  // namespace miq
