// u4 native-width weight store (the reference's `w4t`, src/common/w4.h:55-66):
// the repack of a Q4_K tensor, the per-32-group activation quantizer its GEMV
// reads, and the one-token GEMV over it.
//
// Store layout (kept as the reference defines it, so a caller's planes carry over):
//   vals [N][K/2]     element k of row n in byte (n*K+k)/2, low nibble first
//   scale[g*N+n]      f16 step  d*sc_g      of 32-group g (truncating f16)
//   off  [g*N+n]      f16 offset -dmin*m_g  (so w = step*q + off exactly up to
//                     the f16 rounding of the two constants)
// Activation (act_quant_grp_launch, src/backend/dnnl_gemm.cpp:100-146):
//   xq [M][K] int8, one symmetric scale per 32-group; asa[M][K/32] its f16
//   (round to nearest) scale; xs[M][K/32] the group's code sum; axe/axo[M][K/2]
//   the even / odd elements (a byte of `vals` holds k and k+1).
// GEMV (w4_gemv_impl, src/backend/gpu/kernels/w4_gemv.cpp:79-154):
//   out[n] = alpha * sum_g asa[g]*(step[g][n]*QDOT_g[n] + off[g][n]*xs[g]) + residual[n]
#include "miq_internal.h"
#include "miq_xq.h"

namespace miq {

// ------------------------------------------------------------------ repack

// One thread per (32-group g, row n), n fastest so the scale/off stores of a
// wave are contiguous.  w4.cpp:160-212 (pack_q4_K): group j of a block takes
// nibble (j & 1) of qs[(j/2)*32 + l]; step = f16(d*sc_j), off = f16(-dmin*m_j).
__global__ __launch_bounds__(256) void w4_pack_kernel(const uint8_t *src, int K, int N, uint8_t *vals,
                                                      uint16_t *scale, uint16_t *off) {
    const int ng = K / 32;
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (size_t)ng * N) return;
    const int g = (int)(i / N), n = (int)(i % N);
    const int b = g >> 3, j = g & 7;
    const uint8_t *blk = src + (size_t)n * (size_t)(K / 256) * kQ4KBytes + (size_t)b * kQ4KBytes;
    const uint32_t hd = *reinterpret_cast<const uint32_t *>(blk);
    const uint4 sc12 = *reinterpret_cast<const uint4 *>(blk);  // d, dmin, scales[0..11]
    int sc, m;
    scale_min_k4(j, sc12.y, sc12.z, sc12.w, sc, m);
    const float d = h2f(hd & 0xFFFFu), mn = h2f(hd >> 16);
    scale[i] = (uint16_t)f2h_trunc(d * (float)sc);
    off[i] = (uint16_t)f2h_trunc(-mn * (float)m);
    const uint4 *qs = reinterpret_cast<const uint4 *>(blk + 16 + (j >> 1) * 32);
    const uint4 q0 = qs[0], q1 = qs[1];
    const uint32_t in[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
    const int sh = (j & 1) * 4;
    uint32_t o[4];
#pragma unroll
    for (int w = 0; w < 4; w++) {
        // codes of elements 8w..8w+7 are the nibbles of in[2w], in[2w+1]
        const uint32_t a = (in[2 * w] >> sh) & 0x0F0F0F0Fu, c = (in[2 * w + 1] >> sh) & 0x0F0F0F0Fu;
        // byte i of the output pairs elements 2i (low) and 2i+1 (high)
        const uint32_t lo_a = (a & 0xFFu) | ((a >> 4) & 0xF0u) | ((a >> 8) & 0xFF00u) | ((a >> 12) & 0xF000u);
        const uint32_t lo_c = (c & 0xFFu) | ((c >> 4) & 0xF0u) | ((c >> 8) & 0xFF00u) | ((c >> 12) & 0xF000u);
        o[w] = (lo_a & 0xFFFFu) | (lo_c << 16);
    }
    *reinterpret_cast<uint4 *>(vals + (size_t)n * (K / 2) + (size_t)g * 16) = make_uint4(o[0], o[1], o[2], o[3]);
}

// k5: pack_q5_K (w4.cpp:336-403).  The nibble plane is the u4 one (low 4 bits
// of the Q5_K code: nibble (j & 1) of qs[(j/2)*32 + l]); the fifth bit of
// element l of group j is bit 2*(j/2) + (j & 1) of qh[l] and goes to the hi
// plane's word for the group: bit l/2 for even l, bit 16 + l/2 for odd l.
// Q5_K block: {d @0, dmin @2, scales @4, qh[32] @16, qs[128] @48}, 176 bytes.
__global__ __launch_bounds__(256) void k5_pack_kernel(const uint8_t *src, int K, int N, uint8_t *vals, uint8_t *hi,
                                                      uint16_t *scale, uint16_t *off) {
    const int ng = K / 32;
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (size_t)ng * N) return;
    const int g = (int)(i / N), n = (int)(i % N);
    const int b = g >> 3, j = g & 7;
    const uint8_t *blk = src + (size_t)n * (size_t)(K / 256) * kQ5KBytes + (size_t)b * kQ5KBytes;
    const uint4 sc12 = *reinterpret_cast<const uint4 *>(blk);  // d, dmin, scales[0..11]
    int sc, m;
    scale_min_k4(j, sc12.y, sc12.z, sc12.w, sc, m);
    const float d = h2f(sc12.x & 0xFFFFu), mn = h2f(sc12.x >> 16);
    scale[i] = (uint16_t)f2h_trunc(d * (float)sc);
    off[i] = (uint16_t)f2h_trunc(-mn * (float)m);
    const uint4 *qs = reinterpret_cast<const uint4 *>(blk + 48 + (j >> 1) * 32);
    const uint4 q0 = qs[0], q1 = qs[1];
    const uint32_t in[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
    const int sh = (j & 1) * 4;
    uint32_t o[4];
#pragma unroll
    for (int w = 0; w < 4; w++) {
        const uint32_t a = (in[2 * w] >> sh) & 0x0F0F0F0Fu, c = (in[2 * w + 1] >> sh) & 0x0F0F0F0Fu;
        const uint32_t lo_a = (a & 0xFFu) | ((a >> 4) & 0xF0u) | ((a >> 8) & 0xFF00u) | ((a >> 12) & 0xF000u);
        const uint32_t lo_c = (c & 0xFFu) | ((c >> 4) & 0xF0u) | ((c >> 8) & 0xFF00u) | ((c >> 12) & 0xF000u);
        o[w] = (lo_a & 0xFFFFu) | (lo_c << 16);
    }
    *reinterpret_cast<uint4 *>(vals + (size_t)n * (K / 2) + (size_t)g * 16) = make_uint4(o[0], o[1], o[2], o[3]);
    const uint8_t *qh = blk + 16;
    const int p = 2 * (j >> 1) + (j & 1);
    uint32_t h = 0;
#pragma unroll
    for (int l = 0; l < 32; l++) h |= (uint32_t)((qh[l] >> p) & 1) << ((l & 1) * 16 + (l >> 1));
    *reinterpret_cast<uint32_t *>(hi + (size_t)n * (K / 8) + (size_t)g * 4) = h;
}

// ------------------------------------------------------ activation quantizer

// Two lanes per 32-group, 16 values each; the pair's max and code sum through
// a DPP swap.  dnnl_gemm.cpp:120-146: sc = max/127 (1 for an all-zero group),
// q = clamp(round(v * (1/sc)), -127, 127); asa = f16(sc) rounded to nearest.
__global__ __launch_bounds__(256) void w4_act_kernel(const float *x, const float *up, int x_stride, int up_stride,
                                                     int M, int K, int8_t *xq, uint16_t *asa, float *xs,
                                                     int8_t *axe, int8_t *axo) {
    const int ng = K / 32;
    const int p = blockIdx.x * 128 + (threadIdx.x >> 1), h = threadIdx.x & 1;
    const bool ok = p < M * ng;  // both lanes of a pair agree, the DPP partner is always live
    const int m = ok ? p / ng : 0, g = ok ? p % ng : 0;
    float v[16];
    const float4 *xp = reinterpret_cast<const float4 *>(x + (size_t)m * x_stride + g * 32 + 16 * h);
#pragma unroll
    for (int c = 0; c < 4; c++) {
        float4 a = ok ? xp[c] : make_float4(0.f, 0.f, 0.f, 0.f);
        if (up && ok) {
            const float4 b = reinterpret_cast<const float4 *>(up + (size_t)m * up_stride + g * 32 + 16 * h)[c];
            a = make_float4(silu(a.x) * b.x, silu(a.y) * b.y, silu(a.z) * b.z, silu(a.w) * b.w);
        }
        v[4 * c] = a.x, v[4 * c + 1] = a.y, v[4 * c + 2] = a.z, v[4 * c + 3] = a.w;
    }
    float mx = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; i++) mx = fmaxf(mx, fabsf(v[i]));
    mx = fmaxf(mx, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, mx), 0xB1, 0xF, 0xF, false)));
    const float sc = mx > 0.0f ? mx / 127.0f : 1.0f;
    const float inv = 1.0f / sc;
    int s = 0;
    uint32_t wq[4] = {0, 0, 0, 0}, we[2] = {0, 0}, wo[2] = {0, 0};
#pragma unroll
    for (int i = 0; i < 16; i++) {
        float r = roundf(v[i] * inv);
        r = fminf(fmaxf(r, -127.0f), 127.0f);
        const int q = (int)r;
        s += q;
        const uint32_t b = (uint32_t)q & 0xFFu;
        wq[i >> 2] |= b << (8 * (i & 3));
        if (i & 1) wo[i >> 3] |= b << (8 * ((i >> 1) & 3));
        else we[i >> 3] |= b << (8 * ((i >> 1) & 3));
    }
    s += __builtin_amdgcn_mov_dpp(s, 0xB1, 0xF, 0xF, false);
    if (!ok) return;
    if (xq) *reinterpret_cast<uint4 *>(xq + (size_t)m * K + g * 32 + 16 * h) = make_uint4(wq[0], wq[1], wq[2], wq[3]);
    if (axe) {
        const size_t o = (size_t)m * (K / 2) + g * 16 + 8 * h;
        *reinterpret_cast<uint2 *>(axe + o) = make_uint2(we[0], we[1]);
        *reinterpret_cast<uint2 *>(axo + o) = make_uint2(wo[0], wo[1]);
    }
    if (h == 0) {
        asa[(size_t)m * ng + g] = __builtin_bit_cast(uint16_t, (_Float16)sc);
        xs[(size_t)m * ng + g] = (float)s;
    }
}

// ------------------------------------------------------------------- GEMV

constexpr int kW4MaxSegs = 8;

// One output segment: a store and where its rows go (w4_grp_seg, kernels.h:226-234).
struct W4Seg {
    const uint8_t *vals;
    const uint16_t *scale, *off;
    const uint8_t *hi;  // k5 fifth-bit plane [N][K/8] (K5 kernels only)
    float *out;
    const float *residual;
    float alpha;
    int N, tile0;       // rows; first tile of the segment in the launch
    int out_stride;     // token stride of out / residual (TB > 1)
    uint32_t vals_bytes, meta_bytes, hi_bytes;
};

struct W4Args {
    W4Seg seg[kW4MaxSegs];
    int n_segs, ntiles, K, mstride, tb;
    int kparts, gpp;          // K split across workgroups: parts, groups per part
    float *part;              // kparts > 1: partial sums [kparts][N] (one segment)
    const int8_t *axe, *axo;  // the quantized activation (not Q)
    const uint16_t *asa;
    const float *xs;
    const float *x, *up;      // the fp32 activation (Q: quantized in the launch)
};

constexpr size_t kW4MaxLds = 64 * 1024;

// meta row stride in dwords: >= ng and = 16 mod 64, so the four rows a wave
// reads at once sit on disjoint bank ranges
__host__ __device__ inline int w4_mstride(int ng) { return (ng + 47) / 64 * 64 + 16; }
__host__ __device__ inline size_t w4_lds_bytes(int ng, int rows, int ks, int tb = 1) {
    return (size_t)tb * ng * 40 + (size_t)rows * w4_mstride(ng) * 4 + (size_t)ks * rows * tb * 4;
}

// One workgroup per 4*RW rows, RW*KS waves: wave w takes row-quad w % RW and
// the K-part w / RW (KS parts of whole 16-group runs); 16 lanes per row.  LDS holds the activation
// (even plane, odd plane, {asa, asa*xs} per group) and the tile's (step, off)
// pairs row-major; lane j of a row owns groups j, j+16, ... of its K-part.
// Order of work: the staging loads (activation, then the tile's scale/off runs)
// go out first, then every weight load of the lane; the LDS writes wait only
// for the staging loads (the oldest), so the weights stay in flight across
// the barrier.  The 32-byte scale/off runs of a tile share their lines with
// the neighbouring tiles, so tiles are laid out XCD-major (consecutive tiles
// on one XCD meet in its L2).
// AL: scale/off 16-byte aligned with N % 8 == 0 (16-byte staging loads).
// Staging slots: one activation group and two 8-row scale/off runs per
// thread, so ng <= 64*RW*KS and ng <= 256*KS (the host picks RW, KS to fit).
// A 32-row tile (RW = 8) reads whole 64-byte sectors of the scale/off lines.
// Q: the workgroup quantizes the fp32 activation itself into the same LDS
// image (act_quant_grp's arithmetic, as w4_act_kernel: two lanes per group,
// ng <= NT/2), so the result is bit-identical to miq_w4_act + the plain form.
// Segments: tiles are numbered across the launch's segments; a tile never
// straddles two.
// TB tokens (staged activation, u4 or k5): the LDS image holds A.tb <= TB
// activations (token-major, the planes' own [M][...] order) and each weight
// unit is decoded once for all of them; slots past A.tb are neither staged nor
// computed.
template <int NU, int RW, int KS, bool AL, bool K5, bool Q, int TB>
__global__ __launch_bounds__(64 * RW * KS) void w4_gemv_kernel(W4Args A) {
    constexpr int R = 4 * RW, NT = 64 * RW * KS;
    extern __shared__ __align__(16) uint8_t lds[];
    const int ngt = A.K / 32;
    const int per = (A.ntiles * A.kparts + 7) >> 3;
    const int wid = (blockIdx.x & 7) * per + (blockIdx.x >> 3);
    if (wid >= A.ntiles * A.kparts) return;
    // K part kp covers groups [g0, g0 + ng); tiles of one part are consecutive
    const int kp = wid / A.ntiles, tile = wid % A.ntiles;
    const int g0 = kp * A.gpp, ng = min(A.gpp, ngt - g0);
    W4Seg S = A.seg[0];
#pragma unroll
    for (int q = 1; q < kW4MaxSegs; q++)
        if (q < A.n_segs && tile >= A.seg[q].tile0) S = A.seg[q];
    const int n0 = (tile - S.tile0) * R;
    static_assert(TB == 1 || !Q, "several tokens: a staged activation");
    const int tbl = TB == 1 ? 1 : A.tb;  // live tokens
    // the image is carved for the live tokens, as the host sized it
    uint8_t *le = lds, *lo = lds + (size_t)tbl * ng * 16;
    float2 *lsx = reinterpret_cast<float2 *>(lds + (size_t)tbl * ng * 32);
    uint32_t *lm = reinterpret_cast<uint32_t *>(lds + (size_t)tbl * ng * 40);
    float *lred = reinterpret_cast<float *>(lm + R * A.mstride);

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r = (wave % RW) * 4 + (lane >> 4), j = lane & 15, kq = wave / RW;
    const int n = n0 + r;
    const bool row_ok = n < S.N;
    const int U = (ng + 15) >> 4, UQ = (U + KS - 1) / KS;
    const int u_lo = kq * UQ, u_hi = min(U, u_lo + UQ);

    // staging loads (out-of-range slots read zeros past the buffer ends)
    uint4 se[TB], so[TB];
    uint32_t sa_bits[TB];
    float sxs[TB];
    float4 fx[4], fu[4];
    if constexpr (Q) {
        const uint32_t xb = (uint32_t)A.K * 4;
        const __amdgpu_buffer_rsrc_t rfx = make_rsrc(A.x, xb), rfu = make_rsrc(A.up, A.up ? xb : 0);
        const uint32_t base = (uint32_t)((g0 + (tid >> 1)) * 32 + 16 * (tid & 1)) * 4;  // past K*4: zeros
#pragma unroll
        for (int c = 0; c < 4; c++) {
            fx[c] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rfx, base + 16 * c, 0, 0));
            if (A.up) fu[c] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rfu, base + 16 * c, 0, 0));
        }
    } else {
        // LDS index c = t*ng + g of this K part; the planes are [TB][K/2], [TB][K/32]
        const uint32_t na = (uint32_t)(tbl * ng), nt = (uint32_t)(tbl * ngt);
        const __amdgpu_buffer_rsrc_t re = make_rsrc(A.axe, nt * 16), rod = make_rsrc(A.axo, nt * 16);
        const __amdgpu_buffer_rsrc_t ra = make_rsrc(A.asa, dword_span((size_t)nt * 2)), rx = make_rsrc(A.xs, nt * 4);
#pragma unroll
        for (int t = 0; t < TB; t++) {
            const uint32_t c = (uint32_t)(tid + t * NT);
            const uint32_t ca = c < na ? (c / ng) * ngt + g0 + c % ng : nt;
            se[t] = bload16(re, ca * 16), so[t] = bload16(rod, ca * 16);
            sa_bits[t] = bload4(ra, (ca * 2) & ~3u) >> (16 * (ca & 1));
            sxs[t] = __builtin_bit_cast(float, bload4(rx, ca * 4));
        }
    }
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(S.scale, S.meta_bytes), ro = make_rsrc(S.off, S.meta_bytes);
    uint32_t ms[2][8], mo[2][8];
#pragma unroll
    for (int s = 0; s < 2; s++) {
        const int c = tid + s * NT;
        const int g = c / (R / 8), hf = c % (R / 8);
        const uint32_t e0 = (uint32_t)(g0 + g) * S.N + n0 + 8 * hf;  // first f16 element of this 8-row run
        if constexpr (AL) {
            const uint32_t b = c < (R / 8) * ng ? e0 * 2 : S.meta_bytes;
            const uint4 a = bload16(rs, b), o = bload16(ro, b);
            const uint32_t av[4] = {a.x, a.y, a.z, a.w}, ov[4] = {o.x, o.y, o.z, o.w};
#pragma unroll
            for (int q = 0; q < 4; q++) {
                ms[s][2 * q] = av[q] & 0xFFFFu, ms[s][2 * q + 1] = av[q] >> 16;
                mo[s][2 * q] = ov[q] & 0xFFFFu, mo[s][2 * q + 1] = ov[q] >> 16;
            }
        } else {
#pragma unroll
            for (int q = 0; q < 8; q++) {
                const uint32_t e = c < (R / 8) * ng ? e0 + q : S.meta_bytes;  // e*2 past the end: zeros
                ms[s][q] = bload4(rs, (e * 2) & ~3u) >> (16 * (e & 1)) & 0xFFFFu;
                mo[s][q] = bload4(ro, (e * 2) & ~3u) >> (16 * (e & 1)) & 0xFFFFu;
            }
        }
    }
    // every weight load of the lane
    const __amdgpu_buffer_rsrc_t rv = make_rsrc(S.vals, S.vals_bytes);
    const uint32_t rowb = (uint32_t)n * (uint32_t)(A.K / 2);
    uint4 wv[NU];
#pragma unroll
    for (int i = 0; i < NU; i++) {
        const int u = u_lo + i, g = j + 16 * u;
        wv[i] = bload16(rv, row_ok && u < u_hi && g < ng ? rowb + (uint32_t)(g0 + g) * 16 : S.vals_bytes);
    }
    uint32_t hv[K5 ? NU : 1];
    if constexpr (K5) {
        const __amdgpu_buffer_rsrc_t rh = make_rsrc(S.hi, S.hi_bytes);
#pragma unroll
        for (int i = 0; i < NU; i++) {
            const int u = u_lo + i, g = j + 16 * u;
            hv[i] = bload4(rh, row_ok && u < u_hi && g < ng ? (uint32_t)n * (uint32_t)(A.K / 8) + (g0 + g) * 4 : S.hi_bytes);
        }
    }
    if constexpr (Q) {
        // dnnl_gemm.cpp:120-146: sc = max/127 (1 for an all-zero group),
        // q = clamp(round(v * (1/sc)), -127, 127), asa = f16(sc) to nearest
        const int g = tid >> 1, h = tid & 1;
        float v[16];
#pragma unroll
        for (int c = 0; c < 4; c++) {
            float4 a = fx[c];
            if (A.up) {
                const float4 b = fu[c];
                a = make_float4(silu(a.x) * b.x, silu(a.y) * b.y, silu(a.z) * b.z, silu(a.w) * b.w);
            }
            v[4 * c] = a.x, v[4 * c + 1] = a.y, v[4 * c + 2] = a.z, v[4 * c + 3] = a.w;
        }
        float mx = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; i++) mx = fmaxf(mx, fabsf(v[i]));
        mx = fmaxf(mx, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, mx), 0xB1, 0xF, 0xF, false)));
        const float sc = mx > 0.0f ? mx / 127.0f : 1.0f;
        const float inv = 1.0f / sc;
        int sum = 0;
        uint32_t we[2] = {0, 0}, wo[2] = {0, 0};
#pragma unroll
        for (int i = 0; i < 16; i++) {
            float rr = roundf(v[i] * inv);
            rr = fminf(fmaxf(rr, -127.0f), 127.0f);
            const int q = (int)rr;
            sum += q;
            const uint32_t b = (uint32_t)q & 0xFFu;
            if (i & 1) wo[i >> 3] |= b << (8 * ((i >> 1) & 3));
            else we[i >> 3] |= b << (8 * ((i >> 1) & 3));
        }
        sum += __builtin_amdgcn_mov_dpp(sum, 0xB1, 0xF, 0xF, false);
        if (g < ng) {
            *reinterpret_cast<uint2 *>(le + g * 16 + 8 * h) = make_uint2(we[0], we[1]);
            *reinterpret_cast<uint2 *>(lo + g * 16 + 8 * h) = make_uint2(wo[0], wo[1]);
            if (h == 0) {
                const float sa = (float)(_Float16)sc;
                lsx[g] = make_float2(sa, sa * (float)sum);
            }
        }
    } else {
#pragma unroll
        for (int t = 0; t < TB; t++) {
            const int c = tid + t * NT;
            if (c < tbl * ng) {
                *reinterpret_cast<uint4 *>(le + c * 16) = se[t];
                *reinterpret_cast<uint4 *>(lo + c * 16) = so[t];
                const float sa = h2f(sa_bits[t]);
                lsx[c] = make_float2(sa, sa * sxs[t]);
            }
        }
    }
#pragma unroll
    for (int s = 0; s < 2; s++) {
        const int c = tid + s * NT;
        if (c < (R / 8) * ng) {
            const int g = c / (R / 8), hf = c % (R / 8);
#pragma unroll
            for (int q = 0; q < 8; q++) lm[(8 * hf + q) * A.mstride + g] = ms[s][q] | (mo[s][q] << 16);
        }
    }
    __syncthreads();

    float acc[TB];
#pragma unroll
    for (int t = 0; t < TB; t++) acc[t] = 0.0f;
    const uint32_t *mrow = lm + r * A.mstride;
#pragma unroll
    for (int i = 0; i < NU; i++) {
        const int u = u_lo + i, g = j + 16 * u;
        if (u < u_hi && g < ng) {
            const uint4 w = wv[i];
            uint32_t c[8] = {w.x & 0x0F0F0F0Fu, w.y & 0x0F0F0F0Fu, w.z & 0x0F0F0F0Fu, w.w & 0x0F0F0F0Fu,
                             (w.x >> 4) & 0x0F0F0F0Fu, (w.y >> 4) & 0x0F0F0F0Fu, (w.z >> 4) & 0x0F0F0F0Fu,
                             (w.w >> 4) & 0x0F0F0F0Fu};
            if constexpr (K5) {
                // nibble q of the fifth-bit word holds the bits of word q's four
                // elements; spread them to bit 4 of each byte (q5 = lo4 | bit << 4)
#pragma unroll
                for (int q = 0; q < 8; q++) c[q] |= ((((hv[i] >> (4 * q)) & 0xFu) * 0x00204081u) & 0x01010101u) << 4;
            }
            const uint32_t m = mrow[g];
            const float st = h2f(m & 0xFFFFu), of = h2f(m >> 16);
#pragma unroll
            for (int t = 0; t < TB; t++) {
                if (TB > 1 && t >= tbl) break;
                const uint4 xe = *reinterpret_cast<const uint4 *>(le + (t * ng + g) * 16);
                const uint4 xo = *reinterpret_cast<const uint4 *>(lo + (t * ng + g) * 16);
                int qd = dot4(c[0], xe.x, 0);
                qd = dot4(c[1], xe.y, qd);
                qd = dot4(c[2], xe.z, qd);
                qd = dot4(c[3], xe.w, qd);
                qd = dot4(c[4], xo.x, qd);
                qd = dot4(c[5], xo.y, qd);
                qd = dot4(c[6], xo.z, qd);
                qd = dot4(c[7], xo.w, qd);
                const float2 s = lsx[t * ng + g];
                acc[t] = fmaf(s.x * st, (float)qd, acc[t]);
                acc[t] = fmaf(of, s.y, acc[t]);
            }
        }
    }
#pragma unroll
    for (int t = 0; t < TB; t++) acc[t] = seg_sum<16>(acc[t]);
    if constexpr (KS > 1) {
        if (j == 0) {
#pragma unroll
            for (int t = 0; t < TB; t++) lred[(kq * R + r) * TB + t] = acc[t];
        }
        __syncthreads();
        if (tid >= R) return;
        const int rr = tid;
        if (n0 + rr >= S.N) return;
#pragma unroll
        for (int t = 0; t < TB; t++) {
            if (t >= tbl) break;
            float a = lred[rr * TB + t];
#pragma unroll
            for (int q = 1; q < KS; q++) a += lred[(q * R + rr) * TB + t];
            if (A.kparts > 1) {  // one segment: partial sums [kp][t][n]
                A.part[((size_t)kp * tbl + t) * S.N + n0 + rr] = a;
                continue;
            }
            const size_t o = (size_t)t * S.out_stride + n0 + rr;
            float v = S.alpha * a;
            if (S.residual) v += S.residual[o];
            S.out[o] = v;
        }
    } else if (A.kparts > 1) {  // one segment: partial sums [kp][t][n]
        if (j == 0 && row_ok) {
#pragma unroll
            for (int t = 0; t < TB; t++) {
                if (t >= tbl) break;
                A.part[((size_t)kp * tbl + t) * S.N + n] = acc[t];
            }
        }
    } else if (j == 0 && row_ok) {
#pragma unroll
        for (int t = 0; t < TB; t++) {
            if (t >= tbl) break;
            const size_t o = (size_t)t * S.out_stride + n;
            float v = S.alpha * acc[t];
            if (S.residual) v += S.residual[o];
            S.out[o] = v;
        }
    }
}

// The K parts' partial sums of a split launch ([kp][t][n]), added in part order.
__global__ __launch_bounds__(256) void w4_part_reduce_kernel(const float *part, int kparts, int tb, int N,
                                                             float alpha, const float *residual, float *out,
                                                             int out_stride) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= N * tb) return;
    const int t = i / N, n = i % N;
    float a = part[i];
    for (int q = 1; q < kparts; q++) a += part[(size_t)q * tb * N + i];
    const size_t o = (size_t)t * out_stride + n;
    float v = alpha * a;
    if (residual) v += residual[o];
    out[o] = v;
}

template <int NU, int RW, int KS, bool K5, bool Q> static void launch_w4_nu(hipStream_t s, const W4Args &A, bool al) {
    const int grid = 8 * ((A.ntiles * A.kparts + 7) / 8);
    const dim3 blk(64 * RW * KS);
    const size_t lds = w4_lds_bytes(A.gpp, 4 * RW, KS, A.tb);
    if constexpr (!Q) {
        if (A.tb > 1) {  // several tokens: the 32-row tile with 16-byte staging (the host guarantees both)
            if constexpr (KS == 1) {
                if (A.tb <= 2) hipLaunchKernelGGL((w4_gemv_kernel<NU, RW, KS, true, K5, false, 2>), dim3(grid), blk, lds, s, A);
                else if (A.tb <= 4) hipLaunchKernelGGL((w4_gemv_kernel<NU, RW, KS, true, K5, false, 4>), dim3(grid), blk, lds, s, A);
                else hipLaunchKernelGGL((w4_gemv_kernel<NU, RW, KS, true, K5, false, 8>), dim3(grid), blk, lds, s, A);
            }
            return;
        }
    }
    if (al) hipLaunchKernelGGL((w4_gemv_kernel<NU, RW, KS, true, K5, Q, 1>), dim3(grid), blk, lds, s, A);
    else hipLaunchKernelGGL((w4_gemv_kernel<NU, RW, KS, false, K5, Q, 1>), dim3(grid), blk, lds, s, A);
}

// units per lane NU = ceil(ceil(ng/16) / KS), instantiated at 4, 6, 8, 10, 12
template <int RW, int KS, bool K5, bool Q> static void launch_w4_ks(hipStream_t s, const W4Args &A, bool al) {
    const int nu = ((A.gpp + 15) / 16 + KS - 1) / KS;
    if (nu <= 4) launch_w4_nu<4, RW, KS, K5, Q>(s, A, al);
    else if (nu <= 6) launch_w4_nu<6, RW, KS, K5, Q>(s, A, al);
    else if (nu <= 8) launch_w4_nu<8, RW, KS, K5, Q>(s, A, al);
    else if (nu <= 10) launch_w4_nu<10, RW, KS, K5, Q>(s, A, al);
    else launch_w4_nu<12, RW, KS, K5, Q>(s, A, al);
}

// The in-launch quantizer serves K/32 <= 256 (at most two K-parts).  The
// 1024-thread forms (four K-parts) have 128 VGPRs a lane; the k5 and
// element-staging variants of them spill a few registers at 10-12 units.
template <bool K5, bool Q> static void launch_w4_shape(hipStream_t s, const W4Args &A, bool al, int rw, int ks) {
    if (rw == 8 && ks == 2) {
        if constexpr (!Q) launch_w4_ks<8, 2, K5, Q>(s, A, al);
    } else if (rw == 8) launch_w4_ks<8, 1, K5, Q>(s, A, al);
    else if (ks == 1) launch_w4_ks<4, 1, K5, Q>(s, A, al);
    else if (ks == 2 || Q) launch_w4_ks<4, 2, K5, Q>(s, A, al);
    else if constexpr (!Q) launch_w4_ks<4, 4, K5, Q>(s, A, al);
}

static int w4_checks(int K, int N, const char *who) {
    if (K <= 0 || N <= 0) {
        set_error("%s: empty shape K=%d N=%d", who, K, N);
        return MIQ_EINVAL;
    }
    if (K % 32) {
        set_error("%s: K=%d must be a multiple of 32", who, K);
        return MIQ_UNSUPPORTED;
    }
    if ((size_t)N * (K / 2) >= (1ull << 32) - 4096 || (size_t)(K / 32) * N * 2 >= (1ull << 32) - 4096) {
        set_error("%s: store of N=%d x K=%d exceeds the 4 GiB buffer window", who, N, K);
        return MIQ_UNSUPPORTED;
    }
    return MIQ_OK;
}

// One store of a launch: the segment fields of the reference's w4_grp_seg.
struct W4In {
    const uint8_t *vals, *hi;
    const uint16_t *scale, *off;
    int N;
    float *out;
    float alpha;
    const float *residual;
    int out_stride;
};

// u4 (hi == nullptr) or k5 GEMV over n_segs stores sharing one activation:
// either quantized (axe/axo/asa/xs) or fp32 x (+up), quantized in the launch.
static int run_w4(hipStream_t stream, const W4In *in, int n_segs, const int8_t *axe, const int8_t *axo,
                  const uint16_t *asa, const float *xs, const float *x, const float *up, int K, const char *who,
                  int tb = 1) {
    if (n_segs < 1 || n_segs > kW4MaxSegs) {
        set_error("%s: %d segments (1..%d)", who, n_segs, kW4MaxSegs);
        return n_segs < 1 ? MIQ_EINVAL : MIQ_UNSUPPORTED;
    }
    const bool quant = x != nullptr;
    if (quant ? false : (!axe || !axo || !asa || !xs)) {
        set_error("%s: null activation buffer", who);
        return MIQ_EINVAL;
    }
    if (quant ? (((uintptr_t)x & 15) || ((uintptr_t)up & 15))
              : (((uintptr_t)axe & 15) || ((uintptr_t)axo & 15) || ((uintptr_t)asa & 1) || ((uintptr_t)xs & 3))) {
        set_error("%s: axe/axo (or x/up) must be 16-byte aligned", who);
        return MIQ_UNSUPPORTED;
    }
    const bool k5 = in[0].hi != nullptr;
    bool al = true;
    int maxN = 0;
    for (int i = 0; i < n_segs; i++) {
        const W4In &g = in[i];
        if (!g.vals || !g.scale || !g.off || !g.out || (g.hi != nullptr) != k5) {
            set_error("%s: null buffer in segment %d", who, i);
            return MIQ_EINVAL;
        }
        int rc = w4_checks(K, g.N, who);
        if (rc) return rc;
        if (((uintptr_t)g.vals & 15) || ((uintptr_t)g.scale & 1) || ((uintptr_t)g.off & 1) || ((uintptr_t)g.hi & 3)) {
            set_error("%s: vals must be 16-byte aligned, hi 4-byte, scale/off 2-byte", who);
            return MIQ_UNSUPPORTED;
        }
        al = al && !((uintptr_t)g.scale & 15) && !((uintptr_t)g.off & 15) && g.N % 8 == 0;
        maxN = g.N > maxN ? g.N : maxN;
    }
    const int ng = K / 32;
    // Tile shape.  32 rows (whole 64-byte sectors of the scale/off lines) when
    // the tile's metadata fits the LDS budget and 12 units per lane cover K;
    // else 16 rows with KS K-parts: enough that the staging slots cover ng,
    // and (for short grids) enough waves to keep the weight stream in flight.
    // Measured at 17408 x 5120: 32 rows 14.4 us, 16 rows 14.2-16.0 us, 64 rows
    // (16 waves) 18.7 us; 32 rows with two K-parts inside 20.6 us
    // in bench.py's timing against 17.0.  The in-launch quantizer needs ng <= threads/2.
    // One long-K store: split K across workgroups into parts of at most 160
    // groups (32-row tiles), the parts' sums added by a second small launch.
    // Measured at 5120 x 17408 (bench.py's event timing): 4 parts 18.3 us
    // against 22.0 us for one workgroup per 16 rows with four K-parts inside.
    int kparts = 1, rw_tb = 8;  // rw_tb: the tile of a several-token launch
    if (!quant && n_segs == 1 && ng > 192) kparts = (ng + 159) / 160;
    if (tb > 1) {
        if (tb > 8 || n_segs != 1 || !al || quant) {
            set_error("%s: %d tokens need one store with 16-byte aligned scale/off planes, N %% 8 == 0, and at most 8 tokens",
                      who, tb);
            return MIQ_UNSUPPORTED;
        }
        // K split across workgroups until the tokens' activations and the
        // tile's metadata fit the LDS budget.  Beyond four tokens: 16-row
        // tiles and at least two K parts, so two workgroups share a CU and one
        // loads while the other computes (measured at 17408 x 5120, u4: 8
        // tokens 40.7 -> 31.0 us, 13 tokens 66.1 -> 52.4 us)
        rw_tb = tb > 4 ? 4 : 8;
        if (tb > 4 && ng >= 32) kparts = kparts > 2 ? kparts : 2;
        // k5 at three or four tokens: two K parts as well (its decode holds more
        // registers; 17408 x 5120 at 4 tokens 30.4 -> 24.7 us; u4 is faster with one)
        if (k5 && tb >= 3 && ng >= 32) kparts = kparts > 2 ? kparts : 2;
        for (;; kparts++) {
            const int g = 16 * (((ng + kparts - 1) / kparts + 15) / 16);
            if (g <= 12 * 16 && w4_lds_bytes(g, 4 * rw_tb, 1, tb) <= kW4MaxLds) break;
        }
    }
    // groups per part, in whole 16-group units: the same cut as the in-workgroup
    // K-parts of the 16-row tile (KS parts of ceil(ceil(ng/16)/KS) units), so a
    // split launch adds the same partial sums in the same order as the fused
    // quantize form, and the two stay bit-identical
    const int ngs = 16 * (((ng + kparts - 1) / kparts + 15) / 16);
    kparts = (ng + ngs - 1) / ngs;
    const int U = (ngs + 15) / 16;
    int rw = 4, ks = 1;
    if (quant && ng > 256) {
        set_error("%s: K=%d is more groups than the in-launch quantizer's lanes (K/32 <= 256)", who, K);
        return MIQ_UNSUPPORTED;
    }
    if (tb > 1) {
        rw = rw_tb;
    } else if (U <= 12 && w4_lds_bytes(ngs, 32, 1, tb) <= kW4MaxLds && (!quant || ng <= 256)) {
        rw = 8;
    } else {
        ks = ngs <= 256 ? 1 : (ngs <= 512 ? 2 : 4);
        if (ks < 4 && (maxN + 15) / 16 * ks < 1024 && U > 4 * ks) ks *= 2;
        while (ks < 4 && ((U + ks - 1) / ks > 12 || (quant && ngs > 128 * ks))) ks *= 2;
    }
    if ((U + ks - 1) / ks > 12 || w4_lds_bytes(ngs, 4 * rw, ks, tb) > kW4MaxLds || (quant && ngs > 32 * rw * ks)) {
        set_error("%s: K=%d needs %zu B of LDS or more than 12 loads per lane (limits %zu, 12)%s", who, K,
                  w4_lds_bytes(ngs, 4 * rw, ks, tb), kW4MaxLds, quant ? ", or more groups than the quantizer's lanes" : "");
        return MIQ_UNSUPPORTED;
    }
    W4Args A;
    A.n_segs = n_segs;
    A.K = K;
    if (kparts > 1 && ks != 1) {  // the split form runs one K part per workgroup
        set_error("%s: K split needs one K part per workgroup", who);
        return MIQ_UNSUPPORTED;
    }
    A.mstride = w4_mstride(ngs);
    A.kparts = kparts;
    A.gpp = ngs;
    A.part = nullptr;
    if (kparts > 1) {
        void *ws = nullptr;
        const int rc = workspace_get(stream, kWsW4Part, (size_t)kparts * tb * in[0].N * 4, &ws);
        if (rc) return rc;
        A.part = (float *)ws;
    }
    A.tb = tb;
    A.axe = axe;
    A.axo = axo;
    A.asa = asa;
    A.xs = xs;
    A.x = x;
    A.up = up;
    int tiles = 0;
    for (int i = 0; i < kW4MaxSegs; i++) {
        const W4In &g = in[i < n_segs ? i : 0];
        W4Seg &d = A.seg[i];
        d.vals = g.vals;
        d.scale = g.scale;
        d.off = g.off;
        d.hi = g.hi;
        d.out = g.out;
        d.residual = g.residual;
        d.alpha = g.alpha;
        d.N = g.N;
        d.out_stride = g.out_stride;
        d.tile0 = tiles;
        d.vals_bytes = (uint32_t)((size_t)g.N * (K / 2));
        d.meta_bytes = dword_span((size_t)ng * g.N * 2);
        d.hi_bytes = (uint32_t)((size_t)g.N * (K / 8));
        if (i < n_segs) tiles += (g.N + 4 * rw - 1) / (4 * rw);
    }
    A.ntiles = tiles;
    if (k5) {
        if (quant) launch_w4_shape<true, true>(stream, A, al, rw, ks);
        else launch_w4_shape<true, false>(stream, A, al, rw, ks);
    } else {
        if (quant) launch_w4_shape<false, true>(stream, A, al, rw, ks);
        else launch_w4_shape<false, false>(stream, A, al, rw, ks);
    }
    if (kparts > 1)
        hipLaunchKernelGGL(w4_part_reduce_kernel, dim3((in[0].N * tb + 255) / 256), dim3(256), 0, stream, A.part,
                           kparts, tb, in[0].N, in[0].alpha, in[0].residual, in[0].out, in[0].out_stride);
    return check_launch(who);
}

}  // namespace miq

using namespace miq;

extern "C" {

int miq_w4_pack(hipStream_t stream, uint32_t type, const void *src, int K, int N, uint8_t *vals, uint16_t *scale,
                uint16_t *off) {
    if (!src || !vals || !scale || !off) {
        set_error("miq_w4_pack: null buffer");
        return MIQ_EINVAL;
    }
    if (type != MIQ_TYPE_Q4_K) {
        set_error("miq_w4_pack: type %u has no native 4-bit grid (Q4_K only)", type);
        return MIQ_UNSUPPORTED;
    }
    int rc = w4_checks(K, N, "miq_w4_pack");
    if (rc) return rc;
    if (K % 256) {
        set_error("miq_w4_pack: K=%d must be a multiple of 256", K);
        return MIQ_UNSUPPORTED;
    }
    if (((uintptr_t)src & 15) || ((uintptr_t)vals & 15) || ((uintptr_t)scale & 1) || ((uintptr_t)off & 1)) {
        set_error("miq_w4_pack: src/vals must be 16-byte aligned, scale/off 2-byte aligned");
        return MIQ_UNSUPPORTED;
    }
    const size_t n = (size_t)(K / 32) * N;
    hipLaunchKernelGGL(w4_pack_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream,
                       (const uint8_t *)src, K, N, vals, scale, off);
    return check_launch("miq_w4_pack");
}

int miq_k5_pack(hipStream_t stream, uint32_t type, const void *src, int K, int N, uint8_t *vals, uint8_t *hi,
                uint16_t *scale, uint16_t *off) {
    if (!src || !vals || !hi || !scale || !off) {
        set_error("miq_k5_pack: null buffer");
        return MIQ_EINVAL;
    }
    if (type != MIQ_TYPE_Q5_K) {
        set_error("miq_k5_pack: type %u is not Q5_K", type);
        return MIQ_UNSUPPORTED;
    }
    int rc = w4_checks(K, N, "miq_k5_pack");
    if (rc) return rc;
    if (K % 256) {
        set_error("miq_k5_pack: K=%d must be a multiple of 256", K);
        return MIQ_UNSUPPORTED;
    }
    if (((uintptr_t)src & 15) || ((uintptr_t)vals & 15) || ((uintptr_t)hi & 3) || ((uintptr_t)scale & 1) ||
        ((uintptr_t)off & 1)) {
        set_error("miq_k5_pack: src/vals must be 16-byte aligned, hi 4-byte, scale/off 2-byte aligned");
        return MIQ_UNSUPPORTED;
    }
    const size_t n = (size_t)(K / 32) * N;
    hipLaunchKernelGGL(k5_pack_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream,
                       (const uint8_t *)src, K, N, vals, hi, scale, off);
    return check_launch("miq_k5_pack");
}

int miq_w4_act(hipStream_t stream, const float *x, const float *up, int x_stride, int up_stride, int M, int K,
               int8_t *xq, uint16_t *asa, float *xs, int8_t *axe, int8_t *axo) {
    if (!x || !asa || !xs || (!axe) != (!axo) || M <= 0 || K <= 0) {
        set_error("miq_w4_act: null buffer or empty shape");
        return MIQ_EINVAL;
    }
    if (K % 32) {
        set_error("miq_w4_act: K=%d must be a multiple of 32", K);
        return MIQ_UNSUPPORTED;
    }
    if (((uintptr_t)x & 15) || (x_stride & 3) || (up && (((uintptr_t)up & 15) || (up_stride & 3))) ||
        ((uintptr_t)xq & 15) || ((uintptr_t)axe & 7) || ((uintptr_t)axo & 7) || (M > 1 && x_stride < K)) {
        set_error("miq_w4_act: x/up must be 16-byte aligned with strides a multiple of 4 (>= K), xq 16 B, axe/axo 8 B");
        return MIQ_UNSUPPORTED;
    }
    const size_t pairs = (size_t)M * (K / 32);
    hipLaunchKernelGGL(w4_act_kernel, dim3((unsigned)((pairs + 127) / 128)), dim3(256), 0, stream, x, up, x_stride,
                       up_stride, M, K, xq, asa, xs, axe, axo);
    return check_launch("miq_w4_act");
}

int miq_w4_gemv(hipStream_t stream, const uint8_t *vals, const uint16_t *scale, const uint16_t *off,
                const int8_t *axe, const int8_t *axo, const uint16_t *asa, const float *xs, float *out,
                int out_stride, const float *residual, float alpha, int K, int N) {
    (void)out_stride;  // one output row: out and residual are indexed by n (w4_gemv.cpp:139-149)
    const W4In in{vals, nullptr, scale, off, N, out, alpha, residual, N};
    return run_w4(stream, &in, 1, axe, axo, asa, xs, nullptr, nullptr, K, "miq_w4_gemv");
}

}  // extern "C"

namespace miq {
// M tokens over one u4 (hi == nullptr) or k5 store, in chunks of up to eight
// tokens that share each weight read; a chunk the multi-token form cannot
// take (unaligned scale/off planes, N % 8 != 0) runs token by token.
static int run_w4_tokens(hipStream_t stream, const uint8_t *vals, const uint8_t *hi, const uint16_t *scale,
                         const uint16_t *off, const int8_t *axe, const int8_t *axo, const uint16_t *asa,
                         const float *xs, float *out, int out_stride, const float *residual, float alpha, int M,
                         int K, int N, const char *who) {
    if (M <= 0 || (M > 1 && out_stride < N)) {
        set_error("%s: M=%d, out_stride %d < N %d", who, M, out_stride, N);
        return MIQ_EINVAL;
    }
    if (K <= 0 || K % 32) {
        set_error("%s: K=%d must be a positive multiple of 32", who, K);
        return K <= 0 ? MIQ_EINVAL : MIQ_UNSUPPORTED;
    }
    if (!axe || !axo || !asa || !xs) {
        set_error("%s: null activation buffer", who);
        return MIQ_EINVAL;
    }
    const int ng = K / 32;
    const bool al = !((uintptr_t)scale & 15) && !((uintptr_t)off & 15) && N % 8 == 0;
    for (int m0 = 0; m0 < M;) {
        const W4In in{vals, hi, scale, off, N, out + (size_t)m0 * out_stride, alpha,
                      residual ? residual + (size_t)m0 * out_stride : nullptr, out_stride};
        const int tb = al ? (M - m0 < 8 ? M - m0 : 8) : 1;
        const int rc = run_w4(stream, &in, 1, axe + (size_t)m0 * (K / 2), axo + (size_t)m0 * (K / 2),
                              asa + (size_t)m0 * ng, xs + (size_t)m0 * ng, nullptr, nullptr, K, who, tb);
        if (rc) return rc;
        m0 += tb;
    }
    return MIQ_OK;
}
}  // namespace miq

extern "C" {

int miq_w4_gemm(hipStream_t stream, const uint8_t *vals, const uint16_t *scale, const uint16_t *off,
                const int8_t *axe, const int8_t *axo, const uint16_t *asa, const float *xs, float *out,
                int out_stride, const float *residual, float alpha, int M, int K, int N) {
    return run_w4_tokens(stream, vals, nullptr, scale, off, axe, axo, asa, xs, out, out_stride, residual, alpha, M,
                         K, N, "miq_w4_gemm");
}

int miq_nat_gemm(hipStream_t stream, int fmt, const void *w0, const void *w1, const int8_t *w8,
                 const uint16_t *scale, const uint16_t *off, const uint16_t *lut16, const uint32_t *bit_lut,
                 const int8_t *axe, const int8_t *axo, const int8_t *axg, const uint16_t *asa, const float *xs,
                 float *out, int out_stride, const float *residual, float alpha, int M, int K, int N) {
    (void)w8, (void)lut16, (void)bit_lut, (void)axg;
    // the reference's launcher declines these shapes (w4_gemv.cpp:2409-2419)
    if (M < 2 || M > 32 || K % 32 != 0 || (M > 13 && fmt != 0)) {
        set_error("miq_nat_gemm: M=%d K=%d format %d outside M 2..32 (k5: 2..13), K %% 32 == 0", M, K, fmt);
        return MIQ_UNSUPPORTED;
    }
    if (fmt == 0)
        return run_w4_tokens(stream, (const uint8_t *)w0, nullptr, scale, off, axe, axo, asa, xs, out, out_stride,
                             residual, alpha, M, K, N, "miq_nat_gemm");
    if (fmt == 1) {
        if (!w1) {
            set_error("miq_nat_gemm: k5 needs the fifth-bit plane (w1)");
            return MIQ_EINVAL;
        }
        return run_w4_tokens(stream, (const uint8_t *)w0, (const uint8_t *)w1, scale, off, axe, axo, asa, xs, out,
                             out_stride, residual, alpha, M, K, N, "miq_nat_gemm");
    }
    set_error("miq_nat_gemm: format %d (cb4 / grouped int8 store) is not built; u4 (0) and k5 (1) are", fmt);
    return MIQ_UNSUPPORTED;
}

int miq_k5_gemv(hipStream_t stream, const uint8_t *vals, const uint8_t *hi, const uint16_t *scale,
                const uint16_t *off, const int8_t *axe, const int8_t *axo, const uint16_t *asa, const float *xs,
                float *out, const float *residual, float alpha, int K, int N) {
    if (!hi) {
        set_error("miq_k5_gemv: null buffer");
        return MIQ_EINVAL;
    }
    const W4In in{vals, hi, scale, off, N, out, alpha, residual, N};
    return run_w4(stream, &in, 1, axe, axo, asa, xs, nullptr, nullptr, K, "miq_k5_gemv");
}

int miq_w4_quant_gemv(hipStream_t stream, const miq_w4_seg *segs, int n_segs, int total_rows, const float *x,
                      const float *up, int K) {
    if (!segs || !x || n_segs < 1) {
        set_error("miq_w4_quant_gemv: null buffer or no segment");
        return MIQ_EINVAL;
    }
    if (n_segs > kW4MaxSegs) {
        set_error("miq_w4_quant_gemv: %d segments (at most %d)", n_segs, kW4MaxSegs);
        return MIQ_UNSUPPORTED;
    }
    W4In in[kW4MaxSegs];
    long rows = 0;
    for (int i = 0; i < n_segs; i++) {
        in[i] = W4In{segs[i].vals, nullptr, segs[i].scale, segs[i].off, segs[i].n_rows, segs[i].out, segs[i].alpha,
                     segs[i].residual, segs[i].n_rows};
        rows += segs[i].n_rows;
    }
    if (rows != total_rows) {
        set_error("miq_w4_quant_gemv: total_rows %d != %ld rows in the segments", total_rows, rows);
        return MIQ_EINVAL;
    }
    return run_w4(stream, in, n_segs, nullptr, nullptr, nullptr, nullptr, x, up, K, "miq_w4_quant_gemv");
}

}  // extern "C"
