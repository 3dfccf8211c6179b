// Decode GEMV straight from GGUF blocks: out[t][row] = alpha * sum_k W[row][k]
// * act_t[k] (+ residual) for a few tokens (TB <= 4), int8 packed dots.
//
// Mapping (wave64, 4 waves per workgroup):
//   - a row is split across LPR lanes; lane j of a row takes units j, j+LPR, ...
//     (a unit = 64 weights, see miq_units.h), so the wave holds 64/LPR rows;
//   - the quantized activation (x8, scales, sums) of all TB tokens is staged
//     once per workgroup in LDS; weights stream from HBM through buffer loads
//     (16-byte loads on 16-byte-aligned Q4_K/Q5_K blocks, aligned dwords +
//     byte funnel shifts on the 2-byte-aligned Q6_K/Q8_0 blocks);
//   - each lane accumulates its units' fp32 group terms, then the row's lanes
//     reduce with cross-lane shuffles and one lane writes the output.
// Per-group int32 dots are exact; the fp32 terms follow the reference
// epilogues (i8.cpp:60,120,152; q4exp.cpp:467); only the fp32 summation
// order differs from the CPU (per-lane partials, then a tree).
#include <cstdlib>

#include "miq_internal.h"
#include "miq_units.h"
#include "miq_xq.h"

namespace miq {

// One output segment of a launch: its weight tensor and output; segments of
// a launch share the type, K and the activation (the reference's
// i8_row_gemv_multi, src/backend/backend.h:120-121).  Workgroups
// [wg0, next segment's wg0) serve it.
constexpr int kGemvMaxSegs = 8;
struct GemvSeg {
    const uint8_t *w;
    uint32_t w_bytes;
    int n_rows;
    float *out;
    int out_stride;
    const float *residual;
    float alpha;
    int wg0;
};

struct GemvArgs {
    uint32_t row_bytes;
    int K;
    const int8_t *x8;
    const float *xmeta;
    const int32_t *xsumq;
    const float *x;  // fused form: the fp32 activation of the one token (x8/xmeta/xsumq are outputs)
    int n_segs;
    int n_wg;
    GemvSeg seg[kGemvMaxSegs];
};

// LDS image of the activation: x8 [G][TB][32] bytes, then xmeta and xsumq as
// given ([G*TB] float2 / int2 pairs), each region padded to whole KiB.
template <int TB> struct ActLds {
    const uint32_t *x8;
    const float *sx;   // stride 2 (the float2 pairs)
    const int2 *xs;
};

__host__ __device__ constexpr uint32_t kib_up(uint32_t n) { return (n + 1023u) & ~1023u; }
__host__ __device__ constexpr size_t act_lds_bytes(int K, int TB) {
    return kib_up((uint32_t)K * TB) + 2 * kib_up((uint32_t)(K / 32) * TB * 8);
}

// Stage the activation straight from global memory into LDS (buffer loads with
// the lds bit: no registers held while the weight loads go out).  A wave's
// load covers 1 KiB (64 lanes x 16 bytes); chunks past a region's end read
// zeros and land in its padding.
template <int TB> __device__ __forceinline__ ActLds<TB> stage_dma(uint8_t *lds, const int8_t *x8, const float *xmeta,
                                                                  const int32_t *xsumq, int K) {
    typedef __attribute__((address_space(3))) void *lds_ptr;
    const uint32_t nx = (uint32_t)K * TB, nm = (uint32_t)(K / 32) * TB * 8;
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(x8, nx), rm = make_rsrc(xmeta, nm), rq = make_rsrc(xsumq, nm);
    uint8_t *lx = lds, *lm = lds + kib_up(nx), *lq = lm + kib_up(nm);
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (uint32_t c = wave; c * 1024 < nx; c += 4)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (lds_ptr)(lx + c * 1024), 16, c * 1024 + lane * 16, 0, 0, 0);
    for (uint32_t c = wave; c * 1024 < nm; c += 4) {
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rm, (lds_ptr)(lm + c * 1024), 16, c * 1024 + lane * 16, 0, 0, 0);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rq, (lds_ptr)(lq + c * 1024), 16, c * 1024 + lane * 16, 0, 0, 0);
    }
    return ActLds<TB>{reinterpret_cast<const uint32_t *>(lx), reinterpret_cast<const float *>(lm),
                      reinterpret_cast<const int2 *>(lq)};
}

template <int TB> __device__ __forceinline__ void load_x8(const ActLds<TB> &a, int G, int t, uint32_t (&X)[8]) {
    const uint4 *p = reinterpret_cast<const uint4 *>(a.x8 + ((size_t)G * TB + t) * 8);
    const uint4 v0 = p[0], v1 = p[1];
    X[0] = v0.x; X[1] = v0.y; X[2] = v0.z; X[3] = v0.w;
    X[4] = v1.x; X[5] = v1.y; X[6] = v1.z; X[7] = v1.w;
}

// Header dword c of a Q4_K/Q5_K block (lane c of a quad) plus the unit's codes;
// quad_hdr() gathers the quad's four dwords (DPP quad broadcasts).  The quads
// of a row segment hold units 4m..4m+3 of one block and are uniformly active
// (U is a multiple of 4 and a row spans at least 16 lanes).
__device__ __forceinline__ RawQ4K load_q4k_hw(__amdgpu_buffer_rsrc_t r, uint32_t blk_off, int c) {
    RawQ4K u;
    u.hdr.x = bload4(r, blk_off + 4 * c);
    u.q0 = bload16(r, blk_off + 16 + 32 * c);
    u.q1 = bload16(r, blk_off + 16 + 32 * c + 16);
    return u;
}
// Q5_K: lane c of the quad also loads qh bytes [8c, 8c+8) only; quad_qh()
// gathers the 32 qh bytes every lane needs (the fifth bits of its two groups
// sit in all of them) with DPP quad broadcasts, one load per unit fewer.
__device__ __forceinline__ RawQ5K load_q5k_hw(__amdgpu_buffer_rsrc_t r, uint32_t blk_off, int c) {
    RawQ5K u;
    u.hdr.x = bload4(r, blk_off + 4 * c);
    const uint2 hq = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(r, blk_off + 16 + 8 * c, 0, 0));
    u.h0.x = hq.x;
    u.h0.y = hq.y;
    u.q0 = bload16(r, blk_off + 48 + 32 * c);
    u.q1 = bload16(r, blk_off + 48 + 32 * c + 16);
    return u;
}
__device__ __forceinline__ uint4 quad_hdr(uint32_t w) {
    // dpp quad_perm [k,k,k,k]: every lane of a quad reads the quad's lane k
    return make_uint4((uint32_t)__builtin_amdgcn_mov_dpp((int)w, 0x00, 0xF, 0xF, false),
                      (uint32_t)__builtin_amdgcn_mov_dpp((int)w, 0x55, 0xF, 0xF, false),
                      (uint32_t)__builtin_amdgcn_mov_dpp((int)w, 0xAA, 0xF, 0xF, false),
                      (uint32_t)__builtin_amdgcn_mov_dpp((int)w, 0xFF, 0xF, 0xF, false));
}

__device__ __forceinline__ void quad_qh(RawQ5K &u) {
    const int a = (int)u.h0.x, b = (int)u.h0.y;
    u.h0 = make_uint4((uint32_t)__builtin_amdgcn_mov_dpp(a, 0x00, 0xF, 0xF, false), (uint32_t)__builtin_amdgcn_mov_dpp(b, 0x00, 0xF, 0xF, false),
                      (uint32_t)__builtin_amdgcn_mov_dpp(a, 0x55, 0xF, 0xF, false), (uint32_t)__builtin_amdgcn_mov_dpp(b, 0x55, 0xF, 0xF, false));
    u.h1 = make_uint4((uint32_t)__builtin_amdgcn_mov_dpp(a, 0xAA, 0xF, 0xF, false), (uint32_t)__builtin_amdgcn_mov_dpp(b, 0xAA, 0xF, 0xF, false),
                      (uint32_t)__builtin_amdgcn_mov_dpp(a, 0xFF, 0xF, 0xF, false), (uint32_t)__builtin_amdgcn_mov_dpp(b, 0xFF, 0xF, 0xF, false));
}

#ifndef MIQ_Q4K_PIECES
#define MIQ_Q4K_PIECES 1
#endif
// Q4_K in 16-byte pieces: piece i (0..7) of a block is qs bytes [16i, 16i+16),
// i.e. values 16(i&1)..+15 of groups 2(i>>1) (low nibbles) and 2(i>>1)+1
// (high nibbles).  Lane j of a row takes pieces j, j+LPR, ...; the eight
// lanes of a block are consecutive, so each load instruction reads runs of
// LPR/8 whole 128-byte code areas.  Lane i of the block also loads header
// dword i&3 and its quad rebuilds the header (quad_hdr).  The two lanes of a
// pair (i, i^1) add their half-group dots by one DPP swap; lane i&1 = 0 then
// owns group 2(i>>1)'s term and lane i&1 = 1 group 2(i>>1)+1's.
struct PieceQ4K {
    uint4 hdr;  // .x as loaded: header dword i&3; all four after quad_hdr
    uint4 q;
};
__device__ __forceinline__ PieceQ4K load_q4k_piece(__amdgpu_buffer_rsrc_t r, uint32_t blk_off, int i) {
    PieceQ4K p;
    p.hdr.x = bload4(r, blk_off + 4 * (i & 3));
    p.q = bload16(r, blk_off + 16 + 16 * i);
    return p;
}
// lane i^1's value (DPP quad_perm [1,0,3,2])
__device__ __forceinline__ int pair_swap(int v) { return __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, false); }

// The exact int32 dot of this lane's group (see above): its own half-group
// dot plus the partner lane's.  Every lane of the quad must call it.
__device__ __forceinline__ int piece_dot(const uint32_t (&q)[4], const uint32_t (&X0)[4], const uint32_t (&X1)[4], int h) {
    int lo = 0, hi = 0;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        lo = dot4(q[k] & 0x0F0F0F0Fu, X0[k], lo);
        hi = dot4((q[k] >> 4) & 0x0F0F0F0Fu, X1[k], hi);
    }
    // this lane's group: the low-nibble group for h = 0, the high one for h = 1
    const int mine = h ? hi : lo, other = h ? lo : hi;
    return mine + pair_swap(other);
}

template <int TB>
__device__ __forceinline__ void piece_accumulate(const PieceQ4K &pc, int p, const ActLds<TB> &a, float (&acc)[TB]) {
    const int b = p >> 3, i = p & 7, c = i >> 1, h = i & 1;
    const int G0 = b * 8 + 2 * c, G1 = G0 + 1, Gm = G0 + h;
    const uint32_t q[4] = {pc.q.x, pc.q.y, pc.q.z, pc.q.w};
    int sc, m;
    scale_min_k4(2 * c + h, pc.hdr.y, pc.hdr.z, pc.hdr.w, sc, m);
    const float d = h2f(pc.hdr.x), dm = h2f(pc.hdr.x >> 16);
#pragma unroll
    for (int t = 0; t < TB; t++) {
        const uint4 x0 = reinterpret_cast<const uint4 *>(a.x8 + ((size_t)G0 * TB + t) * 8)[h];
        const uint4 x1 = reinterpret_cast<const uint4 *>(a.x8 + ((size_t)G1 * TB + t) * 8)[h];
        const uint32_t X0[4] = {x0.x, x0.y, x0.z, x0.w}, X1[4] = {x1.x, x1.y, x1.z, x1.w};
        const int wd = piece_dot(q, X0, X1, h);
        const int2 xs = a.xs[Gm * TB + t];
        acc[t] += a.sx[2 * (Gm * TB + t)] * (d * (float)sc * (float)wd - dm * (float)m * (float)(xs.x + xs.y));
    }
}

// Raw bytes of one unit, per type.
template <uint32_t TYPE> struct RawOf;
template <> struct RawOf<MIQ_TYPE_Q4_K> { using T = RawQ4K; };
template <> struct RawOf<MIQ_TYPE_Q5_K> { using T = RawQ5K; };
template <> struct RawOf<MIQ_TYPE_Q6_K> { using T = RawQ6K; };
template <> struct RawOf<MIQ_TYPE_Q8_0> { using T = RawQ80; };

template <uint32_t TYPE>
__device__ __forceinline__ typename RawOf<TYPE>::T load_unit(__amdgpu_buffer_rsrc_t rs, uint32_t row_off, int u) {
    if constexpr (TYPE == MIQ_TYPE_Q4_K) return load_q4k(rs, row_off + (uint32_t)(u >> 2) * kQ4KBytes, u & 3);
    else if constexpr (TYPE == MIQ_TYPE_Q5_K) return load_q5k(rs, row_off + (uint32_t)(u >> 2) * kQ5KBytes, u & 3);
    else if constexpr (TYPE == MIQ_TYPE_Q6_K) return load_q6k(rs, row_off + (uint32_t)(u >> 2) * kQ6KBytes, u & 3);
    else return load_q80(rs, row_off + (uint32_t)u * 68u);
}

// Fold one loaded unit into acc[TB].
template <uint32_t TYPE, int TB>
__device__ __forceinline__ void unit_accumulate(const typename RawOf<TYPE>::T &raw, int u, const ActLds<TB> &a,
                                                float (&acc)[TB]) {
    if constexpr (TYPE == MIQ_TYPE_Q4_K || TYPE == MIQ_TYPE_Q5_K) {
        const int b = u >> 2, c = u & 3;
        const int G0 = b * 8 + 2 * c, G1 = G0 + 1;
        int wd0[TB], wd1[TB];
#pragma unroll
        for (int t = 0; t < TB; t++) {
            uint32_t X0[8], X1[8];
            load_x8(a, G0, t, X0);
            load_x8(a, G1, t, X1);
            if constexpr (TYPE == MIQ_TYPE_Q4_K) dots_q4k(raw, X0, X1, wd0[t], wd1[t]);
            else dots_q5k(raw, c, X0, X1, wd0[t], wd1[t]);
        }
#pragma unroll
        for (int t = 0; t < TB; t++) {
            const int2 s0 = a.xs[G0 * TB + t], s1 = a.xs[G1 * TB + t];
            acc[t] += epi_kq45(raw.hdr, c, wd0[t], wd1[t], a.sx[2 * (G0 * TB + t)], a.sx[2 * (G1 * TB + t)], s0.x + s0.y,
                               s1.x + s1.y);
        }
    } else if constexpr (TYPE == MIQ_TYPE_Q6_K) {
        const int b = u >> 2, c = u & 3;
        const int blk2 = c >> 1, half = c & 1;
        const float d = h2f(raw.dbits);
#pragma unroll
        for (int t = 0; t < TB; t++) {
            uint32_t Xh[4][4];
            const uint32_t *Xp[4];
#pragma unroll
            for (int p = 0; p < 4; p++) {
                const int G = b * 8 + blk2 * 4 + p;
                const uint4 v = reinterpret_cast<const uint4 *>(a.x8 + ((size_t)G * TB + t) * 8)[half];
                Xh[p][0] = v.x; Xh[p][1] = v.y; Xh[p][2] = v.z; Xh[p][3] = v.w;
                Xp[p] = Xh[p];
            }
            int wd[4];
            dots_q6k(raw, Xp, wd);
            // the sub-group scale multiplies the exact dot in integers
            // (|sc * (wd - 32 xsum)| < 2^24), d scales the unit's sum once
            float s = 0.0f;
#pragma unroll
            for (int p = 0; p < 4; p++) {
                const int G = b * 8 + blk2 * 4 + p;
                const int2 xs = a.xs[G * TB + t];
                const int xsh = half ? xs.y : xs.x;
                s = __builtin_fmaf(a.sx[2 * (G * TB + t)], (float)__mul24(wd[p] - 32 * xsh, q6k_scale(raw, c, p)), s);
            }
            acc[t] = __builtin_fmaf(d, s, acc[t]);
        }
    } else {  // Q8_0: unit = blocks 2u, 2u+1
        const float da = h2f(raw.da), db = h2f(raw.db);
        const int G0 = 2 * u, G1 = G0 + 1;
#pragma unroll
        for (int t = 0; t < TB; t++) {
            uint32_t X0[8], X1[8];
            load_x8(a, G0, t, X0);
            load_x8(a, G1, t, X1);
            int wd0, wd1;
            dots_q80(raw, X0, X1, wd0, wd1);
            acc[t] += a.sx[2 * (G0 * TB + t)] * da * (float)wd0 + a.sx[2 * (G1 * TB + t)] * db * (float)wd1;
        }
    }
}

// Waves per SIMD the register budget is set for: five (<= 96 VGPRs) for the
// one-token Q4_K decode, so a CU holds 20 waves and the usual decode grids run
// in one round; otherwise no bound (the compiler's choice, no spills).
template <uint32_t TYPE, int TB, int NU, bool QUANT = false> constexpr int gemv_waves() {
    return (TB == 1 && NU <= 5 && TYPE == MIQ_TYPE_Q4_K) ? (QUANT ? 4 : 5) : 1;
}

// vector-memory loads one load_q4k/q5k/q6k/q80 issues
template <uint32_t TYPE> constexpr int unit_loads() {
    return TYPE == MIQ_TYPE_Q4_K ? 3 : TYPE == MIQ_TYPE_Q5_K ? 4 : TYPE == MIQ_TYPE_Q6_K ? 8 : 5;
}

// One wave per group of 64/LPR rows; lane j of a row owns units j, j+LPR, ...
// (NU per lane).  Order of work, chosen so nothing waits for more than it needs:
// issue the activation staging loads (straight into LDS), issue every weight
// load of the lane, wait for the staging loads (the oldest) and the other
// waves', then fold the units in load order -- each fold waits only for its
// own loads.
// All loads are unconditional buffer loads (an invalid unit reads past the end
// and gets zeros), so the compiler tracks the outstanding loads exactly.
//
// QUANT (one token, K <= 8192): the workgroup quantizes the fp32 activation
// itself (cpu_xq, xq.cpp:10-50: two lanes per 32-value group, 16 values each,
// the group max through a DPP swap) into the LDS image, and workgroup 0 also
// writes x8/xmeta/xsumq as miq_xq would.  The x loads go out before the weight
// loads, so waiting for them leaves the weights in flight.
template <uint32_t TYPE, int LPR, int TB, int NU, bool QUANT>
__global__ __launch_bounds__(256, (gemv_waves<TYPE, TB, NU, QUANT>())) void gemv_kernel(GemvArgs A) {
    extern __shared__ __align__(16) uint8_t lds[];
    ActLds<TB> act;
    float4 xv[2][4];
    if constexpr (QUANT) {
        static_assert(TB == 1, "the fused quantizer serves one token");
        const __amdgpu_buffer_rsrc_t rx = make_rsrc(A.x, (uint32_t)A.K * 4);
        const int pq = threadIdx.x >> 1, hf = threadIdx.x & 1;
#pragma unroll
        for (int r = 0; r < 2; r++) {
            const uint32_t base = (uint32_t)((pq + 128 * r) * 32 + 16 * hf) * 4;  // past K*4: zeros
#pragma unroll
            for (int c = 0; c < 4; c++)
                xv[r][c] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rx, base + 16 * c, 0, 0));
        }
        const uint32_t nx = (uint32_t)A.K * TB, nm = (uint32_t)(A.K / 32) * TB * 8;
        act = ActLds<TB>{reinterpret_cast<const uint32_t *>(lds), reinterpret_cast<const float *>(lds + kib_up(nx)),
                         reinterpret_cast<const int2 *>(lds + kib_up(nx) + kib_up(nm))};
    } else {
        act = stage_dma<TB>(lds, A.x8, A.xmeta, A.xsumq, A.K);
    }
    int si = 0;  // this workgroup's segment (uniform)
#pragma unroll
    for (int q = 1; q < kGemvMaxSegs; q++)
        if (q < A.n_segs && (int)blockIdx.x >= A.seg[q].wg0) si = q;
    const GemvSeg S = A.seg[si];
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(S.w, S.w_bytes);
    constexpr int RPW = 64 / LPR;
    const int lane = threadIdx.x & 63;
    const int row = (((int)blockIdx.x - S.wg0) * 4 + (threadIdx.x >> 6)) * RPW + lane / LPR;
    const int j = lane % LPR;
    const int U = A.K / 64;
    const bool row_ok = row < S.n_rows;
    // pieces for Q4_K at two or more tokens (measured faster there; the unit
    // layout stays at one token, where the pieces' per-piece header work cost more)
    constexpr bool PIECES = MIQ_Q4K_PIECES && TYPE == MIQ_TYPE_Q4_K && TB >= 2;
    using Raw = typename RawOf<TYPE>::T;
    Raw raw[PIECES ? 1 : NU];
    PieceQ4K pcs[PIECES ? 2 * NU : 1];
    if constexpr (PIECES) {
#pragma unroll
        for (int i = 0; i < 2 * NU; i++) {
            const int p = j + i * LPR;
            const bool ok = row_ok && p < 2 * U;
            const uint32_t off = ok ? (uint32_t)row * A.row_bytes + (uint32_t)(p >> 3) * kQ4KBytes : S.w_bytes;
            pcs[i] = load_q4k_piece(rs, off, p & 7);
        }
    } else
#pragma unroll
    for (int i = 0; i < NU; i++) {
        const int u = j + i * LPR;
        const bool ok = row_ok && u < U;
        const uint32_t ub = TYPE == MIQ_TYPE_Q8_0 ? (uint32_t)u * 68u : (uint32_t)(u >> 2) * block_bytes(TYPE);
        const uint32_t off = ok ? (uint32_t)row * A.row_bytes + ub : S.w_bytes;
        // Q4_K/Q5_K: the 4 lanes of a quad hold the 4 units of one block, so each
        // loads one dword of its header and the quad rebuilds it with DPP below
        if constexpr (TYPE == MIQ_TYPE_Q4_K) raw[i] = load_q4k_hw(rs, off, u & 3);
        else if constexpr (TYPE == MIQ_TYPE_Q5_K) raw[i] = load_q5k_hw(rs, off, u & 3);
        else if constexpr (TYPE == MIQ_TYPE_Q6_K) raw[i] = load_q6k(rs, off, u & 3);
        else raw[i] = load_q80(rs, off);
    }
    // the staging loads are the oldest: wait for them only, then for every wave's
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(PIECES ? 2 * NU * 2 : NU * unit_loads<TYPE>()));
    if constexpr (QUANT) {
        const int G = A.K / 32, pq = threadIdx.x >> 1, hf = threadIdx.x & 1;
        uint8_t *lx = lds;
        float *lm = reinterpret_cast<float *>(lds + kib_up((uint32_t)A.K));
        int32_t *lq = reinterpret_cast<int32_t *>(lds + kib_up((uint32_t)A.K) + kib_up((uint32_t)G * 8));
#pragma unroll
        for (int r = 0; r < 2; r++) {
            const int g = pq + 128 * r;
            if (r == 1 && G <= 128) break;
            const float v[16] = {xv[r][0].x, xv[r][0].y, xv[r][0].z, xv[r][0].w, xv[r][1].x, xv[r][1].y,
                                 xv[r][1].z, xv[r][1].w, xv[r][2].x, xv[r][2].y, xv[r][2].z, xv[r][2].w,
                                 xv[r][3].x, xv[r][3].y, xv[r][3].z, xv[r][3].w};
            float mx = 0.0f;
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const float a = fabsf(v[i]);
                mx = mx < a ? a : mx;
            }
            const float mo = __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, mx), 0xB1, 0xF, 0xF, false));
            mx = mx < mo ? mo : mx;  // the group's max over both halves
            const float inv = mx > 0.0f ? 127.0f / mx : 0.0f;
            int sh = 0;
            uint32_t packed[4];
#pragma unroll
            for (int w = 0; w < 4; w++) {
                uint32_t word = 0;
#pragma unroll
                for (int b = 0; b < 4; b++) {
                    float rr = roundf(v[4 * w + b] * inv);
                    rr = rr < 127.0f ? rr : 127.0f;
                    rr = -127.0f > rr ? -127.0f : rr;
                    const int q = (int)rr;
                    sh += q;
                    word |= ((uint32_t)q & 0xFFu) << (8 * b);
                }
                packed[w] = word;
            }
            const float sc = h2f(f2h_trunc(mx > 0.0f ? mx / 127.0f : 0.0f));
            if (g < G) {
                const uint4 codes = make_uint4(packed[0], packed[1], packed[2], packed[3]);
                *reinterpret_cast<uint4 *>(lx + g * 32 + 16 * hf) = codes;
                if (hf == 0) *reinterpret_cast<float2 *>(lm + 2 * g) = make_float2(sc, 0.0f);
                lq[2 * g + hf] = sh;
                if (blockIdx.x == 0) {
                    *reinterpret_cast<uint4 *>(const_cast<int8_t *>(A.x8) + g * 32 + 16 * hf) = codes;
                    if (hf == 0) reinterpret_cast<float2 *>(const_cast<float *>(A.xmeta))[g] = make_float2(sc, 0.0f);
                    const_cast<int32_t *>(A.xsumq)[2 * g + hf] = sh;
                }
            }
        }
    }
    __syncthreads();
    float acc[TB];
#pragma unroll
    for (int t = 0; t < TB; t++) acc[t] = 0.0f;
    if constexpr (PIECES) {
#pragma unroll
        for (int i = 0; i < 2 * NU; i++) {
            const int p = j + i * LPR;
            pcs[i].hdr = quad_hdr(pcs[i].hdr.x);
            // whole quads are in or out of range (2U is a multiple of 8), so the
            // pair swap inside sees only live partners
            if (row_ok && p < 2 * U) piece_accumulate<TB>(pcs[i], p, act, acc);
        }
    } else
#pragma unroll
    for (int i = 0; i < NU; i++) {
        const int u = j + i * LPR;
        if constexpr (TYPE == MIQ_TYPE_Q4_K || TYPE == MIQ_TYPE_Q5_K) raw[i].hdr = quad_hdr(raw[i].hdr.x);
        if constexpr (TYPE == MIQ_TYPE_Q5_K) quad_qh(raw[i]);
        if (row_ok && u < U) unit_accumulate<TYPE, TB>(raw[i], u, act, acc);
    }
#pragma unroll
    for (int t = 0; t < TB; t++) acc[t] = seg_sum<LPR>(acc[t]);
    if (j == 0 && row_ok) {
#pragma unroll
        for (int t = 0; t < TB; t++) {
            const size_t o = (size_t)t * S.out_stride + row;
            float v = S.alpha * acc[t];
            if (S.residual) v += S.residual[o];
            S.out[o] = v;
        }
    }
}

// ------------------------------------------------------------ dispatch

// Lanes per row: among 16, 32, 64 (in order of preference) the one wasting the
// fewest lane slots on a row of U units, with at most 8 units per lane.
static int pick_lpr(int U) {
    const int cand[3] = {16, 32, 64};
    int best = 64;
    long best_w = -1;
    for (int i = 0; i < 3; i++) {
        const int l = cand[i];
        const int nu = (U + l - 1) / l;
        if (nu > 8) continue;
        const long waste = (long)nu * l - U;
        if (best_w < 0 || waste < best_w) {
            best_w = waste;
            best = l;
        }
    }
    return best;
}

template <uint32_t TYPE, int LPR, int TB, int NU, bool Q> static void launch_gemv_nu(hipStream_t s, GemvArgs A) {
    constexpr int rows_per_wg = 4 * (64 / LPR);
    int grid = 0;
    for (int i = 0; i < A.n_segs; i++) {
        A.seg[i].wg0 = grid;
        grid += (A.seg[i].n_rows + rows_per_wg - 1) / rows_per_wg;
    }
    hipLaunchKernelGGL((gemv_kernel<TYPE, LPR, TB, NU, Q>), dim3(grid), dim3(256), act_lds_bytes(A.K, TB), s, A);
}

template <uint32_t TYPE, int LPR, int TB, bool Q = false> static void launch_gemv_t(hipStream_t s, const GemvArgs &A) {
    const int nu = (A.K / 64 + LPR - 1) / LPR;
    if (nu <= 2) launch_gemv_nu<TYPE, LPR, TB, 2, Q>(s, A);
    else if (nu <= 3) launch_gemv_nu<TYPE, LPR, TB, 3, Q>(s, A);
    else if (nu <= 4) launch_gemv_nu<TYPE, LPR, TB, 4, Q>(s, A);
    else if (nu <= 5) launch_gemv_nu<TYPE, LPR, TB, 5, Q>(s, A);
    else if (nu <= 6) launch_gemv_nu<TYPE, LPR, TB, 6, Q>(s, A);
    else launch_gemv_nu<TYPE, LPR, TB, 8, Q>(s, A);
}

template <uint32_t TYPE, int TB, bool Q = false> static void launch_gemv_lpr(hipStream_t s, const GemvArgs &A, int lpr) {
    switch (lpr) {
    case 16: launch_gemv_t<TYPE, 16, TB, Q>(s, A); break;
    case 32: launch_gemv_t<TYPE, 32, TB, Q>(s, A); break;
    default: launch_gemv_t<TYPE, 64, TB, Q>(s, A); break;
    }
}

template <uint32_t TYPE> static void launch_gemv_tb(hipStream_t s, const GemvArgs &A, int TB, int lpr) {
    if (A.x) {  // fused quantizer: one token
        launch_gemv_lpr<TYPE, 1, true>(s, A, lpr);
        return;
    }
    switch (TB) {
    case 1: launch_gemv_lpr<TYPE, 1>(s, A, lpr); break;
    case 2: launch_gemv_lpr<TYPE, 2>(s, A, lpr); break;
    case 3: launch_gemv_lpr<TYPE, 3>(s, A, lpr); break;
    default: launch_gemv_lpr<TYPE, 4>(s, A, lpr); break;
    }
}

constexpr int kGemvMaxTB = 4;
constexpr size_t kGemvMaxLds = 64 * 1024;

// Shape/type/alignment checks shared by every entry point that reads a seg.
int check_seg(const miq_seg *s, int TB, const char *who) {
    if (!s || !s->w || !s->out || !s->x8 || !s->xmeta || !s->xsumq || s->n_rows <= 0 || s->K <= 0 || TB <= 0) {
        set_error("%s: null buffer or empty shape", who);
        return MIQ_EINVAL;
    }
    const uint32_t t = s->type;
    if (t != MIQ_TYPE_Q4_K && t != MIQ_TYPE_Q5_K && t != MIQ_TYPE_Q6_K && t != MIQ_TYPE_Q8_0) {
        set_error("%s: weight type %u is not on the integer path", who, t);
        return MIQ_UNSUPPORTED;
    }
    if (s->K % 32 || (t != MIQ_TYPE_Q8_0 && s->K % 256)) {
        set_error("%s: K=%d must be a multiple of %d", who, s->K, t == MIQ_TYPE_Q8_0 ? 32 : 256);
        return MIQ_UNSUPPORTED;
    }
    const size_t total = (size_t)s->n_rows * miq_row_bytes(t, s->K);
    // loads past a row range use offsets up to w_bytes + 256: keep them inside 32 bits
    if (total >= (1ull << 32) - 4096) {
        set_error("%s: weight tensor of %zu bytes exceeds the 4 GiB buffer window", who, total);
        return MIQ_UNSUPPORTED;
    }
    const uintptr_t wa = (uintptr_t)s->w;
    if ((t == MIQ_TYPE_Q4_K || t == MIQ_TYPE_Q5_K) ? (wa & 15) : (t == MIQ_TYPE_Q8_0 ? (wa & 3) : (wa & 1))) {
        set_error("%s: weight pointer misaligned for type %u", who, t);
        return MIQ_UNSUPPORTED;
    }
    if (((uintptr_t)s->x8 & 15) || ((uintptr_t)s->xmeta & 7) || ((uintptr_t)s->xsumq & 7)) {
        set_error("%s: activation buffers misaligned (x8 16 B, xmeta/xsumq 8 B)", who);
        return MIQ_UNSUPPORTED;
    }
    if (TB > 1 && s->out_stride < s->n_rows) {
        set_error("%s: out_stride %d < n_rows %d", who, s->out_stride, s->n_rows);
        return MIQ_EINVAL;
    }
    return MIQ_OK;
}

bool gemv_fits(const miq_seg *s, int TB) {
    return !q80_any(s) && TB <= kGemvMaxTB && act_lds_bytes(s->K, TB) <= kGemvMaxLds;
}

bool gemv_quant_fits(const miq_seg *s, int TB) {
    return TB == 1 && s->x && !s->act_up && s->K <= 8192 && !((uintptr_t)s->x & 15) && gemv_fits(s, TB);
}

int launch_gemv(hipStream_t stream, const miq_seg *s, int TB, bool quant) { return launch_gemv_multi(stream, s, 1, TB, quant); }

int launch_gemv_multi(hipStream_t stream, const miq_seg *segs, int n_segs, int TB, bool quant) {
    if (n_segs < 1 || n_segs > kGemvMaxSegs) {
        set_error("miq gemv: %d segments (1..%d per launch)", n_segs, kGemvMaxSegs);
        return MIQ_EINVAL;
    }
    const miq_seg *s = segs;
    GemvArgs A{};
    A.x = quant ? s->x : nullptr;
    A.row_bytes = (uint32_t)miq_row_bytes(s->type, s->K);
    A.K = s->K;
    A.x8 = s->x8;
    A.xmeta = s->xmeta;
    A.xsumq = s->xsumq;
    A.n_segs = n_segs;
    for (int i = 0; i < n_segs; i++) {
        GemvSeg &d = A.seg[i];
        d.w = (const uint8_t *)segs[i].w;
        d.w_bytes = dword_span((size_t)segs[i].n_rows * A.row_bytes);
        d.n_rows = segs[i].n_rows;
        d.out = segs[i].out;
        d.out_stride = TB > 1 ? segs[i].out_stride : segs[i].n_rows;
        d.residual = segs[i].residual;
        d.alpha = segs[i].alpha;
    }
    const int lpr = pick_lpr(s->K / 64);
    switch (s->type) {
    case MIQ_TYPE_Q4_K: launch_gemv_tb<MIQ_TYPE_Q4_K>(stream, A, TB, lpr); break;
    case MIQ_TYPE_Q5_K: launch_gemv_tb<MIQ_TYPE_Q5_K>(stream, A, TB, lpr); break;
    case MIQ_TYPE_Q6_K: launch_gemv_tb<MIQ_TYPE_Q6_K>(stream, A, TB, lpr); break;
    default: launch_gemv_tb<MIQ_TYPE_Q8_0>(stream, A, TB, lpr); break;
    }
    return check_launch("miq gemv");
}

// ------------------------------------------------------- parity hook (path 0)

// One thread per (token, row, unit): writes the unit's exact sub-group dots.
template <uint32_t TYPE>
__global__ __launch_bounds__(256) void unit_dots_kernel(const uint8_t *w, uint32_t w_bytes, uint32_t row_bytes, int K,
                                                        int n_rows, const int8_t *x8, int TB, int32_t *out) {
    const int U = K / 64;
    const long gid = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= (long)TB * n_rows * U) return;
    const int u = (int)(gid % U);
    const int row = (int)((gid / U) % n_rows);
    const int t = (int)(gid / ((long)U * n_rows));
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(w, w_bytes);
    const uint32_t row_off = (uint32_t)row * row_bytes;
    const uint32_t *X = reinterpret_cast<const uint32_t *>(x8);
    auto xg = [&](int G, uint32_t (&dst)[8]) {
        const uint4 *p = reinterpret_cast<const uint4 *>(X + ((size_t)G * TB + t) * 8);
        const uint4 v0 = p[0], v1 = p[1];
        dst[0] = v0.x; dst[1] = v0.y; dst[2] = v0.z; dst[3] = v0.w;
        dst[4] = v1.x; dst[5] = v1.y; dst[6] = v1.z; dst[7] = v1.w;
    };
    if constexpr (TYPE == MIQ_TYPE_Q6_K) {
        const int S = K / 16;
        const int b = u >> 2, c = u & 3, blk2 = c >> 1, half = c & 1;
        const RawQ6K raw = load_q6k(rs, row_off + (uint32_t)b * kQ6KBytes, c);
        uint32_t Xf[4][8];
        const uint32_t *Xp[4];
        for (int p = 0; p < 4; p++) {
            xg(b * 8 + blk2 * 4 + p, Xf[p]);
            Xp[p] = Xf[p] + 4 * half;
        }
        int wd[4];
        dots_q6k(raw, Xp, wd);
        int32_t *o = out + ((size_t)t * n_rows + row) * S;
        for (int p = 0; p < 4; p++) o[b * 16 + blk2 * 8 + 2 * p + half] = wd[p];
    } else {
        const int S = K / 32;
        int wd0, wd1, G0;
        uint32_t X0[8], X1[8];
        if constexpr (TYPE == MIQ_TYPE_Q8_0) {
            G0 = 2 * u;
            xg(G0, X0);
            xg(G0 + 1, X1);
            dots_q80(load_q80(rs, row_off + (uint32_t)u * 68u), X0, X1, wd0, wd1);
        } else {
            const int b = u >> 2, c = u & 3;
            G0 = b * 8 + 2 * c;
            xg(G0, X0);
            xg(G0 + 1, X1);
            const uint32_t boff = row_off + (uint32_t)b * block_bytes(TYPE);
            if constexpr (TYPE == MIQ_TYPE_Q4_K) dots_q4k(load_q4k(rs, boff, c), X0, X1, wd0, wd1);
            else dots_q5k(load_q5k(rs, boff, c), c, X0, X1, wd0, wd1);
        }
        int32_t *o = out + ((size_t)t * n_rows + row) * S;
        o[G0] = wd0;
        o[G0 + 1] = wd1;
    }
}

// Parity hook (path 5): the Q4_K piece decoder of the GEMV at two or more
// tokens.  One wave per (token, row, run of eight blocks), lane = piece.
__global__ __launch_bounds__(64) void piece_dots_kernel(const uint8_t *w, uint32_t w_bytes, uint32_t row_bytes, int K,
                                                        int n_rows, const int8_t *x8, int TB, int32_t *out) {
    const int nblk = K / 256, runs = (nblk + 7) / 8;
    const int run = blockIdx.x % runs, row = (blockIdx.x / runs) % n_rows, t = blockIdx.x / (runs * n_rows);
    const int lane = threadIdx.x, p = run * 64 + lane;
    const bool ok = p < 8 * nblk;
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(w, w_bytes);
    PieceQ4K pc = load_q4k_piece(rs, ok ? (uint32_t)row * row_bytes + (uint32_t)(p >> 3) * kQ4KBytes : w_bytes, p & 7);
    const int i = p & 7, c = i >> 1, h = i & 1, G0 = (p >> 3) * 8 + 2 * c;
    const uint4 *X = reinterpret_cast<const uint4 *>(x8);
    const uint4 x0 = ok ? X[((size_t)G0 * TB + t) * 2 + h] : make_uint4(0, 0, 0, 0);
    const uint4 x1 = ok ? X[((size_t)(G0 + 1) * TB + t) * 2 + h] : make_uint4(0, 0, 0, 0);
    const uint32_t q[4] = {pc.q.x, pc.q.y, pc.q.z, pc.q.w};
    const uint32_t X0[4] = {x0.x, x0.y, x0.z, x0.w}, X1[4] = {x1.x, x1.y, x1.z, x1.w};
    const int wd = piece_dot(q, X0, X1, h);
    if (ok) out[((size_t)t * n_rows + row) * (K / 32) + G0 + h] = wd;
}

int launch_piece_dots(hipStream_t stream, const miq_seg *s, int TB, int32_t *out) {
    if (s->type != MIQ_TYPE_Q4_K) {
        set_error("miq_group_dots: path 5 (the GEMV's Q4_K piece decoder) serves Q4_K only");
        return MIQ_UNSUPPORTED;
    }
    const uint32_t rb = (uint32_t)miq_row_bytes(s->type, s->K);
    const uint32_t wb = (uint32_t)((size_t)s->n_rows * rb);
    const long n = (long)TB * s->n_rows * ((s->K / 256 + 7) / 8);
    hipLaunchKernelGGL(piece_dots_kernel, dim3((unsigned)n), dim3(64), 0, stream, (const uint8_t *)s->w, wb, rb, s->K,
                       s->n_rows, s->x8, TB, out);
    return check_launch("miq_group_dots");
}

int launch_unit_dots(hipStream_t stream, const miq_seg *s, int TB, int32_t *out) {
    const uint32_t rb = (uint32_t)miq_row_bytes(s->type, s->K);
    const uint32_t wb = (uint32_t)((size_t)s->n_rows * rb);
    const long n = (long)TB * s->n_rows * (s->K / 64);
    const dim3 grid((unsigned)((n + 255) / 256));
    const uint8_t *w = (const uint8_t *)s->w;
    switch (s->type) {
    case MIQ_TYPE_Q4_K:
        hipLaunchKernelGGL(unit_dots_kernel<MIQ_TYPE_Q4_K>, grid, dim3(256), 0, stream, w, wb, rb, s->K, s->n_rows, s->x8, TB, out);
        break;
    case MIQ_TYPE_Q5_K:
        hipLaunchKernelGGL(unit_dots_kernel<MIQ_TYPE_Q5_K>, grid, dim3(256), 0, stream, w, wb, rb, s->K, s->n_rows, s->x8, TB, out);
        break;
    case MIQ_TYPE_Q6_K:
        hipLaunchKernelGGL(unit_dots_kernel<MIQ_TYPE_Q6_K>, grid, dim3(256), 0, stream, w, wb, rb, s->K, s->n_rows, s->x8, TB, out);
        break;
    default:
        hipLaunchKernelGGL(unit_dots_kernel<MIQ_TYPE_Q8_0>, grid, dim3(256), 0, stream, w, wb, rb, s->K, s->n_rows, s->x8, TB, out);
        break;
    }
    return check_launch("miq_group_dots");
}

}  // namespace miq
