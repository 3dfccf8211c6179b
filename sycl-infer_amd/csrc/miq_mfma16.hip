// Batched decode GEMM for 5..47 tokens on int8 MFMA (v_mfma_i32_16x16x32_i8).
//
// One 32-value activation group is exactly one MFMA K step, so every MFMA
// result is the exact int32 group dot of the reference (i8.cpp:49-57,109-118;
// Q6_K: one 16-sub-group per MFMA by masking half the K lanes; Q8_0:
// q4exp.cpp:457-467).  The fp32 epilogue then applies the scales per group.
//
// Mapping: MFMA A = activations (16 tokens x 32), B = weights (32 x 16 rows),
// C[token][row].  Lane l holds column l%16 (its own weight row, whose block
// header it decodes) and tokens 4*(l/16)+v, v = 0..3.  Weights stream from
// HBM straight into B registers (each weight byte is used by one wave only).
// The dmin*m*xsum term of Q4_K/Q5_K is a rank-G product and runs on fp32 MFMA
// (v_mfma_f32_16x16x4_f32: tokens x 4 groups times 4 groups x rows).
//
// Two forms: the split-K kernel (m16z_kernel, the default), where a workgroup
// of 4 or 8 waves owns a 64- or 128-row tile and one K slice and stages that
// slice's activation in LDS for its waves; and the CU-resident kernel
// (m16c_kernel), one persistent workgroup per CU that stages its K part's
// activation once and streams its share of the row tiles.
#include <cstdlib>

#include "miq_internal.h"
#include "miq_units.h"

namespace miq {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));

struct M16Args {
    const uint8_t *w;
    uint32_t w_bytes;
    uint32_t row_bytes;
    int K;
    int n_rows;
    int TB;  // tokens in the activation layout; this launch covers 16 per blockIdx.y
    const int8_t *x8;
    const float *xmeta;
    const int32_t *xsumq;
    float *out;
    int out_stride;
    const float *residual;
    float alpha;
};

__device__ __forceinline__ v4i mfma_i8(long a, long b, v4i c) {
    return __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ v4f mfma_f32(float a, float b, v4f c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ long pack2(uint32_t lo, uint32_t hi) {
    return (long)(((unsigned long)hi << 32) | lo);
}

// 8 bytes at a 2-byte-aligned offset
__device__ __forceinline__ uint2 bload8_u2(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    const uint32_t a = off & ~3u, sh = off & 3u;
    const uint32_t d0 = bload4(r, a), d1 = bload4(r, a + 4), d2 = bload4(r, a + 8);
    return make_uint2(__builtin_amdgcn_alignbyte(d1, d0, sh), __builtin_amdgcn_alignbyte(d2, d1, sh));
}

// ---------------------------------------------------------------------------
// Weight-side MFMA operands of one 256-value K step for lane (row, h): the 8
// codes at positions 8h..8h+7 of each of the 8 groups, plus the row's scales.
// Shared by the GEMM and its parity hook.

__device__ __forceinline__ uint2 bload8(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0));
}

struct WQ6K {
    uint2 ql[4], qh[2];
    uint32_t scw[4];
    float d;
    __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t rs, uint32_t boff, int h) {
        const uint32_t dl = bload4(rs, (boff + 208) & ~3u);
        d = h2f(__builtin_amdgcn_alignbyte(0u, dl, (boff + 208) & 3u) & 0xFFFFu);
        const uint4 sc16 = bload16_u2(rs, boff + 192);
        scw[0] = sc16.x; scw[1] = sc16.y; scw[2] = sc16.z; scw[3] = sc16.w;
#pragma unroll
        for (int i = 0; i < 4; i++) ql[i] = bload8_u2(rs, boff + (i >> 1) * 64 + (i & 1) * 32 + 8 * h);
#pragma unroll
        for (int i = 0; i < 2; i++) qh[i] = bload8_u2(rs, boff + 128 + i * 32 + 8 * h);
    }
    // signed codes (code - 32) of group g = (blk2 = g>>2, plane = g&3)  (i8.cpp:129-144)
    __device__ __forceinline__ long op(int g) const {
        const int blk2 = g >> 2, p = g & 3;
        const uint2 src = ql[blk2 * 2 + (p & 1)];
        const int nib = (p >= 2) ? 4 : 0;
        const uint32_t c0 = q6_signed(((src.x >> nib) & 0x0F0F0F0Fu) | (((qh[blk2].x >> (2 * p)) & 0x03030303u) << 4));
        const uint32_t c1 = q6_signed(((src.y >> nib) & 0x0F0F0F0Fu) | (((qh[blk2].y >> (2 * p)) & 0x03030303u) << 4));
        return pack2(c0, c1);
    }
    // d * scales[s] (i8.cpp:151)
    __device__ __forceinline__ float ds(int s) const { return d * (float)(int8_t)(scw[s >> 2] >> (8 * (s & 3))); }
    // scales[s], the sub-group's signed 8-bit scale
    __device__ __forceinline__ int sc(int s) const { return (int)(int8_t)(scw[s >> 2] >> (8 * (s & 3))); }
};

struct WQ80 {  // eight Q8_0 blocks
    uint2 q[8];
    float d[8];
    __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t rs, uint32_t boff, int h) {
#pragma unroll
        for (int g = 0; g < 8; g++) {
            const uint32_t b0 = boff + 34u * g;
            const uint32_t dl = bload4(rs, b0 & ~3u);
            d[g] = h2f(__builtin_amdgcn_alignbyte(0u, dl, b0 & 3u) & 0xFFFFu);
            q[g] = bload8_u2(rs, b0 + 2 + 8 * h);
        }
    }
    __device__ __forceinline__ long op(int g) const { return pack2(q[g].x, q[g].y); }
};

// The 6-bit (scale, min) pairs of a Q4_K/Q5_K block header, four per dword as
// bytes (get_scale_min_k4, quant.h:136-144, done for all 8 groups at once):
// groups 0-3 sit in the low 6 bits of scales[0..3] / scales[4..7]; groups 4-7
// take their low nibble from scales[8..11] and their top 2 bits from the top
// of scales[0..3] (scale) / scales[4..7] (min).
__device__ __forceinline__ uint32_t scales_lo(uint4 hdr) { return hdr.y & 0x3F3F3F3Fu; }
__device__ __forceinline__ uint32_t mins_lo(uint4 hdr) { return hdr.z & 0x3F3F3F3Fu; }
__device__ __forceinline__ uint32_t scales_hi(uint4 hdr) {
    return (hdr.w & 0x0F0F0F0Fu) | ((hdr.y >> 2) & 0x30303030u);
}
__device__ __forceinline__ uint32_t mins_hi(uint4 hdr) {
    return ((hdr.w >> 4) & 0x0F0F0F0Fu) | ((hdr.z >> 2) & 0x30303030u);
}
// byte k of w as float (one v_cvt_f32_ubyteN)
__device__ __forceinline__ float byte_f(uint32_t w, int k) { return (float)((w >> (8 * k)) & 0xFFu); }

__host__ __device__ constexpr uint32_t kstep_bytes(uint32_t type) {
    return type == MIQ_TYPE_Q8_0 ? 8u * kQ80Bytes : (uint32_t)block_bytes(type);
}

// activation operand: token tok, group Gi, bytes 8h..8h+7 (zero for padding tokens)
__device__ __forceinline__ long act_op(const int8_t *x8, int TB, int Gi, int tok, bool ok, int h) {
    uint2 v = make_uint2(0, 0);
    if (ok) v = *reinterpret_cast<const uint2 *>(x8 + ((size_t)Gi * TB + tok) * 32 + 8 * h);
    return pack2(v.x, v.y);
}

// Weight operands of one K step for WN row tiles.
template <uint32_t TYPE> struct WOf;
template <> struct WOf<MIQ_TYPE_Q6_K> { using T = WQ6K; };
template <> struct WOf<MIQ_TYPE_Q8_0> { using T = WQ80; };

template <uint32_t TYPE>
__device__ __forceinline__ void wload(typename WOf<TYPE>::T &W, __amdgpu_buffer_rsrc_t rs, uint32_t boff, int h) {
    W.load(rs, boff, h);
}

// ---------------------------------------------------------------------------
// Split-K form (the default).  A workgroup is NW (4 or 8) waves on one
// 16*NW-row x 16-token tile and one K slice of it (a few 256-value K steps);
// wave w owns rows 16w..16w+15.  Workgroups are short and many, and every load
// a workgroup needs is issued at its start: the slice's activation (codes,
// scales, sums) goes to LDS once and is shared by the NW waves, and each wave's weights for
// the whole slice land in registers while the staging completes.  The fold
// then waits for each K step's own loads only.
//
// Slices of one tile run on one XCD (blockIdx % 8 == XCD, the dispatcher's
// placement): blockIdx = 8 * (tile / 8 * S + slice) + tile % 8.  With one
// slice the tile is written directly; otherwise each slice leaves its partial
// in the split-K scratch, and the last slice to arrive (arrival counter) sums
// the S partials in slice order -- deterministic whatever the arrival order --
// applies alpha and the residual and re-arms the counter.  The partials meet
// in the XCD's L2 (stores drained before the arrival is counted, L1-bypassing
// loads); a workgroup that finds itself on another XCD (HW_REG_XCC_ID) falls
// back to agent-scope fences and marks the counter so the reducer fences too.
constexpr size_t kZSlotX = 8 * 512;    // codes of one K step: [group][h][token][8 B]
constexpr size_t kZSlotM = 8 * 16 * 4; // one fp32 per (group, token)
constexpr int kZXcd = 8;
constexpr uint32_t kZFar = 1u << 20;   // counter mark: a partial came from another XCD
// K steps per slice at most (register budget of the weight operands)
template <uint32_t TYPE> constexpr int z_ks() {
    return TYPE == MIQ_TYPE_Q8_0 ? 2 : TYPE == MIQ_TYPE_Q6_K ? 3 : TYPE == MIQ_TYPE_Q5_K ? 5 : 7;
}
// vector-memory loads one wload<TYPE>() issues
template <uint32_t TYPE> constexpr int wloads_per_step() {
    return TYPE == MIQ_TYPE_Q4_K ? 3 : TYPE == MIQ_TYPE_Q5_K ? 4 : TYPE == MIQ_TYPE_Q6_K ? 21 : 32;
}
template <int KS> constexpr size_t z_lds() { return KS * (kZSlotX + 3 * kZSlotM); }

// One weight matrix of a split-K launch.  Several matrices over one
// activation (gate and up) run in one launch, each with the tiles, slices and
// scratch it has alone (so each result is bit-identical to its own launch):
// segment i owns blocks [b0, next b0), a multiple of 8 so that the XCD
// placement holds within it.
constexpr int kZSegs = 8;
struct ZSeg {
    const uint8_t *w;
    float *out;
    const float *residual;
    uint32_t w_bytes;
    int n_rows;
    int out_stride;
    float alpha;
    int b0;         // first block
    int ngrp;       // row groups of 16 * waves rows
    int ntile;      // token tiles x ngrp
    int S;          // K slices per tile
    uint32_t poff;  // this segment's partial tiles, [ntile][S][256 * waves] from part + poff
    uint32_t coff;  // its arrival counters, [ntile] from cnt + coff
};

struct ZArgs {
    M16Args a;      // the shared activation, K, row bytes and tokens (its matrix fields unused)
    int nkb;        // K steps per row (the last one partial for Q8_0 when K % 256 != 0)
    int nseg;
    float *part;    // partial tiles of every segment
    uint32_t *cnt;  // arrival counters, zero between launches
    ZSeg seg[kZSegs];
};

// Q4_K odd-group codes straight from the packed byte: (b & 0xF0) ^ 0x80 per
// byte, i.e. 16*q - 128 as a signed int8, in one v_bitop3.  The MFMA then
// yields I' = 16*I - 128*xsum, so I = (I' + 128*xsum) / 16 exactly.
__device__ __forceinline__ uint32_t q4_hi16(uint32_t w) { return __builtin_amdgcn_bitop3_b32(w, 0xF0F0F0F0u, 0x80808080u, 0x6A); }

// Q4_K/Q5_K operands of one K step for the split-K kernel.  Lane (col, h)
// loads dword h of the block header only (the fold gathers the 4 dwords
// across the lanes with two permlane swaps), and the 128 code bytes as two
// 16-byte pieces: qs bytes [16h, 16h+16) and [64+16h, 64+16h+16) of its row.
// The MFMA wants lane h to hold bytes [32j+8h, 32j+8h+8) of pair j; with the
// rows of 16 lanes indexed by h, a permlane16 swap of the pieces' 8-byte
// halves followed by a permlane32 swap produces exactly that (pairs 0, 1 from
// the first piece, 2, 3 from the second).
struct WZ45 {
    uint32_t hw;
    uint4 qa, qb;
    uint2 qh;
    template <uint32_t TYPE> __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t rs, uint32_t boff, int h) {
        hw = bload4(rs, boff + 4 * h);
        constexpr uint32_t qoff = TYPE == MIQ_TYPE_Q4_K ? 16 : 48;
        qa = bload16(rs, boff + qoff + 16 * h);
        qb = bload16(rs, boff + qoff + 64 + 16 * h);
        qh = make_uint2(0, 0);
        if constexpr (TYPE == MIQ_TYPE_Q5_K) qh = bload8(rs, boff + 16 + 8 * h);
    }
    // Lane (col, h) holds header dword h of row col; lanes col + 16h share the row.
    // permlane32_swap: rows {0,1,2,3} -> {D0,D1,D0,D1} and {D2,D3,D2,D3};
    // permlane16_swap of each spreads one dword over all four rows.
    __device__ __forceinline__ uint4 hdr() const {
        const auto a = __builtin_amdgcn_permlane32_swap(hw, hw, false, false);
        const auto b = __builtin_amdgcn_permlane16_swap(a[0], a[0], false, false);
        const auto c = __builtin_amdgcn_permlane16_swap(a[1], a[1], false, false);
        return make_uint4(b[0], b[1], c[0], c[1]);
    }
    // piece (lo = x,y; hi = z,w) of rows h = 0..3 -> pairs (2c, 2c+1) in MFMA order
    __device__ __forceinline__ static void split(const uint4 &q, uint2 &p0, uint2 &p1) {
        const auto s0 = __builtin_amdgcn_permlane16_swap(q.x, q.z, false, false);
        const auto s1 = __builtin_amdgcn_permlane16_swap(q.y, q.w, false, false);
        const auto t0 = __builtin_amdgcn_permlane32_swap(s0[0], s0[1], false, false);
        const auto t1 = __builtin_amdgcn_permlane32_swap(s1[0], s1[1], false, false);
        p0 = make_uint2(t0[0], t1[0]);
        p1 = make_uint2(t0[1], t1[1]);
    }
    __device__ __forceinline__ void pairs(uint2 (&qs)[4]) const {
        split(qa, qs[0], qs[1]);
        split(qb, qs[2], qs[3]);
    }
    template <uint32_t TYPE> __device__ __forceinline__ long op(const uint2 (&qs)[4], int g) const {
        const uint2 q = qs[g >> 1];
        if constexpr (TYPE == MIQ_TYPE_Q4_K) {
            if (g & 1) return pack2(q4_hi16(q.x), q4_hi16(q.y));
            return pack2(q.x & 0x0F0F0F0Fu, q.y & 0x0F0F0F0Fu);
        } else {
            const int nib = (g & 1) * 4;
            const uint32_t c0 = ((q.x >> nib) & 0x0F0F0F0Fu) | (((qh.x >> g) & 0x01010101u) << 4);
            const uint32_t c1 = ((q.y >> nib) & 0x0F0F0F0Fu) | (((qh.y >> g) & 0x01010101u) << 4);
            return pack2(c0, c1);
        }
    }
};
template <uint32_t TYPE> struct ZOf { using T = WZ45; };
template <> struct ZOf<MIQ_TYPE_Q6_K> { using T = WQ6K; };
template <> struct ZOf<MIQ_TYPE_Q8_0> { using T = WQ80; };

// Fold one staged K step (LDS slot `slot`, K step kb of the row) into the
// 16x16 tile accumulators: acc += per-group fp32 epilogue of the int8 MFMA
// dots; t2 collects the Q4_K/Q5_K dmin*m*xsum term (subtracted at the end).
// LDS slot layout: codes [group][16-byte half][token][16 B] at lx + slot*4 KiB;
// scales lsx and the two code sums ls0/ls1 [slot][group][token].
template <uint32_t TYPE>
__device__ __forceinline__ void z_fold(const int8_t *lx, const float *lsx, const float *ls0, const float *ls1,
                                       int slot, int kb, const typename ZOf<TYPE>::T &Wr, int h, int col, int K,
                                       v4f &acc, v4f &t2) {
        const int8_t *xg = lx + slot * kZSlotX + (h >> 1) * 256 + col * 16 + (h & 1) * 8;
        const float *sg = lsx + slot * 128 + 4 * h;
        if constexpr (TYPE == MIQ_TYPE_Q4_K || TYPE == MIQ_TYPE_Q5_K) {
            const uint4 hd = Wr.hdr();
            uint2 qs[4];
            Wr.pairs(qs);
            const float d = h2f(hd.x), dm = h2f(hd.x >> 16);
            const uint32_t sc4[2] = {scales_lo(hd), scales_hi(hd)};
            const uint32_t m4[2] = {mins_lo(hd), mins_hi(hd)};
            // Q4_K odd groups carry 16x codes (WZ45::op): scale by d/16
            const float dodd = TYPE == MIQ_TYPE_Q4_K ? d * 0.0625f : d;
            // two halves of four groups: four MFMAs in flight, then their epilogue
#pragma unroll
            for (int hf = 0; hf < 2; hf++) {
                v4i I[4];
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    const int g = 4 * hf + k;
                    const long wb = Wr.template op<TYPE>(qs, g);
                    I[k] = mfma_i8(*reinterpret_cast<const long *>(xg + g * 512), wb, v4i{0, 0, 0, 0});
                }
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    const int g = 4 * hf + k;
                    const v4f sx = *reinterpret_cast<const v4f *>(sg + g * 16);
                    const float dsc = ((g & 1) ? dodd : d) * byte_f(sc4[hf], k);
#pragma unroll
                    for (int v = 0; v < 4; v++) acc[v] += sx[v] * (dsc * (float)I[k][v]);
                }
            }
            // dmin*m*xsum (and, for Q4_K odd groups, the -8*d*sc*xsum the 16x
            // codes leave over): tokens x groups times groups x rows
#pragma unroll
            for (int qq = 0; qq < 2; qq++) {
                const int g = 4 * qq + h;
                float b = dm * byte_f(m4[qq] >> (8 * h), 0);
                if constexpr (TYPE == MIQ_TYPE_Q4_K)
                    if (h & 1) b -= 8.0f * d * byte_f(sc4[qq] >> (8 * h), 0);
                const int e = slot * 128 + g * 16 + col;
                t2 = mfma_f32(lsx[e] * (float)(__builtin_bit_cast(int, ls0[e]) + __builtin_bit_cast(int, ls1[e])), b, t2);
            }
        } else if constexpr (TYPE == MIQ_TYPE_Q6_K) {
            // the two 16-value sub-groups' signed 8-bit scales join their dots
            // in integers (|sc0*I0 + sc1*I1| < 2^24: exact, and exact as fp32),
            // one fma per output and group adds sx times that, and d scales the
            // block's sum once
            v4f blk = {0, 0, 0, 0};
#pragma unroll
            for (int g = 0; g < 8; g++) {
                const long xa = *reinterpret_cast<const long *>(xg + g * 512);
                const long wb = Wr.op(g);
                const v4i I0 = mfma_i8(xa, h < 2 ? wb : 0, v4i{0, 0, 0, 0});
                const v4i I1 = mfma_i8(xa, h < 2 ? 0 : wb, v4i{0, 0, 0, 0});
                const v4f sx = *reinterpret_cast<const v4f *>(sg + g * 16);
                const int sc0 = Wr.sc(2 * g), sc1 = Wr.sc(2 * g + 1);
#pragma unroll
                for (int v = 0; v < 4; v++)
                    // 24-bit multiplies (|I| < 2^17, |sc| <= 128): full rate, the same integers
                    blk[v] = __builtin_fmaf(sx[v], (float)(__mul24(I0[v], sc0) + __mul24(I1[v], sc1)), blk[v]);
            }
#pragma unroll
            for (int v = 0; v < 4; v++) acc[v] = __builtin_fmaf(Wr.d, blk[v], acc[v]);
        } else {
#pragma unroll
            for (int g = 0; g < 8; g++) {
                const v4i I = mfma_i8(*reinterpret_cast<const long *>(xg + g * 512), Wr.op(g), v4i{0, 0, 0, 0});
                const v4f sx = *reinterpret_cast<const v4f *>(sg + g * 16);
                // groups past the row end (partial last step) hold the next row's bytes
                const float dg = kb * 8 + g < K / 32 ? Wr.d[g] : 0.0f;
#pragma unroll
                for (int v = 0; v < 4; v++) acc[v] += sx[v] * (dg * (float)I[v]);
            }
        }
}

// Buffer loads straight into LDS, issued as inline asm so that the compiler
// does not track them: its tracking of a load into LDS cannot tell the target
// from other LDS accesses and would wait for every such load before the first
// LDS read.  Lane l writes lds_addr + 16 * l (dwordx4) or + 4 * l (dword),
// lds_addr wave-uniform; the caller orders the loads against their readers
// with an explicit vmcnt and a barrier.  M0 is saved and restored.
__device__ __forceinline__ void z_dma16(__amdgpu_buffer_rsrc_t r, uint32_t lds_addr, uint32_t off) {
    const uint32_t base = __builtin_amdgcn_readfirstlane(lds_addr);
    uint32_t keep;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %1\n\t"
        "buffer_load_dwordx4 %2, %3, 0 offen lds\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(keep)
        : "s"(base), "v"(off), "s"(r)
        : "memory");
}
__device__ __forceinline__ void z_dma4(__amdgpu_buffer_rsrc_t r, uint32_t lds_addr, uint32_t off) {
    const uint32_t base = __builtin_amdgcn_readfirstlane(lds_addr);
    uint32_t keep;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %1\n\t"
        "buffer_load_dword %2, %3, 0 offen lds\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(keep)
        : "s"(base), "v"(off), "s"(r)
        : "memory");
}
// s_waitcnt vmcnt(n) for an n the unrolled caller makes a constant (the
// builtin needs a literal; the switch folds away)
__device__ __forceinline__ void z_wait_vm(int n) {
#define Z_WV(k) case k: __builtin_amdgcn_s_waitcnt(vmcnt_imm(k)); break;
#define Z_WV8(k) Z_WV(k) Z_WV(k + 1) Z_WV(k + 2) Z_WV(k + 3) Z_WV(k + 4) Z_WV(k + 5) Z_WV(k + 6) Z_WV(k + 7)
    switch (n) {
        Z_WV8(0) Z_WV8(8) Z_WV8(16) Z_WV8(24) Z_WV8(32) Z_WV8(40) Z_WV8(48) Z_WV8(56)
    default: __builtin_amdgcn_s_waitcnt(vmcnt_imm(0)); break;
    }
#undef Z_WV8
#undef Z_WV
}

// PD = 0: the slice's whole activation is staged and every weight load of
// the slice issued at entry, then the folds run in load order.  PD = -D
// (bounded form): each wave keeps D K steps in flight, each step being its
// activation slot followed by its weights, and issues the next step after
// each fold.  The loads of a CU return in issue order, so with everything
// issued at entry a workgroup's staging waits behind the whole weight stream
// of the workgroups that started before it on the CU; bounded, it waits
// behind at most D steps of theirs and the folds start early.
template <uint32_t TYPE, int KS, int PD, int NW>
__global__ __launch_bounds__(64 * NW, 16 / NW) void m16z_kernel(ZArgs P) {
    const M16Args &A = P.a;
    extern __shared__ __align__(16) uint8_t lds[];
    static_assert(PD <= 0, "PD: 0 (all at entry) or -D (bounded)");
    int8_t *lx = reinterpret_cast<int8_t *>(lds);
    float *lsx = reinterpret_cast<float *>(lds + KS * kZSlotX);
    float *ls0 = lsx + KS * 128, *ls1 = ls0 + KS * 128;
    __shared__ int lflag;

    int si = 0;
#pragma unroll
    for (int i = 1; i < kZSegs; i++)
        if (i < P.nseg && (int)blockIdx.x >= P.seg[i].b0) si = i;
    const ZSeg &G = P.seg[si];
    const int bx = (int)blockIdx.x - G.b0;  // b0 is a multiple of 8: bx % 8 is still the XCD
    const int x = bx % kZXcd, q = bx / kZXcd;
    const int S = G.S;
    const int tl = q / S, s = q - tl * S;
    const int tile = tl * kZXcd + x;
    if (tile >= G.ntile) return;
    const int nkb = P.nkb;
    const int tt = tile / G.ngrp, rg = tile - tt * G.ngrp;
    float *const part = P.part + G.poff;
    uint32_t *const cnt = P.cnt + G.coff;
    const int kb0 = s * nkb / S, nb = (s + 1) * nkb / S - kb0;

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int col = lane & 15, h = lane >> 4;
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(G.w, G.w_bytes);
    const uint32_t x_bytes = (uint32_t)(A.K / 32) * A.TB * 32;
    const uint32_t m_bytes = (uint32_t)(A.K / 32) * A.TB * 8;
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(A.x8, x_bytes);
    const __amdgpu_buffer_rsrc_t rm = make_rsrc(A.xmeta, m_bytes);
    const __amdgpu_buffer_rsrc_t rq = make_rsrc(A.xsumq, m_bytes);
    using W = typename ZOf<TYPE>::T;

    // ---- every weight load of this wave's 16 rows (a padding row or a step
    // past the slice reads zeros past the end of the tensor)
    const int row = rg * (16 * NW) + wave * 16 + col;
    W wr[KS];
    auto wissue = [&](int i) {
        const uint32_t off = (i < nb && row < G.n_rows) ? (uint32_t)row * A.row_bytes + (uint32_t)(kb0 + i) * kstep_bytes(TYPE)
                                                        : G.w_bytes;
        if constexpr (TYPE == MIQ_TYPE_Q4_K || TYPE == MIQ_TYPE_Q5_K) wr[i].template load<TYPE>(rs, off, h);
        else wload<TYPE>(wr[i], rs, off, h);
    };
    typedef __attribute__((address_space(3))) void *lds_ptr;
    const int tb = A.TB;
    if constexpr (PD >= 0) {
        // ---- activation of the slice, straight from global memory into LDS
        // (buffer loads with the lds bit: no registers held).  Per slot (K step):
        // codes [group][16-byte half][token][16 B], then fp32 scales and the two
        // code sums per (group, token).  A lane's 16-byte piece lands at
        // base + 16 * lane, so piece p = 64w + lane of wave w sits at 16p.
        // codes: four 1 KiB pieces per slot, piece j of the workgroup taken by wave j % NW
#pragma unroll
        for (int jj = 0; jj < (KS * 4 + NW - 1) / NW; jj++) {
            const int j = wave + NW * jj;
            if (j < KS * 4) {
                const int i = j >> 2, c = j & 3;
                const int p = c * 64 + lane;
                const int gl = p >> 5, hp = (p >> 4) & 1, tk = p & 15;
                const int t = tt * 16 + tk;
                const uint32_t off = (i < nb && t < tb) ? (uint32_t)(((kb0 + i) * 8 + gl) * tb + t) * 32 + 16 * hp : x_bytes;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (lds_ptr)(lx + i * kZSlotX + c * 1024), 16, off, 0, 0, 0);
            }
        }
        // meta: six 64-entry chunks per slot (scale, sum0, sum1; (group, token) 0..63, 64..127)
#pragma unroll
        for (int jj = 0; jj < (KS * 6 + NW - 1) / NW; jj++) {
            const int j = wave + NW * jj;
            if (j < KS * 6) {
                const int i = j / 6, ch = j - 6 * i;
                const int arr = ch >> 1, e = (ch & 1) * 64 + lane;
                const int gl = e >> 4, tk = e & 15;
                const int t = tt * 16 + tk;
                const bool ok = i < nb && t < tb;
                const uint32_t mo = (uint32_t)(((kb0 + i) * 8 + gl) * tb + t) * 8;
                float *dst = (arr == 0 ? lsx : arr == 1 ? ls0 : ls1) + i * 128 + (ch & 1) * 64;
                if (arr == 0) __builtin_amdgcn_raw_ptr_buffer_load_lds(rm, (lds_ptr)dst, 4, ok ? mo : m_bytes, 0, 0, 0);
                else __builtin_amdgcn_raw_ptr_buffer_load_lds(rq, (lds_ptr)dst, 4, ok ? mo + 4 * (arr - 1) : m_bytes, 0, 0, 0);
            }
        }
#pragma unroll
        for (int i = 0; i < KS; i++) wissue(i);
        // the staging loads are the oldest: wait for them only, then for every wave's
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(wloads_per_step<TYPE>() * KS));
        __syncthreads();
    }
    v4f acc = {0, 0, 0, 0}, t2 = {0, 0, 0, 0};
    auto fold = [&](int slot, int kb, const W &Wr) { z_fold<TYPE>(lx, lsx, ls0, ls1, slot, kb, Wr, h, col, A.K, acc, t2); };
    if constexpr (PD < 0) {
        // Bounded form: slot i's activation (four 1 KiB code pieces and six
        // 256-byte scale/sum chunks, piece j taken by wave j % NW, as untracked
        // loads) then K step i's weights; D = -PD steps in flight, the next
        // issued after each fold.  Fold i waits for its own slot and step (the
        // loads return in issue order), then a barrier shows it the other
        // waves' pieces of the slot.
        constexpr int D = -PD < KS ? -PD : KS;
        const uint32_t lds_at = (uint32_t)(uintptr_t)(lds_ptr)lds;
        constexpr int kPieces = 10, kMinStage = kPieces / NW;  // pieces per slot; fewest any wave issues
        constexpr int kJJ = (kPieces + NW - 1) / NW;
        // the lane's part of each of its pieces' source offsets, the same at
        // every step (the step adds a wave-uniform (kb0+i)*8*tb*stride);
        // ~0 where the piece's token is past the batch
        uint32_t pl[kJJ];
#pragma unroll
        for (int jj = 0; jj < kJJ; jj++) {
            const int j = wave + NW * jj;
            pl[jj] = ~0u;
            if (j < 4) {
                const int p = j * 64 + lane;
                const int gl = p >> 5, hp = (p >> 4) & 1, t = tt * 16 + (p & 15);
                if (t < tb) pl[jj] = (uint32_t)(gl * tb + t) * 32 + 16 * hp;
            } else if (j < kPieces) {
                const int ch = j - 4, arr = ch >> 1, e = (ch & 1) * 64 + lane;
                const int gl = e >> 4, t = tt * 16 + (e & 15);
                if (t < tb) pl[jj] = (uint32_t)(gl * tb + t) * 8 + (arr ? 4 * (arr - 1) : 0);
            }
        }
        auto issue = [&](int i) {
            const uint32_t sx = (uint32_t)(kb0 + i) * 8 * tb;  // the step's first (group, token) row
#pragma unroll
            for (int jj = 0; jj < kJJ; jj++) {
                const int j = wave + NW * jj;
                const bool ok = i < nb && pl[jj] != ~0u;
                if (j < 4) {
                    z_dma16(rx, lds_at + (uint32_t)(i * kZSlotX + j * 1024), ok ? pl[jj] + sx * 32 : x_bytes);
                } else if (j < kPieces) {
                    const int ch = j - 4, arr = ch >> 1;
                    const uint32_t dst = lds_at + (uint32_t)(KS * kZSlotX + (arr * KS * 128 + i * 128 + (ch & 1) * 64) * 4);
                    if (arr == 0) z_dma4(rm, dst, ok ? pl[jj] + sx * 8 : m_bytes);
                    else z_dma4(rq, dst, ok ? pl[jj] + sx * 8 : m_bytes);
                }
            }
            wissue(i);
        };
#pragma unroll
        for (int i = 0; i < D; i++) issue(i);
#pragma unroll
        for (int i = 0; i < KS; i++) {
            // loads issued after step i's: the steps up to min(i + D, KS) - 1
            // (steps past the slice read zeros, so every wave issues KS steps)
            z_wait_vm((i + D < KS ? D - 1 : KS - 1 - i) * (kMinStage + wloads_per_step<TYPE>()));
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
            __builtin_amdgcn_s_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
            if (i < nb) fold(i, kb0 + i, wr[i]);
            if (i + D < KS) issue(i + D);
        }
    } else {
#pragma unroll
        for (int i = 0; i < KS; i++)
            if (i < nb) fold(i, kb0 + i, wr[i]);
    }

    // ---- C[token 4h+v][row col]
    auto store = [&](const v4f &val) {
#pragma unroll
        for (int v = 0; v < 4; v++) {
            const int t = tt * 16 + 4 * h + v;
            if (row < G.n_rows && t < A.TB) {
                const size_t o = (size_t)t * G.out_stride + row;
                float r = G.alpha * val[v];
                if (G.residual) r += G.residual[o];
                G.out[o] = r;
            }
        }
    };
    v4f cv;
#pragma unroll
    for (int v = 0; v < 4; v++) cv[v] = acc[v] - t2[v];
    if (S == 1) {
        store(cv);
        return;
    }
    const bool far = (__builtin_amdgcn_s_getreg((3 << 11) | (0 << 6) | 20) & 15) != (uint32_t)x;  // HW_REG_XCC_ID
    constexpr int kTile = 256 * NW;  // fp32 outputs per tile
    *reinterpret_cast<v4f *>(part + ((size_t)tile * S + s) * kTile + threadIdx.x * 4) = cv;
    if (far) __threadfence();  // another XCD will read this partial: write it back past the L2
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint32_t prev = __hip_atomic_fetch_add(cnt + tile, far ? 1u + kZFar : 1u, __ATOMIC_RELAXED,
                                                     __HIP_MEMORY_SCOPE_AGENT);
        const int last = (prev & (kZFar - 1)) == (uint32_t)(S - 1);
        if (last) __hip_atomic_store(cnt + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        lflag = last ? 1 + (prev >= kZFar) : 0;
    }
    __syncthreads();
    const int fl = lflag;
    if (!fl) return;
    if (fl == 2 || far) __threadfence();  // some partial crossed XCDs: drop stale L2 lines first
    // four partials in flight at a time, summed in slice order; glc: past this
    // CU's L1 to the XCD's L2 where they met
    const __amdgpu_buffer_rsrc_t rp = make_rsrc(part, (uint32_t)((size_t)G.ntile * S * kTile * 4));
    const uint32_t pbase = (uint32_t)((size_t)tile * S * kTile + threadIdx.x * 4) * 4;
    v4f sum = {0, 0, 0, 0};
    for (int p0 = 0; p0 < S; p0 += 4) {
        v4f pv[4];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const uint32_t off = p0 + k < S ? pbase + (uint32_t)(p0 + k) * kTile * 4 : 0xFFFFFFF0u;
            pv[k] = __builtin_bit_cast(v4f, __builtin_amdgcn_raw_buffer_load_b128(rp, off, 0, 1));
        }
#pragma unroll
        for (int k = 0; k < 4; k++)
#pragma unroll
            for (int v = 0; v < 4; v++) sum[v] += pv[k][v];
    }
    store(sum);
}

// ---------------------------------------------------------------------------
// CU-resident form for up to 16 tokens (m16c): one persistent workgroup of 16
// waves per CU.  The K blocks are cut into KP parts (as few as let one part's
// activation fit the CU's LDS); the CUs form KP groups of G, CU gi of group kp
// taking the 16-row tiles [gi*NT/G, (gi+1)*NT/G) over K part kp.  The
// workgroup stages its K part's activation into LDS once, before any weight
// load (so no other workgroup's weight stream queues ahead of it on this CU),
// then its 16 waves split the (tile, K step) sequence into equal contiguous
// ranges and stream their weight bytes with PD steps in flight.  A tile that
// one wave covers completely is finished by that wave; the pieces of a tile
// shared by waves meet in LDS and are added in wave order.  With KP > 1 the
// parts of a tile meet in a global partial buffer (their CUs share an XCD),
// the last to arrive adding them in part order.
constexpr int kCWaves = 8;
constexpr int kCMaxSteps = 20;                        // K steps of activation one CU holds
constexpr size_t kCRedOff = kCMaxSteps * (kZSlotX + 3 * kZSlotM);
constexpr size_t kCLds = kCRedOff + (size_t)kCWaves * 2 * 256 * 4;  // + per wave two 16x16 fp32 pieces

struct CArgs {
    M16Args a;
    int nkb;        // K steps per row
    int KP;         // K parts
    int G;          // workgroups per K part
    int NT;         // 16-row tiles
    float *part;    // [NT][KP][256] fp32 (KP > 1)
    uint32_t *cnt;  // [NT] arrival counters, zero between launches (KP > 1)
};

template <uint32_t TYPE> constexpr int c_pd() {  // K steps in flight per wave
    return TYPE == MIQ_TYPE_Q8_0 ? 2 : TYPE == MIQ_TYPE_Q6_K ? 3 : 4;
}

template <uint32_t TYPE>
__global__ __launch_bounds__(64 * kCWaves, 1) void m16c_kernel(CArgs P) {
    constexpr int PD = c_pd<TYPE>(), R = PD + 1;
    const M16Args &A = P.a;
    extern __shared__ __align__(16) uint8_t lds[];
    int8_t *lx = reinterpret_cast<int8_t *>(lds);
    float *lsx = reinterpret_cast<float *>(lds + kCMaxSteps * kZSlotX);
    float *ls0 = lsx + kCMaxSteps * 128, *ls1 = ls0 + kCMaxSteps * 128;
    float *red = reinterpret_cast<float *>(lds + kCRedOff);  // [wave][2][256]

    const int b = blockIdx.x, kp = b / P.G, gi = b - kp * P.G;
    const int kb0 = kp * P.nkb / P.KP, ns = (kp + 1) * P.nkb / P.KP - kb0;
    const int tl0 = gi * P.NT / P.G, ntl = (gi + 1) * P.NT / P.G - tl0;
    if (ntl <= 0) return;
    // the wave index as a wave-uniform value: the (tile, step) bookkeeping
    // below (divisions by the step count) then runs on the scalar unit
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int col = lane & 15, h = lane >> 4;
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(A.w, A.w_bytes);
    const int tb = A.TB;
    const uint32_t x_bytes = (uint32_t)(A.K / 32) * tb * 32;
    const uint32_t m_bytes = (uint32_t)(A.K / 32) * tb * 8;
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(A.x8, x_bytes);
    const __amdgpu_buffer_rsrc_t rm = make_rsrc(A.xmeta, m_bytes);
    const __amdgpu_buffer_rsrc_t rq = make_rsrc(A.xsumq, m_bytes);
    typedef __attribute__((address_space(3))) void *lds_ptr;

    // ---- the K part's activation into LDS: codes (256 16-byte pieces per
    // step, piece p of step i at i*4 KiB + 16p: group p>>5, half (p>>4)&1,
    // token p&15), then scale / sum0 / sum1 (128 dwords per step each).  A
    // lane's piece lands at the wave's base + 16 * lane (4 * lane for dwords).
    const int nblk = ns * 4, nblm = ns * 2;  // 64-piece blocks of codes / of one meta array
    for (int k = wave; k < nblk; k += kCWaves) {
        const int pb = k * 64;
        const int p = pb + lane, i = p >> 8, q = p & 255;
        const int gl = q >> 5, hp = (q >> 4) & 1, tk = q & 15;
        const uint32_t off = (p < ns * 256 && tk < tb) ? (uint32_t)(((kb0 + i) * 8 + gl) * tb + tk) * 32 + 16 * hp : x_bytes;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (lds_ptr)(lx + (size_t)pb * 16), 16, off, 0, 0, 0);
    }
    for (int arr = 0; arr < 3; arr++) {
        float *dst0 = arr == 0 ? lsx : arr == 1 ? ls0 : ls1;
        for (int k = wave; k < nblm; k += kCWaves) {
            const int eb = k * 64;
            const int e = eb + lane, i = e >> 7, gl = (e & 127) >> 4, tk = e & 15;
            const bool ok = e < ns * 128 && tk < tb;
            const uint32_t mo = (uint32_t)(((kb0 + i) * 8 + gl) * tb + tk) * 8;
            if (arr == 0) __builtin_amdgcn_raw_ptr_buffer_load_lds(rm, (lds_ptr)(dst0 + eb), 4, ok ? mo : m_bytes, 0, 0, 0);
            else __builtin_amdgcn_raw_ptr_buffer_load_lds(rq, (lds_ptr)(dst0 + eb), 4, ok ? mo + 4 * (arr - 1) : m_bytes, 0, 0, 0);
        }
    }

    // ---- this wave's range of the (tile, step) sequence
    const int total = ntl * ns;
    const int r0 = wave * total / kCWaves, r1 = (wave + 1) * total / kCWaves;
    using W = typename ZOf<TYPE>::T;
    W wb[R];
    // the (tile, step) of the next weight issue, advanced one step per issue
    // (no division by the step count inside the loop)
    int w_j = r0, w_tau = r0 / ns, w_i = r0 - (r0 / ns) * ns;
    auto wissue = [&](W &Wr) {
        uint32_t off = A.w_bytes;
        if (w_j < r1) {
            const int row = (tl0 + w_tau) * 16 + col;
            if (row < A.n_rows) off = (uint32_t)row * A.row_bytes + (uint32_t)(kb0 + w_i) * kstep_bytes(TYPE);
        }
        w_j++;
        if (++w_i == ns) {
            w_i = 0;
            w_tau++;
        }
        if constexpr (TYPE == MIQ_TYPE_Q4_K || TYPE == MIQ_TYPE_Q5_K) Wr.template load<TYPE>(rs, off, h);
        else wload<TYPE>(Wr, rs, off, h);
    };
#pragma unroll
    for (int u = 0; u < PD; u++) wissue(wb[u]);
    // the staging loads are older than the weight loads: wait for them only
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(wloads_per_step<TYPE>() * PD));
    __syncthreads();

    // ---- finishing a tile: C[token 4h+v][row col] for this K part
    const bool far = (__builtin_amdgcn_s_getreg((3 << 11) | (0 << 6) | 20) & 15) != (uint32_t)(b % 8);  // HW_REG_XCC_ID
    auto store = [&](int tile, const v4f &val) {
        const int row = tile * 16 + col;
#pragma unroll
        for (int v = 0; v < 4; v++) {
            const int t = 4 * h + v;
            if (row < A.n_rows && t < A.TB) {
                const size_t o = (size_t)t * A.out_stride + row;
                float r = A.alpha * val[v];
                if (A.residual) r += A.residual[o];
                A.out[o] = r;
            }
        }
    };
    auto finish = [&](int tile, const v4f &val) {  // one wave
        if (P.KP == 1) {
            store(tile, val);
            return;
        }
        constexpr uint32_t kFar = 1u << 20;
        *reinterpret_cast<v4f *>(P.part + ((size_t)tile * P.KP + kp) * 256 + lane * 4) = val;
        if (far) __threadfence();  // the part's partner may sit on another XCD
        __builtin_amdgcn_s_waitcnt(0);
        uint32_t prev = 0;
        if (lane == 0) prev = __hip_atomic_fetch_add(P.cnt + tile, far ? 1u + kFar : 1u, __ATOMIC_RELAXED,
                                                     __HIP_MEMORY_SCOPE_AGENT);
        prev = __builtin_amdgcn_readfirstlane(prev);
        if ((prev & (kFar - 1)) != (uint32_t)(P.KP - 1)) return;
        if (lane == 0) __hip_atomic_store(P.cnt + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (prev >= kFar || far) __threadfence();
        const __amdgpu_buffer_rsrc_t rp = make_rsrc(P.part + (size_t)tile * P.KP * 256, (uint32_t)P.KP * 1024);
        v4f sum = {0, 0, 0, 0};
        for (int k = 0; k < P.KP; k++)
            sum += __builtin_bit_cast(v4f, __builtin_amdgcn_raw_buffer_load_b128(rp, (uint32_t)(k * 256 + lane * 4) * 4, 0, 1));
        store(tile, sum);
    };

    // ---- stream the range: fold step jj while step jj+PD loads
    v4f acc = {0, 0, 0, 0}, t2 = {0, 0, 0, 0};
    int cur = r0 < r1 ? r0 / ns : 0;  // local tile being accumulated
    auto close = [&](int tau) {       // the wave's piece of local tile tau is complete
        const v4f val = acc - t2;
        const bool whole = r0 <= tau * ns && (tau + 1) * ns <= r1;
        if (whole) finish(tl0 + tau, val);
        else *reinterpret_cast<v4f *>(red + (wave * 2 + (tau * ns <= r0 ? 0 : 1)) * 256 + lane * 4) = val;
        acc = v4f{0, 0, 0, 0};
        t2 = v4f{0, 0, 0, 0};
    };
    int f_tau = cur, f_i = r0 - cur * ns;  // the (tile, step) of the next fold
    for (int j = r0; j < r1; j += R) {
#pragma unroll
        for (int u = 0; u < R; u++) {
            const int jj = j + u;
            wissue(wb[(u + PD) % R]);
            if (jj < r1) {
                const int tau = f_tau, i = f_i;
                if (++f_i == ns) {
                    f_i = 0;
                    f_tau++;
                }
                if (tau != cur) {
                    close(cur);
                    cur = tau;
                }
                // the fold at raised wave priority, so the SIMD's other wave
                // issues its loads in the fold's gaps (Q6_K head: 2 % faster)
                __builtin_amdgcn_s_setprio(1);
                z_fold<TYPE>(lx, lsx, ls0, ls1, i, kb0 + i, wb[u], h, col, A.K, acc, t2);
                __builtin_amdgcn_s_setprio(0);
            }
        }
    }
    if (r0 < r1) close(cur);

    // ---- tiles shared by waves: their pieces meet in LDS, added in wave order
    __syncthreads();
    auto owner = [&](int j) { return ((j + 1) * kCWaves + total - 1) / total - 1; };
    auto rstart = [&](int w) { return w * total / kCWaves; };
    for (int tau = wave; tau < ntl; tau += kCWaves) {
        const int w_lo = owner(tau * ns), w_hi = owner((tau + 1) * ns - 1);
        if (w_lo == w_hi) continue;  // finished by its one wave
        v4f sum = {0, 0, 0, 0};
        for (int w = w_lo; w <= w_hi; w++) {
            const int ws = rstart(w);
            if (ws == rstart(w + 1)) continue;  // an empty range
            sum += *reinterpret_cast<const v4f *>(red + (w * 2 + (tau * ns <= ws ? 0 : 1)) * 256 + lane * 4);
        }
        finish(tl0 + tau, sum);
    }
}

template <uint32_t TYPE> static int launch_m16c(hipStream_t stream, const M16Args &A) {
    int n_cu = 0, rc;
    if ((rc = device_cus(&n_cu))) return rc;
    CArgs P{};
    P.a = A;
    P.nkb = (A.K + 255) / 256;
    P.KP = 1;
    while ((P.nkb + P.KP - 1) / P.KP > kCMaxSteps) P.KP *= 2;
    P.G = n_cu / P.KP;
    if (P.G < 1) {
        set_error("miq mfma16: K=%d needs more K parts than CUs", A.K);
        return MIQ_UNSUPPORTED;
    }
    P.NT = (A.n_rows + 15) / 16;
    if (P.KP > 1) {
        const int rc2 = scratch_get(stream, (size_t)P.NT * P.KP * 1024, (size_t)P.NT, &P.part, &P.cnt);
        if (rc2 != MIQ_OK) return rc2;
    }
    static bool lds_set[64] = {false};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
        set_error("miq mfma16: no current device");
        return MIQ_EHIP;
    }
    if (!lds_set[dev]) {
        if (hipFuncSetAttribute((const void *)m16c_kernel<TYPE>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)kCLds) != hipSuccess) {
            set_error("miq mfma16: cannot raise the LDS limit to %zu bytes", kCLds);
            return MIQ_EHIP;
        }
        lds_set[dev] = true;
    }
    hipLaunchKernelGGL(m16c_kernel<TYPE>, dim3((unsigned)(P.KP * P.G)), dim3(64 * kCWaves), kCLds, stream, P);
    return MIQ_OK;
}

// Slices per tile.  Every workgroup should be resident at once (4 per CU at
// <= 128 VGPRs): then all loads go out in one round and no workgroup waits
// for a slot.  Among the slice counts that allow that, pick the one with the
// least work on the busiest CU, ceil(workgroups / CUs) x steps per slice; if
// none does, the fewest rounds x (steps per slice + a fixed cost).
static int z_slices(int nkb, int ks_max, int ntile, int n_cu, int nw) {
    const int slots = n_cu * 16 / nw;
    const int tpx = (ntile + kZXcd - 1) / kZXcd;
    int best = 0;
    double best_t = 0;
    for (int S = (nkb + ks_max - 1) / ks_max; S <= nkb; S++) {
        const long wg = (long)kZXcd * tpx * S;
        const int steps = (nkb + S - 1) / S;
        double t;
        if (wg <= slots) t = (double)((wg + n_cu - 1) / n_cu) * steps;
        else t = 1e6 + (double)((wg + slots - 1) / slots) * (steps + 2.0);
        if (!best || t < best_t - 1e-9) {
            best = S;
            best_t = t;
        }
    }
    return best;
}

// Segments As[0..nseg) share the activation, K and type; their row groups are
// laid end to end in one grid.
template <uint32_t TYPE> static int launch_m16z(hipStream_t stream, const M16Args *As, int nseg, int TB) {
    const M16Args &A = As[0];
    static int n_cu[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
        set_error("miq mfma16: no current device");
        return MIQ_EHIP;
    }
    if (!n_cu[dev] && hipDeviceGetAttribute(&n_cu[dev], hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) {
        set_error("miq mfma16: cannot query the CU count");
        return MIQ_EHIP;
    }
    constexpr int KS = z_ks<TYPE>();
    // waves per workgroup: 8 (128-row tiles, half the activation staging per
    // weight byte) measured faster for Q4_K, 4 for the others; MIQ_M16_WAVES=4|8
    const int nw_set = sw(kSwM16Waves);
    const int nw = nw_set == 4 || nw_set == 8 ? nw_set : TYPE == MIQ_TYPE_Q4_K ? 8 : 4;
    ZArgs P{};
    P.a = A;
    P.nkb = (A.K + 255) / 256;
    P.nseg = nseg;
    long nwg = 0;
    size_t part_floats = 0, n_cnt = 0;
    for (int i = 0; i < nseg; i++) {
        const M16Args &B = As[i];
        ZSeg &G = P.seg[i];
        G = ZSeg{B.w, B.out, B.residual, B.w_bytes, B.n_rows, B.out_stride, B.alpha, 0, 0, 0, 0, 0, 0};
        G.b0 = (int)nwg;
        G.ngrp = (B.n_rows + 16 * nw - 1) / (16 * nw);
        G.ntile = ((TB + 15) / 16) * G.ngrp;
        G.S = z_slices(P.nkb, KS, G.ntile, n_cu[dev], nw);
        G.poff = (uint32_t)part_floats;
        G.coff = (uint32_t)n_cnt;
        nwg += (long)kZXcd * ((G.ntile + kZXcd - 1) / kZXcd) * G.S;
        if (G.S > 1) {
            part_floats += (size_t)G.ntile * G.S * 256 * nw;
            n_cnt += (size_t)G.ntile;
        }
        if (part_floats * sizeof(float) >= 0xFFFFFFF0u || nwg >= (1L << 31)) {
            set_error("miq mfma16: shape too large for the split-K scratch (%zu bytes)", part_floats * sizeof(float));
            return MIQ_UNSUPPORTED;
        }
    }
    if (part_floats) {
        const int rc = scratch_get(stream, part_floats * sizeof(float), n_cnt, &P.part, &P.cnt);
        if (rc != MIQ_OK) return rc;
    }
    const dim3 grid((unsigned)nwg), block(64 * nw);
    // Q4_K slices of five or more K steps take the bounded form (two steps of
    // activation and weights in flight per wave; measured bit-identical, and
    // faster: 17408x5120 at 16 tokens 21.4 -> 20.5 us, at 8 tokens 21.3 ->
    // 20.1, gate+up in one launch 37.9 -> 35.0; 5120x17408 unchanged; at
    // K = 1024, four steps, 0.2 us slower; no gain for the other types)
    const int steps0 = (P.nkb + P.seg[0].S - 1) / P.seg[0].S;
    if constexpr (TYPE == MIQ_TYPE_Q4_K) {
        if (nw == 8 && steps0 >= 5) {
            hipLaunchKernelGGL((m16z_kernel<TYPE, KS, -2, 8>), grid, block, z_lds<KS>(), stream, P);
            return MIQ_OK;
        }
    }
    if (nw == 8) hipLaunchKernelGGL((m16z_kernel<TYPE, KS, 0, 8>), grid, block, z_lds<KS>(), stream, P);
    else hipLaunchKernelGGL((m16z_kernel<TYPE, KS, 0, 4>), grid, block, z_lds<KS>(), stream, P);
    return MIQ_OK;
}

// Parity hook (paths 1 and 4: the 16-token kernels' decoders, WZ45 for
// Q4_K/Q5_K, WQ6K, WQ80): the MFMA's int32 group dots, written as
// out[(t*n_rows+row)*S+s] (S = K/32; Q6_K: K/16 with the unsigned-code sum
// wd = I + 32*xsum_half restored, the quantity i8.cpp:149 forms).
template <uint32_t TYPE>
__global__ __launch_bounds__(64) void mfma16_dots_kernel(const uint8_t *w, uint32_t w_bytes, uint32_t row_bytes, int K,
                                                         int n_rows, const int8_t *x8, const int32_t *xsumq, int TB,
                                                         int32_t *out) {
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(w, w_bytes);
    const int lane = threadIdx.x, col = lane & 15, h = lane >> 4;
    const int row = blockIdx.x * 16 + col, kb = blockIdx.z, t0 = blockIdx.y * 16;
    const int tok = t0 + col;
    const bool row_ok = row < n_rows;
    const uint32_t boff = (uint32_t)(row_ok ? row : 0) * row_bytes + (uint32_t)kb * kstep_bytes(TYPE);
    const int S = TYPE == MIQ_TYPE_Q6_K ? K / 16 : K / 32;
    auto put = [&](int s, const v4i &I, int add_half) {
#pragma unroll
        for (int v = 0; v < 4; v++) {
            const int t = t0 + 4 * h + v;
            if (row_ok && t < TB) {
                int val = I[v];
                if (add_half >= 0) val += 32 * xsumq[((size_t)(s >> 1) * TB + t) * 2 + add_half];
                if (add_half == -2) {  // Q4_K odd group from 16x codes: I = (I' + 128*xsum) / 16
                    const int32_t *xs = xsumq + ((size_t)s * TB + t) * 2;
                    val = (val + 128 * (xs[0] + xs[1])) / 16;
                }
                out[((size_t)t * n_rows + row) * S + s] = val;
            }
        }
    };
    if constexpr (TYPE == MIQ_TYPE_Q6_K) {
        WQ6K W;
        W.load(rs, boff, h);
#pragma unroll
        for (int g = 0; g < 8; g++) {
            const long xa = act_op(x8, TB, kb * 8 + g, tok, tok < TB, h);
            const long wb = row_ok ? W.op(g) : 0;
            put(kb * 16 + 2 * g, mfma_i8(xa, h < 2 ? wb : 0, v4i{0, 0, 0, 0}), 0);
            put(kb * 16 + 2 * g + 1, mfma_i8(xa, h < 2 ? 0 : wb, v4i{0, 0, 0, 0}), 1);
        }
    } else {
        long wbs[8];
        if constexpr (TYPE == MIQ_TYPE_Q8_0) {
            WQ80 W;
            W.load(rs, boff, h);
#pragma unroll
            for (int g = 0; g < 8; g++) wbs[g] = W.op(g);
        } else {
            WZ45 W;
            W.load<TYPE>(rs, boff, h);
            uint2 qs[4];
            W.pairs(qs);
#pragma unroll
            for (int g = 0; g < 8; g++) wbs[g] = W.op<TYPE>(qs, g);  // Q4_K odd groups as 16x codes
        }
#pragma unroll
        for (int g = 0; g < 8; g++) {
            const long xa = act_op(x8, TB, kb * 8 + g, tok, tok < TB, h);
            put(kb * 8 + g, mfma_i8(xa, row_ok ? wbs[g] : 0, v4i{0, 0, 0, 0}),
                TYPE == MIQ_TYPE_Q4_K && (g & 1) ? -2 : -1);
        }
    }
}

int launch_mfma16_dots(hipStream_t stream, const miq_seg *s, int TB, int32_t *out) {
    const uint32_t rb = (uint32_t)miq_row_bytes(s->type, s->K);
    const uint32_t wb = (uint32_t)((size_t)s->n_rows * rb);
    const dim3 grid((s->n_rows + 15) / 16, (TB + 15) / 16, s->K / 256);
    const uint8_t *w = (const uint8_t *)s->w;
    switch (s->type) {
    case MIQ_TYPE_Q4_K: hipLaunchKernelGGL(mfma16_dots_kernel<MIQ_TYPE_Q4_K>, grid, dim3(64), 0, stream, w, wb, rb, s->K, s->n_rows, s->x8, s->xsumq, TB, out); break;
    case MIQ_TYPE_Q5_K: hipLaunchKernelGGL(mfma16_dots_kernel<MIQ_TYPE_Q5_K>, grid, dim3(64), 0, stream, w, wb, rb, s->K, s->n_rows, s->x8, s->xsumq, TB, out); break;
    case MIQ_TYPE_Q6_K: hipLaunchKernelGGL(mfma16_dots_kernel<MIQ_TYPE_Q6_K>, grid, dim3(64), 0, stream, w, wb, rb, s->K, s->n_rows, s->x8, s->xsumq, TB, out); break;
    default: hipLaunchKernelGGL(mfma16_dots_kernel<MIQ_TYPE_Q8_0>, grid, dim3(64), 0, stream, w, wb, rb, s->K, s->n_rows, s->x8, s->xsumq, TB, out); break;
    }
    return check_launch("miq_group_dots (mfma)");
}

bool mfma16_fits(const miq_seg *s) { (void)s; return true; }

static M16Args m16_args(const miq_seg *s, int TB) {
    M16Args A;
    A.w = (const uint8_t *)s->w;
    A.row_bytes = (uint32_t)miq_row_bytes(s->type, s->K);
    A.w_bytes = dword_span((size_t)s->n_rows * A.row_bytes);
    A.K = s->K;
    A.n_rows = s->n_rows;
    A.TB = TB;
    A.x8 = s->x8;
    A.xmeta = s->xmeta;
    A.xsumq = s->xsumq;
    A.out = s->out;
    A.out_stride = TB > 1 ? s->out_stride : s->n_rows;
    A.residual = s->residual;
    A.alpha = s->alpha;
    return A;
}

// Whether launch_mfma16 runs this segment on the split-K kernel (the form the
// multi-segment launch shares).
static bool m16z_form(const miq_seg *s, int TB, int n_cu) {
    const int m16_form = sw(kSwM16Form);
    const bool cu_form = TB <= 16 && (m16_form == 3 || (m16_form == 0 && (long)(s->n_rows + 15) / 16 >= 8L * n_cu));
    return !cu_form;
}

int launch_mfma16_multi(hipStream_t stream, const miq_seg *segs, int n_segs, int TB) {
    int n_cu = 0;
    if (const int rc = device_cus(&n_cu)) return rc;
    bool z = n_segs > 1 && n_segs <= kZSegs;
    for (int i = 0; z && i < n_segs; i++) z = mfma16_fits(&segs[i]) && m16z_form(&segs[i], TB, n_cu);
    if (!z) {
        for (int i = 0; i < n_segs; i++)
            if (const int rc = launch_mfma16(stream, &segs[i], TB)) return rc;
        return MIQ_OK;
    }
    M16Args As[kZSegs];
    for (int i = 0; i < n_segs; i++) As[i] = m16_args(&segs[i], TB);
    int rc;
    switch (segs[0].type) {
    case MIQ_TYPE_Q4_K: rc = launch_m16z<MIQ_TYPE_Q4_K>(stream, As, n_segs, TB); break;
    case MIQ_TYPE_Q5_K: rc = launch_m16z<MIQ_TYPE_Q5_K>(stream, As, n_segs, TB); break;
    case MIQ_TYPE_Q6_K: rc = launch_m16z<MIQ_TYPE_Q6_K>(stream, As, n_segs, TB); break;
    default: rc = launch_m16z<MIQ_TYPE_Q8_0>(stream, As, n_segs, TB); break;
    }
    if (rc != MIQ_OK) return rc;
    return check_launch("miq mfma16 (segments)");
}

int launch_mfma16(hipStream_t stream, const miq_seg *s, int TB) {
    const M16Args A = m16_args(s, TB);
    // MIQ_M16_FORM: 0 (default) the CU-resident form for up to 16 tokens when
    // a CU gets at least 8 tiles (its activation staging is then amortized;
    // measured: Q6_K 151936x5120 206 us against 218 us split-K, while at
    // 17408x5120 split-K wins 21 us to 23 us), else split-K; 2 split-K, 3 the
    // CU-resident form wherever it applies
    const int m16_form = sw(kSwM16Form);
    int n_cu = 0;
    if (m16_form == 0 || m16_form == 3) {
        const int rc = device_cus(&n_cu);
        if (rc != MIQ_OK) return rc;
    }
    const bool cu_form = TB <= 16 && (m16_form == 3 || (m16_form == 0 && (long)(A.n_rows + 15) / 16 >= 8L * n_cu));
    int rc;
    if (cu_form) {
        switch (s->type) {
        case MIQ_TYPE_Q4_K: rc = launch_m16c<MIQ_TYPE_Q4_K>(stream, A); break;
        case MIQ_TYPE_Q5_K: rc = launch_m16c<MIQ_TYPE_Q5_K>(stream, A); break;
        case MIQ_TYPE_Q6_K: rc = launch_m16c<MIQ_TYPE_Q6_K>(stream, A); break;
        default: rc = launch_m16c<MIQ_TYPE_Q8_0>(stream, A); break;
        }
    } else {
        switch (s->type) {
        case MIQ_TYPE_Q4_K: rc = launch_m16z<MIQ_TYPE_Q4_K>(stream, &A, 1, TB); break;
        case MIQ_TYPE_Q5_K: rc = launch_m16z<MIQ_TYPE_Q5_K>(stream, &A, 1, TB); break;
        case MIQ_TYPE_Q6_K: rc = launch_m16z<MIQ_TYPE_Q6_K>(stream, &A, 1, TB); break;
        default: rc = launch_m16z<MIQ_TYPE_Q8_0>(stream, &A, 1, TB); break;
        }
    }
    if (rc != MIQ_OK) return rc;
    return check_launch("miq mfma16");
}

}  // namespace miq
