// Chunked-prefill GEMM for Q4_K / Q5_K with the activation scale inside the
// MFMA operand: out[t][n] = alpha * sum_k W[n][k] * act_t[k] (+ residual).
//
// The reference's per-group term (i8.cpp:40-61, 96-121) is
//   sx[t,g] * (d[n] * sc[n,g] * I[t,n,g] - dmin[n] * m[n,g] * xsum[t,g])
// with I the exact int32 dot of the group's codes.  Written per value k of
// group g, the first part is d[n] * (q[n,k]*sc[n,g]) * (x8[t,k]*sx[t,g]):
//   - q*sc is an integer <= 31*63 = 1953: exact in fp16;
//   - x8*sx is a 7-bit integer times an f16 scale (cpu_xq stores sx as an f16
//     value), at most 18 significant bits.  Scaled by a power of two 2^E per
//     (token, 256-value block) it splits into hi = fp16(v) and lo = v - hi,
//     both exact fp16 values (lo needs at most 8 bits; E keeps |v| <= 2^15;
//     exact for every group whose scale is within 2^21 of its block's largest).
// So two fp16 MFMAs per 32 values (hi and lo) accumulate a whole 256-value
// block in fp32 with exact products and no per-group epilogue.  One
// accumulator serves the whole K range: it holds the output in units of
// D[n] * 2^-E[t] of the current block (D = d, or the last nonzero d of the row
// when a block's d is 0, whose codes then enter as 0).  At a block end the
// min term, sum_g (-(dmin/D)*m)[n,g] * (sx*xsum*2^E)[t,g], is added by two
// bf16 MFMAs (both factors split into three bf16 pieces, the six products of
// pieces that reach 2^-24 laid out along K), and the accumulator is rescaled
// to the next block's units (one multiply per output per block); the store
// multiplies by the last block's unit.  The kernel is MFMA-bound by
// construction: the VALU decodes weights (q*sc) once per workgroup and
// rescales once per block.
//
// Pre-pass (pfx_prep_kernel), one thread per (256-value block, token): the
// hi / lo planes [K/32][TB][32] fp16 (group-major like x8), and per (block,
// token) 128 bytes: the bf16 pieces of sx*xsum*2^E' in the six products'
// order (E' the next block's exponent), 2^-E and 2^-E'.
//
// GEMM: a workgroup of 4 waves owns 256 rows x 128 tokens; wave w owns rows
// 128*(w&1).. and tokens 64*(w>>1).. as 8 x 4 tiles of v_mfma_f32_16x16x32_f16
// (A = weights: lane l holds row l%16, k 8*(l/16)..+8; B = activations,
// token l%16; C: lane l holds rows 4*(l/16)+v of token l%16).  K runs in
// stages of one 32-value group through triple-buffered LDS: while the MFMAs
// of stage s run, each wave reads its operands of stage s+1 into registers
// and the workgroup writes stage s+2 (its 256 rows' codes decoded to q*sc, one
// row per thread, and the hi / lo planes), from registers loaded two stages
// (activations) or three (raw weight bytes) ahead.  Tiles are dealt to workgroups stream-K, as in
// the fp16 prefill kernel (miq_pf16.hip).
#include <algorithm>
#include <type_traits>

#include "miq_internal.h"

namespace miq {

namespace {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef __bf16 b8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int kXM = 128;  // tokens per workgroup
constexpr int kXN = 256;  // weight rows per workgroup

// LDS map (bytes).  64-byte rows (W, XH, XL: 32 fp16) store 16-byte chunk c
// of row r at chunk c ^ ((r >> 1) & 3), 128-byte rows (M, U: 64 bf16) at
// c ^ ((r >> 1) & 7).  The first was chosen by measuring SQ_LDS_BANK_CONFLICT
// on gfx950 over every XOR-linear swizzle of the row's low four bits: it is
// conflict-free for the operand reads (16 rows, one chunk each per 16 lanes),
// the decode writes (two threads per row, two chunks each) and the copy
// writes (four threads per row); the second reads conflict-free.
constexpr int kLW = 0;                     // W  [3][256 rows][32] fp16 q*sc
constexpr int kLH = kLW + 3 * kXN * 64;    // XH [3][128 tokens][32] fp16 hi
constexpr int kLL = kLH + 3 * kXM * 64;    // XL [3][128 tokens][32] fp16 lo
constexpr int kLM = kLL + 3 * kXM * 64;    // M  [256 rows][64] bf16 pieces of -(dmin/D)*m (this block)
constexpr int kLU = kLM + kXN * 128;       // U  [128 tokens][64] bf16 pieces of sx*xsum*2^E, 2^-E (this block)
constexpr int kLD = kLU + kXM * 128;       // D [256] (this block's unit), FR [256] = D / next block's D,
                                           // FT [128] = 2^-E / next block's 2^-E, fp32
constexpr int kLBytes = kLD + (2 * kXN + kXM) * 4;

__host__ __device__ constexpr int swz4(int r) { return (r >> 1) & 3; }
__host__ __device__ constexpr int swz8(int r) { return (r >> 1) & 7; }
__device__ __forceinline__ int xswz(int r, int c) { return r * 64 + ((c ^ swz4(r & 15)) << 4); }
__device__ __forceinline__ int wswz(int r, int c) { return r * 128 + ((c ^ swz8(r & 15)) << 4); }

// Order of the bf16 piece products along the min term's K (8 groups each):
// (a0,b0) (a0,b1) (a1,b0) (a0,b2) (a1,b1) (a2,b0), then 16 zero slots; A side
// a = pieces of -(dmin/D')*m (per row), B side b = pieces of sx*xsum*2^E' (per
// token), D' and E' the next block's; B slots 56 and 58 hold 2^-E and 2^-E'
// as fp32 (A is zero there)
constexpr int kPieceA[8] = {0, 0, 1, 0, 1, 2, -1, -1};
constexpr int kPieceB[8] = {0, 1, 0, 2, 1, 0, -1, -1};

struct PxArgs {
    const uint8_t *w;
    uint32_t w_bytes;
    uint32_t row_bytes;
    int K;
    int n_rows;
    int TB;
    const _Float16 *xh;   // [K/32][TB][32]
    const _Float16 *xl;   // [K/32][TB][32]
    const uint16_t *u3;   // [K/256][TB][64]
    float *out;
    int out_stride;
    const float *residual;
    float alpha;
    int vec_out;
    int rounds;           // data-parallel rounds of one tile per workgroup
    int xmap;             // stream-K ranges dealt per XCD
    float *part;          // [2 * workgroups][32][256 threads][4] partial sums (stream-K)
    uint32_t *cnt;        // [tile] arrival counters, zero between launches
};

__device__ __forceinline__ uint16_t bf16_trunc(float f) { return (uint16_t)(__builtin_bit_cast(uint32_t, f) >> 16); }
__device__ __forceinline__ float bf16_val(uint16_t b) { return __builtin_bit_cast(float, (uint32_t)b << 16); }
// three bf16 pieces by truncation, each exact: v == p0 + p1 + p2 for v of <= 24 significant bits
__device__ __forceinline__ void bf16_split3(float v, uint16_t (&p)[3]) {
    p[0] = bf16_trunc(v);
    const float r1 = v - bf16_val(p[0]);
    p[1] = bf16_trunc(r1);
    p[2] = bf16_trunc(r1 - bf16_val(p[1]));
}

// ---------------------------------------------------------------- pre-pass
__global__ __launch_bounds__(256) void pfx_prep_kernel(const int8_t *__restrict__ x8, const float *__restrict__ xmeta,
                                                       const int32_t *__restrict__ xsumq, int TB, int K,
                                                       _Float16 *__restrict__ xh, _Float16 *__restrict__ xl,
                                                       uint16_t *__restrict__ u3) {
    const long e = (long)blockIdx.x * blockDim.x + threadIdx.x;
    const int nb = K / 256;
    if (e >= (long)nb * TB) return;
    const int b = (int)(e / TB), t = (int)(e % TB);
    float sx[8];
    int xs[8];
    float mx = 0.0f, mn = 0.0f;
#pragma unroll
    for (int g = 0; g < 8; g++) {
        const size_t gi = (size_t)(8 * b + g) * TB + t;
        sx[g] = xmeta[gi * 2];
        xs[g] = xsumq[gi * 2] + xsumq[gi * 2 + 1];
        mx = fmaxf(mx, fabsf(sx[g]));
        if (b + 1 < nb) mn = fmaxf(mn, fabsf(xmeta[((size_t)(8 * b + 8 + g) * TB + t) * 2]));
    }
    // 2^E with 127 * mx * 2^E <= 2^15 (mx = f * 2^ex, f in [0.5, 1)); En: the
    // same for the next block (this block's own for the last)
    auto expo = [](float m) {
        int ex = 0;
        (void)frexpf(m, &ex);
        const int E = m > 0.0f ? 8 - ex : 0;
        return E > 100 ? 100 : (E < -100 ? -100 : E);
    };
    const int E = expo(mx), En = b + 1 < nb ? expo(mn) : E;
    const float p = ldexpf(1.0f, E), pn = ldexpf(1.0f, En);
    uint16_t up[8][3];
#pragma unroll
    for (int g = 0; g < 8; g++) {
        const size_t gi = (size_t)(8 * b + g) * TB + t;
        const float s = sx[g] * p;  // exact (a power of two)
        const uint4 *src = reinterpret_cast<const uint4 *>(x8 + gi * 32);
        const uint4 a = src[0], c = src[1];
        const uint32_t wv[8] = {a.x, a.y, a.z, a.w, c.x, c.y, c.z, c.w};
        _Float16 hv[32], lv[32];
#pragma unroll
        for (int k = 0; k < 8; k++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float v = (float)(int)(int8_t)(wv[k] >> (8 * i)) * s;  // <= 18 significant bits: exact
                const _Float16 h = (_Float16)v;
                hv[4 * k + i] = h;
                lv[4 * k + i] = (_Float16)(v - (float)h);  // exact difference, exact in fp16
            }
        uint4 *dh = reinterpret_cast<uint4 *>(xh + gi * 32);
        uint4 *dl = reinterpret_cast<uint4 *>(xl + gi * 32);
#pragma unroll
        for (int q = 0; q < 4; q++) {
            dh[q] = __builtin_bit_cast(uint4, *reinterpret_cast<const h8 *>(hv + 8 * q));
            dl[q] = __builtin_bit_cast(uint4, *reinterpret_cast<const h8 *>(lv + 8 * q));
        }
        bf16_split3(sx[g] * (float)xs[g] * pn, up[g]);  // 11 x 12 significant bits: exact
    }
    uint32_t o[32];
#pragma unroll
    for (int c = 0; c < 8; c++)
#pragma unroll
        for (int q = 0; q < 4; q++)
            o[4 * c + q] = kPieceB[c] < 0 ? 0u
                                          : (uint32_t)up[2 * q][kPieceB[c] < 0 ? 0 : kPieceB[c]] |
                                                ((uint32_t)up[2 * q + 1][kPieceB[c] < 0 ? 0 : kPieceB[c]] << 16);
    o[28] = __builtin_bit_cast(uint32_t, ldexpf(1.0f, -E));   // slot 56: 2^-E
    o[29] = __builtin_bit_cast(uint32_t, ldexpf(1.0f, -En));  // slot 58: the next block's 2^-E
    uint4 *du = reinterpret_cast<uint4 *>(u3 + ((size_t)b * TB + t) * 64);
#pragma unroll
    for (int q = 0; q < 8; q++) du[q] = make_uint4(o[4 * q], o[4 * q + 1], o[4 * q + 2], o[4 * q + 3]);
}

// ---------------------------------------------------------------- GEMM
// bytes k0, k1 of v as two halves 0x64xx = 1024 + byte
__device__ __forceinline__ uint32_t pk_bytes(uint32_t v, int k0, int k1) {
    return __builtin_amdgcn_perm(v, 0x64646464u, (uint32_t)((4 + k0) | ((4 + k1) << 16)));
}

template <uint32_t TYPE> struct PxBlk {  // the raw bytes of one block of one row that stay in registers
    uint4 hdr;
    uint4 qh0, qh1;  // Q5_K: qh[32]
};

template <uint32_t TYPE>
__device__ __forceinline__ void px_load_hdr(PxBlk<TYPE> &B, __amdgpu_buffer_rsrc_t rw, uint32_t boff) {
    B.hdr = bload16(rw, boff);
    if constexpr (TYPE == MIQ_TYPE_Q5_K) {
        B.qh0 = bload16(rw, boff + 16);
        B.qh1 = bload16(rw, boff + 32);
    }
}

// the 32 qs bytes of group pair j (groups 2j, 2j+1)
template <uint32_t TYPE>
__device__ __forceinline__ void px_load_qs(uint4 (&q)[2], __amdgpu_buffer_rsrc_t rw, uint32_t boff, int j) {
    constexpr uint32_t qoff = TYPE == MIQ_TYPE_Q4_K ? 16 : 48;
    q[0] = bload16(rw, boff + qoff + 32 * j);
    q[1] = bload16(rw, boff + qoff + 32 * j + 16);
}

// Group g of row r as q*sc fp16 into the W buffer (its four chunks).
template <uint32_t TYPE>
__device__ __forceinline__ void px_decode(const PxBlk<TYPE> &B, const uint4 (&q4)[2], int g, uint8_t *wbuf, int r,
                                          bool row_ok) {
    const uint32_t q[8] = {q4[0].x, q4[0].y, q4[0].z, q4[0].w, q4[1].x, q4[1].y, q4[1].z, q4[1].w};
    int sc, m;
    scale_min_k4(g, B.hdr.y, B.hdr.z, B.hdr.w, sc, m);
    sc *= (int)(row_ok & ((B.hdr.x & 0x7FFFu) != 0));  // 0 for a row past the tensor, or d == 0
    const h2 sc2 = h2{(_Float16)sc, (_Float16)sc};
    const h2 nsc2 = h2{(_Float16)(-1024 * sc), (_Float16)(-1024 * sc)};
    uint32_t ow[16];
#pragma unroll
    for (int k = 0; k < 8; k++) {
        uint32_t c = (g & 1) ? (q[k] >> 4) & 0x0F0F0F0Fu : q[k] & 0x0F0F0F0Fu;
        if constexpr (TYPE == MIQ_TYPE_Q5_K) {
            const uint32_t hq[8] = {B.qh0.x, B.qh0.y, B.qh0.z, B.qh0.w, B.qh1.x, B.qh1.y, B.qh1.z, B.qh1.w};
            c |= ((hq[k] >> g) & 0x01010101u) << 4;
        }
        // (1024 + code) * sc - 1024 * sc = code * sc, one rounding of an exact value
        ow[2 * k] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(__builtin_bit_cast(h2, pk_bytes(c, 0, 1)), sc2, nsc2));
        ow[2 * k + 1] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(__builtin_bit_cast(h2, pk_bytes(c, 2, 3)), sc2, nsc2));
    }
#pragma unroll
    for (int c = 0; c < 4; c++)
        *reinterpret_cast<uint4 *>(wbuf + xswz(r, c)) = make_uint4(ow[4 * c], ow[4 * c + 1], ow[4 * c + 2], ow[4 * c + 3]);
}

// The block's min-term A row (row r's eight chunks: pieces of -(dmin/D)*m in
// the product order) and its unit D.
template <uint32_t TYPE>
__device__ __forceinline__ void px_block_meta(const PxBlk<TYPE> &B, float D, uint8_t *mbuf, float *dbuf, int r,
                                              bool row_ok) {
    const float f = row_ok ? -h2f(B.hdr.x >> 16) / D : 0.0f;
    uint16_t pc[8][3];
#pragma unroll
    for (int g = 0; g < 8; g++) {
        int sc, m;
        scale_min_k4(g, B.hdr.y, B.hdr.z, B.hdr.w, sc, m);
        bf16_split3(f * (float)m, pc[g]);
    }
#pragma unroll
    for (int c = 0; c < 8; c++) {  // chunk = product c over groups 0..7 (constant indices)
        const int pa = kPieceA[c];
        uint32_t wv[4];
#pragma unroll
        for (int q = 0; q < 4; q++)
            wv[q] = pa < 0 ? 0u : (uint32_t)pc[2 * q][pa < 0 ? 0 : pa] | ((uint32_t)pc[2 * q + 1][pa < 0 ? 0 : pa] << 16);
        *reinterpret_cast<uint4 *>(mbuf + wswz(r, c)) = make_uint4(wv[0], wv[1], wv[2], wv[3]);
    }
    dbuf[r] = D;
}

// a block's unit: its d, or the previous unit when d is 0
__device__ __forceinline__ float px_unit(uint32_t hdr_x, float prev) {
    const float d = h2f(hdr_x);
    return d != 0.0f ? d : prev;
}

// MFMA operands of one stage for one wave: 8 row tiles (A), 4 token tiles hi / lo (B)
struct PxOps {
    h8 a[8], bh[4], bl[4];
};

template <uint32_t TYPE>
__global__ __launch_bounds__(256) void pfx_kernel(PxArgs A) {
    extern __shared__ __align__(16) uint8_t lds[];
    __shared__ int lflag;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wr = wave & 1, wt = wave >> 1;
    const int li = lane & 15, lq = lane >> 4;
    const int mt = (A.TB + kXM - 1) / kXM;
    const int nt = (A.n_rows + kXN - 1) / kXN;
    const int K = A.K, nkb = K / 256, G = K / 32;
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(A.w, A.w_bytes);
    const uint32_t xbytes = (uint32_t)G * A.TB * 64, ubytes = (uint32_t)nkb * A.TB * 128;
    const __amdgpu_buffer_rsrc_t rxh = make_rsrc(A.xh, xbytes), rxl = make_rsrc(A.xl, xbytes);
    const __amdgpu_buffer_rsrc_t ru = make_rsrc(A.u3, ubytes);
    // operand offsets: the swizzle terms depend on li only (tiles are 16 rows)
    const int a_off = xswz(li, lq);
    const int m_off0 = wswz(li, lq);      // 128-byte rows, chunk lq
    const int m_off1 = wswz(li, lq + 4);  // chunk lq + 4
    const int e_off = wswz(li, 7);        // chunk 7: 2^-E, then 2^-E' (+4 bytes)
    // copy role: token ctok, chunks 2*ch, 2*ch+1 of its X rows and 4*ch.. of its U row
    const int ctok = tid >> 1, ch = tid & 1;
    // decode role: row r
    const int r = tid;
    float *Dl = reinterpret_cast<float *>(lds + kLD);  // D, FR, FT
    f4 cb[8][4];

    // Blocks [kb0, kb1) of tile (n0, t0): cb ends holding the tile's outputs.
    auto run = [&](int n0, int t0, int kb0, int kb1) {
        const bool row_ok = n0 + r < A.n_rows;
        const uint32_t wbase = row_ok ? (uint32_t)(n0 + r) * A.row_bytes : A.w_bytes;
        auto boff = [&](int kb) { return kb < kb1 && row_ok ? wbase + (uint32_t)kb * block_bytes(TYPE) : A.w_bytes; };
        // Stage s = group 8*kb0 + s.  Tokens past TB read the next group's data
        // or, past the buffer, zeros: they feed only output columns that are
        // never stored.  So do stages past the range (never decoded).
        const uint32_t xoff0 = ((uint32_t)(8 * kb0) * A.TB + t0 + ctok) * 64 + 32 * ch;
        auto xload = [&](uint4 (&xr)[4], int s) {
            const uint32_t off = xoff0 + (uint32_t)s * A.TB * 64;
            xr[0] = bload16(rxh, off);
            xr[1] = bload16(rxh, off + 16);
            xr[2] = bload16(rxl, off);
            xr[3] = bload16(rxl, off + 16);
        };
        auto xstore = [&](const uint4 (&xr)[4], int buf) {
            uint8_t *h = lds + kLH + buf * kXM * 64, *l = lds + kLL + buf * kXM * 64;
            *reinterpret_cast<uint4 *>(h + xswz(ctok, 2 * ch)) = xr[0];
            *reinterpret_cast<uint4 *>(h + xswz(ctok, 2 * ch + 1)) = xr[1];
            *reinterpret_cast<uint4 *>(l + xswz(ctok, 2 * ch)) = xr[2];
            *reinterpret_cast<uint4 *>(l + xswz(ctok, 2 * ch + 1)) = xr[3];
        };
        const uint32_t uoff0 = (uint32_t)(t0 + ctok) * 128 + 64 * ch;
        auto uload = [&](uint4 (&ur)[4], int kb) {
#pragma unroll
            for (int i = 0; i < 4; i++) ur[i] = bload16(ru, uoff0 + (uint32_t)kb * A.TB * 128 + 16 * i);
        };
        auto ustore = [&](const uint4 (&ur)[4]) {
#pragma unroll
            for (int i = 0; i < 4; i++) *reinterpret_cast<uint4 *>(lds + kLU + wswz(ctok, 4 * ch + i)) = ur[i];
        };
        // this wave's operands of the stage in LDS buffer `buf`
        auto opload = [&](PxOps &o, int buf) {
            const uint8_t *Wl = lds + kLW + buf * kXN * 64 + (128 * wr) * 64 + a_off;
            const uint8_t *Hl = lds + kLH + buf * kXM * 64 + (64 * wt) * 64 + a_off;
            const uint8_t *Ll = lds + kLL + buf * kXM * 64 + (64 * wt) * 64 + a_off;
#pragma unroll
            for (int tt = 0; tt < 4; tt++) {
                o.bh[tt] = *reinterpret_cast<const h8 *>(Hl + tt * 16 * 64);
                o.bl[tt] = *reinterpret_cast<const h8 *>(Ll + tt * 16 * 64);
            }
#pragma unroll
            for (int rt = 0; rt < 8; rt++) o.a[rt] = *reinterpret_cast<const h8 *>(Wl + rt * 16 * 64);
        };

#pragma unroll
        for (int a = 0; a < 8; a++)
#pragma unroll
            for (int b = 0; b < 4; b++) cb[a][b] = f4{0, 0, 0, 0};

        PxBlk<TYPE> bcur, bnxt;
        uint4 qs[2][2];  // group pairs: slot = pair & 1
        uint4 xa[4], xb[4], ur[4];
        PxOps op0, op1;
        float dcur;  // decode role: the unit D of the current block
        __syncthreads();    // the previous segment is done with every LDS buffer
        // prologue: stages 0 and 1 decoded into buffers 0 and 1; stage 2 and 3
        // activations in flight (xa, xb); block kb0's U in flight
        px_load_hdr<TYPE>(bcur, rw, boff(kb0));
        dcur = px_unit(bcur.hdr.x, 1.0f);
        px_load_qs<TYPE>(qs[0], rw, boff(kb0), 0);
        px_load_qs<TYPE>(qs[1], rw, boff(kb0), 1);
        uload(ur, kb0);
        xload(xa, 0);
        xload(xb, 1);
        px_decode<TYPE>(bcur, qs[0], 0, lds + kLW, r, row_ok);
        px_decode<TYPE>(bcur, qs[0], 1, lds + kLW + kXN * 64, r, row_ok);
        px_load_qs<TYPE>(qs[0], rw, boff(kb0), 2);
        xstore(xa, 0);
        xstore(xb, 1);
        xload(xa, 2);
        xload(xb, 3);
        __syncthreads();
        opload(op0, 0);
        int b3 = 0;  // stage s lives in LDS buffer b3 = s % 3

        for (int kb = kb0; kb < kb1; kb++) {
            // one unrolled block: stages s = 8*(kb-kb0) + g
            auto stage = [&](auto g_c) {
                constexpr int g = decltype(g_c)::value;
                const int s = 8 * (kb - kb0) + g;
                const int b1 = b3 == 2 ? 0 : b3 + 1, b2 = b1 == 2 ? 0 : b1 + 1;  // stages s+1, s+2
                PxOps &oc = *((g & 1) ? &op1 : &op0);  // stage s
                PxOps &on = *((g & 1) ? &op0 : &op1);  // stage s+1
                uint4(&xr)[4] = *((g & 1) ? &xb : &xa);  // stage s+2, then s+4
                if constexpr (g == 0) px_load_hdr<TYPE>(bnxt, rw, boff(kb + 1));
                // the next stage's operands (written before the last barrier)
                // (past the range: a stale buffer, never computed on)
                opload(on, b1);
                // ---- MFMAs of stage s: per token tile, the hi MFMAs of the eight row
                // tiles, then the lo ones
#pragma unroll
                for (int tt = 0; tt < 4; tt++) {
#pragma unroll
                    for (int rt = 0; rt < 8; rt++)
                        cb[rt][tt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(oc.a[rt], oc.bh[tt], cb[rt][tt], 0, 0, 0);
#pragma unroll
                    for (int rt = 0; rt < 8; rt++)
                        cb[rt][tt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(oc.a[rt], oc.bl[tt], cb[rt][tt], 0, 0, 0);
                }
                if constexpr (g == 7) {
                    // block end: rescale to the next block's units, then the min term
                    // (in those units) on bf16 MFMA
                    const uint8_t *Ul = lds + kLU + (64 * wt) * 128;
                    const uint8_t *Ml = lds + kLM + (128 * wr) * 128;
                    b8 ua[4], ub[4];
                    float ft[4];
#pragma unroll
                    for (int tt = 0; tt < 4; tt++) {
                        ua[tt] = *reinterpret_cast<const b8 *>(Ul + tt * 16 * 128 + m_off0);
                        ub[tt] = *reinterpret_cast<const b8 *>(Ul + tt * 16 * 128 + m_off1);
                        ft[tt] = Dl[2 * kXN + 64 * wt + 16 * tt + li];
                    }
#pragma unroll
                    for (int rt = 0; rt < 8; rt++) {
                        const f4 fr = *reinterpret_cast<const f4 *>(Dl + kXN + 128 * wr + 16 * rt + 4 * lq);
#pragma unroll
                        for (int tt = 0; tt < 4; tt++) cb[rt][tt] *= fr * ft[tt];
                    }
#pragma unroll
                    for (int rt = 0; rt < 8; rt++) {
                        const b8 ma = *reinterpret_cast<const b8 *>(Ml + rt * 16 * 128 + m_off0);
                        const b8 mb = *reinterpret_cast<const b8 *>(Ml + rt * 16 * 128 + m_off1);
#pragma unroll
                        for (int tt = 0; tt < 4; tt++)
                            cb[rt][tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ma, ua[tt], cb[rt][tt], 0, 0, 0);
#pragma unroll
                        for (int tt = 0; tt < 4; tt++)
                            cb[rt][tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(mb, ub[tt], cb[rt][tt], 0, 0, 0);
                    }
                }
                // ---- stage s+2 into buffer b2: group gn of block kb + (g >= 6)
                // (past the range: zero weights from past the tensor into a buffer
                // whose operands are never computed on)
                {
                    constexpr int gn = (g + 2) & 7;
                    const PxBlk<TYPE> &bd = g >= 6 ? bnxt : bcur;
                    px_decode<TYPE>(bd, qs[(gn >> 1) & 1], gn, lds + kLW + b2 * kXN * 64, r, row_ok);
                    xstore(xr, b2);
                    if constexpr (gn & 1) {  // pair P = gn>>1 decoded: its slot takes pair P + 2
                        constexpr int P = gn >> 1;
                        const int blk = kb + (g >= 6) + (P + 2 > 3);
                        px_load_qs<TYPE>(qs[P & 1], rw, boff(blk), (P + 2) & 3);
                    }
                }
                xload(xr, s + 4);
                // This block's U and the token factors FT = 2^-E / 2^-E' at its first
                // stage, its min-term rows, FR = D / D' and D' mid-block (the
                // previous block's end read them before the last barrier).
                if constexpr (g == 0) {
                    ustore(ur);
                    if (ch == 1) Dl[2 * kXN + ctok] = __builtin_bit_cast(float, ur[3].x) / __builtin_bit_cast(float, ur[3].y);
                }
                if constexpr (g == 2) uload(ur, kb + 1);
                if constexpr (g == 5) {
                    const float dn = px_unit(bnxt.hdr.x, dcur);  // D' (the current unit past the range)
                    px_block_meta<TYPE>(bcur, dn, lds + kLM, Dl, r, row_ok);
                    Dl[kXN + r] = dcur / dn;
                    dcur = dn;
                }
                if constexpr (g == 7) bcur = bnxt;
                b3 = b1;
                __builtin_amdgcn_sched_barrier(0);
                __syncthreads();
            };
            stage(std::integral_constant<int, 0>{});
            stage(std::integral_constant<int, 1>{});
            stage(std::integral_constant<int, 2>{});
            stage(std::integral_constant<int, 3>{});
            stage(std::integral_constant<int, 4>{});
            stage(std::integral_constant<int, 5>{});
            stage(std::integral_constant<int, 6>{});
            stage(std::integral_constant<int, 7>{});
        }
        // to output units: the units after the last block, D' per row and 2^-E' per token
        const uint8_t *Ul = lds + kLU + (64 * wt) * 128;
#pragma unroll
        for (int rt = 0; rt < 8; rt++) {
            const f4 d4 = *reinterpret_cast<const f4 *>(Dl + 128 * wr + 16 * rt + 4 * lq);
#pragma unroll
            for (int tt = 0; tt < 4; tt++)
                cb[rt][tt] *= d4 * *reinterpret_cast<const float *>(Ul + tt * 16 * 128 + e_off + 4);
        }
    };

    auto store = [&](int n0, int t0) {
#pragma unroll
        for (int rt = 0; rt < 8; rt++) {
            const int row = n0 + 128 * wr + 16 * rt + 4 * lq;
#pragma unroll
            for (int tt = 0; tt < 4; tt++) {
                const int t = t0 + 64 * wt + 16 * tt + li;
                if (t >= A.TB) continue;
                const size_t o = (size_t)t * A.out_stride + row;
                if (A.vec_out && row + 3 < A.n_rows) {
                    f4 v = cb[rt][tt] * A.alpha;
                    if (A.residual) v += *reinterpret_cast<const f4 *>(A.residual + o);
                    *reinterpret_cast<f4 *>(A.out + o) = v;
                } else {
#pragma unroll
                    for (int v = 0; v < 4; v++) {
                        if (row + v >= A.n_rows) break;
                        float val = A.alpha * cb[rt][tt][v];
                        if (A.residual) val += A.residual[o + v];
                        A.out[o + v] = val;
                    }
                }
            }
        }
    };

    // Schedule (the fp16 prefill kernel's): `rounds` data-parallel rounds of
    // one tile per workgroup, XCD-major; then every remaining tile's K blocks
    // dealt out as equal contiguous ranges (stream-K), per XCD when `xmap`.
    // A tile covered by one range is stored directly; otherwise each range
    // writes a partial and the last contributor to arrive adds them in range
    // order (deterministic) and stores.
    const int P = gridDim.x, w = blockIdx.x;
    const long T = (long)nt * mt;
    const long F = (long)A.rounds * P, sk = T - F;
    const bool xmap = A.xmap;
    const int NG = xmap ? 8 : 1, x = xmap ? w % 8 : 0, Pg = P / NG, vl = xmap ? w / 8 : w;
    const long tx0 = F + x * sk / NG, tx1 = F + (x + 1) * sk / NG;
    const long base = tx0 * nkb, total = sk > 0 ? (tx1 - tx0) * nkb : 0;
    auto rstart = [&](int u) { return base + u * total / Pg; };
    auto owner = [&](long blk) { return (int)(((blk - base + 1) * Pg + total - 1) / total) - 1; };
    const long bs = total > 0 ? rstart(vl) : 0, be = total > 0 ? rstart(vl + 1) : 0;
    const int v = x * Pg + vl;
    constexpr uint32_t kFar = 1u << 20;
    int k = 0;
    long b0 = bs;
    for (;;) {
        long t;
        int kb0, kb1;
        bool dp;
        if (k < A.rounds) {
            dp = true;
            t = (long)k * P + (w % 8) * (P / 8) + w / 8;
            k++;
            if (t >= T) continue;
            kb0 = 0;
            kb1 = nkb;
        } else if (b0 < be) {
            dp = false;
            t = b0 / nkb;
            const long tb1 = (t + 1) * nkb;
            kb0 = (int)(b0 - t * nkb);
            kb1 = (int)((be < tb1 ? be : tb1) - t * nkb);
        } else {
            break;
        }
        const int n0 = (int)(t % nt) * kXN, t0 = (int)(t / nt) * kXM;
        run(n0, t0, kb0, kb1);
        if (dp) {
            store(n0, t0);
            continue;
        }
        const bool head = b0 == bs;
        b0 = t * nkb + kb1;
        if (kb0 == 0 && kb1 == nkb) {
            store(n0, t0);
            continue;
        }
        const long tb0 = t * nkb, tb1 = tb0 + nkb;
        const int slot = 2 * v + (head ? 0 : 1);
        f4 *mine = reinterpret_cast<f4 *>(A.part) + (size_t)slot * 32 * 256;
#pragma unroll
        for (int a = 0; a < 8; a++)
#pragma unroll
            for (int c = 0; c < 4; c++) mine[(4 * a + c) * 256 + tid] = cb[a][c];
        const int v_lo = owner(tb0), v_hi = owner(tb1 - 1);
        int n_contrib = 0;
        for (int u = v_lo; u <= v_hi; u++) n_contrib += rstart(u) < rstart(u + 1);
        const bool far = !xmap || (__builtin_amdgcn_s_getreg((3 << 11) | (0 << 6) | 20) & 15) != (uint32_t)x;  // HW_REG_XCC_ID
        if (far) __threadfence();
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (tid == 0) {
            const uint32_t prev = __hip_atomic_fetch_add(A.cnt + t, far ? 1u + kFar : 1u, __ATOMIC_RELAXED,
                                                         __HIP_MEMORY_SCOPE_AGENT);
            const int last = (prev & (kFar - 1)) == (uint32_t)(n_contrib - 1);
            if (last) __hip_atomic_store(A.cnt + t, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            lflag = last ? 1 + (prev >= kFar) : 0;
        }
        __syncthreads();
        const int fl = lflag;
        if (!fl) continue;
        if (fl == 2 || far) __threadfence();
#pragma unroll
        for (int a = 0; a < 8; a++)
#pragma unroll
            for (int c = 0; c < 4; c++) cb[a][c] = f4{0, 0, 0, 0};
        for (int u = v_lo; u <= v_hi; u++) {
            const long us = rstart(u);
            if (us == rstart(u + 1)) continue;
            const int sl = 2 * (x * Pg + u) + (us >= tb0 ? 0 : 1);
            const __amdgpu_buffer_rsrc_t rp = make_rsrc(A.part + (size_t)sl * 32 * 256 * 4, 32 * 256 * 16);
#pragma unroll
            for (int a = 0; a < 8; a++)
#pragma unroll
                for (int c = 0; c < 4; c++)
                    cb[a][c] += __builtin_bit_cast(
                        f4, __builtin_amdgcn_raw_buffer_load_b128(rp, ((uint32_t)(4 * a + c) * 256 + tid) * 16, 0, 1));
        }
        store(n0, t0);
    }
}

size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

}  // namespace

bool pfx_serves(const miq_seg *s) { return s->type == MIQ_TYPE_Q4_K || s->type == MIQ_TYPE_Q5_K; }

int launch_pfx(hipStream_t stream, const miq_seg *s, int TB) {
    const int K = s->K;
    const size_t x_bytes = (size_t)TB * K * 2, u_bytes = (size_t)(K / 256) * TB * 128;
    if (x_bytes >= 0xFFFFFFF0u || (size_t)s->n_rows * miq_row_bytes(s->type, K) >= 0xFFFFF000u) {
        set_error("miq prefill: %d x %d activation or the weight tensor exceeds the 4 GiB buffer window", TB, K);
        return MIQ_UNSUPPORTED;
    }
    int n_cu = 0;
    if (int rc = device_cus(&n_cu)) return rc;
    const int mt = (TB + kXM - 1) / kXM;
    const int nt = (s->n_rows + kXN - 1) / kXN;
    const long T = (long)nt * mt, nkb = K / 256;
    // one resident workgroup per CU; data-parallel rounds while a round fills at
    // least half the workgroups, else every tile through stream-K
    long P = n_cu - n_cu % 8;
    if (P < 8) P = n_cu;
    long rounds = T / P, sk = T % P;
    if (sk * 2 >= P) {
        rounds += 1;
        sk = 0;
    } else if (sk > 0) {
        rounds = 0;
        sk = T;
    }
    if (rounds == 0 && sk * nkb < P) P = sk * nkb >= 8 ? sk * nkb / 8 * 8 : sk * nkb;
    const size_t part_bytes = (size_t)2 * P * 32 * 256 * 16;
    const size_t ws_bytes = 2 * align_up(x_bytes, 256) + align_up(u_bytes, 256) + part_bytes;
    void *ws = nullptr;
    if (int rc = workspace_get(stream, kWsPrefill, ws_bytes, &ws)) return rc;
    void *cw = nullptr;
    if (int rc = workspace_get(stream, kWsPrefillCnt, (size_t)T * 4, &cw, true)) return rc;
    uint8_t *p = reinterpret_cast<uint8_t *>(ws);
    PxArgs A;
    A.xh = reinterpret_cast<const _Float16 *>(p);
    A.xl = reinterpret_cast<const _Float16 *>(p + align_up(x_bytes, 256));
    A.u3 = reinterpret_cast<const uint16_t *>(p + 2 * align_up(x_bytes, 256));
    A.part = reinterpret_cast<float *>(p + 2 * align_up(x_bytes, 256) + align_up(u_bytes, 256));
    A.cnt = reinterpret_cast<uint32_t *>(cw);
    const long n = (long)(K / 256) * TB;
    hipLaunchKernelGGL(pfx_prep_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, s->x8, s->xmeta,
                       s->xsumq, TB, K, const_cast<_Float16 *>(A.xh), const_cast<_Float16 *>(A.xl),
                       const_cast<uint16_t *>(A.u3));
    A.w = (const uint8_t *)s->w;
    A.row_bytes = (uint32_t)miq_row_bytes(s->type, K);
    A.w_bytes = dword_span((size_t)s->n_rows * A.row_bytes);
    A.K = K;
    A.n_rows = s->n_rows;
    A.TB = TB;
    A.out = s->out;
    A.out_stride = s->out_stride;
    A.residual = s->residual;
    A.alpha = s->alpha;
    A.vec_out = ((uintptr_t)s->out % 16 == 0) && (s->out_stride % 4 == 0) &&
                (!s->residual || (uintptr_t)s->residual % 16 == 0);
    A.rounds = (int)rounds;
    A.xmap = sk >= 8 && P % 8 == 0;
    static bool lds_set[64] = {false};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
        set_error("miq prefill: no current device");
        return MIQ_EHIP;
    }
    if (!lds_set[dev]) {
        if (hipFuncSetAttribute((const void *)pfx_kernel<MIQ_TYPE_Q4_K>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                kLBytes) != hipSuccess ||
            hipFuncSetAttribute((const void *)pfx_kernel<MIQ_TYPE_Q5_K>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                kLBytes) != hipSuccess) {
            set_error("miq prefill: cannot raise the LDS limit to %d bytes", kLBytes);
            return MIQ_EHIP;
        }
        lds_set[dev] = true;
    }
    if (s->type == MIQ_TYPE_Q4_K) hipLaunchKernelGGL(pfx_kernel<MIQ_TYPE_Q4_K>, dim3((unsigned)P), dim3(256), kLBytes, stream, A);
    else hipLaunchKernelGGL(pfx_kernel<MIQ_TYPE_Q5_K>, dim3((unsigned)P), dim3(256), kLBytes, stream, A);
    return check_launch("miq prefill");
}

}  // namespace miq
