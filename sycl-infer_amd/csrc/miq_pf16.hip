// Chunked-prefill GEMM for Q4_K / Q5_K on fp16 MFMA with exact integer
// arithmetic: out[t][n] = alpha * sum_k W[n][k] * act_t[k] (+ residual).
//
// Why fp16 and still exact.  Per 32-value group g the reference forms the
// int32 dot I = sum q*x8 and adds sx*(d*sc*I - dmin*m*xsum) (i8.cpp:40-61,
// 96-121).  Here the weight operand is q*sc (an integer <= 31*63 = 1953, exact
// in fp16) and the activation operand is x8 (exact in fp16); every product is
// exact in fp32 and every partial sum of a group is an integer below 2^24, so
// one v_mfma_f32_16x16x32_f16 (K = 32 = one group) returns sc*I exactly.  The
// epilogue is then one fp32 fma per output and group (acc_b += sx*C), the
// block's d and dmin are applied once per 256 values (acc += d*acc_b -
// dmin*T), and T = sum_g m_g * (sx*xsum)_g runs on bf16 MFMA with sx*xsum
// split into three bf16 terms (24 significant bits) against the exact m.
// Int8 MFMA would need cvt + mul + fma per output and group instead.
//
// Structure.  A pre-pass (pf_prep_kernel) converts the quantized activation
// to a token-major fp16 copy, per-(group, token) scales and the bf16 split of
// sx*xsum, all in a per-device workspace.  The GEMM workgroup owns 128 rows x
// 128 tokens (4 waves, 64 x 64 each = 4 x 4 MFMA tiles) and walks K in stages
// of 64 values: the activation of the next stage streams straight into LDS
// (buffer loads with the lds bit, double-buffered) while the current one is
// computed; the raw weight bytes of the next stage are held in registers and
// decoded to q*sc fp16 in LDS at the top of the stage.
//
// MFMA layout (16x16x32): A = weight rows x 32 K, B = 32 K x tokens; lane l
// holds C[rows 4*(l/16) + v][token l%16], so a lane's token scale is one value
// per tile and its four rows are consecutive (one 16-byte store per tile).
#include <algorithm>
#include <cstdlib>
#include <type_traits>

#include "miq_internal.h"
#include "miq_units.h"

namespace miq {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef __bf16 b8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void *lds_ptr;

constexpr int kPM = 128;  // tokens per workgroup
constexpr int kPN = 128;  // weight rows per workgroup
constexpr int kPK = 64;   // K values per stage (two 32-value groups; four stages per block)

// LDS map (bytes), about 75 KiB so two workgroups share a CU
constexpr int kLW = 0;                        // W  [128 rows][64 K] fp16, swizzled 16-byte chunks
constexpr int kLX = kLW + kPN * kPK * 2;      // X  2 x [128 tokens][64 K] fp16, swizzled
constexpr int kLS = kLX + 2 * kPM * kPK * 2;  // SX 2 x [8 groups][2][16][4] fp32 (token = 64*w + 16*tt + j)
constexpr int kLU = kLS + 2 * 8 * kPM * 4;    // U  2 x [128 tokens][32] bf16 (hi, mid, lo of sx*xsum; 8 zero)
constexpr int kLM = kLU + 2 * kPM * 64;       // M  [128 rows][8] bf16 (the block's m per group)
constexpr int kLD = kLM + kPN * 16;           // D, DMIN [128] fp32 each
constexpr int kLBytes = kLD + 2 * kPN * 4;
// Q6_K: W as two planes (hi at kLW, lo after it), no U / M / DMIN
constexpr int kLWLo = kLW + kPN * kPK * 2;
template <uint32_t TYPE> constexpr int lds_x() { return TYPE == MIQ_TYPE_Q6_K ? kLWLo + kPN * kPK * 2 : kLX; }
template <uint32_t TYPE> constexpr int lds_s() { return lds_x<TYPE>() + 2 * kPM * kPK * 2; }
template <uint32_t TYPE> constexpr int lds_d() { return TYPE == MIQ_TYPE_Q6_K ? lds_s<TYPE>() + 2 * 8 * kPM * 4 : kLD; }
static_assert(lds_d<MIQ_TYPE_Q6_K>() + kPN * 4 <= kLBytes, "Q6_K LDS map fits the common size");

// 16-byte chunk c (0..7) of LDS row r: rows are 128 bytes, chunks XOR-swizzled
// so the 16 consecutive rows an operand read touches hit distinct banks
__device__ __forceinline__ int pswz(int r, int c) { return r * 128 + ((c ^ ((r >> 1) & 7)) << 4); }

struct PfArgs {
    const uint8_t *w;
    uint32_t w_bytes;
    uint32_t row_bytes;
    int K;
    int n_rows;
    int TB;
    const _Float16 *x16;  // [TB][K]
    const float *sx;      // [K/32][TB]
    const __bf16 *u3;     // [K/256][TB][32]
    float *out;
    int out_stride;
    const float *residual;
    float alpha;
    int vec_out;          // out / residual allow 16-byte row stores
    int rounds;           // data-parallel rounds of one tile per workgroup
    int xmap;             // stream-K ranges are dealt to the 8 XCDs
    float *part;          // [2 * workgroups][256 threads][64] partial sums (stream-K)
    uint32_t *cnt;        // [tile] arrival counters, zero between launches
    int32_t *dots;        // parity form: [TB][n_rows][K/32] MFMA group results
};

// ---------------------------------------------------------------- pre-pass
// Eight lanes per (256-value block, token), lane l taking group 8b + l:
// x8 -> fp16 (token-major), sx, and the three-term bf16 split of
// u = sx * (s0 + s1).  The eight lanes of a (block, token) write its 512
// fp16 bytes and its 64-byte u3 record as whole runs; consecutive (block,
// token) items are consecutive tokens, so the x8 reads are runs too.
__device__ __forceinline__ uint16_t bf16_trunc(float f) { return (uint16_t)(__builtin_bit_cast(uint32_t, f) >> 16); }
__device__ __forceinline__ float bf16_val(uint16_t b) { return __builtin_bit_cast(float, (uint32_t)b << 16); }

__global__ __launch_bounds__(256) void pf_prep_kernel(const int8_t *x8, const float *xmeta, const int32_t *xsumq, int TB,
                                                      int K, _Float16 *x16, float *sx, uint16_t *u3) {
    const int nb = K / 256;
    const long e8 = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (e8 >= (long)nb * TB * 8) return;
    const int l = (int)(e8 & 7);
    const long bt = e8 >> 3;
    const int b = (int)(bt / TB), t = (int)(bt % TB);
    const int g = 8 * b + l;
    const size_t gi = (size_t)g * TB + t;
    const uint4 *src = reinterpret_cast<const uint4 *>(x8 + gi * 32);
    const uint4 a = src[0], c = src[1];
    const uint32_t w[8] = {a.x, a.y, a.z, a.w, c.x, c.y, c.z, c.w};
    _Float16 hv[32];
#pragma unroll
    for (int k = 0; k < 8; k++)
#pragma unroll
        for (int i = 0; i < 4; i++) hv[4 * k + i] = (_Float16)(int)(int8_t)(w[k] >> (8 * i));
    uint4 *dst = reinterpret_cast<uint4 *>(x16 + (size_t)t * K + g * 32);
#pragma unroll
    for (int q = 0; q < 4; q++) dst[q] = __builtin_bit_cast(uint4, *reinterpret_cast<const h8 *>(hv + 8 * q));
    const float sv = xmeta[gi * 2];
    sx[gi] = sv;
    const float u = sv * (float)(xsumq[gi * 2] + xsumq[gi * 2 + 1]);
    const uint16_t hi = bf16_trunc(u);
    const float r1 = u - bf16_val(hi);
    const uint16_t mid = bf16_trunc(r1);
    const uint16_t lo = bf16_trunc(r1 - bf16_val(mid));
    uint16_t *ub = u3 + ((size_t)b * TB + t) * 32;
    ub[l] = hi;
    ub[8 + l] = mid;
    ub[16 + l] = lo;
    ub[24 + l] = 0;
}

// ---------------------------------------------------------------- GEMM
// Raw weight bytes of one stage for thread (row r = tid/2, nibble half hh =
// tid&1): the block header and the 32 qs bytes holding groups 2kq (low
// nibbles) and 2kq+1 (high nibbles), plus qh for Q5_K.  Thread hh decodes
// group 2kq + hh.
template <uint32_t TYPE> struct PfRaw {
    uint4 hdr, q0, q1;
    uint4 h0, h1;  // Q5_K qh[32]
};

// Q6_K: thread (r, hh) decodes group g = 2kq + hh = plane p = g & 3 of the
// 128-value half blk2 = g >> 2: 32 ql bytes at blk2*64 + (p&1)*32, the 32 qh
// bytes at 128 + blk2*32, scales[2g], scales[2g+1] and d.  Blocks are 210
// bytes (2-byte aligned): each 32-byte run is loaded as the dword-aligned
// 32 bytes plus the dword after them and realigned by the shift sh.
template <> struct PfRaw<MIQ_TYPE_Q6_K> {
    uint4 l0, l1, h0, h1;
    uint32_t le, he, sc, dd, sh;
};

template <uint32_t TYPE>
__device__ __forceinline__ void pf_wload(PfRaw<TYPE> &R, __amdgpu_buffer_rsrc_t rw, uint32_t boff, int j) {
    if constexpr (TYPE == MIQ_TYPE_Q6_K) {
        const int g = 2 * j + (threadIdx.x & 1), blk2 = g >> 2, p = g & 3;
        const uint32_t lo = boff + blk2 * 64 + (p & 1) * 32, ho = boff + 128 + blk2 * 32;
        R.sh = boff & 3u;
        R.l0 = bload16(rw, lo & ~3u);
        R.l1 = bload16(rw, (lo & ~3u) + 16);
        R.le = bload4(rw, (lo & ~3u) + 32);
        R.h0 = bload16(rw, ho & ~3u);
        R.h1 = bload16(rw, (ho & ~3u) + 16);
        R.he = bload4(rw, (ho & ~3u) + 32);
        R.sc = bload4(rw, (boff + 192 + 2 * g) & ~3u);  // the two scale bytes never straddle a dword
        R.dd = bload4(rw, (boff + 208) & ~3u);
        return;
    } else {
    R.hdr = bload16(rw, boff);
    constexpr uint32_t qoff = TYPE == MIQ_TYPE_Q4_K ? 16 : 48;
    R.q0 = bload16(rw, boff + qoff + 32 * j);
    R.q1 = bload16(rw, boff + qoff + 32 * j + 16);
    if constexpr (TYPE == MIQ_TYPE_Q5_K) {
        R.h0 = bload16(rw, boff + 16);
        R.h1 = bload16(rw, boff + 32);
    }
    }
}

// bytes k0, k1 of v as two halves 0x64xx = 1024 + byte
__device__ __forceinline__ uint32_t pk_bytes(uint32_t v, int k0, int k1) {
    return __builtin_amdgcn_perm(v, 0x64646464u, (uint32_t)((4 + k0) | ((4 + k1) << 16)));
}

// Q6_K group g = 2kq + hh of row r: the signed codes v = code - 32 of its two
// 16-value sub-groups with scales sc0, sc1 as two fp16 planes whose sum is
// v * sc exactly: sc = 2*s2 + s1 (s1 = sc & 1), hi = v * 2*s2 (|v*s2| <= 2048,
// so hi is an exact fp16), lo = s1 ? v : 0.  d into D at block starts.
__device__ __forceinline__ void pf_wdecode_q6k(const PfRaw<MIQ_TYPE_Q6_K> &R, uint8_t *lds, int r, int hh, int kq,
                                               bool row_ok) {
    const int g = 2 * kq + hh, p = g & 3;
    const uint32_t sh = R.sh;
    const uint32_t lw[9] = {R.l0.x, R.l0.y, R.l0.z, R.l0.w, R.l1.x, R.l1.y, R.l1.z, R.l1.w, R.le};
    const uint32_t hw[9] = {R.h0.x, R.h0.y, R.h0.z, R.h0.w, R.h1.x, R.h1.y, R.h1.z, R.h1.w, R.he};
    // the scale bytes sit at byte (sh + 2g) & 3 of R.sc: 0 or 2
    const uint32_t scw = R.sc >> (8 * ((sh + 2 * g) & 3u));
    const int sc[2] = {row_ok ? (int)(int8_t)(scw & 0xFF) : 0, row_ok ? (int)(int8_t)((scw >> 8) & 0xFF) : 0};
    const h2 bias = h2{(_Float16)-1056, (_Float16)-1056};  // 1024 + code - 1056 = code - 32
    uint32_t hiw[16], low[16];
#pragma unroll
    for (int k = 0; k < 8; k++) {
        const uint32_t l = __builtin_amdgcn_alignbyte(lw[k + 1], lw[k], sh);
        const uint32_t h = __builtin_amdgcn_alignbyte(hw[k + 1], hw[k], sh);
        const uint32_t c = ((p >= 2 ? (l >> 4) : l) & 0x0F0F0F0Fu) | (((h >> (2 * p)) & 0x03030303u) << 4);
        const int s = sc[k >> 2];
        const h2 m2 = h2{(_Float16)(s & ~1), (_Float16)(s & ~1)};
        const bool odd = s & 1;
        const h2 a = __builtin_bit_cast(h2, pk_bytes(c, 0, 1)) + bias;
        const h2 b = __builtin_bit_cast(h2, pk_bytes(c, 2, 3)) + bias;
        hiw[2 * k] = __builtin_bit_cast(uint32_t, a * m2);
        hiw[2 * k + 1] = __builtin_bit_cast(uint32_t, b * m2);
        low[2 * k] = odd ? __builtin_bit_cast(uint32_t, a) : 0u;
        low[2 * k + 1] = odd ? __builtin_bit_cast(uint32_t, b) : 0u;
    }
#pragma unroll
    for (int c = 0; c < 4; c++) {
        *reinterpret_cast<uint4 *>(lds + kLW + pswz(r, 4 * hh + c)) = make_uint4(hiw[4 * c], hiw[4 * c + 1], hiw[4 * c + 2], hiw[4 * c + 3]);
        *reinterpret_cast<uint4 *>(lds + kLWLo + pswz(r, 4 * hh + c)) = make_uint4(low[4 * c], low[4 * c + 1], low[4 * c + 2], low[4 * c + 3]);
    }
    if (kq == 0 && hh == 0) {
        const uint32_t dsh = (sh + 208) & 3u;  // 0 or 2
        reinterpret_cast<float *>(lds + lds_d<MIQ_TYPE_Q6_K>())[r] = row_ok ? h2f((R.dd >> (8 * dsh)) & 0xFFFFu) : 0.0f;
    }
}

// Group g = 2kq + hh of row r as q*sc fp16 into W (chunks 4hh..4hh+3), its m
// into M, and (block start) d / dmin into D.
template <uint32_t TYPE>
__device__ __forceinline__ void pf_wdecode(const PfRaw<TYPE> &R, uint8_t *lds, int r, int hh, int kq, bool row_ok) {
    if constexpr (TYPE == MIQ_TYPE_Q6_K) {
        pf_wdecode_q6k(R, lds, r, hh, kq, row_ok);
        return;
    } else {
    const uint32_t q[8] = {R.q0.x, R.q0.y, R.q0.z, R.q0.w, R.q1.x, R.q1.y, R.q1.z, R.q1.w};
    const int g = 2 * kq + hh;
    int sc, m;
    scale_min_k4(g, R.hdr.y, R.hdr.z, R.hdr.w, sc, m);
    if (!row_ok) sc = m = 0;
    const h2 sc2 = h2{(_Float16)sc, (_Float16)sc};
    const h2 nsc2 = h2{(_Float16)(-1024 * sc), (_Float16)(-1024 * sc)};
    uint32_t outw[16];
#pragma unroll
    for (int k = 0; k < 8; k++) {
        uint32_t c = hh ? (q[k] >> 4) & 0x0F0F0F0Fu : q[k] & 0x0F0F0F0Fu;
        if constexpr (TYPE == MIQ_TYPE_Q5_K) {
            const uint32_t hq[8] = {R.h0.x, R.h0.y, R.h0.z, R.h0.w, R.h1.x, R.h1.y, R.h1.z, R.h1.w};
            c |= ((hq[k] >> g) & 0x01010101u) << 4;
        }
        // (1024 + code) * sc - 1024 * sc = code * sc: one rounding of an exact value
        const h2 a = __builtin_bit_cast(h2, pk_bytes(c, 0, 1));
        const h2 b = __builtin_bit_cast(h2, pk_bytes(c, 2, 3));
        outw[2 * k] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(a, sc2, nsc2));
        outw[2 * k + 1] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(b, sc2, nsc2));
    }
#pragma unroll
    for (int c = 0; c < 4; c++)
        *reinterpret_cast<uint4 *>(lds + kLW + pswz(r, 4 * hh + c)) =
            make_uint4(outw[4 * c], outw[4 * c + 1], outw[4 * c + 2], outw[4 * c + 3]);
    reinterpret_cast<uint16_t *>(lds + kLM + r * 16)[g] = bf16_trunc((float)m);
    if (kq == 0 && hh == 0) {
        reinterpret_cast<float *>(lds + kLD)[r] = row_ok ? h2f(R.hdr.x) : 0.0f;
        reinterpret_cast<float *>(lds + kLD)[kPN + r] = row_ok ? h2f(R.hdr.x >> 16) : 0.0f;
    }
    }
}

// DOTS: the parity form -- every group's MFMA result (sc * I, exact in fp32)
// goes to A.dots instead of the epilogue; one tile per workgroup
template <uint32_t TYPE, bool DOTS = false>
__global__ __launch_bounds__(256, 2) void pf16_kernel(PfArgs A) {
    extern __shared__ __align__(16) uint8_t lds[];
    __shared__ int lflag;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wr = wave & 1, wt = wave >> 1;  // wave's 64-row / 64-token quarter
    const int li = lane & 15, lq = lane >> 4;
    // LDS byte offsets of this lane's operand chunks, group gl of a stage
    // (pswz with row 64*w + 16*tile + li: the swizzle term (row >> 1) & 7 is
    // (li >> 1) & 7 for every tile, so tile t adds t * 2048)
    const int aoff[2] = {pswz(64 * wr + li, lq), pswz(64 * wr + li, 4 + lq)};
    const int boff[2] = {pswz(64 * wt + li, lq), pswz(64 * wt + li, 4 + lq)};
    const int mt = (A.TB + kPM - 1) / kPM;
    const int nt = (A.n_rows + kPN - 1) / kPN;
    const int K = A.K, nkb = K / 256;

    const __amdgpu_buffer_rsrc_t rw = make_rsrc(A.w, A.w_bytes);
    const uint32_t xb = (uint32_t)A.TB * K * 2, sb = (uint32_t)(K / 32) * A.TB * 4, ub = (uint32_t)nkb * A.TB * 64;
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(A.x16, xb);
    const __amdgpu_buffer_rsrc_t rsx = make_rsrc(A.sx, sb);
    const __amdgpu_buffer_rsrc_t ru = make_rsrc(A.u3, ub);
    const int xr0 = wave * 32 + (lane >> 3), xc = lane & 7;
    const int wrow = tid >> 1, whh = tid & 1;
    f4 acc[4][4], ab[4][4];

    // Blocks [kb0, kb1) of tile (n0, t0) into acc.
    auto run = [&](int n0, int t0, int kb0, int kb1) {
        // Activation of stage s into X buffer s & 1 (and, on block starts, SX / U
        // of the block).  X: LDS chunk p = 64*(4*wave + i) + lane holds token r =
        // p/8 at swizzled chunk p%8; SX: dword [g][w][j][tt]; U: 16-byte chunk
        // [token][4].  A token past TB reads past the X buffer (zeros); its SX / U
        // entries feed only outputs that are never stored.
        auto stage_act = [&](int s) {
            const int kb = s >> 2, bb = kb & 1;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int r = xr0 + 8 * i;
                const uint32_t off = (uint32_t)(t0 + r) * K * 2 + (uint32_t)s * kPK * 2 + ((xc ^ ((r >> 1) & 7)) << 4);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (lds_ptr)(lds + lds_x<TYPE>() + (s & 1) * kPM * kPK * 2 + (wave * 4 + i) * 1024),
                                                         16, off, 0, 0, 0);
            }
            if (!(s & 3)) {
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int p = (wave * 4 + i) * 64 + lane;
                    const int g = p >> 7, rem = p & 127;
                    const int t = t0 + (rem >> 6) * 64 + (rem & 3) * 16 + ((rem >> 2) & 15);
                    const uint32_t off = ((uint32_t)(kb * 8 + g) * A.TB + t) * 4;
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsx, (lds_ptr)(lds + lds_s<TYPE>() + bb * 4096 + (wave * 4 + i) * 256), 4,
                                                             off, 0, 0, 0);
                }
                if constexpr (TYPE != MIQ_TYPE_Q6_K)  // Q6_K has no dmin term
#pragma unroll
                for (int i = 0; i < 2; i++) {
                    const int p = (wave * 2 + i) * 64 + lane;
                    const uint32_t off = ((uint32_t)kb * A.TB + t0 + (p >> 2)) * 64 + (p & 3) * 16;
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(ru, (lds_ptr)(lds + kLU + bb * 8192 + (wave * 2 + i) * 1024), 16,
                                                             off, 0, 0, 0);
                }
            }
        };
        const bool wrow_ok = n0 + wrow < A.n_rows;
        const uint32_t wbase = wrow_ok ? (uint32_t)(n0 + wrow) * A.row_bytes : A.w_bytes;
        const int s0 = 4 * kb0, s1 = 4 * kb1;
        auto wload = [&](PfRaw<TYPE> &R, int s) {
            const uint32_t boff = s < s1 && wrow_ok ? wbase + (uint32_t)(s >> 2) * block_bytes(TYPE) : A.w_bytes;
            pf_wload<TYPE>(R, rw, boff, s & 3);
        };
#pragma unroll
        for (int a = 0; a < 4; a++)
#pragma unroll
            for (int b = 0; b < 4; b++) {
                acc[a][b] = f4{0, 0, 0, 0};
                ab[a][b] = f4{0, 0, 0, 0};
            }
        PfRaw<TYPE> R;
        __syncthreads();  // the previous range is done with every LDS buffer
        stage_act(s0);
        wload(R, s0);
        for (int s = s0; s < s1; s++) {
            const int kq = s & 3, bb = (s >> 2) & 1;
            // Order within a stage: the barrier (its fence waits for this
            // wave's stage-s activation DMA, issued one stage back), the decode
            // (it waits for R, loaded right after that DMA), a barrier, then
            // the next stage's activation DMA and weight loads, then the MFMAs.
            // Issued before the decode, the DMA made the decode's and the
            // second barrier's waits include it at every stage; issued here, a
            // whole MFMA phase covers its latency.
            __syncthreads();  // stage s-1 is done with W, X[(s+1)&1] and (block end) M / D / U / SX
            pf_wdecode<TYPE>(R, lds, wrow, whh, kq, wrow_ok);
            __syncthreads();  // W of stage s is written
            if (s + 1 < s1) stage_act(s + 1);
            wload(R, s + 1);

            const uint8_t *Wl = lds + kLW + aoff[0];
            const uint8_t *Xl = lds + lds_x<TYPE>() + (s & 1) * kPM * kPK * 2 + boff[0];
            const float *SX = reinterpret_cast<const float *>(lds + lds_s<TYPE>() + bb * 4096);
            // group gl of the stage; the first group of a block starts ab (no
            // separate clear at the block end)
            auto group = [&](auto gl_c, auto first_c) {
                constexpr int gl = decltype(gl_c)::value;
                constexpr bool first = decltype(first_c)::value;
                const int g = 2 * kq + gl;
                h8 av[4], bv[4];
#pragma unroll
                for (int rt = 0; rt < 4; rt++)
                    av[rt] = *reinterpret_cast<const h8 *>(Wl + (aoff[gl] - aoff[0]) + rt * 2048);
#pragma unroll
                for (int tt = 0; tt < 4; tt++)
                    bv[tt] = *reinterpret_cast<const h8 *>(Xl + (boff[gl] - boff[0]) + tt * 2048);
                const f4 sxv = *reinterpret_cast<const f4 *>(SX + g * 128 + wt * 64 + li * 4);
                // 16 tiles; each MFMA is issued two tiles ahead of its epilogue so
                // its latency hides behind the previous tiles' fmas
                // Q6_K: the lo plane's MFMA accumulates onto the hi plane's
                h8 al[TYPE == MIQ_TYPE_Q6_K ? 4 : 1];
                if constexpr (TYPE == MIQ_TYPE_Q6_K)
#pragma unroll
                    for (int rt = 0; rt < 4; rt++)
                        al[rt] = *reinterpret_cast<const h8 *>(Wl + (kLWLo - kLW) + (aoff[gl] - aoff[0]) + rt * 2048);
                auto mm = [&](int q) {
                    const f4 h = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[q >> 2], bv[q & 3], f4{0, 0, 0, 0}, 0, 0, 0);
                    if constexpr (TYPE == MIQ_TYPE_Q6_K) return __builtin_amdgcn_mfma_f32_16x16x32_f16(al[q >> 2], bv[q & 3], h, 0, 0, 0);
                    else return h;
                };
                f4 c[3];
                c[0] = mm(0);
                c[1] = mm(1);
#pragma unroll
                for (int p = 0; p < 16; p++) {
                    if (p + 2 < 16) c[(p + 2) % 3] = mm(p + 2);
                    const int rt = p >> 2, tt = p & 3;
                    if constexpr (DOTS) {
                        const int t = t0 + 64 * wt + 16 * tt + li, G = 8 * (s >> 2) + g;
#pragma unroll
                        for (int v = 0; v < 4; v++) {
                            const int row = n0 + 64 * wr + 16 * rt + 4 * lq + v;
                            if (t < A.TB && row < A.n_rows)
                                A.dots[((size_t)t * A.n_rows + row) * (A.K / 32) + G] = (int32_t)c[p % 3][v];
                        }
                        continue;
                    }
#pragma unroll
                    for (int v = 0; v < 4; v++) {
                        if constexpr (first) ab[rt][tt][v] = sxv[tt] * c[p % 3][v];
                        else ab[rt][tt][v] = __builtin_fmaf(sxv[tt], c[p % 3][v], ab[rt][tt][v]);
                    }
                }
            };
            using I0 = std::integral_constant<int, 0>;
            using I1 = std::integral_constant<int, 1>;
            // the stage's MFMAs and their epilogue at raised wave priority: the
            // other wave on the SIMD then fills the issue gaps with its decode
            // and loads (measured 5 % faster at configs[3] and the Q6_K side line)
            __builtin_amdgcn_s_setprio(1);
            if (kq == 0) group(I0{}, std::true_type{});
            else group(I0{}, std::false_type{});
            group(I1{}, std::false_type{});
            __builtin_amdgcn_s_setprio(0);
            if (kq == 3 && TYPE == MIQ_TYPE_Q6_K) {
                // block end: acc += d * ab (ab holds sum_g sx * (sc . I) of the block)
                const float *D = reinterpret_cast<const float *>(lds + lds_d<TYPE>());
#pragma unroll
                for (int rt = 0; rt < 4; rt++) {
                    const f4 d4 = *reinterpret_cast<const f4 *>(D + 64 * wr + 16 * rt + 4 * lq);
#pragma unroll
                    for (int tt = 0; tt < 4; tt++)
#pragma unroll
                        for (int v = 0; v < 4; v++) acc[rt][tt][v] = __builtin_fmaf(d4[v], ab[rt][tt][v], acc[rt][tt][v]);
                }
            } else if (kq == 3) {
                // block end: acc += d * ab - dmin * (m . sx*xsum) (the next block's
                // first group overwrites ab).
                // The bf16 MFMA's K slots are (m, m, m, 0) x (hi, mid, lo, 0).
                const uint8_t *Ul = lds + kLU + bb * 8192;
                const float *D = reinterpret_cast<const float *>(lds + kLD);
                b8 mv[4], uv[4];
#pragma unroll
                for (int rt = 0; rt < 4; rt++) {
                    const uint4 mrow = *reinterpret_cast<const uint4 *>(lds + kLM + (64 * wr + 16 * rt + li) * 16);
                    mv[rt] = __builtin_bit_cast(b8, lq == 3 ? make_uint4(0, 0, 0, 0) : mrow);
                }
#pragma unroll
                for (int tt = 0; tt < 4; tt++) uv[tt] = *reinterpret_cast<const b8 *>(Ul + (64 * wt + 16 * tt + li) * 64 + 16 * lq);
#pragma unroll
                for (int rt = 0; rt < 4; rt++) {
                    const f4 d4 = *reinterpret_cast<const f4 *>(D + 64 * wr + 16 * rt + 4 * lq);
                    const f4 dm4 = *reinterpret_cast<const f4 *>(D + kPN + 64 * wr + 16 * rt + 4 * lq);
#pragma unroll
                    for (int tt = 0; tt < 4; tt++) {
                        const f4 T = __builtin_amdgcn_mfma_f32_16x16x32_bf16(mv[rt], uv[tt], f4{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
                        for (int v = 0; v < 4; v++) {
                            acc[rt][tt][v] = __builtin_fmaf(d4[v], ab[rt][tt][v], acc[rt][tt][v]);
                            acc[rt][tt][v] = __builtin_fmaf(-dm4[v], T[v], acc[rt][tt][v]);
                        }
                    }
                }
            }
        }
    };

    // C[row][token]: lane holds rows 4*lq .. 4*lq+3 of each row tile for one token
    auto store = [&](int n0, int t0) {
#pragma unroll
        for (int rt = 0; rt < 4; rt++) {
            const int row = n0 + 64 * wr + 16 * rt + 4 * lq;
#pragma unroll
            for (int tt = 0; tt < 4; tt++) {
                const int t = t0 + 64 * wt + 16 * tt + li;
                if (t >= A.TB) continue;
                const size_t o = (size_t)t * A.out_stride + row;
                if (A.vec_out && row + 3 < A.n_rows) {
                    f4 v = acc[rt][tt] * A.alpha;
                    if (A.residual) v += *reinterpret_cast<const f4 *>(A.residual + o);
                    *reinterpret_cast<f4 *>(A.out + o) = v;
                } else {
#pragma unroll
                    for (int v = 0; v < 4; v++) {
                        if (row + v >= A.n_rows) break;
                        float val = A.alpha * acc[rt][tt][v];
                        if (A.residual) val += A.residual[o + v];
                        A.out[o + v] = val;
                    }
                }
            }
        }
    };

    // Schedule.  `rounds` data-parallel rounds: in round k workgroup w takes
    // tile k*P + 8*(w%8-th XCD block) + w/8, i.e. each XCD (blockIdx % 8) a
    // run of consecutive tiles (one token tile's activation per L2); tiles past
    // T are skipped.  The remaining `sk` tiles are then split along K over all
    // workgroups (stream-K): XCD x owns sk tiles [x*sk/G, (x+1)*sk/G) and cuts
    // their K blocks into P/G equal contiguous ranges, one per workgroup of the
    // XCD.  A tile covered by one range is stored directly; otherwise each
    // range writes a partial (slot 2v for the tile it starts in, 2v+1 for the
    // one it ends in), and the last contributor to arrive adds the partials in
    // range order (the result does not depend on timing) and stores.  The
    // partials of a tile stay in their XCD's L2 unless a workgroup finds itself
    // on another XCD than blockIdx % 8, or G == 1: then they go through memory.
    const int P = gridDim.x, w = blockIdx.x;
    const long T = (long)nt * mt;
    const long F = (long)A.rounds * P, sk = T - F;
    const bool xmap = A.xmap;
    const int G = xmap ? 8 : 1, x = xmap ? w % 8 : 0, Pg = P / G, vl = xmap ? w / 8 : w;
    const long tx0 = F + x * sk / G, tx1 = F + (x + 1) * sk / G;
    const long base = tx0 * nkb, total = sk > 0 ? (tx1 - tx0) * nkb : 0;
    auto rstart = [&](int u) { return base + u * total / Pg; };
    auto owner = [&](long blk) { return (int)(((blk - base + 1) * Pg + total - 1) / total) - 1; };  // local range
    const long bs = total > 0 ? rstart(vl) : 0, be = total > 0 ? rstart(vl + 1) : 0;
    const int v = x * Pg + vl;  // global range id (partial slots)
    constexpr uint32_t kFar = 1u << 20;
    int k = 0;
    long b0 = bs;
    for (;;) {
        // next segment: a data-parallel tile, else the next piece of this
        // workgroup's stream-K range
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
        const int n0 = (int)(t % nt) * kPN, t0 = (int)(t / nt) * kPM;
        run(n0, t0, kb0, kb1);
        if (dp) {  // a data-parallel tile
            if constexpr (!DOTS) store(n0, t0);
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
        f4 *mine = reinterpret_cast<f4 *>(A.part + ((size_t)slot * 256 + tid) * 64);
#pragma unroll
        for (int a = 0; a < 4; a++)
#pragma unroll
            for (int c = 0; c < 4; c++) mine[4 * a + c] = acc[a][c];
        const int v_lo = owner(tb0), v_hi = owner(tb1 - 1);
        int n_contrib = 0;  // ranges of the tile that hold a block (with few blocks some are empty)
        for (int u = v_lo; u <= v_hi; u++) n_contrib += rstart(u) < rstart(u + 1);
        const bool far = !xmap || (__builtin_amdgcn_s_getreg((3 << 11) | (0 << 6) | 20) & 15) != (uint32_t)x;  // HW_REG_XCC_ID
        if (far) __threadfence();  // a reader on another XCD: write the partial back past the L2
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
        if (fl == 2 || far) __threadfence();  // some partial crossed XCDs: drop stale L2 lines first
#pragma unroll
        for (int a = 0; a < 4; a++)
#pragma unroll
            for (int c = 0; c < 4; c++) acc[a][c] = f4{0, 0, 0, 0};
        for (int u = v_lo; u <= v_hi; u++) {
            const long us = rstart(u);
            if (us == rstart(u + 1)) continue;
            const int sl = 2 * (x * Pg + u) + (us >= tb0 ? 0 : 1);  // range u starts in tile t, or ends in it
            const __amdgpu_buffer_rsrc_t rp = make_rsrc(A.part + (size_t)sl * 256 * 64, 256 * 64 * 4);
#pragma unroll
            for (int a = 0; a < 4; a++)
#pragma unroll
                for (int c = 0; c < 4; c++)
                    acc[a][c] += __builtin_bit_cast(
                        f4, __builtin_amdgcn_raw_buffer_load_b128(rp, ((uint32_t)tid * 64 + (4 * a + c) * 4) * 4, 0, 1));
        }
        store(n0, t0);
    }
}

static size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

static int pf16_lds_limit() {
    static bool lds_set[64] = {false};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
        set_error("miq prefill: no current device");
        return MIQ_EHIP;
    }
    if (!lds_set[dev]) {  // more than 64 KiB of dynamic LDS
        const void *k[5] = {(const void *)pf16_kernel<MIQ_TYPE_Q4_K>, (const void *)pf16_kernel<MIQ_TYPE_Q5_K>,
                            (const void *)pf16_kernel<MIQ_TYPE_Q6_K>, (const void *)pf16_kernel<MIQ_TYPE_Q4_K, true>,
                            (const void *)pf16_kernel<MIQ_TYPE_Q5_K, true>};
        for (const void *f : k)
            if (hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, kLBytes) != hipSuccess) {
                set_error("miq prefill: cannot raise the LDS limit to %d bytes", kLBytes);
                return MIQ_EHIP;
            }
        lds_set[dev] = true;
    }
    return MIQ_OK;
}

bool pf16_serves(const miq_seg *s) {
    return s->type == MIQ_TYPE_Q4_K || s->type == MIQ_TYPE_Q5_K || s->type == MIQ_TYPE_Q6_K;
}

// The fp16 GEMM against the split-K 16-token kernel, by a cost model fitted
// to measured times (Q4_K / Q5_K / Q6_K at 48..512 tokens, N x K from
// 1024 x 5120 to 17408 x 5120 and 5120 x 17408; NK = N*K in millions, times
// in us):
//   16-token kernel  c16 * ceil(TB / 16) * NK
//   this kernel      a0 + ac * C + cpf * ceil(TB / 128) * NK
// where C is the number of stream-K ranges that meet in a tile (about P / T
// for T tiles on P < T workgroups, else 2): the last of them adds the others'
// partials, so the fixed cost grows with C.  It takes the batch when its
// estimate is lower.
bool pf16_prefers(const miq_seg *s, int TB) {
    double c16, a0, ac, cpf;
    switch (s->type) {
    case MIQ_TYPE_Q4_K: c16 = 0.15; a0 = 44.0; ac = 4.3; cpf = 0.49; break;
    case MIQ_TYPE_Q5_K: c16 = 0.157; a0 = 44.0; ac = 4.3; cpf = 0.52; break;
    default: c16 = 0.255; a0 = 56.0; ac = 3.6; cpf = 0.70; break;  // Q6_K
    }
    int n_cu = 0;
    if (device_cus(&n_cu) != MIQ_OK) n_cu = 256;
    const double P = 2.0 * n_cu;
    const double T = (double)((s->n_rows + kPN - 1) / kPN) * ((TB + kPM - 1) / kPM);
    const double C = T >= P ? 2.0 : P / T;
    const double nk = (double)s->n_rows * s->K * 1e-6;
    return a0 + ac * C + cpf * ((TB + kPM - 1) / kPM) * nk < c16 * ((TB + 15) / 16) * nk;
}

int launch_pf16(hipStream_t stream, const miq_seg *s, int TB) {
    const int K = s->K;
    const size_t x16_bytes = (size_t)TB * K * 2, sx_bytes = (size_t)(K / 32) * TB * 4, u3_bytes = (size_t)(K / 256) * TB * 64;
    if (x16_bytes >= 0xFFFFFFF0u) {
        set_error("miq prefill: activation of %d x %d exceeds the 4 GiB buffer window", TB, K);
        return MIQ_UNSUPPORTED;
    }
    void *ws = nullptr;
    // the tail partials: at most one 64 KiB partial per workgroup of a round
    int n_cu0 = 0;
    if (device_cus(&n_cu0) != MIQ_OK) return MIQ_EHIP;
    const size_t part_bytes = (size_t)2 * (2 * n_cu0 + 8) * 256 * 64 * 4;
    const size_t ws_bytes = align_up(x16_bytes + sx_bytes + u3_bytes, 256) + part_bytes + 256;
    const int rc = workspace_get(stream, kWsPrefill, ws_bytes, &ws);
    if (rc != MIQ_OK) return rc;
    uint8_t *p = reinterpret_cast<uint8_t *>(ws);
    _Float16 *x16 = reinterpret_cast<_Float16 *>(p);
    float *sx = reinterpret_cast<float *>(p + x16_bytes);
    uint16_t *u3 = reinterpret_cast<uint16_t *>(p + x16_bytes + sx_bytes);
    const long n = (long)(K / 32) * TB;  // eight lanes per (block, token): one per group
    hipLaunchKernelGGL(pf_prep_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, s->x8, s->xmeta,
                       s->xsumq, TB, K, x16, sx, u3);
    PfArgs A;
    A.w = (const uint8_t *)s->w;
    A.row_bytes = (uint32_t)miq_row_bytes(s->type, K);
    A.w_bytes = dword_span((size_t)s->n_rows * A.row_bytes);
    A.K = K;
    A.n_rows = s->n_rows;
    A.TB = TB;
    A.x16 = x16;
    A.sx = sx;
    A.u3 = reinterpret_cast<const __bf16 *>(u3);
    A.out = s->out;
    A.out_stride = s->out_stride;
    A.residual = s->residual;
    A.alpha = s->alpha;
    A.vec_out = ((uintptr_t)s->out % 16 == 0) && (s->out_stride % 4 == 0) &&
                (!s->residual || (uintptr_t)s->residual % 16 == 0);
    // One round of resident workgroups (two per CU), each taking an equal
    // share of the tiles' K blocks (stream-K).
    const int mt = (TB + kPM - 1) / kPM;
    const int nt = (s->n_rows + kPN - 1) / kPN;
    const long T = (long)nt * mt, nkb = K / 256;
    int n_cu = 0;
    int rc2 = device_cus(&n_cu);
    if (rc2 != MIQ_OK) return rc2;
    // Data-parallel rounds of one tile per workgroup when the tiles divide
    // evenly over the workgroups, else every tile is split along K (stream-K)
    // over all of them (small shapes: over at most one workgroup per K block).
    // Measured (Q4_K/Q6_K, 128..1024 tokens, 5120x5120, 17408x5120,
    // 5120x17408): stream-K over every tile is never slower than data-parallel
    // rounds plus a stream-K tail or an extra part-filled round, and up to 1.5x
    // faster (a round of 272 tiles on 512 workgroups: 183 us, stream-K 143 us).
    long P = 2L * n_cu - (2L * n_cu) % 8;
    long rounds = T / P, sk = T % P;
    if (sk > 0) {
        rounds = 0;
        sk = T;
    }
    if (rounds == 0 && sk * nkb < P) P = sk * nkb >= 8 ? sk * nkb / 8 * 8 : sk * nkb;
    A.rounds = (int)rounds;
    A.xmap = sk >= 8 && P % 8 == 0;
    const unsigned grid = (unsigned)P;
    void *cw = nullptr;
    if ((rc2 = workspace_get(stream, kWsPrefillCnt, (size_t)T * 4, &cw, true)) != MIQ_OK) return rc2;
    A.cnt = reinterpret_cast<uint32_t *>(cw);
    A.part = reinterpret_cast<float *>(p + align_up(x16_bytes + sx_bytes + u3_bytes, 256));
    if (int rc = pf16_lds_limit()) return rc;
    if (s->type == MIQ_TYPE_Q4_K) hipLaunchKernelGGL(pf16_kernel<MIQ_TYPE_Q4_K>, dim3(grid), dim3(256), kLBytes, stream, A);
    else if (s->type == MIQ_TYPE_Q5_K) hipLaunchKernelGGL(pf16_kernel<MIQ_TYPE_Q5_K>, dim3(grid), dim3(256), kLBytes, stream, A);
    else hipLaunchKernelGGL(pf16_kernel<MIQ_TYPE_Q6_K>, dim3(grid), dim3(256), kLBytes, stream, A);
    return check_launch("miq prefill");
}

// Parity form (miq_group_dots path 2): the pre-pass, then one tile per
// workgroup with every 32-group's MFMA result written to `out`: sc * I for
// Q4_K/Q5_K; for Q6_K the two planes' sum sc0 * I0 + sc1 * I1 of the group's
// 16-value sub-groups, I = sum (q - 32) * x8 (exact in fp32 below 2^24).
int launch_pf16_dots(hipStream_t stream, const miq_seg *s, int TB, int32_t *out) {
    if (s->type != MIQ_TYPE_Q4_K && s->type != MIQ_TYPE_Q5_K && s->type != MIQ_TYPE_Q6_K) {
        set_error("miq_group_dots: path 2 (the fp16 prefill decoder) serves Q4_K, Q5_K and Q6_K");
        return MIQ_UNSUPPORTED;
    }
    const int K = s->K;
    const size_t x16_bytes = (size_t)TB * K * 2, sx_bytes = (size_t)(K / 32) * TB * 4, u3_bytes = (size_t)(K / 256) * TB * 64;
    void *ws = nullptr;
    if (int rc = workspace_get(stream, kWsPrefill, align_up(x16_bytes + sx_bytes + u3_bytes, 256), &ws)) return rc;
    if (int rc = pf16_lds_limit()) return rc;
    uint8_t *p = reinterpret_cast<uint8_t *>(ws);
    _Float16 *x16 = reinterpret_cast<_Float16 *>(p);
    float *sx = reinterpret_cast<float *>(p + x16_bytes);
    uint16_t *u3 = reinterpret_cast<uint16_t *>(p + x16_bytes + sx_bytes);
    const long n = (long)(K / 32) * TB;  // eight lanes per (block, token): one per group
    hipLaunchKernelGGL(pf_prep_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, s->x8, s->xmeta,
                       s->xsumq, TB, K, x16, sx, u3);
    PfArgs A{};
    A.w = (const uint8_t *)s->w;
    A.row_bytes = (uint32_t)miq_row_bytes(s->type, K);
    A.w_bytes = dword_span((size_t)s->n_rows * A.row_bytes);
    A.K = K;
    A.n_rows = s->n_rows;
    A.TB = TB;
    A.x16 = x16;
    A.sx = sx;
    A.u3 = reinterpret_cast<const __bf16 *>(u3);
    A.alpha = 1.0f;
    A.rounds = 1;
    A.xmap = 0;
    A.dots = out;
    const long T = (long)((s->n_rows + kPN - 1) / kPN) * ((TB + kPM - 1) / kPM);
    // one round: tile (w % 8) * (P / 8) + w / 8 of workgroup w is a
    // permutation of 0..P-1 when 8 divides P; tiles past T are skipped
    const unsigned grid = (unsigned)((T + 7) / 8 * 8);
    if (s->type == MIQ_TYPE_Q4_K)
        hipLaunchKernelGGL((pf16_kernel<MIQ_TYPE_Q4_K, true>), dim3(grid), dim3(256), kLBytes, stream, A);
    else if (s->type == MIQ_TYPE_Q5_K)
        hipLaunchKernelGGL((pf16_kernel<MIQ_TYPE_Q5_K, true>), dim3(grid), dim3(256), kLBytes, stream, A);
    else
        hipLaunchKernelGGL((pf16_kernel<MIQ_TYPE_Q6_K, true>), dim3(grid), dim3(256), kLBytes, stream, A);
    return check_launch("miq_group_dots");
}

}  // namespace miq
