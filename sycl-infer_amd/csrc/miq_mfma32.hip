// Chunked-prefill GEMM on int8 MFMA (v_mfma_i32_32x32x32_i8, full rate on
// gfx950): out[t][n] = alpha * sum_k W[n][k] * act_t[k] (+ residual) for many
// tokens.
//
// Workgroup tile: 64 tokens x 128 rows, 4 waves in a 2x2 arrangement, each
// wave 32 tokens x 64 rows = 1x2 MFMA tiles.  The K loop walks one 256-value
// block per step.  Each step the workgroup decodes its 128 rows' Q4_K/Q5_K/
// Q8_0 bytes once into int8 codes in LDS (plus per-(row, group) fp32 scales)
// and copies the 128 tokens' codes and scales next to them; the next step's
// raw bytes are fetched into registers while the current step computes.
//
// One MFMA K step is one 32-value group, so every MFMA result is the exact
// int32 group dot of the reference (i8.cpp:49-57,109-118; q4exp.cpp:457-467);
// the fp32 epilogue applies sx*d*sc per (token, row, group) on the VALU and the
// rank-G dmin*m*xsum term (i8.cpp:60,120) runs on fp32 MFMA
// (v_mfma_f32_32x32x2_f32: tokens x 2 groups times 2 groups x rows).
// MFMA C layout (32x32): lane l, register v -> row 8*(v/4) + 4*(l/32) + v%4
// (tokens), column l%32 (weight rows).
#include "miq_internal.h"
#include "miq_units.h"

namespace miq {

typedef int v4i32 __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int kBM = 64;   // tokens per workgroup
constexpr int kBN = 128;  // weight rows per workgroup
// LDS rows of 256 codes; the 16-byte chunk c of row r lives at chunk c ^ (r & 15),
// so the 32 rows a b128 operand read touches hit distinct banks.
__device__ __forceinline__ int swz(int r, int chunk) { return r * 256 + ((chunk ^ (r & 15)) << 4); }

struct M32Args {
    const uint8_t *w;
    uint32_t w_bytes;
    uint32_t row_bytes;
    int K;
    int n_rows;
    int TB;
    const int8_t *x8;
    const float *xmeta;
    const int32_t *xsumq;
    float *out;
    int out_stride;
    const float *residual;
    float alpha;
    int32_t *dots;  // parity form: [TB][n_rows][K/32] int32 group dots
};

// LDS layout of one step
struct M32Lds {
    uint8_t wq[kBN * 256];        // weight codes [row][256], swizzled chunks
    uint8_t xq[kBM * 256];        // activation codes [token][256], swizzled chunks
    float dsc[8][kBN];            // d*sc per (group, row)
    float dmm[8][kBN];            // dmin*m per (group, row)
    float sx[8][kBM];             // activation scale per (group, token)
    float u[8][kBM];              // sx * (s0 + s1) per (group, token)
};

// Raw bytes one thread fetches for a step: two weight units (Q4_K/Q5_K:
// 16 B header + 32 B qs (+ 32 B qh for Q5_K) of a quarter block; Q8_0: a
// quarter of the 8-block step), four 16-byte activation chunks and one
// chunk each of xmeta / xsumq.
template <uint32_t TYPE> struct M32Raw {
    uint4 w[2][TYPE == MIQ_TYPE_Q5_K ? 5 : (TYPE == MIQ_TYPE_Q8_0 ? 5 : 3)];
    FetchQ6K f6[2];  // Q6_K: unit (row, blk2, half) as fetch_q6k loads it
    uint32_t sh6[2];  // and its block offset's byte shift
    uint4 x[4];
    uint4 m, q;
};

template <uint32_t TYPE>
__device__ __forceinline__ void m32_fetch(M32Raw<TYPE> &R, const M32Args &A, __amdgpu_buffer_rsrc_t rw,
                                          __amdgpu_buffer_rsrc_t rx, __amdgpu_buffer_rsrc_t rm,
                                          __amdgpu_buffer_rsrc_t rq, int n0, int t0, int kb) {
    const int tid = threadIdx.x;
    // weights: unit = (row r, quarter c), 512 units, two per thread
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int unit = tid + 256 * i;
        const int r = unit >> 2, c = unit & 3;
        const int row = n0 + r;
        const uint32_t base = row < A.n_rows ? (uint32_t)row * A.row_bytes : A.w_bytes;
        if constexpr (TYPE == MIQ_TYPE_Q4_K) {
            const uint32_t b = base + (uint32_t)kb * kQ4KBytes;
            R.w[i][0] = bload16(rw, b);
            R.w[i][1] = bload16(rw, b + 16 + 32 * c);
            R.w[i][2] = bload16(rw, b + 32 + 32 * c);
        } else if constexpr (TYPE == MIQ_TYPE_Q5_K) {
            const uint32_t b = base + (uint32_t)kb * kQ5KBytes;
            R.w[i][0] = bload16(rw, b);
            R.w[i][1] = bload16(rw, b + 48 + 32 * c);
            R.w[i][2] = bload16(rw, b + 64 + 32 * c);
            R.w[i][3] = bload16(rw, b + 16);
            R.w[i][4] = bload16(rw, b + 32);
        } else if constexpr (TYPE == MIQ_TYPE_Q6_K) {  // c = blk2 * 2 + half (2-byte aligned blocks)
            R.f6[i] = fetch_q6k(rw, base + (uint32_t)kb * kQ6KBytes, c);
            R.sh6[i] = (base + (uint32_t)kb * kQ6KBytes) & 3u;
        } else {  // Q8_0: quarter c = blocks 2c, 2c+1 of the step (68 bytes, 4-byte aligned)
            const uint32_t b = base + (uint32_t)kb * 272u + 68u * c;
            R.w[i][0] = bload16(rw, b);
            R.w[i][1] = bload16(rw, b + 16);
            R.w[i][2] = bload16(rw, b + 32);
            R.w[i][3] = bload16(rw, b + 48);
            R.w[i][4] = make_uint4(bload4(rw, b + 64), 0, 0, 0);
        }
    }
    // activations: group g, token tt, half hf -> 16-byte chunk; 1024 chunks, 4 per thread
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int ch = tid + 256 * i;
        const int g = ch >> 7, rest = ch & 127, tt = rest >> 1, hf = rest & 1;
        const int t = t0 + tt;
        const uint32_t off = t < A.TB ? ((uint32_t)(kb * 8 + g) * A.TB + t) * 32 + 16 * hf : 0xFFFFFFF0u;
        R.x[i] = bload16(rx, off);
    }
    // scales and sums: group g, token pair p -> 16 bytes of xmeta and of xsumq; 256 chunks
    {
        const int g = tid >> 5, p = tid & 31;
        const int t = t0 + 2 * p;
        const uint32_t off = t < A.TB ? ((uint32_t)(kb * 8 + g) * A.TB + t) * 8 : 0xFFFFFFF0u;
        R.m = bload16(rm, off);
        R.q = bload16(rq, off);
    }
}

template <uint32_t TYPE>
__device__ __forceinline__ void m32_store(const M32Raw<TYPE> &R, M32Lds &L, const M32Args &A, int n0, int t0) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int unit = tid + 256 * i;
        const int r = unit >> 2, c = unit & 3;
        const bool ok = n0 + r < A.n_rows;
        if constexpr (TYPE == MIQ_TYPE_Q4_K || TYPE == MIQ_TYPE_Q5_K) {
            const uint4 hdr = R.w[i][0];
            const uint32_t q[8] = {R.w[i][1].x, R.w[i][1].y, R.w[i][1].z, R.w[i][1].w,
                                   R.w[i][2].x, R.w[i][2].y, R.w[i][2].z, R.w[i][2].w};
            uint32_t lo[8], hi[8];
#pragma unroll
            for (int k = 0; k < 8; k++) {
                lo[k] = q[k] & 0x0F0F0F0Fu;
                hi[k] = (q[k] >> 4) & 0x0F0F0F0Fu;
            }
            if constexpr (TYPE == MIQ_TYPE_Q5_K) {
                const uint32_t h[8] = {R.w[i][3].x, R.w[i][3].y, R.w[i][3].z, R.w[i][3].w,
                                       R.w[i][4].x, R.w[i][4].y, R.w[i][4].z, R.w[i][4].w};
#pragma unroll
                for (int k = 0; k < 8; k++) {
                    lo[k] |= ((h[k] >> (2 * c)) & 0x01010101u) << 4;
                    hi[k] |= ((h[k] >> (2 * c + 1)) & 0x01010101u) << 4;
                }
            }
            // group 2c codes -> chunks 4c, 4c+1; group 2c+1 -> chunks 4c+2, 4c+3
            *reinterpret_cast<uint4 *>(L.wq + swz(r, 4 * c + 0)) = make_uint4(lo[0], lo[1], lo[2], lo[3]);
            *reinterpret_cast<uint4 *>(L.wq + swz(r, 4 * c + 1)) = make_uint4(lo[4], lo[5], lo[6], lo[7]);
            *reinterpret_cast<uint4 *>(L.wq + swz(r, 4 * c + 2)) = make_uint4(hi[0], hi[1], hi[2], hi[3]);
            *reinterpret_cast<uint4 *>(L.wq + swz(r, 4 * c + 3)) = make_uint4(hi[4], hi[5], hi[6], hi[7]);
            const float d = h2f(hdr.x), dm = h2f(hdr.x >> 16);
            int sc0, m0, sc1, m1;
            scale_min_k4(2 * c, hdr.y, hdr.z, hdr.w, sc0, m0);
            scale_min_k4(2 * c + 1, hdr.y, hdr.z, hdr.w, sc1, m1);
            L.dsc[2 * c][r] = ok ? d * (float)sc0 : 0.0f;
            L.dsc[2 * c + 1][r] = ok ? d * (float)sc1 : 0.0f;
            L.dmm[2 * c][r] = ok ? dm * (float)m0 : 0.0f;
            L.dmm[2 * c + 1][r] = ok ? dm * (float)m1 : 0.0f;
        } else if constexpr (TYPE == MIQ_TYPE_Q6_K) {
            // unit c = (blk2, half): plane p's 16 codes are sub-group s = 8*blk2 + 2p + half,
            // LDS chunk s; MFMA group g = 4*blk2 + p takes half 0 / 1 on its two lane halves,
            // whose scales go to dsc[g] / dmm[g]
            const RawQ6K u = dec_q6k(R.f6[i], R.sh6[i]);
            const int blk2 = c >> 1, half = c & 1;
            const uint32_t l0[4] = {u.l0.x, u.l0.y, u.l0.z, u.l0.w};
            const uint32_t l1[4] = {u.l1.x, u.l1.y, u.l1.z, u.l1.w};
            const uint32_t hh[4] = {u.h.x, u.h.y, u.h.z, u.h.w};
            const float d = h2f(u.dbits);
#pragma unroll
            for (int p = 0; p < 4; p++) {
                uint32_t q[4];
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    const uint32_t src = (p & 1) ? l1[k] : l0[k];
                    q[k] = q6_signed(((p >= 2 ? (src >> 4) : src) & 0x0F0F0F0Fu) | (((hh[k] >> (2 * p)) & 0x03030303u) << 4));
                }
                *reinterpret_cast<uint4 *>(L.wq + swz(r, 8 * blk2 + 2 * p + half)) = make_uint4(q[0], q[1], q[2], q[3]);
                const float ds = ok ? d * (float)q6k_scale(u, c, p) : 0.0f;
                if (half) L.dmm[4 * blk2 + p][r] = ds;
                else L.dsc[4 * blk2 + p][r] = ds;
            }
        } else {  // Q8_0 blocks 2c, 2c+1: 68 bytes
            const uint32_t w[17] = {R.w[i][0].x, R.w[i][0].y, R.w[i][0].z, R.w[i][0].w, R.w[i][1].x, R.w[i][1].y,
                                    R.w[i][1].z, R.w[i][1].w, R.w[i][2].x, R.w[i][2].y, R.w[i][2].z, R.w[i][2].w,
                                    R.w[i][3].x, R.w[i][3].y, R.w[i][3].z, R.w[i][3].w, R.w[i][4].x};
            uint32_t a[8], b[8];
#pragma unroll
            for (int k = 0; k < 8; k++) {
                a[k] = __builtin_amdgcn_alignbyte(w[k + 1], w[k], 2);
                b[k] = w[9 + k];
            }
            *reinterpret_cast<uint4 *>(L.wq + swz(r, 4 * c + 0)) = make_uint4(a[0], a[1], a[2], a[3]);
            *reinterpret_cast<uint4 *>(L.wq + swz(r, 4 * c + 1)) = make_uint4(a[4], a[5], a[6], a[7]);
            *reinterpret_cast<uint4 *>(L.wq + swz(r, 4 * c + 2)) = make_uint4(b[0], b[1], b[2], b[3]);
            *reinterpret_cast<uint4 *>(L.wq + swz(r, 4 * c + 3)) = make_uint4(b[4], b[5], b[6], b[7]);
            L.dsc[2 * c][r] = ok ? h2f(w[0]) : 0.0f;
            L.dsc[2 * c + 1][r] = ok ? h2f(w[8] >> 16) : 0.0f;
        }
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int ch = tid + 256 * i;
        const int g = ch >> 7, rest = ch & 127, tt = rest >> 1, hf = rest & 1;
        *reinterpret_cast<uint4 *>(L.xq + swz(tt, 2 * g + hf)) = R.x[i];
    }
    {
        const int g = tid >> 5, p = tid & 31;
        const int t = t0 + 2 * p;
        const float s0 = t < A.TB ? __builtin_bit_cast(float, R.m.x) : 0.0f;
        const float s1 = t + 1 < A.TB ? __builtin_bit_cast(float, R.m.z) : 0.0f;
        L.sx[g][2 * p] = s0;
        L.sx[g][2 * p + 1] = s1;
        L.u[g][2 * p] = s0 * (float)((int)R.q.x + (int)R.q.y);
        L.u[g][2 * p + 1] = s1 * (float)((int)R.q.z + (int)R.q.w);
    }
}

// DOTS: the parity form -- every MFMA result (the exact int32 group dot)
// goes to A.dots and nothing else is computed
template <uint32_t TYPE, bool DOTS = false>
__global__ __launch_bounds__(256, 2) void mfma32_kernel(M32Args A) {
    extern __shared__ __align__(16) uint8_t lds_raw[];
    M32Lds &L = *reinterpret_cast<M32Lds *>(lds_raw);
    const int n0 = blockIdx.x * kBN, t0 = blockIdx.y * kBM;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wt = (wave >> 1) * 32, wn = (wave & 1) * 64;  // wave tile origin (tokens, rows)
    const int l32 = lane & 31, hk = lane >> 5;
    const int nkb = A.K / 256;
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(A.w, A.w_bytes);
    const uint32_t xbytes = (uint32_t)(A.K / 32) * A.TB * 32, mbytes = (uint32_t)(A.K / 32) * A.TB * 8;
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(A.x8, xbytes);
    const __amdgpu_buffer_rsrc_t rm = make_rsrc(A.xmeta, mbytes), rq = make_rsrc(A.xsumq, mbytes);

    v16f acc[2], t2[2];
#pragma unroll
    for (int j = 0; j < 2; j++) {
        acc[j] = v16f{};
        t2[j] = v16f{};
    }

    M32Raw<TYPE> R;
    m32_fetch<TYPE>(R, A, rw, rx, rm, rq, n0, t0, 0);
    for (int kb = 0; kb < nkb; kb++) {
        __syncthreads();  // the previous step's LDS reads are done
        m32_store<TYPE>(R, L, A, n0, t0);
        __syncthreads();
        if (kb + 1 < nkb) m32_fetch<TYPE>(R, A, rw, rx, rm, rq, n0, t0, kb + 1);
#pragma unroll 2
        for (int g = 0; g < 8; g++) {
            // operands: A = tokens (rows i), B = weight rows (columns j); lane half hk takes k 16*hk..16*hk+15
            const v4i32 av = *reinterpret_cast<const v4i32 *>(L.xq + swz(wt + l32, 2 * g + hk));
            v4i32 bv[2];
#pragma unroll
            for (int j = 0; j < 2; j++) bv[j] = *reinterpret_cast<const v4i32 *>(L.wq + swz(wn + 32 * j + l32, 2 * g + hk));
            if constexpr (TYPE == MIQ_TYPE_Q6_K) {
                // two 16-value sub-groups with their own scales: one MFMA per
                // sub-group, the other lane half's weights zeroed
                const v4i32 zero{0, 0, 0, 0};
                v16i I0[2], I1[2];
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    I0[j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, hk ? zero : bv[j], v16i{}, 0, 0, 0);
                    I1[j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, hk ? bv[j] : zero, v16i{}, 0, 0, 0);
                }
                if constexpr (DOTS) {  // the unsigned-code sums wd = I + 32 * xsum of the half (i8.cpp:149)
#pragma unroll
                    for (int j = 0; j < 2; j++) {
                        const int row = n0 + wn + 32 * j + l32;
#pragma unroll
                        for (int v = 0; v < 16; v++) {
                            const int t = t0 + wt + 8 * (v >> 2) + 4 * hk + (v & 3);
                            if (t < A.TB && row < A.n_rows) {
                                const int32_t *xs = A.xsumq + ((size_t)(8 * kb + g) * A.TB + t) * 2;
                                int32_t *o = A.dots + ((size_t)t * A.n_rows + row) * (A.K / 16) + 2 * (8 * kb + g);
                                o[0] = I0[j][v] + 32 * xs[0];
                                o[1] = I1[j][v] + 32 * xs[1];
                            }
                        }
                    }
                    continue;
                }
                float sxr[16];
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const float4 sv = *reinterpret_cast<const float4 *>(&L.sx[g][wt + 8 * q + 4 * hk]);
                    sxr[4 * q + 0] = sv.x;
                    sxr[4 * q + 1] = sv.y;
                    sxr[4 * q + 2] = sv.z;
                    sxr[4 * q + 3] = sv.w;
                }
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    const float ds0 = L.dsc[g][wn + 32 * j + l32], ds1 = L.dmm[g][wn + 32 * j + l32];
#pragma unroll
                    for (int v = 0; v < 16; v++) {
                        acc[j][v] += sxr[v] * (ds0 * (float)I0[j][v]);
                        acc[j][v] += sxr[v] * (ds1 * (float)I1[j][v]);
                    }
                }
                continue;
            }
            v16i I[2];
#pragma unroll
            for (int j = 0; j < 2; j++) I[j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, bv[j], v16i{}, 0, 0, 0);
            if constexpr (DOTS) {
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    const int row = n0 + wn + 32 * j + l32;
#pragma unroll
                    for (int v = 0; v < 16; v++) {
                        const int t = t0 + wt + 8 * (v >> 2) + 4 * hk + (v & 3);
                        if (t < A.TB && row < A.n_rows)
                            A.dots[((size_t)t * A.n_rows + row) * (A.K / 32) + 8 * kb + g] = I[j][v];
                    }
                }
                continue;
            }
            // token scales of this lane's C rows: tokens 8*(v/4) + 4*hk + v%4
            float sxr[16];
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const float4 sv = *reinterpret_cast<const float4 *>(&L.sx[g][wt + 8 * q + 4 * hk]);
                sxr[4 * q + 0] = sv.x;
                sxr[4 * q + 1] = sv.y;
                sxr[4 * q + 2] = sv.z;
                sxr[4 * q + 3] = sv.w;
            }
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const float dsc = L.dsc[g][wn + 32 * j + l32];
#pragma unroll
                for (int v = 0; v < 16; v++) acc[j][v] += sxr[v] * (dsc * (float)I[j][v]);
            }
        }
        if constexpr (TYPE != MIQ_TYPE_Q8_0 && TYPE != MIQ_TYPE_Q6_K && !DOTS) {
            // dmin*m*xsum: A = u (tokens x 2 groups), B = dmin*m (2 groups x rows)
#pragma unroll
            for (int gp = 0; gp < 4; gp++) {
                const int g = 2 * gp + hk;
                const float a = L.u[g][wt + l32];
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    const float b = L.dmm[g][wn + 32 * j + l32];
                    t2[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, t2[j], 0, 0, 0);
                }
            }
        }
    }
    if constexpr (DOTS) return;
    // write: C[token][row]
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int row = n0 + wn + 32 * j + l32;
        if (row >= A.n_rows) continue;
#pragma unroll
        for (int v = 0; v < 16; v++) {
            const int t = t0 + wt + 8 * (v >> 2) + 4 * hk + (v & 3);
            if (t < A.TB) {
                const size_t o = (size_t)t * A.out_stride + row;
                float val = A.alpha * (acc[j][v] - t2[j][v]);
                if (A.residual) val += A.residual[o];
                A.out[o] = val;
            }
        }
    }
}

bool mfma32_serves(const miq_seg *s) {
    // Q8_0 rows whose K is not a whole number of 256-value steps go to the 16-token kernel
    return s->type == MIQ_TYPE_Q4_K || s->type == MIQ_TYPE_Q5_K || s->type == MIQ_TYPE_Q6_K ||
           (s->type == MIQ_TYPE_Q8_0 && s->K % 256 == 0);
}

bool mfma32_fills(const miq_seg *s, int TB) {
    if (s->type != MIQ_TYPE_Q6_K || sw(kSwM32Fill) == 0) return true;  // M32_FILL=0: the tiled kernel at any size
    int cus = 0;
    if (device_cus(&cus) != MIQ_OK) return true;
    // measured (Q6_K, K 5120/17408): 136 or 80 tiles lose to the 16-token kernel by 1.4-2.3x, 272 / 320 tiles win by 1.1-1.7x
    return (long)((s->n_rows + kBN - 1) / kBN) * ((TB + kBM - 1) / kBM) >= cus;
}

int launch_mfma32(hipStream_t stream, const miq_seg *s, int TB, int32_t *dots) {
    M32Args A{};
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
    A.out_stride = s->out_stride;
    A.residual = s->residual;
    A.alpha = s->alpha;
    const dim3 grid((s->n_rows + kBN - 1) / kBN, (TB + kBM - 1) / kBM);
    const size_t lds = sizeof(M32Lds);
    A.dots = dots;
    if (dots) {  // parity form (miq_group_dots path 3)
        switch (s->type) {
        case MIQ_TYPE_Q4_K: hipLaunchKernelGGL((mfma32_kernel<MIQ_TYPE_Q4_K, true>), grid, dim3(256), lds, stream, A); break;
        case MIQ_TYPE_Q5_K: hipLaunchKernelGGL((mfma32_kernel<MIQ_TYPE_Q5_K, true>), grid, dim3(256), lds, stream, A); break;
        case MIQ_TYPE_Q6_K: hipLaunchKernelGGL((mfma32_kernel<MIQ_TYPE_Q6_K, true>), grid, dim3(256), lds, stream, A); break;
        default: hipLaunchKernelGGL((mfma32_kernel<MIQ_TYPE_Q8_0, true>), grid, dim3(256), lds, stream, A); break;
        }
        return check_launch("miq_group_dots");
    }
    switch (s->type) {
    case MIQ_TYPE_Q4_K: hipLaunchKernelGGL(mfma32_kernel<MIQ_TYPE_Q4_K>, grid, dim3(256), lds, stream, A); break;
    case MIQ_TYPE_Q5_K: hipLaunchKernelGGL(mfma32_kernel<MIQ_TYPE_Q5_K>, grid, dim3(256), lds, stream, A); break;
    case MIQ_TYPE_Q6_K: hipLaunchKernelGGL(mfma32_kernel<MIQ_TYPE_Q6_K>, grid, dim3(256), lds, stream, A); break;
    default: hipLaunchKernelGGL(mfma32_kernel<MIQ_TYPE_Q8_0>, grid, dim3(256), lds, stream, A); break;
    }
    return check_launch("miq mfma32");
}

}  // namespace miq
