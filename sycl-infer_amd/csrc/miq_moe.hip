// MoE on the integer path: router, token->expert CSR, expert-grouped GEMV
// (gate/up fused into silu(g)*u, then down) and the weighted reduce.
//
// Reference semantics:
//   router  cpu_moe_route (src/backend/cpu/kernels/moe.cpp:72-137): logits in
//           double, max-subtracted softmax summed in expert order, top-k by
//           rank counting (ties to the lower index), renormalise by
//           max(sum of the selected, 6.103515625e-5)
//   experts cpu_moe_experts_i8 (moe.cpp:476-559): per pair, gate/up integer
//           GEMV on xq(x), h = silu(g)*u, h requantised (quant_row_1 ==
//           cpu_xq), down integer GEMV on xq(h)
//   reduce  cpu_moe_reduce (moe.cpp:562-574): out += sum_j w*acc in double
// The GPU form groups the pairs by expert (the CSR) so each active expert's
// weights are streamed once for all of its pairs, as moe_grp_gate_up_launch /
// moe_grp_down_launch do on the reference GPU (kernels.h:638,718).
#include "miq_internal.h"
#include "miq_units.h"

namespace miq {

// ------------------------------------------------------------------ router
// One workgroup (256 threads) per token.  The max is order-free (a tree); the
// softmax sum and the sum of the selected probabilities run in expert order on
// one thread, as the reference's loops do, over vector LDS reads.
__device__ __forceinline__ float block_max256(float v, float *red) {
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    v = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    __syncthreads();
    return v;
}

__global__ __launch_bounds__(256) void route_kernel(const float *__restrict__ x, int x_stride,
                                                    const float *__restrict__ gate_inp, int n_embd, int n_expert,
                                                    int top_k, float *__restrict__ logits, int32_t *__restrict__ ids,
                                                    float *__restrict__ wts) {
    extern __shared__ __align__(16) float sp[];  // [n_expert rounded to 4] probabilities
    __shared__ float red[4];
    __shared__ float s_inv, s_den;
    __shared__ int sids[64];  // the selected experts by rank (top_k <= 64)
    const int t = blockIdx.x;
    const int ne4 = (n_expert + 3) & ~3;
    float *lg = logits + (size_t)t * n_expert;
    if (gate_inp) {
        // one wave per expert: double-precision dot, as the reference's F32 router
        const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
        const float *xr = x + (size_t)t * x_stride;
        for (int e = wave; e < n_expert; e += blockDim.x / 64) {
            const float *w = gate_inp + (size_t)e * n_embd;
            double a = 0.0;
            for (int k = lane; k < n_embd; k += 64) a += (double)w[k] * (double)xr[k];
            for (int o = 32; o > 0; o >>= 1) a += __shfl_xor(a, o, 64);
            if (lane == 0) lg[e] = (float)a;
        }
        __syncthreads();
    }
    float mx = -3.402823466e38f;
    for (int e = threadIdx.x; e < ne4; e += blockDim.x) {
        const float v = e < n_expert ? lg[e] : -3.402823466e38f;
        sp[e] = v;
        mx = fmaxf(mx, v);
    }
    mx = block_max256(mx, red);
    for (int e = threadIdx.x; e < ne4; e += blockDim.x) sp[e] = e < n_expert ? expf(sp[e] - mx) : 0.0f;
    __syncthreads();
    if (threadIdx.x == 0) {
        float sum = 0.f;
        const float4 *s4 = reinterpret_cast<const float4 *>(sp);
        for (int q = 0; q < ne4 / 4; q++) {  // expert order
            const float4 v = s4[q];
            sum += v.x;
            sum += v.y;
            sum += v.z;
            sum += v.w;
        }
        s_inv = 1.f / sum;
    }
    __syncthreads();
    const float inv = s_inv;
    // the logits scratch ends holding the probabilities, as in cpu_moe_route
    for (int e = threadIdx.x; e < n_expert; e += blockDim.x) lg[e] = sp[e] * inv;
    __syncthreads();
    for (int e = threadIdx.x; e < ne4; e += blockDim.x) sp[e] *= inv;
    __syncthreads();
    // rank of every expert: how many beat it (ties to the lower index); padding scores 0 and loses ties
    const float4 *s4 = reinterpret_cast<const float4 *>(sp);
    for (int e = threadIdx.x; e < n_expert; e += blockDim.x) {
        const float pe = sp[e];
        int rank = 0;
#pragma unroll 4
        for (int q = 0; q < ne4 / 4; q++) {
            const float4 v = s4[q];
            const int f = 4 * q;
            rank += (v.x > pe || (v.x == pe && f < e)) + (v.y > pe || (v.y == pe && f + 1 < e)) +
                    (v.z > pe || (v.z == pe && f + 2 < e)) + (v.w > pe || (v.w == pe && f + 3 < e));
        }
        if (rank < top_k) {
            ids[(size_t)t * top_k + rank] = e;
            sids[rank] = e;
        }
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        // sum of the selected, in expert order
        int sel[64];
        const int k = top_k < 64 ? top_k : 64;
        for (int i = 0; i < k; i++) sel[i] = sids[i];
        for (int i = 1; i < k; i++)
            for (int j2 = i; j2 > 0 && sel[j2 - 1] > sel[j2]; j2--) {
                const int tmp = sel[j2];
                sel[j2] = sel[j2 - 1];
                sel[j2 - 1] = tmp;
            }
        float wsum = 0.f;
        for (int i = 0; i < k; i++) wsum += sp[sel[i]];
        s_den = fmaxf(wsum, 6.103515625e-5f);
    }
    __syncthreads();
    for (int r = threadIdx.x; r < top_k; r += blockDim.x) wts[(size_t)t * top_k + r] = sp[sids[r]] / s_den;
}

// ------------------------------------------------------------------ CSR
// One workgroup of 1024 threads: ids staged in LDS, counts by LDS atomics,
// offsets and the active list by block-wide scans; pairs of one expert keep
// ascending pair order (a pair's slot = the earlier pairs of its expert).
__device__ __forceinline__ int block_scan1024(int v, int *tmp) {  // inclusive
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int o = 1; o < 64; o <<= 1) {
        const int n = __shfl_up(v, o, 64);
        if (lane >= o) v += n;
    }
    if (lane == 63) tmp[wave] = v;
    __syncthreads();
    if (wave == 0) {
        int w = lane < 16 ? tmp[lane] : 0;
        for (int o = 1; o < 16; o <<= 1) {
            const int n = __shfl_up(w, o, 64);
            if (lane >= o) w += n;
        }
        if (lane < 16) tmp[lane] = w;
    }
    __syncthreads();
    const int r = v + (wave ? tmp[wave - 1] : 0);
    __syncthreads();
    return r;
}

__global__ __launch_bounds__(1024) void csr_kernel(const int32_t *__restrict__ ids, int n_pairs, int n_expert,
                                                   int32_t *__restrict__ off, int32_t *__restrict__ pair,
                                                   int32_t *__restrict__ active, int32_t *__restrict__ n_active) {
    extern __shared__ int sm[];
    int *cnt = sm;              // [n_expert]
    int *sid = sm + n_expert;   // [n_pairs]
    __shared__ int tmp[16];
    __shared__ int carry[2];
    for (int e = threadIdx.x; e < n_expert; e += blockDim.x) cnt[e] = 0;
    for (int p = threadIdx.x; p < n_pairs; p += blockDim.x) sid[p] = ids[p];
    if (threadIdx.x < 2) carry[threadIdx.x] = 0;
    __syncthreads();
    for (int p = threadIdx.x; p < n_pairs; p += blockDim.x) {
        const int e = sid[p];
        if (e >= 0 && e < n_expert) atomicAdd(&cnt[e], 1);
    }
    __syncthreads();
    // exclusive scans of the counts (offsets) and of the active flags, 1024 experts at a time
    for (int e0 = 0; e0 < n_expert; e0 += blockDim.x) {
        const int e = e0 + threadIdx.x;
        const int c = e < n_expert ? cnt[e] : 0;
        const int incl = block_scan1024(c, tmp);
        const int aincl = block_scan1024(c > 0, tmp);
        const int base = carry[0] + incl - c, apos = carry[1] + aincl - (c > 0);
        if (e < n_expert) {
            off[e] = base;
            cnt[e] = base;  // from here on cnt holds the offsets
            if (c > 0) active[apos] = e;
        }
        __syncthreads();
        if (threadIdx.x == blockDim.x - 1) {
            carry[0] = base + c;
            carry[1] = apos + (c > 0);
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        off[n_expert] = carry[0];
        *n_active = carry[1];
    }
    __syncthreads();
    for (int p = threadIdx.x; p < n_pairs; p += blockDim.x) {
        const int e = sid[p];
        if (e < 0 || e >= n_expert) continue;
        int r = 0;
        for (int q = 0; q < p; q++) r += sid[q] == e;
        pair[cnt[e] + r] = p;
    }
}

// ------------------------------------------------------------------ grouped GEMV
// Grid (expert slot, row block).  The workgroup of slot a serves expert
// active[a]: its LPR lanes per row stream each weight unit once per chunk of
// four pairs and dot it against every pair's activation.  FUSE: two banks
// (gate, up) and out = silu(g)*u; otherwise one bank and out = the dot.
struct GrpArgs {
    const uint8_t *w0, *w1;
    uint32_t w_bytes;   // bytes of one bank (all experts)
    size_t plane;       // bytes of one expert in a bank
    uint32_t row_bytes;
    int K, n_rows;
    const int32_t *off, *pair, *active, *n_active;
    const int8_t *x8;
    const float *xmeta;
    const int32_t *xsumq;
    int x_tb;    // tokens (rows) of the activation layout
    int tok_div; // activation row of pair p = p / tok_div
    float *out;
    int out_stride;
};

__device__ __forceinline__ void gload_x8(const int8_t *x8, int TB, int G, int t, uint32_t (&X)[8]) {
    const uint4 *p = reinterpret_cast<const uint4 *>(x8 + ((size_t)G * TB + t) * 32);
    const uint4 v0 = p[0], v1 = p[1];
    X[0] = v0.x; X[1] = v0.y; X[2] = v0.z; X[3] = v0.w;
    X[4] = v1.x; X[5] = v1.y; X[6] = v1.z; X[7] = v1.w;
}

// Raw bytes of one weight unit (miq_units.h) and their loader.
template <uint32_t TYPE> struct GRawOf;
template <> struct GRawOf<MIQ_TYPE_Q4_K> { using T = RawQ4K; };
template <> struct GRawOf<MIQ_TYPE_Q5_K> { using T = RawQ5K; };
template <> struct GRawOf<MIQ_TYPE_Q6_K> { using T = RawQ6K; };
template <> struct GRawOf<MIQ_TYPE_Q8_0> { using T = RawQ80; };

// unit u of the row starting at row_off (an out-of-range row_off reads zeros)
template <uint32_t TYPE>
__device__ __forceinline__ typename GRawOf<TYPE>::T grp_load(__amdgpu_buffer_rsrc_t rs, uint32_t row_off, int u) {
    if constexpr (TYPE == MIQ_TYPE_Q4_K) return load_q4k(rs, row_off + (uint32_t)(u >> 2) * kQ4KBytes, u & 3);
    else if constexpr (TYPE == MIQ_TYPE_Q5_K) return load_q5k(rs, row_off + (uint32_t)(u >> 2) * kQ5KBytes, u & 3);
    else if constexpr (TYPE == MIQ_TYPE_Q6_K) return load_q6k(rs, row_off + (uint32_t)(u >> 2) * kQ6KBytes, u & 3);
    else return load_q80(rs, row_off + (uint32_t)u * 68u);
}

// Dot one loaded unit against one activation row (token t of layout TB);
// returns the unit's fp32 contribution (the per-type epilogues of i8.cpp /
// q4exp.cpp).
template <uint32_t TYPE>
__device__ __forceinline__ float unit_term(const typename GRawOf<TYPE>::T &raw, int u, const int8_t *x8,
                                           const float *xmeta, const int32_t *xsumq, int TB, int t) {
    const float2 *xm = reinterpret_cast<const float2 *>(xmeta);
    const int2 *xs = reinterpret_cast<const int2 *>(xsumq);
    if constexpr (TYPE == MIQ_TYPE_Q4_K || TYPE == MIQ_TYPE_Q5_K) {
        const int b = u >> 2, c = u & 3, G0 = b * 8 + 2 * c, G1 = G0 + 1;
        uint32_t X0[8], X1[8];
        gload_x8(x8, TB, G0, t, X0);
        gload_x8(x8, TB, G1, t, X1);
        int wd0, wd1;
        if constexpr (TYPE == MIQ_TYPE_Q4_K) dots_q4k(raw, X0, X1, wd0, wd1);
        else dots_q5k(raw, c, X0, X1, wd0, wd1);
        const int2 s0 = xs[(size_t)G0 * TB + t], s1 = xs[(size_t)G1 * TB + t];
        return epi_kq45(raw.hdr, c, wd0, wd1, xm[(size_t)G0 * TB + t].x, xm[(size_t)G1 * TB + t].x, s0.x + s0.y,
                        s1.x + s1.y);
    } else if constexpr (TYPE == MIQ_TYPE_Q6_K) {
        const int b = u >> 2, c = u & 3, blk2 = c >> 1, half = c & 1;
        uint32_t Xf[4][8];
        const uint32_t *Xp[4];
#pragma unroll
        for (int p = 0; p < 4; p++) {
            gload_x8(x8, TB, b * 8 + blk2 * 4 + p, t, Xf[p]);
            Xp[p] = Xf[p] + 4 * half;
        }
        int wd[4];
        dots_q6k(raw, Xp, wd);
        const float d = h2f(raw.dbits);
        float s = 0.0f;
#pragma unroll
        for (int p = 0; p < 4; p++) {
            const size_t gi = (size_t)(b * 8 + blk2 * 4 + p) * TB + t;
            const int xsh = half ? xs[gi].y : xs[gi].x;
            s += xm[gi].x * (d * (float)q6k_scale(raw, c, p)) * (float)(wd[p] - 32 * xsh);
        }
        return s;
    } else {
        uint32_t X0[8], X1[8];
        gload_x8(x8, TB, 2 * u, t, X0);
        gload_x8(x8, TB, 2 * u + 1, t, X1);
        int wd0, wd1;
        dots_q80(raw, X0, X1, wd0, wd1);
        return xm[(size_t)(2 * u) * TB + t].x * h2f(raw.da) * (float)wd0 +
               xm[(size_t)(2 * u + 1) * TB + t].x * h2f(raw.db) * (float)wd1;
    }
}

__device__ __forceinline__ float silu_dev(float x) { return x / (1.0f + expf(-x)); }

// Workgroup (expert slot, row block); the slot serves expert active[slot].
// Each lane loads its NU weight units of the row (both banks when fused)
// once, then folds them against every pair of the expert in turn: an
// active expert's weights are read once for all of its pairs.
template <uint32_t TYPE, int LPR, int NU, bool FUSE>
__global__ __launch_bounds__(256) void grp_kernel(GrpArgs A) {
    // n_active and active[slot] are fetched together (active[] holds a valid
    // expert id or stale data past n_active, never read then); the weight
    // loads go out next and the pair range is fetched behind them
    const int slot = blockIdx.x;
    const int na = __builtin_nontemporal_load(A.n_active);
    const int e = __builtin_nontemporal_load(A.active + slot);
    if (slot >= na) return;
    constexpr int RPW = 64 / LPR;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int row = (blockIdx.y * 4 + wave) * RPW + lane / LPR;
    const int j = lane % LPR;
    const int U = A.K / 64;
    const __amdgpu_buffer_rsrc_t r0 = make_rsrc(A.w0, A.w_bytes);
    const __amdgpu_buffer_rsrc_t r1 = make_rsrc(FUSE ? A.w1 : A.w0, A.w_bytes);
    const bool row_ok = row < A.n_rows;
    const uint32_t row_off = row_ok ? (uint32_t)((size_t)e * A.plane) + (uint32_t)row * A.row_bytes : A.w_bytes;
    using Raw = typename GRawOf<TYPE>::T;
    Raw w0[NU], w1[NU];
#pragma unroll
    for (int i = 0; i < NU; i++) {
        const int u = j + i * LPR;
        const uint32_t ro = u < U ? row_off : A.w_bytes;
        w0[i] = grp_load<TYPE>(r0, ro, u < U ? u : 0);
        if constexpr (FUSE) w1[i] = grp_load<TYPE>(r1, ro, u < U ? u : 0);
    }
    const int p0 = A.off[e], P = A.off[e + 1] - p0;
    for (int pi = 0; pi < P; pi++) {
        const int p = A.pair[p0 + pi];
        const int tk = p / A.tok_div;
        float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
        for (int i = 0; i < NU; i++) {
            const int u = j + i * LPR;
            if (row_ok && u < U) {
                a0 += unit_term<TYPE>(w0[i], u, A.x8, A.xmeta, A.xsumq, A.x_tb, tk);
                if constexpr (FUSE) a1 += unit_term<TYPE>(w1[i], u, A.x8, A.xmeta, A.xsumq, A.x_tb, tk);
            }
        }
        a0 = seg_sum<LPR>(a0);
        if constexpr (FUSE) a1 = seg_sum<LPR>(a1);
        if (j == 0 && row_ok) A.out[(size_t)p * A.out_stride + row] = FUSE ? silu_dev(a0) * a1 : a0;
    }
}

static int pick_lpr_grp(int U) {
    for (int l : {16, 32, 8, 64, 4})
        if (U % l == 0 && U / l <= 8) return l;
    return 64;
}

template <uint32_t TYPE, int LPR, bool FUSE> static void launch_grp_l(hipStream_t s, const GrpArgs &A, int n_expert) {
    constexpr int rows_per_wg = 4 * (64 / LPR);
    const dim3 grid(n_expert, (A.n_rows + rows_per_wg - 1) / rows_per_wg);
    const int nu = (A.K / 64 + LPR - 1) / LPR;
    if (nu <= 1) hipLaunchKernelGGL((grp_kernel<TYPE, LPR, 1, FUSE>), grid, dim3(256), 0, s, A);
    else if (nu <= 2) hipLaunchKernelGGL((grp_kernel<TYPE, LPR, 2, FUSE>), grid, dim3(256), 0, s, A);
    else if (nu <= 4) hipLaunchKernelGGL((grp_kernel<TYPE, LPR, 4, FUSE>), grid, dim3(256), 0, s, A);
    else hipLaunchKernelGGL((grp_kernel<TYPE, LPR, 8, FUSE>), grid, dim3(256), 0, s, A);
}

template <uint32_t TYPE, bool FUSE> static void launch_grp_t(hipStream_t s, const GrpArgs &A, int n_expert) {
    switch (pick_lpr_grp(A.K / 64)) {
    case 4: launch_grp_l<TYPE, 4, FUSE>(s, A, n_expert); break;
    case 8: launch_grp_l<TYPE, 8, FUSE>(s, A, n_expert); break;
    case 16: launch_grp_l<TYPE, 16, FUSE>(s, A, n_expert); break;
    case 32: launch_grp_l<TYPE, 32, FUSE>(s, A, n_expert); break;
    default: launch_grp_l<TYPE, 64, FUSE>(s, A, n_expert); break;
    }
}

template <bool FUSE> static void launch_grp(hipStream_t s, uint32_t type, const GrpArgs &A, int n_expert) {
    switch (type) {
    case MIQ_TYPE_Q4_K: launch_grp_t<MIQ_TYPE_Q4_K, FUSE>(s, A, n_expert); break;
    case MIQ_TYPE_Q5_K: launch_grp_t<MIQ_TYPE_Q5_K, FUSE>(s, A, n_expert); break;
    case MIQ_TYPE_Q6_K: launch_grp_t<MIQ_TYPE_Q6_K, FUSE>(s, A, n_expert); break;
    default: launch_grp_t<MIQ_TYPE_Q8_0, FUSE>(s, A, n_expert); break;
    }
}

// ------------------------------------------------------------------ reduce
__global__ __launch_bounds__(256) void reduce_kernel(const float *__restrict__ acc, const float *__restrict__ wts,
                                                     int top_k, int n_tok, int n_embd, int acc_stride,
                                                     float *__restrict__ out, int out_stride) {
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long)n_tok * n_embd) return;
    const int t = (int)(i / n_embd), e = (int)(i % n_embd);
    double a = 0.0;
    for (int j = 0; j < top_k; j++) {
        const size_t pr = (size_t)t * top_k + j;
        a += (double)wts[pr] * (double)acc[pr * (size_t)acc_stride + e];
    }
    out[(size_t)t * out_stride + e] += (float)a;
}

// Pairs whose expert id is out of range are not in the CSR; their rows of acc
// are zero (the reference's per-pair path writes zeros for them, moe.cpp:359-364).
__global__ __launch_bounds__(256) void zero_invalid_kernel(const int32_t *__restrict__ ids, int n_pairs, int n_expert,
                                                           float *__restrict__ acc, int acc_stride, int n_embd) {
    const int p = blockIdx.x;
    const int e = ids[p];
    if (e >= 0 && e < n_expert) return;
    for (int r = threadIdx.x; r < n_embd; r += blockDim.x) acc[(size_t)p * acc_stride + r] = 0.0f;
}

// ------------------------------------------------------------------ workspace
struct MoeWs {
    int8_t *x8;
    float *xmeta;
    int32_t *xsumq;
    int32_t *off, *pair, *active, *n_active;
    float *h;
    int8_t *h8;
    float *hmeta;
    int32_t *hsumq;
    size_t bytes;
};

static size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

static MoeWs moe_ws_layout(const miq_moe *M, int n_tok, int top_k, uint8_t *base) {
    const size_t np = (size_t)n_tok * top_k;
    const size_t K = M->n_embd, F = M->n_ff;
    MoeWs w{};
    size_t o = 0;
    auto take = [&](size_t bytes) {
        uint8_t *p = base ? base + o : nullptr;
        o += align256(bytes);
        return p;
    };
    w.x8 = (int8_t *)take(K * n_tok);
    w.xmeta = (float *)take(K / 32 * n_tok * 8);
    w.xsumq = (int32_t *)take(K / 32 * n_tok * 8);
    w.off = (int32_t *)take(4 * (M->n_expert + 1));
    w.pair = (int32_t *)take(4 * np);
    w.active = (int32_t *)take(4 * M->n_expert);
    w.n_active = (int32_t *)take(4);
    w.h = (float *)take(4 * F * np);
    w.h8 = (int8_t *)take(F * np);
    w.hmeta = (float *)take(F / 32 * np * 8);
    w.hsumq = (int32_t *)take(F / 32 * np * 8);
    w.bytes = o;
    return w;
}

static int check_bank(uint32_t type, int K, const void *p, size_t plane, const char *who) {
    if (!p) {
        set_error("%s: null expert bank", who);
        return MIQ_EINVAL;
    }
    if (type != MIQ_TYPE_Q4_K && type != MIQ_TYPE_Q5_K && type != MIQ_TYPE_Q6_K && type != MIQ_TYPE_Q8_0) {
        set_error("%s: expert type %u is not on the integer path", who, type);
        return MIQ_UNSUPPORTED;
    }
    if (K % 64 || (type != MIQ_TYPE_Q8_0 && K % 256)) {
        set_error("%s: K=%d not a multiple of the block", who, K);
        return MIQ_UNSUPPORTED;
    }
    const uintptr_t a = (uintptr_t)p | (uintptr_t)plane;
    if ((type == MIQ_TYPE_Q4_K || type == MIQ_TYPE_Q5_K) ? (a & 15) : (type == MIQ_TYPE_Q8_0 ? (a & 3) : (a & 1))) {
        set_error("%s: bank pointer/plane misaligned for type %u", who, type);
        return MIQ_UNSUPPORTED;
    }
    return MIQ_OK;
}

}  // namespace miq

extern "C" {

int miq_moe_route(hipStream_t stream, const float *x, int x_stride, const float *gate_inp, int n_tok, int n_embd,
                  int n_expert, int top_k, float *logits, int32_t *ids, float *wts) {
    if (!logits || !ids || !wts || n_tok <= 0 || n_expert <= 0 || top_k <= 0 || top_k > n_expert ||
        (gate_inp && (!x || n_embd <= 0 || x_stride < n_embd))) {
        miq::set_error("miq_moe_route: bad arguments");
        return MIQ_EINVAL;
    }
    const size_t lds = (size_t)((n_expert + 3) & ~3) * 4;
    if (lds > 64 * 1024 || top_k > 64) {
        miq::set_error("miq_moe_route: n_expert=%d / top_k=%d too large", n_expert, top_k);
        return MIQ_UNSUPPORTED;
    }
    hipLaunchKernelGGL(miq::route_kernel, dim3(n_tok), dim3(256), lds, stream, x, x_stride, gate_inp, n_embd,
                       n_expert, top_k, logits, ids, wts);
    return miq::check_launch("miq_moe_route");
}

int miq_moe_csr(hipStream_t stream, const int32_t *ids, int n_pairs, int n_expert, int32_t *off, int32_t *pair,
                int32_t *active, int32_t *n_active) {
    if (!ids || !off || !pair || !active || !n_active || n_pairs <= 0 || n_expert <= 0) {
        miq::set_error("miq_moe_csr: bad arguments");
        return MIQ_EINVAL;
    }
    const size_t lds = (size_t)(n_expert + n_pairs) * 4;
    if (lds > 64 * 1024) {
        miq::set_error("miq_moe_csr: n_expert=%d + n_pairs=%d too large", n_expert, n_pairs);
        return MIQ_UNSUPPORTED;
    }
    hipLaunchKernelGGL(miq::csr_kernel, dim3(1), dim3(1024), lds, stream, ids, n_pairs, n_expert, off, pair, active,
                       n_active);
    return miq::check_launch("miq_moe_csr");
}

size_t miq_moe_workspace_bytes(const miq_moe *M, int n_tok, int top_k) {
    if (!M || n_tok <= 0 || top_k <= 0) return 0;
    return miq::moe_ws_layout(M, n_tok, top_k, nullptr).bytes;
}

int miq_moe_experts(hipStream_t stream, const miq_moe *M, const float *x, int x_stride, int n_tok, int top_k,
                    const int32_t *ids, float *acc, int acc_stride, void *workspace, size_t workspace_bytes) {
    using namespace miq;
    if (!M || !x || !ids || !acc || !workspace || n_tok <= 0 || top_k <= 0 || M->n_embd <= 0 || M->n_ff <= 0 ||
        M->n_expert <= 0 || x_stride < M->n_embd || acc_stride < M->n_embd) {
        set_error("miq_moe_experts: bad arguments");
        return MIQ_EINVAL;
    }
    int rc;
    if ((rc = check_bank(M->gate_type, M->n_embd, M->gate, M->gate_plane, "miq_moe_experts gate")) ||
        (rc = check_bank(M->up_type, M->n_embd, M->up, M->up_plane, "miq_moe_experts up")) ||
        (rc = check_bank(M->down_type, M->n_ff, M->down, M->down_plane, "miq_moe_experts down")))
        return rc;
    if (M->n_embd / 64 > 512 || M->n_ff / 64 > 512) {  // the grouped kernel holds at most 8 units per lane
        set_error("miq_moe_experts: n_embd / n_ff above 32768");
        return MIQ_UNSUPPORTED;
    }
    if (M->gate_type != M->up_type || M->gate_plane != M->up_plane) {
        set_error("miq_moe_experts: gate and up banks must share type and plane size");
        return MIQ_UNSUPPORTED;
    }
    const size_t gbytes = M->gate_plane * M->n_expert, dbytes = M->down_plane * M->n_expert;
    if (gbytes >= (1ull << 32) || dbytes >= (1ull << 32)) {
        set_error("miq_moe_experts: expert bank exceeds the 4 GiB buffer window");
        return MIQ_UNSUPPORTED;
    }
    if (((uintptr_t)workspace & 255) || ((uintptr_t)x & 15) || (x_stride & 3)) {
        set_error("miq_moe_experts: workspace must be 256-byte aligned, x 16-byte aligned with stride %% 4");
        return MIQ_UNSUPPORTED;
    }
    const MoeWs w = moe_ws_layout(M, n_tok, top_k, (uint8_t *)workspace);
    if (workspace_bytes < w.bytes) {
        set_error("miq_moe_experts: workspace %zu < %zu bytes", workspace_bytes, w.bytes);
        return MIQ_EINVAL;
    }
    const int np = n_tok * top_k;
    if ((rc = miq_moe_csr(stream, ids, np, M->n_expert, w.off, w.pair, w.active, w.n_active))) return rc;
    if ((rc = launch_xq(stream, x, nullptr, x_stride, 0, w.x8, w.xmeta, w.xsumq, n_tok, M->n_embd))) return rc;
    GrpArgs A{};
    A.w0 = (const uint8_t *)M->gate;
    A.w1 = (const uint8_t *)M->up;
    A.w_bytes = (uint32_t)gbytes;
    A.plane = M->gate_plane;
    A.row_bytes = (uint32_t)miq_row_bytes(M->gate_type, M->n_embd);
    A.K = M->n_embd;
    A.n_rows = M->n_ff;
    A.off = w.off;
    A.pair = w.pair;
    A.active = w.active;
    A.n_active = w.n_active;
    A.x8 = w.x8;
    A.xmeta = w.xmeta;
    A.xsumq = w.xsumq;
    A.x_tb = n_tok;
    A.tok_div = top_k;
    A.out = w.h;
    A.out_stride = M->n_ff;
    launch_grp<true>(stream, M->gate_type, A, M->n_expert);
    if ((rc = check_launch("miq_moe_experts gate/up"))) return rc;
    if ((rc = launch_xq(stream, w.h, nullptr, M->n_ff, 0, w.h8, w.hmeta, w.hsumq, np, M->n_ff))) return rc;
    GrpArgs D = A;
    D.w0 = D.w1 = (const uint8_t *)M->down;
    D.w_bytes = (uint32_t)dbytes;
    D.plane = M->down_plane;
    D.row_bytes = (uint32_t)miq_row_bytes(M->down_type, M->n_ff);
    D.K = M->n_ff;
    D.n_rows = M->n_embd;
    D.x8 = w.h8;
    D.xmeta = w.hmeta;
    D.xsumq = w.hsumq;
    D.x_tb = np;
    D.tok_div = 1;
    D.out = acc;
    D.out_stride = acc_stride;
    launch_grp<false>(stream, M->down_type, D, M->n_expert);
    if ((rc = check_launch("miq_moe_experts down"))) return rc;
    hipLaunchKernelGGL(zero_invalid_kernel, dim3(np), dim3(256), 0, stream, ids, np, M->n_expert, acc, acc_stride,
                       M->n_embd);
    return check_launch("miq_moe_experts zero");
}

int miq_moe_reduce(hipStream_t stream, const float *acc, const float *wts, int top_k, int n_tok, int n_embd,
                   int acc_stride, float *out, int out_stride) {
    if (!acc || !wts || !out || top_k <= 0 || n_tok <= 0 || n_embd <= 0 || acc_stride < n_embd ||
        out_stride < n_embd) {
        miq::set_error("miq_moe_reduce: bad arguments");
        return MIQ_EINVAL;
    }
    const long n = (long)n_tok * n_embd;
    hipLaunchKernelGGL(miq::reduce_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, acc, wts, top_k,
                       n_tok, n_embd, acc_stride, out, out_stride);
    return miq::check_launch("miq_moe_reduce");
}

}  // extern "C"
