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
#include <type_traits>

#include "miq_internal.h"
#include "miq_units.h"
#include "miq_xq.h"

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
    __shared__ int sids[64], sord[64];  // the selected experts by rank / by id (top_k <= 64)
    const int t = blockIdx.x;
    const int ne4 = (n_expert + 3) & ~3;
    float *lg = logits + (size_t)t * n_expert;
    if (gate_inp) {
        // one thread per expert: the reference's F32 router dot (moe.cpp:84-88),
        // a serial double-precision sum in k order.  Each product of two floats
        // is exact in double, so every partial sum rounds as the reference's
        // does and the logit is its value bit for bit.
        const float *xr = x + (size_t)t * x_stride;
        for (int e = threadIdx.x; e < n_expert; e += blockDim.x) {
            const float *w = gate_inp + (size_t)e * n_embd;
            double a = 0.0;
            for (int k = 0; k < n_embd; k++) a += (double)w[k] * (double)xr[k];
            lg[e] = (float)a;
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
    for (int e = threadIdx.x; e < ne4; e += blockDim.x) sp[e] = e < n_expert ? expf_libm(sp[e] - mx) : 0.0f;
    __syncthreads();
    if (threadIdx.x == 0) {
        // expert order; sixteen LDS reads in flight ahead of the dependent adds
        float sum = 0.f;
        const float4 *s4 = reinterpret_cast<const float4 *>(sp);
        const int nq = ne4 / 4;
        int q = 0;
        for (; q + 16 <= nq; q += 16) {
            float4 v[16];
#pragma unroll
            for (int i = 0; i < 16; i++) v[i] = s4[q + i];
#pragma unroll
            for (int i = 0; i < 16; i++) {
                sum += v[i].x;
                sum += v[i].y;
                sum += v[i].z;
                sum += v[i].w;
            }
        }
        for (; q < nq; q++) {
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
    // the logits scratch ends holding the probabilities, as in cpu_moe_route;
    // each thread rescales only its own entries, so one barrier covers both
    for (int e = threadIdx.x; e < ne4; e += blockDim.x) {
        const float pr = sp[e] * inv;
        sp[e] = pr;
        if (e < n_expert) lg[e] = pr;
    }
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
    // the selected ids in increasing order: each goes to the slot given by how
    // many selected ids are smaller (ids are distinct)
    for (int r = threadIdx.x; r < top_k; r += blockDim.x) {
        const int e = sids[r];
        int pos = 0;
        for (int q = 0; q < top_k; q++) pos += sids[q] < e;
        sord[pos] = e;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float wsum = 0.f;  // sum of the selected, in expert order
        for (int i = 0; i < top_k; i++) wsum += sp[sord[i]];
        s_den = fmaxf(wsum, 6.103515625e-5f);
    }
    __syncthreads();
    for (int r = threadIdx.x; r < top_k; r += blockDim.x) wts[(size_t)t * top_k + r] = sp[sids[r]] / s_den;
}

// Router over given logits, one wave per token with V = ceil(n_expert/64)
// experts per lane (lane l holds experts l*V .. l*V+V-1, so walking lanes
// then slots is expert order).  Same arithmetic as route_kernel:
//   max by a wave tree (order-free); p = expf_libm(l - max); the softmax sum and
//   the sum of the selected run strictly in expert order (one lane value at a
//   time, broadcast by readlane); the top_k are taken by k rounds of a wave
//   argmax of (probability, lowest index) -- the order rank counting gives.
template <int R> __device__ __forceinline__ int row_ror(int v) {
    return __builtin_amdgcn_update_dpp(0, v, 0x120 + R, 0xF, 0xF, false);
}
template <int R> __device__ __forceinline__ float row_ror(float v) {
    return __builtin_bit_cast(float, row_ror<R>(__builtin_bit_cast(int, v)));
}

// Top-k order as one unsigned 64-bit key: a probability p >= 0 above every
// smaller one, the lower expert index first among equal p.  The high word is
// p's bits + 1 (the bits of non-negative floats order as the values), the low
// word ~index; a taken or padding slot holds key 0 (below every expert).  A
// NaN probability (from a NaN logit; the caller's logits must be finite) gets
// the high word 0, below every number: the token's ids are then unspecified,
// as in the reference.
__device__ __forceinline__ uint64_t topk_key(float p, int e) {
    const uint32_t hi = p >= 0.0f ? (__builtin_bit_cast(uint32_t, p) & 0x7FFFFFFFu) + 1u : 0u;  // -0 as +0
    return ((uint64_t)hi << 32) | (uint32_t)~e;
}
__device__ __forceinline__ uint64_t umax64(uint64_t a, uint64_t b) { return a > b ? a : b; }
template <int R> __device__ __forceinline__ uint64_t row_ror64(uint64_t v) {
    return ((uint64_t)(uint32_t)row_ror<R>((int)(v >> 32)) << 32) | (uint32_t)row_ror<R>((int)(uint32_t)v);
}
// Wave max of the keys, branch-free: rotations inside each 16-lane row
// (DPP row_ror 8, 4, 2, 1) leave every lane with its row's maximum; a
// permlane32 swap then a permlane16 swap fold the four rows.  Max is
// commutative and associative, so every lane ends with the same key.
__device__ __forceinline__ uint64_t wave_max_key(uint64_t k) {
    k = umax64(k, row_ror64<8>(k));
    k = umax64(k, row_ror64<4>(k));
    k = umax64(k, row_ror64<2>(k));
    k = umax64(k, row_ror64<1>(k));
    uint32_t lo = (uint32_t)k, hi = (uint32_t)(k >> 32);
    const auto l32 = __builtin_amdgcn_permlane32_swap(lo, lo, false, false);
    const auto h32 = __builtin_amdgcn_permlane32_swap(hi, hi, false, false);
    k = umax64(((uint64_t)h32[0] << 32) | l32[0], ((uint64_t)h32[1] << 32) | l32[1]);
    lo = (uint32_t)k;
    hi = (uint32_t)(k >> 32);
    const auto l16 = __builtin_amdgcn_permlane16_swap(lo, lo, false, false);
    const auto h16 = __builtin_amdgcn_permlane16_swap(hi, hi, false, false);
    return umax64(((uint64_t)h16[0] << 32) | l16[0], ((uint64_t)h16[1] << 32) | l16[1]);
}

__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, row_ror<8>(v));
    v = fmaxf(v, row_ror<4>(v));
    v = fmaxf(v, row_ror<2>(v));
    v = fmaxf(v, row_ror<1>(v));
    const int b = __builtin_bit_cast(int, v);
    return fmaxf(fmaxf(__builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 0)),
                       __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 16))),
                 fmaxf(__builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 32)),
                       __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 48))));
}

__device__ __forceinline__ float lane_f(float v, int l) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}

// LDS of route_block for a workgroup of `waves` waves
static constexpr size_t route_lds_bytes(int V, int waves) { return ((size_t)waves * (64 * V + 1) + 64) * 4; }

// Router over given logits for tokens t0 .. t0+nt-1 of one workgroup (nt at
// most its waves), wave w taking token t0+w with V = ceil(n_expert/64) experts
// per lane (lane l holds experts l*V .. l*V+V-1, so walking lanes then slots is
// expert order).  Same arithmetic as route_kernel:
//   max by a wave tree (order-free); p = expf_libm(l - max); the softmax sum runs
//   strictly in expert order -- on one lane of wave 0 per token, over the
//   exps staged in LDS (sp: rows of 64V+1 floats, the pad keeps the tokens'
//   rows on distinct banks), so the sixteen tokens' sums run side by side;
//   the top_k are taken by k rounds of a wave max of (probability, lowest
//   index) keys -- the order rank counting gives; their sum runs in
//   increasing id.
// Every thread of the workgroup calls it (two barriers).
template <int V>
__device__ __forceinline__ void route_block(int t0, int nt, int n_expert, int top_k, float *__restrict__ logits,
                                           int32_t *__restrict__ ids, float *__restrict__ wts, float *sp) {
    constexpr int RS = 64 * V + 1;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    float *ssum = sp + (blockDim.x >> 6) * RS;
    const bool mine = w < nt;
    const int t = t0 + w;
    float *lg = logits + (size_t)t * n_expert;
    float pv[V];
    if (mine) {
        float mx = -3.402823466e38f;
#pragma unroll
        for (int i = 0; i < V; i++) {
            const int e = lane * V + i;
            pv[i] = e < n_expert ? lg[e] : -3.402823466e38f;
            mx = fmaxf(mx, pv[i]);
        }
        mx = wave_max(mx);
#pragma unroll
        for (int i = 0; i < V; i++) {
            pv[i] = lane * V + i < n_expert ? expf_libm(pv[i] - mx) : 0.0f;
            sp[w * RS + lane * V + i] = pv[i];
        }
    }
    __syncthreads();
    if (w == 0 && lane < nt) {
        // the whole padded row (entries past n_expert hold +0, which leaves a
        // sum of positive terms unchanged), read 16 entries ahead of the adds
        // so the chain waits on the adds, not on one LDS latency per entry
        float sum = 0.f;
        const float *row = sp + lane * RS;
        float cur[16], nxt[16];
#pragma unroll
        for (int j = 0; j < 16; j++) cur[j] = row[j];
#pragma unroll
        for (int e0 = 0; e0 < 64 * V; e0 += 16) {
            if (e0 + 16 < 64 * V)
#pragma unroll
                for (int j = 0; j < 16; j++) nxt[j] = row[e0 + 16 + j];
#pragma unroll
            for (int j = 0; j < 16; j++) sum += cur[j];
#pragma unroll
            for (int j = 0; j < 16; j++) cur[j] = nxt[j];
        }
        ssum[lane] = sum;
    }
    __syncthreads();
    if (mine) {
        const float inv = 1.f / ssum[w];
#pragma unroll
        for (int i = 0; i < V; i++) {
            const int e = lane * V + i;
            pv[i] *= inv;
            if (e < n_expert) lg[e] = pv[i];
        }
        uint64_t key[V];
#pragma unroll
        for (int i = 0; i < V; i++) key[i] = lane * V + i < n_expert ? topk_key(pv[i], lane * V + i) : 0;
        int my_id = 0x7fffffff;
        float my_w = 0.0f;
        for (int r = 0; r < top_k; r++) {
            uint64_t best = key[0];
#pragma unroll
            for (int i = 1; i < V; i++) best = umax64(best, key[i]);
            best = wave_max_key(best);
            const int bi = (int)~(uint32_t)best;
#pragma unroll
            for (int i = 0; i < V; i++)
                if (lane * V + i == bi) key[i] = 0;  // taken
            if (lane == r) {
                my_id = bi;
                my_w = __builtin_bit_cast(float, (uint32_t)(best >> 32) - 1u);
            }
        }
        // lane r < top_k holds the r-th pick; its place in increasing id order
        int pos = 0;
        for (int q = 0; q < top_k; q++) pos += __builtin_amdgcn_readlane(my_id, q) < my_id;
        float wsum = 0.f;
        for (int j = 0; j < top_k; j++) {
            const uint64_t m = __ballot(lane < top_k && pos == j);
            wsum += lane_f(my_w, (int)__builtin_ctzll(m));
        }
        const float den = fmaxf(wsum, 6.103515625e-5f);
        if (lane < top_k) {
            ids[(size_t)t * top_k + lane] = my_id;
            wts[(size_t)t * top_k + lane] = my_w / den;
        }
    }
}

// One workgroup of four waves per four tokens.
template <int V>
__global__ __launch_bounds__(256) void route_wave_kernel(int n_tok, int n_expert, int top_k,
                                                         float *__restrict__ logits, int32_t *__restrict__ ids,
                                                         float *__restrict__ wts) {
    extern __shared__ float rsm[];
    const int t0 = blockIdx.x * 4;
    route_block<V>(t0, min(4, n_tok - t0), n_expert, top_k, logits, ids, wts, rsm);
}

// ------------------------------------------------------------------ CSR
// One workgroup (1024 threads for miq_moe_csr, 512 in the experts' set-up
// kernel; any multiple of 64 up to 1024): ids staged in LDS, counts by LDS atomics,
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

__device__ __forceinline__ void csr_block(const int32_t *__restrict__ ids, int n_pairs, int n_expert,
                                          int32_t *__restrict__ off, int32_t *__restrict__ pair,
                                          int32_t *__restrict__ active, int32_t *__restrict__ n_active, int *sm) {
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
    // exclusive scans of the counts (offsets) and of the active flags, 1024
    // experts at a time, as one scan of count | flag << 16 (both sums stay
    // below 2^16: n_pairs and n_expert are bounded by the LDS they use)
    for (int e0 = 0; e0 < n_expert; e0 += blockDim.x) {
        const int e = e0 + threadIdx.x;
        const int c = e < n_expert ? cnt[e] : 0;
        const int both = block_scan1024(c | ((c > 0) << 16), tmp);
        const int incl = both & 0xFFFF, aincl = both >> 16;
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
    // a pair's rank among the earlier pairs of its expert, counted by C
    // adjacent lanes per pair (each over a slice of the earlier pairs, eight
    // LDS reads per batch) and summed across them
    int C = 1;
    while (C < 64 && C * 2 * n_pairs <= (int)blockDim.x) C *= 2;
    const int per = (n_pairs + C - 1) / C;
    for (int k0 = 0; k0 < n_pairs * C; k0 += blockDim.x) {
        const int k = k0 + threadIdx.x, p = k / C, c = k % C;
        const int e = p < n_pairs ? sid[p] : -1;
        int r = 0;
        if (p < n_pairs) {
            const int q1 = min(p, (c + 1) * per);
            int q = c * per;
            for (; q + 8 <= q1; q += 8) {
                int a[8];
#pragma unroll
                for (int j = 0; j < 8; j++) a[j] = sid[q + j];
#pragma unroll
                for (int j = 0; j < 8; j++) r += a[j] == e;
            }
            for (; q < q1; q++) r += sid[q] == e;
        }
        for (int o = 1; o < C; o <<= 1) r += __shfl_xor(r, o, 64);
        if (c == 0 && e >= 0 && e < n_expert) pair[cnt[e] + r] = p;
    }
}

__global__ __launch_bounds__(1024) void csr_kernel(const int32_t *__restrict__ ids, int n_pairs, int n_expert,
                                                   int32_t *__restrict__ off, int32_t *__restrict__ pair,
                                                   int32_t *__restrict__ active, int32_t *__restrict__ n_active) {
    extern __shared__ int sm[];
    csr_block(ids, n_pairs, n_expert, off, pair, active, n_active, sm);
}

// The MoE set-up in one launch: workgroup 0 builds the CSR and zeroes the acc
// rows of pairs whose expert id is out of range (they are in no expert's
// list; the reference's per-pair path writes zeros for them,
// moe.cpp:359-364); the other workgroups quantize the tokens' activations.
struct PrepArgs {
    const int32_t *ids;
    int n_pairs, n_expert;
    int32_t *off, *pair, *active, *n_active;
    float *acc;
    int acc_stride, n_embd;
    const float *x;
    int x_stride;
    int8_t *x8;
    float *xmeta;
    int32_t *xsumq;
    int n_tok, G;
};

template <int LAYOUT> __global__ __launch_bounds__(512) void moe_prep_kernel(PrepArgs P) {
    extern __shared__ int sm[];
    if (blockIdx.x == 0) {
        csr_block(P.ids, P.n_pairs, P.n_expert, P.off, P.pair, P.active, P.n_active, sm);
        const int lane = threadIdx.x & 63;
        for (int p = threadIdx.x >> 6; p < P.n_pairs; p += blockDim.x / 64) {  // a wave per pair
            const int e = sm[P.n_expert + p];  // the ids, staged in LDS by csr_block
            if (e >= 0 && e < P.n_expert) continue;
            for (int r = lane; r < P.n_embd; r += 64) P.acc[(size_t)p * P.acc_stride + r] = 0.0f;
        }
        return;
    }
    const int gid = (blockIdx.x - 1) * blockDim.x + threadIdx.x;
    if (gid < P.n_tok * P.G)
        xq_one<LAYOUT>(P.x, nullptr, P.x_stride, 0, P.x8, P.xmeta, P.xsumq, P.n_tok, P.G, gid);
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

// Activation of one weight unit for one token (layout TB, token t): the
// int8 codes the unit's groups meet, their scales sx and their code sums
// (xsumq holds the two 16-halves of each 32-group).
template <uint32_t TYPE> struct XU {
    uint4 a0, a1, b0, b1;  // groups G0, G1 (8 dwords each)
    float s0, s1;
    int2 q0, q1;
};
template <> struct XU<MIQ_TYPE_Q6_K> {
    uint4 a[4];  // the unit's half (4 dwords) of each of its four groups
    float s[4];
    int q[4];    // xsum of that half
};

template <uint32_t TYPE>
__device__ __forceinline__ XU<TYPE> load_xu(const int8_t *x8, const float *xmeta, const int32_t *xsumq, int TB, int u,
                                            int t) {
    XU<TYPE> x;
    if constexpr (TYPE == MIQ_TYPE_Q6_K) {
        const int b = u >> 2, c = u & 3, blk2 = c >> 1, half = c & 1;
#pragma unroll
        for (int p = 0; p < 4; p++) {
            const size_t gi = (size_t)(b * 8 + blk2 * 4 + p) * TB + t;
            x.a[p] = *reinterpret_cast<const uint4 *>(x8 + gi * 32 + half * 16);
            x.s[p] = xmeta[2 * gi];
            x.q[p] = xsumq[2 * gi + half];
        }
    } else {
        const int G0 = TYPE == MIQ_TYPE_Q8_0 ? 2 * u : (u >> 2) * 8 + 2 * (u & 3);
        const size_t g0 = (size_t)G0 * TB + t, g1 = g0 + TB;
        const uint4 *p0 = reinterpret_cast<const uint4 *>(x8 + g0 * 32);
        const uint4 *p1 = reinterpret_cast<const uint4 *>(x8 + g1 * 32);
        x.a0 = p0[0];
        x.a1 = p0[1];
        x.b0 = p1[0];
        x.b1 = p1[1];
        x.s0 = xmeta[2 * g0];
        x.s1 = xmeta[2 * g1];
        if constexpr (TYPE != MIQ_TYPE_Q8_0) {
            x.q0 = reinterpret_cast<const int2 *>(xsumq)[g0];
            x.q1 = reinterpret_cast<const int2 *>(xsumq)[g1];
        }
    }
    return x;
}

// fp32 contribution of one decoded unit against its activation (the per-type
// epilogues of i8.cpp / q4exp.cpp)
template <uint32_t TYPE>
__device__ __forceinline__ float term_xu(const typename GRawOf<TYPE>::T &raw, int u, const XU<TYPE> &x) {
    if constexpr (TYPE == MIQ_TYPE_Q6_K) {
        const int c = u & 3;
        const uint32_t X[4][4] = {{x.a[0].x, x.a[0].y, x.a[0].z, x.a[0].w},
                                  {x.a[1].x, x.a[1].y, x.a[1].z, x.a[1].w},
                                  {x.a[2].x, x.a[2].y, x.a[2].z, x.a[2].w},
                                  {x.a[3].x, x.a[3].y, x.a[3].z, x.a[3].w}};
        const uint32_t *Xp[4] = {X[0], X[1], X[2], X[3]};
        int wd[4];
        dots_q6k(raw, Xp, wd);
        const float d = h2f(raw.dbits);
        float s = 0.0f;
#pragma unroll
        for (int p = 0; p < 4; p++) s += x.s[p] * (d * (float)q6k_scale(raw, c, p)) * (float)(wd[p] - 32 * x.q[p]);
        return s;
    } else {
        const uint32_t X0[8] = {x.a0.x, x.a0.y, x.a0.z, x.a0.w, x.a1.x, x.a1.y, x.a1.z, x.a1.w};
        const uint32_t X1[8] = {x.b0.x, x.b0.y, x.b0.z, x.b0.w, x.b1.x, x.b1.y, x.b1.z, x.b1.w};
        int wd0, wd1;
        if constexpr (TYPE == MIQ_TYPE_Q8_0) {
            dots_q80(raw, X0, X1, wd0, wd1);
            return x.s0 * h2f(raw.da) * (float)wd0 + x.s1 * h2f(raw.db) * (float)wd1;
        } else {
            if constexpr (TYPE == MIQ_TYPE_Q4_K) dots_q4k(raw, X0, X1, wd0, wd1);
            else dots_q5k(raw, u & 3, X0, X1, wd0, wd1);
            return epi_kq45(raw.hdr, u & 3, wd0, wd1, x.s0, x.s1, x.q0.x + x.q0.y, x.q1.x + x.q1.y);
        }
    }
}

// The same activation read from the token-major unit layout (xq LAYOUT 1 for
// Q4_K/Q5_K/Q8_0 units, 2 for Q6_K units): token t's row is K bytes of codes
// with chunk k of unit u at (k*U + u)*16, then per-unit meta.  Lanes holding
// consecutive units read consecutive 16-byte words.
template <uint32_t TYPE>
__device__ __forceinline__ XU<TYPE> load_xv(const int8_t *x8, const float *xmeta, int K, int u, int t) {
    const int U = K / 64;
    const uint4 *row = reinterpret_cast<const uint4 *>(x8 + (size_t)t * K);
    XU<TYPE> x;
    if constexpr (TYPE == MIQ_TYPE_Q6_K) {
#pragma unroll
        for (int k = 0; k < 4; k++) x.a[k] = row[k * U + u];
        const uint4 *m = reinterpret_cast<const uint4 *>(xmeta) + ((size_t)t * U + u) * 2;
        const uint4 m0 = m[0], m1 = m[1];
        x.s[0] = __uint_as_float(m0.x);
        x.s[1] = __uint_as_float(m0.y);
        x.s[2] = __uint_as_float(m0.z);
        x.s[3] = __uint_as_float(m0.w);
        x.q[0] = (int)m1.x;
        x.q[1] = (int)m1.y;
        x.q[2] = (int)m1.z;
        x.q[3] = (int)m1.w;
    } else {
        x.a0 = row[u];
        x.a1 = row[U + u];
        x.b0 = row[2 * U + u];
        x.b1 = row[3 * U + u];
        const uint4 m = reinterpret_cast<const uint4 *>(xmeta)[(size_t)t * U + u];
        x.s0 = __uint_as_float(m.x);
        x.s1 = __uint_as_float(m.y);
        x.q0 = make_int2((int)m.z, 0);
        x.q1 = make_int2((int)m.w, 0);
    }
    return x;
}

template <uint32_t TYPE>
__device__ __forceinline__ float unit_term(const typename GRawOf<TYPE>::T &raw, int u, const int8_t *x8,
                                           const float *xmeta, const int32_t *xsumq, int TB, int t) {
    return term_xu<TYPE>(raw, u, load_xu<TYPE>(x8, xmeta, xsumq, TB, u, t));
}

__device__ __forceinline__ float silu_dev(float x) { return x / (1.0f + expf_libm(-x)); }

// ---- gate/up in the reference's fp32 order (Q4_K / Q5_K)
//
// h = silu(g)*u is requantised before the down projection, so its codes are
// bytes of the result: g and u must be the reference's fp32 values bit for bit,
// not merely close.  i8_row (i8.cpp:40-61, 96-121, 157-190) forms, per group,
// T = d*sc*wd - dmin*m*xsum (the compiled reference contracts it to one fma of
// (d*sc, wd) minus the rounded (dmin*m)*xsum), the block partial
// acc = fma(xm_g, T_g, acc) over groups 0..7 in order from 0, and the row as the
// block partials added in block order from 0.  Here lane c of a block's quad
// holds groups 2c, 2c+1: the partial runs down the quad by DPP, and the quads'
// partials meet in LDS where the row's first lane adds them in block order.
template <uint32_t TYPE>
__device__ __forceinline__ void ref_group_terms(const typename GRawOf<TYPE>::T &raw, int u, const XU<TYPE> &x, float &T0,
                                                float &T1) {
    const uint32_t X0[8] = {x.a0.x, x.a0.y, x.a0.z, x.a0.w, x.a1.x, x.a1.y, x.a1.z, x.a1.w};
    const uint32_t X1[8] = {x.b0.x, x.b0.y, x.b0.z, x.b0.w, x.b1.x, x.b1.y, x.b1.z, x.b1.w};
    const int c = u & 3;
    int wd0, wd1;
    if constexpr (TYPE == MIQ_TYPE_Q4_K) dots_q4k(raw, X0, X1, wd0, wd1);
    else dots_q5k(raw, c, X0, X1, wd0, wd1);
    const float d = h2f(raw.hdr.x), dm = h2f(raw.hdr.x >> 16);
    int sc0, m0, sc1, m1;
    scale_min_k4(2 * c, raw.hdr.y, raw.hdr.z, raw.hdr.w, sc0, m0);
    scale_min_k4(2 * c + 1, raw.hdr.y, raw.hdr.z, raw.hdr.w, sc1, m1);
    T0 = __builtin_fmaf(d * (float)sc0, (float)wd0, -((dm * (float)m0) * (float)(x.q0.x + x.q0.y)));
    T1 = __builtin_fmaf(d * (float)sc1, (float)wd1, -((dm * (float)m1) * (float)(x.q1.x + x.q1.y)));
}

// The block partial down a quad: lane c adds its groups after lane c-1's;
// lane 3 ends with fma(xm7, T7, ... fma(xm0, T0, 0)).
__device__ __forceinline__ float quad_block_chain(float xm0, float T0, float xm1, float T1, int c) {
    float v = 0.0f;
#pragma unroll
    for (int step = 0; step < 4; step++) {
        // quad_perm [0,0,1,2]: lane c reads lane c-1 (lane 0 its own, replaced by 0)
        const float prev = __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x90, 0xF, 0xF, false));
        const float in = c == 0 ? 0.0f : prev;
        if (c == step) v = __builtin_fmaf(xm1, T1, __builtin_fmaf(xm0, T0, in));
    }
    return v;
}

// Q6_K (i8.cpp:125-155): the block partial is fma(wd_s - 32*xsum_s, (d*sc_s)*xm_s, acc)
// over the 16 sub-groups s in value order; sub-group s = 8*blk2 + 2p + half
// sits in lane 2*blk2 + half of the quad (plane p of that lane's unit), so the
// chain alternates between the quad's lanes.
__device__ __forceinline__ float quad_block_chain_q6k(const float (&P)[4], const float (&V)[4], int c) {
    float v = 0.0f;
#pragma unroll
    for (int s = 0; s < 16; s++) {
        const int owner = 2 * (s >> 3) + (s & 1), prev = s ? 2 * ((s - 1) >> 3) + ((s - 1) & 1) : 0;
        // quad_perm [prev, prev, prev, prev]: every lane reads the previous step's lane
        const int vi = __builtin_bit_cast(int, v);
        const int pv = prev == 0   ? __builtin_amdgcn_mov_dpp(vi, 0x00, 0xF, 0xF, false)
                       : prev == 1 ? __builtin_amdgcn_mov_dpp(vi, 0x55, 0xF, 0xF, false)
                       : prev == 2 ? __builtin_amdgcn_mov_dpp(vi, 0xAA, 0xF, 0xF, false)
                                   : __builtin_amdgcn_mov_dpp(vi, 0xFF, 0xF, 0xF, false);
        const float in = s ? __builtin_bit_cast(float, pv) : 0.0f;
        const int p = (s & 7) >> 1;
        if (c == owner) v = __builtin_fmaf(V[p], P[p], in);
    }
    return v;  // lane 3 (sub-group 15) ends with the block partial
}

// The block partial of this lane's quad for one bank, in the reference's
// order, ending in lane 3 of the quad (zero terms for a dead lane).
template <uint32_t TYPE>
__device__ __forceinline__ float ref_block_partial(const typename GRawOf<TYPE>::T &raw, int u, const XU<TYPE> &x, bool live) {
    if constexpr (TYPE == MIQ_TYPE_Q6_K) {
        float P[4] = {0, 0, 0, 0}, V[4] = {0, 0, 0, 0};
        if (live) {
            const int c = u & 3;
            const uint32_t X[4][4] = {{x.a[0].x, x.a[0].y, x.a[0].z, x.a[0].w},
                                      {x.a[1].x, x.a[1].y, x.a[1].z, x.a[1].w},
                                      {x.a[2].x, x.a[2].y, x.a[2].z, x.a[2].w},
                                      {x.a[3].x, x.a[3].y, x.a[3].z, x.a[3].w}};
            const uint32_t *Xp[4] = {X[0], X[1], X[2], X[3]};
            int wd[4];
            dots_q6k(raw, Xp, wd);
            const float d = h2f(raw.dbits);
#pragma unroll
            for (int p = 0; p < 4; p++) {
                P[p] = ((float)q6k_scale(raw, c, p) * d) * x.s[p];
                V[p] = (float)(wd[p] - 32 * x.q[p]);
            }
        }
        return quad_block_chain_q6k(P, V, u & 3);
    } else {
        float T0 = 0.0f, T1 = 0.0f;
        if (live) ref_group_terms<TYPE>(raw, u, x, T0, T1);
        return quad_block_chain(live ? x.s0 : 0.0f, T0, live ? x.s1 : 0.0f, T1, u & 3);
    }
}

template <uint32_t TYPE> constexpr bool ref_order() {
    return TYPE == MIQ_TYPE_Q4_K || TYPE == MIQ_TYPE_Q5_K || TYPE == MIQ_TYPE_Q6_K;
}

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
    // gate/up in the reference's order: block partials of this wave's rows,
    // [row in wave][block][gate, up] (at most 16 * NU blocks per wave)
    __shared__ float rchain[4][16 * NU][2];
    for (int pi = 0; pi < P; pi++) {
        const int p = A.pair[p0 + pi];
        const int tk = p / A.tok_div;
        if constexpr (FUSE && ref_order<TYPE>()) {
            const int nbr = LPR / 4;  // blocks one lane iteration covers
            float(*rc)[2] = rchain[wave] + (lane / LPR) * (nbr * NU);
#pragma unroll
            for (int i = 0; i < NU; i++) {
                const int u = j + i * LPR;
                const bool live = row_ok && u < U;
                const XU<TYPE> x = load_xu<TYPE>(A.x8, A.xmeta, A.xsumq, A.x_tb, live ? u : 0, tk);
                const float pg = ref_block_partial<TYPE>(w0[i], u, x, live);
                const float pu = ref_block_partial<TYPE>(w1[i], u, x, live);
                if ((j & 3) == 3 && u < U) {
                    rc[(j >> 2) + i * nbr][0] = pg;
                    rc[(j >> 2) + i * nbr][1] = pu;
                }
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            if (j == 0 && row_ok) {
                float g = 0.0f, uu = 0.0f;
                for (int b = 0; b < U / 4; b++) {
                    g += rc[b][0];
                    uu += rc[b][1];
                }
                A.out[(size_t)p * A.out_stride + row] = silu_dev(g) * uu;
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            continue;
        }
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

// Loaded-but-undecoded form of a unit, so the next item's weights can stay in
// flight while the current item computes: Q4_K/Q5_K units are used as
// loaded; Q6_K/Q8_0 units are byte-realigned at decode.
template <uint32_t TYPE> struct GFetch { using T = typename GRawOf<TYPE>::T; };
template <> struct GFetch<MIQ_TYPE_Q6_K> { using T = FetchQ6K; };
template <> struct GFetch<MIQ_TYPE_Q8_0> { using T = FetchQ80; };

template <uint32_t TYPE> __device__ __forceinline__ uint32_t unit_off(uint32_t row_off, int u) {
    if constexpr (TYPE == MIQ_TYPE_Q4_K) return row_off + (uint32_t)(u >> 2) * kQ4KBytes;
    else if constexpr (TYPE == MIQ_TYPE_Q5_K) return row_off + (uint32_t)(u >> 2) * kQ5KBytes;
    else if constexpr (TYPE == MIQ_TYPE_Q6_K) return row_off + (uint32_t)(u >> 2) * kQ6KBytes;
    else return row_off + (uint32_t)u * 68u;
}
template <uint32_t TYPE>
__device__ __forceinline__ typename GFetch<TYPE>::T grp_fetch(__amdgpu_buffer_rsrc_t rs, uint32_t row_off, int u) {
    const uint32_t o = unit_off<TYPE>(row_off, u);
    if constexpr (TYPE == MIQ_TYPE_Q4_K) return load_q4k(rs, o, u & 3);
    else if constexpr (TYPE == MIQ_TYPE_Q5_K) return load_q5k(rs, o, u & 3);
    else if constexpr (TYPE == MIQ_TYPE_Q6_K) return fetch_q6k(rs, o, u & 3);
    else return fetch_q80(rs, o);
}
template <uint32_t TYPE>
__device__ __forceinline__ typename GRawOf<TYPE>::T grp_dec(const typename GFetch<TYPE>::T &f, uint32_t row_off,
                                                            int u) {
    if constexpr (TYPE == MIQ_TYPE_Q6_K) return dec_q6k(f, unit_off<TYPE>(row_off, u));
    else if constexpr (TYPE == MIQ_TYPE_Q8_0) return dec_q80(f);
    else return f;
}

// One work item of the pipelined grouped GEMV: (active expert slot, block of
// 4*64/LPR rows); item i = slot * nrb + row block.
struct GItem {
    int e, row;
    uint32_t ro;  // byte offset of the lane's row in the bank, or w_bytes (reads zeros)
};

template <int LPR, bool DUAL = false>
__device__ __forceinline__ GItem grp_locate(const GrpArgs &A, int item, int nrb, int rsub, bool u_ok) {
    const int slot = item / nrb;
    GItem g;
    g.e = A.active[slot];
    g.row = (item - slot * nrb) * ((DUAL ? 2 : 1) * 4 * (64 / LPR)) + rsub;
    g.ro = (g.row < A.n_rows && u_ok) ? (uint32_t)((size_t)g.e * A.plane) + (uint32_t)g.row * A.row_bytes
                                      : A.w_bytes;
    return g;
}

// Item `cur` (weights c0/c1 in flight) is computed while item `itn`'s weights
// are fetched into n0/n1.  The first pair's activation is loaded before the
// next item's weights, so waiting for it leaves those weights in flight;
// further pairs (fewer at decode sizes) load after the first is done and wait
// for everything.
template <uint32_t TYPE, int LPR, bool FUSE, bool DUAL = false>
__device__ __forceinline__ void grpp_step(const GrpArgs &A, __amdgpu_buffer_rsrc_t r0, __amdgpu_buffer_rsrc_t r1,
                                          int nrb, int rsub, int j, bool u_ok, int u, const GItem &cur,
                                          const typename GFetch<TYPE>::T &c0, const typename GFetch<TYPE>::T &c1,
                                          int itn, int n_items, GItem &nxt, typename GFetch<TYPE>::T &n0,
                                          typename GFetch<TYPE>::T &n1, float (*rchain)[2]) {
    const int p0 = A.off[cur.e], P = A.off[cur.e + 1] - p0;
    const int pa = A.pair[p0], pb = A.pair[P > 1 ? p0 + 1 : p0];
    const XU<TYPE> xa = load_xv<TYPE>(A.x8, A.xmeta, A.K, u, pa / A.tok_div);
    if (itn < n_items) {
        nxt = grp_locate<LPR, DUAL>(A, itn, nrb, rsub, u_ok);
    } else {  // past the last item: a zero fetch, never computed
        nxt.e = 0;
        nxt.row = A.n_rows;
        nxt.ro = A.w_bytes;
    }
    n0 = grp_fetch<TYPE>(r0, nxt.ro, u);
    if constexpr (FUSE || DUAL) n1 = grp_fetch<TYPE>(r1, nxt.ro, u);

    const bool live = cur.row < A.n_rows && u_ok;
    const typename GRawOf<TYPE>::T w0 = grp_dec<TYPE>(c0, cur.ro, u);
    typename GRawOf<TYPE>::T w1;
    if constexpr (FUSE || DUAL) w1 = grp_dec<TYPE>(c1, cur.ro, u);
    auto emit = [&](int p, const XU<TYPE> &x) {
        if constexpr (FUSE && ref_order<TYPE>()) {  // gate/up in the reference's order (see ref_group_terms)
            const float pg = ref_block_partial<TYPE>(w0, u, x, live);
            const float pu = ref_block_partial<TYPE>(w1, u, x, live);
            const int lane = threadIdx.x & 63;
            float(*rc)[2] = rchain + ((threadIdx.x >> 6) * 16 + (lane / LPR) * (LPR / 4));
            if ((j & 3) == 3 && u_ok) {
                rc[j >> 2][0] = pg;
                rc[j >> 2][1] = pu;
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            if (j == 0 && cur.row < A.n_rows) {
                float g = 0.0f, uu = 0.0f;
                for (int b = 0; b < A.K / 256; b++) {
                    g += rc[b][0];
                    uu += rc[b][1];
                }
                A.out[(size_t)p * A.out_stride + cur.row] = silu_dev(g) * uu;
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            return;
        }
        float a0 = live ? term_xu<TYPE>(w0, u, x) : 0.0f, a1 = 0.0f;
        if constexpr (FUSE) a1 = live ? term_xu<TYPE>(w1, u, x) : 0.0f;
        // DUAL: bank 1 is the same matrix 4*64/LPR rows further on
        constexpr int kHalf = 4 * (64 / LPR);
        if constexpr (DUAL) a1 = cur.row + kHalf < A.n_rows && u_ok ? term_xu<TYPE>(w1, u, x) : 0.0f;
        a0 = seg_sum<LPR>(a0);
        if constexpr (FUSE || DUAL) a1 = seg_sum<LPR>(a1);
        if (j == 0 && cur.row < A.n_rows) A.out[(size_t)p * A.out_stride + cur.row] = FUSE ? silu_dev(a0) * a1 : a0;
        if constexpr (DUAL)
            if (j == 0 && cur.row + kHalf < A.n_rows) A.out[(size_t)p * A.out_stride + cur.row + kHalf] = a1;
    };
    emit(pa, xa);
    // the second pair's activation only now: holding it from the step's start
    // cost the registers of a fourth wave per SIMD (gate/up 132 -> 117 VGPRs;
    // experts call 59.3 -> 55.0 us at config 5)
    if (P > 1) emit(pb, load_xv<TYPE>(A.x8, A.xmeta, A.K, u, pb / A.tok_div));
    for (int pi = 2; pi < P; pi++) {
        const int p = A.pair[p0 + pi];
        emit(p, load_xv<TYPE>(A.x8, A.xmeta, A.K, u, p / A.tok_div));
    }
}

// Persistent grouped GEMV for K <= 64*LPR (one unit per lane per bank): the
// grid covers the device once and each workgroup walks the work items
// blockIdx.x, +gridDim.x, ... with the next item's weights always in flight.
// Only items of active experts exist, so no workgroup idles on an inactive
// expert.
template <uint32_t TYPE, int LPR, bool FUSE, bool DUAL = false>
__global__ __launch_bounds__(256) void grpp_kernel(GrpArgs A, int nrb) {
    const int n_items = *A.n_active * nrb;
    int it = blockIdx.x;
    if (it >= n_items) return;
    constexpr int RPW = 64 / LPR;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int rsub = wave * RPW + lane / LPR, j = lane % LPR;
    const bool u_ok = j < A.K / 64;
    const int u = u_ok ? j : 0;
    const __amdgpu_buffer_rsrc_t r0 = make_rsrc(A.w0, A.w_bytes);
    constexpr uint32_t kHalfRows = 4 * (64 / LPR);
    const __amdgpu_buffer_rsrc_t r1 = DUAL ? make_rsrc(A.w0 + kHalfRows * A.row_bytes, A.w_bytes - kHalfRows * A.row_bytes)
                                           : make_rsrc(FUSE ? A.w1 : A.w0, A.w_bytes);
    using F = typename GFetch<TYPE>::T;
    F fa0, fa1, fb0, fb1;
    GItem ga = grp_locate<LPR, DUAL>(A, it, nrb, rsub, u_ok), gb{0, A.n_rows, A.w_bytes};
    fa0 = grp_fetch<TYPE>(r0, ga.ro, u);
    if constexpr (FUSE || DUAL) fa1 = grp_fetch<TYPE>(r1, ga.ro, u);
    const int G = gridDim.x;
    __shared__ float rchain[4 * 16][2];  // gate/up block partials, [wave][row in wave][block]
    while (true) {
        grpp_step<TYPE, LPR, FUSE, DUAL>(A, r0, r1, nrb, rsub, j, u_ok, u, ga, fa0, fa1, it + G, n_items, gb, fb0, fb1, rchain);
        it += G;
        if (it >= n_items) break;
        grpp_step<TYPE, LPR, FUSE, DUAL>(A, r0, r1, nrb, rsub, j, u_ok, u, gb, fb0, fb1, it + G, n_items, ga, fa0, fa1, rchain);
        it += G;
        if (it >= n_items) break;
    }
}

template <uint32_t TYPE, int LPR, bool FUSE, bool DUAL = false>
static int launch_grpp_l(hipStream_t s, const GrpArgs &A, int n_expert) {
    constexpr int rows_per_item = (DUAL ? 2 : 1) * 4 * (64 / LPR);
    const int nrb = (A.n_rows + rows_per_item - 1) / rows_per_item;
    static int occ[64] = {0};
    int dev = 0, cus = 0, rc;
    if ((rc = device_cus(&cus))) return rc;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
        set_error("miq_moe_experts: no current device");
        return MIQ_EHIP;
    }
    if (!occ[dev] && (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ[dev], grpp_kernel<TYPE, LPR, FUSE, DUAL>, 256, 0) !=
                          hipSuccess ||
                      occ[dev] <= 0))
        occ[dev] = 1;
    const long items = (long)n_expert * nrb;
    const int grid = (int)std::min<long>(items, (long)cus * occ[dev]);
    hipLaunchKernelGGL((grpp_kernel<TYPE, LPR, FUSE, DUAL>), dim3(grid), dim3(256), 0, s, A, nrb);
    return MIQ_OK;
}

template <uint32_t TYPE, bool FUSE> static int launch_grpp_t(hipStream_t s, const GrpArgs &A, int n_expert) {
    const int U = A.K / 64;
    if (U <= 4) return launch_grpp_l<TYPE, 4, FUSE>(s, A, n_expert);
    if (U <= 8) {
        // the down projection (K <= 512): two row sets per item, so each
        // pair's activation serves twice the weights (experts call 55.3 ->
        // 54.0 us at config 5)
        if (!FUSE && A.n_rows >= 64) return launch_grpp_l<TYPE, 8, false, true>(s, A, n_expert);
        return launch_grpp_l<TYPE, 8, FUSE>(s, A, n_expert);
    }
    if (U <= 16) return launch_grpp_l<TYPE, 16, FUSE>(s, A, n_expert);
    if (U <= 32) return launch_grpp_l<TYPE, 32, FUSE>(s, A, n_expert);
    return launch_grpp_l<TYPE, 64, FUSE>(s, A, n_expert);
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

// K <= 4096 takes the persistent pipelined kernel (MIQ_MOE_GRP=0 selects the
// one-workgroup-per-(expert, row block) kernel instead); larger K the latter.
// The pipelined kernel reads its activation in the token-major unit layout,
// the other in the group-major one: grp_layout names the xq layout to write.
static int grp_layout(uint32_t type, int K) {
    if (K > 64 * 64 || sw(kSwMoeGrp) == 0) return 0;
    return type == MIQ_TYPE_Q6_K ? 2 : 1;
}

template <bool FUSE> static int launch_grp(hipStream_t s, uint32_t type, const GrpArgs &A, int n_expert, int layout) {
    if (layout) {
        switch (type) {
        case MIQ_TYPE_Q4_K: return launch_grpp_t<MIQ_TYPE_Q4_K, FUSE>(s, A, n_expert);
        case MIQ_TYPE_Q5_K: return launch_grpp_t<MIQ_TYPE_Q5_K, FUSE>(s, A, n_expert);
        case MIQ_TYPE_Q6_K: return launch_grpp_t<MIQ_TYPE_Q6_K, FUSE>(s, A, n_expert);
        default:
            if constexpr (FUSE) return MIQ_UNSUPPORTED;  // no Q8_0 gate/up (checked by the caller)
            else return launch_grpp_t<MIQ_TYPE_Q8_0, false>(s, A, n_expert);
        }
    }
    switch (type) {
    case MIQ_TYPE_Q4_K: launch_grp_t<MIQ_TYPE_Q4_K, FUSE>(s, A, n_expert); break;
    case MIQ_TYPE_Q5_K: launch_grp_t<MIQ_TYPE_Q5_K, FUSE>(s, A, n_expert); break;
    case MIQ_TYPE_Q6_K: launch_grp_t<MIQ_TYPE_Q6_K, FUSE>(s, A, n_expert); break;
    default:
        if constexpr (FUSE) return MIQ_UNSUPPORTED;
        else launch_grp_t<MIQ_TYPE_Q8_0, false>(s, A, n_expert);
        break;
    }
    return MIQ_OK;
}

// ------------------------------------------------------------------ reduce
constexpr int kRedK = 8;  // top-k the weighted reduce serves with all loads issued first
__global__ __launch_bounds__(256) void reduce_kernel(const float *__restrict__ acc, const float *__restrict__ wts,
                                                     int top_k, int n_tok, int n_embd, int acc_stride,
                                                     float *__restrict__ out, int out_stride) {
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long)n_tok * n_embd) return;
    const int t = (int)(i / n_embd), e = (int)(i % n_embd);
    const size_t p0 = (size_t)t * top_k;
    float *const dst = out + (size_t)t * out_stride + e;
    const float prev = *dst;  // loaded with the pairs, not after the sum
    double a = 0.0;
    if (top_k <= kRedK) {
        // every pair's loads go out before the sum (a loop that loads as it
        // adds waits one L2 round trip per pair); the sum keeps pair order
        float w[kRedK], v[kRedK];
#pragma unroll
        for (int j = 0; j < kRedK; j++)
            if (j < top_k) {
                w[j] = wts[p0 + j];
                v[j] = acc[(p0 + j) * (size_t)acc_stride + e];
            }
#pragma unroll
        for (int j = 0; j < kRedK; j++)
            if (j < top_k) a += (double)w[j] * (double)v[j];
    } else {
        for (int j = 0; j < top_k; j++) a += (double)wts[p0 + j] * (double)acc[(p0 + j) * (size_t)acc_stride + e];
    }
    *dst = prev + (float)a;
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
    w.xmeta = (float *)take(K / 32 * n_tok * 16);  // the unit layouts need up to 32 B per 64 values
    w.xsumq = (int32_t *)take(K / 32 * n_tok * 8);
    w.off = (int32_t *)take(4 * (M->n_expert + 1));
    w.pair = (int32_t *)take(4 * np);
    w.active = (int32_t *)take(4 * M->n_expert);
    w.n_active = (int32_t *)take(4);
    w.h = (float *)take(4 * F * np);
    w.h8 = (int8_t *)take(F * np);
    w.hmeta = (float *)take(F / 32 * np * 16);
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
    if (K % 32 || (type != MIQ_TYPE_Q8_0 && K % 256)) {
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
    const int V = (n_expert + 63) / 64;
    const dim3 wgrid((n_tok + 3) / 4), wblock(256);
    if (!gate_inp && V <= 8) {  // given logits, up to 512 experts: one wave per token
        const int vv = V == 1 ? 1 : V == 2 ? 2 : V <= 4 ? 4 : 8;
        const size_t rl = miq::route_lds_bytes(vv, 4);
        if (vv == 1) hipLaunchKernelGGL(miq::route_wave_kernel<1>, wgrid, wblock, rl, stream, n_tok, n_expert, top_k, logits, ids, wts);
        else if (vv == 2) hipLaunchKernelGGL(miq::route_wave_kernel<2>, wgrid, wblock, rl, stream, n_tok, n_expert, top_k, logits, ids, wts);
        else if (vv == 4) hipLaunchKernelGGL(miq::route_wave_kernel<4>, wgrid, wblock, rl, stream, n_tok, n_expert, top_k, logits, ids, wts);
        else hipLaunchKernelGGL(miq::route_wave_kernel<8>, wgrid, wblock, rl, stream, n_tok, n_expert, top_k, logits, ids, wts);
    } else {
        hipLaunchKernelGGL(miq::route_kernel, dim3(n_tok), dim3(256), lds, stream, x, x_stride, gate_inp, n_embd,
                           n_expert, top_k, logits, ids, wts);
    }
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
    if (M->gate_type == MIQ_TYPE_Q8_0 || M->up_type == MIQ_TYPE_Q8_0) {
        // i8_row (i8.cpp:157-190) serves Q4_K/Q5_K/Q6_K gate/up only; Q8_0 is a
        // down-projection type there (q8_0_down_row, q4exp.cpp:442-467)
        set_error("miq_moe_experts: Q8_0 gate/up banks are not on the reference's integer expert path");
        return MIQ_UNSUPPORTED;
    }
    if (M->gate_type != M->up_type || M->gate_plane != M->up_plane) {
        set_error("miq_moe_experts: gate and up banks must share type and plane size");
        return MIQ_UNSUPPORTED;
    }
    const size_t gbytes = M->gate_plane * M->n_expert, dbytes = M->down_plane * M->n_expert;
    if (gbytes >= (1ull << 32) - 4096 || dbytes >= (1ull << 32) - 4096) {
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
    const size_t lds = (size_t)(M->n_expert + np) * 4;
    if (lds > 64 * 1024) {
        set_error("miq_moe_experts: n_expert=%d + pairs=%d too large for the CSR", M->n_expert, np);
        return MIQ_UNSUPPORTED;
    }
    // a Q8_0 down bank with an odd group count (n_ff % 64 == 32) runs on the
    // any-group-count Q8_0 kernel, which reads the group-major layout
    const bool d_any = M->down_type == MIQ_TYPE_Q8_0 && M->n_ff % 64 != 0;
    const int lay_g = grp_layout(M->gate_type, M->n_embd), lay_d = d_any ? 0 : grp_layout(M->down_type, M->n_ff);
    PrepArgs P{ids, np, M->n_expert, w.off, w.pair, w.active, w.n_active, acc, acc_stride, M->n_embd,
               x, x_stride, w.x8, w.xmeta, w.xsumq, n_tok, M->n_embd / 32};
    constexpr int kPrepThreads = 512;  // measured 1 us faster per experts call than 1024 (256: slower)
    const dim3 pgrid(1 + (n_tok * P.G + kPrepThreads - 1) / kPrepThreads);
    if (lay_g == 0) hipLaunchKernelGGL(moe_prep_kernel<0>, pgrid, dim3(kPrepThreads), lds, stream, P);
    else if (lay_g == 1) hipLaunchKernelGGL(moe_prep_kernel<1>, pgrid, dim3(kPrepThreads), lds, stream, P);
    else hipLaunchKernelGGL(moe_prep_kernel<2>, pgrid, dim3(kPrepThreads), lds, stream, P);
    if ((rc = check_launch("miq_moe_experts set-up"))) return rc;
    GrpArgs A{};
    A.w0 = (const uint8_t *)M->gate;
    A.w1 = (const uint8_t *)M->up;
    A.w_bytes = dword_span(gbytes);
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
    if ((rc = launch_grp<true>(stream, M->gate_type, A, M->n_expert, lay_g))) return rc;
    if ((rc = check_launch("miq_moe_experts gate/up"))) return rc;
    if ((rc = launch_xq(stream, w.h, nullptr, M->n_ff, 0, w.h8, w.hmeta, w.hsumq, np, M->n_ff, lay_d))) return rc;
    if (d_any) {
        if ((rc = launch_q80_banked(stream, M->down, M->down_plane, M->n_expert, M->n_ff, M->n_embd, w.h8, w.hmeta,
                                    np, ids, acc, acc_stride)))
            return rc;
        return MIQ_OK;
    }
    GrpArgs D = A;
    D.w0 = D.w1 = (const uint8_t *)M->down;
    D.w_bytes = dword_span(dbytes);
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
    if ((rc = launch_grp<false>(stream, M->down_type, D, M->n_expert, lay_d))) return rc;
    if ((rc = check_launch("miq_moe_experts down"))) return rc;
    return MIQ_OK;
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
