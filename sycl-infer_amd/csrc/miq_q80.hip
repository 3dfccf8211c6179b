// Q8_0 rows of any whole number of 32-value groups (K % 32 == 0).
//
// The reference's native Q8_0 down projection loops G = K/32 groups
// (q8_0_down_row, src/backend/cpu/kernels/q4exp.cpp:442-467): per group the
// int32 dot of the 32 signed codes with the group's activation codes, then
// a += xmeta * d * (float)dot.  The other kernels walk 64-value units, so a row
// with an odd group count (K % 64 == 32, e.g. K = 96 or 5152) comes here: its
// 34-byte blocks then start at 2-byte aligned offsets, and no unit holds a
// group of the next row.
//
// One wave per row.  Lane l takes groups l, l + 64, ...: it loads each block
// as the dword-aligned 36 bytes around it (three buffer loads) and realigns
// the codes by the block's byte shift (0 or 2), so the block's codes are read
// once for a tile of TT tokens; per token it loads the group's 32 activation
// codes and its scale, forms the exact dot with sdot4 and adds the group term.
// The lanes' sums meet by cross-lane shuffles.  Workgroups of four waves (four
// rows) x one token tile.
//
// Banked form (the MoE down projection): token p of the activation is routed
// pair p, whose weights are bank + ids[p] * plane; an id outside
// [0, n_bank) gives a zero row.  A tile then holds one pair (TT = 1).
//
// Parity form: every group's int32 dot goes to dots[(t*n_rows + row)*G + g].
#include "miq_internal.h"

namespace miq {
namespace {

struct Q80Args {
    const uint8_t *w;
    uint32_t w_bytes;   // whole tensor (all banks), rounded up to dwords
    uint32_t row_bytes;
    int G;              // groups per row
    int n_rows;
    int TB;
    const int8_t *x8;   // [(g*TB + t)*32]
    const float *xmeta; // [(g*TB + t)*2]
    float *out;
    int out_stride;
    const float *residual;
    float alpha;
    const int32_t *ids; // banked form: pair -> bank
    int n_bank;
    uint32_t plane;     // bytes per bank
    int32_t *dots;
};

constexpr int kQ80TT = 8;  // tokens per tile

template <int TT, bool BANKED, bool DOTS>
__global__ __launch_bounds__(256) void q80_kernel(Q80Args A) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int t0 = blockIdx.y * TT;
    if (row >= A.n_rows) return;  // whole waves leave: no cross-lane op follows for them
    uint32_t row_off = (uint32_t)row * A.row_bytes;
    bool live = true;
    if constexpr (BANKED) {
        const int e = A.ids[t0];
        live = e >= 0 && e < A.n_bank;
        row_off += live ? (uint32_t)e * A.plane : 0u;
    }
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(A.w, A.w_bytes);
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(A.x8, (uint32_t)A.G * A.TB * 32);
    const __amdgpu_buffer_rsrc_t rm = make_rsrc(A.xmeta, (uint32_t)A.G * A.TB * 8);
    float acc[TT];
#pragma unroll
    for (int i = 0; i < TT; i++) acc[i] = 0.0f;
    for (int g = lane; g < A.G; g += 64) {
        const uint32_t off = row_off + (uint32_t)g * 34u;
        const uint32_t a = off & ~3u, sh = off & 3u;  // sh: 0 or 2
        const uint4 r0 = bload16(rw, a), r1 = bload16(rw, a + 16);
        const uint32_t r8 = bload4(rw, a + 32);
        const uint32_t r[9] = {r0.x, r0.y, r0.z, r0.w, r1.x, r1.y, r1.z, r1.w, r8};
        const float d = h2f((r[0] >> (8 * sh)) & 0xFFFFu);
        uint32_t c[8];  // the codes start 2 bytes after the block: byte 2 of r[0], or r[1]
#pragma unroll
        for (int k = 0; k < 8; k++) c[k] = sh ? r[k + 1] : __builtin_amdgcn_alignbyte(r[k + 1], r[k], 2);
#pragma unroll
        for (int i = 0; i < TT; i++) {
            const int t = t0 + i;
            const uint32_t gi = (uint32_t)g * A.TB + (uint32_t)(t < A.TB ? t : 0);
            const uint4 x0 = bload16(rx, gi * 32), x1 = bload16(rx, gi * 32 + 16);
            const uint32_t x[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
            int qd = 0;
#pragma unroll
            for (int k = 0; k < 8; k++) qd = dot4(c[k], x[k], qd);
            if constexpr (DOTS) {
                if (t < A.TB) A.dots[((size_t)t * A.n_rows + row) * A.G + g] = qd;
            } else {
                const float xm = __builtin_bit_cast(float, bload4(rm, gi * 8));
                acc[i] = __builtin_fmaf(xm * d, (float)qd, acc[i]);
            }
        }
    }
    if constexpr (!DOTS) {
#pragma unroll
        for (int i = 0; i < TT; i++) {
            float v = acc[i];
#pragma unroll
            for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
            const int t = t0 + i;
            if (lane == 0 && t < A.TB) {
                const size_t o = (size_t)t * A.out_stride + row;
                float y = live ? A.alpha * v : 0.0f;
                if (A.residual) y += A.residual[o];
                A.out[o] = y;
            }
        }
    }
}

}  // namespace

bool q80_any(const miq_seg *s) { return s->type == MIQ_TYPE_Q8_0 && s->K % 64 != 0; }

static Q80Args q80_args(const miq_seg *s, int TB) {
    Q80Args A{};
    A.w = (const uint8_t *)s->w;
    A.row_bytes = (uint32_t)miq_row_bytes(MIQ_TYPE_Q8_0, s->K);
    A.w_bytes = dword_span((size_t)s->n_rows * A.row_bytes);
    A.G = s->K / 32;
    A.n_rows = s->n_rows;
    A.TB = TB;
    A.x8 = s->x8;
    A.xmeta = s->xmeta;
    A.out = s->out;
    A.out_stride = s->out_stride;
    A.residual = s->residual;
    A.alpha = s->alpha;
    return A;
}

int launch_q80(hipStream_t stream, const miq_seg *s, int TB, int32_t *dots) {
    if ((size_t)(s->K / 32) * TB * 32 >= 0xFFFFFFF0u) {
        set_error("miq Q8_0: activation of %d x %d exceeds the 4 GiB buffer window", TB, s->K);
        return MIQ_UNSUPPORTED;
    }
    Q80Args A = q80_args(s, TB);
    A.dots = dots;
    const dim3 grid((unsigned)((s->n_rows + 3) / 4), (unsigned)((TB + kQ80TT - 1) / kQ80TT)), block(256);
    if (dots) hipLaunchKernelGGL((q80_kernel<kQ80TT, false, true>), grid, block, 0, stream, A);
    else hipLaunchKernelGGL((q80_kernel<kQ80TT, false, false>), grid, block, 0, stream, A);
    return check_launch(dots ? "miq_group_dots" : "miq Q8_0");
}

int launch_q80_banked(hipStream_t stream, const void *bank, size_t plane, int n_bank, int K, int n_rows,
                      const int8_t *x8, const float *xmeta, int n_pairs, const int32_t *ids, float *out,
                      int out_stride) {
    Q80Args A{};
    A.w = (const uint8_t *)bank;
    A.row_bytes = (uint32_t)miq_row_bytes(MIQ_TYPE_Q8_0, K);
    A.w_bytes = dword_span(plane * (size_t)n_bank);
    A.G = K / 32;
    A.n_rows = n_rows;
    A.TB = n_pairs;
    A.x8 = x8;
    A.xmeta = xmeta;
    A.out = out;
    A.out_stride = out_stride;
    A.alpha = 1.0f;
    A.ids = ids;
    A.n_bank = n_bank;
    A.plane = (uint32_t)plane;
    const dim3 grid((unsigned)((n_rows + 3) / 4), (unsigned)n_pairs), block(256);
    hipLaunchKernelGGL((q80_kernel<1, true, false>), grid, block, 0, stream, A);
    return check_launch("miq_moe_experts (Q8_0 down)");
}

}  // namespace miq
