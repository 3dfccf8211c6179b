/*
 * miq oracle -- TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C, scalar restatement of sycl-infer's CPU integer quantized-matmul
 * path.  It is the checker the HIP kernels are compared against; nothing in the
 * product library links, loads or calls it.  Only tests/, the smoke check in
 * __graft_entry__.py and bench.py's CPU-baseline leg may use it.
 *
 * Every function cites the reference file:line it restates (paths relative to
 * the sycl-infer source root).  Integer dot products are computed exactly with
 * scalar loops; the fp32 epilogues keep the reference's expressions and
 * association order (block partial then row for the one-token form, continuous
 * per-group accumulation for the tiled form).
 *
 * Pinning (what checks each function; see tests/test_oracle_*.py):
 *   f16 conversions      exhaustive 2^16 half->float vs IEEE; truncation
 *                        invariant for float->half; compiled-reference fixtures
 *   get_scale_min_k4     pack/unpack round trip over all 6-bit values
 *   dequantize_row       hand-built bit patterns (Q8_0 d*q), compiled-reference
 *                        fixtures for Q4_K/Q5_K/Q6_K
 *   xq                   compiled-reference fixtures (bit-exact, incl. zero group)
 *                        + the reference unit test's closed form
 *   group dots           brute force over dequantized integer codes
 *   i8_gemv / i8_gemm    compiled-reference fixtures (<=1e-6) and a
 *                        dequantize + double-dot reference (3e-2, as the
 *                        reference's own test)
 *   moe route / reduce   compiled-reference fixtures, closed form invariants
 *   moe experts          composition of the pinned pieces + fixtures
 *   w4 pack              compiled-reference w4_pack (bit-exact) + the
 *                        reference test's round trip against dequantize_row
 *   float->half (rne)    numpy's float16 conversion, every f16 boundary
 *   w4 act               the reference GPU test's make_act closed form, and
 *                        per-group invariants (|q|<=127, max code 127)
 *   k5 pack / gemv       compiled-reference k5_pack (bit-exact); the gemv
 *                        against the Q5_K dequantize x activation double sum
 *   w4 gemv              the dequantize x activation double sum (the
 *                        reference GPU test's formula, 2e-3) and the
 *                        pack identity sum_g step*qdot + off*xs
 */
#ifndef MIQ_ORACLE_H
#define MIQ_ORACLE_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { MIQO_Q8_0 = 8, MIQO_Q4_K = 12, MIQO_Q5_K = 13, MIQO_Q6_K = 14 };

/* src/common/quant.h:67-92 (half->float) and :112-133 (truncating float->half) */
float miqo_half_to_float(uint16_t h);
uint16_t miqo_float_to_half(float f);
/* src/common/quant.h:136-144 */
void miqo_get_scale_min_k4(int j, const uint8_t *q, uint8_t *d, uint8_t *m);
/* src/common/quant.h:1177 (the four types of this path only) */
size_t miqo_row_bytes(uint32_t type, int K);
/* src/common/quant.h:148-210,1074 -- fp32 dequantisation of one row */
void miqo_dequantize_row(uint32_t type, const void *row, float *y, int K);

/* src/backend/cpu/kernels/xq.cpp:10-50 (cpu_xq).  x8[(g*TB+t)*32+i],
 * xmeta[(g*TB+t)*2] = {f16-truncated scale, 0}, xsumq[(g*TB+t)*2+{0,1}]. */
void miqo_xq(const float *x, const float *up, int x_stride, int up_stride, int8_t *x8, float *xmeta,
             int32_t *xsumq, int TB, int K);

/* Exact per-group integer dots, the quantity the fp32 epilogue scales.
 * For Q4_K/Q5_K/Q8_0: one int32 per (t, row, 32-group) = sum q*x8 with q the
 * unsigned 4/5-bit code (Q8_0: signed byte).  For Q6_K: one int32 per
 * (t, row, 16-subgroup) = sum q*x8 with q the unsigned 6-bit code (the -32 is
 * applied in the epilogue, i8.cpp:149-152).  Layout: out[(t*n_rows+row)*S+s]
 * with S = K/32 (K/16 for Q6_K).  i8.cpp:49-57 (Q4_K), :109-118 (Q5_K),
 * :129-150 (Q6_K); q4exp.cpp:70-74,442-470 (Q8_0). */
void miqo_group_dots(uint32_t type, const void *w, int K, int n_rows, const int8_t *x8, int TB, int32_t *out);

/* src/backend/cpu/kernels/i8.cpp:157-190 (i8_row) plus q8_0_down_row's
 * per-group form (q4exp.cpp:442-470) for Q8_0. */
float miqo_i8_row(uint32_t type, const void *wrow, const int8_t *x8, const float *xmeta, const int32_t *xsumq,
                  int TB, int t, int K);

/* Segment descriptor: the fields of cpu_gemv_seg (src/backend/cpu/cpu_types.h:68-86)
 * the integer path reads. */
typedef struct miqo_seg {
    const void *w;
    uint32_t type;
    int32_t K;
    int32_t n_rows;
    float *out;
    int32_t out_stride;
    const float *residual;
    float alpha;
    const int8_t *x8;
    const float *xmeta;
    const int32_t *xsumq;
} miqo_seg;

/* src/backend/cpu/kernels/i8.cpp:498-516 (cpu_i8_gemv): out[row] = alpha*i8_row + residual[row] */
void miqo_i8_gemv(const miqo_seg *s);
/* src/backend/cpu/kernels/i8.cpp:518-546 (cpu_i8_gemm): TB>=2 takes the tiled
 * form (i8.cpp:316-377, per-group accumulation continuous across blocks);
 * out[t*out_stride+row] = alpha*acc + residual[t*out_stride+row]. */
void miqo_i8_gemm(const miqo_seg *s, int TB);

/* src/backend/cpu/kernels/moe.cpp:72-137 (cpu_moe_route).  With gate_inp ==
 * NULL the logits buffer is taken as already filled (n_tok x n_expert). */
void miqo_moe_route(const float *x, int x_stride, const float *gate_inp, int n_tok, int n_embd, int n_expert,
                    int top_k, float *logits, int32_t *ids, float *wts);

/* The integer expert composition of cpu_moe_experts_i8 (moe.cpp:476-559) with
 * every projection a K-quant: per pair p (token p/top_k, expert ids[p]):
 * g,u = i8_row(gate/up rows, xq(x_t)); h = silu(g)*u; xq(h) (quant_row_1,
 * moe.cpp:450-471); acc[p][r] = i8_row(down row r, xq(h)).  Expert e's
 * projection starts at bank + e*plane_bytes. */
typedef struct miqo_moe {
    const void *gate;
    const void *up;
    const void *down;
    uint32_t gate_type, up_type, down_type;
    size_t gate_plane, up_plane, down_plane;
    int n_embd;   /* K of gate/up, rows of down */
    int n_ff;     /* rows of gate/up, K of down */
    int n_expert;
} miqo_moe;
void miqo_moe_experts(const miqo_moe *M, const float *x, int x_stride, int n_tok, int top_k, const int32_t *ids,
                      float *acc, int acc_stride, float *h_out /* optional [np][n_ff] */);
/* src/backend/cpu/kernels/moe.cpp:562-574 (cpu_moe_reduce): out += sum_j w*acc in double */
void miqo_moe_reduce(const float *acc, const float *wts, int top_k, int n_tok, int n_embd, int acc_stride,
                     float *out, int out_stride);

/* ---- u4 native-width store (the reference's "w4t", src/common/w4.h:55-66) ----
 * vals [N][K/2]: element k of row n in byte (n*K+k)/2, nibble (k&1) (low first)
 * scale[g*N+n], off[g*N+n]: f16 step d*sc_j and additive offset -dmin*m_j of
 * 32-group g, converted with the truncating float->half (quant.h:112-133). */

/* src/common/w4.cpp:160-212 (pack_q4_K).  Returns 0, or -1 if K % 256. */
int miqo_w4_pack_q4k(const void *src, int K, int N, uint8_t *vals, uint16_t *scale, uint16_t *off);
/* float->half rounding to nearest even (IEEE binary16), the conversion of
 * sycl::half(float) that act_quant_grp_launch stores the group scale with */
uint16_t miqo_float_to_half_rne(float f);
/* src/backend/dnnl_gemm.cpp:100-146 (act_quant_grp_launch, do_split): per
 * 32-group symmetric int8, xq[m*K+k]; asa[m*ng+g] = half_rne(max/127);
 * xs[m*ng+g] = sum of the group's codes; axe/axo[m*K/2+j] = xq[2j], xq[2j+1]. */
void miqo_w4_act(const float *x, const float *up, int M, int K, int8_t *xq, uint16_t *asa, float *xs, int8_t *axe,
                 int8_t *axo);
/* src/backend/gpu/kernels/w4_gemv.cpp:79-154 (w4_gemv_impl), M == 1:
 * out[n] = alpha * sum_g asa[g]*(step[g][n]*QDOT_g[n] + off[g][n]*xs[g]) + residual[n],
 * QDOT_g = sum over the group's 32 (nibble * int8) products (exact).  The sum
 * over g runs in double here; the kernel's fp32 order is implementation-defined. */
void miqo_w4_gemv(const uint8_t *vals, const uint16_t *scale, const uint16_t *off, const int8_t *axe,
                  const int8_t *axo, const uint16_t *asa, const float *xs, float *out, const float *residual,
                  float alpha, int K, int N);
/* src/common/w4.cpp:336-403 (pack_q5_K): vals as the u4 store, hi[N][K/8]
 * one u32 per (row, group): bit i = fifth bit of element 2i, bit 16+i = of
 * element 2i+1.  Returns 0, or -1 if K % 256. */
int miqo_k5_pack(const void *src, int K, int N, uint8_t *vals, uint8_t *hi, uint16_t *scale, uint16_t *off);
/* src/backend/gpu/kernels/w4_gemv.cpp:1002-1080 (k5_gemv_impl): the u4 formula
 * with q5 = lo4 | bit << 4 */
void miqo_k5_gemv(const uint8_t *vals, const uint8_t *hi, const uint16_t *scale, const uint16_t *off,
                  const int8_t *axe, const int8_t *axo, const uint16_t *asa, const float *xs, float *out,
                  const float *residual, float alpha, int K, int N);

/* silu as the reference defines it (src/backend/cpu/kernels/common.h:31-33) */
float miqo_silu(float x);

/* Count of i < count where y[i] differs in bits from the host libm's
 * expf(bits(first + i)) (NaNs compare equal); *first_bad = the first such
 * input's bits.  The check for the device expf. */
uint64_t miqo_expf_mismatches(uint32_t first, uint32_t count, const float *y, uint32_t *first_bad);
/* The device expf's method restated in C (glibc expf, Arm optimized-routines
 * e_expf.c, FMA build), and the count of inputs in [first, first+count) where
 * it differs in bits from the host libm's expf. */
float miqo_expf_method(float x);
uint64_t miqo_expf_method_mismatches(uint32_t first, uint32_t count, uint32_t *first_bad);

#ifdef __cplusplus
}
#endif
#endif
