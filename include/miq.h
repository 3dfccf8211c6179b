/*
 * miq -- MI355X-native quantized matmul for GGUF inference (C ABI).
 *
 * Drop-in for sycl-infer's quantized-matmul hot path: the int8 activation
 * quantizer, the GGUF K-quant x int8 GEMV used in decode, the batched int8 GEMM
 * used in chunked prefill, and the MoE expert-grouped GEMV with its router,
 * token->expert CSR and weighted reduce.  Every reference interface an entry
 * point replaces is cited next to it (paths relative to the sycl-infer root).
 *
 * Conventions kept from the reference (src/backend/backend.h:13-15,
 * src/backend/gpu/kernels/kernels.h:44-81,585-594):
 *   - the caller owns every input and output buffer (device memory).  The
 *     library keeps per-device scratch of its own (split-K partials and
 *     counters, the prefill workspace, the u4 K-part sums) that a call grows
 *     with hipMalloc the first time a larger shape needs it; a call whose
 *     stream is capturing a graph never allocates and returns MIQ_UNSUPPORTED
 *     instead, so warm each shape up once before capture (as the reference
 *     runs a step eagerly before recording its decode graph,
 *     src/engine/engine.cpp:4528-4583), or call miq_i8_gemm_noalloc.  That
 *     scratch is shared by every stream of a device: calls that use it must
 *     not overlap on one device;
 *   - work is enqueued on the caller's stream and nothing waits on the host;
 *   - status: MIQ_OK (0); MIQ_UNSUPPORTED (1) for a shape/type the kernels do
 *     not serve, so the caller falls back exactly as the reference's `bool`
 *     launchers return false; negative values for invalid arguments or a HIP
 *     launch error (text from miq_last_error());
 *   - calls are expected from one host thread at a time per stream, as the
 *     reference serialises engine execution.
 * Activation format (src/backend/cpu/kernels/xq.cpp:1-50): per 32-value group
 * (g) of token t, x8[(g*TB+t)*32+i] int8, xmeta[(g*TB+t)*2] = {f16-truncated
 * fp32 scale, 0}, xsumq[(g*TB+t)*2+{0,1}] = sums of codes 0..15 and 16..31.
 * Weights: ggml blocks, row-major [n_rows][K/QK] (src/common/quant.h:12-41).
 * The 4-byte word holding a weight tensor's last byte is read whole (a tensor
 * of 2 mod 4 bytes, e.g. an odd number of Q6_K rows of an odd block count).
 */
#ifndef MIQ_H
#define MIQ_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t *hipStream_t;

enum miq_status {
    MIQ_OK = 0,
    MIQ_UNSUPPORTED = 1,
    MIQ_EINVAL = -1,
    MIQ_EHIP = -2,
};

/* ggml type ids of the weight formats on this path (src/model/gguf.h:15-21) */
enum miq_type {
    MIQ_TYPE_Q8_0 = 8,
    MIQ_TYPE_Q4_K = 12,
    MIQ_TYPE_Q5_K = 13,
    MIQ_TYPE_Q6_K = 14,
};

/* One GEMV output segment.  Mirrors gemv_seg (src/backend/gpu/kernels/kernels.h:44-81)
 * and its CPU twin cpu_gemv_seg (src/backend/cpu/cpu_types.h:68-86) field for
 * field on the integer path; `x`/`x_stride`/`act_up` are carried for the
 * caller's xq call and are not read by the GEMV itself.
 * Output is token-major: out[t*out_stride + row] = alpha*acc + residual[same]. */
typedef struct miq_seg {
    const void *w;         /* GGUF blocks [n_rows][K/QK] on the device */
    uint32_t type;         /* enum miq_type */
    int32_t K;             /* input length (multiple of 256 for K-quants, 32 for Q8_0) */
    int32_t n_rows;        /* output rows */
    const float *x;        /* fp32 activations (for miq_xq), row stride x_stride */
    int32_t x_stride;
    const float *act_up;   /* non-null: x is activated as silu(x)*act_up by miq_xq */
    float *out;
    int32_t out_stride;
    const float *residual; /* optional, same layout as out */
    float alpha;
    const int8_t *x8;      /* quantized activation (miq_xq output) */
    const float *xmeta;
    const int32_t *xsumq;
} miq_seg;

/* Library identification and the last error message of this thread. */
const char *miq_version(void);
const char *miq_last_error(void);

/* Bytes of one row of K values in `type` (src/common/quant.h:1177); 0 if unknown. */
size_t miq_row_bytes(uint32_t type, int K);

/* Activation quantizer.  Replaces compute_backend::xq (src/backend/backend.h:104-105),
 * i.e. cpu_xq (src/backend/cpu/kernels/xq.cpp:10) and xq_launch
 * (src/backend/gpu/kernels/kernels.h:440).  Bit-exact with cpu_xq when up == NULL. */
int miq_xq(hipStream_t stream, const float *x, const float *up, int x_stride, int up_stride, int8_t *x8,
           float *xmeta, int32_t *xsumq, int TB, int K);

/* Decode GEMV, one token.  Replaces compute_backend::i8_gemv (src/backend/backend.h:113),
 * i.e. cpu_i8_gemv (src/backend/cpu/kernels/i8.cpp:498); on the GPU side it
 * takes the place of dp4a_gemv_launch (src/backend/gpu/kernels/kernels.h:447). */
int miq_i8_gemv(hipStream_t stream, const miq_seg *seg);

/* Batched decode / chunked-prefill GEMM over TB tokens.  Replaces
 * compute_backend::i8_gemm (src/backend/backend.h:114), i.e. cpu_i8_gemm
 * (src/backend/cpu/kernels/i8.cpp:518), and on the GPU side dp4a_gemm_launch
 * (kernels.h:465) and dnnl_gemm::gemm (src/backend/dnnl_gemm.h:186). */
int miq_i8_gemm(hipStream_t stream, const miq_seg *seg, int TB);

/* Several output segments of one activation in one call: segs[i] carry
 * their own w, type, n_rows, out, out_stride, residual and alpha; every
 * segment must have segs[0]'s K and uses segs[0]'s activation (x8, xmeta,
 * xsumq; the other segments' activation fields are ignored).  Up to 8
 * segments.  At decode sizes (TB <= 3) segments of one type run in a single
 * launch whose workgroups are numbered across them (gate and up of an FFN
 * read as one stream); where every segment takes the split-K 16-token GEMM
 * (4..47 tokens) one launch of it covers all, each segment with the tiles
 * and K slices it has alone; otherwise one launch per segment.  Each segment's
 * outputs equal miq_i8_gemm's for it bit for bit.  Replaces
 * compute_backend::i8_row_gemv_multi (src/backend/backend.h:120-121). */
int miq_i8_gemv_multi(hipStream_t stream, const miq_seg *segs, int n_segs, int TB);

/* The fused form over several segments: quantize segs[0]'s x (and act_up)
 * into segs[0]'s x8/xmeta/xsumq, then every segment as miq_i8_gemv_multi; at
 * one token a single launch does both.  Replaces i8_grp_quant_gemv_launch
 * (src/backend/gpu/kernels/kernels.h:216-219). */
int miq_quant_gemm_multi(hipStream_t stream, const miq_seg *segs, int n_segs, int TB);

/* miq_i8_gemm without any allocation: the split-K partials and arrival
 * counters come from a static device array of the library (16 MiB of partials
 * and 64 Ki counters, held by each GPU the library runs on until the process
 * ends) instead of the grow-on-demand scratch.  No counterpart in the
 * reference: for callers that cannot allocate device memory (code under
 * graph capture that was never warmed up, tight serving loops, harnesses that
 * forbid hipMalloc).  Serves the decode and 16-token kernels (batches that the
 * dispatch gives the fp16 prefill GEMM need a workspace and return
 * MIQ_UNSUPPORTED), and
 * returns MIQ_UNSUPPORTED for a shape whose partials exceed the array.  Every
 * call on one GPU shares its array: calls that overlap on one GPU race. */
int miq_i8_gemm_noalloc(hipStream_t stream, const miq_seg *seg, int TB);

/* The fused form: quantize the segment's activation (x, act_up) into the
 * caller's x8/xmeta/xsumq and run the GEMV/GEMM in one call.  Replaces
 * i8_grp_quant_gemv_launch (src/backend/gpu/kernels/kernels.h:218). */
int miq_quant_gemm(hipStream_t stream, const miq_seg *seg, int TB);

/* Per-group exact int32 dot products of a GEMV/GEMM -- the quantity the
 * reference's fp32 epilogue scales (i8.cpp:49-57,109-118,129-150;
 * q4exp.cpp:457-467).  out[(t*n_rows+row)*S+s], S = K/32 (K/16 for Q6_K).
 * path 0 = the decode kernel's unit decoder, 1 = the 16-token MFMA GEMMs',
 * 2 = the fp16-MFMA prefill GEMM's (it returns sc * dot, the 6-bit group
 * scale folded into the weight operand, exact in fp32; for Q6_K one value per
 * 32-group, S = K/32: sc0 * (dot0 - 32 * xsum0) + sc1 * (dot1 - 32 * xsum1)
 * over its two 16-value sub-groups, i8.cpp:125-155), 3 = the
 * int8-MFMA prefill GEMM's (Q4_K/Q5_K, Q8_0 with K % 256 == 0), 4 = path 1
 * (the split-K and CU-resident 16-token kernels share one decoder per type), 5 = the
 * decode kernel's Q4_K piece decoder (two or more tokens), 6 = the Q8_0
 * kernel for any whole number of 32-value groups (every Q8_0 call with
 * K % 64 == 32 runs it, as does a MoE Q8_0 down bank of such a K; paths 0-5
 * refuse that K).  The MoE experts' grouped GEMV decodes with path 0's unit
 * decoder.  No
 * counterpart in the reference: a parity hook so tests can check the integer
 * core bit-exactly. */
int miq_group_dots(hipStream_t stream, const void *w, uint32_t type, int K, int n_rows, const int8_t *x8,
                   const int32_t *xsumq, int TB, int32_t *out, int path);

/* Set a tuning switch (an A/B form of a kernel choice) by name: M32_MIN_TB,
 * GEMV_MAX_TB, PREFILL_FP16, FUSED_QUANT, M16_WAVES, M16_FORM, MOE_GRP,
 * M32_FILL.  Each
 * starts from the environment variable MIQ_<name> (read once per process) or
 * its default; value INT_MIN restores that.  Every form gives results within
 * the same bounds; the defaults are the measured fastest.  The reference
 * reads its own PF_* switches through si::env (src/common/env.h); this is the
 * library's counterpart, settable at run time. */
int miq_set_switch(const char *name, int value);

/* y[i] = expf(bits(first + i)) for i < count, by the device expf that silu
 * and the router softmax use.  That expf restates the host libm's (glibc)
 * expf, which the reference's cpu_silu and cpu_moe_route call
 * (src/backend/cpu/kernels/common.h:31-33, moe.cpp:107).  No counterpart in
 * the reference: a parity hook so tests can check it against the host expf
 * over whole bit ranges. */
int miq_expf_range(hipStream_t stream, uint32_t first, uint32_t count, float *y);

/* ------------------------------------------------------------------ MoE */

/* Router: logits = gate_inp @ x (fp32 gate_inp [n_expert][n_embd]; with
 * gate_inp == NULL the logits buffer is read as given), softmax, top-k by
 * rank (ties to the lower index), renormalise by max(sum, 6.103515625e-5).
 * Replaces moe_router_launch (kernels.h:595) / cpu_moe_route
 * (src/backend/cpu/kernels/moe.cpp:72).  ids/wts: [n_tok][top_k].  The
 * logits must be finite: a NaN logit makes every probability of its token NaN
 * and the ids unspecified (the reference's rank count then leaves ranks
 * unwritten); here such a token's probabilities sort below every number. */
int miq_moe_route(hipStream_t stream, const float *x, int x_stride, const float *gate_inp, int n_tok, int n_embd,
                  int n_expert, int top_k, float *logits, int32_t *ids, float *wts);

/* Token->expert CSR: off[n_expert+1], pair[n_pairs] (pairs of one expert in
 * ascending pair order), active[n_expert] (experts with >=1 pair, ascending),
 * n_active[1].  Replaces moe_csr_{clear,count,prefix,scatter}_launch
 * (kernels.h:599-606) and the host CSR in moe.cpp:168-185. */
int miq_moe_csr(hipStream_t stream, const int32_t *ids, int n_pairs, int n_expert, int32_t *off, int32_t *pair,
                int32_t *active, int32_t *n_active);

/* Expert banks: expert e's projection starts at bank + e*plane_bytes. */
typedef struct miq_moe {
    const void *gate;
    const void *up;
    const void *down;
    uint32_t gate_type, up_type, down_type;
    size_t gate_plane, up_plane, down_plane;
    int32_t n_embd;   /* K of gate/up, output rows of down */
    int32_t n_ff;     /* output rows of gate/up, K of down */
    int32_t n_expert;
} miq_moe;

/* Workspace the expert call needs for n_pairs routed pairs (device bytes). */
size_t miq_moe_workspace_bytes(const miq_moe *M, int n_tok, int top_k);

/* Routed experts, unweighted: acc[p*acc_stride + r] for every pair p
 * (token p/top_k, expert ids[p]).  Runs, on the stream: CSR, xq(x),
 * grouped gate/up with h = silu(g)*u fused, xq(h), grouped down.  Each active
 * expert's weights are read once for all of its pairs.  Replaces the sequence
 * moe_actq_launch -> moe_grp_gate_up_launch -> moe_actq_launch ->
 * moe_grp_down_launch (kernels.h:626-718; graph.cpp:1011-1082) and, on the
 * CPU, cpu_moe_experts_i8 (moe.cpp:476).  `workspace` holds
 * miq_moe_workspace_bytes() bytes, 256-byte aligned. */
int miq_moe_experts(hipStream_t stream, const miq_moe *M, const float *x, int x_stride, int n_tok, int top_k,
                    const int32_t *ids, float *acc, int acc_stride, void *workspace, size_t workspace_bytes);

/* Weighted reduce: out[t][e] += sum_j wts[t][j]*acc[(t*top_k+j)][e],
 * accumulated in double.  Replaces moe_reduce_launch (kernels.h:753) /
 * cpu_moe_reduce (moe.cpp:562). */
int miq_moe_reduce(hipStream_t stream, const float *acc, const float *wts, int top_k, int n_tok, int n_embd,
                   int acc_stride, float *out, int out_stride);

/* ------------------------------------------------------ host utilities */

/* Encode fp32 rows into GGUF blocks (host memory).  The reference has no
 * K-quant encoder (it only dequantizes); this one follows the published ggml
 * block layout with a min/max fit per group and 6-bit super-block scales.
 * Any valid encoding serves: parity is defined on the produced blocks.
 * No counterpart in the reference. */
int miq_quantize_rows(uint32_t type, const float *x, void *out, int64_t n_rows, int K, int n_threads);


/* ------------------------------------------- u4 native-width store (repack) */
/* The reference's lossless-up-to-f16 repack of Q4_K into a plain nibble plane
 * plus two f16 planes (w4t, src/common/w4.h:55-66):
 *   vals [N][K/2]  element k of row n in byte (n*K+k)/2, low nibble first
 *   scale[g*N+n]   f16 step d*sc_g, off[g*N+n] f16 offset -dmin*m_g (g = k/32),
 *                  both converted with the truncating float->half (quant.h:112-133)
 * 0.625 B per weight against Q4_K's 0.5625. */

/* Replaces w4_pack (src/common/w4.cpp:416-439) for Q4_K at the native group
 * of 32 (pack_q4_K, w4.cpp:160-212); src is the raw Q4_K tensor on the device,
 * the planes are written on the device.  Other types re-quantize lossily in
 * the reference (pack_generic) and return MIQ_UNSUPPORTED here.  K % 256 == 0;
 * src and vals 16-byte aligned. */
int miq_w4_pack(hipStream_t stream, uint32_t type, const void *src, int K, int N, uint8_t *vals, uint16_t *scale,
                uint16_t *off);

/* Per-32-group activation quantizer of the u4 path with the even/odd split.
 * Replaces act_quant_grp_launch with do_split (src/backend/dnnl_gemm.cpp:100-146):
 * xq[m*K+k] int8 (may be NULL); asa[m*K/32+g] f16 scale (round to nearest);
 * xs[m*K/32+g] the group's code sum; axe/axo[m*K/2+j] = xq[2j], xq[2j+1] (both
 * NULL: no split).  With up: the value is silu(x)*up.  x/up 16-byte aligned,
 * strides multiples of 4; xq 16 B, axe/axo 8 B aligned. */
int miq_w4_act(hipStream_t stream, const float *x, const float *up, int x_stride, int up_stride, int M, int K,
               int8_t *xq, uint16_t *asa, float *xs, int8_t *axe, int8_t *axo);

/* One-token GEMV over the u4 store.  Replaces w4_gemv_launch
 * (src/backend/gpu/kernels/kernels.h:240, w4_gemv.cpp:156-187), same arguments:
 *   out[n] = alpha * sum_g asa[g]*(step[g][n]*QDOT_g[n] + off[g][n]*xs[g]) + residual[n]
 * out_stride is unused (one output row, as in the reference).  K % 32 == 0;
 * beyond 6144 the K range is split across workgroups and the parts' sums are
 * added by a second launch (library scratch); vals/axe/axo 16-byte aligned. */
int miq_w4_gemv(hipStream_t stream, const uint8_t *vals, const uint16_t *scale, const uint16_t *off,
                const int8_t *axe, const int8_t *axo, const uint16_t *asa, const float *xs, float *out,
                int out_stride, const float *residual, float alpha, int K, int N);

/* M tokens over the u4 store.  Replaces w4_gemm_launch
 * (src/backend/gpu/kernels/kernels.h:237-239, w4_gemv.cpp:1684-1830), same
 * arguments: activation planes [M][K/2], [M][K/32] as miq_w4_act writes them;
 * out[m*out_stride+n] = alpha * (u4 formula on row m) + residual[m*out_stride+n].
 * Up to eight tokens share each weight read (16-byte aligned scale/off and
 * N % 8 == 0; otherwise token by token); K splits across workgroups where
 * the tokens' activations would not fit the LDS budget. */
int miq_w4_gemm(hipStream_t stream, const uint8_t *vals, const uint16_t *scale, const uint16_t *off,
                const int8_t *axe, const int8_t *axo, const uint16_t *asa, const float *xs, float *out,
                int out_stride, const float *residual, float alpha, int M, int K, int N);

/* Batched native-width GEMM over the u4 (fmt 0) or k5 (fmt 1) store.
 * Replaces nat_gemm_launch (src/backend/gpu/kernels/kernels.h:250-262,
 * w4_gemv.cpp:2403-2503), same arguments: w0 = u4/k5 vals, w1 = the k5 hi
 * plane, scale/off the f16 planes; the activation is miq_w4_act's split planes
 * (axe/axo, asa, xs) for M tokens; out[m*out_stride+n] = alpha * (u4 formula
 * on token m) + residual[m*out_stride+n].  Chunks of up to eight tokens share
 * each weight read (16-byte aligned scale/off and N % 8 == 0; otherwise token
 * by token).  w8, lut16, bit_lut and axg belong to the cb4 and grouped-int8
 * stores (fmt 2, 3), which are not built here: MIQ_UNSUPPORTED.  Where the
 * reference's launcher returns false (M outside 2..32, k5 beyond 13 tokens,
 * K % 32 != 0) this returns MIQ_UNSUPPORTED and launches nothing. */
int miq_nat_gemm(hipStream_t stream, int fmt, const void *w0, const void *w1, const int8_t *w8,
                 const uint16_t *scale, const uint16_t *off, const uint16_t *lut16, const uint32_t *bit_lut,
                 const int8_t *axe, const int8_t *axo, const int8_t *axg, const uint16_t *asa, const float *xs,
                 float *out, int out_stride, const float *residual, float alpha, int M, int K, int N);

/* One u4 output segment of a fused call; mirrors w4_grp_seg
 * (src/backend/gpu/kernels/kernels.h:226-234) field for field. */
typedef struct miq_w4_seg {
    const uint8_t *vals;   /* [n_rows][K/2] nibble plane */
    const uint16_t *scale; /* [K/32][n_rows] f16 step plane */
    const uint16_t *off;   /* [K/32][n_rows] f16 offset plane */
    int32_t n_rows;
    float *out;            /* out[n] = alpha*acc + residual[n] */
    float alpha;
    const float *residual;
} miq_w4_seg;

/* One token: quantize x (silu(x)*up with up) as miq_w4_act does and run every
 * segment's u4 GEMV in the same launch.  Replaces w4_grp_quant_gemv_launch
 * (src/backend/gpu/kernels/kernels.h:216-236, w4_gemv.cpp:747-937); bit-identical
 * to miq_w4_act + one miq_w4_gemv per segment.  total_rows = sum of n_rows;
 * at most 8 segments; x/up 16-byte aligned.  MIQ_UNSUPPORTED (nothing
 * launched) where the reference's launcher returns false: K beyond what one
 * workgroup quantizes (K <= 8192). */
int miq_w4_quant_gemv(hipStream_t stream, const miq_w4_seg *segs, int n_segs, int total_rows, const float *x,
                      const float *up, int K);

/* The reference's native 5-bit store of Q5_K (k5t, src/common/w4.h:104-132):
 * the u4 nibble plane of the low four bits, plus
 *   hi[N][K/8]  per 32-group one 32-bit word: bit i = fifth bit of element 2i,
 *               bit 16+i = fifth bit of element 2i+1
 * and the same scale/off planes (step d*sc_g, offset -dmin*m_g).  0.75 B per
 * weight against Q5_K's 0.6875.  Replaces k5_pack (w4.cpp:336-403,409-414);
 * src is the raw Q5_K tensor on the device.  K % 256 == 0; src and vals
 * 16-byte aligned, hi 4-byte aligned. */
int miq_k5_pack(hipStream_t stream, uint32_t type, const void *src, int K, int N, uint8_t *vals, uint8_t *hi,
                uint16_t *scale, uint16_t *off);

/* One-token GEMV over the k5 store.  Replaces k5_gemv_launch
 * (src/backend/gpu/kernels/kernels.h:263-269, w4_gemv.cpp:1002-1099), same
 * arguments; the activation is miq_w4_act's.  q5 = lo4 | bit << 4, then the
 * u4 formula.  Limits as miq_w4_gemv. */
int miq_k5_gemv(hipStream_t stream, const uint8_t *vals, const uint8_t *hi, const uint16_t *scale,
                const uint16_t *off, const int8_t *axe, const int8_t *axo, const uint16_t *asa, const float *xs,
                float *out, const float *residual, float alpha, int K, int N);

/* ------------------------------------------------------ GGUF files */

/* Per-type block geometry (src/model/gguf.cpp:13-100: ggml_type_name,
 * ggml_blck_size, ggml_type_size, ggml_row_bytes).  An unknown type is "?"
 * or 0 here where the reference throws; row bytes are 0 when n is not a
 * whole number of blocks. */
const char *miq_ggml_type_name(uint32_t type);
size_t miq_ggml_blck_size(uint32_t type);
size_t miq_ggml_type_size(uint32_t type);
size_t miq_ggml_row_bytes(uint32_t type, uint64_t n_elems);

/* An open GGUF model, mapped read-only.  Replaces gguf_file
 * (src/model/gguf.h:102-158).  A file named "...-IIIII-of-NNNNN.gguf" is one
 * shard of a split model: all NNNNN shards are opened and placed in one
 * contiguous reservation, so map_offset below is one offset space over the
 * whole model (gguf.h:103-107, gguf.cpp:345-456). */
typedef struct miq_gguf miq_gguf;
typedef struct miq_gguf_val miq_gguf_val;

typedef struct miq_gguf_desc {
    uint32_t version;
    int32_t n_shards;
    int64_t n_tensors;
    int64_t n_kv;
    int32_t split_count;    /* split.count of the first shard, else the shard count; 1 when single */
    int32_t split_no;       /* split.no of the first shard, else 0 */
    const void *map_base;   /* the whole mapping (reservation for a split model) */
    size_t map_size;
    size_t data_offset;     /* first shard's data section */
} miq_gguf_desc;

typedef struct miq_gguf_shard_info {
    const void *base;       /* inside the mapping */
    size_t size;            /* file bytes */
    size_t data_offset;
} miq_gguf_shard_info;

/* gguf_tensor_info (gguf.h:64-93); pointers stay valid until miq_gguf_close. */
typedef struct miq_gguf_tensor_info {
    const char *name;
    uint32_t type;          /* ggml type id */
    uint32_t n_dims;
    const uint64_t *dims;   /* dims[0] innermost (ggml ne[0]) */
    uint64_t n_elements;
    uint64_t n_rows;        /* product of dims[1:] */
    uint64_t nbytes;        /* 0 for a type without a known block size */
    uint64_t offset;        /* relative to its shard's data section */
    const void *data;       /* host address in the mapping */
    uint64_t map_offset;    /* data - map_base */
    int32_t shard;
} miq_gguf_tensor_info;

/* One kv value, widened as gguf_kv (gguf.h:38-62): integer types in u64 and
 * i64 (sign of their type), float32/float64 in f64, bool 0/1, string in
 * str/str_len, array: n elements of arr_type (read with miq_gguf_val_elem). */
typedef struct miq_gguf_kv {
    uint32_t type;          /* GGUF value type 0..12 */
    uint32_t arr_type;
    uint64_t u64;
    int64_t i64;
    double f64;
    const char *str;
    uint64_t str_len;
    uint64_t n;
} miq_gguf_kv;

/* gguf_file::load (gguf.cpp:345).  NULL on error, with the reference's
 * exception text in miq_last_error() ("not a gguf file", "gguf: unexpected
 * end of file", "gguf: bad data offset", "gguf: split.count does not match
 * the shard file names", ...). */
miq_gguf *miq_gguf_open(const char *path);
/* ~gguf_file (gguf.cpp:183): unmaps and closes every shard. */
void miq_gguf_close(miq_gguf *f);
int miq_gguf_describe(const miq_gguf *f, miq_gguf_desc *out);
/* gguf_file::shards (gguf.h:108-113) */
int miq_gguf_shard(const miq_gguf *f, int i, miq_gguf_shard_info *out);
/* gguf_file::find (gguf.h:136): index of the tensor, -1 when absent. */
int64_t miq_gguf_find(const miq_gguf *f, const char *name);
/* gguf_file::tensors[i] */
int miq_gguf_tensor(const miq_gguf *f, int64_t i, miq_gguf_tensor_info *out);
/* i-th key in sorted order (gguf_file::kv is a std::map), NULL past the end. */
const char *miq_gguf_kv_key(const miq_gguf *f, int64_t i);
/* gguf_file::meta (gguf.h:140): NULL when absent. */
const miq_gguf_val *miq_gguf_meta(const miq_gguf *f, const char *key);
int miq_gguf_val_read(const miq_gguf_val *v, miq_gguf_kv *out);
/* i-th element of an array value, NULL when not an array or out of range. */
const miq_gguf_val *miq_gguf_val_elem(const miq_gguf_val *v, uint64_t i);
/* gguf_file::get_u32 / get_f32 / get_str (gguf.h:144-157). */
uint32_t miq_gguf_get_u32(const miq_gguf *f, const char *key, uint32_t def);
float miq_gguf_get_f32(const miq_gguf *f, const char *key, float def);
const char *miq_gguf_get_str(const miq_gguf *f, const char *key);
/* gguf_file::drop_cache (gguf.cpp:199): drop page cache behind mapping
 * bytes [off, off+len), clipped to each shard's file bytes. */
int miq_gguf_drop_cache(const miq_gguf *f, uint64_t off, uint64_t len);
/* Copy mapping bytes [off, off+len) to device memory `dst` through pinned
 * staging chunks on `stream`; returns when the bytes are on the device.
 * Padding between split shards arrives as zeros.  Takes the place of the
 * contiguous upload weight_store::upload_contiguous (src/backend/weight_store.h:37;
 * no eviction or residency policy).  The staging buffers belong to `f`. */
int miq_gguf_upload(hipStream_t stream, miq_gguf *f, uint64_t off, uint64_t len, void *dst);

#ifdef __cplusplus
}
#endif
#endif /* MIQ_H */
