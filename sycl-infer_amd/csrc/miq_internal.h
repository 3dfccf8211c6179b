// Launchers shared between the miq translation units.
#pragma once

#include "miq_common.h"

namespace miq {

// Per-device split-K scratch (partial tiles + zeroed arrival counters).  Grown
// only outside stream capture (MIQ_UNSUPPORTED if `stream` captures and the
// buffers are too small).
int scratch_get(hipStream_t stream, size_t part_bytes, size_t n_cnt, float **part, uint32_t **cnt);
// Per-device workspace buffers, one per slot, grown on demand (same lifetime,
// sharing and capture rules as the split-K scratch).  `zero`: a new
// allocation is zero-filled (arrival counters that their users return to zero).
enum { kWsPrefill = 0, kWsPrefillCnt = 1, kWsW4Part = 2, kWsSlots = 4 };
int workspace_get(hipStream_t stream, int slot, size_t bytes, void **ptr, bool zero = false);
// Tuning switches (A/B forms of the kernels).  Each starts from the
// environment variable MIQ_<name>, read once per process, else its default;
// miq_set_switch() changes it at run time.
enum Switch {
    kSwM32MinTb, kSwGemvMaxTb, kSwPrefillFp16, kSwFusedQuant, kSwM16Waves, kSwM16Form, kSwMoeGrp, kSwM32Fill, kSwCount
};
int sw(Switch s);
// Compute units of the current device (queried once per device).
int device_cus(int *n);

int check_seg(const miq_seg *s, int TB, const char *who);
int launch_xq(hipStream_t stream, const float *x, const float *up, int x_stride, int up_stride, int8_t *x8,
              float *xmeta, int32_t *xsumq, int TB, int K, int layout = 0);

// dot4 decode GEMV (TB <= 4, activation staged in LDS)
bool gemv_fits(const miq_seg *s, int TB);
int launch_gemv(hipStream_t stream, const miq_seg *s, int TB, bool quant = false);
// every segment in one launch: same type and K, one shared activation (segs[0]'s)
int launch_gemv_multi(hipStream_t stream, const miq_seg *segs, int n_segs, int TB, bool quant = false);
// the one-token GEMV that quantizes seg->x itself (miq_quant_gemm in one launch)
bool gemv_quant_fits(const miq_seg *s, int TB);
int launch_piece_dots(hipStream_t stream, const miq_seg *s, int TB, int32_t *out);
int launch_unit_dots(hipStream_t stream, const miq_seg *s, int TB, int32_t *out);

// int8-MFMA GEMM in 16-token tiles
bool mfma16_fits(const miq_seg *s);
int launch_mfma16(hipStream_t stream, const miq_seg *s, int TB);
int launch_mfma16_multi(hipStream_t stream, const miq_seg *segs, int n_segs, int TB);
int launch_mfma16_dots(hipStream_t stream, const miq_seg *s, int TB, int32_t *out);

// LDS-tiled int8-MFMA GEMM for prefill-sized batches (Q4_K, Q5_K, Q8_0)
bool mfma32_serves(const miq_seg *s);
// Q6_K: the tiled kernel has no K split, so it takes a batch only when its
// tiles cover every CU (else the split-K 16-token kernel is faster)
bool mfma32_fills(const miq_seg *s, int TB);
int launch_mfma32(hipStream_t stream, const miq_seg *s, int TB, int32_t *dots = nullptr);

// fp16-MFMA exact prefill GEMM (Q4_K, Q5_K)
bool pf16_serves(const miq_seg *s);
bool pf16_prefers(const miq_seg *s, int TB);
int launch_pf16(hipStream_t stream, const miq_seg *s, int TB);
int launch_pf16_dots(hipStream_t stream, const miq_seg *s, int TB, int32_t *out);


// Q8_0 rows of any whole number of 32-value groups (the kernels above walk
// 64-value units: K % 64 == 32 comes here); dots != nullptr: the parity form
bool q80_any(const miq_seg *s);
int launch_q80(hipStream_t stream, const miq_seg *s, int TB, int32_t *dots = nullptr);
// the same over expert banks: pair p (activation token p) reads bank ids[p]
int launch_q80_banked(hipStream_t stream, const void *bank, size_t plane, int n_bank, int K, int n_rows,
                      const int8_t *x8, const float *xmeta, int n_pairs, const int32_t *ids, float *out,
                      int out_stride);

// Route a seg to the kernel that serves TB tokens.
int run_gemm(hipStream_t stream, const miq_seg *s, int TB, const char *who);
int run_gemm_multi(hipStream_t stream, const miq_seg *s, int n_segs, int TB, bool one_type, const char *who);

}  // namespace miq
