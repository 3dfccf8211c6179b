// Entry points of the GEMV/GEMM family and the kernel choice by batch size.
//
//   TB <= 3 (and the activation fits LDS)  dot4 GEMV (miq_gemv.hip)
//   TB >= 48, Q4_K/Q5_K/Q6_K               exact fp16-MFMA GEMM, stream-K schedule (miq_pf16.hip),
//                                          where its cost model beats the 16-token kernel;
//                                          MIQ_PREFILL_FP16=0: the int8 kernel below
//   TB >= 48, Q8_0 (and the switch above)  LDS-tiled 32x32 int8-MFMA GEMM (miq_mfma32.hip);
//                                          Q6_K only when its tiles cover every CU
//   otherwise                              16-token int8-MFMA GEMM (miq_mfma16.hip)
// The switch M32_MIN_TB (miq_set_switch, env MIQ_M32_MIN_TB) moves the second
// threshold.
#include "miq_internal.h"

namespace miq {

namespace {
enum Route { kRouteGemv, kRoutePf16, kRouteM32, kRouteM16, kRouteQ80, kRouteNone };

Route route(const miq_seg *s, int TB) {
    if (q80_any(s)) return kRouteQ80;  // Q8_0 with an odd group count: its own kernel at every batch size
    const int min_tb32 = sw(kSwM32MinTb);
    // GEMV_MAX_TB: the largest batch the dot4 GEMV takes (an A/B switch)
    const int gemv_max = sw(kSwGemvMaxTb);
    if (TB <= gemv_max && gemv_fits(s, TB)) return kRouteGemv;
    // PREFILL_FP16: 1 (default) the fp16 GEMM where its cost model beats the
    // 16-token kernel, 2 the fp16 GEMM at every prefill size, 0 the int8
    // tiled kernel instead (A/B switches)
    const int pf_mode = sw(kSwPrefillFp16);
    const bool pf16 = pf_mode == 2 || (pf_mode == 1 && pf16_serves(s) && pf16_prefers(s, TB));
    if (TB >= min_tb32 && pf16 && pf16_serves(s)) return kRoutePf16;
    if (TB >= min_tb32 && (pf_mode == 0 || !pf16_serves(s)) && mfma32_serves(s) && mfma32_fills(s, TB))
        return kRouteM32;
    if (mfma16_fits(s)) return kRouteM16;
    return kRouteNone;
}
}  // namespace

int run_gemm(hipStream_t stream, const miq_seg *s, int TB, const char *who) {
    const int rc = check_seg(s, TB, who);
    if (rc != MIQ_OK) return rc;
    switch (route(s, TB)) {
    case kRouteGemv: return launch_gemv(stream, s, TB);
    case kRoutePf16: return launch_pf16(stream, s, TB);
    case kRouteM32: return launch_mfma32(stream, s, TB);
    case kRouteM16: return launch_mfma16(stream, s, TB);
    case kRouteQ80: return launch_q80(stream, s, TB);
    default: break;
    }
    set_error("%s: K=%d too long for the kernels' LDS staging", who, s->K);
    return MIQ_UNSUPPORTED;
}

// Segments of one activation past the GEMV's batch sizes: one launch of the
// split-K 16-token kernel when every segment goes there, else one call each.
int run_gemm_multi(hipStream_t stream, const miq_seg *s, int n_segs, int TB, bool one_type, const char *who) {
    bool m16 = one_type;
    for (int i = 0; m16 && i < n_segs; i++) m16 = route(&s[i], TB) == kRouteM16;
    if (m16) return launch_mfma16_multi(stream, s, n_segs, TB);
    for (int i = 0; i < n_segs; i++)
        if (const int rc = run_gemm(stream, &s[i], TB, who)) return rc;
    return MIQ_OK;
}

}  // namespace miq

extern "C" {

int miq_i8_gemv(hipStream_t stream, const miq_seg *seg) { return miq::run_gemm(stream, seg, 1, "miq_i8_gemv"); }

int miq_i8_gemm(hipStream_t stream, const miq_seg *seg, int TB) {
    return miq::run_gemm(stream, seg, TB, "miq_i8_gemm");
}

int miq_quant_gemm(hipStream_t stream, const miq_seg *seg, int TB) {
    const int rc = miq::check_seg(seg, TB, "miq_quant_gemm");
    if (rc != MIQ_OK) return rc;
    if (!seg->x) {
        miq::set_error("miq_quant_gemm: seg->x is null");
        return MIQ_EINVAL;
    }
    // one token on the GEMV: quantize inside the GEMV launch (f1, the
    // reference's i8_grp_quant_gemv_launch, kernels.h:216-236)
    const int gemv_max = miq::sw(miq::kSwGemvMaxTb);
    if (miq::sw(miq::kSwFusedQuant) && TB <= gemv_max && miq::gemv_quant_fits(seg, TB)) return miq::launch_gemv(stream, seg, TB, true);
    const int q = miq::launch_xq(stream, seg->x, seg->act_up, seg->x_stride, seg->x_stride,
                                 const_cast<int8_t *>(seg->x8), const_cast<float *>(seg->xmeta),
                                 const_cast<int32_t *>(seg->xsumq), TB, seg->K);
    if (q != MIQ_OK) return q;
    return miq::run_gemm(stream, seg, TB, "miq_quant_gemm");
}

namespace {
// The segments of a multi call: each checked, and each given segs[0]'s
// activation (the shared x8/xmeta/xsumq and, for the fused form, x/act_up).
int multi_segs(const miq_seg *segs, int n_segs, int TB, const char *who, miq_seg *out, bool &one_launch) {
    if (!segs || n_segs < 1 || n_segs > 8) {
        miq::set_error("%s: %d segments (1..8 per call)", who, n_segs);
        return MIQ_EINVAL;
    }
    one_launch = true;
    for (int i = 0; i < n_segs; i++) {
        out[i] = segs[i];
        out[i].x8 = segs[0].x8;
        out[i].xmeta = segs[0].xmeta;
        out[i].xsumq = segs[0].xsumq;
        out[i].x = segs[0].x;
        out[i].x_stride = segs[0].x_stride;
        out[i].act_up = segs[0].act_up;
        if (const int rc = miq::check_seg(&out[i], TB, who)) return rc;
        if (out[i].K != segs[0].K) {
            miq::set_error("%s: segment %d has K=%d, segment 0 K=%d (one shared activation)", who, i, out[i].K, segs[0].K);
            return MIQ_EINVAL;
        }
        one_launch = one_launch && out[i].type == segs[0].type;
    }
    return MIQ_OK;
}
}  // namespace

int miq_i8_gemv_multi(hipStream_t stream, const miq_seg *segs, int n_segs, int TB) {
    miq_seg s[8];
    bool one = false;
    if (const int rc = multi_segs(segs, n_segs, TB, "miq_i8_gemv_multi", s, one)) return rc;
    if (one && TB <= miq::sw(miq::kSwGemvMaxTb) && miq::gemv_fits(&s[0], TB))
        return miq::launch_gemv_multi(stream, s, n_segs, TB);
    return miq::run_gemm_multi(stream, s, n_segs, TB, one, "miq_i8_gemv_multi");
}

int miq_quant_gemm_multi(hipStream_t stream, const miq_seg *segs, int n_segs, int TB) {
    miq_seg s[8];
    bool one = false;
    if (const int rc = multi_segs(segs, n_segs, TB, "miq_quant_gemm_multi", s, one)) return rc;
    if (!s[0].x) {
        miq::set_error("miq_quant_gemm_multi: segs[0].x is null");
        return MIQ_EINVAL;
    }
    if (one && miq::sw(miq::kSwFusedQuant) && TB <= miq::sw(miq::kSwGemvMaxTb) && miq::gemv_quant_fits(&s[0], TB))
        return miq::launch_gemv_multi(stream, s, n_segs, TB, true);
    const int q = miq::launch_xq(stream, s[0].x, s[0].act_up, s[0].x_stride, s[0].x_stride,
                                 const_cast<int8_t *>(s[0].x8), const_cast<float *>(s[0].xmeta),
                                 const_cast<int32_t *>(s[0].xsumq), TB, s[0].K);
    if (q != MIQ_OK) return q;
    if (one && TB <= miq::sw(miq::kSwGemvMaxTb) && miq::gemv_fits(&s[0], TB))
        return miq::launch_gemv_multi(stream, s, n_segs, TB);
    return miq::run_gemm_multi(stream, s, n_segs, TB, one, "miq_quant_gemm_multi");
}

int miq_group_dots(hipStream_t stream, const void *w, uint32_t type, int K, int n_rows, const int8_t *x8,
                   const int32_t *xsumq, int TB, int32_t *out, int path) {
    miq_seg s{};
    s.w = w;
    s.type = type;
    s.K = K;
    s.n_rows = n_rows;
    s.x8 = x8;
    s.out = reinterpret_cast<float *>(out);
    s.out_stride = n_rows;
    s.xsumq = xsumq;
    s.xmeta = reinterpret_cast<const float *>(xsumq);  // not read; satisfies the null check
    const int rc = miq::check_seg(&s, TB, "miq_group_dots");
    if (rc != MIQ_OK) return rc;
    if (path == 6) {
        if (type != MIQ_TYPE_Q8_0) {
            miq::set_error("miq_group_dots: path 6 (the any-group-count Q8_0 decoder) serves Q8_0");
            return MIQ_UNSUPPORTED;
        }
        return miq::launch_q80(stream, &s, TB, out);
    }
    if (miq::q80_any(&s)) {
        miq::set_error("miq_group_dots: Q8_0 with K %% 64 == 32 is served by path 6 only");
        return MIQ_UNSUPPORTED;
    }
    if (path == 0) return miq::launch_unit_dots(stream, &s, TB, out);
    // paths 1 and 4 both name the 16-token kernels' decoders (the split-K
    // and CU-resident forms share one per type)
    if (path == 1 || path == 4) return miq::launch_mfma16_dots(stream, &s, TB, out);
    if (path == 2) return miq::launch_pf16_dots(stream, &s, TB, out);
    if (path == 5) return miq::launch_piece_dots(stream, &s, TB, out);
    if (path == 3) {
        if (!miq::mfma32_serves(&s)) {
            miq::set_error("miq_group_dots: path 3 (the int8 prefill decoder) serves Q4_K, Q5_K and Q8_0 with K %% 256 == 0");
            return MIQ_UNSUPPORTED;
        }
        return miq::launch_mfma32(stream, &s, TB, out);
    }
    miq::set_error("miq_group_dots: unknown path %d", path);
    return MIQ_EINVAL;
}

}  // extern "C"
