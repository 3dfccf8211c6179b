/*
 * miq oracle -- TEST INFRASTRUCTURE ONLY (see miq_oracle.h).  Scalar C
 * restatement of sycl-infer's CPU integer quantized-matmul path; the checker,
 * never the thing measured or shipped.
 */
#include "miq_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------ f16 helpers */

/* src/common/quant.h:67-92 */
float miqo_half_to_float(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) & 1u;
    uint32_t exp = (uint32_t)(h >> 10) & 0x1Fu;
    uint32_t mant = (uint32_t)h & 0x3FFu;
    uint32_t bits;
    if (exp == 0) {
        if (mant == 0) {
            bits = sign << 31;
        } else {
            /* normalise the subnormal: shift until the implicit bit appears */
            int e = 1;
            while (!(mant & 0x400u)) {
                mant <<= 1;
                e--;
            }
            mant &= 0x3FFu;
            bits = (sign << 31) | ((uint32_t)(e + 127 - 15) << 23) | (mant << 13);
        }
    } else if (exp == 31) {
        bits = (sign << 31) | 0x7F800000u | (mant << 13);
    } else {
        bits = (sign << 31) | ((exp + 127 - 15) << 23) | (mant << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* src/common/quant.h:112-133: truncation toward zero on the normal range,
 * truncated subnormals, overflow to infinity. */
uint16_t miqo_float_to_half(float f) {
    uint32_t bits;
    memcpy(&bits, &f, 4);
    const uint32_t sign = (bits >> 16) & 0x8000u;
    const int32_t e32 = (int32_t)((bits >> 23) & 0xFFu);
    const int32_t e16 = e32 - 127 + 15;
    const uint32_t mant = bits & 0x7FFFFFu;
    if (e16 >= 31) return (uint16_t)(sign | 0x7C00u);
    if (e16 <= 0) {
        const int32_t shift = 126 - e32; /* value = (mant|2^23) * 2^(e32-150) = h * 2^-24 */
        if (shift >= 32) return (uint16_t)sign;
        return (uint16_t)(sign | ((mant | 0x800000u) >> shift));
    }
    return (uint16_t)(sign | ((uint32_t)e16 << 10) | (mant >> 13));
}

/* src/common/quant.h:136-144: 6-bit (scale, min) of group j from scales[12] */
void miqo_get_scale_min_k4(int j, const uint8_t *q, uint8_t *d, uint8_t *m) {
    if (j < 4) {
        *d = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *d = (uint8_t)((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

static uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* Block byte sizes, src/common/quant.h:12-41 */
enum { Q4K_BYTES = 144, Q5K_BYTES = 176, Q6K_BYTES = 210, Q80_BYTES = 34 };

size_t miqo_row_bytes(uint32_t type, int K) {
    switch (type) {
    case MIQO_Q4_K: return (size_t)(K / 256) * Q4K_BYTES;
    case MIQO_Q5_K: return (size_t)(K / 256) * Q5K_BYTES;
    case MIQO_Q6_K: return (size_t)(K / 256) * Q6K_BYTES;
    case MIQO_Q8_0: return (size_t)(K / 32) * Q80_BYTES;
    default: return 0;
    }
}

/* ------------------------------------------------------- integer codes */
/* The unsigned code of element i (0..255) of one K-quant block, exactly as the
 * integer kernels extract it:
 *   Q4_K  nibble of qs[(g/2)*32 + i%32], low for even g (i8.cpp:49-52)
 *   Q5_K  + 16 when bit g of qh[i%32] is set (i8.cpp:110-113)
 *   Q6_K  lo4 | 2-bit plane << 4, with the plane/half mapping of i8.cpp:129-144
 * Layout offsets: Q4_K {d@0, dmin@2, scales@4, qs@16}; Q5_K {.., qh@16, qs@48};
 * Q6_K {ql@0, qh@128, scales@192, d@208}. */
static int code_q4k(const uint8_t *blk, int i) {
    const int g = i / 32, l = i % 32;
    const uint8_t b = blk[16 + (g / 2) * 32 + l];
    return (g & 1) ? (b >> 4) : (b & 0xF);
}
static int code_q5k(const uint8_t *blk, int i) {
    const int g = i / 32, l = i % 32;
    const uint8_t b = blk[48 + (g / 2) * 32 + l];
    int q = (g & 1) ? (b >> 4) : (b & 0xF);
    if ((blk[16 + l] >> g) & 1) q |= 16;
    return q;
}
static int code_q6k(const uint8_t *blk, int i) {
    /* sub-group s = i/16 -> blk2 = s>>3, plane = (s&7)>>1, half = s&1 */
    const int s = i / 16, l16 = i % 16;
    const int blk2 = s >> 3, s8 = s & 7, plane = s8 >> 1, half = s8 & 1;
    const uint8_t *ql = blk + blk2 * 64 + ((plane == 1 || plane == 3) ? 32 : 0) + half * 16;
    const uint8_t *qh = blk + 128 + blk2 * 32 + half * 16;
    const int lo = (plane >= 2) ? (ql[l16] >> 4) : (ql[l16] & 0xF);
    const int two = (qh[l16] >> (2 * plane)) & 3;
    return lo | (two << 4);
}

/* ------------------------------------------------------------ dequant */
/* src/common/quant.h:148-210 (Q4_K/Q5_K/Q6_K/Q8_0), one row of K values */
void miqo_dequantize_row(uint32_t type, const void *row, float *y, int K) {
    const uint8_t *p = (const uint8_t *)row;
    if (type == MIQO_Q8_0) {
        for (int b = 0; b < K / 32; b++) {
            const uint8_t *blk = p + (size_t)b * Q80_BYTES;
            const float d = miqo_half_to_float(rd16(blk));
            for (int i = 0; i < 32; i++) y[b * 32 + i] = d * (float)(int8_t)blk[2 + i];
        }
        return;
    }
    const size_t bb = miqo_row_bytes(type, 256);
    for (int b = 0; b < K / 256; b++) {
        const uint8_t *blk = p + (size_t)b * bb;
        float *yb = y + b * 256;
        if (type == MIQO_Q6_K) {
            const float d = miqo_half_to_float(rd16(blk + 208));
            for (int i = 0; i < 256; i++) {
                /* scale index follows the element's 16-wide sub-group in the
                 * storage order of quant.h:195-211: positions n*128 + plane*32 + l
                 * use sc[n*8 + plane*2 + l/16]. */
                const int n = i / 128, r = i % 128, plane = r / 32, l = r % 32;
                const int s_idx = n * 8 + plane * 2 + l / 16;
                /* the code at that position: sub-group (n*8 + plane*2 + l/16) */
                const int code = code_q6k(blk, s_idx * 16 + (l % 16));
                yb[i] = d * (float)(int8_t)blk[192 + s_idx] * (float)(int8_t)(code - 32);
            }
        } else {
            const float d = miqo_half_to_float(rd16(blk));
            const float mn = miqo_half_to_float(rd16(blk + 2));
            for (int g = 0; g < 8; g++) {
                uint8_t sc, m;
                miqo_get_scale_min_k4(g, blk + 4, &sc, &m);
                const float d1 = d * sc, m1 = mn * m;
                for (int l = 0; l < 32; l++) {
                    const int q = (type == MIQO_Q4_K) ? code_q4k(blk, g * 32 + l) : code_q5k(blk, g * 32 + l);
                    yb[g * 32 + l] = d1 * (float)q - m1;
                }
            }
        }
    }
}

/* ------------------------------------------------------------------ xq */
float miqo_silu(float x) { return x / (1.0f + expf(-x)); }

static int same_f32(float a, float b) {
    uint32_t ua, ub;
    memcpy(&ua, &a, 4);
    memcpy(&ub, &b, 4);
    return ua == ub || (isnan(a) && isnan(b));
}

uint64_t miqo_expf_mismatches(uint32_t first, uint32_t count, const float *y, uint32_t *first_bad) {
    uint64_t bad = 0;
    for (uint32_t i = 0; i < count; i++) {
        const uint32_t u = first + i;
        float x;
        memcpy(&x, &u, 4);
        if (!same_f32(expf(x), y[i]) && bad++ == 0 && first_bad) *first_bad = u;
    }
    return bad;
}

/* glibc's expf (sysdeps/ieee754/flt-32/e_expf.c, from Arm optimized-routines):
 * k = round(x*32/ln2) by the 1.5*2^52 shift, r = x*32/ln2 - k,
 * expf(x) = 2^(k/32) * (1 + c2 r + c1 r^2 + c0 r^3), the double 2^(k/32) from a
 * table of 2^(i/32) with k/32's integer part added to the exponent field.  The
 * x86-64 FMA build fuses x*32/ln2 into both the shift and r. */
static uint64_t expf_tab[32];
__attribute__((constructor)) static void expf_tab_init(void) {
    /* tab[i] = bits(2^(i/32)) - (i << 47), from exp2 in double */
    for (int i = 0; i < 32; i++) {
        double v = exp2((double)i / 32.0);
        uint64_t b;
        memcpy(&b, &v, 8);
        expf_tab[i] = b - ((uint64_t)i << 47);
    }
}

float miqo_expf_method(float x) {
    const uint64_t *tab = expf_tab;
    const double inv_ln2_n = 0x1.71547652b82fep+0 * 32.0, shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / 32.0 / 32.0 / 32.0, c1 = 0x1.ebfce50fac4f3p-3 / 32.0 / 32.0,
                 c2 = 0x1.62e42ff0c52d6p-1 / 32.0;
    uint32_t ux;
    memcpy(&ux, &x, 4);
    const uint32_t abstop = (ux >> 20) & 0x7ffu;
    if (abstop >= 0x42bu) {
        if (ux == 0xff800000u) return 0.0f;
        if (abstop >= 0x7f8u) return x + x;
        if (x > 0x1.62e42ep6f) return INFINITY;
        if (x < -0x1.9fe368p6f) return 0.0f;
    }
    double kd = fma(inv_ln2_n, (double)x, shift);
    uint64_t ki;
    memcpy(&ki, &kd, 8);
    kd -= shift;
    const double r = fma(inv_ln2_n, (double)x, -kd);
    const uint64_t tb = tab[ki & 31] + (ki << 47);
    double s;
    memcpy(&s, &tb, 8);
    const double z = fma(c0, r, c1);
    double y = fma(c2, r, 1.0);
    y = fma(z, r * r, y);
    return (float)(y * s);
}

uint64_t miqo_expf_method_mismatches(uint32_t first, uint32_t count, uint32_t *first_bad) {
    uint64_t bad = 0;
    for (uint32_t i = 0; i < count; i++) {
        const uint32_t u = first + i;
        float x;
        memcpy(&x, &u, 4);
        if (!same_f32(expf(x), miqo_expf_method(x)) && bad++ == 0 && first_bad) *first_bad = u;
    }
    return bad;
}

/* src/backend/cpu/kernels/xq.cpp:10-50 */
void miqo_xq(const float *x, const float *up, int x_stride, int up_stride, int8_t *x8, float *xmeta,
             int32_t *xsumq, int TB, int K) {
    const int G = K / 32;
    for (int t = 0; t < TB; t++) {
        for (int g = 0; g < G; g++) {
            float v[32];
            float mx = 0.0f;
            for (int i = 0; i < 32; i++) {
                float a = x[(size_t)t * x_stride + g * 32 + i];
                if (up) a = miqo_silu(a) * up[(size_t)t * up_stride + g * 32 + i];
                v[i] = a;
                const float fa = fabsf(a);
                mx = mx < fa ? fa : mx; /* std::max(mx, |a|) */
            }
            const float scale = mx > 0.0f ? mx / 127.0f : 1.0f;
            const float inv = mx > 0.0f ? 127.0f / mx : 0.0f;
            int32_t s0 = 0, s1 = 0;
            int8_t *dst = x8 + ((size_t)g * TB + t) * 32;
            for (int i = 0; i < 32; i++) {
                float r = roundf(v[i] * inv);
                r = r < 127.0f ? r : 127.0f;   /* std::min(127, r) */
                r = -127.0f > r ? -127.0f : r; /* std::max(-127, .) */
                const int32_t q = (int32_t)r;
                dst[i] = (int8_t)q;
                if (i < 16) s0 += q; else s1 += q;
            }
            const size_t gi = (size_t)g * TB + t;
            xmeta[gi * 2] = miqo_half_to_float(miqo_float_to_half(mx > 0.0f ? scale : 0.0f));
            xmeta[gi * 2 + 1] = 0.0f;
            xsumq[gi * 2 + 0] = s0;
            xsumq[gi * 2 + 1] = s1;
        }
    }
}

/* ---------------------------------------------------------- group dots */
static int32_t dot_group(uint32_t type, const uint8_t *row, int K, const int8_t *x8, int TB, int t, int s) {
    int32_t acc = 0;
    if (type == MIQO_Q8_0) {
        const uint8_t *blk = row + (size_t)s * Q80_BYTES;
        const int8_t *xv = x8 + ((size_t)s * TB + t) * 32;
        for (int i = 0; i < 32; i++) acc += (int32_t)(int8_t)blk[2 + i] * xv[i];
        return acc;
    }
    (void)K;
    if (type == MIQO_Q6_K) {
        const int b = s / 16, sub = s % 16;
        const uint8_t *blk = row + (size_t)b * Q6K_BYTES;
        const int g = b * 8 + sub / 2, half = sub & 1;
        const int8_t *xv = x8 + ((size_t)g * TB + t) * 32 + half * 16;
        for (int i = 0; i < 16; i++) acc += code_q6k(blk, sub * 16 + i) * xv[i];
        return acc;
    }
    const size_t bb = miqo_row_bytes(type, 256);
    const int b = s / 8, g = s % 8;
    const uint8_t *blk = row + (size_t)b * bb;
    const int8_t *xv = x8 + ((size_t)s * TB + t) * 32;
    for (int i = 0; i < 32; i++) {
        const int q = (type == MIQO_Q4_K) ? code_q4k(blk, g * 32 + i) : code_q5k(blk, g * 32 + i);
        acc += q * xv[i];
    }
    return acc;
}

void miqo_group_dots(uint32_t type, const void *w, int K, int n_rows, const int8_t *x8, int TB, int32_t *out) {
    const size_t rb = miqo_row_bytes(type, K);
    const int S = (type == MIQO_Q6_K) ? K / 16 : K / 32;
    for (int t = 0; t < TB; t++)
        for (int r = 0; r < n_rows; r++)
            for (int s = 0; s < S; s++)
                out[((size_t)t * n_rows + r) * S + s] = dot_group(type, (const uint8_t *)w + (size_t)r * rb, K, x8, TB, t, s);
}

/* ------------------------------------------------- per-block epilogues */
/* Q4_K/Q5_K block partial, i8.cpp:40-61 / :96-121:
 *   acc += xmeta * (d*sc*wd - dmin*m*xsum) per group, xsum = s0 + s1 */
static float kq45_block(uint32_t type, const uint8_t *blk, const int8_t *x8, const float *xmeta,
                        const int32_t *xsumq, int TB, int t, int gbase) {
    const float d = miqo_half_to_float(rd16(blk));
    const float dm = miqo_half_to_float(rd16(blk + 2));
    float acc = 0.0f;
    for (int g = 0; g < 8; g++) {
        uint8_t sc, mm;
        miqo_get_scale_min_k4(g, blk + 4, &sc, &mm);
        const size_t ai = (size_t)(gbase + g) * TB + t;
        int32_t wd = 0;
        for (int i = 0; i < 32; i++) {
            const int q = (type == MIQO_Q4_K) ? code_q4k(blk, g * 32 + i) : code_q5k(blk, g * 32 + i);
            wd += q * x8[ai * 32 + i];
        }
        const int32_t xsum = xsumq[ai * 2] + xsumq[ai * 2 + 1];
        acc += xmeta[ai * 2] * (d * sc * (float)wd - dm * mm * (float)xsum);
    }
    return acc;
}

/* Q6_K block partial, i8.cpp:125-155: 16 sub-groups of 16,
 *   acc += xmeta * (d*scales[s]) * (wd - 32*xsum_half) */
static float q6k_block(const uint8_t *blk, const int8_t *x8, const float *xmeta, const int32_t *xsumq, int TB,
                       int t, int gbase) {
    const float d = miqo_half_to_float(rd16(blk + 208));
    float acc = 0.0f;
    for (int s = 0; s < 16; s++) {
        const int half = s & 1;
        const size_t ai = (size_t)(gbase + (s >> 1)) * TB + t;
        int32_t wd = 0;
        for (int i = 0; i < 16; i++) wd += code_q6k(blk, s * 16 + i) * x8[ai * 32 + half * 16 + i];
        const int32_t xsum = xsumq[ai * 2 + half];
        const float ds = d * (float)(int8_t)blk[192 + s];
        acc += xmeta[ai * 2] * ds * (float)(wd - 32 * xsum);
    }
    return acc;
}

/* Q8_0 group term, q4exp.cpp:457-467: a += xmeta * d * (float)sum(q*x8) */
static float q80_group(const uint8_t *blk, const int8_t *x8, const float *xmeta, int TB, int t, int g) {
    const size_t gi = (size_t)g * TB + t;
    const float d = miqo_half_to_float(rd16(blk));
    int32_t qd = 0;
    for (int i = 0; i < 32; i++) qd += (int32_t)(int8_t)blk[2 + i] * x8[gi * 32 + i];
    return xmeta[gi * 2] * d * (float)qd;
}

/* i8.cpp:157-190: block partials summed into the row */
float miqo_i8_row(uint32_t type, const void *wrow, const int8_t *x8, const float *xmeta, const int32_t *xsumq,
                  int TB, int t, int K) {
    const uint8_t *p = (const uint8_t *)wrow;
    float acc = 0.0f;
    if (type == MIQO_Q8_0) {
        for (int g = 0; g < K / 32; g++) acc += q80_group(p + (size_t)g * Q80_BYTES, x8, xmeta, TB, t, g);
        return acc;
    }
    const int nb = K / 256;
    const size_t bb = miqo_row_bytes(type, 256);
    for (int b = 0; b < nb; b++) {
        const uint8_t *blk = p + (size_t)b * bb;
        if (type == MIQO_Q6_K) acc += q6k_block(blk, x8, xmeta, xsumq, TB, t, b * 8);
        else acc += kq45_block(type, blk, x8, xmeta, xsumq, TB, t, b * 8);
    }
    return acc;
}

/* i8.cpp:498-516 */
void miqo_i8_gemv(const miqo_seg *s) {
    const size_t rb = miqo_row_bytes(s->type, s->K);
    for (int row = 0; row < s->n_rows; row++) {
        float v = s->alpha * miqo_i8_row(s->type, (const uint8_t *)s->w + (size_t)row * rb, s->x8, s->xmeta,
                                         s->xsumq, 1, 0, s->K);
        if (s->residual) v += s->residual[row];
        s->out[row] = v;
    }
}

/* The tiled form's per-(row, token) accumulation, i8.cpp:221-314 via
 * i8_gemm_tile_part (:316-349): one float accumulator per (row, token), every
 * group (Q6_K: every 16-sub-group) added in block/group order. */
static float tiled_acc(uint32_t type, const uint8_t *row, const int8_t *x8, const float *xmeta,
                       const int32_t *xsumq, int TB, int t, int K) {
    float acc = 0.0f;
    if (type == MIQO_Q8_0) { /* q8_0_down_row: the same continuous per-group form */
        for (int g = 0; g < K / 32; g++) acc += q80_group(row + (size_t)g * Q80_BYTES, x8, xmeta, TB, t, g);
        return acc;
    }
    const int nb = K / 256;
    const size_t bb = miqo_row_bytes(type, 256);
    for (int b = 0; b < nb; b++) {
        const uint8_t *blk = row + (size_t)b * bb;
        for (int g = 0; g < 8; g++) {
            const size_t ai = (size_t)(b * 8 + g) * TB + t;
            if (type == MIQO_Q6_K) {
                const float d = miqo_half_to_float(rd16(blk + 208));
                for (int half = 0; half < 2; half++) {
                    const int s = 2 * g + half;
                    int32_t wd = 0;
                    for (int i = 0; i < 16; i++) wd += code_q6k(blk, s * 16 + i) * x8[ai * 32 + half * 16 + i];
                    const float ds = d * (float)(int8_t)blk[192 + s];
                    const int32_t xsum = xsumq[ai * 2 + half];
                    acc += xmeta[ai * 2] * ds * (float)(wd - 32 * xsum);
                }
            } else {
                const float d = miqo_half_to_float(rd16(blk));
                const float dm = miqo_half_to_float(rd16(blk + 2));
                uint8_t sc, mm;
                miqo_get_scale_min_k4(g, blk + 4, &sc, &mm);
                const float dsc = d * sc, dmm = dm * mm;
                int32_t wd = 0;
                for (int i = 0; i < 32; i++) {
                    const int q = (type == MIQO_Q4_K) ? code_q4k(blk, g * 32 + i) : code_q5k(blk, g * 32 + i);
                    wd += q * x8[ai * 32 + i];
                }
                acc += xmeta[ai * 2] * (dsc * (float)wd - dmm * (float)(xsumq[ai * 2] + xsumq[ai * 2 + 1]));
            }
        }
    }
    return acc;
}

/* i8.cpp:518-546 (TB == 1 takes the i8_row form, TB >= 2 the tiled form) */
void miqo_i8_gemm(const miqo_seg *s, int TB) {
    const size_t rb = miqo_row_bytes(s->type, s->K);
    for (int t = 0; t < TB; t++) {
        for (int row = 0; row < s->n_rows; row++) {
            const uint8_t *wr = (const uint8_t *)s->w + (size_t)row * rb;
            const float a = (TB >= 2) ? tiled_acc(s->type, wr, s->x8, s->xmeta, s->xsumq, TB, t, s->K)
                                      : miqo_i8_row(s->type, wr, s->x8, s->xmeta, s->xsumq, TB, t, s->K);
            const size_t o = (size_t)t * s->out_stride + row;
            float v = s->alpha * a;
            if (s->residual) v += s->residual[o];
            s->out[o] = v;
        }
    }
}

/* ------------------------------------------------------------------ MoE */
/* moe.cpp:72-137 (the double-accumulated F32 router, fast_f32 = false) */
void miqo_moe_route(const float *x, int x_stride, const float *gate_inp, int n_tok, int n_embd, int n_expert,
                    int top_k, float *logits, int32_t *ids, float *wts) {
    if (gate_inp) {
        for (int t = 0; t < n_tok; t++)
            for (int e = 0; e < n_expert; e++) {
                double a = 0;
                for (int k = 0; k < n_embd; k++)
                    a += (double)gate_inp[(size_t)e * n_embd + k] * (double)x[(size_t)t * x_stride + k];
                logits[(size_t)t * n_expert + e] = (float)a;
            }
    }
    for (int t = 0; t < n_tok; t++) {
        float *p = logits + (size_t)t * n_expert;
        float mx = -3.402823466e38f;
        for (int e = 0; e < n_expert; e++) mx = fmaxf(mx, p[e]);
        float sum = 0.f;
        for (int e = 0; e < n_expert; e++) {
            p[e] = expf(p[e] - mx);
            sum += p[e];
        }
        const float inv = 1.f / sum;
        for (int e = 0; e < n_expert; e++) p[e] *= inv;
        int32_t *ir = ids + (size_t)t * top_k;
        float *wr = wts + (size_t)t * top_k;
        float wsum = 0.f;
        for (int e = 0; e < n_expert; e++) {
            const float pe = p[e];
            int rank = 0;
            for (int f = 0; f < n_expert; f++) {
                const float pf = p[f];
                if (pf > pe || (pf == pe && f < e)) rank++;
            }
            if (rank < top_k) {
                ir[rank] = e;
                wr[rank] = pe;
                wsum += pe;
            }
        }
        const float den = fmaxf(wsum, 6.103515625e-5f);
        for (int j = 0; j < top_k; j++) wr[j] /= den;
    }
}

void miqo_moe_experts(const miqo_moe *M, const float *x, int x_stride, int n_tok, int top_k, const int32_t *ids,
                      float *acc, int acc_stride, float *h_out) {
    const int K = M->n_embd, F = M->n_ff;
    const int G = K / 32, Gd = F / 32;
    int8_t *x8 = (int8_t *)malloc((size_t)K);
    float *xm = (float *)malloc(sizeof(float) * 2 * G);
    int32_t *xs = (int32_t *)malloc(sizeof(int32_t) * 2 * G);
    float *g = (float *)malloc(sizeof(float) * F), *u = (float *)malloc(sizeof(float) * F);
    float *h = (float *)malloc(sizeof(float) * F);
    int8_t *h8 = (int8_t *)malloc((size_t)F);
    float *hm = (float *)malloc(sizeof(float) * 2 * Gd);
    int32_t *hs = (int32_t *)malloc(sizeof(int32_t) * 2 * Gd);
    const size_t grb = miqo_row_bytes(M->gate_type, K), urb = miqo_row_bytes(M->up_type, K);
    const size_t drb = miqo_row_bytes(M->down_type, F);
    for (int p = 0; p < n_tok * top_k; p++) {
        const int t = p / top_k, e = ids[p];
        float *out = acc + (size_t)p * acc_stride;
        if (e < 0 || e >= M->n_expert) { /* moe.cpp:359-364: out-of-range pairs contribute zeros */
            for (int r = 0; r < K; r++) out[r] = 0.f;
            if (h_out) for (int i = 0; i < F; i++) h_out[(size_t)p * F + i] = 0.f;
            continue;
        }
        miqo_xq(x + (size_t)t * x_stride, NULL, K, 0, x8, xm, xs, 1, K); /* quant_row_1 == cpu_xq, TB=1 */
        const uint8_t *gb = (const uint8_t *)M->gate + (size_t)e * M->gate_plane;
        const uint8_t *ub = (const uint8_t *)M->up + (size_t)e * M->up_plane;
        const uint8_t *db = (const uint8_t *)M->down + (size_t)e * M->down_plane;
        for (int i = 0; i < F; i++) {
            g[i] = miqo_i8_row(M->gate_type, gb + (size_t)i * grb, x8, xm, xs, 1, 0, K);
            u[i] = miqo_i8_row(M->up_type, ub + (size_t)i * urb, x8, xm, xs, 1, 0, K);
            h[i] = miqo_silu(g[i]) * u[i];
        }
        if (h_out) memcpy(h_out + (size_t)p * F, h, sizeof(float) * F);
        miqo_xq(h, NULL, F, 0, h8, hm, hs, 1, F);
        for (int r = 0; r < K; r++) out[r] = miqo_i8_row(M->down_type, db + (size_t)r * drb, h8, hm, hs, 1, 0, F);
    }
    free(x8); free(xm); free(xs); free(g); free(u); free(h); free(h8); free(hm); free(hs);
}

/* moe.cpp:562-574 */
void miqo_moe_reduce(const float *acc, const float *wts, int top_k, int n_tok, int n_embd, int acc_stride,
                     float *out, int out_stride) {
    for (int t = 0; t < n_tok; t++)
        for (int e = 0; e < n_embd; e++) {
            double a = 0;
            for (int j = 0; j < top_k; j++) {
                const size_t pr = (size_t)t * top_k + j;
                a += (double)wts[pr] * acc[pr * (size_t)acc_stride + e];
            }
            out[(size_t)t * out_stride + e] += (float)a;
        }
}

/* ------------------------------------------------------- u4 native store */

/* IEEE binary16 round-to-nearest-even of a float (what sycl::half(float)
 * does); NaN stays NaN, |f| >= 65520 becomes inf. */
uint16_t miqo_float_to_half_rne(float f) {
    uint32_t b;
    memcpy(&b, &f, 4);
    const uint16_t sign = (uint16_t)((b >> 16) & 0x8000u);
    const uint32_t a = b & 0x7FFFFFFFu;
    if (a > 0x7F800000u) return (uint16_t)(sign | 0x7E00u | ((a >> 13) & 0x3FFu));
    if (a >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);
    uint32_t h, rem, half;
    if (a >= 0x38800000u) {           /* normal half: rebias the exponent by 112 */
        const uint32_t r = a - 0x38000000u;
        h = r >> 13;
        rem = r & 0x1FFFu;
        half = 0x1000u;
    } else {
        if (a < 0x33000000u) return sign; /* below 2^-25: rounds to zero */
        const uint32_t e = a >> 23, m = (a & 0x7FFFFFu) | 0x800000u;
        const uint32_t shift = 126u - e; /* value = m*2^(e-150) = h*2^-24 */
        h = m >> shift;
        rem = m & ((1u << shift) - 1u);
        half = 1u << (shift - 1u);
    }
    if (rem > half || (rem == half && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

/* src/common/w4.cpp:160-212 (pack_q4_K) */
int miqo_w4_pack_q4k(const void *src, int K, int N, uint8_t *vals, uint16_t *scale, uint16_t *off) {
    if (K % 256 != 0) return -1;
    const size_t rb = miqo_row_bytes(MIQO_Q4_K, K);
    memset(vals, 0, (size_t)N * K / 2);
    for (int n = 0; n < N; n++) {
        for (int b = 0; b < K / 256; b++) {
            const uint8_t *blk = (const uint8_t *)src + (size_t)n * rb + (size_t)b * Q4K_BYTES;
            const float d = miqo_half_to_float(rd16(blk)), mn = miqo_half_to_float(rd16(blk + 2));
            for (int j = 0; j < 8; j++) {
                uint8_t sc, m;
                miqo_get_scale_min_k4(j, blk + 4, &sc, &m);
                const size_t g = (size_t)b * 8 + j;
                scale[g * N + n] = miqo_float_to_half(d * (float)sc);
                off[g * N + n] = miqo_float_to_half(-mn * (float)m);
                for (int l = 0; l < 32; l++) {
                    const size_t idx = (size_t)n * K + g * 32 + l;
                    vals[idx >> 1] |= (uint8_t)(code_q4k(blk, j * 32 + l) << ((idx & 1) * 4));
                }
            }
        }
    }
    return 0;
}

/* src/backend/dnnl_gemm.cpp:100-146 (act_quant_grp_launch with do_split) */
void miqo_w4_act(const float *x, const float *up, int M, int K, int8_t *xq, uint16_t *asa, float *xs, int8_t *axe,
                 int8_t *axo) {
    const int ng = K / 32;
    for (int m = 0; m < M; m++)
        for (int g = 0; g < ng; g++) {
            float v[32], mx = 0.0f;
            for (int i = 0; i < 32; i++) {
                const size_t k = (size_t)m * K + (size_t)g * 32 + i;
                v[i] = up ? miqo_silu(x[k]) * up[k] : x[k];
                mx = fmaxf(mx, fabsf(v[i]));
            }
            const float sc = mx > 0.0f ? mx / 127.0f : 1.0f;
            const float inv = 1.0f / sc;
            int s = 0;
            for (int i = 0; i < 32; i++) {
                int q = (int)roundf(v[i] * inv);
                q = q < -127 ? -127 : (q > 127 ? 127 : q);
                const size_t k = (size_t)m * K + (size_t)g * 32 + i;
                xq[k] = (int8_t)q;
                if (i & 1) axo[k >> 1] = (int8_t)q;
                else axe[k >> 1] = (int8_t)q;
                s += q;
            }
            asa[(size_t)m * ng + g] = miqo_float_to_half_rne(sc);
            xs[(size_t)m * ng + g] = (float)s;
        }
}

/* src/backend/gpu/kernels/w4_gemv.cpp:79-154 (w4_gemv_impl) */
void miqo_w4_gemv(const uint8_t *vals, const uint16_t *scale, const uint16_t *off, const int8_t *axe,
                  const int8_t *axo, const uint16_t *asa, const float *xs, float *out, const float *residual,
                  float alpha, int K, int N) {
    const int ng = K / 32;
    for (int n = 0; n < N; n++) {
        const uint8_t *wrow = vals + (size_t)n * (K / 2);
        double acc = 0.0;
        for (int g = 0; g < ng; g++) {
            int32_t qd = 0;
            for (int j = 0; j < 16; j++) {  /* byte j: elements 2j (low), 2j+1 (high) */
                const uint8_t b = wrow[(size_t)g * 16 + j];
                qd += (int32_t)(b & 0xF) * axe[(size_t)g * 16 + j] + (int32_t)(b >> 4) * axo[(size_t)g * 16 + j];
            }
            const float sa = miqo_half_to_float(asa[g]);
            const float st = miqo_half_to_float(scale[(size_t)g * N + n]);
            const float of = miqo_half_to_float(off[(size_t)g * N + n]);
            acc += (double)(sa * (st * (float)qd + of * xs[g]));
        }
        float v = alpha * (float)acc;
        if (residual) v += residual[n];
        out[n] = v;
    }
}

/* src/common/w4.cpp:336-403 (pack_q5_K) */
int miqo_k5_pack(const void *src, int K, int N, uint8_t *vals, uint8_t *hi, uint16_t *scale, uint16_t *off) {
    if (K % 256 != 0) return -1;
    const size_t rb = miqo_row_bytes(MIQO_Q5_K, K);
    memset(vals, 0, (size_t)N * K / 2);
    memset(hi, 0, (size_t)N * K / 8);
    for (int n = 0; n < N; n++)
        for (int b = 0; b < K / 256; b++) {
            const uint8_t *blk = (const uint8_t *)src + (size_t)n * rb + (size_t)b * Q5K_BYTES;
            const float d = miqo_half_to_float(rd16(blk)), mn = miqo_half_to_float(rd16(blk + 2));
            for (int j = 0; j < 8; j++) {
                uint8_t sc, m;
                miqo_get_scale_min_k4(j, blk + 4, &sc, &m);
                const size_t g = (size_t)b * 8 + j;
                scale[g * N + n] = miqo_float_to_half(d * (float)sc);
                off[g * N + n] = miqo_float_to_half(-mn * (float)m);
                uint32_t h = 0;
                for (int l = 0; l < 32; l++) {
                    const int code = code_q5k(blk, j * 32 + l);  /* 0..31 */
                    const size_t idx = (size_t)n * K + g * 32 + l;
                    vals[idx >> 1] |= (uint8_t)((code & 0xF) << ((idx & 1) * 4));
                    h |= (uint32_t)(code >> 4) << ((l & 1) * 16 + (l >> 1));
                }
                memcpy(hi + (size_t)n * (K / 8) + g * 4, &h, 4);
            }
        }
    return 0;
}

/* src/backend/gpu/kernels/w4_gemv.cpp:1002-1080 (k5_gemv_impl) */
void miqo_k5_gemv(const uint8_t *vals, const uint8_t *hi, const uint16_t *scale, const uint16_t *off,
                  const int8_t *axe, const int8_t *axo, const uint16_t *asa, const float *xs, float *out,
                  const float *residual, float alpha, int K, int N) {
    const int ng = K / 32;
    for (int n = 0; n < N; n++) {
        const uint8_t *wrow = vals + (size_t)n * (K / 2);
        double acc = 0.0;
        for (int g = 0; g < ng; g++) {
            uint32_t h;
            memcpy(&h, hi + (size_t)n * (K / 8) + (size_t)g * 4, 4);
            int32_t qd = 0;
            for (int j = 0; j < 16; j++) {
                const uint8_t b = wrow[(size_t)g * 16 + j];
                const int qe = (b & 0xF) | (int)((h >> j) & 1) << 4, qo = (b >> 4) | (int)((h >> (16 + j)) & 1) << 4;
                qd += qe * axe[(size_t)g * 16 + j] + qo * axo[(size_t)g * 16 + j];
            }
            const float sa = miqo_half_to_float(asa[g]);
            const float st = miqo_half_to_float(scale[(size_t)g * N + n]);
            const float of = miqo_half_to_float(off[(size_t)g * N + n]);
            acc += (double)(sa * (st * (float)qd + of * xs[g]));
        }
        float v = alpha * (float)acc;
        if (residual) v += residual[n];
        out[n] = v;
    }
}
