/*
 * w4a16_oracle.c - CPU oracle for the W4A16 dense-FFN decode path (TEST INFRASTRUCTURE ONLY).
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg load this library, as the
 * checker. The product (the HIP library) never calls it. The contract each function restates is
 * in w4a16_oracle.h; the citations below name the reference lines each one follows.
 */
#include "w4a16_oracle.h"

#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define ORC_GROUP 128
#define ORC_TILE_ROWS 8
#define ORC_QMAX 7
#define ORC_QMIN (-7)

static _Thread_local char g_err[256];

const char *orc_last_error(void) { return g_err; }

static int fail(int status, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return status;
}

/* Round-to-nearest-even by adding 0x7FFF plus the kept LSB to the FP32 bit pattern and keeping
 * the top half (reference csrc/linear_weight.cpp:34-44). A carry out of the mantissa bumps the
 * exponent, so values past the BF16 range become infinity. */
uint16_t orc_f32_to_bf16(float value) {
    uint32_t u;
    memcpy(&u, &value, 4);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

float orc_bf16_to_f32(uint16_t bits) {
    uint32_t u = (uint32_t)bits << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* reference csrc/linear_weight.cpp:57-86 */
int orc_layout_check(long long n, long long k, long long group) {
    if (n <= 0 || k <= 0) return fail(ORC_ERR_RANGE, "empty or negative shape %lld x %lld", n, k);
    if (group != ORC_GROUP) return fail(ORC_ERR_RANGE, "group must be %d, got %lld", ORC_GROUP, group);
    if (k % group) return fail(ORC_ERR_RANGE, "K=%lld is not a multiple of the group", k);
    if (n % ORC_TILE_ROWS) return fail(ORC_ERR_RANGE, "N=%lld is not a multiple of %d", n, ORC_TILE_ROWS);
    return ORC_OK;
}

static inline int nibble_at(const uint8_t *packed, long long flat) {
    const uint8_t b = packed[flat >> 1];
    return (flat & 1) ? (b >> 4) : (b & 0x0F);
}

static inline int sext4(int nib) { return nib >= 8 ? nib - 16 : nib; }

/* reference csrc/linear_weight.cpp:96-102 */
int orc_packed_code(const uint8_t *packed, long long row, long long k, long long k_extent) {
    return sext4(nibble_at(packed, row * k_extent + k));
}

/* reference csrc/linear_weight.cpp:108-176 */
int orc_quantize_int4(long long n, long long k, const float *w, uint8_t *packed,
                      uint16_t *scales) {
    if (!w || !packed || !scales) return fail(ORC_ERR_ARG, "null argument");
    int st = orc_layout_check(n, k, ORC_GROUP);
    if (st) return st;
    const long long gpr = k / ORC_GROUP;
    for (long long i = 0; i < n * k; ++i)
        if (!isfinite(w[i])) return fail(ORC_ERR_VALUE, "element %lld is not finite", i);
    /* Scales first, into a private buffer, so a refused group leaves the outputs untouched. */
    uint16_t *s_tmp = (uint16_t *)malloc((size_t)(n * gpr) * sizeof(uint16_t));
    if (!s_tmp) return fail(ORC_ERR_ARG, "out of memory");
    for (long long r = 0; r < n; ++r) {
        for (long long g = 0; g < gpr; ++g) {
            const float *src = w + r * k + g * ORC_GROUP;
            float amax = 0.0f;
            for (int i = 0; i < ORC_GROUP; ++i) {
                float a = fabsf(src[i]);
                if (a > amax) amax = a;
            }
            uint16_t sb = orc_f32_to_bf16(amax == 0.0f ? 1.0f : amax / 7.0f);
            float s = orc_bf16_to_f32(sb);
            if (!(s > 0.0f) || !isfinite(s)) {
                free(s_tmp);
                return fail(ORC_ERR_VALUE, "row %lld group %lld: scale %g not positive/finite",
                            r, g, (double)s);
            }
            s_tmp[r * gpr + g] = sb;
        }
    }
    for (long long r = 0; r < n; ++r) {
        for (long long kk = 0; kk < k; kk += 2) {
            int nib[2];
            for (int h = 0; h < 2; ++h) {
                const float s = orc_bf16_to_f32(s_tmp[r * gpr + (kk + h) / ORC_GROUP]);
                /* nearbyintf under the default rounding mode rounds half to even. */
                float q = nearbyintf(w[r * k + kk + h] / s);
                if (q > ORC_QMAX) q = ORC_QMAX;
                if (q < ORC_QMIN) q = ORC_QMIN;
                nib[h] = ((int)q) & 0x0F;
            }
            packed[(r * k + kk) >> 1] = (uint8_t)(nib[0] | (nib[1] << 4));
        }
    }
    memcpy(scales, s_tmp, (size_t)(n * gpr) * sizeof(uint16_t));
    free(s_tmp);
    return ORC_OK;
}

/* reference csrc/linear_weight.cpp:178-216 */
int orc_dequantize_int4(long long n, long long k, const uint8_t *packed, const uint16_t *scales,
                        float *out) {
    if (!packed || !scales || !out) return fail(ORC_ERR_ARG, "null argument");
    int st = orc_layout_check(n, k, ORC_GROUP);
    if (st) return st;
    const long long gpr = k / ORC_GROUP;
    for (long long r = 0; r < n; ++r) {
        for (long long g = 0; g < gpr; ++g) {
            const float s = orc_bf16_to_f32(scales[r * gpr + g]);
            if (!(s > 0.0f) || !isfinite(s))
                return fail(ORC_ERR_FORMAT, "row %lld group %lld: bad scale", r, g);
            for (int i = 0; i < ORC_GROUP; ++i) {
                const long long kk = g * ORC_GROUP + i;
                const int nib = nibble_at(packed, r * k + kk);
                if (nib == 0x8)
                    return fail(ORC_ERR_FORMAT, "code -8 at row %lld column %lld", r, kk);
                out[r * k + kk] = (float)sext4(nib) * s;
            }
        }
    }
    return ORC_OK;
}

/* Dequant-then-matmul in double (reference tests/test_quantization_kernel.py:60-70,111-115).
 * The kernel path sign-extends -8 without checking (reference csrc/kernels/gemm_quant.cu:45-48),
 * and so does this product; format refusals are orc_dequantize_int4's job. */
int orc_gemm_f64(long long m, long long n, long long k, const uint16_t *x, const uint8_t *packed,
                 const uint16_t *scales, double *out) {
    if (!x || !packed || !scales || !out) return fail(ORC_ERR_ARG, "null argument");
    if (m < 0 || n <= 0 || k <= 0 || k % ORC_GROUP) return fail(ORC_ERR_RANGE, "bad extents");
    const long long gpr = k / ORC_GROUP;
    double *xd = (double *)malloc((size_t)(m * k) * sizeof(double));
    if (!xd) return fail(ORC_ERR_ARG, "out of memory");
    for (long long i = 0; i < m * k; ++i) xd[i] = (double)orc_bf16_to_f32(x[i]);
#pragma omp parallel for schedule(static)
    for (long long r = 0; r < n; ++r) {
        double acc[64];
        for (long long m0 = 0; m0 < m; m0 += 64) {
            const long long mb = (m - m0) < 64 ? (m - m0) : 64;
            for (long long t = 0; t < mb; ++t) acc[t] = 0.0;
            for (long long kk = 0; kk < k; ++kk) {
                const double w = (double)sext4(nibble_at(packed, r * k + kk)) *
                                 (double)orc_bf16_to_f32(scales[r * gpr + kk / ORC_GROUP]);
                for (long long t = 0; t < mb; ++t) acc[t] += w * xd[(m0 + t) * k + kk];
            }
            for (long long t = 0; t < mb; ++t) out[(m0 + t) * n + r] = acc[t];
        }
    }
    free(xd);
    return ORC_OK;
}

static uint16_t d_to_bf16(double v) { return orc_f32_to_bf16((float)v); }

int orc_gemm_bf16(long long m, long long n, long long k, const uint16_t *x, const uint8_t *packed,
                  const uint16_t *scales, uint16_t *out) {
    double *tmp = (double *)malloc((size_t)(m * n > 0 ? m * n : 1) * sizeof(double));
    if (!tmp) return fail(ORC_ERR_ARG, "out of memory");
    int st = orc_gemm_f64(m, n, k, x, packed, scales, tmp);
    if (!st)
        for (long long i = 0; i < m * n; ++i) out[i] = d_to_bf16(tmp[i]);
    free(tmp);
    return st;
}

/* reference csrc/kernels/silu.cu:61-74: out = bf16((g / (1 + exp(-g))) * u). */
int orc_silu_mul_packed(long long tokens, long long inter, const uint16_t *packed, uint16_t *act) {
    if (!packed || !act) return fail(ORC_ERR_ARG, "null argument");
    if (tokens < 0 || inter < 0) return fail(ORC_ERR_RANGE, "negative extent");
    for (long long t = 0; t < tokens; ++t) {
        for (long long i = 0; i < inter; ++i) {
            const double g = orc_bf16_to_f32(packed[t * 2 * inter + i]);
            const double u = orc_bf16_to_f32(packed[t * 2 * inter + inter + i]);
            act[t * inter + i] = d_to_bf16((g / (1.0 + exp(-g))) * u);
        }
    }
    return ORC_OK;
}

/* reference csrc/kernels/layers.cu:126-145 (gate/up GEMM, packed SiLU x mul, down GEMM). */
static int ffn_core(long long m, long long h, long long inter, const uint16_t *x,
                    const uint8_t *gup, const uint16_t *gus, const uint8_t *dnp,
                    const uint16_t *dns, uint16_t *mid, uint16_t *act, double *out_d) {
    int st = orc_gemm_bf16(m, 2 * inter, h, x, gup, gus, mid);
    if (st) return st;
    st = orc_silu_mul_packed(m, inter, mid, act);
    if (st) return st;
    return orc_gemm_f64(m, h, inter, act, dnp, dns, out_d);
}

int orc_ffn_bf16(long long m, long long h, long long inter, const uint16_t *x,
                 const uint8_t *gup, const uint16_t *gus, const uint8_t *dnp,
                 const uint16_t *dns, uint16_t *out, uint16_t *mid_out, uint16_t *act_out) {
    if (!x || !gup || !gus || !dnp || !dns || !out) return fail(ORC_ERR_ARG, "null argument");
    if (m <= 0 || h <= 0 || inter <= 0) return fail(ORC_ERR_RANGE, "bad extents");
    uint16_t *mid = (uint16_t *)malloc((size_t)(m * 2 * inter) * 2);
    uint16_t *act = (uint16_t *)malloc((size_t)(m * inter) * 2);
    double *od = (double *)malloc((size_t)(m * h) * sizeof(double));
    int st = (!mid || !act || !od) ? fail(ORC_ERR_ARG, "out of memory")
                                   : ffn_core(m, h, inter, x, gup, gus, dnp, dns, mid, act, od);
    if (!st) {
        for (long long i = 0; i < m * h; ++i) out[i] = d_to_bf16(od[i]);
        if (mid_out) memcpy(mid_out, mid, (size_t)(m * 2 * inter) * 2);
        if (act_out) memcpy(act_out, act, (size_t)(m * inter) * 2);
    }
    free(mid);
    free(act);
    free(od);
    return st;
}

int orc_ffn_partial_f32(long long m, long long h, long long inter, const uint16_t *x,
                        const uint8_t *gup, const uint16_t *gus, const uint8_t *dnp,
                        const uint16_t *dns, float *out) {
    if (!x || !gup || !gus || !dnp || !dns || !out) return fail(ORC_ERR_ARG, "null argument");
    if (m <= 0 || h <= 0 || inter <= 0) return fail(ORC_ERR_RANGE, "bad extents");
    uint16_t *mid = (uint16_t *)malloc((size_t)(m * 2 * inter) * 2);
    uint16_t *act = (uint16_t *)malloc((size_t)(m * inter) * 2);
    double *od = (double *)malloc((size_t)(m * h) * sizeof(double));
    int st = (!mid || !act || !od) ? fail(ORC_ERR_ARG, "out of memory")
                                   : ffn_core(m, h, inter, x, gup, gus, dnp, dns, mid, act, od);
    if (!st)
        for (long long i = 0; i < m * h; ++i) out[i] = (float)od[i];
    free(mid);
    free(act);
    free(od);
    return st;
}

/* reference csrc/kernels/flashinfer_norm.cu:22-76 (FlashInfer RMSNorm / GemmaRMSNorm). */
int orc_rmsnorm_bf16(long long rows, long long cols, const uint16_t *x, const uint16_t *w,
                     int norm_style, double eps, uint16_t *out) {
    if (rows < 0 || cols <= 0 || !isfinite(eps) || eps <= 0.0)
        return fail(ORC_ERR_RANGE, "invalid shape or epsilon");
    if (rows == 0) return ORC_OK;
    if (!x || !w || !out) return fail(ORC_ERR_ARG, "null argument");
    if (norm_style != 0 && norm_style != 1) return fail(ORC_ERR_ARG, "norm_style must be 0 or 1");
    const double bias = norm_style == 0 ? 1.0 : 0.0;
    for (long long r = 0; r < rows; ++r) {
        const uint16_t *xr = x + r * cols;
        double ss = 0.0;
        for (long long c = 0; c < cols; ++c) {
            const double v = orc_bf16_to_f32(xr[c]);
            ss += v * v;
        }
        /* the scale in double, rounded once to FP32; then FlashInfer's FP32 products in its
         * order, x * rms first, then times (bias + w) */
        const float rms = (float)(1.0 / sqrt(ss / (double)cols + eps));
        for (long long c = 0; c < cols; ++c) {
            const float xs = orc_bf16_to_f32(xr[c]) * rms;
            const float wb = (float)bias + orc_bf16_to_f32(w[c]);
            out[r * cols + c] = orc_f32_to_bf16(xs * wb);
        }
    }
    return ORC_OK;
}

/* reference csrc/kernels/gdn_norm.cu:121-129. */
int orc_residual_add_bf16(long long n, uint16_t *dst, const uint16_t *src) {
    if (n < 0) return fail(ORC_ERR_RANGE, "negative extent");
    if (n > 0 && (!dst || !src)) return fail(ORC_ERR_ARG, "null argument");
    for (long long i = 0; i < n; ++i)
        dst[i] = orc_f32_to_bf16(orc_bf16_to_f32(dst[i]) + orc_bf16_to_f32(src[i]));
    return ORC_OK;
}

/* reference csrc/kernels/flashinfer_norm.cu:111-175 (residual_norm_kernel and its wrapper). */
int orc_residual_norm_bf16(long long rows, long long cols, uint16_t *residual,
                           const uint16_t *sub, const uint16_t *w, int norm_style, double eps,
                           uint16_t *out) {
    if (rows < 0 || cols <= 0 || !isfinite(eps) || eps <= 0.0)
        return fail(ORC_ERR_RANGE, "invalid shape or epsilon");
    if (rows == 0) return ORC_OK;
    if (!residual || !sub || !w || !out) return fail(ORC_ERR_ARG, "null argument");
    int st = orc_residual_add_bf16(rows * cols, residual, sub);
    if (st) return st;
    return orc_rmsnorm_bf16(rows, cols, residual, w, norm_style, eps, out);
}

/* The reference's in-tree FP32 order (csrc/kernels/flashinfer_norm.cu:136-160, residual_norm_kernel
 * launched with 256 threads a row, :169-171): thread t accumulates fmaf(v, v, .) over columns
 * t, t + 256, ...; each 32-lane warp reduces with __shfl_down offsets 16, 8, 4, 2, 1 (lane 0's
 * value is the pairwise tree (l, l + 16), (l, l + 8), ...); warp 0 then reduces the 8 warp totals
 * (zeros in lanes 8..31) the same way; scale = rsqrt(total / cols + eps) in FP32, taken here as the
 * correctly rounded 1 / sqrtf (the reference's rsqrtf is a hardware approximation whose bits are
 * not specified); out = BF16((v * scale) * (bias + w)) in FP32. rms_out (optional) gets the
 * per-row scale. */
int orc_rmsnorm_f32order_bf16(long long rows, long long cols, const uint16_t *x, const uint16_t *w,
                              int norm_style, float eps, uint16_t *out, float *rms_out) {
    if (rows < 0 || cols <= 0 || !isfinite(eps) || eps <= 0.0f)
        return fail(ORC_ERR_RANGE, "invalid shape or epsilon");
    if (rows == 0) return ORC_OK;
    if (!x || !w || !out) return fail(ORC_ERR_ARG, "null argument");
    if (norm_style != 0 && norm_style != 1) return fail(ORC_ERR_ARG, "norm_style must be 0 or 1");
    enum { kThreads = 256, kWarp = 32 };
    for (long long r = 0; r < rows; ++r) {
        const uint16_t *xr = x + r * cols;
        float lane[kThreads];
        for (int t = 0; t < kThreads; ++t) {
            float s = 0.0f;
            for (long long c = t; c < cols; c += kThreads) {
                const float v = orc_bf16_to_f32(xr[c]);
                s = fmaf(v, v, s);
            }
            lane[t] = s;
        }
        float totals[kWarp];
        for (int wi = 0; wi < kWarp; ++wi) totals[wi] = 0.0f;
        for (int wi = 0; wi < kThreads / kWarp; ++wi) {
            float *l = lane + wi * kWarp;
            for (int off = kWarp / 2; off > 0; off >>= 1)
                for (int i = 0; i < off; ++i) l[i] = l[i] + l[i + off];
            totals[wi] = l[0];
        }
        for (int off = kWarp / 2; off > 0; off >>= 1)
            for (int i = 0; i < off; ++i) totals[i] = totals[i] + totals[i + off];
        const float scale = 1.0f / sqrtf(totals[0] / (float)cols + eps);
        if (rms_out) rms_out[r] = scale;
        for (long long c = 0; c < cols; ++c) {
            float wt = orc_bf16_to_f32(w[c]);
            if (norm_style == 0) wt += 1.0f;
            out[r * cols + c] = orc_f32_to_bf16(orc_bf16_to_f32(xr[c]) * scale * wt);
        }
    }
    return ORC_OK;
}
