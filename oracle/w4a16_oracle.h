/*
 * w4a16_oracle.h - CPU oracle for the W4A16 dense-FFN decode path.
 *
 * TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline
 * leg may load this library, and only as the checker. The product path (the HIP library under
 * haskell-infer-demo_amd/) never calls it and has no CPU fallback.
 *
 * This is a clean-room restatement of the reference's INT4 format arithmetic and of the FFN
 * sequence that consumes it. Each function cites the reference file:line it follows. The
 * format contract (reference csrc/include/linear_weight.h:5-13):
 *   - symmetric signed INT4, groups of 128 along K, BF16 scales s = BF16_RNE(max|g| / 7),
 *     s = 1 for an all-zero group;
 *   - code q = clip(round_half_even(w / s), -7, 7); -8 is reserved invalid;
 *   - two two's-complement nibbles per byte, lower K index in the low nibble, rows of K/2 bytes.
 *
 * Pinning (what checks each function against something other than itself) is listed in
 * tests/test_oracle.py; every function below has at least one such check.
 */
#ifndef W4A16_ORACLE_H
#define W4A16_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    ORC_OK = 0,
    ORC_ERR_ARG = 1,
    ORC_ERR_RANGE = 2,
    ORC_ERR_VALUE = 3,
    ORC_ERR_FORMAT = 4,
};

const char *orc_last_error(void);

/* BF16 round-to-nearest-even and widening (reference csrc/linear_weight.cpp:34-51). */
uint16_t orc_f32_to_bf16(float value);
float orc_bf16_to_f32(uint16_t bits);

/* Shape rule (reference csrc/linear_weight.cpp:57-86): n,k > 0, group == 128, k % 128 == 0,
 * n % 8 == 0. Returns ORC_OK or ORC_ERR_RANGE / ORC_ERR_ARG. */
int orc_layout_check(long long n, long long k, long long group);

/* One code of a row-major packed [n, k/2] payload (reference csrc/linear_weight.cpp:96-102). */
int orc_packed_code(const uint8_t *packed, long long row, long long k, long long k_extent);

/* Quantize FP32 [n, k] -> packed [n*k/2] + BF16 scales [n * k/128] (reference
 * csrc/linear_weight.cpp:108-176). Buffers are untouched on failure. */
int orc_quantize_int4(long long n, long long k, const float *weights, uint8_t *packed,
                      uint16_t *scales);

/* Dequantize to FP32 [n, k]: w = code * f32(scale); refuses nibble 0x8 and a scale that is not
 * positive and finite (reference csrc/linear_weight.cpp:178-216). */
int orc_dequantize_int4(long long n, long long k, const uint8_t *packed, const uint16_t *scales,
                        float *out);

/* out[m, n] = sum_k x[m, k] * (code[n, k] * scale[n, k/128]), accumulated in double, written as
 * double (no rounding). x is BF16 bits [m, k]. This is the dequant-then-matmul the reference's
 * kernel gate compares against (reference tests/test_quantization_kernel.py:60-70,111-115). */
int orc_gemm_f64(long long m, long long n, long long k, const uint16_t *x_bf16,
                 const uint8_t *packed, const uint16_t *scales, double *out);

/* Same, rounded to BF16 through FP32 the way a kernel writes its output
 * (reference csrc/kernels/gemm_quant.cu:199). */
int orc_gemm_bf16(long long m, long long n, long long k, const uint16_t *x_bf16,
                  const uint8_t *packed, const uint16_t *scales, uint16_t *out_bf16);

/* act[t, i] = BF16(silu(g) * u) with g = packed[t, i], u = packed[t, I + i] (the row-interleaved
 * gate-then-up layout, reference csrc/kernels/silu.cu:61-74). Evaluated in double and rounded
 * to FP32, then to BF16. */
int orc_silu_mul_packed(long long tokens, long long inter, const uint16_t *packed_bf16,
                        uint16_t *act_bf16);

/* The INT4 FFN decode sequence of reference csrc/kernels/layers.cu:126-145, with its rounding
 * points: gate/up GEMM -> BF16 [m, 2I]; SiLU x up -> BF16 [m, I]; down GEMM -> BF16 [m, H].
 * gate_up is the F1 pair [2I, H] (gate rows then up rows) and down is [H, I], both in the
 * reference's row-major packed layout. `mid_out` (optional, [m, 2I]) receives the gate/up
 * output and `act_out` (optional, [m, I]) the activation, for stage-by-stage checks. */
int orc_ffn_bf16(long long m, long long hidden, long long inter, const uint16_t *x_bf16,
                 const uint8_t *gu_packed, const uint16_t *gu_scales, const uint8_t *dn_packed,
                 const uint16_t *dn_scales, uint16_t *out_bf16, uint16_t *mid_out,
                 uint16_t *act_out);

/* Same FFN, but the down projection's FP32-accumulated partial is returned unrounded (as FP32)
 * for the tensor-parallel slice, whose output is a partial to be summed across ranks. */
int orc_ffn_partial_f32(long long m, long long hidden, long long inter, const uint16_t *x_bf16,
                        const uint8_t *gu_packed, const uint16_t *gu_scales,
                        const uint8_t *dn_packed, const uint16_t *dn_scales, float *out_f32);

/* RMSNorm ahead of the FFN (reference csrc/kernels/layers.cu:16-25,150-159, which calls
 * kernel_rms_norm_plain / kernel_gemma_rms_norm, csrc/kernels/flashinfer_norm.cu:22-76, i.e.
 * FlashInfer 0.5.3 norm::RMSNorm / GemmaRMSNorm, a third-party header absent from the
 * reference tree). Its published algorithm:
 *   out[r, c] = BF16( x[r, c] * rsqrt(sum_c x[r, c]^2 / cols + eps) * (bias + w[c]) )
 * with bias = 1 for norm_style 0 (Gemma: weight + 1) and 0 for norm_style 1 (plain), all in
 * FP32 there. Here the sum of squares and the root are taken in double and rounded once to
 * FP32 (any FP32 summation order is within an FP32 ULP of it); the two products are FP32 in
 * FlashInfer's order ((x * rms) * (bias + w)), then BF16 RNE. Refuses rows < 0, cols <= 0 and an
 * epsilon that is not finite and positive (flashinfer_norm.cu:25-27). */
int orc_rmsnorm_bf16(long long rows, long long cols, const uint16_t *x_bf16,
                     const uint16_t *w_bf16, int norm_style, double eps, uint16_t *out_bf16);

/* Plan F2's fused residual update and norm (reference csrc/kernels/flashinfer_norm.cu:111-155,
 * in-tree): residual[r, c] <- BF16(residual + sublayer) (stored back), then out = the RMSNorm of
 * the rounded residual, as orc_rmsnorm_bf16 (the reference kernel's FP32 order is the same:
 * value * scale * weight, weight + 1 for Gemma). */
int orc_residual_norm_bf16(long long rows, long long cols, uint16_t *residual,
                           const uint16_t *sublayer, const uint16_t *w_bf16, int norm_style,
                           double eps, uint16_t *out_bf16);

/* The RMSNorm in the reference's in-tree FP32 order (residual_norm_kernel, reference
 * csrc/kernels/flashinfer_norm.cu:136-160): FP32 fmaf partial sums over 256 strided threads, the
 * warp shuffle trees, then 1/sqrt in FP32 (correctly rounded, standing in for rsqrtf), then
 * (v * scale) * (bias + w). rms_out (may be NULL) receives each row's FP32 scale. */
int orc_rmsnorm_f32order_bf16(long long rows, long long cols, const uint16_t *x_bf16,
                              const uint16_t *w_bf16, int norm_style, float eps,
                              uint16_t *out_bf16, float *rms_out);

/* dst[i] <- BF16(f32(dst[i]) + f32(src[i])) (reference csrc/kernels/gdn_norm.cu:121-129). */
int orc_residual_add_bf16(long long n, uint16_t *dst, const uint16_t *src);

#ifdef __cplusplus
}
#endif

#endif /* W4A16_ORACLE_H */
