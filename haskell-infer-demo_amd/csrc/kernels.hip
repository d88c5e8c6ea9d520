/*
 * kernels.hip - gfx950 kernels of the W4A16 dense-FFN decode path and their C-ABI launchers.
 *
 * Weights are read in the tile order described in common.h. The M = 1 kernels are wave64
 * GEMVs: each lane loads one 16-byte piece (32 codes of one row) per step with a single
 * global_load_dwordx4, turns each pair of codes into a BF16 pair with one shift and one
 * and-or (value 1 + u/16, u = nibble ^ 8 = code + 8, exact in BF16), and accumulates with the
 * packed BF16 dot product v_dot2_f32_bf16 against the activation pair. Since
 * code = 16 * v - 24, a piece's contribution is 16 * dot(v, x) - 24 * sum(x), and the per-piece
 * activation sums are computed once per block when the activation is staged in LDS. The
 * group's BF16 scale multiplies each piece's FP32 partial (the association of the reference's
 * tiled kernel, csrc/kernels/gemm_quant.cu:130-142). Lanes of one row are reduced with
 * cross-lane shuffles; the waves of a block (split-K over groups) through LDS.
 */
#include <hip/hip_runtime.h>

#include <cstdio>

#include "common.h"

using namespace w4a16;

namespace {

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

constexpr int kWaves = 4;                 /* waves per GEMV block */
constexpr int kThreads = kWaves * 64;
constexpr int kBatch = 4;                 /* 16-byte pieces in flight per lane */
constexpr int kMaxGemvK = 30720;          /* activation staged in LDS: 2K bytes + sums */

__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                           __builtin_bit_cast(bf16x2_t, b), c, false);
}

/* BF16 pair (1 + u_lo/16, 1 + u_hi/16) for code pair q of a tile word already XORed with
 * 0x88888888 (so each nibble is u = code + 8). */
template <int Q>
__device__ __forceinline__ uint32_t code_pair(uint32_t w) {
    const uint32_t shifted = (Q == 0) ? (w << 3) : (w >> (4 * Q - 3));
    return (shifted & 0x00780078u) | 0x3F803F80u;
}

/* sum_{j<32} code_j * x_j for one 16-byte piece: 16 * dot(v, x) - 24 * xsum. */
__device__ __forceinline__ float piece_dot(uint4 piece, const uint4 *xq, float xsum) {
    float d = 0.0f;
    const uint32_t words[4] = {piece.x, piece.y, piece.z, piece.w};
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        const uint32_t w = words[s] ^ 0x88888888u;
        const uint4 xv = xq[s];
        d = dot2_bf16(code_pair<0>(w), xv.x, d);
        d = dot2_bf16(code_pair<1>(w), xv.y, d);
        d = dot2_bf16(code_pair<2>(w), xv.z, d);
        d = dot2_bf16(code_pair<3>(w), xv.w, d);
    }
    return fmaf(16.0f, d, -24.0f * xsum);
}

/* SiLU with exp computed as 2^n * 2^(r * log2 e), -g = n ln2 + r, |r| <= ln2/2 (Cody-Waite
 * split of ln2 into a 16-bit head and a tail), 2^(.) by v_exp_f32 on the reduced argument and
 * the power of two by v_ldexp_f32. */
__device__ __forceinline__ float silu_f32(float g) {
    const float t = fminf(fmaxf(-g, -200.0f), 200.0f);
    const float n = rintf(t * 1.44269504088896341f);
    float r = fmaf(-n, 0.693145751953125f, t);
    r = fmaf(-n, 1.42860682030941723e-06f, r);
    const float e = ldexpf(__builtin_amdgcn_exp2f(r * 1.44269504088896341f), (int)n);
    return g / (1.0f + e);
}

__device__ __forceinline__ uint16_t silu_mul_bf16(float gate, float up) {
    return bf16_rne(silu_f32(gate) * up);
}

/* One block per 8-row tile; wave w takes the group pairs w, w + kWaves, ...; half-wave h of a
 * step takes group 2*pair + h. PAIR: the tile is 4 gate + 4 up rows and the block writes four
 * BF16(silu(BF16 gate) * BF16 up) values; otherwise eight BF16 outputs (or FP32 if OUT_F32). */
template <bool PAIR, bool OUT_F32>
__global__ __launch_bounds__(kThreads) void gemv_tiles_kernel(
    const uint16_t *__restrict__ x, const uint4 *__restrict__ wt,
    const uint16_t *__restrict__ st, void *__restrict__ out, int K) {
    extern __shared__ uint4 smem4[];
    const int G = K >> 7;
    const int tile = blockIdx.x;
    uint32_t *xs = reinterpret_cast<uint32_t *>(smem4);
    float *xsum = reinterpret_cast<float *>(xs + (K >> 1));
    float *red = xsum + 4 * G;

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int half = lane >> 5;
    const int piece = lane & 31;
    const int kb = piece >> 3;
    const int r = piece & 7;

    /* Issue the first batch of weight loads before staging the activation, so the HBM
     * latency overlaps the staging. */
    const uint4 *wtile = wt + (size_t)tile * G * 32;
    const uint16_t *stile = st + (size_t)tile * G * 8;
    const int pairs = (G + 1) >> 1;
    uint4 buf[kBatch];
    float sc[kBatch];
    int p0 = wave;
#pragma unroll
    for (int b = 0; b < kBatch; ++b) {
        const int g = 2 * (p0 + b * kWaves) + half;
        const bool ok = (p0 + b * kWaves) < pairs && g < G;
        buf[b] = ok ? wtile[(size_t)g * 32 + piece] : make_uint4(0, 0, 0, 0);
        sc[b] = ok ? bf16_widen(stile[g * 8 + r]) : 0.0f;
    }

    const uint32_t *x32 = reinterpret_cast<const uint32_t *>(x);
    for (int i = threadIdx.x; i < (K >> 1); i += kThreads) xs[i] = x32[i];
    __syncthreads();
    for (int i = threadIdx.x; i < 4 * G; i += kThreads) {
        const int g = i >> 2, b = i & 3;
        const uint16_t *xv = reinterpret_cast<const uint16_t *>(xs) + g * 128 + 8 * b;
        float s = 0.0f;
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
            for (int j = 0; j < 8; ++j) s += bf16_widen(xv[32 * q + j]);
        xsum[i] = s;
    }
    __syncthreads();

    float acc = 0.0f;
    for (; p0 < pairs; p0 += kBatch * kWaves) {
        uint4 nbuf[kBatch];
        float nsc[kBatch];
        const int p1 = p0 + kBatch * kWaves;
#pragma unroll
        for (int b = 0; b < kBatch; ++b) {
            const int g = 2 * (p1 + b * kWaves) + half;
            const bool ok = (p1 + b * kWaves) < pairs && g < G;
            nbuf[b] = ok ? wtile[(size_t)g * 32 + piece] : make_uint4(0, 0, 0, 0);
            nsc[b] = ok ? bf16_widen(stile[g * 8 + r]) : 0.0f;
        }
#pragma unroll
        for (int b = 0; b < kBatch; ++b) {
            const int g = 2 * (p0 + b * kWaves) + half;
            if ((p0 + b * kWaves) < pairs && g < G) {
                const uint4 *xq = reinterpret_cast<const uint4 *>(xs) + g * 16 + kb;
                const uint4 xrow[4] = {xq[0], xq[4], xq[8], xq[12]};
                acc = fmaf(piece_dot(buf[b], xrow, xsum[4 * g + kb]), sc[b], acc);
            }
            buf[b] = nbuf[b];
            sc[b] = nsc[b];
        }
    }

    /* Lanes r, r+8, ..., r+56 hold row r's partials. */
    acc += __shfl_xor(acc, 8);
    acc += __shfl_xor(acc, 16);
    acc += __shfl_xor(acc, 32);
    if (lane < 8) red[wave * 8 + lane] = acc;
    __syncthreads();
    if (threadIdx.x < 8) {
        float v = 0.0f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) v += red[w * 8 + threadIdx.x];
        red[kWaves * 8 + threadIdx.x] = v;
    }
    __syncthreads();
    if (PAIR) {
        if (threadIdx.x < 4) {
            const float gate = bf16_widen(bf16_rne(red[kWaves * 8 + threadIdx.x]));
            const float up = bf16_widen(bf16_rne(red[kWaves * 8 + 4 + threadIdx.x]));
            reinterpret_cast<uint16_t *>(out)[tile * 4 + threadIdx.x] = silu_mul_bf16(gate, up);
        }
    } else if (threadIdx.x < 8) {
        const float v = red[kWaves * 8 + threadIdx.x];
        if (OUT_F32)
            reinterpret_cast<float *>(out)[tile * 8 + threadIdx.x] = v;
        else
            reinterpret_cast<uint16_t *>(out)[tile * 8 + threadIdx.x] = bf16_rne(v);
    }
}

__global__ void silu_mul_packed_kernel(uint16_t *__restrict__ out,
                                       const uint16_t *__restrict__ packed, int tokens,
                                       int inter) {
    const int row = blockIdx.y;
    const uint16_t *in = packed + (size_t)row * 2 * inter;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < inter; i += gridDim.x * blockDim.x)
        out[(size_t)row * inter + i] = silu_mul_bf16(bf16_widen(in[i]), bf16_widen(in[inter + i]));
}

/* One thread per tile dword (the inverse of it is w4a16_tile_unpack_host). */
__global__ void tile_pack_kernel(const uint8_t *__restrict__ packed,
                                 const uint16_t *__restrict__ scales, uint32_t *__restrict__ pt,
                                 uint16_t *__restrict__ stl, long long n, long long k, int pair) {
    const long long groups = k >> 7;
    const long long total = (n >> 3) * groups * 128;
    for (long long d = blockIdx.x * (long long)blockDim.x + threadIdx.x; d < total;
         d += (long long)gridDim.x * blockDim.x) {
        const int s = (int)(d & 3);
        const int r = (int)((d >> 2) & 7);
        const int kb = (int)((d >> 5) & 3);
        const long long unit = d >> 7;
        const long long g = unit % groups;
        const long long t = unit / groups;
        const long long row = tile_source_row(t, r, n, pair);
        const long long c0 = g * 128 + 32 * s + 8 * kb;
        const uint32_t word = *reinterpret_cast<const uint32_t *>(packed + row * (k >> 1) + (c0 >> 1));
        pt[d] = spread_nibbles(word);
        if (s == 0 && kb == 0) stl[unit * 8 + r] = scales[row * groups + g];
    }
}

/* One thread per tile dword: eight FP32 outputs code * scale at their row-major positions. */
__global__ void dequant_tiled_kernel(const uint32_t *__restrict__ pt,
                                     const uint16_t *__restrict__ stl, float *__restrict__ out,
                                     long long n, long long k, int pair) {
    const long long groups = k >> 7;
    const long long total = (n >> 3) * groups * 128;
    for (long long d = blockIdx.x * (long long)blockDim.x + threadIdx.x; d < total;
         d += (long long)gridDim.x * blockDim.x) {
        const int s = (int)(d & 3);
        const int r = (int)((d >> 2) & 7);
        const int kb = (int)((d >> 5) & 3);
        const long long unit = d >> 7;
        const long long g = unit % groups;
        const long long t = unit / groups;
        const long long row = tile_source_row(t, r, n, pair);
        const float sc = bf16_widen(stl[unit * 8 + r]);
        const uint32_t word = gather_nibbles(pt[d]);
        const long long c0 = g * 128 + 32 * s + 8 * kb;
#pragma unroll
        for (int j = 0; j < 8; ++j)
            out[row * k + c0 + j] = (float)nibble_code((int)((word >> (4 * j)) & 0xF)) * sc;
    }
}

/* One thread per (row, group): the format's quantizer, bit-exact with the host one. */
__global__ void quantize_kernel(const float *__restrict__ w, uint8_t *__restrict__ packed,
                                uint16_t *__restrict__ scales, int *__restrict__ status,
                                long long n, long long k) {
    const long long groups = k >> 7;
    const long long total = n * groups;
    for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < total;
         i += (long long)gridDim.x * blockDim.x) {
        const long long row = i / groups, g = i % groups;
        const float *src = w + row * k + g * 128;
        float peak = 0.0f;
        bool finite = true;
        for (int j = 0; j < 128; ++j) {
            const float a = fabsf(src[j]);
            finite = finite && (a <= 3.402823466e38f);
            peak = fmaxf(peak, a);
        }
        const uint16_t bits = bf16_rne(peak > 0.0f ? peak / 7.0f : 1.0f);
        const float s = bf16_widen(bits);
        if (!finite || !(s > 0.0f) || !(s <= 3.402823466e38f)) atomicOr(status, 1);
        scales[i] = bits;
        uint32_t *dst = reinterpret_cast<uint32_t *>(packed + row * (k >> 1) + g * 64);
        for (int c = 0; c < 16; ++c) {
            uint32_t word = 0;
#pragma unroll
            for (int j = 0; j < 8; ++j)
                word |= (uint32_t)(quant_code(src[8 * c + j], s) & 0xF) << (4 * j);
            dst[c] = word;
        }
    }
}

int hip_status(hipError_t e, const char *what) {
    if (e == hipSuccess) return W4A16_OK;
    return set_error(W4A16_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

int grid_for(long long work, int block) {
    long long g = (work + block - 1) / block;
    if (g > 65535LL * 16) g = 65535LL * 16;
    return (int)(g < 1 ? 1 : g);
}

size_t gemv_smem(int K) { return (size_t)K * 2 + (size_t)(K / 128) * 16 + (kWaves + 1) * 32; }

template <bool PAIR, bool OUT_F32>
int launch_gemv(const uint16_t *x, const uint8_t *w, const uint16_t *s, void *out, int N, int K,
                hipStream_t stream) {
    const size_t smem = gemv_smem(K);
    hipLaunchKernelGGL((gemv_tiles_kernel<PAIR, OUT_F32>), dim3(N / 8), dim3(kThreads), smem,
                       stream, x, reinterpret_cast<const uint4 *>(w), s, out, K);
    return hip_status(hipGetLastError(), "gemv launch");
}

/* Shape refusals of the reference wrapper (csrc/kernels/gemm_quant.cu:204-231), plus the
 * tile rules this layout adds (N % 8, group == 128). */
int check_gemm_args(const void *a, const void *p, const void *s, const void *o, int M, int N,
                    int K, int group, const char *what) {
    if (M < 0 || N < 0 || K <= 0 || group <= 0)
        return set_error(W4A16_ERR_CONFIG, "%s: negative extent or nonpositive group", what);
    if (M == 0 || N == 0) return 1; /* no-op */
    if (!a || !p || !s || !o) return set_error(W4A16_ERR_CONFIG, "%s: null buffer", what);
    if (K % group != 0)
        return set_error(W4A16_ERR_CONFIG, "%s: K=%d is not a whole number of %d-wide groups",
                         what, K, group);
    if (group % 8 != 0)
        return set_error(W4A16_ERR_CONFIG, "%s: a group must be a multiple of 8; got %d", what,
                         group);
    if (group != W4A16_GROUP)
        return set_error(W4A16_ERR_CONFIG, "%s: the tile order holds 128-wide groups, not %d",
                         what, group);
    if (N % W4A16_TILE_ROWS != 0)
        return set_error(W4A16_ERR_CONFIG, "%s: N=%d is not a whole number of 8-row tiles",
                         what, N);
    if (K > kMaxGemvK)
        return set_error(W4A16_ERR_CONFIG, "%s: K=%d needs more activation staging than one "
                         "block has (max %d)", what, K, kMaxGemvK);
    return 0;
}

}  // namespace

/* ---------------------------------------------------------------------------------------- */
/* C ABI                                                                                     */
/* ---------------------------------------------------------------------------------------- */

extern "C" int gemm_int4_bf16(const uint16_t *a, const uint8_t *packed, const uint16_t *scales,
                              uint16_t *out, int M, int N, int K, int group, void *stream) {
    int st = check_gemm_args(a, packed, scales, out, M, N, K, group, "gemm_int4_bf16");
    if (st) return st > 0 ? W4A16_OK : st;
    hipStream_t s = static_cast<hipStream_t>(stream);
    for (int m = 0; m < M; ++m) {
        st = launch_gemv<false, false>(a + (size_t)m * K, packed, scales, out + (size_t)m * N, N,
                                       K, s);
        if (st) return st;
    }
    return W4A16_OK;
}

extern "C" int gate_up_silu_int4_bf16(const uint16_t *x, const uint8_t *gu_packed,
                                      const uint16_t *gu_scales, uint16_t *act, int M, int hidden,
                                      int inter, void *stream) {
    if (inter < 0) return set_error(W4A16_ERR_CONFIG, "gate_up_silu: negative intermediate");
    int st = check_gemm_args(x, gu_packed, gu_scales, act, M, 2 * inter, hidden, W4A16_GROUP,
                             "gate_up_silu_int4_bf16");
    if (st) return st > 0 ? W4A16_OK : st;
    hipStream_t s = static_cast<hipStream_t>(stream);
    for (int m = 0; m < M; ++m) {
        st = launch_gemv<true, false>(x + (size_t)m * hidden, gu_packed, gu_scales,
                                      act + (size_t)m * inter, 2 * inter, hidden, s);
        if (st) return st;
    }
    return W4A16_OK;
}

static int mlp_common(const uint16_t *normed, const uint8_t *gup, const uint16_t *gus,
                      const uint8_t *dnp, const uint16_t *dns, void *out, bool out_f32,
                      uint16_t *act, int M, int hidden, int inter, void *stream) {
    if (M < 0 || hidden <= 0 || inter <= 0)
        return set_error(W4A16_ERR_CONFIG, "mlp_int4: bad extents M=%d hidden=%d inter=%d", M,
                         hidden, inter);
    if (M == 0) return W4A16_OK;
    if (!act || !out) return set_error(W4A16_ERR_CONFIG, "mlp_int4: null buffer");
    int st = check_gemm_args(act, dnp, dns, out, M, hidden, inter, W4A16_GROUP, "mlp_int4 down");
    if (st < 0) return st;
    st = gate_up_silu_int4_bf16(normed, gup, gus, act, M, hidden, inter, stream);
    if (st) return st;
    hipStream_t s = static_cast<hipStream_t>(stream);
    for (int m = 0; m < M; ++m) {
        st = out_f32 ? launch_gemv<false, true>(act + (size_t)m * inter, dnp, dns,
                                                static_cast<float *>(out) + (size_t)m * hidden,
                                                hidden, inter, s)
                     : launch_gemv<false, false>(act + (size_t)m * inter, dnp, dns,
                                                 static_cast<uint16_t *>(out) + (size_t)m * hidden,
                                                 hidden, inter, s);
        if (st) return st;
    }
    return W4A16_OK;
}

extern "C" int mlp_int4_bf16(const uint16_t *normed, const uint8_t *gup, const uint16_t *gus,
                             const uint8_t *dnp, const uint16_t *dns, uint16_t *out,
                             uint16_t *act_ws, int M, int hidden, int inter, void *stream) {
    return mlp_common(normed, gup, gus, dnp, dns, out, false, act_ws, M, hidden, inter, stream);
}

extern "C" int mlp_int4_partial_f32(const uint16_t *normed, const uint8_t *gup,
                                    const uint16_t *gus, const uint8_t *dnp, const uint16_t *dns,
                                    float *out_f32, uint16_t *act_ws, int M, int hidden,
                                    int inter, void *stream) {
    return mlp_common(normed, gup, gus, dnp, dns, out_f32, true, act_ws, M, hidden, inter, stream);
}

extern "C" int silu_mul_packed_bf16(uint16_t *out, const uint16_t *packed, int tokens, int inter,
                                    void *stream) {
    if (tokens < 0 || inter < 0)
        return set_error(W4A16_ERR_CONFIG, "silu_mul_packed: negative extent");
    if (tokens == 0 || inter == 0) return W4A16_OK;
    if (!out || !packed) return set_error(W4A16_ERR_CONFIG, "silu_mul_packed: null buffer");
    const int block = 256;
    hipLaunchKernelGGL(silu_mul_packed_kernel, dim3((inter + block - 1) / block, tokens),
                       dim3(block), 0, static_cast<hipStream_t>(stream), out, packed, tokens,
                       inter);
    return hip_status(hipGetLastError(), "silu_mul_packed launch");
}

extern "C" int w4a16_tile_pack_device(long long n, long long k, int pair, const uint8_t *packed,
                                      const uint16_t *scales, uint8_t *packed_tiled,
                                      uint16_t *scales_tiled, void *stream) {
    if (!packed || !scales || !packed_tiled || !scales_tiled)
        return set_error(W4A16_ERR_CONFIG, "tile_pack_device: null argument");
    int st = w4a16_layout_init(n, k, W4A16_GROUP, nullptr, nullptr);
    if (st) return st;
    if (pair != 0 && pair != 1) return set_error(W4A16_ERR_CONFIG, "tile_pack_device: bad pair");
    const long long total = (n / 8) * (k / 128) * 128;
    hipLaunchKernelGGL(tile_pack_kernel, dim3(grid_for(total, 256)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), packed, scales,
                       reinterpret_cast<uint32_t *>(packed_tiled), scales_tiled, n, k, pair);
    return hip_status(hipGetLastError(), "tile_pack launch");
}

extern "C" int w4a16_dequant_tiled_device(long long n, long long k, int pair,
                                          const uint8_t *packed_tiled,
                                          const uint16_t *scales_tiled, float *out,
                                          void *stream) {
    if (!packed_tiled || !scales_tiled || !out)
        return set_error(W4A16_ERR_CONFIG, "dequant_tiled_device: null argument");
    int st = w4a16_layout_init(n, k, W4A16_GROUP, nullptr, nullptr);
    if (st) return st;
    if (pair != 0 && pair != 1) return set_error(W4A16_ERR_CONFIG, "dequant_tiled: bad pair");
    const long long total = (n / 8) * (k / 128) * 128;
    hipLaunchKernelGGL(dequant_tiled_kernel, dim3(grid_for(total, 256)), dim3(256), 0,
                       static_cast<hipStream_t>(stream),
                       reinterpret_cast<const uint32_t *>(packed_tiled), scales_tiled, out, n, k,
                       pair);
    return hip_status(hipGetLastError(), "dequant_tiled launch");
}

extern "C" int w4a16_quantize_device(long long n, long long k, const float *weights,
                                     uint8_t *packed, uint16_t *scales, int *status_dev,
                                     void *stream) {
    if (!weights || !packed || !scales || !status_dev)
        return set_error(W4A16_ERR_CONFIG, "quantize_device: null argument");
    int st = w4a16_layout_init(n, k, W4A16_GROUP, nullptr, nullptr);
    if (st) return st;
    const long long total = n * (k / 128);
    hipLaunchKernelGGL(quantize_kernel, dim3(grid_for(total, 256)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), weights, packed, scales, status_dev, n,
                       k);
    return hip_status(hipGetLastError(), "quantize launch");
}
