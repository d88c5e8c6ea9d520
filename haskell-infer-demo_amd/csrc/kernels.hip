/*
 * kernels.hip - gfx950 kernels of the W4A16 dense-FFN decode path and their C-ABI launchers.
 *
 * Weights are read in the tile order described in common.h. The M = 1 kernels are wave64
 * GEMVs: each lane loads one 16-byte piece (32 codes of one row) per step with a single
 * buffer_load_dwordx4, turns each pair of codes into a BF16 pair with one v_perm_b32 (value
 * 0.5 + u/32, u = nibble ^ 8 = code + 8, exact in BF16), and accumulates with the packed BF16
 * dot product v_dot2_f32_bf16 against the activation pair. Since code = 32 v - 24, a piece's
 * contribution is 32 * dot(v, x) - 24 * sum(x); the per-piece activation sums are computed once
 * per block when the activation is staged in LDS. The
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

constexpr int kMaxLoads = 12;     /* 16-byte pieces in flight per lane (all of a wave's share) */
constexpr int kMaxGemvK = 30464;  /* activation staged in LDS: 2K bytes + sums within 64 KiB */

__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                           __builtin_bit_cast(bf16x2_t, b), c, false);
}

/* Code pairs as BF16. A tile word's low nibbles [j0, j4, j1, j5] (one per byte) and high
 * nibbles [j2, j6, j3, j7] are moved to bits 3-6 of their bytes with the sign bit flipped
 * (u = code + 8), and v_perm_b32 places two of them under the byte 0x3F: the BF16 value is
 * 2^-1 * (1 + u/16) = 0.5 + u/32 = 0.75 + code/32, exact. Keeping the nibble in the top mantissa
 * bits keeps the offset small (0.75 against a code step of 1/32), so the FP32 sums lose little
 * to the offset that is subtracted afterwards. */
constexpr uint32_t kMagic = 0x3F3F3F3Fu;
constexpr uint32_t kSelLo = 0x04020400u; /* bytes 0 and 2 of the nibble word */
constexpr uint32_t kSelHi = 0x04030401u; /* bytes 1 and 3 */

/* sum_{j<32} code_j * x_j for one 16-byte piece: 32 * dot(v, x) - 24 * xsum. Four independent
 * accumulators (one per dword) keep the dot-product chains short. */
__device__ __forceinline__ float piece_dot(uint4 piece, const uint4 *xq, float xsum) {
    const uint32_t words[4] = {piece.x, piece.y, piece.z, piece.w};
    float d[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        const uint32_t t = ((words[s] << 3) ^ 0x40404040u) & 0x78787878u;
        const uint32_t t2 = ((words[s] >> 1) ^ 0x40404040u) & 0x78787878u;
        const uint4 xv = xq[s];
        float a = dot2_bf16(__builtin_amdgcn_perm(kMagic, t, kSelLo), xv.x, 0.0f);
        a = dot2_bf16(__builtin_amdgcn_perm(kMagic, t2, kSelLo), xv.y, a);
        a = dot2_bf16(__builtin_amdgcn_perm(kMagic, t, kSelHi), xv.z, a);
        d[s] = dot2_bf16(__builtin_amdgcn_perm(kMagic, t2, kSelHi), xv.w, a);
    }
    return fmaf(32.0f, (d[0] + d[1]) + (d[2] + d[3]), -24.0f * xsum);
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

/* Raw buffer access: an offset past num_records reads 0 without a branch, which keeps every
 * load of a wave unconditional (a predicated global load is compiled as a branch plus a wait). */
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes,
                                             0x00020000);
}

__device__ __forceinline__ uint4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0);
    return __builtin_bit_cast(uint4, v);
}

__device__ __forceinline__ uint16_t buf_load_u16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b16(r, (int)off, 0, 0);
}

constexpr uint32_t kOob = 0x80000000u; /* an offset no buffer here reaches: reads return 0 */

/* A block holds TB consecutive 8-row tiles and W = TB * SK waves: wave w works on tile w / SK and
 * takes the group pairs (w % SK) + SK * i of it; half-wave h of a step takes group 2 * pair + h.
 * The activation loads are issued first, then every weight and scale load of the wave, so one
 * wait covers the activation and the weights stream while it is staged into LDS.
 * PAIR: a tile is 4 gate + 4 up rows and yields four BF16(silu(BF16 gate) x BF16 up) values;
 * otherwise eight BF16 outputs (or FP32 if OUT_F32). */
template <bool PAIR, bool OUT_F32, int TB, int SK>
__global__ __launch_bounds__(TB * SK * 64) void gemv_tiles_kernel(
    const uint16_t *__restrict__ x, const uint8_t *__restrict__ wt,
    const uint16_t *__restrict__ st, void *__restrict__ out, int N, int K) {
    constexpr int W = TB * SK;
    /* the largest K this configuration is launched for: SK * kMaxLoads group pairs */
    constexpr int kMaxK = (256 * kMaxLoads * SK < kMaxGemvK) ? 256 * kMaxLoads * SK : kMaxGemvK;
    constexpr int kXIters = (kMaxK / 8 + W * 64 - 1) / (W * 64);
    extern __shared__ uint4 smem4[];
    const int G = K >> 7;
    const int P = (G + 1) >> 1;
    const int tiles = N >> 3;
    float *xsum = reinterpret_cast<float *>(smem4 + (K >> 3));
    float *red = xsum + 4 * G;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    /* wave-uniform, made scalar so the buffer descriptors below live in SGPRs */
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int tile = blockIdx.x * TB + wave / SK;
    const int ks = wave % SK;
    const int half = lane >> 5;
    const int piece = lane & 31;
    const int kb = piece >> 3;
    const int r = piece & 7;

    /* 1. activation loads (L2-resident; the first ones to return) */
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(x, (uint32_t)K * 2);
    const int xchunks = K >> 3;
    uint4 xv[kXIters];
#pragma unroll
    for (int it = 0; it < kXIters; ++it) {
        const int i = it * W * 64 + tid;
        xv[it] = buf_load16(xr, i < xchunks ? (uint32_t)i * 16 : kOob);
    }

    /* 2. every weight piece and scale of this wave */
    const bool tile_ok = tile < tiles;
    const size_t tile_bytes = (size_t)G * 512;
    const __amdgpu_buffer_rsrc_t wr =
        make_rsrc(wt + (size_t)(tile_ok ? tile : 0) * tile_bytes, tile_ok ? (uint32_t)tile_bytes : 0);
    const __amdgpu_buffer_rsrc_t sr =
        make_rsrc(st + (size_t)(tile_ok ? tile : 0) * G * 8, tile_ok ? (uint32_t)G * 16 : 0);
    uint4 buf[kMaxLoads];
    uint16_t sbits[kMaxLoads];
#pragma unroll
    for (int i = 0; i < kMaxLoads; ++i) {
        const int p = ks + i * SK;
        const int g = 2 * p + half;
        const bool ok = p < P && g < G;
        buf[i] = buf_load16(wr, ok ? (uint32_t)(g * 512 + piece * 16) : kOob);
        sbits[i] = buf_load_u16(sr, ok ? (uint32_t)(g * 16 + r * 2) : kOob);
    }

    /* 3. stage the activation and the per-(group, kb) sums of the codes' x values */
#pragma unroll
    for (int it = 0; it < kXIters; ++it) {
        const int i = it * W * 64 + tid;
        if (i < xchunks) smem4[i] = xv[it];
        const uint32_t w4[4] = {xv[it].x, xv[it].y, xv[it].z, xv[it].w};
        float s8 = 0.0f;
#pragma unroll
        for (int q = 0; q < 4; ++q)
            s8 += bf16_widen((uint16_t)(w4[q] & 0xFFFFu)) + bf16_widen((uint16_t)(w4[q] >> 16));
        /* chunk i = 16 g + 4 s + kb: add the four s of one (g, kb) */
        s8 += __shfl_xor(s8, 4);
        s8 += __shfl_xor(s8, 8);
        if (i < xchunks && ((i >> 2) & 3) == 0) xsum[(i >> 4) * 4 + (i & 3)] = s8;
    }
    __syncthreads();

    /* 4. dot products; a piece past the tile's groups has scale 0 (its loads read 0) and reads
     * the activation of the last group, so it adds exactly 0 without a branch */
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < kMaxLoads; ++i) {
        if (ks + i * SK < P) { /* wave-uniform */
            const int g = min(2 * (ks + i * SK) + half, G - 1);
            const uint4 *xq = smem4 + g * 16 + kb;
            const uint4 xrow[4] = {xq[0], xq[4], xq[8], xq[12]};
            acc = fmaf(piece_dot(buf[i], xrow, xsum[4 * g + kb]), bf16_widen(sbits[i]), acc);
        }
    }

    /* 5. lanes r, r+8, ..., r+56 hold row r's partials; then the SK waves of a tile */
    acc += __shfl_xor(acc, 8);
    acc += __shfl_xor(acc, 16);
    acc += __shfl_xor(acc, 32);
    float row_sum = acc;
    if (SK > 1) {
        if (lane < 8) red[wave * 8 + lane] = acc;
        __syncthreads();
        if (ks == 0 && lane < 8) {
            row_sum = 0.0f;
#pragma unroll
            for (int w = 0; w < SK; ++w) row_sum += red[(wave + w) * 8 + lane];
        }
    }
    if (ks != 0 || !tile_ok) return;
    if (PAIR) {
        /* lane r < 4 has gate row r, lane r + 4 the matching up row */
        const float upv = __shfl_down(row_sum, 4);
        if (lane < 4) {
            const float gate = bf16_widen(bf16_rne(row_sum));
            const float up = bf16_widen(bf16_rne(upv));
            reinterpret_cast<uint16_t *>(out)[tile * 4 + lane] = silu_mul_bf16(gate, up);
        }
    } else if (lane < 8) {
        if (OUT_F32)
            reinterpret_cast<float *>(out)[tile * 8 + lane] = row_sum;
        else
            reinterpret_cast<uint16_t *>(out)[tile * 8 + lane] = bf16_rne(row_sum);
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

size_t gemv_smem(int K, int waves) {
    return (size_t)K * 2 + (size_t)(K / 128) * 16 + (size_t)waves * 32;
}

template <bool PAIR, bool OUT_F32, int TB, int SK>
int launch_gemv_cfg(const uint16_t *x, const uint8_t *w, const uint16_t *s, void *out, int N,
                    int K, hipStream_t stream) {
    const int tiles = N / 8;
    hipLaunchKernelGGL((gemv_tiles_kernel<PAIR, OUT_F32, TB, SK>), dim3((tiles + TB - 1) / TB),
                       dim3(TB * SK * 64), gemv_smem(K, TB * SK), stream, x, w, s, out, N, K);
    return hip_status(hipGetLastError(), "gemv launch");
}

/* Split-K: the smallest power of two keeping a wave at <= kMaxLoads pieces; tiles per block
 * then fill four waves where the split leaves room. */
template <bool PAIR, bool OUT_F32>
int launch_gemv(const uint16_t *x, const uint8_t *w, const uint16_t *s, void *out, int N, int K,
                hipStream_t stream) {
    const int pairs = (K / 128 + 1) / 2;
    int sk = 1;
    while (sk < 16 && (pairs + sk - 1) / sk > kMaxLoads) sk *= 2;
    switch (sk) {
        case 1: return launch_gemv_cfg<PAIR, OUT_F32, 4, 1>(x, w, s, out, N, K, stream);
        case 2: return launch_gemv_cfg<PAIR, OUT_F32, 2, 2>(x, w, s, out, N, K, stream);
        case 4: return launch_gemv_cfg<PAIR, OUT_F32, 1, 4>(x, w, s, out, N, K, stream);
        case 8: return launch_gemv_cfg<PAIR, OUT_F32, 1, 8>(x, w, s, out, N, K, stream);
        default: return launch_gemv_cfg<PAIR, OUT_F32, 1, 16>(x, w, s, out, N, K, stream);
    }
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
