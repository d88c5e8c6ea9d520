/*
 * kernels.hip - gfx950 kernels of the W4A16 dense-FFN decode path and their C-ABI launchers.
 *
 * Weights are read in the tile order described in common.h. The M = 1 kernels are wave64
 * GEMVs: each lane loads one 16-byte piece (32 codes of one row) per step with a single
 * buffer_load_dwordx4, turns each pair of codes into a BF16 pair with at most one shift and one
 * v_bitop3_b32 (value 0.5 + u/32, u = nibble ^ 8 = code + 8, exact in BF16), and accumulates with
 * the packed BF16 dot product v_dot2c_f32_bf16 against the activation pair, whose activation
 * operand is broadcast over DPP from the lane of its quad that holds it. Since code = 32 v - 24,
 * a piece's contribution is 32 * dot(v, x) - 24 * sum(x), with the per-piece activation sums
 * formed by DPP adds (or once when the activation is staged in LDS). The group's BF16 scale multiplies each
 * piece's FP32 partial (the association of the reference's tiled kernel,
 * csrc/kernels/gemm_quant.cu:130-142). Lanes of one row are reduced with DPP moves within rows
 * of 16 lanes and shuffles across them.
 *
 *   gemv_tiles_kernel   M = 1, block-staged activation (gate/up with the fused SiLU x up
 *                       epilogue, short-K linears); optional RMSNorm (and residual) prologue
 *   gemv_xwave_kernel   M = 1, long K (the down projection) and K = 1792..3072 (with the
 *                       fused SiLU x up epilogue for gate/up): each wave loads only its own
 *                       pairs' activation, no LDS before the reduction; optional residual epilogue
 *   gemv_mfma1_kernel   M = 1 or 2 on v_mfma_f32_16x16x32_bf16 with a block-diagonal operand, one
 *                       tile a block, wave-local activation: the C1 down projection's 37 to 48
 *                       group pairs, linears of 7 to 12 and 17 to 20 pairs, and at M = 2 the
 *                       gate/up pair
 *   gemv_rows_kernel    2 <= M <= 8: the GEMV's block structure on v_mfma_f32_16x16x32_bf16 with
 *                       a block-diagonal operand, activation loaded straight into LDS
 *   gemv_rows16_kernel  9 <= M <= 16, short K: the same with a tile pair a wave
 *   gemv_rows16x_kernel long K, no pair (the down projection): a tile pair a block, each lane
 *                       loading its MFMA A operand from memory into registers (no LDS staging,
 *                       no K split across blocks); 4 <= M <= 16 inside the FFN entry points,
 *                       which keep the intermediate chunk-major for it, 8 <= M <= 15 on
 *                       row-major rows in gemm_int4_bf16
 *   mfma_gemm_kernel    2 <= M <= 16 where the above do not fit: v_mfma_f32_16x16x32_bf16, K
 *                       split across blocks
 *   rmsnorm_kernel, residual_add_kernel, silu_mul_packed_kernel: the norm, the residual update
 *                       and the standalone SiLU x up
 *   tile_pack_kernel, dequant_tiled_kernel, quantize_kernel: the load-time re-layout and the
 *                       checks of it
 */
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <mutex>

#include "common.h"

using namespace w4a16;

namespace {

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

constexpr int kMaxLoads = 12;     /* group pairs one wave holds when it takes a whole tile (norm prologue) */
constexpr int kMaxGemvK = 30464;  /* block-staged GEMV: 2K bytes of activation + sums in 64 KiB */
constexpr int kMaxRowK = 49152;   /* M = 1: the reference's limit (K * 2 <= 96 KiB of staging) */
constexpr int kMaxAnyK = 1 << 20; /* M > 1 (the MFMA form stages only its K range) */
constexpr size_t kMaxLds = 163840; /* LDS a block can allocate on gfx950 */

/* Cross-lane moves on the DPP path (a VALU operand modifier, no LDS round trip). quad_perm
 * patterns permute within groups of four lanes, row_ror:n rotates within rows of sixteen, and
 * row_half_mirror reverses each group of eight. */
constexpr int kDppQuadSwap1 = 0xB1;      /* quad_perm [1,0,3,2]: lane ^ 1 */
constexpr int kDppQuadSwap2 = 0x4E;      /* quad_perm [2,3,0,1]: lane ^ 2 */
constexpr int kDppRowRor4 = 0x124;       /* row_ror:4 */
constexpr int kDppRowRor8 = 0x128;       /* row_ror:8: lane ^ 8 within a row */
constexpr int kDppRowShl4 = 0x104;       /* row_shl:4: lane l reads lane l + 4 of its row */

/* The value of v in the lane the DPP pattern names (a lane with no source reads 0: the bound
 * control that lets the compiler fold the move into the VALU instruction that uses it, e.g. one
 * v_add_f32_dpp instead of a v_mov_b32_dpp and a v_add_f32). */
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}

/* v + v[l ^ 16] and v + v[l ^ 32] over the wave, on every lane, by the gfx950 lane swaps
 * (v_permlane16_swap_b32 exchanges the odd rows of sixteen lanes of its first operand with the
 * even rows of its second, v_permlane32_swap_b32 the upper half of the first with the lower half
 * of the second; both operands hold v, so the two results are the lane's value and its partner's).
 * A VALU exchange instead of an LDS-crossbar shuffle; the sum is the same FP32 add as
 * v + __shfl_xor(v, 16 or 32). Inline asm because the compiler builtin does not keep its two
 * results apart when both operands are one value; the waits cover the hazards the compiler
 * cannot see inside the asm. */
__device__ __forceinline__ float lane_sum16(float v) {
    float x = v, y = v;
    asm volatile("s_nop 1\n v_permlane16_swap_b32 %0, %1\n s_nop 1" : "+v"(x), "+v"(y));
    return x + y;
}
__device__ __forceinline__ float lane_sum32(float v) {
    float x = v, y = v;
    asm volatile("s_nop 1\n v_permlane32_swap_b32 %0, %1\n s_nop 1" : "+v"(x), "+v"(y));
    return x + y;
}

/* Code pairs as BF16. In a tile word the pair (j = 2q, 2q+1) sits at bits 3 + 4q and 19 + 4q
 * (the word is stored rotated left by 3 bits, so the odd code of q = 3 wraps round to bits 31 and
 * 0-2): pair 0 already sits at bits 3-6 of its two 16-bit halves, pairs 1 and 2 get there by a
 * right shift of 4q and pair 3 by a rotation of 12 (v_alignbit_b32), and one v_bitop3_b32 then
 * computes (s & 0x00780078) ^ 0x3F403F40: it keeps the two nibbles, flips their sign bits
 * (u = code + 8) and sets the exponent byte 0x3F (the mask and the constant are disjoint but for
 * the sign bits). Three shifts and four bit operations a word, where a pair order that needs a
 * shift for every pair costs four and four. The BF16 value is 2^-1 * (1 + u/16) = 0.5 + u/32 =
 * 0.75 + code/32, exact. Keeping the nibble in the top mantissa bits keeps the offset small
 * (0.75 against a code step of 1/32), so the FP32 sums lose little to the offset that is
 * subtracted afterwards. */
__device__ __forceinline__ uint32_t code_pair(uint32_t shifted) {
    return (shifted & 0x00780078u) ^ 0x3F403F40u;
}

/* The four BF16 code pairs of a tile word, in k order. */
__device__ __forceinline__ uint4 code_pairs(uint32_t word) {
    uint4 v;
    v.x = code_pair(word);
    v.y = code_pair(word >> 4);
    v.z = code_pair(word >> 8);
    v.w = code_pair(__builtin_amdgcn_alignbit(word, word, 12));
    return v;
}

/* (1/32) sum_{j<32} code_j * x_j for one 16-byte piece (row r, k block kb of a group):
 * dot(v, x) - 0.75 xsum, with v = 0.75 + code/32 from the unpack above and xsum the sum of the 32
 * x values; the chain starts from a0 = -0.75 xsum (quad_offset) and callers multiply their
 * accumulated sum by 32 (exact) once.
 * The activation comes from the lane's quad through DPP: quad lane s holds the 8 values
 * 32 s + 8 kb + (0..7) of the group as four dwords, and every v_dot2c reads its activation
 * operand from quad lane s by a quad_perm broadcast, so no lane needs more than its own 16 bytes
 * of activation. The 16 products form one dependent v_dot2c chain in the order (s, dword) (the
 * accumulator forwards, so splitting it only adds combining work). The compiler does not fold a DPP move into v_dot2c, hence the inline asm, and it
 * cannot see the two hazards inside it: a VALU write of a register that a DPP operand reads
 * needs two wait states before the first instruction (the leading s_nop 1), and a v_dot2c result
 * needs a wait state before a following VALU instruction reads it (the trailing s_nop 1; without
 * it the last product is lost, which the compiler guards against in its own code the same way).
 * The sum is bit-identical to the same chain written in plain HIP with the activation in LDS. */
__device__ __forceinline__ float piece_dot_dpp(uint4 piece, uint4 xq, float a0) {
    const uint32_t w[4] = {piece.x, piece.y, piece.z, piece.w};
    uint32_t c[16];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        const uint4 v = code_pairs(w[s]);
        c[4 * s] = v.x;
        c[4 * s + 1] = v.y;
        c[4 * s + 2] = v.z;
        c[4 * s + 3] = v.w;
    }
    float a = a0;
#define W4A16_DOT2_DPP(S, X, C)                                                                  \
    "v_dot2c_f32_bf16_dpp %0, " X ", " C " quad_perm:[" S "," S "," S "," S "] row_mask:0xf "   \
    "bank_mask:0xf\n"
    asm volatile("s_nop 1\n"
                 W4A16_DOT2_DPP("0", "%1", "%5") W4A16_DOT2_DPP("0", "%2", "%6")
                 W4A16_DOT2_DPP("0", "%3", "%7") W4A16_DOT2_DPP("0", "%4", "%8")
                 W4A16_DOT2_DPP("1", "%1", "%9") W4A16_DOT2_DPP("1", "%2", "%10")
                 W4A16_DOT2_DPP("1", "%3", "%11") W4A16_DOT2_DPP("1", "%4", "%12")
                 W4A16_DOT2_DPP("2", "%1", "%13") W4A16_DOT2_DPP("2", "%2", "%14")
                 W4A16_DOT2_DPP("2", "%3", "%15") W4A16_DOT2_DPP("2", "%4", "%16")
                 W4A16_DOT2_DPP("3", "%1", "%17") W4A16_DOT2_DPP("3", "%2", "%18")
                 W4A16_DOT2_DPP("3", "%3", "%19") W4A16_DOT2_DPP("3", "%4", "%20")
                 "s_nop 1\n"
                 : "+v"(a)
                 : "v"(xq.x), "v"(xq.y), "v"(xq.z), "v"(xq.w), "v"(c[0]), "v"(c[1]), "v"(c[2]),
                   "v"(c[3]), "v"(c[4]), "v"(c[5]), "v"(c[6]), "v"(c[7]), "v"(c[8]), "v"(c[9]),
                   "v"(c[10]), "v"(c[11]), "v"(c[12]), "v"(c[13]), "v"(c[14]), "v"(c[15]));
#undef W4A16_DOT2_DPP
    return a;
}

/* The sum of the eight BF16 values of a 16-byte chunk as four chained packed dot products with
 * (1, 1): exact products, FP32 sums, one VALU instruction per two values (unpacking each value
 * to FP32 and adding costs three). */
__device__ __forceinline__ float chunk_sum8(uint4 v) {
    const bf16x2_t one = __builtin_bit_cast(bf16x2_t, 0x3F803F80u);
    float s = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, v.x), one, 0.0f, false);
    s = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, v.y), one, s, false);
    s = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, v.z), one, s, false);
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, v.w), one, s, false);
}

/* -0.75 times the sum of the 32 activation values a quad of lanes holds (8 a lane): the lane's
 * chunk sum, then the quad's four lane sums by two DPP adds (each one v_add_f32_dpp). The start
 * value of a piece's dot chain. */
__device__ __forceinline__ float quad_offset(uint4 v) {
    float s8 = chunk_sum8(v);
    s8 += dpp_f32<kDppQuadSwap1>(s8);
    s8 += dpp_f32<kDppQuadSwap2>(s8);
    return -0.75f * s8;
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

/* Index of element (m, i) of an M x cols activation: row-major, or (cm) chunk-major, i.e.
 * [cols / 8 chunks][M rows][8 values], where one 16-byte chunk of every row sits together, so
 * the MFMA A operands of all rows at one k block are contiguous in memory. */
__device__ __forceinline__ size_t act_index(int m, int i, int M, int cols, int cm) {
    return cm ? ((size_t)(i >> 3) * M + m) * 8 + (i & 7) : (size_t)m * cols + i;
}

/* Two packed BF16 sums, each BF16(f32(a) + f32(b)) (the residual update of reference
 * csrc/kernels/gdn_norm.cu:121-129 and flashinfer_norm.cu:124-126). */
__device__ __forceinline__ uint32_t bf16_add2(uint32_t a, uint32_t b) {
    const float lo = bf16_widen((uint16_t)(a & 0xFFFFu)) + bf16_widen((uint16_t)(b & 0xFFFFu));
    const float hi = bf16_widen((uint16_t)(a >> 16)) + bf16_widen((uint16_t)(b >> 16));
    return (uint32_t)bf16_rne(lo) | ((uint32_t)bf16_rne(hi) << 16);
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

/* A weight piece: read once per call, so the load carries the non-temporal hint. */
__device__ __forceinline__ uint4 buf_load16_stream(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 2);
    return __builtin_bit_cast(uint4, v);
}

__device__ __forceinline__ uint16_t buf_load_u16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b16(r, (int)off, 0, 0);
}

constexpr uint32_t kOob = 0x80000000u; /* an offset no buffer here reaches: reads return 0 */

/* Load order. A wave's vector memory loads complete in issue order (one vmcnt counter), so every
 * kernel issues its 2-byte scale loads first and then the weight pieces in the order its pairs
 * are computed, each fixed in place by a scheduling barrier, with a use of the loads on the
 * skipped path of a pair's branch so that none is sunk into the branch. Left to itself the
 * compiler issued the scales after all the weights, and the first pair's scale FMA then waited
 * for the whole weight stream of the wave (with the scales first C4 16.26 -> 15.88 us, C0 4.26 ->
 * 4.19, C1 within the noise; outputs bit-identical). */

/* u / d for 0 <= u < 69905 and 1 <= d <= 16 as (u * ceil(2^20 / d)) >> 20: exact in that range
 * (the rounding excess of the multiplier, at most 15 / 2^20 per unit of u, stays below 1 / d),
 * and with d wave-uniform the multiplier is one scalar computation, where an integer division
 * costs a few dozen VALU instructions per use. div_magic(d) gives the multiplier. */
__device__ __forceinline__ uint32_t div_magic(int d) { return ((1u << 20) + (uint32_t)d - 1u) / (uint32_t)d; }
__device__ __forceinline__ int div_small(int u, uint32_t magic) {
    return (int)(((uint32_t)u * magic) >> 20);
}

/* s_waitcnt immediate that waits until at most N vector memory operations are outstanding
 * (vmcnt in bits 3:0 and 15:14; expcnt and lgkmcnt at their maxima, i.e. not waited on):
 * with the NL weight and NL scale loads of a wave issued last, N = 2 NL waits for everything
 * issued before them. */
template <int NL>
constexpr int kVmcntWeights = ((2 * NL) & 15) | (7 << 4) | (15 << 8) | (((2 * NL) >> 4) << 14);

/* s_waitcnt "at most C - 2 i vector memory operations outstanding" for an unrolled loop index i
 * (the builtin takes only a constant; i >= 4 waits for everything) */
constexpr int vm_enc(int c) { return (c & 15) | (7 << 4) | (15 << 8) | ((c >> 4) << 14); }
template <int C>
__device__ __forceinline__ void wait_vm(int i) {
    switch (i) {
        case 0: __builtin_amdgcn_s_waitcnt(vm_enc(C > 0 ? C : 0)); break;
        case 1: __builtin_amdgcn_s_waitcnt(vm_enc(C - 2 > 0 ? C - 2 : 0)); break;
        case 2: __builtin_amdgcn_s_waitcnt(vm_enc(C - 4 > 0 ? C - 4 : 0)); break;
        case 3: __builtin_amdgcn_s_waitcnt(vm_enc(C - 6 > 0 ? C - 6 : 0)); break;
        default: __builtin_amdgcn_s_waitcnt(vm_enc(0)); break;
    }
}

/* A block holds TB consecutive 8-row tiles and W = TB * SK waves: wave w works on tile w / SK and
 * takes the group pairs (w % SK) + SK * i of it; half-wave h of a step takes group 2 * pair + h.
 * The activation loads are issued first, then every weight and scale load of the wave, so one
 * wait covers the activation and the weights stream while it is staged into LDS.
 * PAIR: a tile is 4 gate + 4 up rows and yields four BF16(silu(BF16 gate) x BF16 up) values;
 * otherwise eight BF16 outputs (or FP32 if OUT_F32). NL: the loads (group pairs) a wave holds,
 * SK * NL >= pairs; sizing it to the shape keeps the VGPR count low enough for 8 waves a SIMD. */
template <bool PAIR, bool OUT_F32, int TB, int SK, bool NORM, int NL>
__global__ __launch_bounds__(TB * SK * 64) void gemv_tiles_kernel(
    const uint16_t *__restrict__ x, const uint8_t *__restrict__ wt,
    const uint16_t *__restrict__ st, void *__restrict__ out, int N, int K,
    const uint16_t *__restrict__ norm_w, float norm_bias, float eps,
    const uint16_t *__restrict__ sub) {
    constexpr int W = TB * SK;
    /* the largest K this configuration is launched for: SK * NL group pairs */
    constexpr int kMaxK = (256 * NL * SK < kMaxGemvK) ? 256 * NL * SK : kMaxGemvK;
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
        /* chunks past K fall outside the descriptor's range and read zeros */
        xv[it] = buf_load16(xr, (uint32_t)(it * W * 64 + tid) * 16);
    }
    uint4 nv[NORM ? kXIters : 1];
    uint4 sv[NORM ? kXIters : 1];
    if (NORM) {
        const __amdgpu_buffer_rsrc_t nr = make_rsrc(norm_w, (uint32_t)K * 2);
        /* a null sublayer reads as zeros (an empty buffer descriptor) */
        const __amdgpu_buffer_rsrc_t ur = make_rsrc(sub, sub ? (uint32_t)K * 2 : 0u);
#pragma unroll
        for (int it = 0; it < kXIters; ++it) {
            const int i = it * W * 64 + tid;
            nv[it] = buf_load16(nr, i < xchunks ? (uint32_t)i * 16 : kOob);
            sv[it] = buf_load16(ur, i < xchunks ? (uint32_t)i * 16 : kOob);
        }
    }

    /* 2. every weight piece and scale of this wave */
    const bool tile_ok = tile < tiles;
    const size_t tile_bytes = (size_t)G * 512;
    const __amdgpu_buffer_rsrc_t wr =
        make_rsrc(wt + (size_t)(tile_ok ? tile : 0) * tile_bytes, tile_ok ? (uint32_t)tile_bytes : 0);
    const __amdgpu_buffer_rsrc_t sr =
        make_rsrc(st + (size_t)(tile_ok ? tile : 0) * G * 8, tile_ok ? (uint32_t)G * 16 : 0);
    uint4 buf[NL];
    uint16_t sbits[NL];
#pragma unroll
    for (int i = 0; i < NL; ++i) { /* the scales first: loads return in issue order */
        /* a group past the tile (g >= G, which covers p >= P) is past both descriptors' ranges
         * and reads zeros, so no offset needs a condition */
        const int g = 2 * (ks + i * SK) + half;
        sbits[i] = buf_load_u16(sr, (uint32_t)(g * 16 + r * 2));
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < NL; ++i) {
        const int g = 2 * (ks + i * SK) + half;
        buf[i] = buf_load16_stream(wr, (uint32_t)(g * 512 + piece * 16));
        __builtin_amdgcn_sched_barrier(0);
    }

    /* 2b. NORM: the activation is the RMSNorm of x, formed here (every block sees all of x):
     * BF16(x * rsqrt(sum x^2 / K + eps) * (norm_bias + w)), the FP32 order of the reference's
     * norm (FlashInfer RMSNorm / GemmaRMSNorm behind csrc/kernels/flashinfer_norm.cu:22-76) */
    if (NORM) {
        /* keep the weight loads above: without this fence the scheduler hoists the sum of
         * squares over them, and the weights would wait for the activation's round trip */
        __builtin_amdgcn_sched_barrier(0);
        if (sub) { /* plan F2: the norm reads BF16(residual + sublayer) */
#pragma unroll
            for (int it = 0; it < kXIters; ++it) {
                const uint32_t a4[4] = {xv[it].x, xv[it].y, xv[it].z, xv[it].w};
                const uint32_t b4[4] = {sv[it].x, sv[it].y, sv[it].z, sv[it].w};
                uint32_t o4[4];
#pragma unroll
                for (int q = 0; q < 4; ++q) o4[q] = bf16_add2(a4[q], b4[q]);
                xv[it] = make_uint4(o4[0], o4[1], o4[2], o4[3]);
            }
        }
        /* the sum of squares in FP64 and the scale rounded once to FP32: the correctly
         * rounded scale whatever the summation order (each square of a BF16 value is exact in
         * FP64); one double a wave in the reduction area */
        double ss = 0.0;
#pragma unroll
        for (int it = 0; it < kXIters; ++it) {
            const uint32_t w4[4] = {xv[it].x, xv[it].y, xv[it].z, xv[it].w};
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const double lo = bf16_widen((uint16_t)(w4[q] & 0xFFFFu));
                const double hi = bf16_widen((uint16_t)(w4[q] >> 16));
                ss = fma(lo, lo, ss);
                ss = fma(hi, hi, ss);
            }
        }
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) ss += __shfl_xor(ss, o);
        double *dred = reinterpret_cast<double *>(red);
        if (lane == 0) dred[wave] = ss;
        __syncthreads();
        double total = 0.0;
        for (int w = 0; w < W; ++w) total += dred[w];
        const float rms = (float)(1.0 / sqrt(total / (double)K + (double)eps));
#pragma unroll
        for (int it = 0; it < kXIters; ++it) {
            uint32_t w4[4] = {xv[it].x, xv[it].y, xv[it].z, xv[it].w};
            const uint32_t n4[4] = {nv[it].x, nv[it].y, nv[it].z, nv[it].w};
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float lo = bf16_widen((uint16_t)(w4[q] & 0xFFFFu)) * rms *
                                 (norm_bias + bf16_widen((uint16_t)(n4[q] & 0xFFFFu)));
                const float hi = bf16_widen((uint16_t)(w4[q] >> 16)) * rms *
                                 (norm_bias + bf16_widen((uint16_t)(n4[q] >> 16)));
                /* v_cvt_pk_bf16_f32: round-to-nearest-even of both, packed (finite values:
                 * the same bits as bf16_rne) */
                const bf16x2_t packed = {(__bf16)lo, (__bf16)hi};
                w4[q] = __builtin_bit_cast(uint32_t, packed);
            }
            xv[it] = make_uint4(w4[0], w4[1], w4[2], w4[3]);
        }
        __syncthreads(); /* red is reused by the split-K reduction */
    }

    /* 3. stage the activation and the per-(group, kb) sums of the codes' x values */
#pragma unroll
    for (int it = 0; it < kXIters; ++it) {
        const int i = it * W * 64 + tid;
        if (i < xchunks) smem4[i] = xv[it];
        float s8 = chunk_sum8(xv[it]);
        /* chunk i = 16 g + 4 s + kb (16 consecutive chunks are one DPP row): add the four s
         * of one (g, kb), i.e. the lanes congruent mod 4 within the row, by two rotations */
        s8 += dpp_f32<kDppRowRor4>(s8);
        s8 += dpp_f32<kDppRowRor8>(s8);
        if (i < xchunks && ((i >> 2) & 3) == 0) xsum[(i >> 4) * 4 + (i & 3)] = s8;
    }
    __syncthreads();

    /* 4. dot products; a piece past the tile's groups has scale 0 (its loads read 0) and reads
     * the activation of the last group, so it adds exactly 0 without a branch */
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < NL; ++i) {
        if (ks + i * SK < P) { /* wave-uniform */
            const int g = min(2 * (ks + i * SK) + half, G - 1);
            /* one 16-byte chunk a lane: quad lane s reads chunk 4 s + kb of group g, and the
             * dot products take it from there over DPP */
            const uint4 xq = smem4[g * 16 + 4 * (lane & 3) + kb];
            acc = fmaf(piece_dot_dpp(buf[i], xq, -0.75f * xsum[4 * g + kb]), bf16_widen(sbits[i]),
                       acc);
        } else { /* keeps the pair's loads ahead of the branch, in issue order */
            asm volatile("" ::"v"(buf[i].x), "v"(sbits[i]));
        }
    }
    acc *= 32.0f; /* piece_dot_dpp returns its sum over 32 */

    /* 5. lanes r, r+8, ..., r+56 hold row r's partials; then the SK waves of a tile */
    acc += dpp_f32<kDppRowRor8>(acc);
    acc = lane_sum32(lane_sum16(acc));
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
        const float upv = dpp_f32<kDppRowShl4>(row_sum);
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

/* Split-K combine without fences. Each block of a tile stores its FP32 partials into mailbox
 * slots: one 64-bit atomic word holding the value in its low half and a written-flag of 1 in its
 * high half, so a reader that sees the flag sees that value (one atomic object; no ordering
 * between locations is needed). The block then counts its arrival on the tile's counter
 * (relaxed). The one that takes the last arrival waits on each slot's flag (it is set: the
 * writer stored it before counting, so it becomes visible; the wait is bounded all the same),
 * sums the slots in split order (independent of arrival order) and clears every slot and the
 * counter, so the next kernel, which the kernel boundary orders after these stores, finds them
 * empty. Slots are cleared when the scratch is allocated. Agent-scope release/acquire fences
 * would give the same guarantee through a write-back and an invalidation of the L2 caches, which
 * multiplied the time of these kernels several times. */
constexpr int kSlotWaitPolls = 1 << 16;

__device__ __forceinline__ void slot_put(uint64_t *slot, float v) {
    __hip_atomic_store(slot, (1ull << 32) | __float_as_uint(v), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ uint64_t slot_peek(const uint64_t *slot) {
    return __hip_atomic_load(const_cast<uint64_t *>(slot), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

/* Bounded waits that gave up since the host last read this word (per device; read and cleared
 * by w4a16_split_wait_status). A wait that gives up means a combine summed a slot that was never
 * written, so the call's output is wrong: the count turns that into an error the host can see. */
__device__ unsigned g_slot_wait_timeouts;

/* The value of a slot whose first read was `w`, waiting (at most `polls` polls) for its flag if
 * needed; clears it. A wait that gives up counts itself in g_slot_wait_timeouts and returns 0. */
__device__ __forceinline__ float slot_take(uint64_t *slot, uint64_t w, int polls = kSlotWaitPolls) {
    for (int n = 0; (w >> 32) == 0 && n < polls; ++n) {
        __builtin_amdgcn_s_sleep(1);
        w = slot_peek(slot);
    }
    if ((w >> 32) == 0) {
        __hip_atomic_fetch_add(&g_slot_wait_timeouts, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        w = 0;
    }
    __hip_atomic_store(slot, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return __uint_as_float((uint32_t)w);
}

/* One wave waiting on the slot at `slot` with the given poll bound (status path test). */
__global__ __launch_bounds__(64) void slot_wait_probe_kernel(uint64_t *slot, int polls, float *out) {
    const float v = slot_take(slot, slot_peek(slot), polls);
    if (threadIdx.x == 0) out[0] = v;
}

/* Counts one block's arrival (lane 0) and returns the count before it on every lane. */
__device__ __forceinline__ unsigned split_arrive(unsigned *counter, int lane) {
    unsigned prev = 0;
    if (lane == 0) prev = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return __shfl(prev, 0);
}

/* The end of an M = 1 GEMV tile: eight lanes (one DPP row of sixteen, in order) hold its eight
 * row sums, row r on the lane this call passes r. PAIR: row r < 4 is gate row r and row r + 4
 * the matching up row, and the lanes of r < 4 write BF16(silu(gate) x up); otherwise eight FP32
 * or BF16 rows, with the plan-F2 residual update when residual is given. */
template <bool PAIR, bool OUT_F32>
__device__ __forceinline__ void gemv_row_epilogue(float row_sum, int r, int tile, void *out,
                                                  uint16_t *residual, const uint16_t *sub) {
    if (PAIR) {
        /* row r < 4 is gate row r, r + 4 the matching up row, four lanes further in the same
         * row of sixteen lanes */
        const float upv = dpp_f32<kDppRowShl4>(row_sum);
        if (r < 4) {
            const float gate = bf16_widen(bf16_rne(row_sum));
            const float up = bf16_widen(bf16_rne(upv));
            reinterpret_cast<uint16_t *>(out)[tile * 4 + r] = silu_mul_bf16(gate, up);
        }
    } else if (OUT_F32) {
        reinterpret_cast<float *>(out)[tile * 8 + r] = row_sum;
    } else {
        const int row = tile * 8 + r;
        const uint16_t o = bf16_rne(row_sum);
        if (residual) {
            /* plan F2 epilogue: residual <- BF16(BF16(residual + sub) + out), the updates of
             * reference csrc/layer_dispatch.cu:193-209 (this row's inputs are read before
             * its output is written, so sub may alias out); with no sub the residual already
             * holds BF16(residual + sub) and only the second update is made */
            const uint16_t rsum =
                sub ? (uint16_t)(bf16_add2(residual[row], sub[row]) & 0xFFFFu) : residual[row];
            residual[row] = (uint16_t)(bf16_add2(rsum, o) & 0xFFFFu);
        }
        reinterpret_cast<uint16_t *>(out)[row] = o;
    }
}

/* GEMV with wave-local activation: as gemv_tiles_kernel, but each wave loads only the
 * activation of its own group pairs (512 bytes a pair, 8 bytes a lane, issued with its weight
 * loads) into a private LDS slice, and forms the per-(group, kb) sums with shuffles. No block
 * barrier stands between a wave's loads and its dot products, so a wave starts as soon as its
 * own data arrives. Suits a long K (the down projection), where staging the whole activation per
 * block costs a round trip before any compute can start.
 *
 * One 8-row tile is split over BS blocks of SK waves: global wave gw = part * SK + wave takes
 * the group pairs gw + i * SK * BS (i < NP). The SK waves of a block meet in LDS; with BS > 1 the
 * blocks of a tile store FP32 row partials with agent-scope stores, count on the tile's
 * agent-scope counter, and the last to arrive adds the BS partials in block order (independent
 * of arrival order), writes the row and resets the counter. */
template <bool PAIR, bool OUT_F32, int SK, int NP, int BS>
__global__ __launch_bounds__(SK * 64) void gemv_xwave_kernel(
    const uint16_t *__restrict__ x, const uint8_t *__restrict__ wt,
    const uint16_t *__restrict__ st, void *__restrict__ out, int N, int K, uint64_t *partial,
    unsigned *counters, uint16_t *residual, const uint16_t *sub) {
    extern __shared__ uint4 smem4[];
    const int G = K >> 7;
    const int P = (G + 1) >> 1;
    const int tile = blockIdx.x / BS;
    const int part = blockIdx.x % BS;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int gw = part * SK + wave;
    constexpr int kStride = SK * BS;
    const int half = lane >> 5;
    const int piece = lane & 31;
    const int kb = piece >> 3;
    const int r = piece & 7;
    float *red = reinterpret_cast<float *>(smem4);

    /* 1. this wave's scales, then its activation and weight piece pair by pair. Pair p holds
     * values [256 p, 256 p + 256) as 32 chunks of 8; a quad of lanes (same half and kb, lane & 3 = s)
     * loads the chunks c = 16 half + 4 s + kb, the 32 values that each piece (half, kb, r) of
     * the quad multiplies (the quads r < 4 and r >= 4 load the same chunks). */
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(x, (uint32_t)K * 2);
    const int xchunk = 16 * half + 4 * (lane & 3) + kb;
    const size_t tile_bytes = (size_t)G * 512;
    const __amdgpu_buffer_rsrc_t wr = make_rsrc(wt + (size_t)tile * tile_bytes, (uint32_t)tile_bytes);
    const __amdgpu_buffer_rsrc_t sr = make_rsrc(st + (size_t)tile * G * 8, (uint32_t)G * 16);
    uint4 xv[NP];
    uint4 buf[NP];
    uint16_t sbits[NP];
#pragma unroll
    for (int i = 0; i < NP; ++i) { /* g >= G (and so p >= P) is past the tile: zeros */
        const int g = 2 * (gw + i * kStride) + half;
        sbits[i] = buf_load_u16(sr, (uint32_t)(g * 16 + r * 2));
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < NP; ++i) { /* p >= P reads past K: zeros */
        const int g = 2 * (gw + i * kStride) + half;
        xv[i] = buf_load16(xr, (uint32_t)((gw + i * kStride) * 512 + xchunk * 16));
        buf[i] = buf_load16_stream(wr, (uint32_t)(g * 512 + piece * 16));
        __builtin_amdgcn_sched_barrier(0);
    }

    /* 2. per pair: the (half, kb) activation sum over the quad (two DPP adds), then the dot
     * products with the activation broadcast from the quad's lanes */
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < NP; ++i) {
        if (gw + i * kStride < P) { /* wave-uniform: every lane of the wave takes part */
            acc = fmaf(piece_dot_dpp(buf[i], xv[i], quad_offset(xv[i])), bf16_widen(sbits[i]), acc);
        } else { /* keeps the pair's loads ahead of the branch, in issue order */
            asm volatile("" ::"v"(buf[i].x), "v"(xv[i].x), "v"(sbits[i]));
        }
    }
    acc *= 32.0f; /* piece_dot_dpp returns its sum over 32 */

    /* 3. lanes r, r+8, ..., r+56 hold row r's partials; then the SK waves of the block */
    acc += dpp_f32<kDppRowRor8>(acc);
    acc = lane_sum32(lane_sum16(acc));
    if (lane < 8) red[wave * 8 + lane] = acc;
    __syncthreads();
    if (wave != 0 || lane >= 8) return;
    float row_sum = 0.0f;
#pragma unroll
    for (int w = 0; w < SK; ++w) row_sum += red[w * 8 + lane];

    /* 4. the BS blocks of the tile */
    if (BS > 1) {
        uint64_t *pp = partial + (size_t)tile * BS * 8;
        slot_put(pp + part * 8 + lane, row_sum);
        if (split_arrive(&counters[tile], lane) != BS - 1) return;
        uint64_t w[BS];
#pragma unroll
        for (int j = 0; j < BS; ++j) w[j] = slot_peek(pp + j * 8 + lane);
        row_sum = 0.0f;
#pragma unroll
        for (int j = 0; j < BS; ++j) row_sum += slot_take(pp + j * 8 + lane, w[j]);
        if (lane == 0)
            __hip_atomic_store(&counters[tile], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    gemv_row_epilogue<PAIR, OUT_F32>(row_sum, lane, tile, out, residual, sub);
}

size_t xwave_smem(int waves, int np) { return (void)np, (size_t)waves * 32; }
constexpr int kXwaveWaves = 16;


/* ------------------------------------------------------------------------------------------
 * MFMA form (M = 1..16 activation rows): v_mfma_f32_16x16x32_bf16 with the activation as the A
 * operand (lane l holds row l % 16, k-block l / 16) and sixteen weight rows as B (lane l holds
 * weight row l % 16 of a tile pair, the same k-block): lanes 0-7 carry tile 2p, lanes 8-15 tile
 * 2p + 1, and lane l's 16-byte piece (kb = l / 16, r = l % 8) supplies one MFMA per dword, so a
 * group of one tile pair is four MFMAs and the matrix core, not the VALU, does the FMAs. Only
 * the rows < M of A are non-zero. B holds v = 0.75 + code/32 (see the unpack above) and the group
 * result is 32 * D - 24 * X with X the group's activation sum. Each wave owns one tile pair over
 * the block's K range (GS groups, all loads issued up front); the four waves of a block share the
 * staged activation of that range. When K is split over S blocks, every block writes its FP32
 * partial and the last one to arrive on a tile pair (device-scope counter) sums the S partials in
 * split order - the result does not depend on arrival order - and resets the counter.
 * ---------------------------------------------------------------------------------------- */
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

/* groups per wave (16-byte loads in flight per lane). 8 keeps the kernel near 80 VGPRs, so six
 * waves a SIMD stay resident; medians of interleaved graph runs of the C1 FFN at M = 2/4/8/16:
 * 20.0/22.2/23.9/30.1 us at 8 against 21.3/27.4/30.3/38.6 at 20 (4: 23.0/25.4/28.2/33.9). */
constexpr int kGMax = 8;
constexpr int kMfmaWaves = 4;   /* tile pairs per block */
enum { kOutBf16 = 0, kOutPairSilu = 1, kOutF32 = 2 };

__device__ __forceinline__ bf16x8_t unpack8(uint32_t word) {
    return __builtin_bit_cast(bf16x8_t, code_pairs(word));
}


/* M = 1 or 2 rows on the matrix cores. The block and wave decomposition of gemv_xwave_kernel (one
 * 8-row tile a block, wave w taking the group pairs w + SK i), but a pair's products go to
 * v_mfma_f32_16x16x32_bf16 with a block-diagonal operand: lane l loads piece (kb = l / 16,
 * row r = l % 8) of group 2p + a, a = (l / 8) % 2, which is B column n = 8a + r for k block kb,
 * and A row 8a + 4t carries activation row t (t < M) of group 2p + a, every other row zero, so
 * D[8a + 4t][8a + r] is row r's dot product with activation row t over group 2p + a (the
 * off-diagonal quadrants mix the groups and are not read). Four MFMAs a pair, one per piece
 * dword, take B = 0.75 + code/32 from the unpack; a fifth, issued first, takes the constant
 * -0.75 as B and an A whose row 8a + 4t + s holds slice s (the 32 values of k block s of every
 * kb) of activation row t over group 2p + a, which adds -0.75 times each slice's sum to those
 * rows of D. Rows 8a + 4t .. 8a + 4t + 3 of D sit in the four accumulator registers of lane
 * 16 (2a + t) + n, so the group's result is the sum of that lane's four registers, and one FMA
 * with the scale folds it in: the VALU does only the unpack and that sum (33 instructions a pair
 * against 54 on the v_dot2 path, whatever M).
 *
 * Operands. A wave's activation for pair p (M x 512 bytes, in k order) goes straight into a
 * private 1 KiB LDS slice by one direct load (lanes 0-31 row 0; lanes 32-63 row 1 when M = 2,
 * otherwise past the buffer, so that half holds zeros), and at M = 2 a 256-byte zero area after
 * each slice serves the rows that carry nothing: every A operand is one ds_read_b128 whose address is fixed per
 * lane (the pair and the k block in the instruction's offset). No block barrier stands before
 * the MFMAs; the SK waves meet in LDS once at the end. */
template <bool PAIR, bool OUT_F32, int SK, int NP, int M>
__global__ __launch_bounds__(SK * 64) void gemv_mfma1_kernel(
    const uint16_t *__restrict__ x, const uint8_t *__restrict__ wt,
    const uint16_t *__restrict__ st, void *__restrict__ out, int N, int K, uint16_t *residual,
    const uint16_t *sub) {
    static_assert(M == 1 || M == 2, "one or two activation rows");
    /* a pair's slice in 16-byte chunks: 1 KiB of rows, then at M = 2 256 bytes of zeros; its
     * zero chunks: M = 1 the second half (the direct load's lanes past the buffer), M = 2 the
     * area after it */
    constexpr int STRIDE = M == 2 ? 80 : 64;
    constexpr int ZERO = M == 2 ? 64 : 32;
    extern __shared__ uint4 smem4[];
    const int G = K >> 7;
    const int P = (G + 1) >> 1;
    const int tile = blockIdx.x;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n = lane & 15, kb = lane >> 4;
    const int a = n >> 3, r = n & 7;
    uint4 *slice = smem4 + wave * NP * STRIDE;
    float *red = reinterpret_cast<float *>(smem4 + SK * NP * STRIDE);

    /* 1. the zero areas, the scales, then pair by pair the weight piece and the pair's activation
     * into its slice (a pair past K reads zeros everywhere); each pair waits below for its own
     * slice only, so its MFMAs start while the later pairs' loads are in flight */
    if (M == 2) {
#pragma unroll
        for (int i = 0; i < NP; ++i) reinterpret_cast<uint32_t *>(slice + i * STRIDE + 64)[lane] = 0u;
    }
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(x, (uint32_t)K * 2 * M);
    const size_t tile_bytes = (size_t)G * 512;
    const __amdgpu_buffer_rsrc_t wr = make_rsrc(wt + (size_t)tile * tile_bytes, (uint32_t)tile_bytes);
    const __amdgpu_buffer_rsrc_t sr = make_rsrc(st + (size_t)tile * G * 8, (uint32_t)G * 16);
    uint4 buf[NP];
    uint16_t sbits[NP];
#pragma unroll
    for (int i = 0; i < NP; ++i) {
        const int g = 2 * (wave + i * SK) + a;
        sbits[i] = buf_load_u16(sr, (uint32_t)(g * 16 + r * 2));
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < NP; ++i) {
        {
            const int g = 2 * (wave + i * SK) + a;
            buf[i] = buf_load16_stream(wr, (uint32_t)(g * 512 + (kb * 8 + r) * 16));
        }
        __builtin_amdgcn_sched_barrier(0);
        {
            const int c = (wave + i * SK) * 512 + (lane & 31) * 16;
            const uint32_t off = c >= K * 2 ? kOob
                                 : lane < 32 ? (uint32_t)c
                                 : M == 2    ? (uint32_t)(K * 2 + c)
                                             : kOob;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                xr, (__attribute__((address_space(3))) void *)(slice + i * STRIDE), 16, off, 0, 0, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
    }

    /* 2. A chunks: 32 t + 16 a + 4 s + kb of a slice is row t's k block kb of slice s of group
     * 2p + a; ZERO + kb reads zeros. cmain: row 8a + 4t (plus 4 s a dword); coff: row
     * 8a + 4t + s */
    const int ta = (n >> 2) & 1;
    const int cmain = (n & 3) == 0 && ta < M ? 32 * ta + 16 * a + kb : ZERO + kb;
    const int coff = ta < M ? 32 * ta + 16 * a + 4 * (n & 3) + kb : ZERO + kb;
    uint4 offs = make_uint4(0xBF40BF40u, 0xBF40BF40u, 0xBF40BF40u, 0xBF40BF40u); /* BF16 -0.75 */
    asm volatile("" : "+v"(offs.x), "+v"(offs.y), "+v"(offs.z), "+v"(offs.w)); /* kept in place */
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < NP; ++i) {
        if (wave + i * SK < P) { /* wave-uniform */
            /* the slice of pair i has landed: 2 (NP - 1 - i) loads were issued after it */
            wait_vm<2 * (NP - 1)>(i);
            const uint4 *sl = slice + i * STRIDE;
            f32x4_t d = {0.0f, 0.0f, 0.0f, 0.0f};
            d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, sl[coff]),
                                                        __builtin_bit_cast(bf16x8_t, offs), d, 0, 0, 0);
            const uint32_t words[4] = {buf[i].x, buf[i].y, buf[i].z, buf[i].w};
#pragma unroll
            for (int t = 0; t < 4; ++t)
                d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                    __builtin_bit_cast(bf16x8_t, sl[cmain + 4 * t]), unpack8(words[t]), d, 0, 0, 0);
            acc = fmaf((d[0] + d[1]) + (d[2] + d[3]), bf16_widen(sbits[i]), acc);
        } else {
            /* a use on this path too, so the compiler keeps the pair's loads ahead of the branch
             * (sunk into it, they would no longer sit where the waits above count them) */
            asm volatile("" ::"v"(buf[i].x), "v"(sbits[i]));
        }
    }

    /* 3. lane 16 t + r holds row r's sum for activation row t over group 2p, lane 40 + 16 t + r
     * over group 2p + 1: after the lane swap, lane 8 + 16 t + r holds the latter, which a row
     * rotation by 8 brings to lane 16 t + r */
    {
        float t = acc, u = acc;
        asm volatile("s_nop 1\n v_permlane32_swap_b32 %0, %1\n s_nop 1" : "+v"(t), "+v"(u));
        acc += dpp_f32<kDppRowRor8>(u);
    }
    const int trow = lane >> 4;
    if (r == n && trow < M) red[(wave * M + trow) * 8 + r] = acc;
    __syncthreads();
    if (wave != 0 || lane >= 8 * M) return;
    /* lane 8 t + r finishes row r of activation row t (rows r and r + 4 in one DPP row) */
    const int t = lane >> 3, rr = lane & 7;
    float row_sum = 0.0f;
#pragma unroll
    for (int w = 0; w < SK; ++w) row_sum += red[(w * M + t) * 8 + rr];
    const size_t ocols = PAIR ? (size_t)N / 2 : (size_t)N;
    void *out_t = OUT_F32 ? (void *)(reinterpret_cast<float *>(out) + t * ocols)
                          : (void *)(reinterpret_cast<uint16_t *>(out) + t * ocols);
    gemv_row_epilogue<PAIR, OUT_F32>(32.0f * row_sum, rr, tile, out_t,
                                     residual ? residual + t * ocols : nullptr,
                                     sub ? sub + t * ocols : nullptr);
}

size_t mfma1_smem(int waves, int np, int m) {
    return (size_t)waves * np * (m == 2 ? 1280 : 1024) + (size_t)waves * 64;
}

template <int OUT, int XPRE, int MI>
__global__ __launch_bounds__(kMfmaWaves * 64) void mfma_gemm_kernel(
    const uint16_t *__restrict__ x, int M, const uint8_t *__restrict__ wt,
    const uint16_t *__restrict__ st, void *__restrict__ out, int N, int K, int S, int GS,
    uint64_t *__restrict__ partial, unsigned *__restrict__ counters, uint16_t *residual, int cm) {
    extern __shared__ uint4 smem4[];
    const int G = K >> 7;
    const int tiles = N >> 3;
    const int NT = (tiles + 1) >> 1;
    const int ks = blockIdx.x % S;
    const int g0 = ks * GS;
    const int ng = min(GS, G - g0);
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int tp = (int)(blockIdx.x / S) * kMfmaWaves + wave;
    const int n = lane & 15;
    const int q = lane >> 4;
    const int tile = 2 * tp + (n >> 3);
    const int r = n & 7;

    /* 1. the activation chunks of this block's K range (8 BF16 each; row m, chunk c) */
    const int cpr = ng * 16;            /* chunks per activation row */
    const int chunks = M * cpr;
    const uint32_t ndiv = div_magic(ng); /* row of chunk i: (i / 16) / ng, ng <= 8 */
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(x, (uint32_t)M * K * 2);
    uint4 xv[XPRE];
#pragma unroll
    for (int it = 0; it < XPRE; ++it) {
        const int i = it * kMfmaWaves * 64 + tid;
        const int m = div_small(i >> 4, ndiv), c = i - m * cpr;
        xv[it] = buf_load16(xr, i < chunks ? (uint32_t)((m * K + g0 * 128 + c * 8) * 2) : kOob);
    }

    /* 2. every weight piece and scale of this wave's tile pair and K range */
    const __amdgpu_buffer_rsrc_t wr = make_rsrc(wt, (uint32_t)((size_t)N * K / 2));
    const __amdgpu_buffer_rsrc_t sr = make_rsrc(st, (uint32_t)((size_t)N * G * 2));
    const bool tile_ok = tp < NT && tile < tiles;
    uint4 buf[kGMax];
    uint16_t sbits[kGMax];
#pragma unroll
    for (int i = 0; i < kGMax; ++i) { /* the scales first: loads return in issue order */
        const bool ok = tile_ok && i < ng;
        const uint32_t unit = (uint32_t)(tile * G + g0 + i);
        sbits[i] = buf_load_u16(sr, ok ? (unit * 8 + r) * 2 : kOob);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < kGMax; ++i) {
        const bool ok = tile_ok && i < ng;
        const uint32_t unit = (uint32_t)(tile * G + g0 + i);
        buf[i] = buf_load16_stream(wr, ok ? (unit * 32 + q * 8 + r) * 16 : kOob);
        __builtin_amdgcn_sched_barrier(0);
    }

    /* 3. stage the activation (row-major [M][ng*128] BF16, then one zero row that the lanes of
     * rows >= M read as their A operand) and the group sums X[m][g] */
    uint4 *zero_row = smem4 + chunks;
    for (int i = tid; i < cpr; i += kMfmaWaves * 64) zero_row[i] = make_uint4(0, 0, 0, 0);
    float *xsum = reinterpret_cast<float *>(smem4 + chunks + cpr);
    auto stage = [&](int i, uint4 v) {
        if (i < chunks) smem4[i] = v;
        float s8 = chunk_sum8(v);
        /* 16 consecutive chunks make one group of one row */
        s8 += dpp_f32<kDppQuadSwap1>(s8);
        s8 += dpp_f32<kDppQuadSwap2>(s8);
        s8 += dpp_f32<kDppRowRor4>(s8);
        s8 += dpp_f32<kDppRowRor8>(s8);
        if (i < chunks && (i & 15) == 0) xsum[i >> 4] = s8;
    };
#pragma unroll
    for (int it = 0; it < XPRE; ++it) stage(it * kMfmaWaves * 64 + tid, xv[it]);
    for (int i0 = XPRE * kMfmaWaves * 64; i0 < chunks; i0 += kMfmaWaves * 64) {
        const int i = i0 + tid;
        const int m = div_small(i >> 4, ndiv), c = i - m * cpr;
        stage(i, buf_load16(xr, i < chunks ? (uint32_t)((m * K + g0 * 128 + c * 8) * 2) : kOob));
    }
    __syncthreads();
    if (tp >= NT) return;

    /* 4. four MFMAs per group, then scale and offset correction into acc[i] (row 4q + i; only
     * the MI first D registers can hold rows < M when M <= 4). Two groups are processed
     * together so their MFMA chains interleave. */
    const uint4 *arow_base = smem4 + (n < M ? n * cpr : chunks) + q;
    f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
    auto group_mfma = [&](int gl) {
        const uint32_t words[4] = {buf[gl].x, buf[gl].y, buf[gl].z, buf[gl].w};
        const uint4 *xa = arow_base + gl * 16;
        f32x4_t d = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int s = 0; s < 4; ++s)
            d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, xa[4 * s]),
                                                        unpack8(words[s]), d, 0, 0, 0);
        return d;
    };
    auto group_fold = [&](int gl, const f32x4_t &d) {
        const float sc = bf16_widen(sbits[gl]);
#pragma unroll
        for (int i = 0; i < MI; ++i) {
            const int m = min(4 * q + i, M - 1);
            acc[i] = fmaf(sc, fmaf(32.0f, d[i], -24.0f * xsum[m * ng + gl]), acc[i]);
        }
    };
#pragma unroll
    for (int gl = 0; gl < kGMax; gl += 2) {
        if (gl + 1 < ng) { /* block-uniform */
            const f32x4_t d0 = group_mfma(gl);
            const f32x4_t d1 = group_mfma(gl + 1);
            group_fold(gl, d0);
            group_fold(gl + 1, d1);
        } else if (gl < ng) {
            group_fold(gl, group_mfma(gl));
        }
    }

    /* 5. split-K combine: publish, count, and let the last arrival sum in split order (mailbox
     * slots, see slot_put). Only the rows < M are published and read. */
    if (S > 1) {
        uint64_t *mine = partial + ((size_t)ks * NT + tp) * 16 * M;
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if (4 * q + i < M) slot_put(mine + (4 * q + i) * 16 + n, acc[i]);
        if (split_arrive(&counters[tp], lane) != (unsigned)(S - 1)) return;
        /* the S partials are read in batches of 8 with every load issued before any is summed
         * (each is a round trip to the coherence point), then summed in split order */
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i] = 0.0f;
        for (int k0 = 0; k0 < S; k0 += 8) {
            uint64_t v[8][MI];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                uint64_t *src = partial + ((size_t)(k0 + j) * NT + tp) * 16 * M;
#pragma unroll
                for (int i = 0; i < MI; ++i)
                    v[j][i] = (k0 + j < S && 4 * q + i < M) ? slot_peek(src + (4 * q + i) * 16 + n) : 0ull;
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                uint64_t *src = partial + ((size_t)(k0 + j) * NT + tp) * 16 * M;
#pragma unroll
                for (int i = 0; i < MI; ++i)
                    if (k0 + j < S && 4 * q + i < M) acc[i] += slot_take(src + (4 * q + i) * 16 + n, v[j][i]);
            }
        }
        if (lane == 0)
            __hip_atomic_store(&counters[tp], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }

    /* 6. epilogue */
    if (OUT == kOutPairSilu) {
        const int inter = N >> 1;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float upv = __shfl_down(acc[i], 4);
            const int m = 4 * q + i;
            if (r < 4 && m < M && tile < tiles) {
                const float gate = bf16_widen(bf16_rne(acc[i]));
                const float up = bf16_widen(bf16_rne(upv));
                reinterpret_cast<uint16_t *>(out)[act_index(m, tile * 4 + r, M, inter, cm)] =
                    silu_mul_bf16(gate, up);
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int m = 4 * q + i;
            if (m < M && tile < tiles) {
                const size_t o = (size_t)m * N + tile * 8 + r;
                if (OUT == kOutF32) {
                    reinterpret_cast<float *>(out)[o] = acc[i];
                } else {
                    const uint16_t ob = bf16_rne(acc[i]);
                    /* plan F2: the residual, already BF16(residual + sublayer), gains the output */
                    if (residual) residual[o] = (uint16_t)(bf16_add2(residual[o], ob) & 0xFFFFu);
                    reinterpret_cast<uint16_t *>(out)[o] = ob;
                }
            }
        }
    }
}

/* ------------------------------------------------------------------------------------------
 * Few rows (2 <= M <= 8) on the GEMV's block structure: TB tiles a block, SK waves a tile, NL
 * group pairs a wave, the activation staged in LDS once per block, no split-K across blocks.
 * The inner product runs on v_mfma_f32_16x16x32_bf16 with a block-diagonal operand: lane l
 * loads the 16-byte piece (row r = l & 7, kb = q = l >> 4) of group 2p + a, a = (l >> 3) & 1, so
 * B column n = 8a + r is tile row r of one group of the pair and the 32-wide k block of MFMA t
 * (the piece's dword t) is k = 32 t + 8 kb + j in both groups. A row 8a + m holds activation row
 * m of group 2p + a at the same k, so D[8a + m][8a + r] is row r's group sum for row m (the other
 * quadrants mix the groups and are not used). B holds 0.75 + code/32; four more MFMAs against a
 * constant -0.75 operand take the offset out inside the accumulator, so the VALU only unpacks
 * codes and applies the scale. Lane l's D rows are 4q + i (a = q >> 1, m = 4 (q & 1) + i);
 * lanes l and l ^ 40 hold the two groups of a pair for the same (r, m).
 *
 * The activation goes from memory straight into LDS (buffer_load ... lds, 16 bytes a lane),
 * every load issued before the weight loads, in the order [pair][row m][a][16 chunks] with
 * chunk c in slot c ^ (2 m + a): one load instruction reads four 256-byte runs (whole cache
 * lines; the order [pair][chunk][row][a] read 64-byte half lines from M = 5), and the 16 lanes
 * of one ds_read_b128 pass (one k block, rows 8a + m) hit 16 distinct 16-byte bank slots.
 * Chunks of a group past K are loaded as zeros.
 * ---------------------------------------------------------------------------------------- */
template <bool PAIR, bool OUT_F32, int TB, int SK, int NL, int MI>
__global__ __launch_bounds__(TB * SK * 64) void gemv_rows_kernel(
    const uint16_t *__restrict__ x, int M, const uint8_t *__restrict__ wt,
    const uint16_t *__restrict__ st, void *__restrict__ out, int N, int K, uint16_t *residual,
    int cm) {
    constexpr int W = TB * SK;
    extern __shared__ uint4 smem4[];
    const int G = K >> 7;
    const int P = (G + 1) >> 1;
    const int tiles = N >> 3;
    const int cpr = K >> 3;             /* 16-byte chunks a row in memory */
    const int nlds = P * 32 * M;        /* staged chunks (both groups of every pair) */
    const int nins = (nlds + 63) >> 6;  /* 1 KiB load instructions */
    float *red = reinterpret_cast<float *>(smem4 + nins * 64); /* [W][8 rows][8 tile rows] */

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int tile = blockIdx.x * TB + wave / SK;
    const int ks = wave % SK;
    const int q = lane >> 4;
    const int a = (lane >> 3) & 1;
    const int r = lane & 7;

    /* 1. the activation, straight into LDS: instruction j of the block (wave j % W) fills
     * staged chunks 64 j .. 64 j + 63 */
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(x, (uint32_t)M * cpr * 16);
    int xloads = 0;
    /* staged chunk pos holds chunk c of row m of group 2 p + a, pos = ((p M + m) 2 + a) 16 +
     * (c ^ (2 m + a)): one instruction reads four (row, group) runs of 256 contiguous bytes */
    const uint32_t mdiv = div_magic(M); /* t2 < P * M <= 640 */
    auto staged = [&](int pos, int &m, int &g, int &c) {
        const int seg = pos >> 4, aa = seg & 1, t2 = seg >> 1;
        const int pq = div_small(t2, mdiv);
        m = t2 - pq * M;
        g = 2 * pq + aa;
        c = (pos & 15) ^ ((2 * m + aa) & 15);
    };
    for (int j = wave; j < nins; j += W) {
        const int pos = j * 64 + lane;
        int m, g, c;
        staged(pos, m, g, c);
        const bool ok = pos < nlds && g < G;
        const uint32_t off = ok ? (uint32_t)((m * cpr + g * 16 + c) * 16) : kOob;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            xr, (__attribute__((address_space(3))) void *)(smem4 + j * 64), 16, off, 0, 0, 0);
        ++xloads;
    }
    /* 2. every weight piece and scale of this wave */
    const bool tile_ok = tile < tiles;
    const size_t tile_bytes = (size_t)G * 512;
    const __amdgpu_buffer_rsrc_t wr =
        make_rsrc(wt + (size_t)(tile_ok ? tile : 0) * tile_bytes, tile_ok ? (uint32_t)tile_bytes : 0);
    const __amdgpu_buffer_rsrc_t sr =
        make_rsrc(st + (size_t)(tile_ok ? tile : 0) * G * 8, tile_ok ? (uint32_t)G * 16 : 0);
    uint4 buf[NL];
    uint16_t sbits[NL];
#pragma unroll
    for (int i = 0; i < NL; ++i) {
        const int p = ks + i * SK;
        const int g = 2 * p + a;
        const bool ok = p < P && g < G;
        buf[i] = buf_load16_stream(wr, ok ? (uint32_t)(g * 512 + (q * 8 + r) * 16) : kOob);
        sbits[i] = buf_load_u16(sr, ok ? (uint32_t)(g * 16 + r * 2) : kOob);
    }

    /* 3. wait for this wave's activation loads only (issued first; memory ops complete in
     * order of the counter), then for every wave's */
    (void)xloads;
    __builtin_amdgcn_s_waitcnt(kVmcntWeights<NL>);
    __syncthreads();

    /* 4. eight MFMAs a pair. A piece past the tile's groups has scale 0 (its loads read 0) and
     * its staged activation is zero, so it adds exactly 0 without a branch; lanes of A rows
     * m >= M read row M - 1 (their D rows are not used). */
    const int arow = min(r, M - 1);
    const uint4 *abase = smem4 + (arow * 2 + a) * 16;
    const int aswz = (2 * arow + a) & 15;
    const uint4 offs = make_uint4(0xBF40BF40u, 0xBF40BF40u, 0xBF40BF40u, 0xBF40BF40u);
    f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int i = 0; i < NL; ++i) {
        const int p = ks + i * SK;
        if (p < P) { /* wave-uniform */
            const uint4 *xa = abase + p * 32 * M;
            const uint32_t words[4] = {buf[i].x, buf[i].y, buf[i].z, buf[i].w};
            f32x4_t d = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const bf16x8_t av = __builtin_bit_cast(bf16x8_t, xa[(4 * t + q) ^ aswz]);
                d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, unpack8(words[t]), d, 0, 0, 0);
                d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, __builtin_bit_cast(bf16x8_t, offs),
                                                            d, 0, 0, 0);
            }
            const float sc = bf16_widen(sbits[i]);
#pragma unroll
            for (int j = 0; j < MI; ++j) acc[j] = fmaf(sc, d[j], acc[j]);
        }
    }

    /* 5. the pair's two groups (lanes l, l ^ 40), then the SK waves of a tile in LDS; the
     * code step 1/32 is applied once here (a power of two: exact) */
#pragma unroll
    for (int j = 0; j < MI; ++j) acc[j] = 32.0f * (acc[j] + __shfl_xor(acc[j], 40));
    if ((lane & 40) == 0) {
#pragma unroll
        for (int j = 0; j < MI; ++j) red[wave * 64 + (4 * q + j) * 8 + r] = acc[j];
    }
    __syncthreads();
    if (ks != 0 || !tile_ok) return;
    const int m = lane >> 3;
    float row_sum = 0.0f;
#pragma unroll
    for (int w = 0; w < SK; ++w) row_sum += red[(wave + w) * 64 + lane];
    if (PAIR) {
        /* lane r < 4 of row m has gate row r, lane r + 4 the matching up row */
        const float upv = __shfl_down(row_sum, 4);
        if (r < 4 && m < M) {
            const float gate = bf16_widen(bf16_rne(row_sum));
            const float up = bf16_widen(bf16_rne(upv));
            reinterpret_cast<uint16_t *>(out)[act_index(m, tile * 4 + r, M, N >> 1, cm)] =
                silu_mul_bf16(gate, up);
        }
    } else if (m < M) {
        const size_t o = (size_t)m * N + tile * 8 + r;
        if (OUT_F32) {
            reinterpret_cast<float *>(out)[o] = row_sum;
        } else {
            const uint16_t ob = bf16_rne(row_sum);
            /* plan F2: the residual, already BF16(residual + sublayer), gains the output */
            if (residual) residual[o] = (uint16_t)(bf16_add2(residual[o], ob) & 0xFFFFu);
            reinterpret_cast<uint16_t *>(out)[o] = ob;
        }
    }
}

/* Up to 16 rows (9 <= M <= 16), short K: as gemv_rows_kernel, but a wave owns a tile pair and a
 * load covers one group of both tiles (lane l: piece (row l & 7, kb = l >> 4) of tile
 * 2 tp + ((l >> 3) & 1)), so all sixteen B columns share the k range and all sixteen A rows are
 * activation rows. A block holds blockDim / 64 waves: TP tile pairs of SK waves (both runtime),
 * NL groups a wave (group ks + i SK). The rows are staged in the order [group][row][16 chunks],
 * chunk c of row m in slot c ^ (m & 15): one staging instruction then reads four rows' 256
 * contiguous bytes each (whole cache lines; the order [group][chunk][row] read 16 rows x 64
 * bytes, half lines, and measured C3 M = 16 / 12 20.1 / 19.1 us against 19.4 / 18.6), and the 16
 * lanes of one ds_read_b128 pass (rows n, one chunk) hit 16 distinct 16-byte bank slots. */
template <bool PAIR, bool OUT_F32, int NL>
__global__ __launch_bounds__(1024) void gemv_rows16_kernel(
    const uint16_t *__restrict__ x, int M, const uint8_t *__restrict__ wt,
    const uint16_t *__restrict__ st, void *__restrict__ out, int N, int K, int TP, int SK, int cm) {
    const int W = TP * SK;
    extern __shared__ uint4 smem4[];
    const int G = K >> 7;
    const int tiles = N >> 3;
    const int cpr = K >> 3;
    const int nlds = G * 16 * M;
    const int nins = (nlds + 63) >> 6;
    f32x4_t *red = reinterpret_cast<f32x4_t *>(smem4 + nins * 64); /* [W][64 lanes] */

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int tp = blockIdx.x * TP + wave / SK;
    const int ks = wave % SK;
    const int q = lane >> 4;
    const int n = lane & 15;
    const int r = n & 7;
    const int tile = 2 * tp + (n >> 3);

    /* 1. the activation, straight into LDS */
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(x, (uint32_t)M * cpr * 16);
    const uint32_t mdiv = div_magic(M); /* pos / 16 < G * M <= 640 within the LDS limit */
    for (int j = wave; j < nins; j += W) {
        const int pos = j * 64 + lane;
        const int g = div_small(pos >> 4, mdiv);
        const int m = (pos >> 4) - g * M;
        const int c = (pos & 15) ^ (m & 15);
        const uint32_t off = pos < nlds ? (uint32_t)((m * cpr + g * 16 + c) * 16) : kOob;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            xr, (__attribute__((address_space(3))) void *)(smem4 + j * 64), 16, off, 0, 0, 0);
    }

    /* The staged rows land before any weight load is issued. Issued behind the weight loads of
     * the block's other waves, the staging loads (L2 hits) waited for their HBM misses: the
     * barrier released at 4 us of an 8.5 us kernel at M = 16 (block stamps), and staging first
     * takes C3 M = 9 / 12 / 16 from 17.49 / 18.08 / 18.83 to 16.66 / 17.28 / 18.00 us. */
    __builtin_amdgcn_s_waitcnt(vm_enc(0));
    __syncthreads();
    /* 2. every weight piece and scale of this wave (a tile past N reads zeros) */
    const bool tile_ok = tile < tiles;
    const __amdgpu_buffer_rsrc_t wr = make_rsrc(wt, (uint32_t)((size_t)N * K / 2));
    const __amdgpu_buffer_rsrc_t sr = make_rsrc(st, (uint32_t)((size_t)N * G * 2));
    uint4 buf[NL];
    uint16_t sbits[NL];
#pragma unroll
    for (int i = 0; i < NL; ++i) { /* the scales first: loads return in issue order */
        const int g = ks + i * SK;
        const bool ok = tile_ok && g < G;
        const uint32_t unit = (uint32_t)(tile * G + g);
        sbits[i] = buf_load_u16(sr, ok ? unit * 16 + (uint32_t)r * 2 : kOob);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < NL; ++i) {
        const int g = ks + i * SK;
        const bool ok = tile_ok && g < G;
        const uint32_t unit = (uint32_t)(tile * G + g);
        buf[i] = buf_load16_stream(wr, ok ? unit * 512 + (uint32_t)(q * 8 + r) * 16 : kOob);
        __builtin_amdgcn_sched_barrier(0);
    }

    /* 3. eight MFMAs a group (the offset ones as in gemv_rows_kernel) */
    const int arow = min(n, M - 1);
    const uint4 *abase = smem4 + arow * 16;
    const uint4 offs = make_uint4(0xBF40BF40u, 0xBF40BF40u, 0xBF40BF40u, 0xBF40BF40u);
    f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int i = 0; i < NL; ++i) {
        const int g = ks + i * SK;
        if (g < G) { /* wave-uniform */
            const uint4 *xa = abase + g * 16 * M;
            const uint32_t words[4] = {buf[i].x, buf[i].y, buf[i].z, buf[i].w};
            f32x4_t d = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const bf16x8_t av = __builtin_bit_cast(bf16x8_t, xa[(4 * t + q) ^ (arow & 15)]);
                d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, unpack8(words[t]), d, 0, 0, 0);
                d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, __builtin_bit_cast(bf16x8_t, offs),
                                                            d, 0, 0, 0);
            }
            const float sc = bf16_widen(sbits[i]);
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[j] = fmaf(sc, d[j], acc[j]);
        } else { /* keeps the pair's loads ahead of the branch, in issue order */
            asm volatile("" ::"v"(buf[i].x), "v"(sbits[i]));
        }
    }

    /* 4. the SK waves of a tile pair in LDS; lane (n, q) then holds rows 4 q + j of column n */
    red[wave * 64 + lane] = acc;
    __syncthreads();
    if (ks != 0) return;
    f32x4_t sum = red[wave * 64 + lane];
#pragma unroll
    for (int w = 1; w < SK; ++w) {
        const f32x4_t v = red[(wave + w) * 64 + lane];
#pragma unroll
        for (int j = 0; j < 4; ++j) sum[j] += v[j];
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float row_sum = 32.0f * sum[j];
        const int m = 4 * q + j;
        if (PAIR) {
            /* column r < 4 of a tile has gate row r, column r + 4 the matching up row */
            const float upv = __shfl_down(row_sum, 4);
            if (r < 4 && m < M && tile_ok) {
                const float gate = bf16_widen(bf16_rne(row_sum));
                const float up = bf16_widen(bf16_rne(upv));
                reinterpret_cast<uint16_t *>(out)[act_index(m, tile * 4 + r, M, N >> 1, cm)] =
                    silu_mul_bf16(gate, up);
            }
        } else if (m < M && tile_ok) {
            const size_t o = (size_t)m * N + tile * 8 + r;
            if (OUT_F32)
                reinterpret_cast<float *>(out)[o] = row_sum;
            else
                reinterpret_cast<uint16_t *>(out)[o] = bf16_rne(row_sum);
        }
    }
}

/* Up to 16 rows, long K, no PAIR: one tile pair a block of 16 waves, wave ks taking groups
 * ks + 16 i, and every lane loading its own MFMA A operand (row n, the 8 values of k block q
 * of each 32-wide slice) straight from memory into registers instead of staging the rows in
 * LDS. The A bytes of a block are M K 2 (from L2: every block reads the same rows), against
 * 16 K / 2 bytes of weight, but nothing is shared across the waves of a block, so no LDS pass
 * or block barrier stands before the MFMAs and no K split crosses blocks: the 16 waves meet
 * in LDS once, at the end. Suits the down projection (N small, K long), where the LDS-staged
 * rows no longer fit and splitting K across blocks costs a combine through the coherence
 * point. The weight loads of every group are issued first, then the A loads, kept D groups
 * ahead of the MFMAs. Lanes of A rows >= M load zeros (no memory traffic).
 *
 * With CM the activation is chunk-major ([K / 8 chunks][M rows][8 values], written so by the
 * gate/up kernels inside the FFN entry points): the A operands of one MFMA are then 64 M
 * contiguous bytes, M / 2 whole cache lines, where the row-major rows give 16 half lines. The
 * A stream is what bounds this kernel (down at M = 16 without its A loads: 6.0 us against
 * 13.1), and the chunk-major order takes it from 13.1 to 8.6-8.7 us.
 *
 * More than 16 row-major rows (gemm_int4_bf16 beyond M = 16): blockIdx.y takes rows
 * 16 y .. 16 y + 15, so the slices run in one launch and their blocks read each weight tile at
 * about the same time (the repeats are served by the caches). */
template <bool OUT_F32, int NL, int D, bool CM>
__global__ __launch_bounds__(1024) void gemv_rows16x_kernel(
    const uint16_t *__restrict__ x, int M, const uint8_t *__restrict__ wt,
    const uint16_t *__restrict__ st, void *__restrict__ out, int N, int K,
    uint16_t *residual) {
    if (!CM && blockIdx.y > 0) {
        const int m0 = (int)blockIdx.y * 16;
        x += (size_t)m0 * K;
        out = static_cast<char *>(out) + (size_t)m0 * N * (OUT_F32 ? 4 : 2);
        if (residual) residual += (size_t)m0 * N;
        M -= m0;
    }
    if (M > 16) M = 16;
    constexpr int SK = 16;
    __shared__ f32x4_t red[SK * 64];
    const int G = K >> 7;
    const int tiles = N >> 3;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int ks = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int tp = blockIdx.x;
    const int q = lane >> 4;
    const int n = lane & 15;
    const int r = n & 7;
    const int tile = 2 * tp + (n >> 3);

    /* 1. every weight piece and scale of this wave (a tile past N reads zeros) */
    const bool tile_ok = tile < tiles;
    const __amdgpu_buffer_rsrc_t wr = make_rsrc(wt, (uint32_t)((size_t)N * K / 2));
    const __amdgpu_buffer_rsrc_t sr = make_rsrc(st, (uint32_t)((size_t)N * G * 2));
    uint4 buf[NL];
    uint16_t sbits[NL];
#pragma unroll
    for (int i = 0; i < NL; ++i) { /* the scales first: loads return in issue order */
        const int g = ks + i * SK;
        const bool ok = tile_ok && g < G;
        const uint32_t unit = (uint32_t)(tile * G + g);
        sbits[i] = buf_load_u16(sr, ok ? unit * 16 + (uint32_t)r * 2 : kOob);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < NL; ++i) {
        const int g = ks + i * SK;
        const bool ok = tile_ok && g < G;
        const uint32_t unit = (uint32_t)(tile * G + g);
        buf[i] = buf_load16_stream(wr, ok ? unit * 512 + (uint32_t)(q * 8 + r) * 16 : kOob);
        __builtin_amdgcn_sched_barrier(0);
    }

    /* 2. the A operands of group i: for MFMA t, row n, k = 128 g + 32 t + 8 q .. + 7 */
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(x, (uint32_t)M * K * 2);
    const bool row_ok = n < M;
    const uint32_t row_off = (uint32_t)(n * K + q * 8) * 2;
    uint4 av[D][4];
    auto load_a = [&](int i) {
        const int g = ks + i * SK;
        const bool ok = row_ok && g < G;
#pragma unroll
        for (int t = 0; t < 4; ++t)
            av[i % D][t] = buf_load16(
                xr, !ok ? kOob
                    : CM ? (uint32_t)(((g * 16 + 4 * t + q) * M + n) * 16)
                         : row_off + (uint32_t)(g * 128 + 32 * t) * 2);
    };
#pragma unroll
    for (int i = 0; i < D && i < NL; ++i) load_a(i);

    /* 3. eight MFMAs a group (the offset ones as in gemv_rows_kernel) */
    const uint4 offs = make_uint4(0xBF40BF40u, 0xBF40BF40u, 0xBF40BF40u, 0xBF40BF40u);
    f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int i = 0; i < NL; ++i) {
        if (ks + i * SK < G) { /* wave-uniform */
            const uint32_t words[4] = {buf[i].x, buf[i].y, buf[i].z, buf[i].w};
            f32x4_t d = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const bf16x8_t a = __builtin_bit_cast(bf16x8_t, av[i % D][t]);
                d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, unpack8(words[t]), d, 0, 0, 0);
                d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, __builtin_bit_cast(bf16x8_t, offs),
                                                            d, 0, 0, 0);
            }
            const float sc = bf16_widen(sbits[i]);
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[j] = fmaf(sc, d[j], acc[j]);
        } else { /* keeps the pair's loads ahead of the branch, in issue order */
            asm volatile("" ::"v"(buf[i].x), "v"(sbits[i]));
        }
        if (i + D < NL) load_a(i + D);
    }

    /* 4. the 16 waves in LDS, summed in wave order; lane (n, q) holds rows 4 q + j of column n */
    red[ks * 64 + lane] = acc;
    __syncthreads();
    if (ks != 0) return;
    f32x4_t sum = acc;
#pragma unroll
    for (int w = 1; w < SK; ++w) {
        const f32x4_t v = red[w * 64 + lane];
#pragma unroll
        for (int j = 0; j < 4; ++j) sum[j] += v[j];
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float row_sum = 32.0f * sum[j];
        const int m = 4 * q + j;
        if (m < M && tile_ok) {
            const size_t o = (size_t)m * N + tile * 8 + r;
            if (OUT_F32) {
                reinterpret_cast<float *>(out)[o] = row_sum;
            } else {
                const uint16_t ob = bf16_rne(row_sum);
                /* plan F2: the residual, already BF16(residual + sublayer), gains the output */
                if (residual) residual[o] = (uint16_t)(bf16_add2(residual[o], ob) & 0xFFFFu);
                reinterpret_cast<uint16_t *>(out)[o] = ob;
            }
        }
    }
}

/* Beyond 16 row-major rows (gemm_int4_bf16): gemv_rows16x_kernel's layout (16 waves a block,
 * wave ks taking groups ks + 16 i, A loaded per lane from memory, one LDS meeting at the end),
 * but a wave takes TPW adjacent tile pairs and runs each A operand against all of them, so a
 * block reads its 16 rows of A once for TPW tile pairs: the A bytes the CUs take in (every block
 * reads all of K for its rows) shrink TPW times. blockIdx.y takes rows 16 y .. 16 y + 15. */
template <bool OUT_F32, int NL, int D, int TPW>
__global__ __launch_bounds__(1024) void gemv_rows16w_kernel(
    const uint16_t *__restrict__ x, int M, const uint8_t *__restrict__ wt,
    const uint16_t *__restrict__ st, void *__restrict__ out, int N, int K) {
    {
        const int m0 = (int)blockIdx.y * 16;
        x += (size_t)m0 * K;
        out = static_cast<char *>(out) + (size_t)m0 * N * (OUT_F32 ? 4 : 2);
        M = min(16, M - m0);
    }
    constexpr int SK = 16;
    extern __shared__ f32x4_t redw[]; /* [SK][TPW][64 lanes] */
    const int G = K >> 7;
    const int tiles = N >> 3;
    const int lane = threadIdx.x & 63;
    const int ks = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int q = lane >> 4;
    const int n = lane & 15;
    const int r = n & 7;
    int tile[TPW];
#pragma unroll
    for (int p = 0; p < TPW; ++p) tile[p] = 2 * ((int)blockIdx.x * TPW + p) + (n >> 3);

    /* 1. every scale, then every weight piece of this wave (a tile past N reads zeros) */
    const __amdgpu_buffer_rsrc_t wr = make_rsrc(wt, (uint32_t)((size_t)N * K / 2));
    const __amdgpu_buffer_rsrc_t sr = make_rsrc(st, (uint32_t)((size_t)N * G * 2));
    uint4 buf[NL][TPW];
    uint16_t sbits[NL][TPW];
#pragma unroll
    for (int i = 0; i < NL; ++i)
#pragma unroll
        for (int p = 0; p < TPW; ++p) {
            const int g = ks + i * SK;
            const bool ok = tile[p] < tiles && g < G;
            const uint32_t unit = (uint32_t)(tile[p] * G + g);
            sbits[i][p] = buf_load_u16(sr, ok ? unit * 16 + (uint32_t)r * 2 : kOob);
        }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < NL; ++i) {
#pragma unroll
        for (int p = 0; p < TPW; ++p) {
            const int g = ks + i * SK;
            const bool ok = tile[p] < tiles && g < G;
            const uint32_t unit = (uint32_t)(tile[p] * G + g);
            buf[i][p] = buf_load16_stream(wr, ok ? unit * 512 + (uint32_t)(q * 8 + r) * 16 : kOob);
        }
        __builtin_amdgcn_sched_barrier(0);
    }

    /* 2. the A operands of group i: for MFMA t, row n, k = 128 g + 32 t + 8 q .. + 7 */
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(x, (uint32_t)M * K * 2);
    const bool row_ok = n < M;
    const uint32_t row_off = (uint32_t)(n * K + q * 8) * 2;
    uint4 av[D][4];
    auto load_a = [&](int i) {
        const int g = ks + i * SK;
        const bool ok = row_ok && g < G;
#pragma unroll
        for (int t = 0; t < 4; ++t)
            av[i % D][t] = buf_load16(xr, ok ? row_off + (uint32_t)(g * 128 + 32 * t) * 2 : kOob);
    };
#pragma unroll
    for (int i = 0; i < D && i < NL; ++i) load_a(i);

    /* 3. per group and tile pair, four product MFMAs and four offset MFMAs, as rows16x */
    const uint4 offs = make_uint4(0xBF40BF40u, 0xBF40BF40u, 0xBF40BF40u, 0xBF40BF40u);
    f32x4_t acc[TPW];
#pragma unroll
    for (int p = 0; p < TPW; ++p) acc[p] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int i = 0; i < NL; ++i) {
        if (ks + i * SK < G) { /* wave-uniform */
#pragma unroll
            for (int p = 0; p < TPW; ++p) {
                const uint32_t words[4] = {buf[i][p].x, buf[i][p].y, buf[i][p].z, buf[i][p].w};
                f32x4_t d = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const bf16x8_t a = __builtin_bit_cast(bf16x8_t, av[i % D][t]);
                    d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, unpack8(words[t]), d, 0, 0, 0);
                    d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, __builtin_bit_cast(bf16x8_t, offs),
                                                                d, 0, 0, 0);
                }
                const float sc = bf16_widen(sbits[i][p]);
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[p][j] = fmaf(sc, d[j], acc[p][j]);
            }
        } else {
#pragma unroll
            for (int p = 0; p < TPW; ++p) asm volatile("" ::"v"(buf[i][p].x), "v"(sbits[i][p]));
        }
        if (i + D < NL) load_a(i + D);
    }

    /* 4. the 16 waves in LDS, summed in wave order; lane (n, q) holds rows 4 q + j of column n */
#pragma unroll
    for (int p = 0; p < TPW; ++p) redw[(ks * TPW + p) * 64 + lane] = acc[p];
    __syncthreads();
    if (ks >= TPW) return;
    const int p = ks; /* wave p finishes tile pair p */
    f32x4_t sum = redw[p * 64 + lane];
    for (int w = 1; w < SK; ++w) {
        const f32x4_t v = redw[(w * TPW + p) * 64 + lane];
#pragma unroll
        for (int j = 0; j < 4; ++j) sum[j] += v[j];
    }
    const int tl = 2 * ((int)blockIdx.x * TPW + p) + (n >> 3);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int m = 4 * q + j;
        if (m < M && tl < tiles) {
            const size_t o = (size_t)m * N + tl * 8 + r;
            const float row_sum = 32.0f * sum[j];
            if (OUT_F32) reinterpret_cast<float *>(out)[o] = row_sum;
            else reinterpret_cast<uint16_t *>(out)[o] = bf16_rne(row_sum);
        }
    }
}

/* RMSNorm of each row (one block a row): BF16(x * rsqrt(sum x^2 / cols + eps) * (bias + w)),
 * FP32 arithmetic (reference csrc/kernels/flashinfer_norm.cu:22-76). Each thread holds CH
 * 8-value chunks of the row, all loaded before any use, so a row costs one load round trip;
 * cols % 8 == 0 and cols <= CH * 8 * 256 (the launcher checks). */
template <int CH>
__global__ __launch_bounds__(256) void rmsnorm_kernel(uint16_t *__restrict__ out,
                                                      uint16_t *x,
                                                      const uint16_t *__restrict__ w, int cols,
                                                      float bias, float eps,
                                                      const uint16_t *sub) {
    __shared__ double red[4];
    const int chunks = cols >> 3;
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(x + (size_t)blockIdx.x * cols, (uint32_t)cols * 2);
    const __amdgpu_buffer_rsrc_t wr = make_rsrc(w, (uint32_t)cols * 2);
    const __amdgpu_buffer_rsrc_t ur =
        make_rsrc(sub ? sub + (size_t)blockIdx.x * cols : sub, sub ? (uint32_t)cols * 2 : 0u);
    uint4 xv[CH], wv[CH], uv[CH];
#pragma unroll
    for (int c = 0; c < CH; ++c) {
        const int i = c * 256 + threadIdx.x;
        xv[c] = buf_load16(xr, i < chunks ? (uint32_t)i * 16 : kOob);
        wv[c] = buf_load16(wr, i < chunks ? (uint32_t)i * 16 : kOob);
        uv[c] = buf_load16(ur, i < chunks ? (uint32_t)i * 16 : kOob);
    }
    if (sub) {
        /* plan F2 (reference csrc/kernels/flashinfer_norm.cu:111-155): the residual becomes
         * BF16(x + sub), is stored back, and the norm reads the rounded value */
        uint4 *xrow = reinterpret_cast<uint4 *>(x + (size_t)blockIdx.x * cols);
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            const int i = c * 256 + threadIdx.x;
            xv[c] = make_uint4(bf16_add2(xv[c].x, uv[c].x), bf16_add2(xv[c].y, uv[c].y),
                               bf16_add2(xv[c].z, uv[c].z), bf16_add2(xv[c].w, uv[c].w));
            if (i < chunks) xrow[i] = xv[c];
        }
    }
    /* the sum of squares in FP64 and the scale rounded once to FP32: the correctly rounded
     * scale whatever the summation order (each square of a BF16 value is exact in FP64) */
    double ss = 0.0;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
        const uint32_t w4[4] = {xv[c].x, xv[c].y, xv[c].z, xv[c].w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const double lo = bf16_widen((uint16_t)(w4[q] & 0xFFFFu));
            const double hi = bf16_widen((uint16_t)(w4[q] >> 16));
            ss = fma(lo, lo, ss);
            ss = fma(hi, hi, ss);
        }
    }
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) ss += __shfl_xor(ss, o);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    const double total = (red[0] + red[1]) + (red[2] + red[3]);
    const float rms = (float)(1.0 / sqrt(total / (double)cols + (double)eps));
    uint4 *orow = reinterpret_cast<uint4 *>(out + (size_t)blockIdx.x * cols);
#pragma unroll
    for (int c = 0; c < CH; ++c) {
        const int i = c * 256 + threadIdx.x;
        const uint32_t x4[4] = {xv[c].x, xv[c].y, xv[c].z, xv[c].w};
        const uint32_t n4[4] = {wv[c].x, wv[c].y, wv[c].z, wv[c].w};
        uint32_t o4[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float lo = bf16_widen((uint16_t)(x4[q] & 0xFFFFu)) * rms *
                             (bias + bf16_widen((uint16_t)(n4[q] & 0xFFFFu)));
            const float hi = bf16_widen((uint16_t)(x4[q] >> 16)) * rms *
                             (bias + bf16_widen((uint16_t)(n4[q] >> 16)));
            const bf16x2_t packed = {(__bf16)lo, (__bf16)hi};
            o4[q] = __builtin_bit_cast(uint32_t, packed);
        }
        if (i < chunks) orow[i] = make_uint4(o4[0], o4[1], o4[2], o4[3]);
    }
}

/* dst <- BF16(dst + src), 8 elements a thread (reference csrc/kernels/gdn_norm.cu:121-129). */
__global__ __launch_bounds__(256) void residual_add_kernel(uint16_t *__restrict__ dst,
                                                           const uint16_t *__restrict__ src,
                                                           long long chunks) {
    const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
    if (i >= chunks) return;
    uint4 *d = reinterpret_cast<uint4 *>(dst) + i;
    const uint4 a = *d, b = reinterpret_cast<const uint4 *>(src)[i];
    *d = make_uint4(bf16_add2(a.x, b.x), bf16_add2(a.y, b.y), bf16_add2(a.z, b.z),
                    bf16_add2(a.w, b.w));
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

/* Events that time one of the calling thread's next kernel launches (w4a16_time_next_launch): it
 * goes through hipExtLaunchKernel, whose events take the dispatch's own start and end times
 * (the times a kernel trace reports), and the pair is then forgotten. */
thread_local hipEvent_t t_next_launch_events[2] = {nullptr, nullptr};
thread_local int t_launches_to_skip = 0;

template <typename... Params, typename... Args>
void launch_k(void (*kernel)(Params...), dim3 grid, dim3 block, size_t smem, hipStream_t stream,
              Args... args) {
    hipEvent_t start = t_next_launch_events[0], stop = t_next_launch_events[1];
    if ((start || stop) && t_launches_to_skip > 0) {
        --t_launches_to_skip;
        start = stop = nullptr;
    }
    if (start || stop) {
        t_next_launch_events[0] = t_next_launch_events[1] = nullptr;
        hipExtLaunchKernelGGL(kernel, grid, block, (uint32_t)smem, stream, start, stop, 0u,
                              static_cast<Params>(args)...);
    } else {
        hipLaunchKernelGGL(kernel, grid, block, smem, stream, static_cast<Params>(args)...);
    }
}

int grid_for(long long work, int block) {
    long long g = (work + block - 1) / block;
    if (g > 65535LL * 16) g = 65535LL * 16;
    return (int)(g < 1 ? 1 : g);
}

size_t gemv_smem(int K, int waves) {
    return (size_t)K * 2 + (size_t)(K / 128) * 16 + (size_t)waves * 32;
}

/* Optional RMSNorm prologue of a GEMV (gate/up only): weight, bias (1 Gemma, 0 plain), eps. */
struct NormArgs {
    const uint16_t *w = nullptr;
    float bias = 0.0f, eps = 0.0f;
    const uint16_t *sub = nullptr; /* plan F2: normalise BF16(x + sub) */
};

template <bool PAIR, bool OUT_F32, int TB, int SK, int NL>
int launch_gemv_cfg(const uint16_t *x, const uint8_t *w, const uint16_t *s, void *out, int N,
                    int K, hipStream_t stream, const NormArgs *norm = nullptr) {
    const int tiles = N / 8;
    if (SK * NL < (K / 128 + 1) / 2)
        return set_error(W4A16_ERR_CONFIG, "internal: a %d x %d gemv shape covers %d of %d group pairs",
                         SK, NL, SK * NL, (K / 128 + 1) / 2);
    if (norm)
        launch_k((gemv_tiles_kernel<PAIR, OUT_F32, TB, SK, true, NL>),
                           dim3((tiles + TB - 1) / TB), dim3(TB * SK * 64), gemv_smem(K, TB * SK),
                           stream, x, w, s, out, N, K, norm->w, norm->bias, norm->eps, norm->sub);
    else
        launch_k((gemv_tiles_kernel<PAIR, OUT_F32, TB, SK, false, NL>),
                           dim3((tiles + TB - 1) / TB), dim3(TB * SK * 64), gemv_smem(K, TB * SK),
                           stream, x, w, s, out, N, K, nullptr, 0.0f, 0.0f, nullptr);
    return hip_status(hipGetLastError(), "gemv launch");
}

int split_scratch(size_t partial_bytes, size_t ncounters, uint64_t **partial, unsigned **counters);

template <bool OUT_F32, int NP, int SK, int BS, bool PAIR = false>
int launch_xwave_np(const uint16_t *x, const uint8_t *w, const uint16_t *s, void *out, int N,
                    int K, hipStream_t stream, uint16_t *residual = nullptr,
                    const uint16_t *sub = nullptr) {
    if (SK * BS * NP < (K / 128 + 1) / 2)
        return set_error(W4A16_ERR_CONFIG, "internal: a %d x %d x %d wave-local shape covers %d of %d "
                         "group pairs", BS, SK, NP, BS * SK * NP, (K / 128 + 1) / 2);
    uint64_t *partial = nullptr;
    unsigned *counters = nullptr;
    if (BS > 1) {
        int st = split_scratch((size_t)(N / 8) * BS * 8 * sizeof(uint64_t), (size_t)(N / 8),
                               &partial, &counters);
        if (st) return st;
    }
    launch_k((gemv_xwave_kernel<PAIR, OUT_F32, SK, NP, BS>), dim3(N / 8 * BS), dim3(SK * 64),
                       xwave_smem(SK, NP), stream, x, w, s, out, N, K, partial, counters, residual,
                       sub);
    return hip_status(hipGetLastError(), "gemv launch");
}

template <bool OUT_F32, int SK, int NP, bool PAIR = false, int M = 1>
int launch_mfma1(const uint16_t *x, const uint8_t *w, const uint16_t *s, void *out, int N, int K,
                 hipStream_t stream, uint16_t *residual = nullptr, const uint16_t *sub = nullptr) {
    if (SK * NP < (K / 128 + 1) / 2)
        return set_error(W4A16_ERR_CONFIG, "internal: a %d x %d matrix-core gemv shape covers %d of %d "
                         "group pairs", SK, NP, SK * NP, (K / 128 + 1) / 2);
    launch_k((gemv_mfma1_kernel<PAIR, OUT_F32, SK, NP, M>), dim3(N / 8), dim3(SK * 64),
                       mfma1_smem(SK, NP, M), stream, x, w, s, out, N, K, residual, sub);
    return hip_status(hipGetLastError(), "gemv launch");
}

/* The wave-local kernel for a K of more than kMaxLoads group pairs: up to 48 pairs one block of
 * 16 waves a tile (12 waves at 33 to 36 pairs); beyond, the tile split over BS blocks of 8 waves holding at most 3 pairs each
 * (K = 17408: 12.9 against 13.7 us). residual / sub: the plan-F2 epilogue (BF16 output only).
 * Returns 1 when K is beyond its shapes. */
template <bool OUT_F32>
int launch_xwave(const uint16_t *x, const uint8_t *w, const uint16_t *s, void *out, int N, int K,
                 hipStream_t stream, uint16_t *residual = nullptr, const uint16_t *sub = nullptr) {
    const int pairs = (K / 128 + 1) / 2;
    /* 33 to 36 pairs (K = 8320..9216; C4's down, K = 8704): twelve waves of three pairs,
     * 7.6-7.7 us against 8.1-8.4 for sixteen waves (interleaved bench runs, one box). At 38
     * pairs (C1's down) thirteen waves only tie sixteen. */
    if (pairs > 32 && pairs <= 36)
        return launch_xwave_np<OUT_F32, 3, 12, 1>(x, w, s, out, N, K, stream, residual, sub);
    /* 17 to 20 pairs (C5, K = 5120): the matrix-core form, ten waves of two pairs, 3.97 us
     * against 4.08 for the v_dot2 kernel of the same shape (matrix-core 7 x 3: 4.16, 5 x 4:
     * 4.27; the v_dot2 kernel: 16 waves of which twelve held one pair 4.21, 3 x 7 4.17, 4 x 5
     * 4.35, 5 x 4 4.43; interleaved runs, one box) */
    if (pairs > 16 && pairs <= 20)
        return launch_mfma1<OUT_F32, 10, 2>(x, w, s, out, N, K, stream, residual, sub);
    /* 37 to 48 pairs (C1's down, K = 9728): the matrix-core form, C1 11.45 against 11.59-11.70
     * us for the v_dot2 kernel of the same shape; thirteen waves of three pairs up to 39 pairs
     * (11.35-11.45 against 11.42-11.46 for sixteen, 10 x 4: 11.54-11.58; interleaved runs, one
     * box), sixteen beyond. At 34 and 68 pairs (C4, C2) the two forms tie. */
    if (pairs > 36 && pairs <= 39)
        return launch_mfma1<OUT_F32, 13, 3>(x, w, s, out, N, K, stream, residual, sub);
    if (pairs > 39 && pairs <= 48)
        return launch_mfma1<OUT_F32, 16, 3>(x, w, s, out, N, K, stream, residual, sub);
    switch ((pairs + kXwaveWaves - 1) / kXwaveWaves) {
        case 1: return launch_xwave_np<OUT_F32, 1, kXwaveWaves, 1>(x, w, s, out, N, K, stream, residual, sub);
        case 2: return launch_xwave_np<OUT_F32, 2, kXwaveWaves, 1>(x, w, s, out, N, K, stream, residual, sub);
        case 3: return launch_xwave_np<OUT_F32, 3, kXwaveWaves, 1>(x, w, s, out, N, K, stream, residual, sub);
        default: break;
    }
    switch ((pairs + 23) / 24) {
        case 3: return launch_xwave_np<OUT_F32, 3, 8, 3>(x, w, s, out, N, K, stream, residual, sub);
        case 4: return launch_xwave_np<OUT_F32, 3, 8, 4>(x, w, s, out, N, K, stream, residual, sub);
        case 5: return launch_xwave_np<OUT_F32, 3, 8, 5>(x, w, s, out, N, K, stream, residual, sub);
        case 6: return launch_xwave_np<OUT_F32, 3, 8, 6>(x, w, s, out, N, K, stream, residual, sub);
        case 7: return launch_xwave_np<OUT_F32, 3, 8, 7>(x, w, s, out, N, K, stream, residual, sub);
        case 8: return launch_xwave_np<OUT_F32, 3, 8, 8>(x, w, s, out, N, K, stream, residual, sub);
        default: return 1;
    }
}

/* Block shapes (measured on MI355X, graph-replayed, weights rotated past the MALL):
 * - a long K (more group pairs than one wave holds, the down projection) runs the wave-local
 *   activation kernel: at K = 9728 / 8704 / 17408 it takes 5.85 / 8.35 / 12.9 us against
 *   6.2 / 9.7 / 15.7 us for the block-staged kernel;
 * - 7 to 12 group pairs (K = 1792..3072, the C0/C1 gate/up) run it too, one tile of four waves
 *   holding three pairs each: C1 gate/up 7.53 against 7.79 us, C0 5.0 against 5.43 (medians of
 *   interleaved runs; at K = 5120 it only ties the block-staged 1 x 4 x 5, 17.6-17.9 against
 *   17.4-18.4 us, which stays);
 * - otherwise the block-staged kernel with few loads a wave (NL) and several waves a tile, which
 *   keeps 8 waves a SIMD resident. Medians of 7 interleaved graph runs, whole C1 FFN (gate/up
 *   shape varied, same down kernel): 2 tiles x 2 waves x 5 pairs 13.9 us; 1 x 4 x 3 14.4;
 *   2 x 4 x 3 14.1; 4 x 1 x 10 14.7; 2 x 2 x 12 (12 loads a wave, 4 waves a SIMD) 14.9. At
 *   K = 5120, 1 x 4 x 5 takes 19.8 us for the C4 FFN against 20.4 for 2 x 2 x 12. */
template <bool PAIR, bool OUT_F32>
int launch_gemv(const uint16_t *x, const uint8_t *w, const uint16_t *s, void *out, int N, int K,
                hipStream_t stream, const NormArgs *norm = nullptr) {
    const int pairs = (K / 128 + 1) / 2;
    if (!PAIR && !norm && pairs > kMaxLoads) {
        const int st = launch_xwave<OUT_F32>(x, w, s, out, N, K, stream);
        if (st <= 0) return st;
    }
    /* 7 to 12 pairs without the pair (C0, K = 2560): the matrix-core form, C0 4.30 us at five
     * waves of two pairs against 4.51 for the v_dot2 kernel's four of three (4 x 3: 4.40, 6 x 3,
     * 8 x 2, 10 x 2, 4 x 4: 4.56-5.72); for gate/up (the pair) the two tie, and the v_dot2 kernel
     * stays */
    if (!PAIR && !norm && pairs > 6 && pairs <= 10) return launch_mfma1<OUT_F32, 5, 2>(x, w, s, out, N, K, stream);
    if (!PAIR && !norm && pairs > 10 && pairs <= 12) return launch_mfma1<OUT_F32, 4, 3>(x, w, s, out, N, K, stream);
    if (!norm && pairs > 6 && pairs <= 12)
        return launch_xwave_np<OUT_F32, 3, 4, 1, PAIR>(x, w, s, out, N, K, stream);
    if (norm) {
        /* every block normalises all of x, yet the small-load shape still wins over fewer,
         * larger blocks (C1 norm + FFN medians: 2 x 2 x 5 14.9 us, 4 x 1 x 10 15.4, 4 x 2 x 5
         * 15.5; the FFN alone 13.9) */
        if (pairs <= 10) return launch_gemv_cfg<PAIR, OUT_F32, 2, 2, 5>(x, w, s, out, N, K, stream, norm);
        if (pairs <= 12) return launch_gemv_cfg<PAIR, OUT_F32, 2, 2, 6>(x, w, s, out, N, K, stream, norm);
        return set_error(W4A16_ERR_CONFIG, "gemv: the RMSNorm prologue needs K <= 3072");
    }
    if (pairs <= 3) return launch_gemv_cfg<PAIR, OUT_F32, 4, 1, 3>(x, w, s, out, N, K, stream);
    if (pairs <= 6) return launch_gemv_cfg<PAIR, OUT_F32, 2, 2, 3>(x, w, s, out, N, K, stream);
    if (pairs <= 20) return launch_gemv_cfg<PAIR, OUT_F32, 1, 4, 5>(x, w, s, out, N, K, stream);
    if (pairs <= 48) return launch_gemv_cfg<PAIR, OUT_F32, 1, 8, 6>(x, w, s, out, N, K, stream);
    if (pairs <= 96) return launch_gemv_cfg<PAIR, OUT_F32, 1, 16, 6>(x, w, s, out, N, K, stream);
    return launch_gemv_cfg<PAIR, OUT_F32, 1, 16, 8>(x, w, s, out, N, K, stream);
}

/* Few-row kernel: LDS for both groups of every pair of the M rows (whole 1 KiB load
 * instructions) and the wave reduction. */
size_t rows_smem(int M, int K, int waves) {
    const int P = (K / 128 + 1) / 2;
    return (size_t)((P * 32 * M + 63) / 64) * 1024 + (size_t)waves * 256;
}

template <bool PAIR, bool OUT_F32, int TB, int SK, int NL>
int launch_rows_mi(const uint16_t *x, int M, const uint8_t *w, const uint16_t *s, void *out,
                   int N, int K, hipStream_t stream, uint16_t *residual = nullptr, int cm = 0) {
    if (SK * NL < (K / 128 + 1) / 2)
        return set_error(W4A16_ERR_CONFIG, "internal: a %d x %d few-row shape covers %d of %d group pairs",
                         SK, NL, SK * NL, (K / 128 + 1) / 2);
    const size_t smem = rows_smem(M, K, TB * SK);
    if (smem > kMaxLds) return 1;
    const dim3 grid((N / 8 + TB - 1) / TB), block(TB * SK * 64);
    if (M == 2)
        launch_k((gemv_rows_kernel<PAIR, OUT_F32, TB, SK, NL, 2>), grid, block, smem,
                           stream, x, M, w, s, out, N, K, residual, cm);
    else
        launch_k((gemv_rows_kernel<PAIR, OUT_F32, TB, SK, NL, 4>), grid, block, smem,
                           stream, x, M, w, s, out, N, K, residual, cm);
    return hip_status(hipGetLastError(), "gemv rows launch");
}

/* 2 <= M <= 8 on the few-row kernel; returns 1 when the shape is not applicable (the staged
 * rows past the LDS of a block, or more than 80 group pairs). Shapes from sweeps of the C1 FFN
 * (graph-replayed, weights rotated past the MALL; gate/up K = 2560, down K = 9728):
 * - short K (gate/up): the M = 1 GEMV's shapes up to M = 4; from M = 5 twice the tiles a block,
 *   which halves the activation staged per tile (M = 8: 4 x 2 x 5 11.0 us, 2 x 2 x 5 12.0);
 * - long K (down): two tiles of eight waves a block (M = 2 / 4 / 8: 6.6 / 7.8 / 9.3 us; one tile
 *   of 8 or 16 waves: 7.0 / 8.8-9.1 / 14.3, the M = 8 rows filling 155 KB of LDS a block). */
/* 9 <= M <= 16, short K: tile-pair waves. Each block stages all M rows (80 KB at M = 16,
 * K = 2560, so at most two blocks a CU), which makes the grid's balance the lever: one block a
 * CU, TP = ceil(tile pairs / CUs) tile pairs of SK = 16 / TP waves. C1 gate/up at M = 16
 * (1216 tile pairs): 5 x 3 waves 11.7 us; 6 x 2 11.9, 5 x 2 12.1, 8 x 2 13.4, 3 x 5 14.8,
 * 4 x 4 17.0, 2 x 8 17.6, 1 x 4 24.4 (the split-K MFMA form: 16.3). */
size_t rows16_smem(int M, int K, int waves) {
    return (size_t)((K / 128 * 16 * M + 63) / 64) * 1024 + (size_t)waves * 1024;
}

template <bool PAIR, bool OUT_F32, int NL>
int launch_rows16_nl(const uint16_t *x, int M, const uint8_t *w, const uint16_t *s, void *out,
                     int N, int K, int TP, int SK, hipStream_t stream, int cm) {
    const size_t smem = rows16_smem(M, K, TP * SK);
    if (smem > kMaxLds) return 1;
    const int pairs = (N / 8 + 1) / 2;
    launch_k((gemv_rows16_kernel<PAIR, OUT_F32, NL>), dim3((pairs + TP - 1) / TP),
                       dim3(TP * SK * 64), smem, stream, x, M, w, s, out, N, K, TP, SK, cm);
    return hip_status(hipGetLastError(), "gemv rows16 launch");
}

int device_cus();

template <bool OUT_F32, bool CM, int NL>
int launch_rows16x_nl(const uint16_t *x, int M, const uint8_t *w, const uint16_t *s, void *out,
                      int N, int K, hipStream_t stream, uint16_t *residual) {
    constexpr int D = NL <= 5 ? NL : NL <= 9 ? 4 : 3;
    const int pairs = (N / 8 + 1) / 2;
    launch_k((gemv_rows16x_kernel<OUT_F32, NL, D, CM>), dim3(pairs, CM ? 1 : (M + 15) / 16),
             dim3(1024), 0, stream, x, M, w, s, out, N, K, residual);
    return hip_status(hipGetLastError(), "gemv rows16x launch");
}

/* Long-K rows without LDS staging (gemv_rows16x_kernel): one tile pair a block of 16 waves. */
template <bool OUT_F32, bool CM = false>
int launch_rows16x(const uint16_t *x, int M, const uint8_t *w, const uint16_t *s, void *out, int N,
                   int K, hipStream_t stream, uint16_t *residual = nullptr) {
    const int nl = (K / 128 + 15) / 16;
    if (nl <= 2) return launch_rows16x_nl<OUT_F32, CM, 2>(x, M, w, s, out, N, K, stream, residual);
    if (nl <= 3) return launch_rows16x_nl<OUT_F32, CM, 3>(x, M, w, s, out, N, K, stream, residual);
    if (nl <= 4) return launch_rows16x_nl<OUT_F32, CM, 4>(x, M, w, s, out, N, K, stream, residual);
    if (nl <= 5) return launch_rows16x_nl<OUT_F32, CM, 5>(x, M, w, s, out, N, K, stream, residual);
    if (nl <= 6) return launch_rows16x_nl<OUT_F32, CM, 6>(x, M, w, s, out, N, K, stream, residual);
    if (nl <= 8) return launch_rows16x_nl<OUT_F32, CM, 8>(x, M, w, s, out, N, K, stream, residual);
    if (nl <= 9) return launch_rows16x_nl<OUT_F32, CM, 9>(x, M, w, s, out, N, K, stream, residual);
    if (nl <= 12) return launch_rows16x_nl<OUT_F32, CM, 12>(x, M, w, s, out, N, K, stream, residual);
    return 1;
}

/* Beyond 16 row-major rows: gemv_rows16w_kernel with as many tile pairs a wave (4, 2 or 1) as
 * still leaves a block a CU across the 16-row slices. Returns 1 when K is beyond its shapes. */
template <bool OUT_F32, int NL, int TPW>
int launch_rows16w_t(const uint16_t *x, int M, const uint8_t *w, const uint16_t *s, void *out,
                     int N, int K, hipStream_t stream) {
    constexpr int D = TPW >= 4 ? 1 : 2;
    const int pairs = (N / 8 + 1) / 2;
    launch_k((gemv_rows16w_kernel<OUT_F32, NL, D, TPW>), dim3((pairs + TPW - 1) / TPW, (M + 15) / 16),
             dim3(1024), (size_t)16 * TPW * 64 * sizeof(f32x4_t), stream, x, M, w, s, out, N, K);
    return hip_status(hipGetLastError(), "gemv rows16w launch");
}

template <bool OUT_F32, int NL>
int launch_rows16w_nl(const uint16_t *x, int M, const uint8_t *w, const uint16_t *s, void *out,
                      int N, int K, hipStream_t stream) {
    const int pairs = (N / 8 + 1) / 2;
    const int slices = (M + 15) / 16;
    const int cus = device_cus();
    if ((pairs / 4) * slices >= cus) return launch_rows16w_t<OUT_F32, NL, 4>(x, M, w, s, out, N, K, stream);
    if ((pairs / 2) * slices >= cus) return launch_rows16w_t<OUT_F32, NL, 2>(x, M, w, s, out, N, K, stream);
    return 1;
}

template <bool OUT_F32>
int launch_rows16w(const uint16_t *x, int M, const uint8_t *w, const uint16_t *s, void *out, int N,
                   int K, hipStream_t stream) {
    const int nl = (K / 128 + 15) / 16;
    if (nl <= 2) return launch_rows16w_nl<OUT_F32, 2>(x, M, w, s, out, N, K, stream);
    if (nl <= 3) return launch_rows16w_nl<OUT_F32, 3>(x, M, w, s, out, N, K, stream);
    return 1;
}

template <bool PAIR, bool OUT_F32>
int launch_rows16(const uint16_t *x, int M, const uint8_t *w, const uint16_t *s, void *out, int N,
                  int K, hipStream_t stream, int cm = 0) {
    const int G = K / 128;
    const int pairs = (N / 8 + 1) / 2;
    const int TP = std::min(16, (pairs + device_cus() - 1) / device_cus());
    const int SK = std::max(1, 16 / TP);
    const int nl = (G + SK - 1) / SK;
    if (nl <= 2) return launch_rows16_nl<PAIR, OUT_F32, 2>(x, M, w, s, out, N, K, TP, SK, stream, cm);
    if (nl <= 4) return launch_rows16_nl<PAIR, OUT_F32, 4>(x, M, w, s, out, N, K, TP, SK, stream, cm);
    if (nl <= 6) return launch_rows16_nl<PAIR, OUT_F32, 6>(x, M, w, s, out, N, K, TP, SK, stream, cm);
    if (nl <= 8) return launch_rows16_nl<PAIR, OUT_F32, 8>(x, M, w, s, out, N, K, TP, SK, stream, cm);
    if (nl <= 12) return launch_rows16_nl<PAIR, OUT_F32, 12>(x, M, w, s, out, N, K, TP, SK, stream, cm);
    return 1;
}

template <bool PAIR, bool OUT_F32>
int launch_rows(const uint16_t *x, int M, const uint8_t *w, const uint16_t *s, void *out, int N,
                int K, hipStream_t stream, uint16_t *residual = nullptr, int cm = 0) {
    /* long K (the staged rows would not fit LDS): registers-fed A from M = 8 (9 with the
     * residual epilogue) to 15; at 16 the split-K MFMA form is faster. C1 down, medians of
     * interleaved whole-call runs, split-K or LDS-staged against rows16x: M = 8 20.5 / 19.9 us,
     * 10 22.7 / 21.0, 13 23.9 / 22.6, 14 24.2 / 23.4, 15 24.2 / 23.9, 16 24.4 / 24.6; at M = 8
     * plan F2 23.3 against 23.6, and M = 4 and 6 tie. */
    if (!PAIR && M >= (residual ? 9 : 8) && M <= 15 && rows16_smem(M, K, 16) > kMaxLds)
        return launch_rows16x<OUT_F32>(x, M, w, s, out, N, K, stream, residual);
    if (M > 8 && M <= 16 && !residual)
        return launch_rows16<PAIR, OUT_F32>(x, M, w, s, out, N, K, stream, cm);
    if (M < 2 || M > 8) return 1;
    const int pairs = (K / 128 + 1) / 2;
    /* two rows on the matrix-core GEMV: the gate/up pair at 7 to 12 group pairs (four waves of
     * three) and the long K of the C1 down projection, 37 to 48 pairs (sixteen of three). Whole
     * C1 FFN call at M = 2: 12.58-12.66 us against 13.70-13.99 on this kernel's few-row form
     * (down alone 12.82-12.90, gate/up alone 13.55; gate/up as five waves of two ties; down as
     * thirteen of three 12.58 with the gate/up; interleaved runs, one box). */
    if (M == 2 && !cm) {
        if (PAIR && pairs > 6 && pairs <= 12)
            return launch_mfma1<OUT_F32, 4, 3, true, 2>(x, w, s, out, N, K, stream);
        if (!PAIR && pairs > 36 && pairs <= 48)
            return launch_mfma1<OUT_F32, 16, 3, false, 2>(x, w, s, out, N, K, stream, residual);
    }
    if (pairs <= 12 && M <= 4) {
        if (pairs <= 3) return launch_rows_mi<PAIR, OUT_F32, 4, 1, 3>(x, M, w, s, out, N, K, stream, residual, cm);
        if (pairs <= 6) return launch_rows_mi<PAIR, OUT_F32, 2, 2, 3>(x, M, w, s, out, N, K, stream, residual, cm);
        if (pairs <= 10) return launch_rows_mi<PAIR, OUT_F32, 2, 2, 5>(x, M, w, s, out, N, K, stream, residual, cm);
        return launch_rows_mi<PAIR, OUT_F32, 2, 2, 6>(x, M, w, s, out, N, K, stream, residual, cm);
    }
    if (pairs <= 12) {
        if (pairs <= 3) return launch_rows_mi<PAIR, OUT_F32, 8, 1, 3>(x, M, w, s, out, N, K, stream, residual, cm);
        if (pairs <= 6) return launch_rows_mi<PAIR, OUT_F32, 4, 2, 3>(x, M, w, s, out, N, K, stream, residual, cm);
        if (pairs <= 10) return launch_rows_mi<PAIR, OUT_F32, 4, 2, 5>(x, M, w, s, out, N, K, stream, residual, cm);
        return launch_rows_mi<PAIR, OUT_F32, 4, 2, 6>(x, M, w, s, out, N, K, stream, residual, cm);
    }
    if (pairs <= 20) return launch_rows_mi<PAIR, OUT_F32, 2, 4, 5>(x, M, w, s, out, N, K, stream, residual, cm);
    if (pairs <= 40) return launch_rows_mi<PAIR, OUT_F32, 2, 8, 5>(x, M, w, s, out, N, K, stream, residual, cm);
    if (pairs <= 48) return launch_rows_mi<PAIR, OUT_F32, 2, 8, 6>(x, M, w, s, out, N, K, stream, residual, cm);
    if (pairs <= 80) return launch_rows_mi<PAIR, OUT_F32, 2, 8, 10>(x, M, w, s, out, N, K, stream, residual, cm);
    return 1;
}

/* Compute units of the current device (cached per device; 256 if the query fails). */
int device_cus() {
    static int cus[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cus[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            n <= 0)
            n = 256;
        cus[dev] = n;
    }
    return cus[dev];
}

/* Split-K scratch for the MFMA form: FP32 partials and per-tile-pair arrival counters, one set
 * per device, grown on demand (growth allocates, so it cannot happen under graph capture, and
 * synchronises the device; counters are zeroed when allocated and every kernel leaves them
 * zero). Outgrown buffers stay allocated until the process ends (at most the size of the current
 * one in total, since sizes double), so graphs captured before a growth stay valid. Calls that
 * overlap in time on one device share the scratch, so they must be ordered on one stream. */
struct SplitScratch {
    uint64_t *partial = nullptr; /* mailbox slots (slot_put) */
    size_t partial_bytes = 0;
    unsigned *counters = nullptr;
    size_t ncounters = 0;
};
std::mutex g_scratch_mu;
SplitScratch g_scratch[64];

/* While an allocation-free entry point runs on this thread, the split-K kernels take their
 * partials and counters from the static scratch array below instead of the growable buffer. */
struct FixedScratch {
    bool active = false;
    uint64_t *partial = nullptr; /* mailbox slots (slot_put) */
    size_t partial_bytes = 0;
    unsigned *counters = nullptr;
    size_t ncounters = 0;
};
thread_local FixedScratch t_fixed;

int split_scratch(size_t partial_bytes, size_t ncounters, uint64_t **partial, unsigned **counters) {
    if (t_fixed.active) {
        /* the entry point checked its shapes against these sizes before launching anything */
        if (partial_bytes > t_fixed.partial_bytes || ncounters > t_fixed.ncounters)
            return set_error(W4A16_ERR_CONFIG, "split-K needs %zu bytes and %zu counters, beyond the "
                             "static scratch (%zu bytes, %zu counters)", partial_bytes, ncounters,
                             t_fixed.partial_bytes, t_fixed.ncounters);
        *partial = t_fixed.partial;
        *counters = t_fixed.counters;
        return W4A16_OK;
    }
    int dev = 0;
    int st = hip_status(hipGetDevice(&dev), "hipGetDevice");
    if (st) return st;
    if (dev < 0 || dev >= 64) return set_error(W4A16_ERR_CONFIG, "device ordinal %d out of range", dev);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    SplitScratch &sc = g_scratch[dev];
    if (sc.partial_bytes < partial_bytes) {
        size_t want = (size_t)4 << 20;
        while (want < partial_bytes) want *= 2;
        /* the outgrown buffer is kept, not freed: a kernel still in flight, or a graph
         * captured earlier, may hold its address */
        sc.partial = nullptr;
        sc.partial_bytes = 0;
        if (hipMalloc((void **)&sc.partial, want) != hipSuccess)
            return set_error(W4A16_ERR_ALLOC, "split-K scratch: hipMalloc(%zu) failed", want);
        /* every slot starts empty (flag 0); kernels leave the slots they use empty */
        st = hip_status(hipMemset(sc.partial, 0, want), "hipMemset split-K slots");
        if (!st) st = hip_status(hipDeviceSynchronize(), "hipDeviceSynchronize");
        if (st) return st;
        sc.partial_bytes = want;
    }
    if (sc.ncounters < ncounters) {
        size_t want = 65536;
        while (want < ncounters) want *= 2;
        sc.counters = nullptr; /* kept, as above; every kernel leaves its counters zero */
        sc.ncounters = 0;
        if (hipMalloc((void **)&sc.counters, want * sizeof(unsigned)) != hipSuccess)
            return set_error(W4A16_ERR_ALLOC, "split-K counters: hipMalloc failed");
        st = hip_status(hipMemset(sc.counters, 0, want * sizeof(unsigned)), "hipMemset counters");
        if (!st) st = hip_status(hipDeviceSynchronize(), "hipDeviceSynchronize");
        if (st) return st;
        sc.ncounters = want;
    }
    *partial = sc.partial;
    *counters = sc.counters;
    return W4A16_OK;
}

struct MfmaPlan {
    int S, GS, xpre, grid;
    size_t smem, partial_bytes, ncounters;
};

/* K split: at most kGMax groups per wave, activation range within 32 KiB of LDS, and enough
 * blocks that the waves cover the chip several times over. */
MfmaPlan plan_mfma(int M, int N, int K) {
    MfmaPlan p{};
    const int G = K / 128;
    const int NT = (N / 8 + 1) / 2;
    const int gmax = std::max(1, std::min(kGMax, 128 / M));
    int S = (G + gmax - 1) / gmax;
    const int nblk = (NT + kMfmaWaves - 1) / kMfmaWaves;
    while ((long long)nblk * kMfmaWaves * S < 1024 && (G + S) / (S + 1) >= 4) ++S;
    p.GS = (G + S - 1) / S;
    p.S = (G + p.GS - 1) / p.GS;
    const int chunks = M * p.GS * 16;
    const int pre = (chunks + kMfmaWaves * 64 - 1) / (kMfmaWaves * 64);
    p.xpre = pre <= 1 ? 1 : pre <= 2 ? 2 : pre <= 4 ? 4 : 8;
    p.grid = nblk * p.S;
    p.smem = (size_t)(chunks + p.GS * 16) * 16 + (size_t)M * p.GS * 4;
    p.partial_bytes = p.S > 1 ? (size_t)p.S * NT * 16 * M * sizeof(uint64_t) : 0;
    p.ncounters = p.S > 1 ? (size_t)NT : 0;
    return p;
}

/* ---- The allocation-free scratch ------------------------------------------------------------
 * For callers that cannot allocate device memory (code under HIP graph capture, serving loops,
 * harnesses that forbid hipMalloc): the split-K partials and arrival counters in one static
 * device array, 256 KiB of counters then 32 MiB of partial slots (an FP32 value and a
 * written-flag each, see slot_put), which each GPU holds for the life of the process. The host-side name `scratch` is only a stand-in for the device array, so
 * host code uses the address hipGetSymbolAddress returns for the current device, never the name. */
constexpr size_t kFixedCounters = 65536;
constexpr size_t kFixedPartialBytes = (size_t)32 << 20;
static __device__ __align__(256) unsigned char scratch[kFixedCounters * 4 + kFixedPartialBytes];

__global__ void zero_words_kernel(unsigned *p, size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        p[i] = 0u;
}

void *g_fixed_base[64]; /* per device: the address of `scratch` there (under g_scratch_mu) */

/* The device's scratch address, looked up (and the whole array cleared by a fill kernel on
 * `stream`, which a graph capture may record) on the first call on that device. */
int fixed_scratch(hipStream_t stream, unsigned char **base) {
    int dev = 0;
    int st = hip_status(hipGetDevice(&dev), "hipGetDevice");
    if (st) return st;
    if (dev < 0 || dev >= 64) return set_error(W4A16_ERR_CONFIG, "device ordinal %d out of range", dev);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_fixed_base[dev]) {
        /* the one-time clear below must run, not be recorded into a graph that may never be
         * replayed: the first call on a device is refused under capture */
        hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
        st = hip_status(hipStreamIsCapturing(stream, &cap), "hipStreamIsCapturing");
        if (st) return st;
        if (cap != hipStreamCaptureStatusNone)
            return set_error(W4A16_ERR_STATE, "mlp_int4_bf16_noalloc: the first call on device %d "
                             "clears the static scratch and must be made outside graph capture",
                             dev);
        void *p = nullptr;
        st = hip_status(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
        if (st) return st;
        if (!p) return set_error(W4A16_ERR_HIP, "hipGetSymbolAddress(scratch) returned no address");
        launch_k(zero_words_kernel, dim3(2048), dim3(256), 0, stream,
                           static_cast<unsigned *>(p), sizeof(scratch) / 4);
        st = hip_status(hipGetLastError(), "scratch clear");
        if (st) return st;
        g_fixed_base[dev] = p;
    }
    *base = static_cast<unsigned char *>(g_fixed_base[dev]);
    return W4A16_OK;
}

/* An upper bound of the split-K scratch one [M, K] x [N, K]^T product of this library can ask
 * for, whichever kernel it is routed to: the wave-local GEMV's tile split (at most 8 blocks a
 * tile, M = 1) and the MFMA form's plan for a 16-row slice (smaller slices need less). */
void split_bound(int M, int N, int K, size_t *partial_bytes, size_t *ncounters) {
    const size_t tiles = (size_t)N / 8;
    size_t pb = tiles * 8 * 8 * sizeof(uint64_t), nc = tiles;
    const MfmaPlan p = plan_mfma(std::min(std::max(M, 1), 16), N, K);
    pb = std::max(pb, p.partial_bytes);
    nc = std::max(nc, p.ncounters);
    *partial_bytes = pb;
    *ncounters = nc;
}

template <int OUT, int XPRE>
int launch_mfma_x(const MfmaPlan &p, const uint16_t *x, int M, const uint8_t *w,
                  const uint16_t *s, void *out, int N, int K, uint64_t *partial, unsigned *counters,
                  hipStream_t stream, uint16_t *residual, int cm) {
    if (M == 1)
        launch_k((mfma_gemm_kernel<OUT, XPRE, 1>), dim3(p.grid), dim3(kMfmaWaves * 64),
                           p.smem, stream, x, M, w, s, out, N, K, p.S, p.GS, partial, counters,
                           residual, cm);
    else if (M == 2)
        launch_k((mfma_gemm_kernel<OUT, XPRE, 2>), dim3(p.grid), dim3(kMfmaWaves * 64),
                           p.smem, stream, x, M, w, s, out, N, K, p.S, p.GS, partial, counters,
                           residual, cm);
    else
        launch_k((mfma_gemm_kernel<OUT, XPRE, 4>), dim3(p.grid), dim3(kMfmaWaves * 64),
                           p.smem, stream, x, M, w, s, out, N, K, p.S, p.GS, partial, counters,
                           residual, cm);
    return hip_status(hipGetLastError(), "mfma gemm launch");
}

/* M <= 16 rows of x against a tile-order weight. */
template <int OUT>
int launch_mfma(const uint16_t *x, int M, const uint8_t *w, const uint16_t *s, void *out, int N,
                int K, hipStream_t stream, uint16_t *residual = nullptr, int cm = 0) {
    const MfmaPlan p = plan_mfma(M, N, K);
    uint64_t *partial = nullptr;
    unsigned *counters = nullptr;
    if (p.S > 1) {
        int st = split_scratch(p.partial_bytes, p.ncounters, &partial, &counters);
        if (st) return st;
    }
    switch (p.xpre) {
        case 1: return launch_mfma_x<OUT, 1>(p, x, M, w, s, out, N, K, partial, counters, stream, residual, cm);
        case 2: return launch_mfma_x<OUT, 2>(p, x, M, w, s, out, N, K, partial, counters, stream, residual, cm);
        case 4: return launch_mfma_x<OUT, 4>(p, x, M, w, s, out, N, K, partial, counters, stream, residual, cm);
        default: return launch_mfma_x<OUT, 8>(p, x, M, w, s, out, N, K, partial, counters, stream, residual, cm);
    }
}

/* Every device buffer of the compute entry points starts on a 16-byte boundary: the kernels
 * move 16 bytes a lane (buffer and direct-to-LDS loads). Allocator pointers always do. */
bool misaligned(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) != 0; }

/* Whether byte ranges [a, a + an) and [b, b + bn) share a byte. A kernel that reads one while
 * its other blocks write the other would race, so such pairs are refused. */
bool overlap(const void *a, size_t an, const void *b, size_t bn) {
    const uintptr_t x = reinterpret_cast<uintptr_t>(a), y = reinterpret_cast<uintptr_t>(b);
    return an && bn && x < y + bn && y < x + an;
}

/* Shape refusals of the reference wrapper (csrc/kernels/gemm_quant.cu:204-231), plus the
 * tile rules this layout adds (N % 8, group == 128) and 16-byte aligned buffers. */
int check_gemm_args(const void *a, const void *p, const void *s, const void *o, int M, int N,
                    int K, int group, const char *what, size_t out_bytes = 0) {
    if (M < 0 || N < 0 || K <= 0 || group <= 0)
        return set_error(W4A16_ERR_CONFIG, "%s: negative extent or nonpositive group", what);
    if (M == 0 || N == 0) return 1; /* no-op */
    if (!a || !p || !s || !o) return set_error(W4A16_ERR_CONFIG, "%s: a device pointer is null", what);
    if (misaligned(a) || misaligned(p) || misaligned(s) || misaligned(o))
        return set_error(W4A16_ERR_CONFIG, "%s: device buffers must be 16-byte aligned", what);
    if (K % group != 0)
        return set_error(W4A16_ERR_CONFIG, "%s: K=%d leaves a partial scale group of %d",
                         what, K, group);
    if (group % 8 != 0)
        return set_error(W4A16_ERR_CONFIG, "%s: group %d does not split into 8-code dwords", what,
                         group);
    if (group != W4A16_GROUP)
        return set_error(W4A16_ERR_CONFIG, "%s: the tile order holds 128-wide groups, not %d",
                         what, group);
    if (N % W4A16_TILE_ROWS != 0)
        return set_error(W4A16_ERR_CONFIG, "%s: N=%d rows do not fill 8-row tiles", what, N);
    if (M == 1 && K > kMaxRowK)
        return set_error(W4A16_ERR_CONFIG, "%s: K=%d at M=1 needs more than 96 KiB of activation "
                         "staging (max K %d)", what, K, kMaxRowK);
    if (K > kMaxAnyK)
        return set_error(W4A16_ERR_CONFIG, "%s: K=%d exceeds this build's limit %d", what, K,
                         kMaxAnyK);
    if ((unsigned long long)N * (unsigned long long)K / 2 >= (1ull << 32))
        return set_error(W4A16_ERR_CONFIG, "%s: a %d x %d operand exceeds the 4 GiB a buffer "
                         "descriptor addresses", what, N, K);
    const size_t wbytes = (size_t)N * K / 2, sbytes = (size_t)N * (K / 128) * 2;
    if (overlap(a, (size_t)M * K * 2, o, out_bytes) || overlap(p, wbytes, o, out_bytes) ||
        overlap(s, sbytes, o, out_bytes))
        return set_error(W4A16_ERR_CONFIG, "%s: the output overlaps an input", what);
    return 0;
}

}  // namespace

/* ---------------------------------------------------------------------------------------- */
/* C ABI                                                                                     */
/* ---------------------------------------------------------------------------------------- */

/* Rows of x: M = 1 takes the v_dot2 GEMV; 2 <= M <= 16 the few-row MFMA kernels where their
 * staged rows fit a block's LDS, otherwise the split-K MFMA form, one pass over the weight for
 * all rows; larger M runs on 16-row slices. */
template <int OUT>
static int run_rows(const uint16_t *x, int M, const uint8_t *w, const uint16_t *s, void *out,
                    int N, int K, hipStream_t stream, int cm = 0) {
    constexpr bool PAIR = OUT == kOutPairSilu;
    constexpr bool F32 = OUT == kOutF32;
    const int out_cols = PAIR ? N / 2 : N;
    const size_t out_elem = F32 ? 4 : 2;
    /* beyond 16 rows (no pair, row-major): all the 16-row slices in one launch of the
     * registers-fed kernel, and at exactly 16 rows where the LDS-staged kernel cannot hold K */
    if (!PAIR && !cm && M > 16) {
        const int st = launch_rows16w<F32>(x, M, w, s, out, N, K, stream);
        if (st <= 0) return st;
    }
    if (!PAIR && !cm && (M > 16 || (M == 16 && rows16_smem(16, K, 16) > kMaxLds))) {
        const int st = launch_rows16x<F32>(x, M, w, s, out, N, K, stream);
        if (st <= 0) return st;
    }
    for (int m0 = 0; m0 < M; m0 += 16) {
        const int rows = std::min(16, M - m0);
        const uint16_t *xs = x + (size_t)m0 * K;
        void *os = static_cast<char *>(out) + (size_t)m0 * out_cols * out_elem;
        /* one row: the v_dot2 GEMVs, except a pair operand past the block-staged kernel's K
         * (then the MFMA form with one live row) */
        const bool gemv = rows == 1 && (!PAIR || K <= kMaxGemvK);
        int st = gemv ? launch_gemv<PAIR, F32>(xs, w, s, os, N, K, stream)
                      : launch_rows<PAIR, F32>(xs, rows, w, s, os, N, K, stream, nullptr, cm);
        if (st > 0) st = launch_mfma<OUT>(xs, rows, w, s, os, N, K, stream, nullptr, cm);
        if (st) return st;
    }
    return W4A16_OK;
}

extern "C" int gemm_int4_bf16(const uint16_t *a, const uint8_t *packed, const uint16_t *scales,
                              uint16_t *out, int M, int N, int K, int group, void *stream) {
    int st = check_gemm_args(a, packed, scales, out, M, N, K, group, "gemm_int4_bf16",
                             (size_t)std::max(M, 0) * std::max(N, 0) * 2);
    if (st) return st > 0 ? W4A16_OK : st;
    return run_rows<kOutBf16>(a, M, packed, scales, out, N, K, static_cast<hipStream_t>(stream));
}

extern "C" int gate_up_silu_int4_bf16(const uint16_t *x, const uint8_t *gu_packed,
                                      const uint16_t *gu_scales, uint16_t *act, int M, int hidden,
                                      int inter, void *stream) {
    if (inter < 0) return set_error(W4A16_ERR_CONFIG, "gate_up_silu: negative intermediate");
    int st = check_gemm_args(x, gu_packed, gu_scales, act, M, 2 * inter, hidden, W4A16_GROUP,
                             "gate_up_silu_int4_bf16", (size_t)std::max(M, 0) * inter * 2);
    if (st) return st > 0 ? W4A16_OK : st;
    return run_rows<kOutPairSilu>(x, M, gu_packed, gu_scales, act, 2 * inter, hidden,
                                  static_cast<hipStream_t>(stream));
}

/* Inside the FFN entry points the gate/up kernel writes the intermediate chunk-major for a
 * down projection on gemv_rows16x_kernel<CM> when K is long (64 to 192 groups: at most 12 a
 * wave) and 4 <= M <= 16. C1 FFN call, interleaved runs, previous routes against this one:
 * M = 3 15.8 / 15.1-15.4 us (plan F2 18.3 / 18.6: not taken), 4 16.6 / 15.9, 6 18.8 / 16.7,
 * 8 20.0 / 17.4, 12 22.5 / 19.1, 16 24.4 / 20.1; M = 2 ties. */
static bool chunk_major_down(int M, int inter) {
    const int G = inter / W4A16_GROUP;
    return M >= 4 && M <= 16 && G >= 64 && G <= 192;
}

static int mlp_common(const uint16_t *normed, const uint8_t *gup, const uint16_t *gus,
                      const uint8_t *dnp, const uint16_t *dns, void *out, bool out_f32,
                      uint16_t *act, int M, int hidden, int inter, void *stream) {
    if (M < 0 || hidden <= 0 || inter <= 0)
        return set_error(W4A16_ERR_CONFIG, "mlp_int4: bad extents M=%d hidden=%d inter=%d", M,
                         hidden, inter);
    if (M == 0) return W4A16_OK;
    if (!act || !out) return set_error(W4A16_ERR_CONFIG, "mlp_int4: null buffer");
    int st = check_gemm_args(act, dnp, dns, out, M, hidden, inter, W4A16_GROUP, "mlp_int4 down",
                             (size_t)M * hidden * (out_f32 ? 4 : 2));
    if (st < 0) return st;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (chunk_major_down(M, inter)) {
        st = check_gemm_args(normed, gup, gus, act, M, 2 * inter, hidden, W4A16_GROUP,
                             "mlp_int4 gate/up", (size_t)M * inter * 2);
        if (st < 0) return st;
        st = run_rows<kOutPairSilu>(normed, M, gup, gus, act, 2 * inter, hidden, s, 1);
        if (st) return st;
        return out_f32 ? launch_rows16x<true, true>(act, M, dnp, dns, out, hidden, inter, s)
                       : launch_rows16x<false, true>(act, M, dnp, dns, out, hidden, inter, s);
    }
    st = gate_up_silu_int4_bf16(normed, gup, gus, act, M, hidden, inter, stream);
    if (st) return st;
    return out_f32 ? run_rows<kOutF32>(act, M, dnp, dns, out, hidden, inter, s)
                   : run_rows<kOutBf16>(act, M, dnp, dns, out, hidden, inter, s);
}

extern "C" int mlp_int4_bf16(const uint16_t *normed, const uint8_t *gup, const uint16_t *gus,
                             const uint8_t *dnp, const uint16_t *dns, uint16_t *out,
                             uint16_t *act_ws, int M, int hidden, int inter, void *stream) {
    return mlp_common(normed, gup, gus, dnp, dns, out, false, act_ws, M, hidden, inter, stream);
}

/* Grows the per-device split-K scratch (current device) to the worst case of every FFN call of
 * 1..max_rows rows at this shape, so that such calls never allocate afterwards. The loader calls
 * it once per store, outside any capture. */
int reserve_split_scratch(int max_rows, int hidden, int inter) {
    size_t pb = 0, nc = 0;
    for (int m = 1; m <= std::max(1, std::min(max_rows, 16)); ++m) {
        size_t a, b, c, d;
        split_bound(m, 2 * inter, hidden, &a, &b);
        split_bound(m, hidden, inter, &c, &d);
        pb = std::max(pb, std::max(a, c));
        nc = std::max(nc, std::max(b, d));
    }
    uint64_t *partial = nullptr;
    unsigned *counters = nullptr;
    return split_scratch(pb, nc, &partial, &counters);
}

extern "C" int mlp_int4_bf16_noalloc(const uint16_t *normed, const uint8_t *gup,
                                     const uint16_t *gus, const uint8_t *dnp, const uint16_t *dns,
                                     uint16_t *out, uint16_t *act_ws, int M, int hidden, int inter,
                                     void *stream) {
    if (M < 0 || hidden <= 0 || inter <= 0)
        return set_error(W4A16_ERR_CONFIG, "mlp_int4_bf16_noalloc: bad extents M=%d hidden=%d inter=%d",
                         M, hidden, inter);
    if (M == 0) return W4A16_OK;
    if ((long long)2 * inter > INT32_MAX)
        return set_error(W4A16_ERR_CONFIG, "mlp_int4_bf16_noalloc: intermediate %d too large", inter);
    size_t pb_gu, nc_gu, pb_dn, nc_dn;
    split_bound(M, 2 * inter, hidden, &pb_gu, &nc_gu);
    split_bound(M, hidden, inter, &pb_dn, &nc_dn);
    const size_t pb = std::max(pb_gu, pb_dn), nc = std::max(nc_gu, nc_dn);
    if (pb > kFixedPartialBytes || nc > kFixedCounters)
        return set_error(W4A16_ERR_CONFIG, "mlp_int4_bf16_noalloc: M=%d hidden=%d inter=%d may need %zu "
                         "bytes of split-K partials and %zu counters; the static scratch holds %zu "
                         "and %zu", M, hidden, inter, pb, nc, kFixedPartialBytes, kFixedCounters);
    hipStream_t s = static_cast<hipStream_t>(stream);
    unsigned char *base = nullptr;
    int st = fixed_scratch(s, &base);
    if (st) return st;
    t_fixed.partial = reinterpret_cast<uint64_t *>(base + kFixedCounters * 4);
    t_fixed.partial_bytes = kFixedPartialBytes;
    t_fixed.counters = reinterpret_cast<unsigned *>(base);
    t_fixed.ncounters = kFixedCounters;
    t_fixed.active = true;
    st = mlp_common(normed, gup, gus, dnp, dns, out, false, act_ws, M, hidden, inter, stream);
    t_fixed.active = false;
    return st;
}

extern "C" int mlp_int4_partial_f32(const uint16_t *normed, const uint8_t *gup,
                                    const uint16_t *gus, const uint8_t *dnp, const uint16_t *dns,
                                    float *out_f32, uint16_t *act_ws, int M, int hidden,
                                    int inter, void *stream) {
    return mlp_common(normed, gup, gus, dnp, dns, out_f32, true, act_ws, M, hidden, inter, stream);
}

/* ---- RMSNorm and the norm-fused MLP (reference forward_mlp, csrc/kernels/layers.cu:150-159) ---- */

static int norm_args(const uint16_t *w, int style, float eps, int cols, int rows, NormArgs *na,
                     const char *what) {
    if (rows < 0 || cols <= 0 || !std::isfinite(eps) || eps <= 0.0f)
        return set_error(W4A16_ERR_CONFIG, "%s: invalid shape or epsilon", what);
    if (style != 0 && style != 1)
        return set_error(W4A16_ERR_CONFIG, "%s: norm_style %d is neither 0 (gemma) nor 1 (plain)",
                         what, style);
    if (rows > 0 && !w) return set_error(W4A16_ERR_CONFIG, "%s: null norm weight", what);
    if (rows > 0 && misaligned(w))
        return set_error(W4A16_ERR_CONFIG, "%s: the norm weight must be 16-byte aligned", what);
    na->w = w;
    na->bias = style == 0 ? 1.0f : 0.0f;
    na->eps = eps;
    return W4A16_OK;
}

static int launch_rmsnorm(uint16_t *out, const uint16_t *x, const uint16_t *w, int cols, int rows,
                          float bias, float eps, hipStream_t s, const uint16_t *sub = nullptr) {
    const int ch = (cols / 8 + 255) / 256;
    if (cols % 8 || ch > 8)
        return set_error(W4A16_ERR_CONFIG, "rmsnorm: cols=%d must be a multiple of 8 and <= 16384",
                         cols);
    if (ch <= 1) launch_k(rmsnorm_kernel<1>, dim3(rows), dim3(256), 0, s, out, const_cast<uint16_t *>(x), w, cols, bias, eps, sub);
    else if (ch <= 2) launch_k(rmsnorm_kernel<2>, dim3(rows), dim3(256), 0, s, out, const_cast<uint16_t *>(x), w, cols, bias, eps, sub);
    else if (ch <= 4) launch_k(rmsnorm_kernel<4>, dim3(rows), dim3(256), 0, s, out, const_cast<uint16_t *>(x), w, cols, bias, eps, sub);
    else launch_k(rmsnorm_kernel<8>, dim3(rows), dim3(256), 0, s, out, const_cast<uint16_t *>(x), w, cols, bias, eps, sub);
    return hip_status(hipGetLastError(), "rmsnorm launch");
}

extern "C" int w4a16_rmsnorm_bf16(uint16_t *out, const uint16_t *x, const uint16_t *weight,
                                  int cols, int rows, int norm_style, float eps, void *stream) {
    NormArgs na;
    int st = norm_args(weight, norm_style, eps, cols, rows, &na, "w4a16_rmsnorm_bf16");
    if (st) return st;
    if (rows == 0) return W4A16_OK;
    if (!out || !x) return set_error(W4A16_ERR_CONFIG, "w4a16_rmsnorm_bf16: null buffer");
    if (misaligned(out) || misaligned(x))
        return set_error(W4A16_ERR_CONFIG, "w4a16_rmsnorm_bf16: buffers must be 16-byte aligned");
    return launch_rmsnorm(out, x, weight, cols, rows, na.bias, eps, static_cast<hipStream_t>(stream));
}

static int mlp_norm_common(const uint16_t *residual, const uint16_t *norm_w, int norm_style,
                           float eps, const uint8_t *gup, const uint16_t *gus, const uint8_t *dnp,
                           const uint16_t *dns, void *out, bool out_f32, uint16_t *ws, int M,
                           int hidden, int inter, void *stream) {
    if (M < 0 || hidden <= 0 || inter <= 0)
        return set_error(W4A16_ERR_CONFIG, "mlp_int4_norm: bad extents M=%d hidden=%d inter=%d", M,
                         hidden, inter);
    NormArgs na;
    int st = norm_args(norm_w, norm_style, eps, hidden, M, &na, "mlp_int4_norm");
    if (st) return st;
    if (M == 0) return W4A16_OK;
    if (!residual || !ws || !out) return set_error(W4A16_ERR_CONFIG, "mlp_int4_norm: null buffer");
    st = check_gemm_args(residual, gup, gus, ws, M, 2 * inter, hidden, W4A16_GROUP,
                         "mlp_int4_norm gate/up");
    if (st < 0) return st;
    st = check_gemm_args(ws, dnp, dns, out, M, hidden, inter, W4A16_GROUP, "mlp_int4_norm down");
    if (st < 0) return st;
    {
        const size_t ws_bytes = (size_t)M * (hidden + inter) * 2, row_bytes = (size_t)M * hidden * 2;
        if (overlap(residual, row_bytes, ws, ws_bytes) ||
            overlap(out, (size_t)M * hidden * (out_f32 ? 4 : 2), ws, ws_bytes) ||
            overlap(norm_w, (size_t)hidden * 2, ws, ws_bytes))
            return set_error(W4A16_ERR_CONFIG, "mlp_int4_norm: the workspace overlaps another buffer");
    }
    hipStream_t s = static_cast<hipStream_t>(stream);
    uint16_t *normed = ws;                          /* [M, hidden] (M > 1) */
    uint16_t *act = ws + (size_t)M * hidden;        /* [M, inter] */
    /* The prologue costs every gate/up block a normalisation of the whole row, so it pays only
     * while a block's waves each hold all of K, at one row (C1 norm + FFN 12.8 us fused against
     * 13.7 with a separate norm launch; at H = 5120 the separate launch is cheaper, 35.0 against
     * 38.4 us). At M = 2 the separate norm, then the two-row matrix-core kernels, beats the
     * few-row kernel's own prologue: C1 14.6-14.7 against 15.6-15.8 us, C2 38.3 against 42.8. */
    st = 1;
    if (M == 1 && (hidden / W4A16_GROUP + 1) / 2 <= kMaxLoads)
        st = launch_gemv<true, false>(residual, gup, gus, act, 2 * inter, hidden, s, &na);
    const bool cm = st > 0 && chunk_major_down(M, inter);
    if (st > 0) {
        st = launch_rmsnorm(normed, residual, norm_w, hidden, M, na.bias, eps, s);
        if (!st) st = run_rows<kOutPairSilu>(normed, M, gup, gus, act, 2 * inter, hidden, s, cm);
    }
    if (st) return st;
    if (cm)
        return out_f32 ? launch_rows16x<true, true>(act, M, dnp, dns, out, hidden, inter, s)
                       : launch_rows16x<false, true>(act, M, dnp, dns, out, hidden, inter, s);
    return out_f32 ? run_rows<kOutF32>(act, M, dnp, dns, out, hidden, inter, s)
                   : run_rows<kOutBf16>(act, M, dnp, dns, out, hidden, inter, s);
}

extern "C" int mlp_int4_norm_bf16(const uint16_t *residual, const uint16_t *norm_w,
                                  int norm_style, float eps, const uint8_t *gup,
                                  const uint16_t *gus, const uint8_t *dnp, const uint16_t *dns,
                                  uint16_t *out, uint16_t *ws, int M, int hidden, int inter,
                                  void *stream) {
    return mlp_norm_common(residual, norm_w, norm_style, eps, gup, gus, dnp, dns, out, false, ws,
                           M, hidden, inter, stream);
}

/* Plan F2 around the INT4 MLP (reference csrc/layer_dispatch.cu:183-209): residual <-
 * BF16(residual + sublayer); normed = RMSNorm(residual); out = MLP(normed); residual <-
 * BF16(residual + out). At M = 1 with a one-wave gate/up tile and a wave-local down kernel the
 * whole sequence is two launches: the gate/up kernel normalises BF16(residual + sublayer) in its
 * staging (writing nothing back, since every block reads the residual), and the down kernel's
 * epilogue forms both residual updates for its rows. Otherwise a norm kernel stores the first
 * update, and an add kernel the second. sublayer may alias out (as in the reference, where the
 * mixer output and the layer output share a buffer). */
extern "C" int mlp_int4_residual_norm_bf16(uint16_t *residual, const uint16_t *sublayer,
                                           const uint16_t *norm_w, int norm_style, float eps,
                                           const uint8_t *gup, const uint16_t *gus,
                                           const uint8_t *dnp, const uint16_t *dns, uint16_t *out,
                                           uint16_t *ws, int M, int hidden, int inter,
                                           void *stream) {
    if (M < 0 || hidden <= 0 || inter <= 0)
        return set_error(W4A16_ERR_CONFIG, "mlp_int4_residual_norm: bad extents M=%d hidden=%d inter=%d",
                         M, hidden, inter);
    NormArgs na;
    int st = norm_args(norm_w, norm_style, eps, hidden, M, &na, "mlp_int4_residual_norm");
    if (st) return st;
    if (M == 0) return W4A16_OK;
    if (!residual || !sublayer || !ws || !out)
        return set_error(W4A16_ERR_CONFIG, "mlp_int4_residual_norm: null buffer");
    if (misaligned(sublayer))
        return set_error(W4A16_ERR_CONFIG, "mlp_int4_residual_norm: the sublayer must be 16-byte aligned");
    if (hidden % 8)
        return set_error(W4A16_ERR_CONFIG, "mlp_int4_residual_norm: hidden=%d is not a multiple of 8",
                         hidden);
    st = check_gemm_args(residual, gup, gus, ws, M, 2 * inter, hidden, W4A16_GROUP,
                         "mlp_int4_residual_norm gate/up");
    if (st < 0) return st;
    st = check_gemm_args(ws, dnp, dns, out, M, hidden, inter, W4A16_GROUP,
                         "mlp_int4_residual_norm down");
    if (st < 0) return st;
    {
        const size_t ws_bytes = (size_t)M * (hidden + inter) * 2, row_bytes = (size_t)M * hidden * 2;
        if (overlap(residual, row_bytes, ws, ws_bytes) || overlap(sublayer, row_bytes, ws, ws_bytes) ||
            overlap(out, row_bytes, ws, ws_bytes) || overlap(norm_w, (size_t)hidden * 2, ws, ws_bytes))
            return set_error(W4A16_ERR_CONFIG,
                             "mlp_int4_residual_norm: the workspace overlaps another buffer");
        /* the sublayer may alias the output exactly (the reference's layer_out); the residual,
         * updated in place beside the output, may not overlap it */
        if (overlap(residual, row_bytes, out, row_bytes) ||
            (sublayer != out && overlap(sublayer, row_bytes, out, row_bytes)))
            return set_error(W4A16_ERR_CONFIG,
                             "mlp_int4_residual_norm: the output overlaps the residual or, other "
                             "than exactly, the sublayer");
    }
    hipStream_t s = static_cast<hipStream_t>(stream);
    uint16_t *normed = ws;
    uint16_t *act = ws + (size_t)M * hidden;
    const int gu_pairs = (hidden / W4A16_GROUP + 1) / 2;
    const int dn_pairs = (inter / W4A16_GROUP + 1) / 2;
    if (M == 1 && gu_pairs <= kMaxLoads && dn_pairs > kMaxLoads) {
        na.sub = sublayer;
        st = launch_gemv<true, false>(residual, gup, gus, act, 2 * inter, hidden, s, &na);
        if (st) return st;
        st = launch_xwave<false>(act, dnp, dns, out, hidden, inter, s, residual, sublayer);
        if (st <= 0) return st;
        return set_error(W4A16_ERR_CONFIG, "mlp_int4_residual_norm: K=%d beyond the down kernels",
                         inter);
    }
    const bool cm = chunk_major_down(M, inter);
    st = launch_rmsnorm(normed, residual, norm_w, hidden, M, na.bias, eps, s, sublayer);
    if (!st) st = run_rows<kOutPairSilu>(normed, M, gup, gus, act, 2 * inter, hidden, s, cm);
    if (st) return st;
    if (cm) return launch_rows16x<false, true>(act, M, dnp, dns, out, hidden, inter, s, residual);
    if (M == 1 && dn_pairs > kMaxLoads) {
        /* the down kernel adds the output into the (already updated) residual itself */
        st = launch_xwave<false>(act, dnp, dns, out, hidden, inter, s, residual, nullptr);
        if (st <= 0) return st;
    }
    if (M >= 2 && M <= 16) { /* the few-row or MFMA down kernel adds into the residual */
        st = launch_rows<false, false>(act, M, dnp, dns, out, hidden, inter, s, residual);
        if (st > 0) st = launch_mfma<kOutBf16>(act, M, dnp, dns, out, hidden, inter, s, residual);
        return st;
    }
    st = run_rows<kOutBf16>(act, M, dnp, dns, out, hidden, inter, s);
    if (st) return st;
    const long long chunks = (long long)M * hidden / 8;
    launch_k(residual_add_kernel, dim3((unsigned)((chunks + 255) / 256)), dim3(256), 0, s,
                       residual, out, chunks);
    return hip_status(hipGetLastError(), "residual add launch");
}

extern "C" int mlp_int4_norm_partial_f32(const uint16_t *residual, const uint16_t *norm_w,
                                         int norm_style, float eps, const uint8_t *gup,
                                         const uint16_t *gus, const uint8_t *dnp,
                                         const uint16_t *dns, float *out_f32, uint16_t *ws, int M,
                                         int hidden, int inter, void *stream) {
    return mlp_norm_common(residual, norm_w, norm_style, eps, gup, gus, dnp, dns, out_f32, true,
                           ws, M, hidden, inter, stream);
}

extern "C" int silu_mul_packed_bf16(uint16_t *out, const uint16_t *packed, int tokens, int inter,
                                    void *stream) {
    if (tokens < 0 || inter < 0)
        return set_error(W4A16_ERR_CONFIG, "silu_mul_packed: negative extent");
    if (tokens == 0 || inter == 0) return W4A16_OK;
    if (!out || !packed) return set_error(W4A16_ERR_CONFIG, "silu_mul_packed: null buffer");
    if (misaligned(out) || misaligned(packed))
        return set_error(W4A16_ERR_CONFIG, "silu_mul_packed: buffers must be 16-byte aligned");
    const int block = 256;
    launch_k(silu_mul_packed_kernel, dim3((inter + block - 1) / block, tokens),
                       dim3(block), 0, static_cast<hipStream_t>(stream), out, packed, tokens,
                       inter);
    return hip_status(hipGetLastError(), "silu_mul_packed launch");
}

extern "C" int w4a16_tile_pack_device(long long n, long long k, int pair, const uint8_t *packed,
                                      const uint16_t *scales, uint8_t *packed_tiled,
                                      uint16_t *scales_tiled, void *stream) {
    if (!packed || !scales || !packed_tiled || !scales_tiled)
        return set_error(W4A16_ERR_CONFIG, "tile_pack_device: null argument");
    if (misaligned(packed) || misaligned(scales) || misaligned(packed_tiled) || misaligned(scales_tiled))
        return set_error(W4A16_ERR_CONFIG, "tile_pack_device: device buffers must be 16-byte aligned");
    int st = w4a16_layout_init(n, k, W4A16_GROUP, nullptr, nullptr);
    if (st) return st;
    if (pair != 0 && pair != 1) return set_error(W4A16_ERR_CONFIG, "tile_pack_device: bad pair");
    const long long total = (n / 8) * (k / 128) * 128;
    launch_k(tile_pack_kernel, dim3(grid_for(total, 256)), dim3(256), 0,
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
    if (misaligned(packed_tiled) || misaligned(scales_tiled) || misaligned(out))
        return set_error(W4A16_ERR_CONFIG, "dequant_tiled_device: device buffers must be 16-byte aligned");
    int st = w4a16_layout_init(n, k, W4A16_GROUP, nullptr, nullptr);
    if (st) return st;
    if (pair != 0 && pair != 1) return set_error(W4A16_ERR_CONFIG, "dequant_tiled: bad pair");
    const long long total = (n / 8) * (k / 128) * 128;
    launch_k(dequant_tiled_kernel, dim3(grid_for(total, 256)), dim3(256), 0,
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
    if (misaligned(weights) || misaligned(packed) || misaligned(scales) || misaligned(status_dev))
        return set_error(W4A16_ERR_CONFIG, "quantize_device: device buffers must be 16-byte aligned");
    int st = w4a16_layout_init(n, k, W4A16_GROUP, nullptr, nullptr);
    if (st) return st;
    const long long total = n * (k / 128);
    launch_k(quantize_kernel, dim3(grid_for(total, 256)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), weights, packed, scales, status_dev, n,
                       k);
    return hip_status(hipGetLastError(), "quantize launch");
}

/* ---------------------------------------------------------------------------------------- */
/* Status of the bounded split-K waits                                                      */
/* ---------------------------------------------------------------------------------------- */

extern "C" int w4a16_split_wait_status(void *stream) {
    hipStream_t s = (hipStream_t)stream;
    unsigned count = 0;
    int st = hip_status(hipMemcpyFromSymbolAsync(&count, HIP_SYMBOL(g_slot_wait_timeouts),
                                                 sizeof(count), 0, hipMemcpyDeviceToHost, s),
                        "split_wait_status read");
    if (st) return st;
    if ((st = hip_status(hipStreamSynchronize(s), "split_wait_status sync"))) return st;
    if (count == 0) return W4A16_OK;
    const unsigned zero = 0;
    st = hip_status(hipMemcpyToSymbolAsync(HIP_SYMBOL(g_slot_wait_timeouts), &zero, sizeof(zero),
                                           0, hipMemcpyHostToDevice, s),
                    "split_wait_status clear");
    if (!st) st = hip_status(hipStreamSynchronize(s), "split_wait_status sync");
    if (st) return st;
    return set_error(W4A16_ERR_HIP,
                     "split_wait_status: %u split-K combine wait(s) gave up on an unwritten "
                     "partial since the last check; outputs of the calls in between are wrong",
                     count);
}

extern "C" int w4a16_debug_slot_wait(void *slot, int polls, float *out, void *stream) {
    if (!slot || !out || polls < 0)
        return set_error(W4A16_ERR_CONFIG, "debug_slot_wait: null pointer or negative bound");
    if (misaligned(slot) || misaligned(out))
        return set_error(W4A16_ERR_CONFIG, "debug_slot_wait: device buffers must be 16-byte aligned");
    launch_k(slot_wait_probe_kernel, dim3(1), dim3(64), 0, (hipStream_t)stream,
                       reinterpret_cast<uint64_t *>(slot), polls, out);
    return hip_status(hipGetLastError(), "debug_slot_wait launch");
}

extern "C" int w4a16_time_next_launch(int skip, void *start_event, void *stop_event) {
    if (skip < 0) return set_error(W4A16_ERR_CONFIG, "time_next_launch: skip %d is negative", skip);
    t_launches_to_skip = skip;
    t_next_launch_events[0] = (hipEvent_t)start_event;
    t_next_launch_events[1] = (hipEvent_t)stop_event;
    return W4A16_OK;
}
