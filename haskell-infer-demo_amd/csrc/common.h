/*
 * common.h - Definitions shared by the host code and the gfx950 kernels.
 *
 * Tile order. An [N, K] INT4 weight (N % 8 == 0, K % 128 == 0) is stored on the device as
 * N/8 row tiles x K/128 groups "units" of 512 bytes, unit (t, g) at byte (t * G + g) * 512 with
 * G = K/128, so one tile's groups are contiguous. Inside a unit, 32 pieces of 16 bytes: piece
 * p = kb * 8 + r holds row r of the tile and, in its dword s (0..3), the eight codes
 * k = g*128 + 32*s + 8*kb + j, j = 0..7. Inside that dword the code for j = 2q sits at bits
 * [3+4q, 6+4q] and the code for j = 2q+1 at bits [19+4q, 22+4q], modulo 32 (the dword is rotated
 * left by 3 bits, so the code j = 7 occupies bits 31 and 0-2), so a mask, after no shift for
 * q = 0, a shift for q = 1, 2 and a rotation for q = 3, puts the pair (k, k+1) at bits 3-6 of the
 * two halves of a register, which is the operand shape of the packed BF16 dot product and of
 * the MFMA B operand. A wave's 64 lanes, each loading one
 * 16-byte piece, read 1 KiB contiguous (two units of one tile).
 *
 * The BF16 scales follow the same unit order: scale (t, g, r) at index (t * G + g) * 8 + r.
 *
 * For the F1 gate/up pair ([2I, K], gate rows then up rows), tile t holds gate rows 4t..4t+3
 * in r = 0..3 and up rows 4t..4t+3 in r = 4..7, so one tile produces four SiLU(gate) x up
 * outputs. The nibble values themselves are never changed: the re-layout is a permutation.
 */
#ifndef W4A16_COMMON_H
#define W4A16_COMMON_H

#include <cmath>
#include <cstdint>
#include <cstring>

#include "../../include/w4a16.h"

#if defined(__HIP__) || defined(__HIPCC__)
#define W4A16_HD __host__ __device__ inline
#else
#define W4A16_HD inline
#endif

namespace w4a16 {

int set_error(int status, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();
const char *error_text(); /* the calling thread's last reason (what w4a16_last_error returns) */

/* BF16 round-to-nearest-even of an FP32 bit pattern (the format's own rounding rule,
 * reference csrc/linear_weight.cpp:34-44). */
W4A16_HD uint16_t bf16_rne(float v) {
    uint32_t u;
    std::memcpy(&u, &v, 4);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

W4A16_HD float bf16_widen(uint16_t b) {
    const uint32_t u = (uint32_t)b << 16;
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

/* Two's-complement nibble -> code in [-8, 7]. */
W4A16_HD int nibble_code(int nib) { return nib >= 8 ? nib - 16 : nib; }

/* q = clip(round_half_even(w / s), -7, 7) (reference csrc/linear_weight.cpp:159-163). */
W4A16_HD int quant_code(float w, float s) {
    float q = rintf(w / s);
    q = q > 7.0f ? 7.0f : q;
    q = q < -7.0f ? -7.0f : q;
    return (int)q;
}

/* Row of the source (artifact) weight that tile t, tile row r holds. */
W4A16_HD long long tile_source_row(long long t, int r, long long n, int pair) {
    if (!pair) return 8 * t + r;
    return r < 4 ? 4 * t + r : n / 2 + 4 * t + (r - 4);
}

/* Index (in dwords) of dword s of piece (kb, r) of unit (t, g). */
W4A16_HD long long tile_dword_index(long long t, long long g, long long groups, int kb, int r,
                                    int s) {
    return (((t * groups + g) * 32 + kb * 8 + r) << 2) + s;
}

/* Artifact word (nibble j of eight consecutive codes at bits 4j) -> tile word (even j at
 * 3 + 4*(j/2), odd j at 19 + 4*(j/2), modulo 32), and back. */
W4A16_HD uint32_t spread_nibbles(uint32_t w) {
    uint32_t out = 0;
    for (int q = 0; q < 4; ++q) {
        out |= ((w >> (8 * q)) & 0xFu) << (4 * q);
        out |= ((w >> (8 * q + 4)) & 0xFu) << (16 + 4 * q);
    }
    return (out << 3) | (out >> 29);
}

W4A16_HD uint32_t gather_nibbles(uint32_t t) {
    t = (t >> 3) | (t << 29);
    uint32_t out = 0;
    for (int q = 0; q < 4; ++q) {
        out |= ((t >> (4 * q)) & 0xFu) << (8 * q);
        out |= ((t >> (16 + 4 * q)) & 0xFu) << (8 * q + 4);
    }
    return out;
}

}  // namespace w4a16

#endif /* W4A16_COMMON_H */
