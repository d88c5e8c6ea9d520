/*
 * format.cpp - Host side of the INT4 artifact format and of the tile order (CPU only).
 *
 * The artifact format is the reference's (csrc/include/linear_weight.h:5-13); this file is the
 * product's own implementation of its converter-side arithmetic (quantize, dequantize, shape
 * rule) and of the host half of the re-layout the loader performs before upload.
 */
#include "common.h"

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

namespace w4a16 {

static thread_local char t_error[512];

int set_error(int status, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(t_error, sizeof(t_error), fmt, ap);
    va_end(ap);
    return status;
}

void clear_error() { t_error[0] = '\0'; }

const char *error_text() { return t_error; }

}  // namespace w4a16

using namespace w4a16;

extern "C" const char *w4a16_last_error(void) { return error_text(); }

/* ---------------------------------------------------------------------------------------- */
/* BF16 and the shape rule                                                                   */
/* ---------------------------------------------------------------------------------------- */

extern "C" int w4a16_abi_version(void) { return W4A16_ABI_VERSION; }

extern "C" uint16_t w4a16_f32_to_bf16(float value) { return bf16_rne(value); }

extern "C" float w4a16_bf16_to_f32(uint16_t bits) { return bf16_widen(bits); }

/* reference csrc/linear_weight.cpp:57-86 */
extern "C" int w4a16_layout_init(long long n, long long k, long long group,
                                 long long *packed_bytes, long long *scale_count) {
    if (n <= 0 || k <= 0)
        return set_error(W4A16_ERR_CONFIG, "layout: shape %lld x %lld has an empty or negative side", n, k);
    if (group != W4A16_GROUP)
        return set_error(W4A16_ERR_CONFIG,
                         "layout: group %lld requested; the INT4 artifact format is fixed at %d "
                         "values per scale", group, W4A16_GROUP);
    if (k % group != 0)
        return set_error(W4A16_ERR_CONFIG,
                         "layout: K=%lld leaves a partial scale group (K %% %lld = %lld)", k, group,
                         k % group);
    if (n % W4A16_TILE_ROWS != 0)
        return set_error(W4A16_ERR_CONFIG, "layout: N=%lld rows do not fill %d-row tiles (N %% %d = %lld)",
                         n, W4A16_TILE_ROWS, W4A16_TILE_ROWS, n % W4A16_TILE_ROWS);
    if (packed_bytes) *packed_bytes = n * k / 2;
    if (scale_count) *scale_count = n * (k / group);
    return W4A16_OK;
}

/* ---------------------------------------------------------------------------------------- */
/* Quantize / dequantize (reference csrc/linear_weight.cpp:108-216)                         */
/* ---------------------------------------------------------------------------------------- */

extern "C" int w4a16_quantize_int4(long long n, long long k, const float *weights,
                                   uint8_t *packed, uint16_t *scales) {
    if (!weights || !packed || !scales) return set_error(W4A16_ERR_CONFIG, "quantize: null argument");
    long long pbytes = 0, nscales = 0;
    int st = w4a16_layout_init(n, k, W4A16_GROUP, &pbytes, &nscales);
    if (st) return st;
    const long long groups = k / W4A16_GROUP;
    for (long long i = 0; i < n * k; ++i)
        if (!std::isfinite(weights[i]))
            return set_error(W4A16_ERR_CONFIG, "quantize: weight %lld (row %lld) is NaN or infinite", i, i / k);
    /* Every group's scale is derived (and checked) before any output byte is written, so a
     * refusal leaves the caller's buffers as they were. */
    std::vector<uint16_t> sc((size_t)nscales);
    for (long long row = 0; row < n; ++row) {
        for (long long g = 0; g < groups; ++g) {
            const float *w = weights + row * k + g * W4A16_GROUP;
            float peak = 0.0f;
            for (int i = 0; i < W4A16_GROUP; ++i) peak = std::fmax(peak, std::fabs(w[i]));
            const uint16_t bits = bf16_rne(peak > 0.0f ? peak / 7.0f : 1.0f);
            const float s = bf16_widen(bits);
            if (!(s > 0.0f) || !std::isfinite(s))
                return set_error(W4A16_ERR_CONFIG,
                                 "quantize: absmax/7 of row %lld group %lld becomes BF16 %g, "
                                 "unusable as a scale", row, g, (double)s);
            sc[(size_t)(row * groups + g)] = bits;
        }
    }
    for (long long row = 0; row < n; ++row) {
        const float *w = weights + row * k;
        uint8_t *dst = packed + row * (k / 2);
        for (long long c = 0; c < k; c += 2) {
            uint8_t byte = 0;
            for (int h = 0; h < 2; ++h) {
                const float s = bf16_widen(sc[(size_t)(row * groups + (c + h) / W4A16_GROUP)]);
                const int q = quant_code(w[c + h], s);
                byte |= (uint8_t)((q & 0xF) << (4 * h));
            }
            dst[c / 2] = byte;
        }
    }
    std::memcpy(scales, sc.data(), sc.size() * sizeof(uint16_t));
    return W4A16_OK;
}

extern "C" int w4a16_dequantize_int4(long long n, long long k, const uint8_t *packed,
                                     const uint16_t *scales, float *out) {
    if (!packed || !scales || !out) return set_error(W4A16_ERR_CONFIG, "dequantize: null argument");
    int st = w4a16_layout_init(n, k, W4A16_GROUP, nullptr, nullptr);
    if (st) return st;
    const long long groups = k / W4A16_GROUP;
    for (long long row = 0; row < n; ++row) {
        for (long long c = 0; c < k; ++c) {
            const float s = bf16_widen(scales[row * groups + c / W4A16_GROUP]);
            if (!(s > 0.0f) || !std::isfinite(s))
                return set_error(W4A16_ERR_WEIGHTS,
                                 "dequantize: scale of row %lld group %lld is zero, negative or "
                                 "non-finite", row, c / W4A16_GROUP);
            const int nib = (packed[(row * k + c) >> 1] >> (4 * (c & 1))) & 0xF;
            if (nib == 0x8)
                return set_error(W4A16_ERR_WEIGHTS,
                                 "dequantize: nibble 0x8 (code -8, never written by the "
                                 "quantizer) at row %lld column %lld", row, c);
            out[row * k + c] = (float)nibble_code(nib) * s;
        }
    }
    return W4A16_OK;
}

/* ---------------------------------------------------------------------------------------- */
/* Tile order (host)                                                                         */
/* ---------------------------------------------------------------------------------------- */

static int tile_args(long long n, long long k, int pair, const void *a, const void *b,
                     const void *c, const void *d, const char *what) {
    if (!a || !b || !c || !d) return set_error(W4A16_ERR_CONFIG, "%s: null argument", what);
    int st = w4a16_layout_init(n, k, W4A16_GROUP, nullptr, nullptr);
    if (st) return st;
    if (pair != 0 && pair != 1) return set_error(W4A16_ERR_CONFIG, "%s: pair must be 0 or 1", what);
    if (pair && (n % 8) != 0)
        return set_error(W4A16_ERR_CONFIG, "%s: a gate/up pair needs I %% 4 == 0 (n=%lld)", what, n);
    return W4A16_OK;
}

extern "C" int w4a16_tile_pack_host(long long n, long long k, int pair, const uint8_t *packed,
                                    const uint16_t *scales, uint8_t *packed_tiled,
                                    uint16_t *scales_tiled) {
    int st = tile_args(n, k, pair, packed, scales, packed_tiled, scales_tiled, "tile_pack_host");
    if (st) return st;
    const long long groups = k / W4A16_GROUP;
    const long long tiles = n / W4A16_TILE_ROWS;
    uint32_t *dst = reinterpret_cast<uint32_t *>(packed_tiled);
    for (long long t = 0; t < tiles; ++t) {
        for (int r = 0; r < W4A16_TILE_ROWS; ++r) {
            const long long row = tile_source_row(t, r, n, pair);
            const uint8_t *src = packed + row * (k / 2);
            for (long long g = 0; g < groups; ++g) {
                scales_tiled[(t * groups + g) * W4A16_TILE_ROWS + r] = scales[row * groups + g];
                for (int kb = 0; kb < 4; ++kb) {
                    for (int s = 0; s < 4; ++s) {
                        const long long c0 = g * W4A16_GROUP + 32 * s + 8 * kb;
                        uint32_t word;
                        std::memcpy(&word, src + c0 / 2, 4);
                        dst[tile_dword_index(t, g, groups, kb, r, s)] = spread_nibbles(word);
                    }
                }
            }
        }
    }
    return W4A16_OK;
}

extern "C" int w4a16_tile_unpack_host(long long n, long long k, int pair,
                                      const uint8_t *packed_tiled, const uint16_t *scales_tiled,
                                      uint8_t *packed, uint16_t *scales) {
    int st = tile_args(n, k, pair, packed_tiled, scales_tiled, packed, scales, "tile_unpack_host");
    if (st) return st;
    const long long groups = k / W4A16_GROUP;
    const long long tiles = n / W4A16_TILE_ROWS;
    const uint32_t *src = reinterpret_cast<const uint32_t *>(packed_tiled);
    for (long long t = 0; t < tiles; ++t) {
        for (int r = 0; r < W4A16_TILE_ROWS; ++r) {
            const long long row = tile_source_row(t, r, n, pair);
            uint8_t *dst = packed + row * (k / 2);
            for (long long g = 0; g < groups; ++g) {
                scales[row * groups + g] = scales_tiled[(t * groups + g) * W4A16_TILE_ROWS + r];
                for (int kb = 0; kb < 4; ++kb) {
                    for (int s = 0; s < 4; ++s) {
                        const long long c0 = g * W4A16_GROUP + 32 * s + 8 * kb;
                        const uint32_t word = gather_nibbles(src[tile_dword_index(t, g, groups, kb, r, s)]);
                        std::memcpy(dst + c0 / 2, &word, 4);
                    }
                }
            }
        }
    }
    return W4A16_OK;
}
