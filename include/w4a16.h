/*
 * w4a16.h - C ABI of the MI355X (gfx950) weight-only INT4 dense-FFN decode path.
 *
 * The artifact format is the reference's frozen INT4 format (reference
 * csrc/include/linear_weight.h:5-13): symmetric signed INT4 codes in 128-wide K groups, BF16
 * scales, two two's-complement nibbles per byte with the lower K index in the low nibble,
 * row-major packed [N, K/2] plus row-major scales [N, K/128]. Nothing here changes it.
 *
 * On the device the library keeps a re-laid copy ("tile order") of every weight: a pure
 * permutation of the nibbles and of the scales, chosen so one wave64 load instruction moves
 * 1 KiB of one 8-row tile and so the fused gate/up kernel sees gate row i and up row i in the
 * same tile. Compute entry points take device pointers in tile order; w4a16_tile_pack_* produce
 * it from the artifact layout, and w4a16_tile_unpack_host is the exact inverse.
 *
 * Conventions (all entry points):
 *   - BF16 tensors are passed as uint16_t bit patterns, FP32 as float.
 *   - Every function returns W4A16_OK (0) or a negative W4A16_ERR_* status and never throws;
 *     the reason is in the calling thread's w4a16_last_error().
 *   - `stream` is a hipStream_t (NULL = the default stream). Device entry points are
 *     asynchronous on it and perform no host synchronisation.
 *   - Device pointers must come from hipMalloc (or a torch CUDA tensor) on the current device
 *     and start on a 16-byte boundary (the kernels move 16 bytes a lane); a misaligned buffer
 *     is refused with W4A16_ERR_CONFIG before anything is launched. So is an output or
 *     workspace that overlaps a buffer the same call reads while writing it (plan F2's
 *     sublayer may alias its output exactly).
 *   - Compute calls that overlap in time on one device must be ordered on one stream: the
 *     split-K kernels of the small-M path share one per-device scratch buffer. The first call
 *     of a shape through the stateless entry points may grow that buffer (an allocation and a
 *     device synchronisation), so make it before capturing calls into a HIP graph, or use
 *     mlp_int4_bf16_noalloc, which never allocates. A store's loader reserves the buffer for
 *     every shape its forwards can take, so engine_ffn_forward* never allocate.
 */
#ifndef W4A16_H
#define W4A16_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes mirror the engine's ENGINE_* codes (reference csrc/include/engine.h:264-270). */
#define W4A16_OK 0
#define W4A16_ERR_HIP (-1)     /* HIP runtime error (reference ENGINE_ERR_CUDA) */
#define W4A16_ERR_ALLOC (-2)   /* device allocation failed */
#define W4A16_ERR_WEIGHTS (-3) /* artifact missing, malformed, hash or shape mismatch */
#define W4A16_ERR_CONFIG (-4)  /* invalid argument or unsupported shape */
#define W4A16_ERR_STATE (-5)   /* invalid handle state */

#define W4A16_GROUP 128
#define W4A16_TILE_ROWS 8

/* Version of this ABI (no reference counterpart). 2: W4A16EngineConfig gained its trailing
 * int4_max_rows field and the store handle is W4A16Store (was EngineHandle); a caller built
 * against version 1 passes a shorter config struct and must be rebuilt. w4a16_abi_version()
 * returns the version the library was built with, so a binding can refuse a mismatch. */
#define W4A16_ABI_VERSION 2
int w4a16_abi_version(void);

/* Thread-local reason for the last failure on this thread ("" if none).
 * Replaces linear_last_error / quant_manifest_last_error / engine_last_error
 * (reference csrc/linear_weight.cpp:16-28, csrc/quant_manifest.c:29-41). */
const char *w4a16_last_error(void);

/* ---------------------------------------------------------------------------------------
 * Format (host, CPU only). Same rules as the reference's linear_weight.h.
 * ------------------------------------------------------------------------------------- */

/* Extents of an [n, k] weight: refuses n,k <= 0, group != 128, k % 128, n % 8.
 * Replaces linear_layout_init (reference csrc/linear_weight.cpp:57-86). */
int w4a16_layout_init(long long n, long long k, long long group, long long *packed_bytes,
                      long long *scale_count);

/* BF16 round-to-nearest-even (reference csrc/linear_weight.cpp:34-51). */
uint16_t w4a16_f32_to_bf16(float value);
float w4a16_bf16_to_f32(uint16_t bits);

/* The converter's quantizer: FP32 [n, k] row-major -> artifact payload + BF16 scales.
 * Replaces linear_quantize_int4 (reference csrc/linear_weight.cpp:108-176). */
int w4a16_quantize_int4(long long n, long long k, const float *weights, uint8_t *packed,
                        uint16_t *scales);

/* The format's dequantizer (refuses nibble 0x8 and bad scales).
 * Replaces linear_dequantize_int4 (reference csrc/linear_weight.cpp:178-216). */
int w4a16_dequantize_int4(long long n, long long k, const uint8_t *packed,
                          const uint16_t *scales, float *out);

/* ---------------------------------------------------------------------------------------
 * Tile order (new; the reference uploads row-major: csrc/engine.cu:2370-2395).
 *
 * `pair` = 0: an ordinary [n, k] weight. `pair` = 1: the F1 gate/up pair [n = 2I, k] whose
 * rows 0..I-1 are gate and I..2I-1 are up (reference scripts/quantize_weights.py:236-276);
 * tile t then holds gate rows 4t..4t+3 and up rows 4t..4t+3 (needs I % 4 == 0).
 * Both buffers keep their artifact sizes (n*k/2 bytes and n*k/128 scales).
 * ------------------------------------------------------------------------------------- */
int w4a16_tile_pack_host(long long n, long long k, int pair, const uint8_t *packed,
                         const uint16_t *scales, uint8_t *packed_tiled, uint16_t *scales_tiled);
int w4a16_tile_unpack_host(long long n, long long k, int pair, const uint8_t *packed_tiled,
                           const uint16_t *scales_tiled, uint8_t *packed, uint16_t *scales);
/* The same permutation on the device (artifact layout already uploaded). */
int w4a16_tile_pack_device(long long n, long long k, int pair, const uint8_t *packed,
                           const uint16_t *scales, uint8_t *packed_tiled,
                           uint16_t *scales_tiled, void *stream);
/* Dequantize a tile-order weight to FP32 row-major [n, k] on the device: the check that the
 * re-laid operand is bit-exact with the format's dequantizer. */
int w4a16_dequant_tiled_device(long long n, long long k, int pair, const uint8_t *packed_tiled,
                               const uint16_t *scales_tiled, float *out, void *stream);
/* Quantize FP32 [n, k] on the device, bit-exact with w4a16_quantize_int4 (used to produce
 * large synthetic weight sets quickly). Writes the artifact (row-major) layout. Inputs must be
 * finite and every group's rounded scale positive; violations are reported through
 * `status_dev` (one int32 on the device, left 0 on success). */
int w4a16_quantize_device(long long n, long long k, const float *weights, uint8_t *packed,
                          uint16_t *scales, int *status_dev, void *stream);

/* ---------------------------------------------------------------------------------------
 * Compute (device pointers, tile order).
 * ------------------------------------------------------------------------------------- */

/* out[M, N] (BF16) = a[M, K] (BF16) x W^T, FP32 accumulation, W in tile order (pair = 0).
 * Same refusals as the reference wrapper: M,N < 0, K <= 0 or group <= 0; M == 0 or N == 0 is a
 * no-op; null buffers; K % group; group % 8; at M = 1, K * 2 > 96 KiB (K > 49152). The tile
 * order adds N % 8 and group == 128 (both always true of the format's artifacts), and this build
 * refuses K > 2^20 and an operand of 4 GiB or more. Replaces gemm_int4_bf16 (reference
 * csrc/include/layers.h:376-377, csrc/kernels/gemm_quant.cu:204-254), which throws instead. */
int gemm_int4_bf16(const uint16_t *a, const uint8_t *packed, const uint16_t *scales,
                   uint16_t *out, int M, int N, int K, int group, void *stream);

/* act[t, i] = BF16(silu(g) * u) over the row-interleaved [tokens, 2I] buffer.
 * Replaces kernel_silu_mul_packed (reference csrc/kernels/silu.cu:78-95). */
int silu_mul_packed_bf16(uint16_t *out, const uint16_t *packed, int tokens, int intermediate,
                         void *stream);

/* act[M, I] (BF16) = BF16(silu(BF16(x W_gate^T)) * BF16(x W_up^T)) from the gate/up pair in
 * tile order (pair = 1), one kernel: the [M, 2I] gate/up output never reaches memory. */
int gate_up_silu_int4_bf16(const uint16_t *x, const uint8_t *gu_packed,
                           const uint16_t *gu_scales, uint16_t *act, int M, int hidden,
                           int intermediate, void *stream);

/* The INT4 branch of the dense MLP (reference csrc/kernels/layers.cu:126-145): fused
 * gate/up/SiLU, then down. `act_ws` is caller workspace of M * intermediate BF16; it holds the
 * intermediate in the order the down kernel reads: row-major [M, I], except chunk-major
 * ([I / 8][M][8]) for 4 <= M <= 16 with I / 128 in 64..192. out [M, hidden] BF16. */
int mlp_int4_bf16(const uint16_t *normed, const uint8_t *gu_packed, const uint16_t *gu_scales,
                  const uint8_t *dn_packed, const uint16_t *dn_scales, uint16_t *out,
                  uint16_t *act_ws, int M, int hidden, int intermediate, void *stream);

/* No counterpart in the reference: mlp_int4_bf16 for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). Same
 * arguments, kernels and results; the split-K partials and counters live in a static device
 * array of the library (256 KiB of counters and 32 MiB of partial slots a GPU, held until the
 * process ends) instead of the growable per-device buffer, so no call allocates or
 * synchronises. Shapes whose worst-case split-K need exceeds that array are refused with
 * W4A16_ERR_CONFIG before anything is launched (every BASELINE shape up to M = 16 fits). The
 * first call on a device looks the array up and clears the array with a kernel on `stream`.
 * Every call on one GPU shares the array: calls that overlap in time on one GPU race, so order
 * them on one stream. */
int mlp_int4_bf16_noalloc(const uint16_t *normed, const uint8_t *gu_packed,
                          const uint16_t *gu_scales, const uint8_t *dn_packed,
                          const uint16_t *dn_scales, uint16_t *out, uint16_t *act_ws, int M,
                          int hidden, int intermediate, void *stream);

/* Tensor-parallel slice: as mlp_int4_bf16, but the down projection's FP32 partial is written
 * unrounded (out_f32 [M, hidden]), to be summed across ranks before rounding. */
int mlp_int4_partial_f32(const uint16_t *normed, const uint8_t *gu_packed,
                         const uint16_t *gu_scales, const uint8_t *dn_packed,
                         const uint16_t *dn_scales, float *out_f32, uint16_t *act_ws, int M,
                         int hidden, int intermediate, void *stream);

/* RMSNorm of `rows` rows of `cols` BF16 values: out = BF16(x * rsqrt(mean(x^2) + eps) * (b + w)),
 * b = 1 for norm_style 0 (Gemma, weight + 1) and 0 for norm_style 1 (plain); the sum of
 * squares in FP64, the scale rounded once to FP32, the products in FP32.
 * Replaces kernel_gemma_rms_norm / kernel_rms_norm_plain (reference
 * csrc/kernels/flashinfer_norm.cu:22-76, chosen by layer_norm, csrc/kernels/layers.cu:16-25),
 * with their refusals (rows < 0, cols <= 0, eps not finite and positive; rows == 0 no-op), plus
 * this kernel's own: cols a multiple of 8 and at most 16384, rows 16-byte aligned. */
int w4a16_rmsnorm_bf16(uint16_t *out, const uint16_t *x, const uint16_t *weight, int cols,
                       int rows, int norm_style, float eps, void *stream);

/* forward_mlp (reference csrc/kernels/layers.cu:150-159): the post-attention RMSNorm of the
 * residual [M, hidden], then the INT4 MLP. At M = 1 (hidden up to 3072) the norm is formed
 * inside the gate/up kernel's activation staging (no separate launch, no normed round trip;
 * the normed part of ws is then left unwritten); other M normalise into ws first. ws: M * (hidden +
 * intermediate) BF16 (normed, then act in the order mlp_int4_bf16 gives it). The norm's scale is rounded once to FP32 from an FP64
 * sum of squares; the products are FlashInfer's FP32 ones in its order. */
int mlp_int4_norm_bf16(const uint16_t *residual, const uint16_t *norm_w, int norm_style,
                       float eps, const uint8_t *gu_packed, const uint16_t *gu_scales,
                       const uint8_t *dn_packed, const uint16_t *dn_scales, uint16_t *out,
                       uint16_t *ws, int M, int hidden, int intermediate, void *stream);

/* Plan F2 around the INT4 MLP (reference csrc/layer_dispatch.cu:183-209 with
 * kernel_residual_norm, csrc/kernels/flashinfer_norm.cu:111-175, and kernel_residual_add,
 * csrc/kernels/gdn_norm.cu:121-136), for a dense layer without tensor parallelism:
 *   residual <- BF16(residual + sublayer); out = MLP(RMSNorm(residual));
 *   residual <- BF16(residual + out).
 * residual [M, hidden] is updated in place; sublayer may alias out. ws as mlp_int4_norm_bf16.
 * At M = 1 this is two launches (the norm in the gate/up staging, both residual updates in the
 * down projection's epilogue). */
int mlp_int4_residual_norm_bf16(uint16_t *residual, const uint16_t *sublayer,
                                const uint16_t *norm_w, int norm_style, float eps,
                                const uint8_t *gu_packed, const uint16_t *gu_scales,
                                const uint8_t *dn_packed, const uint16_t *dn_scales,
                                uint16_t *out, uint16_t *ws, int M, int hidden, int intermediate,
                                void *stream);

/* Same, with the tensor-parallel FP32 partial of the down projection (as mlp_int4_partial_f32). */
int mlp_int4_norm_partial_f32(const uint16_t *residual, const uint16_t *norm_w, int norm_style,
                              float eps, const uint8_t *gu_packed, const uint16_t *gu_scales,
                              const uint8_t *dn_packed, const uint16_t *dn_scales,
                              float *out_f32, uint16_t *ws, int M, int hidden, int intermediate,
                              void *stream);

/* ---------------------------------------------------------------------------------------
 * Sidecar and artifacts (host). Status values are the reference reader's QuantManifestStatus
 * (reference csrc/include/quant_manifest.h:55-63): 0 ok, 1 arg, 2 syntax, 3 format, 4 shape,
 * 5 io, 6 hash; the reason is in w4a16_last_error().
 * ------------------------------------------------------------------------------------- */

/* Parse and validate a weights.manifest.json document (no file access). Replaces
 * quant_manifest_parse (reference csrc/quant_manifest.c:895-1063). */
int w4a16_manifest_check(const char *json, int *entries, int *pairs);

/* Read root/file, requiring `bytes`, the dtype and the SHA-256 the manifest recorded. Replaces
 * quant_artifact_read (reference csrc/quant_manifest.c:1085-1139). */
int w4a16_artifact_verify(const char *root, const char *file, const char *dtype, long long bytes,
                          const char *sha256_hex, const char *want_dtype);

/* Lowercase hex SHA-256 of a buffer into out_hex65 (64 digits + NUL). Replaces sha256_hex
 * (reference csrc/include/sha256.h:41). */
int w4a16_sha256_hex(const void *data, size_t len, char *out_hex65);

/* ---------------------------------------------------------------------------------------
 * The INT4 FFN operand store (load and decode dispatch).
 * ------------------------------------------------------------------------------------- */

/* The store's handle. It carries the part of the reference engine that the INT4 path reads:
 * the descriptor's dense layers and FFN sizes, the tensor-parallel degree and this handle's
 * rank (one handle per GPU), the device it was created on, and the device operands it loads.
 * Its type name is the library's own: the reference engine's opaque EngineHandle is a
 * different struct, and an engine that holds one store per device keeps both side by side. */
typedef struct W4A16Store W4A16Store;

typedef struct W4A16EngineConfig {
    int num_layers;
    const unsigned char *layer_is_dense; /* num_layers flags; NULL = every layer dense */
    int hidden;                          /* hidden_size */
    int intermediate;                    /* the checkpoint's full intermediate_size */
    int tp_size;                         /* replicated tensor parallelism degree */
    int tp_rank;                         /* this handle's rank */
    int ep_size;                         /* expert parallelism (> 1 is refused at load) */
    int max_tokens;                      /* workspace rows: the largest M a forward accepts */
    int int4_max_rows;                   /* verify rows routed to INT4 (0 = 1, decode only) */
} W4A16EngineConfig;

/* Device operands of one layer, in tile order (the reference's LayerWeights::{gate_up_i4,
 * gate_up_i4_scales, down_i4, down_i4_scales, i4_group}, reference csrc/include/layers.h:158-165). */
typedef struct W4A16FfnOperands {
    const uint8_t *gate_up_packed;
    const uint16_t *gate_up_scales;
    const uint8_t *down_packed;
    const uint16_t *down_scales;
    int hidden;
    int intermediate; /* this rank's share */
    int group;
} W4A16FfnOperands;

/* No reference counterpart: the reference engine_create (csrc/include/engine.h:69-72) builds
 * these fields from its descriptor. The store belongs to the device current at this call; the
 * device entry points below refuse to run it from another. int4_max_rows must lie in
 * 0..min(16, max_tokens). NULL on a bad configuration (w4a16_last_error()). */
W4A16Store *w4a16_engine_create(const W4A16EngineConfig *cfg);
void w4a16_engine_destroy(W4A16Store *store);

/* Load the INT4 operands of every dense layer from manifest_dir (weights.manifest.json + the
 * artifacts it names): validated, SHA-256 checked, sliced to this rank with the global scales,
 * uploaded and re-laid on the store's device; all-or-nothing. W4A16_OK, W4A16_ERR_CONFIG for a
 * null argument, otherwise W4A16_ERR_WEIGHTS with the reason in w4a16_last_error().
 * The loader of reference csrc/engine.cu:2207-2428, for an engine that defines the public
 * engine_load_quantized_ffn itself and calls this per rank from inside it. */
int w4a16_load_quantized_ffn(W4A16Store *store, const char *manifest_dir);

/* Standalone aliases, for a caller with no engine of its own (a Haskell program or a ctypes
 * harness linking only this library): the same loader under the reference's public name
 * (reference csrc/include/engine.h:98, src/Infer/FFI/Engine.hs:114-115), its handle argument
 * being this library's store, and the thread's last failure under the engine's name. Inside the
 * library nothing calls either name: the library binds its own calls locally, so an engine
 * whose definitions of these names come first in the load order (and call
 * w4a16_load_quantized_ffn) cannot be re-entered by them. Translation units that also see the
 * engine's engine.h define W4A16_NO_ENGINE_ALIASES before including this header. */
#ifndef W4A16_NO_ENGINE_ALIASES
int engine_load_quantized_ffn(W4A16Store *store, const char *manifest_dir);
const char *engine_last_error(void);
#endif

/* The INT4 routing predicate of mlp_from_normed (reference csrc/kernels/layers.cu:126, there
 * `tokens == 1 && gate_up_i4 && down_i4`): 1 if `layer` holds INT4 operands and either
 * tokens == 1 (decode) or verify_rows is nonzero and tokens <= the store's int4_max_rows
 * (speculative verification); 0 otherwise, so prefill (verify_rows = 0, tokens > 1) stays on
 * the engine's BF16 weights and its logits stay bit-identical to a BF16-only engine's. */
int engine_ffn_routes_int4(const W4A16Store *store, int layer, int tokens, int verify_rows);

/* Number of dense layers holding INT4 operands (the reference's quantized_ffn_layers). */
int engine_quantized_ffn_layers(const W4A16Store *store);

/* The layer's device operands (W4A16_ERR_STATE if the layer has none). */
int engine_ffn_operands(const W4A16Store *store, int layer, W4A16FfnOperands *out);

/* The INT4 branch of forward_mlp_prepared for one layer (reference csrc/kernels/layers.cu:126-145
 * and 163-169): normed [tokens, hidden] BF16 -> out [tokens, hidden] BF16 on `stream`, using the
 * handle's workspace. Every forward below refuses (W4A16_ERR_CONFIG, before any launch) tokens
 * above max(1, int4_max_rows), and a call made while another device than the store's is current.
 * Under tensor parallelism the _partial_f32 form returns this rank's FP32
 * down-projection partial, to be summed across ranks before rounding. */
int engine_ffn_forward(W4A16Store *store, int layer, const uint16_t *normed, uint16_t *out,
                       int tokens, void *stream);
int engine_ffn_forward_partial_f32(W4A16Store *store, int layer, const uint16_t *normed,
                                   float *out, int tokens, void *stream);

/* forward_mlp (reference csrc/kernels/layers.cu:150-159) on a loaded layer: the post-attention
 * RMSNorm of residual [tokens, hidden] with the caller's norm weight (LayerWeights::post_norm_w,
 * kept by the engine with its BF16 weights; style and eps as ModelDims::norm_style / rms_eps),
 * then the INT4 MLP (see mlp_int4_norm_bf16). */
int engine_ffn_forward_norm(W4A16Store *store, int layer, const uint16_t *residual,
                            const uint16_t *norm_w, int norm_style, float eps, uint16_t *out,
                            int tokens, void *stream);
int engine_ffn_forward_norm_partial_f32(W4A16Store *store, int layer, const uint16_t *residual,
                                        const uint16_t *norm_w, int norm_style, float eps,
                                        float *out, int tokens, void *stream);

/* Plan F2 on a loaded layer (see mlp_int4_residual_norm_bf16); refused under tensor parallelism,
 * where the residual add follows the cross-rank sum (reference csrc/layer_dispatch.cu:166-169). */
int engine_ffn_forward_residual_norm(W4A16Store *store, int layer, uint16_t *residual,
                                     const uint16_t *sublayer, const uint16_t *norm_w,
                                     int norm_style, float eps, uint16_t *out, int tokens,
                                     void *stream);

/* ---------------------------------------------------------------------------------------
 * Status of the split-K combines (no counterpart in the reference, whose kernels have no
 * cross-block waits).
 *
 * The split-K kernels finish a tile in the last of its blocks to arrive, which waits (bounded)
 * for each partner's partial. A wait that gives up leaves a wrong output and counts itself in a
 * per-device word. w4a16_split_wait_status synchronises `stream`, reads and clears the current
 * device's word, and returns W4A16_OK, or W4A16_ERR_HIP with the count in w4a16_last_error()
 * when any wait gave up since the previous check (a hip error of its own is also returned).
 * ------------------------------------------------------------------------------------- */
int w4a16_split_wait_status(void *stream);

/* Test hook for the path above: one wave waits at most `polls` polls on the 8-byte slot at
 * device address `slot` (16-byte aligned; a slot whose high half is zero is unwritten), stores
 * what it took into out[0] (0.0 when the wait gave up) and clears the slot. The wait ends on
 * its own, whatever the slot holds. Asynchronous on `stream`. */
int w4a16_debug_slot_wait(void *slot, int polls, float *out, void *stream);

/* Measurement hook (no counterpart in the reference): of the calling thread's next kernel
 * launches by this library, the one after `skip` untimed launches records `start_event` /
 * `stop_event` (hipEvent_t, either may be NULL) at that dispatch's own start and end, through
 * hipExtLaunchKernel; later launches are untimed until the next call. bench.py uses it to time
 * one kernel of a call live, on the stream it is launched on, as a kernel trace times it
 * (skip = 1: the down kernel of an FFN call). W4A16_OK, or W4A16_ERR_CONFIG for skip < 0. */
int w4a16_time_next_launch(int skip, void *start_event, void *stop_event);

/* ---------------------------------------------------------------------------------------
 * Test bridges (host pointers, artifact layout; synchronous).
 * ------------------------------------------------------------------------------------- */

/* Same symbol and argument meaning as the reference bridge
 * (reference tests/kernels/kernel_bridge.cu:83-95): host buffers in the artifact layout; the
 * library uploads, re-lays, runs gemm_int4_bf16 and downloads. Returns 0, or nonzero on a
 * refusal or error. */
int test_gemm_int4(void *out, const void *a, const void *packed, const void *scales, int M,
                   int N, int K, int group);

/* Same as the reference bridge's test_silu_mul_packed (kernel_bridge.cu:66-78). */
int test_silu_mul_packed(void *out, const void *packed, int tokens, int intermediate);

#ifdef __cplusplus
}
#endif

#endif /* W4A16_H */
