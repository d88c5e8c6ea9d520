/*
 * engine.cpp - The dense-FFN INT4 operand store behind engine_load_quantized_ffn, and the
 * decode-time FFN dispatch that reads it.
 *
 * A W4A16Store carries what the loader needs from the reference engine's descriptor (layer
 * count, which layers are dense, hidden and intermediate sizes, the tensor-parallel degree and
 * this handle's rank, the device) and owns the device operands of every dense layer. The loader
 * (w4a16_load_quantized_ffn, and engine_load_quantized_ffn for callers with no engine) follows
 * reference csrc/engine.cu:2207-2428:
 *   - parse and validate weights.manifest.json;
 *   - refuse expert parallelism, a sidecar that does not cover every dense layer with an
 *     mlpGateUp pair and an mlpDown entry, and shapes that are not the checkpoint's;
 *   - slice this rank's rows (gate/up: out_dim) and columns (down: in_dim) exactly as the
 *     reference's slice_rows does, keeping the global scales, and refuse a column split that is
 *     not on a 128-wide group boundary;
 *   - read each artifact with its size, dtype and SHA-256 checked;
 *   - upload, then re-lay into tile order on the device (a permutation; the artifact is never
 *     re-quantized).
 * Loading is all-or-nothing: on any refusal every buffer this call allocated is freed and the
 * handle keeps what it had. Every failure after argument checking returns W4A16_ERR_WEIGHTS
 * with the reason in the thread's last error, as the reference's catch-all does
 * (engine.cu:2423-2427).
 *
 * Both exported loader names call one internal function, and nothing in the library calls an
 * exported name: an engine that defines engine_load_quantized_ffn itself and calls
 * w4a16_load_quantized_ffn from it never gets its own function called back (the library is also
 * linked with -Bsymbolic-functions and exports only the names of include/w4a16.h).
 */
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstring>
#include <fstream>
#include <memory>
#include <sstream>
#include <string>
#include <vector>

#include "loader.h"

using namespace w4a16;

namespace {

struct DevBuf {
    void *ptr = nullptr;
    size_t bytes = 0;
    DevBuf() = default;
    DevBuf(const DevBuf &) = delete;
    DevBuf &operator=(const DevBuf &) = delete;
    DevBuf(DevBuf &&o) noexcept : ptr(o.ptr), bytes(o.bytes) { o.ptr = nullptr; o.bytes = 0; }
    DevBuf &operator=(DevBuf &&o) noexcept {
        if (this != &o) { release(); ptr = o.ptr; bytes = o.bytes; o.ptr = nullptr; o.bytes = 0; }
        return *this;
    }
    ~DevBuf() { release(); }
    void release() {
        if (ptr) (void)hipFree(ptr);
        ptr = nullptr;
        bytes = 0;
    }
    int alloc(size_t n) {
        release();
        if (hipMalloc(&ptr, n) != hipSuccess) {
            ptr = nullptr;
            return set_error(W4A16_ERR_ALLOC, "hipMalloc(%zu) failed", n);
        }
        bytes = n;
        return W4A16_OK;
    }
};

struct LayerOperands {
    bool loaded = false;
    DevBuf gu_packed, gu_scales, dn_packed, dn_scales; /* tile order */
};

}  // namespace

struct W4A16Store {
    W4A16EngineConfig cfg;
    int device = -1;     /* the device current at create; -1 if none was visible */
    int int4_rows = 1;   /* tokens routed to INT4: 1, or int4_max_rows for verify rows */
    std::vector<unsigned char> dense;
    int local_inter = 0; /* intermediate columns this rank holds */
    std::vector<LayerOperands> layers;
    DevBuf act_ws;       /* [int4_rows, hidden + local_inter] BF16 (normed, then act) */
    int quantized_layers = 0;
};

namespace {

std::string join_error(const char *prefix) {
    std::string s = prefix;
    s += w4a16_last_error();
    return s;
}

/* rows [row_off, row_off + rows) of a row-major [*, row_bytes_src] buffer, bytes
 * [col_byte, col_byte + row_bytes) of each (reference csrc/engine.cu:2194-2205). */
void slice_rows(uint8_t *dst, const uint8_t *src, long long src_row_bytes, long long row_off,
                long long rows, long long col_byte, long long row_bytes) {
    for (long long i = 0; i < rows; ++i)
        std::memcpy(dst + i * row_bytes, src + (row_off + i) * src_row_bytes + col_byte, (size_t)row_bytes);
}

/* Upload an artifact-layout weight and re-lay it into tile order in `packed` / `scales`. */
int upload_tiled(const std::vector<uint8_t> &p, const std::vector<uint8_t> &s, long long n,
                 long long k, int pair, DevBuf *packed, DevBuf *scales) {
    DevBuf sp, ss;
    int st = sp.alloc(p.size());
    if (!st) st = ss.alloc(s.size());
    if (!st) st = packed->alloc(p.size());
    if (!st) st = scales->alloc(s.size());
    if (st) return st;
    if (hipMemcpy(sp.ptr, p.data(), p.size(), hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(ss.ptr, s.data(), s.size(), hipMemcpyHostToDevice) != hipSuccess)
        return set_error(W4A16_ERR_HIP, "upload of INT4 operands failed");
    st = w4a16_tile_pack_device(n, k, pair, static_cast<const uint8_t *>(sp.ptr),
                                static_cast<const uint16_t *>(ss.ptr),
                                static_cast<uint8_t *>(packed->ptr),
                                static_cast<uint16_t *>(scales->ptr), nullptr);
    if (st) return st;
    if (hipDeviceSynchronize() != hipSuccess) return set_error(W4A16_ERR_HIP, "re-layout failed");
    return W4A16_OK;
}

int read_text(const std::string &path, std::string *out) {
    std::ifstream f(path, std::ios::binary);
    if (!f) return set_error(W4A16_ERR_WEIGHTS, "cannot open %s", path.c_str());
    std::stringstream ss;
    ss << f.rdbuf();
    *out = ss.str();
    return W4A16_OK;
}

/* Makes the store's device current for the duration of an upload and restores the caller's. */
struct DeviceScope {
    int prev = -1;
    bool changed = false, entered = false;
    int enter(int dev) {
        entered = true;
        if (dev < 0) return set_error(W4A16_ERR_STATE, "the store was created with no device visible");
        if (hipGetDevice(&prev) != hipSuccess) return set_error(W4A16_ERR_HIP, "hipGetDevice failed");
        if (prev != dev) {
            if (hipSetDevice(dev) != hipSuccess) return set_error(W4A16_ERR_HIP, "hipSetDevice(%d) failed", dev);
            changed = true;
        }
        return W4A16_OK;
    }
    ~DeviceScope() {
        if (changed) (void)hipSetDevice(prev);
    }
};

int load_impl(W4A16Store *eng, const std::string &root) {
    const W4A16EngineConfig &c = eng->cfg;
    std::string json;
    int st = read_text(root + "/weights.manifest.json", &json);
    if (st) return st;
    Manifest m;
    if (manifest_parse(json, &m) != kManifestOk) return W4A16_ERR_WEIGHTS;
    if (c.ep_size > 1)
        return set_error(W4A16_ERR_WEIGHTS, "the converter quantizes whole tensors and no expert role is "
                         "admitted, so a quantized expert-parallel engine is refused");
    int dense = 0, covered = 0;
    for (int l = 0; l < c.num_layers; ++l) {
        if (!eng->dense[l]) continue;
        ++dense;
        if (m.find_pair("mlpGateUp", l) >= 0 && m.find_entry(l, "mlpDown") >= 0) ++covered;
    }
    if (dense == 0) return set_error(W4A16_ERR_WEIGHTS, "this engine has no dense FFN layer to quantize");
    if (covered != dense)
        return set_error(W4A16_ERR_WEIGHTS, "the sidecar covers %d of %d dense layers", covered, dense);

    const long long H = c.hidden, I = c.intermediate, r = c.tp_rank;
    const long long li = eng->local_inter;
    DeviceScope on_device; /* entered before the first upload, after the host-side checks */
    std::vector<LayerOperands> staged(c.num_layers);
    for (int l = 0; l < c.num_layers; ++l) {
        if (!eng->dense[l]) continue;
        const PairEntry &pair = m.pairs[m.find_pair("mlpGateUp", l)];
        const Entry &down = m.entries[m.find_entry(l, "mlpDown")];
        /* the loader slices gate rows then up rows, so the pair must say exactly that (the
         * reference reader admits any two member roles that have entries) */
        if (pair.member_role[0] != "mlpGate" || pair.member_role[1] != "mlpUp")
            return set_error(W4A16_ERR_WEIGHTS, "layer %d's mlpGateUp pair lists members [%s, %s]; the loader "
                             "needs [mlpGate, mlpUp] in that order", l, pair.member_role[0].c_str(),
                             pair.member_role[1].c_str());
        if (pair.n != 2 * I || pair.k != H)
            return set_error(W4A16_ERR_WEIGHTS, "layer %d's mlpGateUp pair is [%lld, %lld], the checkpoint's gate+up is "
                             "[%lld, %lld]", l, pair.n, pair.k, 2 * I, H);
        if (down.n != H || down.k != I)
            return set_error(W4A16_ERR_WEIGHTS, "layer %d's mlpDown is [%lld, %lld], the checkpoint's is [%lld, %lld]",
                             l, down.n, down.k, H, I);
        if (pair.group != down.group)
            return set_error(W4A16_ERR_WEIGHTS, "layer %d's gate/up and down disagree on the group width", l);
        /* this rank's extents: gate/up rows [r*li, (r+1)*li) of each half, down columns the same */
        const long long col_off = r * li;
        if (col_off % down.group != 0 || li % down.group != 0)
            return set_error(W4A16_ERR_WEIGHTS, "layer %d's rank %lld splits K at a non-group boundary (column %lld), "
                             "which cannot retain the global scales", l, r, col_off);
        std::vector<uint8_t> gp, gs, dp, ds;
        if (artifact_read(root, pair.packed, "u8", &gp) || artifact_read(root, pair.scales, "bf16", &gs) ||
            artifact_read(root, down.packed, "u8", &dp) || artifact_read(root, down.scales, "bf16", &ds))
            return W4A16_ERR_WEIGHTS;
        const long long G = H / W4A16_GROUP, Gd = I / W4A16_GROUP, lGd = li / W4A16_GROUP;
        std::vector<uint8_t> sgp((size_t)(2 * li * H / 2)), sgs((size_t)(2 * li * G * 2));
        slice_rows(sgp.data(), gp.data(), H / 2, col_off, li, 0, H / 2);
        slice_rows(sgp.data() + li * H / 2, gp.data(), H / 2, I + col_off, li, 0, H / 2);
        slice_rows(sgs.data(), gs.data(), G * 2, col_off, li, 0, G * 2);
        slice_rows(sgs.data() + li * G * 2, gs.data(), G * 2, I + col_off, li, 0, G * 2);
        std::vector<uint8_t> sdp((size_t)(H * li / 2)), sds((size_t)(H * lGd * 2));
        slice_rows(sdp.data(), dp.data(), I / 2, 0, H, col_off / 2, li / 2);
        slice_rows(sds.data(), ds.data(), Gd * 2, 0, H, col_off / W4A16_GROUP * 2, lGd * 2);
        LayerOperands &op = staged[l];
        if (!on_device.entered && (st = on_device.enter(eng->device))) return st;
        if ((st = upload_tiled(sgp, sgs, 2 * li, H, 1, &op.gu_packed, &op.gu_scales)) ||
            (st = upload_tiled(sdp, sds, H, li, 0, &op.dn_packed, &op.dn_scales)))
            return set_error(W4A16_ERR_WEIGHTS, "%s", join_error("upload: ").c_str());
        op.loaded = true;
    }
    if (!on_device.entered && (st = on_device.enter(eng->device))) return st;
    DevBuf ws;
    if (ws.alloc((size_t)eng->int4_rows * (size_t)(H + li) * 2)) return W4A16_ERR_WEIGHTS;
    /* the split-K scratch at its worst case for this store's shapes, so forwards never allocate
     * (or synchronise), also on the first call of a shape under graph capture */
    if ((st = reserve_split_scratch(eng->int4_rows, (int)H, (int)li)))
        return set_error(W4A16_ERR_WEIGHTS, "%s", join_error("split-K scratch: ").c_str());
    /* commit: only now does the handle see the new operands */
    eng->layers.swap(staged);
    eng->act_ws = std::move(ws);
    eng->quantized_layers = dense;
    return W4A16_OK;
}

}  // namespace

/* The one loader body behind both exported names. */
static int load_store(W4A16Store *eng, const char *manifest_dir, const char *what) {
    if (!eng || !manifest_dir) return set_error(W4A16_ERR_CONFIG, "%s: null argument", what);
    try {
        const int st = load_impl(eng, manifest_dir);
        if (st) {
            const std::string why = error_text();
            return set_error(W4A16_ERR_WEIGHTS, "%s: %s", what, why.c_str());
        }
        return W4A16_OK;
    } catch (const std::exception &e) {
        return set_error(W4A16_ERR_WEIGHTS, "%s: %s", what, e.what());
    }
}

extern "C" const char *engine_last_error(void) { return error_text(); }

extern "C" W4A16Store *w4a16_engine_create(const W4A16EngineConfig *cfg) {
    if (!cfg) {
        set_error(W4A16_ERR_CONFIG, "engine_create: null config");
        return nullptr;
    }
    const W4A16EngineConfig &c = *cfg;
    if (c.num_layers <= 0 || c.hidden <= 0 || c.intermediate <= 0 || c.tp_size <= 0 ||
        c.tp_rank < 0 || c.tp_rank >= c.tp_size || c.max_tokens <= 0 || c.ep_size <= 0) {
        set_error(W4A16_ERR_CONFIG, "engine_create: bad configuration");
        return nullptr;
    }
    if (c.int4_max_rows < 0 || c.int4_max_rows > c.max_tokens || c.int4_max_rows > 16) {
        set_error(W4A16_ERR_CONFIG, "engine_create: int4_max_rows %d is outside 0..min(16, "
                  "max_tokens = %d)", c.int4_max_rows, c.max_tokens);
        return nullptr;
    }
    if (c.intermediate % c.tp_size != 0) {
        set_error(W4A16_ERR_CONFIG, "engine_create: intermediate %d does not split over tp=%d",
                  c.intermediate, c.tp_size);
        return nullptr;
    }
    auto eng = std::make_unique<W4A16Store>();
    eng->cfg = c;
    eng->cfg.layer_is_dense = nullptr; /* copied below; the caller's array need not outlive us */
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess) dev = -1;
    eng->device = dev;
    eng->int4_rows = c.int4_max_rows > 0 ? c.int4_max_rows : 1;
    eng->dense.assign((size_t)c.num_layers, 1);
    if (c.layer_is_dense)
        for (int l = 0; l < c.num_layers; ++l) eng->dense[l] = c.layer_is_dense[l] ? 1 : 0;
    eng->local_inter = c.intermediate / c.tp_size;
    eng->layers.resize((size_t)c.num_layers);
    return eng.release();
}

extern "C" void w4a16_engine_destroy(W4A16Store *eng) {
    if (!eng) return;
    DeviceScope on_device; /* free the buffers on the device that holds them */
    if (eng->device >= 0) (void)on_device.enter(eng->device);
    delete eng;
}

extern "C" int w4a16_load_quantized_ffn(W4A16Store *eng, const char *manifest_dir) {
    return load_store(eng, manifest_dir, "w4a16_load_quantized_ffn");
}

extern "C" int engine_load_quantized_ffn(W4A16Store *eng, const char *manifest_dir) {
    return load_store(eng, manifest_dir, "engine_load_quantized_ffn");
}

extern "C" int engine_quantized_ffn_layers(const W4A16Store *eng) {
    return eng ? eng->quantized_layers : 0;
}

static bool layer_loaded(const W4A16Store *eng, int layer) {
    return layer >= 0 && layer < eng->cfg.num_layers && eng->layers[layer].loaded;
}

extern "C" int engine_ffn_routes_int4(const W4A16Store *eng, int layer, int tokens, int verify_rows) {
    if (!eng || !layer_loaded(eng, layer)) return 0;
    return tokens == 1 || (verify_rows && tokens >= 1 && tokens <= eng->int4_rows);
}

/* What every forward checks before it launches: the row count against the INT4 routing limit
 * (prefill rows stay on the engine's BF16 path), and that the store's device is current. */
static int forward_checks(const W4A16Store *eng, int tokens, const char *what) {
    if (!eng) return set_error(W4A16_ERR_CONFIG, "%s: null store", what);
    if (tokens < 0 || tokens > eng->int4_rows)
        return set_error(W4A16_ERR_CONFIG, "%s: %d tokens; this store routes at most %d rows to INT4 "
                         "(int4_max_rows), larger batches stay on the BF16 weights", what, tokens,
                         eng->int4_rows);
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev != eng->device)
        return set_error(W4A16_ERR_STATE, "%s: the store's operands are on device %d, device %d is "
                         "current", what, eng->device, dev);
    return W4A16_OK;
}

extern "C" int engine_ffn_operands(const W4A16Store *eng, int layer, W4A16FfnOperands *out) {
    if (!eng || !out) return set_error(W4A16_ERR_CONFIG, "engine_ffn_operands: null argument");
    if (!layer_loaded(eng, layer))
        return set_error(W4A16_ERR_STATE, "engine_ffn_operands: layer %d has no INT4 operands", layer);
    const LayerOperands &op = eng->layers[layer];
    out->gate_up_packed = static_cast<const uint8_t *>(op.gu_packed.ptr);
    out->gate_up_scales = static_cast<const uint16_t *>(op.gu_scales.ptr);
    out->down_packed = static_cast<const uint8_t *>(op.dn_packed.ptr);
    out->down_scales = static_cast<const uint16_t *>(op.dn_scales.ptr);
    out->hidden = eng->cfg.hidden;
    out->intermediate = eng->local_inter;
    out->group = W4A16_GROUP;
    return W4A16_OK;
}

static int ffn_forward(W4A16Store *eng, int layer, const uint16_t *normed, void *out,
                       bool partial, int tokens, void *stream) {
    int st = forward_checks(eng, tokens, "engine_ffn_forward");
    if (st) return st;
    W4A16FfnOperands op;
    if ((st = engine_ffn_operands(eng, layer, &op))) return st;
    uint16_t *act = static_cast<uint16_t *>(eng->act_ws.ptr);
    return partial ? mlp_int4_partial_f32(normed, op.gate_up_packed, op.gate_up_scales, op.down_packed,
                                          op.down_scales, static_cast<float *>(out), act, tokens,
                                          op.hidden, op.intermediate, stream)
                   : mlp_int4_bf16(normed, op.gate_up_packed, op.gate_up_scales, op.down_packed,
                                   op.down_scales, static_cast<uint16_t *>(out), act, tokens,
                                   op.hidden, op.intermediate, stream);
}

extern "C" int engine_ffn_forward(W4A16Store *eng, int layer, const uint16_t *normed,
                                  uint16_t *out, int tokens, void *stream) {
    return ffn_forward(eng, layer, normed, out, false, tokens, stream);
}

extern "C" int engine_ffn_forward_partial_f32(W4A16Store *eng, int layer,
                                              const uint16_t *normed, float *out, int tokens,
                                              void *stream) {
    return ffn_forward(eng, layer, normed, out, true, tokens, stream);
}

static int ffn_forward_norm(W4A16Store *eng, int layer, const uint16_t *residual,
                            const uint16_t *norm_w, int norm_style, float eps, void *out,
                            bool partial, int tokens, void *stream) {
    int st = forward_checks(eng, tokens, "engine_ffn_forward_norm");
    if (st) return st;
    W4A16FfnOperands op;
    if ((st = engine_ffn_operands(eng, layer, &op))) return st;
    uint16_t *ws = static_cast<uint16_t *>(eng->act_ws.ptr);
    return partial ? mlp_int4_norm_partial_f32(residual, norm_w, norm_style, eps, op.gate_up_packed,
                                               op.gate_up_scales, op.down_packed, op.down_scales,
                                               static_cast<float *>(out), ws, tokens, op.hidden,
                                               op.intermediate, stream)
                   : mlp_int4_norm_bf16(residual, norm_w, norm_style, eps, op.gate_up_packed,
                                        op.gate_up_scales, op.down_packed, op.down_scales,
                                        static_cast<uint16_t *>(out), ws, tokens, op.hidden,
                                        op.intermediate, stream);
}

extern "C" int engine_ffn_forward_norm(W4A16Store *eng, int layer, const uint16_t *residual,
                                       const uint16_t *norm_w, int norm_style, float eps,
                                       uint16_t *out, int tokens, void *stream) {
    return ffn_forward_norm(eng, layer, residual, norm_w, norm_style, eps, out, false, tokens,
                            stream);
}

extern "C" int engine_ffn_forward_norm_partial_f32(W4A16Store *eng, int layer,
                                                   const uint16_t *residual,
                                                   const uint16_t *norm_w, int norm_style,
                                                   float eps, float *out, int tokens,
                                                   void *stream) {
    return ffn_forward_norm(eng, layer, residual, norm_w, norm_style, eps, out, true, tokens,
                            stream);
}

extern "C" int engine_ffn_forward_residual_norm(W4A16Store *eng, int layer, uint16_t *residual,
                                                const uint16_t *sublayer, const uint16_t *norm_w,
                                                int norm_style, float eps, uint16_t *out,
                                                int tokens, void *stream) {
    int st = forward_checks(eng, tokens, "engine_ffn_forward_residual_norm");
    if (st) return st;
    if (eng->cfg.tp_size > 1)
        return set_error(W4A16_ERR_CONFIG, "engine_ffn_forward_residual_norm: tensor parallelism "
                         "adds the residual after the cross-rank sum; use engine_ffn_forward_norm_partial_f32");
    W4A16FfnOperands op;
    if ((st = engine_ffn_operands(eng, layer, &op))) return st;
    return mlp_int4_residual_norm_bf16(residual, sublayer, norm_w, norm_style, eps,
                                       op.gate_up_packed, op.gate_up_scales, op.down_packed,
                                       op.down_scales, out, static_cast<uint16_t *>(eng->act_ws.ptr),
                                       tokens, op.hidden, op.intermediate, stream);
}
