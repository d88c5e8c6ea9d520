/*
 * bridge.cpp - Synchronous host-pointer test bridges with the reference's symbols and argument
 * meaning (reference tests/kernels/kernel_bridge.cu:66-95).
 *
 * The reference bridge hands host pointers straight to its kernel. Here the bridge owns the
 * device copies explicitly: upload the artifact-layout operands, re-lay them into tile order on
 * the device, run the product entry point, download, free.
 */
#include <hip/hip_runtime.h>

#include <cstdio>

#include "common.h"

using namespace w4a16;

namespace {

struct DeviceBuffers {
    void *p[6] = {nullptr, nullptr, nullptr, nullptr, nullptr, nullptr};
    ~DeviceBuffers() {
        for (void *q : p)
            if (q) (void)hipFree(q);
    }
};

int hip_check(hipError_t e, const char *what) {
    if (e == hipSuccess) return 0;
    return set_error(W4A16_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

}  // namespace

extern "C" int test_gemm_int4(void *out, const void *a, const void *packed, const void *scales,
                              int M, int N, int K, int group) {
    if (M < 0 || N < 0 || K <= 0 || group <= 0) {
        set_error(W4A16_ERR_CONFIG, "test_gemm_int4: negative extent or nonpositive group");
        std::fprintf(stderr, "test_gemm_int4: %s\n", w4a16_last_error());
        return -1;
    }
    if (M == 0 || N == 0) return 0;
    if (!out || !a || !packed || !scales) {
        set_error(W4A16_ERR_CONFIG, "test_gemm_int4: null buffer");
        return -1;
    }
    long long pbytes = 0, nscales = 0;
    if (w4a16_layout_init(N, K, group, &pbytes, &nscales) != W4A16_OK) {
        std::fprintf(stderr, "test_gemm_int4: %s\n", w4a16_last_error());
        return -1;
    }
    DeviceBuffers d;
    const size_t a_bytes = (size_t)M * K * 2, o_bytes = (size_t)M * N * 2;
    int st = 0;
    st = st ? st : hip_check(hipMalloc(&d.p[0], a_bytes), "hipMalloc a");
    st = st ? st : hip_check(hipMalloc(&d.p[1], (size_t)pbytes), "hipMalloc packed");
    st = st ? st : hip_check(hipMalloc(&d.p[2], (size_t)nscales * 2), "hipMalloc scales");
    st = st ? st : hip_check(hipMalloc(&d.p[3], (size_t)pbytes), "hipMalloc packed_tiled");
    st = st ? st : hip_check(hipMalloc(&d.p[4], (size_t)nscales * 2), "hipMalloc scales_tiled");
    st = st ? st : hip_check(hipMalloc(&d.p[5], o_bytes), "hipMalloc out");
    st = st ? st : hip_check(hipMemcpy(d.p[0], a, a_bytes, hipMemcpyHostToDevice), "copy a");
    st = st ? st : hip_check(hipMemcpy(d.p[1], packed, (size_t)pbytes, hipMemcpyHostToDevice), "copy packed");
    st = st ? st : hip_check(hipMemcpy(d.p[2], scales, (size_t)nscales * 2, hipMemcpyHostToDevice), "copy scales");
    st = st ? st : w4a16_tile_pack_device(N, K, 0, (const uint8_t *)d.p[1], (const uint16_t *)d.p[2],
                                          (uint8_t *)d.p[3], (uint16_t *)d.p[4], nullptr);
    st = st ? st : gemm_int4_bf16((const uint16_t *)d.p[0], (const uint8_t *)d.p[3],
                                  (const uint16_t *)d.p[4], (uint16_t *)d.p[5], M, N, K, group,
                                  nullptr);
    st = st ? st : hip_check(hipDeviceSynchronize(), "synchronize");
    st = st ? st : hip_check(hipMemcpy(out, d.p[5], o_bytes, hipMemcpyDeviceToHost), "copy out");
    if (st) {
        std::fprintf(stderr, "test_gemm_int4: %s\n", w4a16_last_error());
        return -1;
    }
    return 0;
}

extern "C" int test_silu_mul_packed(void *out, const void *packed, int tokens, int intermediate) {
    if (tokens < 0 || intermediate < 0) return -1;
    if (tokens == 0 || intermediate == 0) return 0;
    if (!out || !packed) return -1;
    DeviceBuffers d;
    const size_t in_bytes = (size_t)tokens * intermediate * 4, out_bytes = (size_t)tokens * intermediate * 2;
    int st = 0;
    st = st ? st : hip_check(hipMalloc(&d.p[0], in_bytes), "hipMalloc packed");
    st = st ? st : hip_check(hipMalloc(&d.p[1], out_bytes), "hipMalloc out");
    st = st ? st : hip_check(hipMemcpy(d.p[0], packed, in_bytes, hipMemcpyHostToDevice), "copy in");
    st = st ? st : silu_mul_packed_bf16((uint16_t *)d.p[1], (const uint16_t *)d.p[0], tokens,
                                        intermediate, nullptr);
    st = st ? st : hip_check(hipDeviceSynchronize(), "synchronize");
    st = st ? st : hip_check(hipMemcpy(out, d.p[1], out_bytes, hipMemcpyDeviceToHost), "copy out");
    if (st) {
        std::fprintf(stderr, "test_silu_mul_packed: %s\n", w4a16_last_error());
        return -1;
    }
    return 0;
}
