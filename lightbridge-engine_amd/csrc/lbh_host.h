// lbh_host.h — host-side state shared by the C-ABI translation units:
// the context and matrix objects behind the opaque handles of
// include/lightbridge_hip.h, and the error-reporting helpers every entry point
// uses (status codes and payloads of QuantError / KernelError).
#pragma once
#include <hip/hip_runtime.h>

#include <cstring>

#include "../../include/lightbridge_hip.h"
#include "lbh_internal.h"

struct lbh_ctx {
    int device;
    int cu_count;
    hipStream_t stream;
    lbh::DevStatus *status;        // device
    lbh::DevStatus *status_host;   // pinned mirror
    lbh::GemvTuning tuning;
    int gemm_shape;           // K-quant GEMM staging (0: registers, two blocks ahead; 1: direct to LDS)
    uint8_t *scratch;         // this device's copy of the library's static scratch array (lbh_api.hip)
};

struct lbh_matrix {
    int device;
    int32_t type;
    size_t rows, k, nb;
    uint8_t *planes;
    size_t bytes;
    uint8_t *gemm_a;     // MFMA-ready copy for token batches (lbh_matrix_prepare_gemm), or NULL
};

namespace {

lbh_status fail(lbh_error *err, lbh_status st, int ty = 0, uint64_t index = 0, uint64_t expected = 0,
                uint64_t actual = 0, uint32_t bits = 0, uint32_t field = 0, uint64_t row = 0) {
    if (err) {
        std::memset(err, 0, sizeof(*err));
        err->status = st;
        err->ty = ty;
        err->index = index;
        err->expected = expected;
        err->actual = actual;
        err->bits = bits;
        err->field = field;
        err->row = row;
    }
    return st;
}

lbh_status hip_fail(lbh_error *err, hipError_t e) {
    lbh_status st = fail(err, LBH_HIP_ERROR);
    if (err) err->hip_error = (int32_t)e;
    return st;
}

#define HIP_TRY(expr)                              \
    do {                                           \
        hipError_t e_ = (expr);                    \
        if (e_ != hipSuccess) return hip_fail(err, e_); \
    } while (0)

lbh_status ok(lbh_error *err) {
    if (err) {
        std::memset(err, 0, sizeof(*err));
        err->status = LBH_OK;
    }
    return LBH_OK;
}

struct DeviceGuard {
    int prev = -1;
    explicit DeviceGuard(int dev) {
        if (hipGetDevice(&prev) != hipSuccess) prev = -1;
        if (prev != dev) (void)hipSetDevice(dev);
    }
    ~DeviceGuard() {
        int cur;
        if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev) (void)hipSetDevice(prev);
    }
};

}  // namespace
