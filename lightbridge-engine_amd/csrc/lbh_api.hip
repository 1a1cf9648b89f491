// lbh_api.hip — host side of the C ABI declared in include/lightbridge_hip.h.
//
// Validation order and error payloads follow the reference entry points they
// replace (cited per function); outputs are untouched on any error: device
// validation kernels run first and every compute kernel skips its writes when
// a validation word is set.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstring>
#include <new>

#include "../../include/lightbridge_hip.h"
#include "lbh_internal.h"

using namespace lbh;

struct lbh_ctx {
    int device;
    hipStream_t stream;
    DevStatus *status;        // device
    DevStatus *status_host;   // pinned mirror
};

struct lbh_matrix {
    int device;
    int32_t type;
    size_t rows, k, nb;
    uint8_t *planes;
    size_t bytes;
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

size_t block_bytes(int ty) { return (size_t)layout_of(ty).block_bytes; }

MatView view_of(const lbh_matrix *m) {
    MatView v;
    v.planes = m->planes;
    v.type = m->type;
    v.nb = (int32_t)m->nb;
    v.rows = (int32_t)m->rows;
    v.pad = 0;
    v.units = (long long)(m->rows * m->nb);
    return v;
}

// Reads the status mirror after the stream drained.
lbh_status read_status(lbh_ctx *ctx, lbh_error *err) {
    HIP_TRY(hipMemcpyAsync(ctx->status_host, ctx->status, sizeof(DevStatus), hipMemcpyDeviceToHost, ctx->stream));
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    return LBH_OK;
}

uint32_t read_f32_bits(lbh_ctx *ctx, const float *p) {
    uint32_t v = 0;
    (void)hipMemcpy(&v, p, 4, hipMemcpyDeviceToHost);
    return v;
}

// validate_logical_elements (crates/bridge-quant-layout/src/q8_k.rs:188-200).
lbh_status check_elements(int ty, size_t n, lbh_error *err) {
    if (n == 0) return fail(err, LBH_ZERO_LOGICAL_ELEMENTS, ty);
    if (n % 256) return fail(err, LBH_LOGICAL_ELEMENTS_NOT_DIVISIBLE, ty, 0, 256, n);
    return LBH_OK;
}

}  // namespace

extern "C" {

const char *lbh_backend_name(void) { return "hip_gfx950_q8_k"; }

int32_t lbh_device_count(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return 0;
    int good = 0;
    for (int i = 0; i < n; ++i) {
        hipDeviceProp_t prop;
        if (hipGetDeviceProperties(&prop, i) == hipSuccess && std::strncmp(prop.gcnArchName, "gfx950", 6) == 0) ++good;
    }
    return good;
}

lbh_status lbh_ctx_create(int32_t device, void *stream, lbh_ctx **out, lbh_error *err) {
    if (!out) return fail(err, LBH_NULL_ARGUMENT);
    *out = nullptr;
    int n = 0;
    HIP_TRY(hipGetDeviceCount(&n));
    if (device < 0 || device >= n) return fail(err, LBH_INVALID_PARAMETER, 0, (uint64_t)device, (uint64_t)n);
    hipDeviceProp_t prop;
    HIP_TRY(hipGetDeviceProperties(&prop, device));
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) return fail(err, LBH_UNSUPPORTED_SHAPE);
    DeviceGuard g(device);
    lbh_ctx *c = new (std::nothrow) lbh_ctx();
    if (!c) return fail(err, LBH_HIP_ERROR);
    c->device = device;
    c->stream = static_cast<hipStream_t>(stream);
    hipError_t e = hipMalloc(&c->status, sizeof(DevStatus));
    if (e == hipSuccess) e = hipHostMalloc(&c->status_host, sizeof(DevStatus), hipHostMallocDefault);
    if (e == hipSuccess) e = launch_reset_status(c->status, c->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    if (e != hipSuccess) {
        if (c->status) (void)hipFree(c->status);
        delete c;
        return hip_fail(err, e);
    }
    *out = c;
    return ok(err);
}

lbh_status lbh_ctx_destroy(lbh_ctx *ctx) {
    if (!ctx) return LBH_NULL_ARGUMENT;
    DeviceGuard g(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    (void)hipFree(ctx->status);
    (void)hipHostFree(ctx->status_host);
    delete ctx;
    return LBH_OK;
}

lbh_status lbh_ctx_set_stream(lbh_ctx *ctx, void *stream) {
    if (!ctx) return LBH_NULL_ARGUMENT;
    ctx->stream = static_cast<hipStream_t>(stream);
    return LBH_OK;
}

lbh_status lbh_ctx_synchronize(lbh_ctx *ctx, lbh_error *err) {
    if (!ctx) return fail(err, LBH_NULL_ARGUMENT);
    DeviceGuard g(ctx->device);
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    return ok(err);
}

// ------------------------------------------------------------------ Q8_K

lbh_status lbh_quantize_row_q8_k_into(lbh_ctx *ctx, const float *input, size_t n, uint8_t *encoded,
                                      size_t encoded_len, lbh_error *err) {
    if (!ctx) return fail(err, LBH_NULL_ARGUMENT);
    lbh_status st = check_elements(LBH_Q8_K, n, err);
    if (st) return st;
    const size_t want = n / 256 * 292;
    if (encoded_len != want) return fail(err, LBH_ENCODED_LENGTH_MISMATCH, LBH_Q8_K, 0, want, encoded_len);
    if (!input || !encoded) return fail(err, LBH_NULL_ARGUMENT);
    DeviceGuard g(ctx->device);
    HIP_TRY(launch_reset_status(ctx->status, ctx->stream));
    HIP_TRY(launch_find_nonfinite(input, (long long)n, &ctx->status->first_bad_input, ctx->stream));
    HIP_TRY(launch_quantize_q8k(input, encoded, (long long)(n / 256), ctx->status, ctx->stream));
    st = read_status(ctx, err);
    if (st) return st;
    const unsigned long long bad = ctx->status_host->first_bad_input;
    if (bad != ~0ull)
        return fail(err, LBH_NON_FINITE_ACTIVATION, LBH_Q8_K, bad, 0, 0, read_f32_bits(ctx, input + bad));
    return ok(err);
}

lbh_status lbh_quantize_q8_k_rows(lbh_ctx *ctx, const float *input, size_t rows, size_t n, uint8_t *encoded) {
    if (!ctx || !input || !encoded) return LBH_NULL_ARGUMENT;
    if (n == 0) return LBH_ZERO_LOGICAL_ELEMENTS;
    if (n % 256) return LBH_LOGICAL_ELEMENTS_NOT_DIVISIBLE;
    DeviceGuard g(ctx->device);
    return launch_quantize_q8k(input, encoded, (long long)(rows * (n / 256)), nullptr, ctx->stream) == hipSuccess
               ? LBH_OK
               : LBH_HIP_ERROR;
}

// -------------------------------------------------------------- matrices

lbh_status lbh_matrix_create(lbh_ctx *ctx, int32_t ty, size_t rows, size_t k, const void *bytes, size_t byte_len,
                             int32_t on_device, lbh_matrix **out, lbh_error *err) {
    if (!ctx || !out) return fail(err, LBH_NULL_ARGUMENT);
    *out = nullptr;
    if (!is_dot_type(ty)) return fail(err, LBH_UNSUPPORTED_TYPE, ty);
    lbh_status st = check_elements(ty, k, err);
    if (st) return st;
    if (rows == 0) return fail(err, LBH_DIMENSION_MISMATCH, ty, 0, 1, 0);
    const size_t nb = k / 256, want = rows * nb * block_bytes(ty);
    if (byte_len != want) return fail(err, LBH_ENCODED_LENGTH_MISMATCH, ty, 0, want, byte_len);
    if (!bytes) return fail(err, LBH_NULL_ARGUMENT);
    if (nb > 64 || rows > 0x7fffffffull) return fail(err, LBH_UNSUPPORTED_SHAPE, ty, 0, 64, nb);
    DeviceGuard g(ctx->device);
    uint8_t *staging = nullptr, *planes = nullptr;
    const uint8_t *src = static_cast<const uint8_t *>(bytes);
    hipError_t e = hipMalloc(&planes, want);
    if (e == hipSuccess && !on_device) {
        e = hipMalloc(&staging, want);
        if (e == hipSuccess) e = hipMemcpyAsync(staging, bytes, want, hipMemcpyHostToDevice, ctx->stream);
        src = staging;
    }
    const long long U = (long long)(rows * nb);
    if (e == hipSuccess) e = launch_reset_status(ctx->status, ctx->stream);
    if (e == hipSuccess) e = launch_validate_scales(ty, src, U, &ctx->status->first_bad_scale, ctx->stream);
    if (e == hipSuccess) e = launch_repack(ty, src, planes, U, 1, ctx->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(ctx->status_host, ctx->status, sizeof(DevStatus), hipMemcpyDeviceToHost, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (staging) (void)hipFree(staging);
    if (e != hipSuccess) {
        if (planes) (void)hipFree(planes);
        return hip_fail(err, e);
    }
    const unsigned long long bad = ctx->status_host->first_bad_scale;
    if (bad != ~0ull) {
        (void)hipFree(planes);
        const unsigned long long u = bad / 2;
        const uint32_t field = (uint32_t)(bad & 1);
        uint16_t bits = 0;
        const uint8_t *p = static_cast<const uint8_t *>(bytes) + u * block_bytes(ty) + 2 * field;
        if (on_device)
            (void)hipMemcpy(&bits, p, 2, hipMemcpyDeviceToHost);
        else
            std::memcpy(&bits, p, 2);
        // NonFiniteScale { ty, block_index, field, bits } (k_quants.rs:196-204) of the first bad row.
        return fail(err, LBH_NON_FINITE_SCALE, ty, u % nb, 0, 0, bits, field, u / nb);
    }
    lbh_matrix *m = new (std::nothrow) lbh_matrix();
    if (!m) {
        (void)hipFree(planes);
        return fail(err, LBH_HIP_ERROR);
    }
    m->device = ctx->device;
    m->type = ty;
    m->rows = rows;
    m->k = k;
    m->nb = nb;
    m->planes = planes;
    m->bytes = want;
    *out = m;
    return ok(err);
}

lbh_status lbh_matrix_destroy(lbh_matrix *m) {
    if (!m) return LBH_NULL_ARGUMENT;
    DeviceGuard g(m->device);
    (void)hipFree(m->planes);  // hipFree waits for work that may still read the planes
    delete m;
    return LBH_OK;
}

lbh_status lbh_matrix_read_ggml(lbh_ctx *ctx, const lbh_matrix *m, void *host, size_t len, lbh_error *err) {
    if (!ctx || !m || !host) return fail(err, LBH_NULL_ARGUMENT);
    if (len != m->bytes) return fail(err, LBH_ENCODED_LENGTH_MISMATCH, m->type, 0, m->bytes, len);
    DeviceGuard g(ctx->device);
    uint8_t *tmp = nullptr;
    HIP_TRY(hipMalloc(&tmp, m->bytes));
    hipError_t e = launch_repack(m->type, m->planes, tmp, (long long)(m->rows * m->nb), 0, ctx->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(host, tmp, m->bytes, hipMemcpyDeviceToHost, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    (void)hipFree(tmp);
    if (e != hipSuccess) return hip_fail(err, e);
    return ok(err);
}

size_t lbh_matrix_rows(const lbh_matrix *m) { return m ? m->rows : 0; }
size_t lbh_matrix_k(const lbh_matrix *m) { return m ? m->k : 0; }
int32_t lbh_matrix_type(const lbh_matrix *m) { return m ? m->type : -1; }
size_t lbh_matrix_bytes(const lbh_matrix *m) { return m ? m->bytes : 0; }

// ------------------------------------------------------------------ gemv

namespace {

// prepare_llama_q8k (crates/bridge-kernels-reference/src/gemv.rs:245-272) minus the
// per-row scale scan, which matrix upload performed once.
lbh_status gemv_checked(lbh_ctx *ctx, const lbh_matrix *m, const float *input, size_t input_len, float *out,
                        size_t out_len, uint8_t *q8, size_t q8_len, int accumulate, float scale, lbh_error *err) {
    if (!ctx || !m) return fail(err, LBH_NULL_ARGUMENT);
    // gemv_accumulate_scaled_into validates the scale before anything else (gemv.rs:126).
    if (accumulate && !std::isfinite(scale)) {
        uint32_t bits;
        std::memcpy(&bits, &scale, 4);
        return fail(err, LBH_NON_FINITE_VALUE, m->type, 0, 0, 0, bits, 2);
    }
    // validate_dimensions (gemv.rs:195-211).
    if (input_len != m->k) return fail(err, LBH_DIMENSION_MISMATCH, m->type, 0, m->k, input_len);
    if (out_len != m->rows) return fail(err, LBH_DIMENSION_MISMATCH, m->type, 1, m->rows, out_len);
    const size_t need = m->k / 256 * 292;
    if (q8_len < need) return fail(err, LBH_SCRATCH_TOO_SMALL, LBH_Q8_K, 0, need, q8_len);
    if (!input || !out || !q8) return fail(err, LBH_NULL_ARGUMENT);
    DeviceGuard g(ctx->device);
    HIP_TRY(launch_reset_status(ctx->status, ctx->stream));
    if (accumulate) HIP_TRY(launch_find_nonfinite(out, (long long)out_len, &ctx->status->first_bad_dest, ctx->stream));
    HIP_TRY(launch_find_nonfinite(input, (long long)input_len, &ctx->status->first_bad_input, ctx->stream));
    HIP_TRY(launch_quantize_q8k(input, q8, (long long)(m->k / 256), ctx->status, ctx->stream));
    GemvArgs a{};
    a.m = view_of(m);
    a.q8 = q8;
    a.y = out;
    a.coef = scale;
    a.accumulate = accumulate;
    a.block_sums = nullptr;
    a.status = ctx->status;
    HIP_TRY(launch_gemv(a, ctx->stream));
    lbh_status st = read_status(ctx, err);
    if (st) return st;
    if (ctx->status_host->first_bad_dest != ~0ull) {
        const unsigned long long i = ctx->status_host->first_bad_dest;
        return fail(err, LBH_NON_FINITE_VALUE, m->type, i, 0, 0, read_f32_bits(ctx, out + i), 3);
    }
    if (ctx->status_host->first_bad_input != ~0ull) {
        const unsigned long long i = ctx->status_host->first_bad_input;
        return fail(err, LBH_NON_FINITE_VALUE, m->type, i, 0, 0, read_f32_bits(ctx, input + i), 0);
    }
    return ok(err);
}

}  // namespace

lbh_status lbh_gemv_into(lbh_ctx *ctx, const lbh_matrix *m, const float *input, size_t input_len, float *output,
                         size_t output_len, uint8_t *q8, size_t q8_len, lbh_error *err) {
    return gemv_checked(ctx, m, input, input_len, output, output_len, q8, q8_len, 0, 0.0f, err);
}

lbh_status lbh_gemv_accumulate_scaled_into(lbh_ctx *ctx, const lbh_matrix *m, const float *input, size_t input_len,
                                           float *dest, size_t dest_len, float scale, uint8_t *q8, size_t q8_len,
                                           lbh_error *err) {
    return gemv_checked(ctx, m, input, input_len, dest, dest_len, q8, q8_len, 1, scale, err);
}

lbh_status lbh_gemv_q8_k(lbh_ctx *ctx, const lbh_matrix *m, const uint8_t *q8, float *y, float coef,
                         int32_t accumulate) {
    if (!ctx || !m || !q8 || !y) return LBH_NULL_ARGUMENT;
    DeviceGuard g(ctx->device);
    GemvArgs a{};
    a.m = view_of(m);
    a.q8 = q8;
    a.y = y;
    a.coef = coef;
    a.accumulate = accumulate;
    return launch_gemv(a, ctx->stream) == hipSuccess ? LBH_OK : LBH_HIP_ERROR;
}

lbh_status lbh_gemv_block_sums(lbh_ctx *ctx, const lbh_matrix *m, const uint8_t *q8, int32_t *out) {
    if (!ctx || !m || !q8 || !out) return LBH_NULL_ARGUMENT;
    DeviceGuard g(ctx->device);
    float *y = nullptr;
    if (hipMallocAsync(reinterpret_cast<void **>(&y), m->rows * sizeof(float), ctx->stream) != hipSuccess)
        return LBH_HIP_ERROR;
    GemvArgs a{};
    a.m = view_of(m);
    a.q8 = q8;
    a.y = y;
    a.block_sums = out;
    hipError_t e = launch_gemv(a, ctx->stream);
    (void)hipFreeAsync(y, ctx->stream);
    return e == hipSuccess ? LBH_OK : LBH_HIP_ERROR;
}

lbh_status lbh_debug_f16_to_f32(lbh_ctx *ctx, const uint16_t *in, float *out, size_t n, lbh_error *err) {
    if (!ctx || !in || !out) return fail(err, LBH_NULL_ARGUMENT);
    DeviceGuard g(ctx->device);
    HIP_TRY(launch_f16_to_f32(in, out, (long long)n, ctx->stream));
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    return ok(err);
}

}  // extern "C"
