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
#include <memory>
#include <mutex>
#include <new>

#include "../../include/lightbridge_hip.h"
#include "lbh_cache.h"
#include "lbh_host.h"
#include "lbh_internal.h"
#include "lbh_math.h"

using namespace lbh;

// Device scratch of the entry points that allocate nothing (lbh_gemm_q8_k_noalloc):
// one copy per GPU, held until the process ends.  Host code never uses this
// name as an address: each device's copy is looked up once with
// hipGetSymbolAddress (scratch_of_device) and only that pointer is passed on.
static __device__ __align__(256) uint8_t scratch[LBH_NOALLOC_SCRATCH_BYTES];

namespace {

// Per-device address of `scratch`, looked up once per device with that device
// current (lbh_ctx_create makes it current before calling this).
constexpr int MAX_DEVICES = 64;
std::mutex g_scratch_mu;
uint8_t *g_scratch_ptr[MAX_DEVICES];

// Use guard of a device's scratch: the stream of the last eager call and an
// event recorded after its launches (created with the lookup, kept until the
// process ends, as the array is).  A call on another stream while that event
// is pending would overwrite tiles the earlier GEMM may still read.
struct ScratchUse {
    hipEvent_t done = nullptr;
    hipStream_t last = nullptr;
    bool pending = false;
};
ScratchUse g_scratch_use[MAX_DEVICES];

hipError_t scratch_of_device(int device, uint8_t **out) {
    if (device < 0 || device >= MAX_DEVICES) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[device]) {
        void *p = nullptr;
        hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        if (!g_scratch_use[device].done) {
            e = hipEventCreateWithFlags(&g_scratch_use[device].done, hipEventDisableTiming);
            if (e != hipSuccess) return e;
        }
        g_scratch_ptr[device] = static_cast<uint8_t *>(p);
    }
    *out = g_scratch_ptr[device];
    return hipSuccess;
}

size_t block_bytes(int ty) { return (size_t)layout_of(ty).block_bytes; }

MatView view_of(const lbh_matrix *m) {
    MatView v;
    v.planes = m->planes;
    v.type = m->type;
    v.nb = (int32_t)m->nb;
    v.rows = (int32_t)m->rows;
    v.order = MAT_ROW_MAJOR;
    v.units = (long long)(m->rows * m->nb);
    v.bytes = (long long)m->bytes;
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
    c->cu_count = prop.multiProcessorCount;
    c->tuning.lpu = 0;
    c->tuning.max_blocks = 0;
    c->tuning.cu_count = prop.multiProcessorCount;
    c->stream = static_cast<hipStream_t>(stream);
    hipError_t e = scratch_of_device(device, &c->scratch);
    if (e == hipSuccess) e = hipMalloc(&c->status, sizeof(DevStatus));
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

lbh_status lbh_ctx_set_tuning(lbh_ctx *ctx, int32_t key, int32_t value) {
    if (!ctx) return LBH_NULL_ARGUMENT;
    switch (key) {
    case LBH_TUNE_GEMV_LPU:
        if (value != 0 && value != 1 && value != 2 && value != 4) return LBH_INVALID_PARAMETER;
        ctx->tuning.lpu = value;
        return LBH_OK;
    case LBH_TUNE_GEMV_MAX_BLOCKS:
        if (value < 0) return LBH_INVALID_PARAMETER;
        ctx->tuning.max_blocks = value;
        return LBH_OK;
    case LBH_TUNE_GEMV_DEPTH:
        if (value < 0 || value > 4) return LBH_INVALID_PARAMETER;
        ctx->tuning.depth = value;
        return LBH_OK;
    case LBH_TUNE_GEMM_SHAPE:
        if (value < 0 || value > 3) return LBH_INVALID_PARAMETER;
        ctx->gemm_shape = value;
        return LBH_OK;
    default: return LBH_INVALID_PARAMETER;
    }
}

int32_t lbh_ctx_cu_count(const lbh_ctx *ctx) { return ctx ? ctx->cu_count : 0; }

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

// An F32 matrix (the reference routes it to dot_f32_row in every mode,
// gemv.rs:88-101, :128-146): stored in the router layout (w[(j * rows + r) * 4
// + c] = row r, input 4j + c) so the sequential row chains read coalesced
// lines; k must be a multiple of 256 (the chains' step), rows < 2^31.
static lbh_status create_f32(lbh_ctx *ctx, size_t rows, size_t k, const void *bytes, size_t byte_len,
                             int32_t on_device, lbh_matrix **out, lbh_error *err) {
    if (k == 0) return fail(err, LBH_ZERO_LOGICAL_ELEMENTS, LBH_F32);
    if (rows == 0) return fail(err, LBH_DIMENSION_MISMATCH, LBH_F32, 0, 1, 0);
    if (rows > SIZE_MAX / 4 / k) return fail(err, LBH_ARITHMETIC_OVERFLOW, LBH_F32);
    const size_t want = rows * k * 4;
    if (byte_len != want) return fail(err, LBH_ENCODED_LENGTH_MISMATCH, LBH_F32, 0, want, byte_len);
    if (!bytes) return fail(err, LBH_NULL_ARGUMENT);
    if (k % 256 || rows > 0x7ffffff0ull) return fail(err, LBH_UNSUPPORTED_SHAPE, LBH_F32, 0, 256, k);
    DeviceGuard g(ctx->device);
    uint8_t *staging = nullptr, *planes = nullptr;
    const uint8_t *src = static_cast<const uint8_t *>(bytes);
    hipError_t e = hipMalloc(&planes, want);
    if (e == hipSuccess && !on_device) {
        e = hipMalloc(&staging, want);
        if (e == hipSuccess) e = hipMemcpyAsync(staging, bytes, want, hipMemcpyHostToDevice, ctx->stream);
        src = staging;
    }
    if (e == hipSuccess)
        e = launch_f32_layout(reinterpret_cast<const float *>(src), reinterpret_cast<float *>(planes), (long long)rows,
                              (long long)k, 1, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (staging) (void)hipFree(staging);
    if (e != hipSuccess) {
        if (planes) (void)hipFree(planes);
        return hip_fail(err, e);
    }
    lbh_matrix *m = new (std::nothrow) lbh_matrix();
    if (!m) {
        (void)hipFree(planes);
        return fail(err, LBH_HIP_ERROR);
    }
    m->device = ctx->device;
    m->type = LBH_F32;
    m->rows = rows;
    m->k = k;
    m->nb = k / 256;
    m->planes = planes;
    m->bytes = want;
    *out = m;
    return ok(err);
}

lbh_status lbh_matrix_create(lbh_ctx *ctx, int32_t ty, size_t rows, size_t k, const void *bytes, size_t byte_len,
                             int32_t on_device, lbh_matrix **out, lbh_error *err) {
    if (!ctx || !out) return fail(err, LBH_NULL_ARGUMENT);
    *out = nullptr;
    if (ty == LBH_F32) return create_f32(ctx, rows, k, bytes, byte_len, on_device, out, err);
    if (!is_dot_type(ty)) return fail(err, LBH_UNSUPPORTED_TYPE, ty);
    lbh_status st = check_elements(ty, k, err);
    if (st) return st;
    if (rows == 0) return fail(err, LBH_DIMENSION_MISMATCH, ty, 0, 1, 0);
    const size_t nb = k / 256, want = rows * nb * block_bytes(ty);
    if (byte_len != want) return fail(err, LBH_ENCODED_LENGTH_MISMATCH, ty, 0, want, byte_len);
    if (!bytes) return fail(err, LBH_NULL_ARGUMENT);
    if (nb > 64 || rows > 0x7fffffffull) return fail(err, LBH_UNSUPPORTED_SHAPE, ty, 0, 64, nb);
    // Kernels address the planes with 32-bit buffer offsets.
    if (want >= (1ull << 32)) return fail(err, LBH_UNSUPPORTED_SHAPE, ty, 0, (1ull << 32) - 1, want);
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

// Tensor bytes pulled through the caller's reader in chunks of this size
// (a multiple of the block size), double-buffered in pinned host memory.
constexpr size_t STREAM_CHUNK_BYTES = 32u << 20;

lbh_status lbh_matrix_create_streamed(lbh_ctx *ctx, int32_t ty, size_t rows, size_t k, lbh_byte_reader reader,
                                      void *user, lbh_matrix **out, lbh_error *err) {
    if (!ctx || !out || !reader) return fail(err, LBH_NULL_ARGUMENT);
    *out = nullptr;
    if (!is_dot_type(ty)) return fail(err, LBH_UNSUPPORTED_TYPE, ty);
    lbh_status st = check_elements(ty, k, err);
    if (st) return st;
    if (rows == 0) return fail(err, LBH_DIMENSION_MISMATCH, ty, 0, 1, 0);
    const size_t nb = k / 256, bb = block_bytes(ty), want = rows * nb * bb;
    if (nb > 64 || rows > 0x7fffffffull) return fail(err, LBH_UNSUPPORTED_SHAPE, ty, 0, 64, nb);
    if (want >= (1ull << 32)) return fail(err, LBH_UNSUPPORTED_SHAPE, ty, 0, (1ull << 32) - 1, want);
    const long long U = (long long)(rows * nb);
    long long per = (long long)(STREAM_CHUNK_BYTES / bb);
    if (per > U) per = U;
    const size_t cb = (size_t)per * bb;
    const bool kq = ty == LBH_Q4_K || ty == LBH_Q5_K;
    DeviceGuard g(ctx->device);
    uint8_t *planes = nullptr, *host[2] = {nullptr, nullptr}, *dev[2] = {nullptr, nullptr};
    hipEvent_t done[2] = {nullptr, nullptr};
    bool pending[2] = {false, false};
    hipError_t e = hipMalloc(&planes, want);
    for (int b = 0; b < 2 && e == hipSuccess; ++b) {
        e = hipHostMalloc(&host[b], cb, hipHostMallocDefault);
        if (e == hipSuccess) e = hipMalloc(&dev[b], cb);
        if (e == hipSuccess) e = hipEventCreateWithFlags(&done[b], hipEventDisableTiming);
    }
    st = e == hipSuccess ? LBH_OK : hip_fail(err, e);
    // Chunk i: wait until its host buffer's previous DMA is done, read, check
    // the scales on the host (validate_scales, k_quants.rs:178-208: first
    // offending block in order, d before dmin), then DMA and repack the units
    // on the stream while the host reads chunk i + 1 into the other buffer.
    for (long long u0 = 0, i = 0; st == LBH_OK && u0 < U; u0 += per, ++i) {
        const int b = (int)(i & 1);
        const long long n = U - u0 < per ? U - u0 : per;
        if (pending[b]) {
            e = hipEventSynchronize(done[b]);
            if (e != hipSuccess) {
                st = hip_fail(err, e);
                break;
            }
        }
        const int32_t code = reader(user, (uint64_t)u0 * bb, host[b], (size_t)n * bb);
        if (code != 0) {
            st = fail(err, (lbh_status)LBH_SOURCE_READ_FAILED, ty, (uint64_t)u0 * bb, 0, (uint64_t)(int64_t)code);
            break;
        }
        for (long long j = 0; j < n && st == LBH_OK; ++j) {
            const uint8_t *blk = host[b] + (size_t)j * bb;
            for (int f = 0; f < (kq ? 2 : 1); ++f) {
                const uint32_t h = blk[2 * f] | ((uint32_t)blk[2 * f + 1] << 8);
                if ((h & 0x7c00u) == 0x7c00u) {
                    const long long u = u0 + j;
                    st = fail(err, LBH_NON_FINITE_SCALE, ty, (uint64_t)(u % (long long)nb), 0, 0, h, (uint32_t)f,
                              (uint64_t)(u / (long long)nb));
                    break;
                }
            }
        }
        if (st != LBH_OK) break;
        e = hipMemcpyAsync(dev[b], host[b], (size_t)n * bb, hipMemcpyHostToDevice, ctx->stream);
        if (e == hipSuccess) e = launch_repack_range(ty, dev[b], planes, U, u0, n, ctx->stream);
        if (e == hipSuccess) e = hipEventRecord(done[b], ctx->stream);
        if (e != hipSuccess) st = hip_fail(err, e);
        pending[b] = true;
    }
    e = hipStreamSynchronize(ctx->stream);
    if (st == LBH_OK && e != hipSuccess) st = hip_fail(err, e);
    for (int b = 0; b < 2; ++b) {
        if (host[b]) (void)hipHostFree(host[b]);
        if (dev[b]) (void)hipFree(dev[b]);
        if (done[b]) (void)hipEventDestroy(done[b]);
    }
    if (st != LBH_OK) {
        if (planes) (void)hipFree(planes);
        return st;
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
    if (m->gemm_a) (void)hipFree(m->gemm_a);
    delete m;
    return LBH_OK;
}

lbh_status lbh_matrix_read_ggml(lbh_ctx *ctx, const lbh_matrix *m, void *host, size_t len, lbh_error *err) {
    if (!ctx || !m || !host) return fail(err, LBH_NULL_ARGUMENT);
    if (len != m->bytes) return fail(err, LBH_ENCODED_LENGTH_MISMATCH, m->type, 0, m->bytes, len);
    DeviceGuard g(ctx->device);
    uint8_t *tmp = nullptr;
    HIP_TRY(hipMalloc(&tmp, m->bytes));
    hipError_t e = m->type == LBH_F32
                       ? launch_f32_layout(reinterpret_cast<const float *>(m->planes), reinterpret_cast<float *>(tmp),
                                           (long long)m->rows, (long long)m->k, 0, ctx->stream)
                       : launch_repack(m->type, m->planes, tmp, (long long)(m->rows * m->nb), 0, ctx->stream);
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

// The device scans of a checked matvec report in the reference's order: the
// destination (gemv_accumulate_scaled_into, gemv.rs:127) before the
// dimensions, the input (validate_dimensions, gemv.rs:195-211) before the
// scratch size (prepare_llama_q8k, gemv.rs:258-264).  A host-side error that
// the reference checks after a scan is reported only once the scan is known
// clean, which costs a synchronisation on error paths only.
lbh_status dest_error(lbh_ctx *ctx, int ty, const float *dest, lbh_error *err) {
    const unsigned long long i = ctx->status_host->first_bad_dest;
    return fail(err, LBH_NON_FINITE_VALUE, ty, i, 0, 0, read_f32_bits(ctx, dest + i), 3);
}

lbh_status input_error(lbh_ctx *ctx, int ty, const float *input, lbh_error *err) {
    const unsigned long long i = ctx->status_host->first_bad_input;
    return fail(err, LBH_NON_FINITE_VALUE, ty, i, 0, 0, read_f32_bits(ctx, input + i), 0);
}

// Scale and destination checks of an accumulating call (gemv.rs:126-127), then
// validate_dimensions (gemv.rs:195-211) including the input scan.  On success
// the scans are queued (not yet read) and the status words are live.
lbh_status check_gemv_args(lbh_ctx *ctx, const lbh_matrix *m, const float *input, size_t input_len, float *out,
                           size_t out_len, int accumulate, float scale, lbh_error *err) {
    if (accumulate && !std::isfinite(scale)) {
        uint32_t bits;
        std::memcpy(&bits, &scale, 4);
        return fail(err, LBH_NON_FINITE_VALUE, m->type, 0, 0, 0, bits, 2);
    }
    if (!input || !out) return fail(err, LBH_NULL_ARGUMENT);
    HIP_TRY(launch_reset_status(ctx->status, ctx->stream));
    if (accumulate) HIP_TRY(launch_find_nonfinite(out, (long long)out_len, &ctx->status->first_bad_dest, ctx->stream));
    if (input_len != m->k || out_len != m->rows) {
        if (accumulate) {
            lbh_status st = read_status(ctx, err);
            if (st) return st;
            if (ctx->status_host->first_bad_dest != ~0ull) return dest_error(ctx, m->type, out, err);
        }
        if (input_len != m->k) return fail(err, LBH_DIMENSION_MISMATCH, m->type, 0, m->k, input_len);
        return fail(err, LBH_DIMENSION_MISMATCH, m->type, 1, m->rows, out_len);
    }
    HIP_TRY(launch_find_nonfinite(input, (long long)input_len, &ctx->status->first_bad_input, ctx->stream));
    return LBH_OK;
}

// The scans' verdict after the compute launch (which skipped its writes if
// any scan fired): destination first, then input.
lbh_status scan_verdict(lbh_ctx *ctx, int ty, const float *input, const float *out, lbh_error *err) {
    lbh_status st = read_status(ctx, err);
    if (st) return st;
    if (ctx->status_host->first_bad_dest != ~0ull) return dest_error(ctx, ty, out, err);
    if (ctx->status_host->first_bad_input != ~0ull) return input_error(ctx, ty, input, err);
    return ok(err);
}

// The sequential row chains of an F32 matrix (dot_f32_row, gemv.rs:286-303),
// optionally accumulating (gemv.rs:161-171); skip_if as RouterArgs.
hipError_t launch_f32_gemv(lbh_ctx *ctx, const lbh_matrix *m, const float *x, float *y, float coef, int accumulate,
                           const DevStatus *skip_if) {
    RouterArgs a{};
    a.w = reinterpret_cast<const float *>(m->planes);
    a.x = x;
    a.logits = y;
    a.n_experts = (int32_t)m->rows;
    a.hidden = (int32_t)m->k;
    a.accumulate = accumulate;
    a.coef = coef;
    a.skip_if = skip_if;
    a.timeout = &ctx->status->pad;   // a chain whose bounded wait gave up
    return launch_f32_chains(a, ctx->stream);
}

// gemv_into / gemv_accumulate_scaled_into / the DequantF32 forms on an F32
// matrix (every mode computes dot_f32_row, gemv.rs:88-101, :128-146): the
// accumulate checks and validate_dimensions as check_gemv_args, then
// prepare_dequant's finite-weight check in row-major order (gemv.rs:230-240:
// NonFiniteValue "GEMV weights", index 0 of the one-element decoded block;
// `row` and `actual` give the weight's row and column), then the chains.
lbh_status f32_checked(lbh_ctx *ctx, const lbh_matrix *m, const float *input, size_t input_len, float *out,
                       size_t out_len, int accumulate, float scale, lbh_error *err) {
    DeviceGuard g(ctx->device);
    lbh_status st = check_gemv_args(ctx, m, input, input_len, out, out_len, accumulate, scale, err);
    if (st) return st;
    HIP_TRY(launch_find_nonfinite_f32w(reinterpret_cast<const float *>(m->planes), (long long)m->rows, (long long)m->k,
                                       &ctx->status->first_bad_scale, ctx->stream));
    HIP_TRY(launch_f32_gemv(ctx, m, input, out, scale, accumulate, ctx->status));
    st = scan_verdict(ctx, LBH_F32, input, out, err);
    if (st) return st;
    const unsigned long long w = ctx->status_host->first_bad_scale;
    if (w != ~0ull) {
        const uint64_t r = w / m->k, c = w % m->k;
        const uint32_t bits = read_f32_bits(ctx, reinterpret_cast<const float *>(m->planes) +
                                                      ((c / 4) * m->rows + r) * 4 + c % 4);
        return fail(err, LBH_NON_FINITE_VALUE, LBH_F32, 0, 0, c, bits, 1, r);
    }
    if (ctx->status_host->pad != 0) return fail(err, LBH_DEVICE_TIMEOUT, LBH_F32);
    return ok(err);
}

// prepare_llama_q8k (crates/bridge-kernels-reference/src/gemv.rs:245-272) minus the
// per-row scale scan, which matrix upload performed once.
lbh_status gemv_checked(lbh_ctx *ctx, const lbh_matrix *m, const float *input, size_t input_len, float *out,
                        size_t out_len, uint8_t *q8, size_t q8_len, int accumulate, float scale, lbh_error *err) {
    if (!ctx || !m) return fail(err, LBH_NULL_ARGUMENT);
    // F32: dot_f32_row in every mode; the Q8_K scratch is not used (gemv.rs:88-101).
    if (m->type == LBH_F32) return f32_checked(ctx, m, input, input_len, out, out_len, accumulate, scale, err);
    DeviceGuard g(ctx->device);
    lbh_status st = check_gemv_args(ctx, m, input, input_len, out, out_len, accumulate, scale, err);
    if (st) return st;
    const size_t need = m->k / 256 * 292;
    if (q8_len < need || !q8) {
        st = scan_verdict(ctx, m->type, input, out, err);
        if (st) return st;
        if (!q8) return fail(err, LBH_NULL_ARGUMENT);
        return fail(err, LBH_SCRATCH_TOO_SMALL, LBH_Q8_K, 0, need, q8_len);
    }
    GemvArgs a{};
    a.m = view_of(m);
    a.x = input;        // quantized inside the matvec kernel ...
    a.q8_out = q8;      // ... and published to the caller's scratch (gemv.rs:267)
    a.y = out;
    a.coef = scale;
    a.accumulate = accumulate;
    a.block_sums = nullptr;
    a.status = ctx->status;
    HIP_TRY(launch_gemv(a, ctx->tuning, ctx->stream));
    return scan_verdict(ctx, m->type, input, out, err);
}

// validate_vec_dot_q8_k_inner (crates/bridge-quant-layout/src/q8_k.rs:121-161)
// for `rows` consecutive rows of raw GGML bytes: type, logical elements, exact
// weight and Q8_K lengths, then per row in order the weight scales
// (validate_scales, k_quants.rs:178-208) and the Q8_K scales
// (validate_q8_scales, q8_k.rs:208-222).  Queues the scans (and, when y is
// given, the dot kernel, which skips its writes if a scan fires) and reports
// the first failure in the reference's order.
lbh_status vec_dot_checked(lbh_ctx *ctx, int32_t ty, const uint8_t *w, size_t w_len, size_t rows, const uint8_t *q8,
                           size_t q8_len, size_t n, float *y, size_t y_len, lbh_error *err) {
    if (!ctx) return fail(err, LBH_NULL_ARGUMENT);
    if (!is_dot_type(ty)) return fail(err, LBH_UNSUPPORTED_TYPE, ty);
    lbh_status st = check_elements(ty, n, err);
    if (st) return st;
    if (rows == 0) return fail(err, LBH_DIMENSION_MISMATCH, ty, 0, 1, 0);
    const size_t nb = n / 256, bb = block_bytes(ty);
    if (rows > SIZE_MAX / (nb * bb)) return fail(err, LBH_ARITHMETIC_OVERFLOW, ty);
    const size_t want_w = rows * nb * bb, want_q8 = nb * 292;
    if (w_len != want_w) return fail(err, LBH_ENCODED_LENGTH_MISMATCH, ty, 0, want_w, w_len);
    if (q8_len != want_q8) return fail(err, LBH_ENCODED_LENGTH_MISMATCH, LBH_Q8_K, 0, want_q8, q8_len);
    if (y && y_len != rows) return fail(err, LBH_OUTPUT_LENGTH_MISMATCH, ty, 0, rows, y_len);
    if (!w || !q8) return fail(err, LBH_NULL_ARGUMENT);
    if (nb > 64) return fail(err, LBH_UNSUPPORTED_SHAPE, ty, 0, 64, nb);
    DeviceGuard g(ctx->device);
    const long long U = (long long)(rows * nb);
    HIP_TRY(launch_reset_status(ctx->status, ctx->stream));
    HIP_TRY(launch_validate_scales(ty, w, U, &ctx->status->first_bad_scale, ctx->stream));
    // The first non-finite Q8_K block goes to the input word: the dot kernel skips on it.
    HIP_TRY(launch_find_nonfinite_q8(q8, (long long)nb, &ctx->status->first_bad_input, ctx->stream));
    if (y) HIP_TRY(launch_dot_ggml(ty, w, (long long)rows, (int)nb, q8, y, ctx->status, ctx->stream));
    st = read_status(ctx, err);
    if (st) return st;
    const unsigned long long bad_w = ctx->status_host->first_bad_scale, bad_q8 = ctx->status_host->first_bad_input;
    auto scale_error = [&]() {
        const unsigned long long u = bad_w / 2;
        const uint32_t field = (uint32_t)(bad_w & 1);
        uint16_t bits = 0;
        (void)hipMemcpy(&bits, w + u * bb + 2 * field, 2, hipMemcpyDeviceToHost);
        // NonFiniteScale { ty, block_index, field, bits } (k_quants.rs:196-204) of row u / nb.
        return fail(err, LBH_NON_FINITE_SCALE, ty, u % nb, 0, 0, bits, field, u / nb);
    };
    // Row 0's weight scales precede the Q8_K scales, which precede later rows' weights.
    if (bad_w != ~0ull && bad_w / 2 < nb) return scale_error();
    if (bad_q8 != ~0ull) {
        uint32_t bits = 0;
        (void)hipMemcpy(&bits, q8 + bad_q8 * 292, 4, hipMemcpyDeviceToHost);
        // NonFiniteQ8Scale { block_index, bits } (q8_k.rs:216-219).
        return fail(err, LBH_NON_FINITE_Q8_SCALE, LBH_Q8_K, bad_q8, 0, 0, bits);
    }
    if (bad_w != ~0ull) return scale_error();
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
    if (!is_dot_type(m->type)) return LBH_UNSUPPORTED_TYPE;   // F32: lbh_gemv_into / lbh_gemv_dequant_*
    DeviceGuard g(ctx->device);
    GemvArgs a{};
    a.m = view_of(m);
    a.q8 = q8;
    a.y = y;
    a.coef = coef;
    a.accumulate = accumulate;
    return launch_gemv(a, ctx->tuning, ctx->stream) == hipSuccess ? LBH_OK : LBH_HIP_ERROR;
}

lbh_status lbh_gemv_f32(lbh_ctx *ctx, const lbh_matrix *m, const float *x, uint8_t *q8_out, float *y, float coef,
                        int32_t accumulate) {
    if (!ctx || !m || !x || !y) return LBH_NULL_ARGUMENT;
    if (!is_dot_type(m->type)) return LBH_UNSUPPORTED_TYPE;   // F32: lbh_gemv_into / lbh_gemv_dequant_*
    DeviceGuard g(ctx->device);
    GemvArgs a{};
    a.m = view_of(m);
    a.x = x;
    a.q8_out = q8_out;
    a.y = y;
    a.coef = coef;
    a.accumulate = accumulate;
    return launch_gemv(a, ctx->tuning, ctx->stream) == hipSuccess ? LBH_OK : LBH_HIP_ERROR;
}

lbh_status lbh_gemv_block_sums(lbh_ctx *ctx, const lbh_matrix *m, const uint8_t *q8, int32_t *out) {
    if (!ctx || !m || !q8 || !out) return LBH_NULL_ARGUMENT;
    if (!is_dot_type(m->type)) return LBH_UNSUPPORTED_TYPE;   // F32: lbh_gemv_into / lbh_gemv_dequant_*
    DeviceGuard g(ctx->device);
    GemvArgs a{};
    a.m = view_of(m);
    a.q8 = q8;
    a.y = nullptr;   // the row values are not stored
    a.block_sums = out;
    return launch_gemv(a, ctx->tuning, ctx->stream) == hipSuccess ? LBH_OK : LBH_HIP_ERROR;
}

lbh_status lbh_validate_vec_dot_q8_k(lbh_ctx *ctx, int32_t ty, const uint8_t *weights, size_t weights_len,
                                     size_t rows, const uint8_t *q8, size_t q8_len, size_t logical_elements,
                                     lbh_error *err) {
    return vec_dot_checked(ctx, ty, weights, weights_len, rows, q8, q8_len, logical_elements, nullptr, 0, err);
}

lbh_status lbh_vec_dot_q8_k_into(lbh_ctx *ctx, int32_t ty, const uint8_t *weights, size_t weights_len, size_t rows,
                                 const uint8_t *q8, size_t q8_len, size_t logical_elements, float *out, size_t out_len,
                                 lbh_error *err) {
    if (!out) return fail(err, LBH_NULL_ARGUMENT);
    return vec_dot_checked(ctx, ty, weights, weights_len, rows, q8, q8_len, logical_elements, out, out_len, err);
}

lbh_status lbh_gemv_q8_k_into(lbh_ctx *ctx, const lbh_matrix *m, const uint8_t *q8, size_t q8_len, float *y,
                              size_t y_len, float coef, int32_t accumulate, lbh_error *err) {
    if (!ctx || !m) return fail(err, LBH_NULL_ARGUMENT);
    if (!is_dot_type(m->type)) return fail(err, LBH_UNSUPPORTED_TYPE, m->type);   // prepare_llama_q8k, gemv.rs:252-257
    if (accumulate && !std::isfinite(coef)) {
        uint32_t bits;
        std::memcpy(&bits, &coef, 4);
        return fail(err, LBH_NON_FINITE_VALUE, m->type, 0, 0, 0, bits, 2);
    }
    if (!y) return fail(err, LBH_NULL_ARGUMENT);
    DeviceGuard g(ctx->device);
    HIP_TRY(launch_reset_status(ctx->status, ctx->stream));
    if (accumulate) HIP_TRY(launch_find_nonfinite(y, (long long)y_len, &ctx->status->first_bad_dest, ctx->stream));
    const size_t want_q8 = m->nb * 292;
    if (y_len != m->rows || q8_len != want_q8 || !q8) {
        if (accumulate) {
            lbh_status st = read_status(ctx, err);
            if (st) return st;
            if (ctx->status_host->first_bad_dest != ~0ull) return dest_error(ctx, m->type, y, err);
        }
        if (y_len != m->rows) return fail(err, LBH_DIMENSION_MISMATCH, m->type, 1, m->rows, y_len);
        if (!q8) return fail(err, LBH_NULL_ARGUMENT);
        return fail(err, LBH_ENCODED_LENGTH_MISMATCH, LBH_Q8_K, 0, want_q8, q8_len);
    }
    HIP_TRY(launch_find_nonfinite_q8(q8, (long long)m->nb, &ctx->status->first_bad_input, ctx->stream));
    GemvArgs a{};
    a.m = view_of(m);
    a.q8 = q8;
    a.y = y;
    a.coef = coef;
    a.accumulate = accumulate;
    a.status = ctx->status;
    HIP_TRY(launch_gemv(a, ctx->tuning, ctx->stream));
    lbh_status st = read_status(ctx, err);
    if (st) return st;
    if (ctx->status_host->first_bad_dest != ~0ull) return dest_error(ctx, m->type, y, err);
    const unsigned long long b = ctx->status_host->first_bad_input;
    if (b != ~0ull) {
        uint32_t bits = 0;
        (void)hipMemcpy(&bits, q8 + b * 292, 4, hipMemcpyDeviceToHost);
        return fail(err, LBH_NON_FINITE_Q8_SCALE, LBH_Q8_K, b, 0, 0, bits);
    }
    return ok(err);
}

// DequantF32 mode: gemv_dequant_f32_into (gemv.rs:33-41) and the DequantF32 arm of
// gemv_accumulate_scaled_into (gemv.rs:146-151).  prepare_dequant's per-block
// weight check (gemv.rs:232-240) cannot fire here: upload required finite d /
// dmin, and with finite scales every decoded weight is finite (at most
// 65504 * 63 * 31 in magnitude).  The reference's decoded-block scratch has no
// device counterpart (the kernel decodes into registers).
static lbh_status dequant_checked(lbh_ctx *ctx, const lbh_matrix *m, const float *input, size_t input_len, float *out,
                                  size_t out_len, int accumulate, float scale, lbh_error *err) {
    if (!ctx || !m) return fail(err, LBH_NULL_ARGUMENT);
    if (m->type == LBH_F32) return f32_checked(ctx, m, input, input_len, out, out_len, accumulate, scale, err);
    DeviceGuard g(ctx->device);
    lbh_status st = check_gemv_args(ctx, m, input, input_len, out, out_len, accumulate, scale, err);
    if (st) return st;
    HIP_TRY(launch_gemv_dequant(view_of(m), input, out, scale, accumulate, ctx->status, ctx->stream));
    return scan_verdict(ctx, m->type, input, out, err);
}

lbh_status lbh_gemv_dequant_into(lbh_ctx *ctx, const lbh_matrix *m, const float *input, size_t input_len,
                                 float *output, size_t output_len, lbh_error *err) {
    return dequant_checked(ctx, m, input, input_len, output, output_len, 0, 0.0f, err);
}

lbh_status lbh_gemv_dequant_accumulate_scaled_into(lbh_ctx *ctx, const lbh_matrix *m, const float *input,
                                                   size_t input_len, float *dest, size_t dest_len, float scale,
                                                   lbh_error *err) {
    return dequant_checked(ctx, m, input, input_len, dest, dest_len, 1, scale, err);
}

lbh_status lbh_gemv_dequant_f32(lbh_ctx *ctx, const lbh_matrix *m, const float *x, float *y, float coef,
                                int32_t accumulate) {
    if (!ctx || !m || !x || !y) return LBH_NULL_ARGUMENT;
    DeviceGuard g(ctx->device);
    const hipError_t e = m->type == LBH_F32 ? launch_f32_gemv(ctx, m, x, y, coef, accumulate, nullptr)
                                            : launch_gemv_dequant(view_of(m), x, y, coef, accumulate, nullptr, ctx->stream);
    return e == hipSuccess ? LBH_OK : LBH_HIP_ERROR;
}

lbh_status lbh_debug_empty_kernel(lbh_ctx *ctx) {
    if (!ctx) return LBH_NULL_ARGUMENT;
    DeviceGuard g(ctx->device);
    return launch_empty(ctx->stream) == hipSuccess ? LBH_OK : LBH_HIP_ERROR;
}

lbh_status lbh_debug_read_matrix(lbh_ctx *ctx, const lbh_matrix *m, uint32_t *sink, int32_t grid, int32_t unroll,
                                 int32_t slab) {
    if (!ctx || !m || !sink) return LBH_NULL_ARGUMENT;
    if (grid < 1 || grid > LBH_DEBUG_READ_MAX_GRID || (unroll != 1 && unroll != 2 && unroll != 4 && unroll != 8))
        return LBH_INVALID_PARAMETER;
    DeviceGuard g(ctx->device);
    return launch_stream_read(m->planes, (long long)m->bytes, sink, grid, unroll, slab != 0, ctx->stream) == hipSuccess
               ? LBH_OK
               : LBH_HIP_ERROR;
}

lbh_status lbh_debug_f16_to_f32(lbh_ctx *ctx, const uint16_t *in, float *out, size_t n, lbh_error *err) {
    if (!ctx || !in || !out) return fail(err, LBH_NULL_ARGUMENT);
    DeviceGuard g(ctx->device);
    HIP_TRY(launch_f16_to_f32(in, out, (long long)n, ctx->stream));
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    return ok(err);
}



}  // extern "C"

// ===================================================================== MoE

struct lbh_moe {
    int device;
    size_t n_experts, hidden, ffn_r, ffn_s;   // n_experts = 0: routed experts come from `cache`
    lbh_expert_cache *cache;
    int type_gate_r, type_down_r;
    ExpertDev *experts_dev;
    ExpertDev *experts_host;  // the same table on the host (host-given routing passes planes as arguments)
    ExpertDev shared;
    int has_shared;
    float *h;
    int h_stride;
    MoeStatus *status;
    MoeStatus *status_host;
    int wg_r, wg_s, tile_d;   // gate/up workgroups (routed, shared stream); down rows per workgroup
    int wg_s_given;           // shared-stream workgroups of the routing-given gate/up launch
    // Batched decode scratch (lbh_moe_reserve_batch): capacity and one allocation.
    size_t cap_tokens, cap_k;
    uint8_t *batch_mem;
    BatchArgs batch;          // scratch pointers; per-call fields are filled in per call
    uint32_t *batch_ids;      // device copies of host routing (checked entry)
    float *batch_coefs;
    int32_t *plan_host;       // pinned
    int tc, rt_gu_r, rt_gu_s, rt_d_r, rt_d_s;
    int mx_min;               // batched IQ chunks of >= mx_min tokens on the matrix cores (0: none)
    int mx_split_gu, mx_split_d;   // waves sharing a 16-row tile of those streams (1, 2, 4)
    hipStream_t side;         // batched calls: second stream and fork/join events
    hipEvent_t ev[4];
    uint8_t *shared_gemm_mem; // MFMA-ready copies of a K-quant shared expert (batched calls)
    size_t gemm_off[3];       // A offsets of gate, up, down in shared_gemm_mem
    // Single-token decode with a shared expert: its gate/up and down run on
    // side1 beside the routed experts (fork / join events); d_shared holds its
    // raw down rows for the routed launch's combine.
    hipStream_t side1;
    hipEvent_t sev[2];
    float *d_shared;
    float *dq;                // DequantF32 checked forward: one expert's gate and up values
    int two_stream;           // 1: the async forwards use side1, 0: one stream (default, measured faster)
    // 16-row tile copies of routed IQ matrices for the batched matrix-core
    // streams (lbh_moe_make_batch_tile_copies): one allocation, and the
    // streams' expert table (tile views where copied, else the row-major ones).
    uint8_t *tile_mem;
    size_t tile_bytes;
    ExpertDev *experts_mx_dev;
    int engine_set;           // lbh_moe_set_batch_engine was called: the copies leave the engine alone
};

namespace {

// Batched launch shapes measured on MI355X at the configs[3] shapes (64 tokens,
// hidden 4096, routed ffn 1536): with the matrix cores on, chunks of 16 tokens
// (one instruction's width); the VALU streams alone do best with chunks of 8.
constexpr int MX_MIN_DEFAULT = 4;
void set_batch_defaults(lbh_moe *m, int mx_min) {
    m->mx_min = mx_min;
    m->mx_split_gu = 4, m->mx_split_d = 2;
    m->tc = mx_min > 0 ? 16 : 8;
    m->rt_gu_r = 64, m->rt_gu_s = 64, m->rt_d_r = 160, m->rt_d_s = 64;
}
// With the tile copies (lbh_moe_make_batch_tile_copies) a step's 16 rows of a
// block are two whole lines, so one wave per 16-row tile and chunks from two
// tokens on the matrix cores measured fastest, the VALU keeping the one-token
// chunks (configs[3]: 360-362 us; 369-371 from three tokens, 379 from four;
// without copies the split tiles and 4-token chunks stay the defaults: 430 us
// there against 477-555 us for these settings).
constexpr int MX_MIN_TILED = 2;
void set_engine_for_copies(lbh_moe *m, bool copies) {
    if (m->engine_set) return;
    m->mx_min = copies ? MX_MIN_TILED : MX_MIN_DEFAULT;
    m->mx_split_gu = copies ? 1 : 4;
    m->mx_split_d = copies ? 1 : 2;
}

void free_moe(lbh_moe *m) {
    if (!m) return;
    DeviceGuard g(m->device);
    if (m->experts_dev) (void)hipFree(m->experts_dev);
    delete[] m->experts_host;
    if (m->batch_mem) (void)hipFree(m->batch_mem);
    if (m->shared_gemm_mem) (void)hipFree(m->shared_gemm_mem);
    if (m->tile_mem) (void)hipFree(m->tile_mem);
    if (m->experts_mx_dev) (void)hipFree(m->experts_mx_dev);
    if (m->plan_host) (void)hipHostFree(m->plan_host);
    for (int i = 0; i < 4; ++i)
        if (m->ev[i]) (void)hipEventDestroy(m->ev[i]);
    if (m->side) (void)hipStreamDestroy(m->side);
    for (int i = 0; i < 2; ++i)
        if (m->sev[i]) (void)hipEventDestroy(m->sev[i]);
    if (m->side1) (void)hipStreamDestroy(m->side1);
    if (m->d_shared) (void)hipFree(m->d_shared);
    if (m->h) (void)hipFree(m->h);
    if (m->dq) (void)hipFree(m->dq);
    if (m->status) (void)hipFree(m->status);
    if (m->status_host) (void)hipHostFree(m->status_host);
    delete m;
}

bool moe_types_supported(int gr, int ts_gate, int dr, int ts_down) {
    const bool g = gr == LBH_IQ2_S && (ts_gate == LBH_Q4_K || ts_gate == LBH_IQ2_S);
    const bool d = (dr == LBH_IQ3_S && (ts_down == LBH_Q5_K || ts_down == LBH_IQ3_S)) ||
                   (dr == LBH_IQ2_S && (ts_down == LBH_IQ2_S || ts_down == LBH_IQ3_S));
    return g && d;
}

MoeArgs moe_args(const lbh_moe *m, const float *x, float *y) {
    MoeArgs a{};
    a.experts = m->experts_dev;
    a.shared = m->shared;
    a.has_shared = m->has_shared;
    a.hidden = (int32_t)m->hidden;
    a.ffn_r = (int32_t)m->ffn_r;
    a.ffn_s = (int32_t)(m->has_shared ? m->ffn_s : m->ffn_r);
    a.x = x;
    a.y = y;
    a.h = m->h;
    a.h_stride = m->h_stride;
    a.tiles_r = m->wg_r;
    a.tiles_s = m->has_shared ? m->wg_s_given : 0;
    a.tile_d = m->tile_d;
    a.stop_step = 0x7fffffff;
    a.type_gate_r = m->type_gate_r;
    a.type_down_r = m->type_down_r;
    a.routed_shape = m->experts_host[0];
    a.d_shared = m->d_shared;
    return a;
}

// The shared expert's gate/up and down on the layer's second stream (forked
// from and joined back to `s`) beside the routed launches `routed` enqueues on
// s; the routed down's combine adds d_shared last, the reference's order.
// Captured into a graph, the fork and join become graph edges.
hipError_t forward_two_streams(lbh_moe *m, const MoeArgs &a, hipStream_t s,
                               hipError_t (*routed_gate_up)(const MoeArgs &, hipStream_t)) {
    MoeArgs sh = a;
    sh.gate_part = 2, sh.down_part = 2;
    sh.route_dev = nullptr;            // the shared stream never reads the routing
    sh.select_in_kernel = 0;
    sh.skip_shared_gate_up = 0;
    MoeArgs rt = a;
    rt.gate_part = 1, rt.down_part = 1;
    rt.skip_shared_gate_up = 0;
    hipError_t e = hipEventRecord(m->sev[0], s);
    if (e == hipSuccess) e = hipStreamWaitEvent(m->side1, m->sev[0], 0);
    if (e == hipSuccess) e = launch_moe_gate_up(sh, m->side1);
    if (e == hipSuccess) e = launch_moe_down(sh, m->side1);
    if (e == hipSuccess) e = hipEventRecord(m->sev[1], m->side1);
    if (e == hipSuccess) e = routed_gate_up(rt, s);
    if (e == hipSuccess) e = hipStreamWaitEvent(s, m->sev[1], 0);
    if (e == hipSuccess) e = launch_moe_down(rt, s);
    return e;
}

// Host-given routing: the routed experts' planes go into the arguments.
void set_routed_planes(MoeArgs &a, const lbh_moe *m, const uint32_t *ids, size_t n) {
    a.routed_given = 1;
    for (size_t i = 0; i < n; ++i) {
        const ExpertDev &e = m->experts_host[ids[i]];
        a.routed_planes[i][0] = e.gate.planes;
        a.routed_planes[i][1] = e.up.planes;
        a.routed_planes[i][2] = e.down.planes;
    }
}

// The layer object from validated routed views: `table` (owned) holds the
// n_experts resident experts, or, when n_experts == 0, one entry with the
// routed shape of `cache` (null planes).
lbh_status build_moe(lbh_ctx *ctx, size_t n_experts, ExpertDev *table, lbh_expert_cache *cache, size_t hidden,
                     size_t ffn_r, int tg, int td, size_t gate_bytes, const lbh_matrix *shared_gate,
                     const lbh_matrix *shared_up, const lbh_matrix *shared_down, lbh_moe **out, lbh_error *err) {
    const bool has_shared = shared_gate != nullptr;
    size_t ffn_s = 0;
    if (has_shared) {
        ffn_s = shared_gate->rows;
        if (shared_gate->k != hidden || shared_up->k != hidden || shared_up->rows != ffn_s ||
            shared_up->type != shared_gate->type || shared_down->rows != hidden || shared_down->k != ffn_s) {
            delete[] table;
            return fail(err, LBH_DIMENSION_MISMATCH, shared_gate->type, n_experts, hidden, shared_gate->k);
        }
    }
    if (!moe_types_supported(tg, has_shared ? shared_gate->type : tg, td, has_shared ? shared_down->type : td)) {
        delete[] table;
        return fail(err, LBH_UNSUPPORTED_TYPE, tg);
    }
    if (hidden / 256 > 64 || ffn_r / 256 > 64 || ffn_s / 256 > 64) {
        delete[] table;
        return fail(err, LBH_UNSUPPORTED_SHAPE);
    }
    DeviceGuard guard(ctx->device);
    lbh_moe *m = new (std::nothrow) lbh_moe();
    if (!m) {
        delete[] table;
        return fail(err, LBH_HIP_ERROR);
    }
    m->experts_host = table;
    m->cache = cache;
    m->device = ctx->device;
    m->n_experts = n_experts;
    m->hidden = hidden;
    m->ffn_r = ffn_r;
    m->ffn_s = ffn_s;
    m->type_gate_r = tg;
    m->type_down_r = td;
    m->has_shared = has_shared;
    if (has_shared) {
        m->shared.gate = view_of(shared_gate);
        m->shared.up = view_of(shared_up);
        m->shared.down = view_of(shared_down);
    }
    // Gate/up workgroups (measured on the configs[2] shapes): two per CU for
    // the routed stream.  The shared stream of the routing-given launch takes
    // the rest of one round of resident workgroups (512 + 256 at three per
    // CU: 34.1 us per token, against 35.4 with its byte share of two per CU
    // and 37.5-38.0 once the grid spills into a second round).  Beside the
    // router chains, and in the device-router path's selecting launch, which
    // runs the routed stream on wg_r + wg_s workgroups, the byte share stays
    // (55.7 us per token, 56.3 with a full round): every routed workgroup
    // there selects the route from the logits in its prologue.
    {
        const double br = 8.0 * 2.0 * (double)gate_bytes;
        const double bs = has_shared ? 2.0 * (double)shared_gate->bytes : 0.0;
        const int total = 2 * ctx->cu_count;
        m->wg_s = has_shared ? (int)(total * bs / (br + bs) + 0.5) : 0;
        if (has_shared && m->wg_s < 1) m->wg_s = 1;
        m->wg_r = total;
        m->wg_s_given = m->wg_s;
        if (has_shared) {
            const int round = moe_gate_up_resident_per_cu(tg, shared_gate->type, (int)hidden) * ctx->cu_count;
            if (round - m->wg_r > m->wg_s) m->wg_s_given = round - m->wg_r;
        }
    }
    m->tile_d = 16;
    // The down kernel stages the Q8_K of every routed expert's h (up to
    // MOE_MAX_ROUTED) and the shared expert's in LDS: refuse layers whose
    // largest launch would not fit a workgroup.
    {
        const int lds = moe_down_lds_bytes(td, has_shared ? shared_down->type : td, MOE_MAX_ROUTED, has_shared,
                                           (int)ffn_r, (int)ffn_s, m->tile_d);
        if (lds > MOE_MAX_LDS) {
            free_moe(m);   // owns the table
            return fail(err, LBH_UNSUPPORTED_SHAPE, td, 0, MOE_MAX_LDS, (uint64_t)lds);
        }
    }
    set_batch_defaults(m, MX_MIN_DEFAULT);
    const size_t max_ffn = ffn_r > ffn_s ? ffn_r : ffn_s;
    m->h_stride = (int)max_ffn;
    const size_t slots = MOE_MAX_ROUTED + 1;
    hipError_t e = hipSuccess;
    if (n_experts > 0) {
        e = hipMalloc(&m->experts_dev, n_experts * sizeof(ExpertDev));
        if (e == hipSuccess) e = hipMemcpy(m->experts_dev, table, n_experts * sizeof(ExpertDev), hipMemcpyHostToDevice);
    }
    if (e == hipSuccess) e = hipMalloc(&m->h, slots * max_ffn * sizeof(float));
    if (e == hipSuccess) e = hipMalloc(&m->dq, 2 * max_ffn * sizeof(float));
    if (e == hipSuccess && has_shared) {
        m->two_stream = 0;   // measured slower on MI355X (see lbh_moe_set_streams)
        e = hipMalloc(&m->d_shared, hidden * sizeof(float));
        if (e == hipSuccess) e = hipStreamCreateWithFlags(&m->side1, hipStreamNonBlocking);
        for (int i = 0; i < 2 && e == hipSuccess; ++i) e = hipEventCreateWithFlags(&m->sev[i], hipEventDisableTiming);
    }
    if (e == hipSuccess) e = hipMalloc(&m->status, sizeof(MoeStatus));
    if (e == hipSuccess) e = hipHostMalloc(&m->status_host, sizeof(MoeStatus), hipHostMallocDefault);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) {
        free_moe(m);
        return hip_fail(err, e);
    }
    *out = m;
    return ok(err);
}

}  // namespace

extern "C" {

lbh_status lbh_moe_create(lbh_ctx *ctx, const lbh_matrix *const *gate, const lbh_matrix *const *up,
                          const lbh_matrix *const *down, size_t n_experts, const lbh_matrix *shared_gate,
                          const lbh_matrix *shared_up, const lbh_matrix *shared_down, lbh_moe **out, lbh_error *err) {
    if (!ctx || !out || !gate || !up || !down) return fail(err, LBH_NULL_ARGUMENT);
    *out = nullptr;
    if (n_experts == 0) return fail(err, LBH_DIMENSION_MISMATCH, 0, 3, 1, 0);
    const bool has_shared = shared_gate || shared_up || shared_down;
    if (has_shared && !(shared_gate && shared_up && shared_down)) return fail(err, LBH_NULL_ARGUMENT);
    for (size_t e = 0; e < n_experts; ++e)
        if (!gate[e] || !up[e] || !down[e]) return fail(err, LBH_NULL_ARGUMENT, 0, e);
    const size_t hidden = gate[0]->k, ffn_r = gate[0]->rows;
    const int tg = gate[0]->type, td = down[0]->type;
    // SwiGluExpert shape rules (activation.rs:6-60): gate/up [ffn, hidden], down [hidden, ffn].
    for (size_t e = 0; e < n_experts; ++e) {
        const lbh_matrix *g = gate[e], *u = up[e], *d = down[e];
        if (g->type != tg || u->type != tg || d->type != td) return fail(err, LBH_UNSUPPORTED_TYPE, g->type, e);
        if (g->k != hidden || u->k != hidden) return fail(err, LBH_DIMENSION_MISMATCH, g->type, e, hidden, g->k);
        if (g->rows != ffn_r || u->rows != ffn_r) return fail(err, LBH_DIMENSION_MISMATCH, g->type, e, ffn_r, g->rows);
        if (d->rows != hidden || d->k != ffn_r) return fail(err, LBH_DIMENSION_MISMATCH, d->type, e, hidden, d->rows);
        if (g->device != ctx->device || u->device != ctx->device || d->device != ctx->device)
            return fail(err, LBH_INVALID_PARAMETER, 0, e);
    }
    ExpertDev *table = new (std::nothrow) ExpertDev[n_experts];
    if (!table) return fail(err, LBH_HIP_ERROR);
    for (size_t e = 0; e < n_experts; ++e) {
        table[e].gate = view_of(gate[e]);
        table[e].up = view_of(up[e]);
        table[e].down = view_of(down[e]);
    }
    return build_moe(ctx, n_experts, table, nullptr, hidden, ffn_r, tg, td, gate[0]->bytes, shared_gate, shared_up,
                     shared_down, out, err);
}

lbh_status lbh_moe_destroy(lbh_moe *m) {
    if (!m) return LBH_NULL_ARGUMENT;
    free_moe(m);
    return LBH_OK;
}

lbh_status lbh_moe_set_streams(lbh_moe *m, int32_t two_streams) {
    if (!m) return LBH_NULL_ARGUMENT;
    if (two_streams && !m->side1) return LBH_INVALID_PARAMETER;   // no shared expert
    m->two_stream = two_streams ? 1 : 0;
    return LBH_OK;
}

lbh_status lbh_moe_set_tiles(lbh_moe *m, int32_t wg_routed, int32_t wg_shared, int32_t tile_d) {
    if (!m) return LBH_NULL_ARGUMENT;
    if (wg_routed < 1 || wg_routed > 65536 || wg_shared < 1 || wg_shared > 65536 || tile_d < 1 || tile_d > 256)
        return LBH_INVALID_PARAMETER;
    if (moe_down_lds_bytes(m->type_down_r, m->has_shared ? m->shared.down.type : m->type_down_r, MOE_MAX_ROUTED,
                           m->has_shared, (int)m->ffn_r, (int)m->ffn_s, tile_d) > MOE_MAX_LDS)
        return LBH_UNSUPPORTED_SHAPE;
    m->wg_r = wg_routed;
    m->wg_s = wg_shared;
    m->wg_s_given = wg_shared;
    m->tile_d = tile_d;
    return LBH_OK;
}

lbh_status lbh_moe_forward(lbh_ctx *ctx, lbh_moe *m, const uint32_t *ids, const float *coefs, size_t n_routed,
                           const float *x, float *y) {
    if (!ctx || !m || !ids || !coefs || !x || !y) return LBH_NULL_ARGUMENT;
    if (n_routed == 0 || n_routed > MOE_MAX_ROUTED) return LBH_UNSUPPORTED_SHAPE;
    MoeArgs a = moe_args(m, x, y);
    a.route.n = (int32_t)n_routed;
    for (size_t i = 0; i < n_routed; ++i) {
        if (ids[i] >= m->n_experts) return LBH_INVALID_PARAMETER;   // never index past the expert table
        a.route.ids[i] = ids[i];
        a.route.coefs[i] = coefs[i];
    }
    a.n_launch = (int32_t)n_routed;
    set_routed_planes(a, m, ids, n_routed);
    DeviceGuard g(ctx->device);
    if (m->has_shared && m->two_stream)
        return forward_two_streams(m, a, ctx->stream, launch_moe_gate_up) == hipSuccess ? LBH_OK : LBH_HIP_ERROR;
    if (launch_moe_gate_up(a, ctx->stream) != hipSuccess) return LBH_HIP_ERROR;
    if (launch_moe_down(a, ctx->stream) != hipSuccess) return LBH_HIP_ERROR;
    return LBH_OK;
}

lbh_status lbh_moe_create_cached(lbh_ctx *ctx, lbh_expert_cache *cache, const lbh_matrix *shared_gate,
                                 const lbh_matrix *shared_up, const lbh_matrix *shared_down, lbh_moe **out,
                                 lbh_error *err) {
    if (!ctx || !cache || !out) return fail(err, LBH_NULL_ARGUMENT);
    *out = nullptr;
    const bool has_shared = shared_gate || shared_up || shared_down;
    if (has_shared && !(shared_gate && shared_up && shared_down)) return fail(err, LBH_NULL_ARGUMENT);
    CacheShape sh;
    cache_shape(cache, &sh);
    if (sh.device != ctx->device) return fail(err, LBH_INVALID_PARAMETER);
    ExpertDev *table = new (std::nothrow) ExpertDev[1];
    if (!table) return fail(err, LBH_HIP_ERROR);
    table[0] = sh.views;
    return build_moe(ctx, 0, table, cache, sh.hidden, sh.ffn, sh.type_gate_up, sh.type_down,
                     (size_t)sh.views.gate.bytes, shared_gate, shared_up, shared_down, out, err);
}

// The streaming MoE step of the runtime (hy3_scalar.rs:575-626): the routed
// experts are the leased cache entries, in the caller's (ascending id) order.
lbh_status lbh_moe_forward_leased(lbh_ctx *ctx, lbh_moe *m, const lbh_expert_lease *leases, const float *coefs,
                                  size_t n_routed, const float *x, float *y) {
    if (!ctx || !m || !leases || !coefs || !x || !y) return LBH_NULL_ARGUMENT;
    if (!m->cache) return LBH_INVALID_PARAMETER;
    if (n_routed == 0 || n_routed > MOE_MAX_ROUTED) return LBH_UNSUPPORTED_SHAPE;
    MoeArgs a = moe_args(m, x, y);
    a.route.n = (int32_t)n_routed;
    a.routed_given = 1;
    DeviceGuard g(ctx->device);
    for (size_t i = 0; i < n_routed; ++i) {
        if (i > 0 && leases[i].expert == leases[i - 1].expert) return LBH_DUPLICATE_ROUTED_EXPERT;   // moe.rs:94-105
        if (i > 0 && leases[i].expert < leases[i - 1].expert) return LBH_ROUTED_EXPERT_ORDER;
        const uint8_t *planes[3];
        hipEvent_t ready;
        if (!cache_lease_planes(m->cache, &leases[i], planes, &ready)) return LBH_INVALID_PARAMETER;
        if (hipStreamWaitEvent(ctx->stream, ready, 0) != hipSuccess) return LBH_HIP_ERROR;
        a.route.ids[i] = leases[i].expert;
        a.route.coefs[i] = coefs[i];
        for (int k = 0; k < 3; ++k) a.routed_planes[i][k] = planes[k];
    }
    a.n_launch = (int32_t)n_routed;
    // The slots are read on this call's stream, whichever stream the cache was
    // created on: once the first launch that reads them is queued, every lease
    // records that use, also when a later launch fails (a refill must wait for
    // the queued reader).
    if (launch_moe_gate_up(a, ctx->stream) != hipSuccess) return LBH_HIP_ERROR;
    const bool down_ok = launch_moe_down(a, ctx->stream) == hipSuccess;
    bool noted = true;
    for (size_t i = 0; i < n_routed; ++i) noted = cache_note_use(m->cache, &leases[i], ctx->stream) && noted;
    return down_ok && noted ? LBH_OK : LBH_HIP_ERROR;
}

lbh_status lbh_moe_routed_by_id_into(lbh_ctx *ctx, lbh_moe *m, const uint32_t *ids, const float *coefs,
                                     size_t n_routed, const float *input, size_t input_len, float *output,
                                     size_t output_len, lbh_error *err) {
    if (!ctx || !m) return fail(err, LBH_NULL_ARGUMENT);
    // moe.rs:73-92
    if (n_routed == 0) return fail(err, LBH_DIMENSION_MISMATCH, 0, 3, 1, 0);
    if (input_len != m->hidden) return fail(err, LBH_DIMENSION_MISMATCH, 0, 0, m->hidden, input_len);
    if (output_len != m->hidden) return fail(err, LBH_DIMENSION_MISMATCH, 0, 1, m->hidden, output_len);
    if (!ids || !coefs || !input || !output) return fail(err, LBH_NULL_ARGUMENT);
    if (n_routed > MOE_MAX_ROUTED) return fail(err, LBH_UNSUPPORTED_SHAPE, 0, 0, MOE_MAX_ROUTED, n_routed);
    // Per-expert checks (moe.rs:94-129) run interleaved with that expert's
    // preflight in the reference: find the first failing index here, preflight
    // the experts before it on the device, and report whichever comes first.
    size_t i_host = n_routed;
    lbh_error host_err{};
    for (size_t i = 0; i < n_routed && i_host == n_routed; ++i) {
        uint32_t bits;
        std::memcpy(&bits, &coefs[i], 4);
        if ((bits & 0x7f800000u) == 0x7f800000u) {
            fail(&host_err, LBH_NON_FINITE_VALUE, 0, 0, 0, 0, bits, 6);
            i_host = i;
        } else if (i > 0 && ids[i] == ids[i - 1]) {
            fail(&host_err, LBH_DUPLICATE_ROUTED_EXPERT, 0, ids[i]);
            i_host = i;
        } else if (i > 0 && ids[i] < ids[i - 1]) {
            fail(&host_err, LBH_ROUTED_EXPERT_ORDER, 0, ids[i], ids[i - 1], ids[i]);
            i_host = i;
        } else if (ids[i] >= m->n_experts) {
            fail(&host_err, LBH_INVALID_PARAMETER, 0, ids[i], m->n_experts, ids[i]);
            i_host = i;
        }
    }
    if (i_host == 0) {
        if (err) *err = host_err;
        return (lbh_status)host_err.status;
    }
    DeviceGuard g(ctx->device);
    MoeArgs a = moe_args(m, input, output);
    a.route.n = (int32_t)n_routed;
    for (size_t i = 0; i < i_host; ++i) {
        a.route.ids[i] = ids[i];
        a.route.coefs[i] = coefs[i];
    }
    set_routed_planes(a, m, ids, i_host);
    a.status = m->status;
    a.check = 1;
    a.n_launch = (int32_t)i_host;
    if (i_host < n_routed) a.has_shared = 0;   // the reference stops before the shared preflight
    HIP_TRY(launch_moe_reset_status(m->status, ctx->stream));
    HIP_TRY(launch_find_nonfinite(input, (long long)input_len, &m->status->first_bad_input, ctx->stream));
    HIP_TRY(launch_moe_gate_up(a, ctx->stream));
    if (i_host == n_routed) {
        HIP_TRY(launch_moe_down(a, ctx->stream));
    }
    HIP_TRY(hipMemcpyAsync(m->status_host, m->status, sizeof(MoeStatus), hipMemcpyDeviceToHost, ctx->stream));
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    const MoeStatus st = *m->status_host;
    if (st.first_bad_input != ~0ull)   // gemv_into's validate_dimensions on the first expert
        return fail(err, LBH_NON_FINITE_VALUE, m->type_gate_r, st.first_bad_input, 0, 0,
                    read_f32_bits(ctx, input + st.first_bad_input), 0);
    if (st.first_bad_swiglu != ~0ull) {   // apply_swiglu (activation.rs:170-178)
        const unsigned order = (unsigned)(st.first_bad_swiglu >> 32), lane = (unsigned)st.first_bad_swiglu;
        const int slot = order < n_routed ? (int)order : MOE_SHARED_SLOT;
        return fail(err, LBH_NON_FINITE_VALUE, 0, lane, 0, 0,
                    read_f32_bits(ctx, m->h + (size_t)slot * m->h_stride + lane), 5);
    }
    if (i_host < n_routed) {
        if (err) *err = host_err;
        return (lbh_status)host_err.status;
    }
    if (st.first_bad_fold != ~0ull) {
        // The accumulation call after step i* rejects the non-finite
        // destination (gemv.rs:126-127), leaving the output as it stood after
        // step i*: recompute the combine up to that step.
        const int step = (int)(st.first_bad_fold >> 32);
        const unsigned row = (unsigned)st.first_bad_fold;
        a.check = 0;
        a.stop_step = step;
        HIP_TRY(launch_moe_down(a, ctx->stream));
        HIP_TRY(hipStreamSynchronize(ctx->stream));
        return fail(err, LBH_NON_FINITE_VALUE, 0, row, 0, 0, read_f32_bits(ctx, output + row), 3);
    }
    return ok(err);
}

// moe_routed_by_id_into in the DequantF32 mode (moe.rs:64-147 with
// ReferenceExecutionMode::DequantF32, the mode of the CLI's dequant-f32
// backend): every matvec is dot_dequant_row (gemv_dequant_f32_into,
// gemv.rs:33-41), on the f32 input with no Q8_K step.  The reference's order:
// per routed expert its checks (moe.rs:94-129) and its preflight
// (swiglu_project_into: gate, up, SwiGLU, down into scratch), the shared
// expert's preflight, then output.fill(0) and one accumulating pass per expert
// in id order and the shared expert at 1.0 (expert_swiglu_accumulate_into,
// activation.rs:104-144), each first rejecting a non-finite destination
// (gemv.rs:126-127).  The preflight's down projection cannot fail (its input
// h was just checked finite and uploaded weights decode finite), so only gate,
// up and SwiGLU run there, and the accumulating passes reuse that h (the same
// values the reference computes again).
lbh_status lbh_moe_routed_by_id_dequant_f32_into(lbh_ctx *ctx, lbh_moe *m, const uint32_t *ids, const float *coefs,
                                                 size_t n_routed, const float *input, size_t input_len, float *output,
                                                 size_t output_len, lbh_error *err) {
    if (!ctx || !m) return fail(err, LBH_NULL_ARGUMENT);
    if (n_routed == 0) return fail(err, LBH_DIMENSION_MISMATCH, 0, 3, 1, 0);
    if (input_len != m->hidden) return fail(err, LBH_DIMENSION_MISMATCH, 0, 0, m->hidden, input_len);
    if (output_len != m->hidden) return fail(err, LBH_DIMENSION_MISMATCH, 0, 1, m->hidden, output_len);
    if (!ids || !coefs || !input || !output) return fail(err, LBH_NULL_ARGUMENT);
    if (n_routed > MOE_MAX_ROUTED) return fail(err, LBH_UNSUPPORTED_SHAPE, 0, 0, MOE_MAX_ROUTED, n_routed);
    DeviceGuard g(ctx->device);
    // The first routed expert's gate gemv_into scans the input (gemv.rs:195-211)
    // after that expert's own checks.
    auto input_scan = [&]() -> lbh_status {
        HIP_TRY(launch_reset_status(ctx->status, ctx->stream));
        HIP_TRY(launch_find_nonfinite(input, (long long)input_len, &ctx->status->first_bad_input, ctx->stream));
        const lbh_status st = read_status(ctx, err);
        if (st) return st;
        if (ctx->status_host->first_bad_input != ~0ull) return input_error(ctx, m->type_gate_r, input, err);
        return LBH_OK;
    };
    float *gbuf = m->dq, *ubuf = m->dq + m->h_stride;
    auto preflight = [&](const ExpertDev &e, int slot, size_t ffn) -> lbh_status {
        float *h = m->h + (size_t)slot * m->h_stride;
        HIP_TRY(launch_gemv_dequant(e.gate, input, gbuf, 0.0f, 0, nullptr, ctx->stream));
        HIP_TRY(launch_gemv_dequant(e.up, input, ubuf, 0.0f, 0, nullptr, ctx->stream));
        HIP_TRY(launch_expf(gbuf, h, (long long)ffn, 1, ubuf, ctx->stream));   // SwiGLU, activation.rs:170-178
        HIP_TRY(launch_reset_status(ctx->status, ctx->stream));
        HIP_TRY(launch_find_nonfinite(h, (long long)ffn, &ctx->status->first_bad_input, ctx->stream));
        const lbh_status st = read_status(ctx, err);
        if (st) return st;
        const unsigned long long bad = ctx->status_host->first_bad_input;
        if (bad != ~0ull) return fail(err, LBH_NON_FINITE_VALUE, 0, bad, 0, 0, read_f32_bits(ctx, h + bad), 5);
        return LBH_OK;
    };
    for (size_t i = 0; i < n_routed; ++i) {
        uint32_t bits;
        std::memcpy(&bits, &coefs[i], 4);
        if ((bits & 0x7f800000u) == 0x7f800000u) return fail(err, LBH_NON_FINITE_VALUE, 0, 0, 0, 0, bits, 6);
        if (i > 0 && ids[i] == ids[i - 1]) return fail(err, LBH_DUPLICATE_ROUTED_EXPERT, 0, ids[i]);
        if (i > 0 && ids[i] < ids[i - 1]) return fail(err, LBH_ROUTED_EXPERT_ORDER, 0, ids[i], ids[i - 1], ids[i]);
        if (ids[i] >= m->n_experts) return fail(err, LBH_INVALID_PARAMETER, 0, ids[i], m->n_experts, ids[i]);
        lbh_status st = i == 0 ? input_scan() : LBH_OK;
        if (!st) st = preflight(m->experts_host[ids[i]], (int)i, m->ffn_r);
        if (st) return st;
    }
    if (m->has_shared) {
        const lbh_status st = preflight(m->shared, MOE_SHARED_SLOT, m->ffn_s);
        if (st) return st;
    }
    // output.fill(0.0) (moe.rs:141), then the accumulating passes.  A [sync]
    // entry point: its memset never goes into a captured graph.
    HIP_TRY(hipMemsetAsync(output, 0, output_len * sizeof(float), ctx->stream));
    auto accumulate = [&](const MatView &down, int slot, float coef) -> lbh_status {
        HIP_TRY(launch_reset_status(ctx->status, ctx->stream));
        HIP_TRY(launch_find_nonfinite(output, (long long)output_len, &ctx->status->first_bad_dest, ctx->stream));
        HIP_TRY(launch_gemv_dequant(down, m->h + (size_t)slot * m->h_stride, output, coef, 1, ctx->status,
                                    ctx->stream));
        const lbh_status st = read_status(ctx, err);
        if (st) return st;
        if (ctx->status_host->first_bad_dest != ~0ull) return dest_error(ctx, 0, output, err);
        return LBH_OK;
    };
    for (size_t i = 0; i < n_routed; ++i) {
        const lbh_status st = accumulate(m->experts_host[ids[i]].down, (int)i, coefs[i]);
        if (st) return st;
    }
    if (m->has_shared) {
        const lbh_status st = accumulate(m->shared.down, MOE_SHARED_SLOT, 1.0f);
        if (st) return st;
    }
    return ok(err);
}

lbh_status lbh_debug_expf(lbh_ctx *ctx, const float *in, float *out, size_t n, int32_t swiglu, const float *up,
                          lbh_error *err) {
    if (!ctx || !in || !out || (swiglu && !up)) return fail(err, LBH_NULL_ARGUMENT);
    DeviceGuard g(ctx->device);
    HIP_TRY(launch_expf(in, out, (long long)n, swiglu, up, ctx->stream));
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    return ok(err);
}

void lbh_debug_expf_host(const float *in, float *out, size_t n, int32_t swiglu, const float *up) {
    for (size_t i = 0; i < n; ++i) out[i] = swiglu ? swiglu_ref(in[i], up[i]) : expf_libm(in[i]);
}

}  // extern "C"

// ================================================================== K-quant GEMM (token batches)

namespace {

MatGemm gemm_view(const lbh_matrix *m, float *y, int ldy) {
    MatGemm g;
    g.a = m->gemm_a;
    g.y = y;
    g.rows = (int32_t)m->rows;
    g.ldy = ldy;
    return g;
}

hipError_t prepare_gemm(lbh_matrix *m, hipStream_t s) {
    if (m->gemm_a) return hipSuccess;
    const int rows = (int)m->rows, nb = (int)m->nb;
    hipError_t e = hipMalloc(&m->gemm_a, gemm_a_bytes(rows, nb));
    if (e == hipSuccess) e = launch_prep_a(view_of(m), m->gemm_a, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) {
        if (m->gemm_a) (void)hipFree(m->gemm_a);
        m->gemm_a = nullptr;
    }
    return e;
}

}  // namespace

extern "C" {

lbh_status lbh_matrix_prepare_gemm(lbh_ctx *ctx, lbh_matrix *m, lbh_error *err) {
    if (!ctx || !m) return fail(err, LBH_NULL_ARGUMENT);
    if (m->type != LBH_Q4_K && m->type != LBH_Q5_K) return fail(err, LBH_UNSUPPORTED_TYPE, m->type);
    if (m->device != ctx->device) return fail(err, LBH_INVALID_PARAMETER);
    DeviceGuard g(ctx->device);
    HIP_TRY(prepare_gemm(m, ctx->stream));
    return ok(err);
}

size_t lbh_matrix_device_bytes(const lbh_matrix *m) {
    if (!m) return 0;
    return m->bytes + (m->gemm_a ? gemm_a_bytes((int)m->rows, (int)m->nb) : 0);
}

size_t lbh_gemm_workspace_bytes(size_t n_tokens, size_t k) {
    if (n_tokens == 0 || k == 0 || k % 256) return 0;
    return gemm_b_bytes((int)n_tokens, (int)(k / 256));
}

}  // extern "C"

namespace {

// The activation tiles go to `bt` (the caller's workspace or this device's
// static scratch), then the GEMM reads them: no allocation either way.
lbh_status gemm_q8_k_into(lbh_ctx *ctx, const lbh_matrix *m, const uint8_t *q8, size_t n_tokens, float *y,
                          uint8_t *bt) {
    const int nb = (int)m->nb;
    DeviceGuard g(ctx->device);
    GemmArgs a{};
    a.b = bt;
    a.nb = nb;
    a.n_tokens = (int32_t)n_tokens;
    a.n_mat = 1;
    a.shape = ctx->gemm_shape;
    a.mat[0] = gemm_view(m, y, (int)m->rows);
    if (launch_prep_b(q8, (int)n_tokens, nb, bt, ctx->stream) != hipSuccess)
        return LBH_HIP_ERROR;
    return launch_kq_gemm(a, ctx->stream) == hipSuccess ? LBH_OK : LBH_HIP_ERROR;
}

}  // namespace

extern "C" {

lbh_status lbh_gemm_q8_k(lbh_ctx *ctx, const lbh_matrix *m, const uint8_t *q8, size_t n_tokens, float *y,
                         void *workspace, size_t workspace_len) {
    if (!ctx || !m || !q8 || !y || !workspace) return LBH_NULL_ARGUMENT;
    if (!m->gemm_a) return LBH_INVALID_PARAMETER;   // lbh_matrix_prepare_gemm first
    if (n_tokens == 0 || n_tokens > (size_t)1 << 20) return LBH_UNSUPPORTED_SHAPE;
    if (workspace_len < gemm_b_bytes((int)n_tokens, (int)m->nb)) return LBH_SCRATCH_TOO_SMALL;
    return gemm_q8_k_into(ctx, m, q8, n_tokens, y, static_cast<uint8_t *>(workspace));
}

lbh_status lbh_gemm_q8_k_noalloc(lbh_ctx *ctx, const lbh_matrix *m, const uint8_t *q8, size_t n_tokens, float *y,
                                 lbh_error *err) {
    if (!ctx || !m || !q8 || !y) return fail(err, LBH_NULL_ARGUMENT);
    if (!m->gemm_a) return fail(err, LBH_INVALID_PARAMETER, m->type);   // lbh_matrix_prepare_gemm first
    if (!ctx->scratch) return fail(err, LBH_HIP_ERROR);
    if (n_tokens == 0 || n_tokens > (size_t)1 << 20) return fail(err, LBH_UNSUPPORTED_SHAPE, m->type, 0, 1, n_tokens);
    const size_t need = gemm_b_bytes((int)n_tokens, (int)m->nb);
    if (need > LBH_NOALLOC_SCRATCH_BYTES)
        return fail(err, LBH_SCRATCH_TOO_SMALL, LBH_Q8_K, n_tokens, need, LBH_NOALLOC_SCRATCH_BYTES);
    // Eager calls: refuse a call on another stream while the last one is
    // pending, then mark this one.  Under stream capture nothing runs yet and
    // events may be neither queried nor recorded: the caller orders replays.
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    const hipError_t ce = hipStreamIsCapturing(ctx->stream, &cap);
    if (ce != hipSuccess) return hip_fail(err, ce);
    const bool eager = cap == hipStreamCaptureStatusNone;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    ScratchUse &use = g_scratch_use[ctx->device];
    if (eager && use.pending && use.last != ctx->stream) {
        const hipError_t q = hipEventQuery(use.done);
        if (q == hipErrorNotReady) return fail(err, LBH_SCRATCH_IN_USE, LBH_Q8_K, 0, 0, n_tokens);
        if (q != hipSuccess) return hip_fail(err, q);
        use.pending = false;
    }
    const lbh_status st = gemm_q8_k_into(ctx, m, q8, n_tokens, y, ctx->scratch);
    if (st != LBH_OK) return fail(err, st);
    if (eager) {
        DeviceGuard g(ctx->device);
        const hipError_t re = hipEventRecord(use.done, ctx->stream);
        if (re != hipSuccess) return hip_fail(err, re);
        use.last = ctx->stream;
        use.pending = true;
    }
    return ok(err);
}

}  // extern "C"

// ================================================================== batched MoE decode

namespace {

BatchArgs batch_args(const lbh_moe *m, const uint32_t *ids, const float *coefs, size_t n_tokens, size_t top_k,
                     const float *x, float *y) {
    BatchArgs a = m->batch;
    a.experts = m->experts_dev;
    a.experts_mx = m->experts_mx_dev ? m->experts_mx_dev : m->experts_dev;
    a.shared = m->shared;
    a.has_shared = m->has_shared;
    a.hidden = (int32_t)m->hidden;
    a.ffn_r = (int32_t)m->ffn_r;
    a.ffn_s = (int32_t)(m->has_shared ? m->ffn_s : m->ffn_r);
    a.n_experts = (int32_t)m->n_experts;
    a.n_tokens = (int32_t)n_tokens;
    a.top_k = (int32_t)top_k;
    a.ids = ids;
    a.coefs = coefs;
    a.x = x;
    a.y = y;
    const long long pairs = (long long)n_tokens * (long long)top_k;
    const long long hit = pairs < (long long)m->n_experts ? pairs : (long long)m->n_experts;
    // Chunks per expert are ceil(count / tc): at most pairs / tc + (experts hit).
    long long mc = pairs / m->tc + hit;
    a.max_chunks = (int32_t)(mc < pairs ? mc : pairs);
    a.tc = m->tc;
    a.rt_gu_r = m->rt_gu_r;
    a.rt_gu_s = m->rt_gu_s;
    a.rt_d_r = m->rt_d_r;
    a.rt_d_s = m->rt_d_s;
    a.type_gate_r = m->type_gate_r;
    a.type_down_r = m->type_down_r;
    a.mx = m->mx_min > 0 ? 1 : 0;
    a.mx_min = m->mx_min > 0 ? m->mx_min : BATCH_MAX_TC + 1;
    a.mx_split_gu = m->mx_split_gu;
    a.mx_split_d = m->mx_split_d;
    a.vc = a.mx ? (a.tc < a.mx_min - 1 ? a.tc : a.mx_min - 1) : a.tc;
    if (a.vc < 1) a.vc = 1;
    return a;
}

bool is_kquant(int ty) { return ty == LBH_Q4_K || ty == LBH_Q5_K; }

BatchStreams batch_streams(const lbh_moe *m) {
    BatchStreams b{};
    b.side = m->side;
    b.fork[0] = m->ev[0], b.fork[1] = m->ev[1], b.join[0] = m->ev[2], b.join[1] = m->ev[3];
    return b;
}

}  // namespace

extern "C" {

lbh_status lbh_moe_reserve_batch(lbh_moe *m, size_t max_tokens, size_t top_k, lbh_error *err) {
    if (!m) return fail(err, LBH_NULL_ARGUMENT);
    if (max_tokens == 0 || max_tokens > (size_t)BATCH_MAX_TOKENS)
        return fail(err, LBH_UNSUPPORTED_SHAPE, 0, 0, BATCH_MAX_TOKENS, max_tokens);
    if (top_k == 0 || top_k > (size_t)MOE_MAX_ROUTED || top_k > m->n_experts)
        return fail(err, LBH_UNSUPPORTED_SHAPE, 0, 1, MOE_MAX_ROUTED, top_k);
    if (m->n_experts > (size_t)BATCH_MAX_EXPERTS) return fail(err, LBH_UNSUPPORTED_SHAPE, 0, 2, BATCH_MAX_EXPERTS, m->n_experts);
    const int tsg = m->has_shared ? m->shared.gate.type : LBH_IQ2_S;
    const int tsd = m->has_shared ? m->shared.down.type : LBH_IQ3_S;
    if (!batch_types_supported(m->type_gate_r, m->type_down_r, tsg, tsd)) return fail(err, LBH_UNSUPPORTED_TYPE, m->type_gate_r);
    DeviceGuard g(m->device);
    if (m->batch_mem) {
        (void)hipFree(m->batch_mem);
        m->batch_mem = nullptr;
    }
    const size_t T = max_tokens, P = max_tokens * top_k;
    const size_t nbh = m->hidden / 256, nbr = m->ffn_r / 256, ffn_s = m->has_shared ? m->ffn_s : m->ffn_r;
    const size_t nbs = ffn_s / 256;
    size_t off = 0;
    auto take = [&](size_t bytes) {
        const size_t o = off;
        off += (bytes + 255) & ~(size_t)255;
        return o;
    };
    const size_t o_plan = take(16), o_ce = take(P * 4), o_cp = take(P * 4), o_cn = take(P * 4);
    const size_t o_pt = take(P * 4), o_po = take(P * 4);
    const size_t o_q8x = take(T * nbh * 292), o_q8xr = take(T * nbh * 292);
    const size_t o_gr = take(P * m->ffn_r * 4), o_ur = take(P * m->ffn_r * 4);
    const size_t o_gs = take(T * ffn_s * 4), o_us = take(T * ffn_s * 4);
    const size_t o_q8hr = take(P * nbr * 292), o_q8hs = take(T * nbs * 292);
    const size_t o_dr = take(P * m->hidden * 4), o_ds = take(T * m->hidden * 4);
    const size_t o_ids = take(P * 4), o_coefs = take(P * 4);
    // operand copies of the Q8_K rows for the matrix-core IQ streams
    const size_t o_xqm = take(T * nbh * 256), o_xdm = take(T * nbh * 4);
    const size_t o_hqr = take(P * nbr * 256), o_hdr = take(P * nbr * 4);
    const size_t o_hqs = take(T * nbs * 256), o_hds = take(T * nbs * 4);
    // A K-quant shared expert runs on the matrix cores: gate/up outputs and the
    // GEMM activation tiles of x and of the shared h.
    const bool sgemm = m->has_shared && is_kquant(m->shared.gate.type) && is_kquant(m->shared.down.type);
    size_t o_bx = 0, o_bh = 0;
    if (sgemm) {
        o_bx = take(gemm_b_bytes((int)T, (int)nbh));
        o_bh = take(gemm_b_bytes((int)T, (int)nbs));
    }
    hipError_t e = hipMalloc(&m->batch_mem, off);
    if (e == hipSuccess) e = hipMemset(m->batch_mem, 0, off);
    // default priority, non-blocking: it only ever waits on the caller's stream through events
    if (e == hipSuccess && !m->side) e = hipStreamCreateWithFlags(&m->side, hipStreamNonBlocking);
    for (int i = 0; i < 4 && e == hipSuccess; ++i)
        if (!m->ev[i]) e = hipEventCreateWithFlags(&m->ev[i], hipEventDisableTiming);
    if (e == hipSuccess && !m->plan_host) e = hipHostMalloc(&m->plan_host, 16, hipHostMallocDefault);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) {
        if (m->batch_mem) (void)hipFree(m->batch_mem);
        m->batch_mem = nullptr;
        m->cap_tokens = m->cap_k = 0;
        return hip_fail(err, e);
    }
    uint8_t *b = m->batch_mem;
    BatchArgs &a = m->batch;
    a = BatchArgs{};
    a.plan = reinterpret_cast<int32_t *>(b + o_plan);
    a.chunk_expert = reinterpret_cast<int32_t *>(b + o_ce);
    a.chunk_p0 = reinterpret_cast<int32_t *>(b + o_cp);
    a.chunk_n = reinterpret_cast<int32_t *>(b + o_cn);
    a.pair_token = reinterpret_cast<int32_t *>(b + o_pt);
    a.pair_of = reinterpret_cast<int32_t *>(b + o_po);
    a.q8x = b + o_q8x;
    a.q8x_rm = b + o_q8xr;
    a.g_r = reinterpret_cast<float *>(b + o_gr);
    a.u_r = reinterpret_cast<float *>(b + o_ur);
    a.g_s = reinterpret_cast<float *>(b + o_gs);
    a.u_s = reinterpret_cast<float *>(b + o_us);
    a.q8h_r = b + o_q8hr;
    a.q8h_s = b + o_q8hs;
    a.d_r = reinterpret_cast<float *>(b + o_dr);
    a.d_s = reinterpret_cast<float *>(b + o_ds);
    a.xq_mx = b + o_xqm;
    a.xd_mx = reinterpret_cast<float *>(b + o_xdm);
    a.hq_mx_r = b + o_hqr;
    a.hd_mx_r = reinterpret_cast<float *>(b + o_hdr);
    a.hq_mx_s = b + o_hqs;
    a.hd_mx_s = reinterpret_cast<float *>(b + o_hds);
    m->batch_ids = reinterpret_cast<uint32_t *>(b + o_ids);
    m->batch_coefs = reinterpret_cast<float *>(b + o_coefs);
    a.shared_gemm = sgemm ? 1 : 0;
    if (sgemm) {
        a.bx = b + o_bx;
        a.bh = b + o_bh;
        if (!m->shared_gemm_mem) {
            // MFMA-ready copies of the shared gate, up and down (built once).
            const MatView v[3] = {m->shared.gate, m->shared.up, m->shared.down};
            size_t so = 0, oa[3];
            for (int i = 0; i < 3; ++i) {
                oa[i] = so;
                so += (gemm_a_bytes(v[i].rows, v[i].nb) + 255) & ~(size_t)255;
            }
            e = hipMalloc(&m->shared_gemm_mem, so);
            for (int i = 0; i < 3 && e == hipSuccess; ++i) e = launch_prep_a(v[i], m->shared_gemm_mem + oa[i], nullptr);
            if (e == hipSuccess) e = hipDeviceSynchronize();
            if (e != hipSuccess) {
                if (m->shared_gemm_mem) (void)hipFree(m->shared_gemm_mem);
                m->shared_gemm_mem = nullptr;
                (void)hipFree(m->batch_mem);
                m->batch_mem = nullptr;
                m->cap_tokens = m->cap_k = 0;
                return hip_fail(err, e);
            }
            m->gemm_off[0] = oa[0], m->gemm_off[1] = oa[1], m->gemm_off[2] = oa[2];
        }
        uint8_t *g = m->shared_gemm_mem;
        const int ffs = (int)ffn_s, hid = (int)m->hidden;
        a.sg = MatGemm{g + m->gemm_off[0], a.g_s, ffs, ffs};
        a.su = MatGemm{g + m->gemm_off[1], a.u_s, ffs, ffs};
        a.sd = MatGemm{g + m->gemm_off[2], a.d_s, hid, hid};
    }
    m->cap_tokens = max_tokens;
    m->cap_k = top_k;
    return ok(err);
}

lbh_status lbh_moe_set_batch_tiles(lbh_moe *m, int32_t tokens_per_chunk, int32_t rows_gate_up_routed,
                                   int32_t rows_gate_up_shared, int32_t rows_down_routed, int32_t rows_down_shared) {
    if (!m) return LBH_NULL_ARGUMENT;
    if (tokens_per_chunk < 1 || tokens_per_chunk > BATCH_MAX_TC) return LBH_INVALID_PARAMETER;
    const int v[4] = {rows_gate_up_routed, rows_gate_up_shared, rows_down_routed, rows_down_shared};
    for (int i = 0; i < 4; ++i)
        if (v[i] < 1 || v[i] > 65536) return LBH_INVALID_PARAMETER;
    const int tc_old = m->tc;
    m->tc = tokens_per_chunk;
    const BatchArgs probe = batch_args(m, nullptr, nullptr, 1, 1, nullptr, nullptr);
    m->tc = tc_old;
    for (int st = 0; st < 5; ++st)
        if (batch_lds_bytes(probe, st) > 160 * 1024) return LBH_UNSUPPORTED_SHAPE;
    m->tc = tokens_per_chunk;
    m->rt_gu_r = v[0], m->rt_gu_s = v[1], m->rt_d_r = v[2], m->rt_d_s = v[3];
    return LBH_OK;
}

lbh_status lbh_moe_set_batch_engine(lbh_moe *m, int32_t mx_min_tokens, int32_t mx_rows_gate_up,
                                    int32_t mx_rows_down) {
    if (!m) return LBH_NULL_ARGUMENT;
    auto rows_ok = [](int32_t r) { return r == 0 || r == 16 || r == 32 || r == 64; };
    if (mx_min_tokens < 0 || mx_min_tokens > BATCH_MAX_TC || !rows_ok(mx_rows_gate_up) || !rows_ok(mx_rows_down))
        return LBH_INVALID_PARAMETER;
    const lbh_moe saved = *m;
    set_batch_defaults(m, mx_min_tokens);
    if (mx_rows_gate_up) m->mx_split_gu = 64 / mx_rows_gate_up;
    if (mx_rows_down) m->mx_split_d = 64 / mx_rows_down;
    const BatchArgs probe = batch_args(m, nullptr, nullptr, 1, 1, nullptr, nullptr);
    for (int st = 0; st < 5; ++st)
        if (batch_lds_bytes(probe, st) > 160 * 1024) {
            *m = saved;
            return LBH_UNSUPPORTED_SHAPE;
        }
    m->engine_set = 1;
    return LBH_OK;
}

lbh_status lbh_moe_make_batch_tile_copies(lbh_ctx *ctx, lbh_moe *m, const uint32_t *experts, size_t n_experts,
                                          lbh_error *err) {
    if (!ctx || !m || (!experts && n_experts > 0)) return fail(err, LBH_NULL_ARGUMENT);
    if (m->n_experts == 0 || !m->experts_host) return fail(err, LBH_INVALID_PARAMETER);   // cache-backed layer
    if (ctx->device != m->device) return fail(err, LBH_INVALID_PARAMETER);
    for (size_t i = 0; i < n_experts; ++i)
        if (experts[i] >= m->n_experts) return fail(err, LBH_INVALID_PARAMETER, 0, i, m->n_experts, experts[i]);
    // experts == NULL: every routed expert; an empty list drops the copies.
    std::unique_ptr<char[]> pick(new (std::nothrow) char[m->n_experts]());
    if (!pick) return fail(err, LBH_HIP_ERROR);
    for (size_t e = 0; e < m->n_experts; ++e) pick[e] = experts ? 0 : 1;
    for (size_t i = 0; i < n_experts; ++i) pick[experts[i]] = 1;
    // The matrix-core streams' matrices: IQ2_S / IQ3_S, whole 16-row tiles.
    auto copyable = [](const MatView &v) { return (v.type == LBH_IQ2_S || v.type == LBH_IQ3_S) && v.rows % 16 == 0; };
    auto align = [](size_t b) { return (b + 255) & ~(size_t)255; };
    size_t total = 0;
    for (size_t e = 0; e < m->n_experts; ++e) {
        if (!pick[e]) continue;
        const ExpertDev &x = m->experts_host[e];
        for (const MatView *v : {&x.gate, &x.up, &x.down})
            if (copyable(*v)) total += align((size_t)v->bytes);
    }
    DeviceGuard g(ctx->device);
    uint8_t *mem = nullptr;
    ExpertDev *table = nullptr;
    std::unique_ptr<ExpertDev[]> host(new (std::nothrow) ExpertDev[m->n_experts]);
    if (!host) return fail(err, LBH_HIP_ERROR);
    if (total > 0) {
        hipError_t e = hipMalloc(&mem, total);
        if (e == hipSuccess) e = hipMalloc(&table, m->n_experts * sizeof(ExpertDev));
        size_t off = 0;
        for (size_t x = 0; x < m->n_experts && e == hipSuccess; ++x) {
            host[x] = m->experts_host[x];
            if (!pick[x]) continue;
            for (MatView *v : {&host[x].gate, &host[x].up, &host[x].down}) {
                if (!copyable(*v) || e != hipSuccess) continue;
                e = launch_units_to_tiles(*v, mem + off, ctx->stream);
                v->planes = mem + off;
                v->order = MAT_TILE16;
                off += align((size_t)v->bytes);
            }
        }
        if (e == hipSuccess)
            e = hipMemcpyAsync(table, host.get(), m->n_experts * sizeof(ExpertDev), hipMemcpyHostToDevice, ctx->stream);
        if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
        if (e != hipSuccess) {
            (void)hipStreamSynchronize(ctx->stream);
            if (mem) (void)hipFree(mem);
            if (table) (void)hipFree(table);
            return hip_fail(err, e);
        }
    }
    // Batched calls still in flight on any stream may read the old copies.
    if (m->tile_mem || m->experts_mx_dev) {
        HIP_TRY(hipDeviceSynchronize());
        if (m->tile_mem) (void)hipFree(m->tile_mem);
        if (m->experts_mx_dev) (void)hipFree(m->experts_mx_dev);
    }
    m->tile_mem = mem;
    m->tile_bytes = total;
    m->experts_mx_dev = table;
    set_engine_for_copies(m, table != nullptr);
    return ok(err);
}

size_t lbh_moe_batch_tile_copy_bytes(const lbh_moe *m) { return m ? m->tile_bytes : 0; }

static lbh_status forward_batch(lbh_ctx *ctx, lbh_moe *m, const uint32_t *ids, const float *coefs, size_t n_tokens,
                                size_t top_k, const float *x, float *y, int residual) {
    if (!ctx || !m || !ids || !coefs || !x || !y) return LBH_NULL_ARGUMENT;
    if (n_tokens == 0 || top_k == 0) return LBH_DIMENSION_MISMATCH;
    if (!m->batch_mem || n_tokens > m->cap_tokens || top_k > m->cap_k) return LBH_SCRATCH_TOO_SMALL;
    DeviceGuard g(ctx->device);
    BatchArgs a = batch_args(m, ids, coefs, n_tokens, top_k, x, y);
    a.residual = residual;
    a.gemm_shape = ctx->gemm_shape;
    const BatchStreams bs = batch_streams(m);
    if (launch_moe_batch(a, ctx->stream, &bs) != hipSuccess) return LBH_HIP_ERROR;
    return LBH_OK;
}

lbh_status lbh_moe_forward_batch(lbh_ctx *ctx, lbh_moe *m, const uint32_t *ids, const float *coefs, size_t n_tokens,
                                 size_t top_k, const float *x, float *y) {
    return forward_batch(ctx, m, ids, coefs, n_tokens, top_k, x, y, 0);
}

lbh_status lbh_moe_forward_batch_residual(lbh_ctx *ctx, lbh_moe *m, const uint32_t *ids, const float *coefs,
                                          size_t n_tokens, size_t top_k, const float *x, float *hidden) {
    return forward_batch(ctx, m, ids, coefs, n_tokens, top_k, x, hidden, 1);
}

lbh_status lbh_moe_routed_by_id_batch_into(lbh_ctx *ctx, lbh_moe *m, const uint32_t *ids, const float *coefs,
                                           size_t n_tokens, size_t top_k, const float *input, size_t input_len,
                                           float *output, size_t output_len, lbh_error *err) {
    if (!ctx || !m) return fail(err, LBH_NULL_ARGUMENT);
    if (top_k == 0) return fail(err, LBH_DIMENSION_MISMATCH, 0, 3, 1, 0);
    if (n_tokens == 0) return fail(err, LBH_DIMENSION_MISMATCH, 0, 4, 1, 0);
    if (input_len != n_tokens * m->hidden) return fail(err, LBH_DIMENSION_MISMATCH, 0, 0, n_tokens * m->hidden, input_len);
    if (output_len != n_tokens * m->hidden)
        return fail(err, LBH_DIMENSION_MISMATCH, 0, 1, n_tokens * m->hidden, output_len);
    if (!ids || !coefs || !input || !output) return fail(err, LBH_NULL_ARGUMENT);
    if (!m->batch_mem || n_tokens > m->cap_tokens || top_k > m->cap_k)
        return fail(err, LBH_SCRATCH_TOO_SMALL, 0, 0, m->cap_tokens * m->cap_k, n_tokens * top_k);
    // Each token's routing under the rules of moe_routed_by_id_into (moe.rs:94-129).
    for (size_t t = 0; t < n_tokens; ++t) {
        const uint32_t *id = ids + t * top_k;
        const float *cf = coefs + t * top_k;
        for (size_t i = 0; i < top_k; ++i) {
            uint32_t bits;
            std::memcpy(&bits, &cf[i], 4);
            if ((bits & 0x7f800000u) == 0x7f800000u) return fail(err, LBH_NON_FINITE_VALUE, 0, 0, 0, 0, bits, 6, t);
            if (i > 0 && id[i] == id[i - 1]) return fail(err, LBH_DUPLICATE_ROUTED_EXPERT, 0, id[i], 0, 0, 0, 0, t);
            if (i > 0 && id[i] < id[i - 1])
                return fail(err, LBH_ROUTED_EXPERT_ORDER, 0, id[i], id[i - 1], id[i], 0, 0, t);
            if (id[i] >= m->n_experts) return fail(err, LBH_INVALID_PARAMETER, 0, id[i], m->n_experts, id[i], 0, 0, t);
        }
    }
    DeviceGuard g(ctx->device);
    HIP_TRY(launch_reset_status(ctx->status, ctx->stream));
    HIP_TRY(launch_find_nonfinite(input, (long long)input_len, &ctx->status->first_bad_input, ctx->stream));
    lbh_status st = read_status(ctx, err);
    if (st) return st;
    if (ctx->status_host->first_bad_input != ~0ull) {
        const unsigned long long i = ctx->status_host->first_bad_input;
        return fail(err, LBH_NON_FINITE_VALUE, m->type_gate_r, i % m->hidden, 0, 0, read_f32_bits(ctx, input + i), 0,
                    i / m->hidden);
    }
    HIP_TRY(hipMemcpyAsync(m->batch_ids, ids, n_tokens * top_k * 4, hipMemcpyHostToDevice, ctx->stream));
    HIP_TRY(hipMemcpyAsync(m->batch_coefs, coefs, n_tokens * top_k * 4, hipMemcpyHostToDevice, ctx->stream));
    BatchArgs a = batch_args(m, m->batch_ids, m->batch_coefs, n_tokens, top_k, input, output);
    a.gemm_shape = ctx->gemm_shape;
    const BatchStreams bs = batch_streams(m);
    HIP_TRY(launch_moe_batch(a, ctx->stream, &bs));
    HIP_TRY(hipMemcpyAsync(m->plan_host, a.plan, 8, hipMemcpyDeviceToHost, ctx->stream));
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    if (m->plan_host[1]) return fail(err, LBH_INVALID_PARAMETER, 0, (uint64_t)m->plan_host[1]);
    return ok(err);
}

lbh_status lbh_route_experts_batch(lbh_ctx *ctx, const float *logits, size_t n_tokens, size_t n_experts, size_t top_k,
                                   int32_t mode, float weight_scale, const float *bias, uint32_t *ids, float *coefs) {
    if (!ctx || !logits || !ids || !coefs || (mode == 1 && !bias)) return LBH_NULL_ARGUMENT;
    if (mode != 0 && mode != 1) return LBH_INVALID_PARAMETER;
    if (n_tokens == 0 || n_experts == 0 || n_experts > 256 || top_k == 0 || top_k > n_experts ||
        top_k > (size_t)MOE_MAX_ROUTED)
        return LBH_UNSUPPORTED_SHAPE;
    RouteBatchArgs a{};
    a.r.bias = bias;
    a.r.n_experts = (int32_t)n_experts;
    a.r.top_k = (int32_t)top_k;
    a.r.mode = mode;
    a.r.weight_scale = weight_scale;
    a.logits = logits;
    a.ids = ids;
    a.coefs = coefs;
    a.n_tokens = (int32_t)n_tokens;
    DeviceGuard g(ctx->device);
    return launch_route_batch(a, ctx->stream) == hipSuccess ? LBH_OK : LBH_HIP_ERROR;
}

}  // extern "C"

// ================================================================== router

struct lbh_router {
    int device;
    size_t n_experts, hidden;
    float *w;            // transposed, interleaved by four (RouterArgs::w)
    float *bias;         // [n_experts] or NULL
    float *logits;
    MoeRoute *route;     // device
    MoeRoute *route_host;
    // [0] first invalid selection input of route_into, [1] ring give-up of the
    // block decodes (sticky until lbh_router_take_status), [2..4] their
    // rejected selections (RouterArgs::reject), [5] ring give-up of route_into.
    unsigned long long *status;
    unsigned long long *status_host;
    long long spin_limit;              // RouterArgs::spin_limit (0: default)
};

namespace {

void free_router(lbh_router *r) {
    if (!r) return;
    DeviceGuard g(r->device);
    if (r->w) (void)hipFree(r->w);
    if (r->bias) (void)hipFree(r->bias);
    if (r->logits) (void)hipFree(r->logits);
    if (r->route) (void)hipFree(r->route);
    if (r->status) (void)hipFree(r->status);
    if (r->route_host) (void)hipHostFree(r->route_host);
    if (r->status_host) (void)hipHostFree(r->status_host);
    delete r;
}

constexpr int ROUTER_STATUS_WORDS = 6;

// NonFiniteValue of a rejected selection (routing.rs:72-77): `bad` as
// select_route codes it ((expert << 2) | field: 0 logit, 1 bias, 2 selection
// score), with that expert's logit and bias bits; the score is recomputed.
lbh_status selection_error(unsigned long long bad, uint32_t logit_bits, uint32_t bias_bits, lbh_error *err) {
    const uint64_t e = bad >> 2;
    const uint32_t field = (uint32_t)(bad & 3);
    float l, bv;
    std::memcpy(&l, &logit_bits, 4);
    std::memcpy(&bv, &bias_bits, 4);
    const float v = field == 0 ? l : field == 1 ? bv : 1.0f / (1.0f + expf_libm(-l)) + bv;
    uint32_t vb;
    std::memcpy(&vb, &v, 4);
    return fail(err, LBH_NON_FINITE_VALUE, LBH_F32, e, 0, 0, vb, 8 + field);
}

RouterArgs router_args(const lbh_router *r, const float *x, size_t top_k, int32_t mode, float scale) {
    RouterArgs a{};
    a.w = r->w;
    a.bias = r->bias;
    a.x = x;
    a.logits = r->logits;
    a.route = r->route;
    a.n_experts = (int32_t)r->n_experts;
    a.hidden = (int32_t)r->hidden;
    a.top_k = (int32_t)top_k;
    a.mode = mode;
    a.weight_scale = scale;
    a.spin_limit = r->spin_limit;
    a.timeout = r->status + 1;
    a.reject = r->status + 2;
    return a;
}

}  // namespace

extern "C" {

lbh_status lbh_router_create(lbh_ctx *ctx, const float *weights, size_t n_experts, size_t hidden, const float *bias,
                             int32_t on_device, lbh_router **out, lbh_error *err) {
    if (!ctx || !weights || !out) return fail(err, LBH_NULL_ARGUMENT);
    *out = nullptr;
    if (n_experts == 0 || n_experts > 256) return fail(err, LBH_UNSUPPORTED_SHAPE, LBH_F32, 0, 256, n_experts);
    if (hidden == 0 || hidden % 256) return fail(err, LBH_DIMENSION_MISMATCH, LBH_F32, 0, 256, hidden);
    DeviceGuard g(ctx->device);
    lbh_router *r = new (std::nothrow) lbh_router();
    if (!r) return fail(err, LBH_HIP_ERROR);
    r->device = ctx->device;
    r->n_experts = n_experts;
    r->hidden = hidden;
    const hipMemcpyKind kind = on_device ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice;
    // Device layout: transposed and interleaved by four, so the lane of expert
    // e reads w[e][4j..4j+3] at ((j * n_experts) + e) * 16 bytes.
    const size_t count = n_experts * hidden;
    float *src = new (std::nothrow) float[count];
    float *dst = new (std::nothrow) float[count];
    hipError_t e = (src && dst) ? hipSuccess : hipErrorOutOfMemory;
    if (e == hipSuccess)
        e = hipMemcpy(src, weights, count * sizeof(float), on_device ? hipMemcpyDeviceToHost : hipMemcpyHostToHost);
    if (e == hipSuccess) {
        for (size_t x = 0; x < n_experts; ++x)
            for (size_t i = 0; i < hidden; ++i) dst[((i / 4) * n_experts + x) * 4 + (i % 4)] = src[x * hidden + i];
        e = hipMalloc(&r->w, count * sizeof(float));
    }
    if (e == hipSuccess) e = hipMemcpy(r->w, dst, count * sizeof(float), hipMemcpyHostToDevice);
    delete[] src;
    delete[] dst;
    if (e == hipSuccess && bias) {
        e = hipMalloc(&r->bias, n_experts * sizeof(float));
        if (e == hipSuccess) e = hipMemcpy(r->bias, bias, n_experts * sizeof(float), kind);
    }
    if (e == hipSuccess) e = hipMalloc(&r->logits, n_experts * sizeof(float));
    if (e == hipSuccess) e = hipMalloc(&r->route, sizeof(MoeRoute));
    if (e == hipSuccess) e = hipMemset(r->route, 0, sizeof(MoeRoute));
    if (e == hipSuccess) e = hipMalloc(&r->status, ROUTER_STATUS_WORDS * sizeof(unsigned long long));
    if (e == hipSuccess) e = hipMemset(r->status, 0, ROUTER_STATUS_WORDS * sizeof(unsigned long long));
    if (e == hipSuccess) e = hipHostMalloc(&r->route_host, sizeof(MoeRoute), hipHostMallocDefault);
    if (e == hipSuccess)
        e = hipHostMalloc(&r->status_host, ROUTER_STATUS_WORDS * sizeof(unsigned long long), hipHostMallocDefault);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) {
        free_router(r);
        return hip_fail(err, e);
    }
    *out = r;
    return ok(err);
}

lbh_status lbh_router_set_spin_limit(lbh_router *r, int64_t limit) {
    if (!r) return LBH_NULL_ARGUMENT;
    r->spin_limit = limit;
    return LBH_OK;
}

lbh_status lbh_router_destroy(lbh_router *r) {
    if (!r) return LBH_NULL_ARGUMENT;
    free_router(r);
    return LBH_OK;
}

lbh_status lbh_router_route_into(lbh_ctx *ctx, lbh_router *r, const float *x, size_t x_len, size_t top_k, int32_t mode,
                                 float weight_scale, uint32_t *ids, float *coefs, float *logits_host, lbh_error *err) {
    if (!ctx || !r || !x || !ids || !coefs) return fail(err, LBH_NULL_ARGUMENT);
    if (x_len != r->hidden) return fail(err, LBH_DIMENSION_MISMATCH, LBH_F32, 0, r->hidden, x_len);
    if (mode != 0 && mode != 1) return fail(err, LBH_INVALID_PARAMETER, 0, (uint64_t)mode);
    if (mode == 1 && !r->bias) return fail(err, LBH_NULL_ARGUMENT);
    // route_experts_into (routing.rs:48-71): top-k range, then weight_scale.
    if (top_k == 0 || top_k > r->n_experts) return fail(err, LBH_INVALID_PARAMETER, 0, top_k, r->n_experts, top_k);
    if (top_k > MOE_MAX_ROUTED) return fail(err, LBH_UNSUPPORTED_SHAPE, 0, top_k, MOE_MAX_ROUTED, top_k);
    uint32_t sbits;
    std::memcpy(&sbits, &weight_scale, 4);
    if (mode == 1 && (sbits & 0x7f800000u) == 0x7f800000u) return fail(err, LBH_NON_FINITE_VALUE, 0, 0, 0, 0, sbits, 7);
    DeviceGuard g(ctx->device);
    RouterArgs a = router_args(r, x, top_k, mode, weight_scale);
    a.status = r->status;
    a.timeout = r->status + 5;   // the block decodes' give-up word stays for lbh_router_take_status
    a.reject = nullptr;
    // The router matvec is gemv_into on an F32 matrix: its input must be finite (gemv.rs:195-211).
    HIP_TRY(launch_reset_status(ctx->status, ctx->stream));
    HIP_TRY(launch_find_nonfinite(x, (long long)x_len, &ctx->status->first_bad_input, ctx->stream));
    HIP_TRY(hipMemsetAsync(r->status + 5, 0, sizeof(unsigned long long), ctx->stream));
    HIP_TRY(launch_router(a, ctx->stream));
    HIP_TRY(hipMemcpyAsync(r->status_host, r->status, ROUTER_STATUS_WORDS * sizeof(unsigned long long),
                           hipMemcpyDeviceToHost, ctx->stream));
    HIP_TRY(hipMemcpyAsync(r->route_host, r->route, sizeof(MoeRoute), hipMemcpyDeviceToHost, ctx->stream));
    lbh_status st = read_status(ctx, err);
    if (st) return st;
    if (ctx->status_host->first_bad_input != ~0ull) {
        const unsigned long long i = ctx->status_host->first_bad_input;
        return fail(err, LBH_NON_FINITE_VALUE, LBH_F32, i, 0, 0, read_f32_bits(ctx, x + i), 0);
    }
    // A router chain whose bounded ring wait gave up left NaN logits behind.
    if (r->status_host[5] != 0) return fail(err, LBH_DEVICE_TIMEOUT, LBH_F32);
    const unsigned long long bad = r->status_host[0];
    if (bad != ~0ull) {
        const uint64_t e = bad >> 2;
        return selection_error(bad, read_f32_bits(ctx, r->logits + e), r->bias ? read_f32_bits(ctx, r->bias + e) : 0u,
                               err);
    }
    for (size_t i = 0; i < top_k; ++i) {
        ids[i] = r->route_host->ids[i];
        coefs[i] = r->route_host->coefs[i];
    }
    if (logits_host) HIP_TRY(hipMemcpy(logits_host, r->logits, r->n_experts * sizeof(float), hipMemcpyDeviceToHost));
    return ok(err);
}

lbh_status lbh_router_take_status(lbh_ctx *ctx, lbh_router *r, uint64_t *rejected, lbh_error *err) {
    if (!ctx || !r) return fail(err, LBH_NULL_ARGUMENT);
    if (rejected) *rejected = 0;
    DeviceGuard g(ctx->device);
    HIP_TRY(hipMemcpyAsync(r->status_host, r->status, ROUTER_STATUS_WORDS * sizeof(unsigned long long),
                           hipMemcpyDeviceToHost, ctx->stream));
    HIP_TRY(hipMemsetAsync(r->status + 1, 0, 4 * sizeof(unsigned long long), ctx->stream));
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    const unsigned long long n = r->status_host[2];
    if (rejected) *rejected = n;
    if (r->status_host[1] != 0) return fail(err, LBH_DEVICE_TIMEOUT, LBH_F32);
    if (n != 0) {
        const unsigned long long v = r->status_host[4];
        return selection_error(r->status_host[3], (uint32_t)v, (uint32_t)(v >> 32), err);
    }
    return ok(err);
}

static lbh_status block_forward(lbh_ctx *ctx, lbh_moe *m, lbh_router *r, const float *x, size_t top_k, int32_t mode,
                                float weight_scale, float *y, int residual) {
    if (!ctx || !m || !r || !x || !y) return LBH_NULL_ARGUMENT;
    if (r->n_experts != m->n_experts || r->hidden != m->hidden) return LBH_DIMENSION_MISMATCH;
    if (top_k == 0 || top_k > r->n_experts || top_k > MOE_MAX_ROUTED) return LBH_INVALID_PARAMETER;
    if (mode != 0 && (mode != 1 || !r->bias)) return LBH_INVALID_PARAMETER;
    DeviceGuard g(ctx->device);
    MoeArgs a = moe_args(m, x, y);
    // Beside the router chains the shared stream keeps its byte share (wg_s);
    // the selecting routed launch, which takes tiles_r + tiles_s workgroups,
    // fills the same round as the routing-given launch (55.2 vs 55.7 us per
    // token at the configs[2] shapes).
    if (m->has_shared) {
        a.tiles_s = m->wg_s;
        a.tiles_r = m->wg_r + m->wg_s_given - m->wg_s;
    }
    a.residual = residual;
    a.router = router_args(r, x, top_k, mode, weight_scale);
    a.route_dev = r->route;
    a.route.n = (int32_t)top_k;
    a.n_launch = (int32_t)top_k;
    a.select_in_kernel = 1;
    if (m->has_shared && m->two_stream) {
        // The router chains, then the routed gate/up (selecting from the
        // logits) and down + combine on the caller's stream; the shared
        // expert's whole FFN beside them on the second stream.
        hipError_t e = forward_two_streams(m, a, ctx->stream, [](const MoeArgs &rt, hipStream_t s) {
            hipError_t e2 = launch_router_logits(rt.router, s);
            return e2 == hipSuccess ? launch_moe_gate_up(rt, s) : e2;
        });
        return e == hipSuccess ? LBH_OK : LBH_HIP_ERROR;
    }
    if (m->has_shared) {
        // Router chains beside the shared gate/up, then the routed gate/up
        // (selecting from the logits), then down + combine.
        a.skip_shared_gate_up = 1;
        if (launch_moe_router_shared(a, ctx->stream) != hipSuccess) return LBH_HIP_ERROR;
    } else if (launch_router_logits(a.router, ctx->stream) != hipSuccess) {
        return LBH_HIP_ERROR;
    }
    if (launch_moe_gate_up(a, ctx->stream) != hipSuccess) return LBH_HIP_ERROR;
    if (launch_moe_down(a, ctx->stream) != hipSuccess) return LBH_HIP_ERROR;
    return LBH_OK;
}

lbh_status lbh_moe_block_forward(lbh_ctx *ctx, lbh_moe *m, lbh_router *r, const float *x, size_t top_k, int32_t mode,
                                 float weight_scale, float *y) {
    return block_forward(ctx, m, r, x, top_k, mode, weight_scale, y, 0);
}

lbh_status lbh_moe_block_forward_residual(lbh_ctx *ctx, lbh_moe *m, lbh_router *r, const float *x, size_t top_k,
                                          int32_t mode, float weight_scale, float *hidden) {
    return block_forward(ctx, m, r, x, top_k, mode, weight_scale, hidden, 1);
}

}  // extern "C"
