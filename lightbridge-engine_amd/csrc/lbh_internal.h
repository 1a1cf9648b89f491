// lbh_internal.h — declarations shared by the kernel and C-ABI translation units.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "lbh_layout.h"

namespace lbh {

// Per-context device status words written by validation kernels and read by
// compute kernels, which skip all writes when a word is set (atomicity).
struct DevStatus {
    unsigned long long first_bad_input;   // first non-finite input lane, ~0ull when none
    unsigned long long first_bad_dest;    // first non-finite destination lane
    unsigned long long first_bad_scale;   // weight upload: 2 * unit + field
    unsigned long long pad;
};

// A matrix in the device layout (lbh_layout.h).
struct MatView {
    const uint8_t *planes;
    int32_t type;
    int32_t nb;        // 256-element blocks per row
    int32_t rows;
    int32_t pad;
    long long units;   // rows * nb
};

struct GemvArgs {
    MatView m;
    const uint8_t *q8;            // (nb) Q8_K blocks
    float *y;
    float coef;
    int32_t accumulate;
    int32_t *block_sums;          // optional integer-stage export
    const DevStatus *status;      // optional: skip when any validation word is set
};

hipError_t launch_quantize_q8k(const float *x, uint8_t *out, long long nblocks, const DevStatus *st,
                               hipStream_t s);
hipError_t launch_find_nonfinite(const float *x, long long n, unsigned long long *first, hipStream_t s);
hipError_t launch_reset_status(DevStatus *st, hipStream_t s);
hipError_t launch_gemv(const GemvArgs &a, hipStream_t s);
hipError_t launch_repack(int ty, const uint8_t *ggml, uint8_t *planes, long long units, int to_device,
                         hipStream_t s);
hipError_t launch_validate_scales(int ty, const uint8_t *ggml, long long units,
                                  unsigned long long *first, hipStream_t s);
hipError_t launch_f16_to_f32(const uint16_t *in, float *out, long long n, hipStream_t s);

}  // namespace lbh
