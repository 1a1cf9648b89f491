// lbh_kernels.hip — gfx950 support kernels of the quantized-dot path: Q8_K
// quantization, input/scale validation, and the lossless repack between the
// GGML block layout and the chunk-major device layout (lbh_layout.h).
#include <hip/hip_runtime.h>

#include "lbh_dev.h"
#include "lbh_internal.h"

namespace lbh {

// --------------------------------------------------------------- Q8_K quant

// Four blocks per wave, 16 per workgroup: quantize_row_q8_k_into (q8_k.rs:35-73).
__global__ void __launch_bounds__(256) k_quantize_q8k(const float *__restrict__ x, uint8_t *__restrict__ out,
                                                      long long nblocks, const DevStatus *st) {
    if (st && (st->first_bad_input != ~0ull || st->first_bad_dest != ~0ull)) return;
    const long long first = ((long long)blockIdx.x * 4 + (threadIdx.x >> 6)) * 4;
    if (first >= nblocks) return;
    quantize_blocks_wave(x, out, first, nblocks);
}

__global__ void k_find_nonfinite(const float *__restrict__ x, long long n, unsigned long long *first) {
    for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long long)gridDim.x * blockDim.x) {
        if ((__float_as_uint(x[i]) & 0x7f800000u) == 0x7f800000u) atomicMin(first, (unsigned long long)i);
    }
}

// One thread per (row, group of four inputs).
__global__ void k_f32_layout(const float *__restrict__ src, float *__restrict__ dst, long long rows, long long k,
                             int to_device) {
    const long long k4 = k / 4, n = rows * k4;
    for (long long t = (long long)blockIdx.x * blockDim.x + threadIdx.x; t < n; t += (long long)gridDim.x * blockDim.x) {
        const long long j = t / rows, r = t - j * rows;   // consecutive threads: consecutive rows of one group
        const long long g = r * k + 4 * j, d = (j * rows + r) * 4;
        if (to_device)
            *reinterpret_cast<float4 *>(dst + d) = *reinterpret_cast<const float4 *>(src + g);
        else
            *reinterpret_cast<float4 *>(dst + g) = *reinterpret_cast<const float4 *>(src + d);
    }
}

__global__ void k_find_nonfinite_f32w(const float *__restrict__ w, long long rows, long long k,
                                      unsigned long long *first) {
    const long long n = rows * k;
    for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long long)gridDim.x * blockDim.x) {
        if ((__float_as_uint(w[i]) & 0x7f800000u) == 0x7f800000u) {
            const long long q = i / 4, c = i - 4 * q, j = q / rows, r = q - j * rows;
            atomicMin(first, (unsigned long long)(r * k + 4 * j + c));
        }
    }
}

__global__ void k_reset_status(DevStatus *st) {
    if (threadIdx.x == 0) {
        st->first_bad_input = ~0ull;
        st->first_bad_dest = ~0ull;
        st->first_bad_scale = ~0ull;
        st->pad = 0;
    }
}

// ------------------------------------------------------------ repack / scan

// Device-layout offset of byte p of unit u (lbh_layout.h).
__device__ __forceinline__ long long dev_offset(int ty, long long U, long long u, int p) {
    const TypeLayout L = layout_of(ty);
    const long long chunk_base = (long long)L.nchunk * U * 16;
    auto chunk = [&](int c, int byte) { return (long long)c * U * 16 + u * 16 + byte; };
    if (ty == T_IQ2_S) {
        if (p < 2) return chunk_base + u * 2 + p;
        const int q = p - 2;
        return chunk(q / 16, q % 16);
    }
    if (ty == T_IQ3_S) {
        if (p < 2) return chunk_base + 12 * U + u * 2 + p;
        if (p < 66) return chunk((p - 2) / 16, (p - 2) % 16);
        if (p < 74) return chunk_base + u * 12 + (p - 66);
        if (p < 106) return chunk(4 + (p - 74) / 16, (p - 74) % 16);
        return chunk_base + u * 12 + 8 + (p - 106);
    }
    if (p < 16) return chunk(0, p);
    if (ty == T_Q4_K) {
        const int q = p - 16, idx = (q / 32) * 32 + residue_pos(q % 32);
        return chunk(1 + idx / 16, idx % 16);
    }
    if (p < 48) {
        const int idx = residue_pos(p - 16);
        return chunk(1 + idx / 16, idx % 16);
    }
    const int q = p - 48, idx = (q / 32) * 32 + residue_pos(q % 32);
    return chunk(3 + idx / 16, idx % 16);
}

// The IQ2_S sign dword of one group in its device encoding (iq2s_encode):
// byte i, bit k = bit 4k + i of the GGML dword (bit b of sign byte j is the
// sign of weight 8j + b = 4k + i, k = 2j + b / 4).  Per output byte: every
// fourth bit from i, compressed.
__device__ __forceinline__ uint32_t iq2s_sign_dword(uint32_t o) {
    uint32_t r = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        uint32_t x = (o >> i) & 0x11111111u;    // bit 4k
        x = (x | (x >> 3)) & 0x03030303u;       // bits 2m, 2m + 1 -> byte m bits 0-1
        x = (x | (x >> 6)) & 0x000f000fu;
        x = (x | (x >> 12)) & 0xffu;
        r |= x << (8 * i);
    }
    return r;
}

// The IQ2_S qh dword of groups 4j .. 4j + 3 in its device encoding: byte l,
// bits 2k, 2k + 1 = bits 2l, 2l + 1 of GGML byte k (a 4 x 4 transpose of
// 2-bit fields).
__device__ __forceinline__ uint32_t iq2s_qh_dword(uint32_t o) {
    uint32_t r = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k)
#pragma unroll
        for (int l = 0; l < 4; ++l) r |= ((o >> (8 * k + 2 * l)) & 3u) << (8 * l + 2 * k);
    return r;
}

// One unit's GGML bytes `g` to the device layout (IQ2_S through its bit
// encoding, iq2s_encode), and back.
template <int TY>
__device__ __forceinline__ void unit_to_device(const uint8_t *g, uint8_t *dst, long long U, long long u) {
    constexpr int BB = layout_of(TY).block_bytes;
    if constexpr (TY == T_IQ2_S) {
        // d, then 20 dwords (qs 0-7, signs 8-15, qh 16-17, scales 18-19):
        // halfword loads from an even address (every block of a buffer that
        // starts even), else byte loads
        uint32_t v[20], d;
        if ((reinterpret_cast<uintptr_t>(g) & 1u) == 0) {
            const uint16_t *h = reinterpret_cast<const uint16_t *>(g);
            d = h[0];
#pragma unroll
            for (int i = 0; i < 20; ++i) v[i] = (uint32_t)h[1 + 2 * i] | ((uint32_t)h[2 + 2 * i] << 16);
        } else {
            d = (uint32_t)g[0] | ((uint32_t)g[1] << 8);
#pragma unroll
            for (int i = 0; i < 20; ++i)
                v[i] = (uint32_t)g[2 + 4 * i] | ((uint32_t)g[3 + 4 * i] << 8) | ((uint32_t)g[4 + 4 * i] << 16) |
                       ((uint32_t)g[5 + 4 * i] << 24);
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = ((v[i] & 0x1f1f1f1fu) << 3) | ((v[i] >> 5) & 0x07070707u);
#pragma unroll
        for (int i = 8; i < 16; ++i) v[i] = iq2s_sign_dword(v[i]);
        v[16] = iq2s_qh_dword(v[16]), v[17] = iq2s_qh_dword(v[17]);
        uint4 *c = reinterpret_cast<uint4 *>(dst + u * 16);
        const long long cs = U;   // chunk plane stride in uint4
#pragma unroll
        for (int k = 0; k < 5; ++k) c[k * cs] = make_uint4(v[4 * k], v[4 * k + 1], v[4 * k + 2], v[4 * k + 3]);
        reinterpret_cast<uint16_t *>(dst + 5 * U * 16)[u] = (uint16_t)d;
    } else {
        for (int p = 0; p < BB; ++p) dst[dev_offset(TY, U, u, p)] = g[p];
    }
}

template <int TY>
__device__ __forceinline__ void unit_to_ggml(const uint8_t *src, uint8_t *g, long long U, long long u) {
    constexpr int BB = layout_of(TY).block_bytes;
    if constexpr (TY == T_IQ2_S) {
        uint8_t e[BB], out[BB];
        for (int p = 0; p < BB; ++p) e[p] = src[dev_offset(TY, U, u, p)];
        iq2s_decode(e, out);
        for (int p = 0; p < BB; ++p) g[p] = out[p];
    } else {
        for (int p = 0; p < BB; ++p) g[p] = src[dev_offset(TY, U, u, p)];
    }
}

template <int TY>
__global__ void k_repack(const uint8_t *__restrict__ src, uint8_t *__restrict__ dst, long long U, int to_device) {
    constexpr int BB = layout_of(TY).block_bytes;
    for (long long u = (long long)blockIdx.x * blockDim.x + threadIdx.x; u < U; u += (long long)gridDim.x * blockDim.x) {
        if (to_device)
            unit_to_device<TY>(src + u * BB, dst, U, u);
        else
            unit_to_ggml<TY>(src, dst + u * BB, U, u);
    }
}

// Units [u0, u0 + n) of a matrix of U units, GGML bytes of those units
// contiguous at `src`, into their places in the device layout.
template <int TY>
__global__ void k_repack_range(const uint8_t *__restrict__ src, uint8_t *__restrict__ dst, long long U, long long u0,
                               long long n) {
    constexpr int BB = layout_of(TY).block_bytes;
    for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long long)gridDim.x * blockDim.x)
        unit_to_device<TY>(src + i * BB, dst, U, u0 + i);
}

// The same device-layout bytes with the units in 16-row tile order
// (unit_index MAT_TILE16): one thread per destination unit, every plane's
// piece of the unit copied whole.  rows % 16 == 0.
template <int TY>
__global__ void k_units_to_tiles(const uint8_t *__restrict__ src, uint8_t *__restrict__ dst, long long rows, int nb) {
    constexpr TypeLayout L = layout_of(TY);
    const long long U = rows * nb;
    for (long long ut = (long long)blockIdx.x * blockDim.x + threadIdx.x; ut < U; ut += (long long)gridDim.x * blockDim.x) {
        const long long tile = ut / (16LL * nb), rem = ut - tile * 16LL * nb;
        const long long b = rem >> 4, r = tile * 16 + (rem & 15);
        const long long u = r * nb + b;
#pragma unroll
        for (int c = 0; c < L.nchunk; ++c)
            reinterpret_cast<uint4 *>(dst + c * U * 16)[ut] = reinterpret_cast<const uint4 *>(src + c * U * 16)[u];
        const long long base = L.nchunk * U * 16;
#pragma unroll
        for (int t = 0; t < L.tail / 4; ++t)
            reinterpret_cast<uint32_t *>(dst + base)[ut * (L.tail / 4) + t] =
                reinterpret_cast<const uint32_t *>(src + base)[u * (L.tail / 4) + t];
        if constexpr (L.dplane)
            reinterpret_cast<uint16_t *>(dst + base + L.tail * U)[ut] =
                reinterpret_cast<const uint16_t *>(src + base + L.tail * U)[u];
    }
}

// First non-finite f16 d / dmin in unit order (validate_scales, k_quants.rs:178-208).
template <int TY>
__global__ void k_validate_scales(const uint8_t *__restrict__ ggml, long long U, unsigned long long *first) {
    constexpr int BB = layout_of(TY).block_bytes;
    constexpr bool KQ = TY == T_Q4_K || TY == T_Q5_K;
    for (long long u = (long long)blockIdx.x * blockDim.x + threadIdx.x; u < U; u += (long long)gridDim.x * blockDim.x) {
        const uint8_t *b = ggml + u * BB;
        const uint32_t d = b[0] | (b[1] << 8);
        if ((d & 0x7c00u) == 0x7c00u) atomicMin(first, (unsigned long long)(2 * u));
        if (KQ) {
            const uint32_t m = b[2] | (b[3] << 8);
            if ((m & 0x7c00u) == 0x7c00u) atomicMin(first, (unsigned long long)(2 * u + 1));
        }
    }
}

__global__ void k_f16_to_f32(const uint16_t *in, float *out, long long n) {
    for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long long)gridDim.x * blockDim.x)
        out[i] = f16_to_f32(in[i]);
}

// ------------------------------------------------------- floor measurement

// Reference points for the matvecs' roofline: an empty kernel (the launch
// floor) and plain reads of a byte range with 16-byte non-temporal loads (the
// memory floor of reading a matrix's planes), in one of several launch shapes
// so that a caller can take the fastest: U loads per lane in flight, either
// grid-strided over the whole range or over one contiguous slab per
// workgroup.  The loaded words are XOR-folded and one word per wave is stored
// so no load can be dropped.
__global__ void k_empty() {}

typedef unsigned v4u32 __attribute__((ext_vector_type(4)));

template <int U>
__global__ void __launch_bounds__(256) k_stream_read(const uint4 *__restrict__ src, long long n16, uint32_t *sink,
                                                     int slab) {
    const v4u32 *p = reinterpret_cast<const v4u32 *>(src);
    uint32_t acc = 0;
    long long i0, end, stride;
    if (slab) {
        const long long per = (n16 + gridDim.x - 1) / gridDim.x;
        i0 = (long long)blockIdx.x * per + threadIdx.x;
        end = min((long long)(blockIdx.x + 1) * per, n16);
        stride = blockDim.x;
    } else {
        i0 = (long long)blockIdx.x * blockDim.x + threadIdx.x;
        end = n16;
        stride = (long long)gridDim.x * blockDim.x;
    }
    for (long long i = i0; i < end; i += U * stride) {
        v4u32 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const long long j = i + u * stride;
            v[u] = j < end ? __builtin_nontemporal_load(p + j) : v4u32{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int u = 0; u < U; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    for (int off = 32; off >= 1; off >>= 1) acc ^= __shfl_xor(acc, off, 64);
    if ((threadIdx.x & 63) == 0) sink[(blockIdx.x * blockDim.x + threadIdx.x) >> 6] = acc;
}

hipError_t launch_empty(hipStream_t s) {
    hipLaunchKernelGGL(k_empty, dim3(1), dim3(64), 0, s);
    return hipGetLastError();
}

hipError_t launch_stream_read(const void *src, long long bytes, uint32_t *sink, int grid, int unroll, int slab,
                              hipStream_t s) {
    if (bytes < 16 || grid < 1 || grid > 65536) return hipErrorInvalidValue;
    const uint4 *p = static_cast<const uint4 *>(src);
    switch (unroll) {
    case 1: hipLaunchKernelGGL(k_stream_read<1>, dim3(grid), dim3(256), 0, s, p, bytes / 16, sink, slab); break;
    case 2: hipLaunchKernelGGL(k_stream_read<2>, dim3(grid), dim3(256), 0, s, p, bytes / 16, sink, slab); break;
    case 4: hipLaunchKernelGGL(k_stream_read<4>, dim3(grid), dim3(256), 0, s, p, bytes / 16, sink, slab); break;
    case 8: hipLaunchKernelGGL(k_stream_read<8>, dim3(grid), dim3(256), 0, s, p, bytes / 16, sink, slab); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// ---------------------------------------------------------------- launchers

static inline int cdiv(long long a, long long b) { return (int)((a + b - 1) / b); }

hipError_t launch_quantize_q8k(const float *x, uint8_t *out, long long nblocks, const DevStatus *st, hipStream_t s) {
    if (nblocks <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_quantize_q8k, dim3(cdiv(nblocks, 16)), dim3(256), 0, s, x, out, nblocks, st);
    return hipGetLastError();
}

hipError_t launch_find_nonfinite(const float *x, long long n, unsigned long long *first, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    int grid = cdiv(n, 256);
    grid = grid > 4096 ? 4096 : grid;
    hipLaunchKernelGGL(k_find_nonfinite, dim3(grid), dim3(256), 0, s, x, n, first);
    return hipGetLastError();
}

hipError_t launch_f32_layout(const float *src, float *dst, long long rows, long long k, int to_device, hipStream_t s) {
    if (rows <= 0 || k <= 0 || k % 4) return hipErrorInvalidValue;
    long long grid = (rows * (k / 4) + 255) / 256;
    grid = grid > 65536 ? 65536 : grid;
    hipLaunchKernelGGL(k_f32_layout, dim3((int)grid), dim3(256), 0, s, src, dst, rows, k, to_device);
    return hipGetLastError();
}

hipError_t launch_find_nonfinite_f32w(const float *w, long long rows, long long k, unsigned long long *first,
                                      hipStream_t s) {
    if (rows <= 0 || k <= 0) return hipSuccess;
    long long grid = (rows * k + 255) / 256;
    grid = grid > 4096 ? 4096 : grid;
    hipLaunchKernelGGL(k_find_nonfinite_f32w, dim3((int)grid), dim3(256), 0, s, w, rows, k, first);
    return hipGetLastError();
}

hipError_t launch_reset_status(DevStatus *st, hipStream_t s) {
    hipLaunchKernelGGL(k_reset_status, dim3(1), dim3(64), 0, s, st);
    return hipGetLastError();
}

hipError_t launch_repack(int ty, const uint8_t *src, uint8_t *dst, long long U, int to_device, hipStream_t s) {
    int grid = cdiv(U, 256);
    grid = grid > 8192 ? 8192 : grid;
    switch (ty) {
    case T_IQ2_S: hipLaunchKernelGGL(k_repack<T_IQ2_S>, dim3(grid), dim3(256), 0, s, src, dst, U, to_device); break;
    case T_IQ3_S: hipLaunchKernelGGL(k_repack<T_IQ3_S>, dim3(grid), dim3(256), 0, s, src, dst, U, to_device); break;
    case T_Q4_K: hipLaunchKernelGGL(k_repack<T_Q4_K>, dim3(grid), dim3(256), 0, s, src, dst, U, to_device); break;
    case T_Q5_K: hipLaunchKernelGGL(k_repack<T_Q5_K>, dim3(grid), dim3(256), 0, s, src, dst, U, to_device); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_repack_range(int ty, const uint8_t *src, uint8_t *dst, long long U, long long u0, long long n,
                               hipStream_t s) {
    if (n <= 0) return hipSuccess;
    int grid = cdiv(n, 256);
    grid = grid > 8192 ? 8192 : grid;
    switch (ty) {
    case T_IQ2_S: hipLaunchKernelGGL(k_repack_range<T_IQ2_S>, dim3(grid), dim3(256), 0, s, src, dst, U, u0, n); break;
    case T_IQ3_S: hipLaunchKernelGGL(k_repack_range<T_IQ3_S>, dim3(grid), dim3(256), 0, s, src, dst, U, u0, n); break;
    case T_Q4_K: hipLaunchKernelGGL(k_repack_range<T_Q4_K>, dim3(grid), dim3(256), 0, s, src, dst, U, u0, n); break;
    case T_Q5_K: hipLaunchKernelGGL(k_repack_range<T_Q5_K>, dim3(grid), dim3(256), 0, s, src, dst, U, u0, n); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_units_to_tiles(const MatView &m, uint8_t *dst, hipStream_t s) {
    if (m.rows % 16 != 0) return hipErrorInvalidValue;
    int grid = cdiv(m.units, 256);
    grid = grid > 8192 ? 8192 : grid;
    switch (m.type) {
    case T_IQ2_S:
        hipLaunchKernelGGL(k_units_to_tiles<T_IQ2_S>, dim3(grid), dim3(256), 0, s, m.planes, dst, (long long)m.rows, m.nb);
        break;
    case T_IQ3_S:
        hipLaunchKernelGGL(k_units_to_tiles<T_IQ3_S>, dim3(grid), dim3(256), 0, s, m.planes, dst, (long long)m.rows, m.nb);
        break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_validate_scales(int ty, const uint8_t *ggml, long long U, unsigned long long *first, hipStream_t s) {
    int grid = cdiv(U, 256);
    grid = grid > 8192 ? 8192 : grid;
    switch (ty) {
    case T_IQ2_S: hipLaunchKernelGGL(k_validate_scales<T_IQ2_S>, dim3(grid), dim3(256), 0, s, ggml, U, first); break;
    case T_IQ3_S: hipLaunchKernelGGL(k_validate_scales<T_IQ3_S>, dim3(grid), dim3(256), 0, s, ggml, U, first); break;
    case T_Q4_K: hipLaunchKernelGGL(k_validate_scales<T_Q4_K>, dim3(grid), dim3(256), 0, s, ggml, U, first); break;
    case T_Q5_K: hipLaunchKernelGGL(k_validate_scales<T_Q5_K>, dim3(grid), dim3(256), 0, s, ggml, U, first); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_f16_to_f32(const uint16_t *in, float *out, long long n, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    int grid = cdiv(n, 256);
    grid = grid > 4096 ? 4096 : grid;
    hipLaunchKernelGGL(k_f16_to_f32, dim3(grid), dim3(256), 0, s, in, out, n);
    return hipGetLastError();
}

}  // namespace lbh
