// lbh_dot.hip — the checked per-row dot over caller-supplied GGML and Q8_K
// bytes, the Q8_K scale scan, and the DequantF32 matvec.
//
// k_dot_ggml: y[r] = vec_dot_q8_k(ty, row r, q8, K) (crates/bridge-quant-layout/
// src/q8_k.rs:80-89) for rows given as raw GGML bytes in device memory (no
// upload, no device layout).  The bytes are gathered with byte loads (the
// caller's pointers carry no alignment guarantee) into the same register
// slices the matvec kernels load from the chunk-major layout, so the integer
// stage and the f32 fold are the matvec's (lbh_rows.h: row_dot); only the
// load path differs, which makes this kernel an independent check of the
// device layout too.
//
// k_gemv_dequant: the DequantF32 execution mode (crates/bridge-kernels-reference/
// src/gemv.rs:12-16, compute_dequant_into :230-243, dot_dequant_row :305-328):
// y[r] = ((0 + w[r][0] * x[0]) + w[r][1] * x[1]) + ... over all K elements in
// order, w the exact f32 decode of the packed block (k_quants.rs:242-300,
// iq2_s.rs:9-39, iq3_s.rs:9-53).  The sum is one dependent chain of K adds per
// row, so the kernel splits the work as a pipeline: three producer waves
// decode one block of 24 rows and multiply it by x into LDS while the
// consumer wave (one lane per row) adds the previous block's 256 products in
// order.
#include <hip/hip_runtime.h>

#include "lbh_internal.h"
#include "lbh_rows.h"

namespace lbh {

// --------------------------------------------------------- byte gathering

__device__ __forceinline__ uint32_t gb32(const uint8_t *p) {
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

// Dword t of a 32-byte group in residue-major order: bytes t, t + 8, t + 16, t + 24.
__device__ __forceinline__ uint32_t grm32(const uint8_t *g, int t) {
    return (uint32_t)g[t] | ((uint32_t)g[t + 8] << 8) | ((uint32_t)g[t + 16] << 16) | ((uint32_t)g[t + 24] << 24);
}

// One GGML block at `blk` into the one-lane-per-unit slice of its type (IQ2_S
// through its device encoding, iq2s_encode).
__device__ __forceinline__ void load_slice_ggml(const uint8_t *blk, WSlice<T_IQ2_S, 1> &w) {
    uint8_t g[82], e[82];
#pragma unroll
    for (int i = 0; i < 82; ++i) g[i] = blk[i];
    iq2s_encode(g, e);
    w.d = (uint32_t)e[0] | ((uint32_t)e[1] << 8);
#pragma unroll
    for (int i = 0; i < 8; ++i) w.qs[i] = gb32(e + 2 + 4 * i), w.sg[i] = gb32(e + 34 + 4 * i);
    w.qh = gb32(e + 66), w.qh2 = gb32(e + 70), w.sc = gb32(e + 74), w.sc2 = gb32(e + 78);
}

__device__ __forceinline__ void load_slice_ggml(const uint8_t *blk, WSlice<T_IQ3_S, 1> &w) {
    w.d = (uint32_t)blk[0] | ((uint32_t)blk[1] << 8);
#pragma unroll
    for (int i = 0; i < 16; ++i) w.qs[i] = gb32(blk + 2 + 4 * i);
#pragma unroll
    for (int i = 0; i < 8; ++i) w.sg[i] = gb32(blk + 74 + 4 * i);
    w.qh = gb32(blk + 66), w.qh2 = gb32(blk + 70), w.sc = gb32(blk + 106);
}

template <int TY>
__device__ __forceinline__ void load_slice_ggml(const uint8_t *blk, WSliceKQ<TY, 1> &w) {
    constexpr int QS = TY == T_Q5_K ? 48 : 16;
    w.hdr = make_uint4(gb32(blk), gb32(blk + 4), gb32(blk + 8), gb32(blk + 12));
    if constexpr (TY == T_Q5_K) {
#pragma unroll
        for (int t = 0; t < 8; ++t) w.qh[t] = grm32(blk + 16, t);
    }
#pragma unroll
    for (int g = 0; g < 4; ++g)
#pragma unroll
        for (int t = 0; t < 8; ++t) w.q[g][t] = grm32(blk + QS + 32 * g, t);
}

// ------------------------------------------------------------- raw row dots

struct DotGgmlArgs {
    const uint8_t *w;          // rows x row_bytes GGML bytes
    const uint8_t *q8;         // nb Q8_K blocks
    float *y;                  // [rows]
    long long rows;
    int32_t nb;
    int32_t pad;
    const DevStatus *status;   // skip every write when a validation word is set
};

constexpr int DOT_THREADS = 256;

template <int TY>
__global__ void __launch_bounds__(DOT_THREADS) k_dot_ggml(DotGgmlArgs p) {
    constexpr int GB = GridLDS<TY>::BYTES > 0 ? GridLDS<TY>::BYTES : 16;
    constexpr int BB = layout_of(TY).block_bytes;
    __shared__ __align__(16) uint8_t s_grid[GB];
    __shared__ __align__(16) uint8_t s_q8[64 * 292];
    __shared__ FoldLDS<TY> s_fold[DOT_THREADS / 64];
    if (p.status && (p.status->first_bad_input != ~0ull || p.status->first_bad_scale != ~0ull)) return;

    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    const int nb = p.nb;
    fill_grid<TY>(s_grid);
    for (int i = threadIdx.x; i < nb * 292; i += DOT_THREADS) s_q8[i] = p.q8[i];
    __syncthreads();

    const LaneMap<1> L(lane, nb);
    ActOf<TY, 1> act;
    load_act(s_q8 + L.b * 292, 0, act);
    const long long items = (p.rows + L.rpw - 1) / L.rpw;
    for (long long it = (long long)blockIdx.x * (DOT_THREADS / 64) + wid; it < items;
         it += (long long)gridDim.x * (DOT_THREADS / 64)) {
        const long long r = it * L.rpw + L.slot;
        const bool on = L.lane_on && r < p.rows;
        WOf<TY, 1> w{};
        if (on) load_slice_ggml(p.w + (r * nb + L.b) * BB, w);
        const float v = row_dot<TY, 1>(w, act, on, L, s_grid, s_fold[wid], nullptr, 0);
        if (on && L.leader()) p.y[r] = v;
    }
}

// First block whose Q8_K d is not finite (validate_q8_scales, q8_k.rs:208-222).
__global__ void k_find_nonfinite_q8(const uint8_t *__restrict__ q8, long long nblocks, unsigned long long *first) {
    for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < nblocks;
         i += (long long)gridDim.x * blockDim.x)
        if ((gb32(q8 + i * 292) & 0x7f800000u) == 0x7f800000u) atomicMin(first, (unsigned long long)i);
}

// --------------------------------------------------------- DequantF32 matvec

constexpr int DQ_ROWS = 24;            // rows per workgroup: 8 producer threads per row
constexpr int DQ_STRIDE = 256 + 4;     // floats per product row in LDS

struct DequantArgs {
    MatView m;
    const float *x;
    float *y;
    float coef;
    int32_t accumulate;
    const DevStatus *status;   // skip every write when the input scan found a non-finite lane
};

// The 32 products w * x of group `sub` (32 consecutive elements) of unit u.
// Decode formulas and their f32 operation order: k_quants.rs:242-300 (K-quants,
// sub-block j = sub), iq2_s.rs:9-39 and iq3_s.rs:9-53 (group g = sub).
template <int TY>
__device__ __forceinline__ void dequant_group(const Planes &P, uint32_t u, int sub, const float *x, float *out) {
    if constexpr (TY == T_Q4_K || TY == T_Q5_K) {
        constexpr int QS0 = TY == T_Q5_K ? 3 : 1;
        const uint4 hdr = bld128(P, u * 16, 0);
        const int g = sub >> 1, hi = sub & 1;
        const uint4 q0 = bld128(P, u * 16, (QS0 + 2 * g) * P.U16), q1 = bld128(P, u * 16, (QS0 + 2 * g + 1) * P.U16);
        const uint32_t q[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
        uint32_t h[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        if constexpr (TY == T_Q5_K) {
            const uint4 h0 = bld128(P, u * 16, P.U16), h1 = bld128(P, u * 16, 2 * P.U16);
            h[0] = h0.x, h[1] = h0.y, h[2] = h0.z, h[3] = h0.w, h[4] = h1.x, h[5] = h1.y, h[6] = h1.z, h[7] = h1.w;
        }
        int32_t sc, mn;
        scale_min_of(hdr.y, hdr.z, hdr.w, sub, sc, mn);
        const float d1 = __fmul_rn(f16_to_f32(hdr.x & 0xffffu), (float)sc);
        const float m1 = __fmul_rn(f16_to_f32(hdr.x >> 16), (float)mn);
#pragma unroll
        for (int l = 0; l < 32; ++l) {
            // element l of the group's 32 bytes sits in residue-major dword l % 8, byte l / 8
            uint32_t qv = (byte_of(q[l % 8], l / 8) >> (4 * hi)) & 15u;
            if constexpr (TY == T_Q5_K) qv += ((byte_of(h[l % 8], l / 8) >> sub) & 1u) * 16u;
            const float w = __fsub_rn(__fmul_rn(d1, (float)qv), m1);
            out[l] = __fmul_rn(w, x[l]);
        }
    } else if constexpr (TY == T_IQ2_S) {
        const float d = f16_to_f32(bld16(P, u * 2, 5 * P.U16));
        // device encoding (lbh_layout.h): rotated qs bytes, the qh dword of
        // groups 4 (sub / 4) .. + 3, bit-sliced sign dword
        const uint32_t qs = bld32(P, u * 16 + 4 * (sub & 3), (sub >> 2) * P.U16);
        const uint32_t sg = bld32(P, u * 16 + 4 * (sub & 3), (2 + (sub >> 2)) * P.U16);
        const uint32_t qh = bld32(P, u * 16 + 4 * (sub >> 2), 4 * P.U16);
        const uint32_t sc = bld8(P, u * 16 + 8 + sub, 4 * P.U16);
        const float bs[2] = {__fmul_rn(__fmul_rn(d, __fadd_rn(0.5f, (float)(sc & 15u))), 0.25f),
                             __fmul_rn(__fmul_rn(d, __fadd_rn(0.5f, (float)(sc >> 4))), 0.25f)};
#pragma unroll
        for (int lg = 0; lg < 4; ++lg) {
            const uint32_t h = (byte_of(qh, lg) >> (2 * (sub & 3))) & 3u;
            const uint32_t idx = iq2s_unrot_q(byte_of(qs, lg)) | (h << 8);
            const uint64_t grid = c_iq2s_grid[idx];
#pragma unroll
            for (int l = 0; l < 8; ++l) {
                // weight 8 lg + l of the group: bit 2 lg + l / 4 of sign byte l % 4
                const float sign = (byte_of(sg, l & 3) >> (2 * lg + (l >> 2))) & 1u ? -1.0f : 1.0f;
                const float w = __fmul_rn(__fmul_rn(bs[lg >> 1], (float)((grid >> (8 * l)) & 0xffu)), sign);
                out[8 * lg + l] = __fmul_rn(w, x[8 * lg + l]);
            }
        }
    } else {  // IQ3_S
        const uint32_t tail_base = 6 * P.U16;
        const float d = f16_to_f32(bld16(P, u * 2, 6 * P.U16 + 12 * P.U));
        const uint2 qs = bld64(P, u * 16 + 8 * (sub & 1), (sub >> 1) * P.U16);
        const uint32_t sg = bld32(P, u * 16 + 4 * (sub & 3), (4 + (sub >> 2)) * P.U16);
        const uint32_t qh = bld8(P, u * 12 + sub, tail_base);
        const uint32_t ps = bld8(P, u * 12 + 8 + (sub >> 1), tail_base);
        const float sc = __fmul_rn(d, (float)(1u + 2u * ((ps >> (4 * (sub & 1))) & 15u)));
#pragma unroll
        for (int lg = 0; lg < 4; ++lg) {
            const uint32_t qq = lg < 2 ? qs.x : qs.y;
            const int sh = 16 * (lg & 1);
            const uint32_t i1 = ((qq >> sh) & 0xffu) | ((qh << (8 - 2 * lg)) & 0x100u);
            const uint32_t i2 = ((qq >> (sh + 8)) & 0xffu) | ((qh << (7 - 2 * lg)) & 0x100u);
            const uint32_t g1 = c_iq3s_grid[i1], g2 = c_iq3s_grid[i2];
            const uint32_t s = byte_of(sg, lg);
#pragma unroll
            for (int l = 0; l < 4; ++l) {
                const float s1 = (s >> l) & 1u ? -1.0f : 1.0f;
                const float s2 = (s >> (l + 4)) & 1u ? -1.0f : 1.0f;
                const float w1 = __fmul_rn(__fmul_rn(sc, (float)byte_of(g1, l)), s1);
                const float w2 = __fmul_rn(__fmul_rn(sc, (float)byte_of(g2, l)), s2);
                out[8 * lg + l] = __fmul_rn(w1, x[8 * lg + l]);
                out[8 * lg + 4 + l] = __fmul_rn(w2, x[8 * lg + 4 + l]);
            }
        }
    }
}

template <int TY>
__global__ void __launch_bounds__(256) k_gemv_dequant(DequantArgs p) {
    __shared__ __align__(16) float s_prod[2][DQ_ROWS * DQ_STRIDE];
    // A non-finite input or (accumulating) destination: the reference rejects
    // the call before it writes (gemv.rs:126-127, :195-211).
    if (p.status && (p.status->first_bad_input != ~0ull || p.status->first_bad_dest != ~0ull)) return;
    const int nb = p.m.nb;
    const int rows = p.m.rows;
    const int r0 = blockIdx.x * DQ_ROWS;
    const Planes P = make_planes(p.m.planes, p.m.units, p.m.bytes);
    const int tid = threadIdx.x;
    float sum = 0.0f;
    // Step s: producers fill block s, the consumer adds block s - 1.
    for (int s = 0; s <= nb; ++s) {
        if (tid >= 64) {
            if (s < nb) {
                const int t = tid - 64, slot = t >> 3, sub = t & 7;
                int r = r0 + slot;
                r = r < rows ? r : rows - 1;   // rows past the matrix decode a real row; never stored
                float xv[32], out[32];
                const float4 *xs = reinterpret_cast<const float4 *>(p.x + (long long)s * 256 + 32 * sub);
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const float4 f = xs[i];
                    xv[4 * i] = f.x, xv[4 * i + 1] = f.y, xv[4 * i + 2] = f.z, xv[4 * i + 3] = f.w;
                }
                dequant_group<TY>(P, (uint32_t)(r * nb + s), sub, xv, out);
                float4 *dst = reinterpret_cast<float4 *>(&s_prod[s & 1][slot * DQ_STRIDE + 32 * sub]);
#pragma unroll
                for (int i = 0; i < 8; ++i) dst[i] = make_float4(out[4 * i], out[4 * i + 1], out[4 * i + 2], out[4 * i + 3]);
            }
        } else if (s > 0 && tid < DQ_ROWS) {
            const float4 *src = reinterpret_cast<const float4 *>(&s_prod[(s - 1) & 1][tid * DQ_STRIDE]);
            for (int i = 0; i < 64; ++i) {
                const float4 v = src[i];
                sum = __fadd_rn(sum, v.x);
                sum = __fadd_rn(sum, v.y);
                sum = __fadd_rn(sum, v.z);
                sum = __fadd_rn(sum, v.w);
            }
        }
        __syncthreads();
    }
    const int r = r0 + tid;
    if (tid < DQ_ROWS && r < rows) {
        if (p.accumulate)
            p.y[r] = __fadd_rn(p.y[r], __fmul_rn(p.coef, sum));
        else
            p.y[r] = sum;
    }
}

// ---------------------------------------------------------------- launchers

hipError_t launch_dot_ggml(int ty, const uint8_t *w, long long rows, int nb, const uint8_t *q8, float *y,
                           const DevStatus *st, hipStream_t s) {
    if (rows <= 0) return hipSuccess;
    if (nb < 1 || nb > 64) return hipErrorInvalidValue;
    DotGgmlArgs a{w, q8, y, rows, nb, 0, st};
    const long long items = (rows + (64 / nb) - 1) / (64 / nb);
    long long grid = (items + 3) / 4;
    grid = grid > 4096 ? 4096 : grid;
    switch (ty) {
    case T_IQ2_S: hipLaunchKernelGGL(k_dot_ggml<T_IQ2_S>, dim3((int)grid), dim3(DOT_THREADS), 0, s, a); break;
    case T_IQ3_S: hipLaunchKernelGGL(k_dot_ggml<T_IQ3_S>, dim3((int)grid), dim3(DOT_THREADS), 0, s, a); break;
    case T_Q4_K: hipLaunchKernelGGL(k_dot_ggml<T_Q4_K>, dim3((int)grid), dim3(DOT_THREADS), 0, s, a); break;
    case T_Q5_K: hipLaunchKernelGGL(k_dot_ggml<T_Q5_K>, dim3((int)grid), dim3(DOT_THREADS), 0, s, a); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_find_nonfinite_q8(const uint8_t *q8, long long nblocks, unsigned long long *first, hipStream_t s) {
    if (nblocks <= 0) return hipSuccess;
    long long grid = (nblocks + 255) / 256;
    grid = grid > 1024 ? 1024 : grid;
    hipLaunchKernelGGL(k_find_nonfinite_q8, dim3((int)grid), dim3(256), 0, s, q8, nblocks, first);
    return hipGetLastError();
}

hipError_t launch_gemv_dequant(const MatView &m, const float *x, float *y, float coef, int accumulate,
                               const DevStatus *st, hipStream_t s) {
    if (m.rows < 1 || m.nb < 1) return hipErrorInvalidValue;
    DequantArgs a{m, x, y, coef, accumulate, st};
    const int grid = (m.rows + DQ_ROWS - 1) / DQ_ROWS;
    switch (m.type) {
    case T_IQ2_S: hipLaunchKernelGGL(k_gemv_dequant<T_IQ2_S>, dim3(grid), dim3(256), 0, s, a); break;
    case T_IQ3_S: hipLaunchKernelGGL(k_gemv_dequant<T_IQ3_S>, dim3(grid), dim3(256), 0, s, a); break;
    case T_Q4_K: hipLaunchKernelGGL(k_gemv_dequant<T_Q4_K>, dim3(grid), dim3(256), 0, s, a); break;
    case T_Q5_K: hipLaunchKernelGGL(k_gemv_dequant<T_Q5_K>, dim3(grid), dim3(256), 0, s, a); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace lbh
