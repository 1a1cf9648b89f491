// lbh_kernels.hip — gfx950 kernels of the quantized-dot path.
//
// Arithmetic contract (bit-identical to the reference CPU path,
// crates/bridge-quant-layout/src/q8_k.rs):
//   * integer block sums are exact int32 (v_dot4_i32_i8 on signed bytes);
//   * every f32 operation is a separately rounded IEEE op in the reference's
//     order (built with -ffp-contract=off; __fmul_rn/__fadd_rn where the order
//     matters), divides are correctly rounded, denormals are preserved.
#include <hip/hip_runtime.h>

#include "lbh_internal.h"

namespace lbh {

#include "lbh_iq_grids.inc"

__constant__ uint64_t c_iq2s_grid[1024] = {LBH_IQ2S_GRID_VALUES};
__constant__ uint32_t c_iq3s_grid[512] = {LBH_IQ3S_GRID_VALUES};

// ------------------------------------------------------------------ helpers

__device__ __forceinline__ float f16_to_f32(uint32_t h16) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(h16)));
}

__device__ __forceinline__ int dot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4(static_cast<int>(a), static_cast<int>(b), c, false);
}

__device__ __forceinline__ uint32_t perm(uint32_t s0, uint32_t s1, uint32_t sel) {
    return __builtin_amdgcn_perm(s0, s1, sel);
}

// Byte-wise negation of grid magnitudes (all bytes in 1..63: no carries).
__device__ __forceinline__ uint32_t neg_bytes(uint32_t g) { return (g ^ 0xffffffffu) + 0x01010101u; }

// perm selector applying four sign bits: byte i takes the negated magnitude
// (selector 4 + i, from S0) when bit i is set, else the magnitude (selector i).
// nib * 0x810204 moves bit i to bit 8i+2 with no carries between terms.
__device__ __forceinline__ uint32_t sign_sel(uint32_t nib) {
    return ((nib * 0x810204u) & 0x04040404u) | 0x03020100u;
}

__device__ __forceinline__ uint32_t signed_mag(uint32_t g, uint32_t nib) {
    return perm(neg_bytes(g), g, sign_sel(nib));
}

__device__ __forceinline__ uint32_t byte_of(uint32_t v, int i) { return (v >> (8 * i)) & 0xffu; }

__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ uint32_t ld_u32(const uint8_t *p) { return *reinterpret_cast<const uint32_t *>(p); }

__device__ __forceinline__ bool status_set(const DevStatus *st) {
    return st && (st->first_bad_input != ~0ull || st->first_bad_dest != ~0ull);
}

// --------------------------------------------------------------- Q8_K quant

// nearest_int (q8_k.rs:224-228).
__device__ __forceinline__ int32_t nearest_int(float v) {
    const float s = __fadd_rn(v, 12582912.0f);
    const int32_t b = __float_as_int(s);
    return (b & 0x007fffff) - 0x00400000;
}

// One wave per 256-element block: quantize_row_q8_k_into (q8_k.rs:35-73).
__global__ void __launch_bounds__(256) k_quantize_q8k(const float *__restrict__ x, uint8_t *__restrict__ out,
                                                      long long nblocks, const DevStatus *st) {
    if (status_set(st)) return;
    const int lane = threadIdx.x & 63;
    const long long blk = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (blk >= nblocks) return;
    const float4 v = reinterpret_cast<const float4 *>(x + blk * 256)[lane];
    const float xs[4] = {v.x, v.y, v.z, v.w};
    // First-index arg-max of |x|: key = (bits(|x|) << 32) | (255 - index).
    unsigned long long key = 0;
    for (int i = 0; i < 4; ++i) {
        const unsigned long long k =
            ((unsigned long long)__float_as_uint(fabsf(xs[i])) << 32) | (unsigned)(255 - (lane * 4 + i));
        key = k > key ? k : key;
    }
    for (int off = 32; off >= 1; off >>= 1) {
        const unsigned long long o = __shfl_xor(key, off, 64);
        key = o > key ? o : key;
    }
    uint8_t *ob = out + blk * 292;
    const float amax = __uint_as_float((uint32_t)(key >> 32));
    uint32_t packed = 0;
    int32_t qsum = 0;
    float d = 0.0f;
    if (amax != 0.0f) {
        const int idx = 255 - (int)(key & 0xffu);
        const float mine = xs[idx & 3];
        const float maxv = __shfl(mine, idx >> 2, 64);
        const float iscale = -127.0f / maxv;
        for (int i = 0; i < 4; ++i) {
            int32_t q = nearest_int(__fmul_rn(iscale, xs[i]));
            q = q < 127 ? q : 127;
            const int8_t q8 = static_cast<int8_t>(q);
            packed |= (uint32_t)(uint8_t)q8 << (8 * i);
            qsum += q8;
        }
        d = 1.0f / iscale;
    }
    *reinterpret_cast<uint32_t *>(ob + 4 + lane * 4) = packed;
    qsum += __shfl_xor(qsum, 1, 64);
    qsum += __shfl_xor(qsum, 2, 64);
    if ((lane & 3) == 0) {
        const uint16_t s16 = static_cast<uint16_t>(static_cast<int16_t>(qsum));
        ob[260 + (lane >> 1)] = static_cast<uint8_t>(s16 & 0xff);
        ob[261 + (lane >> 1)] = static_cast<uint8_t>(s16 >> 8);
    }
    if (lane == 0) *reinterpret_cast<uint32_t *>(ob) = __float_as_uint(d);
}

__global__ void k_find_nonfinite(const float *__restrict__ x, long long n, unsigned long long *first) {
    for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long long)gridDim.x * blockDim.x) {
        if ((__float_as_uint(x[i]) & 0x7f800000u) == 0x7f800000u) atomicMin(first, (unsigned long long)i);
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

template <int TY>
__global__ void k_repack(const uint8_t *__restrict__ src, uint8_t *__restrict__ dst, long long U, int to_device) {
    constexpr int BB = layout_of(TY).block_bytes;
    for (long long u = (long long)blockIdx.x * blockDim.x + threadIdx.x; u < U; u += (long long)gridDim.x * blockDim.x) {
        for (int p = 0; p < BB; ++p) {
            const long long o = dev_offset(TY, U, u, p);
            if (to_device)
                dst[o] = src[u * BB + p];
            else
                dst[u * BB + p] = src[o];
        }
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

// ------------------------------------------------------------------- gemv

// Activation block held in registers by a lane for the whole kernel
// (the lane's K-range is fixed; rows stream past it).
struct ActIQ {
    uint32_t q[64];
    float d8;
};

struct ActKQ {
    uint32_t t[8][8];   // [sub-block][residue]: the 4 bytes 32j + t + 8k, k = 0..3
    int32_t bsp[8];     // bsums[2j] + bsums[2j+1]
    float d8;
};

__device__ __forceinline__ void load_act(const uint8_t *blk, ActIQ &a) {
    a.d8 = __uint_as_float(ld_u32(blk));
#pragma unroll
    for (int i = 0; i < 64; ++i) a.q[i] = ld_u32(blk + 4 + 4 * i);
}

__device__ __forceinline__ void load_act(const uint8_t *blk, ActKQ &a) {
    a.d8 = __uint_as_float(ld_u32(blk));
    uint32_t n[64];
#pragma unroll
    for (int i = 0; i < 64; ++i) n[i] = ld_u32(blk + 4 + 4 * i);
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            uint32_t v = 0;
#pragma unroll
            for (int k = 0; k < 4; ++k) v |= byte_of(n[8 * j + 2 * k + t / 4], t % 4) << (8 * k);
            a.t[j][t] = v;
        }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const uint32_t w = ld_u32(blk + 260 + 4 * j);
        a.bsp[j] = (int32_t)(int16_t)(w & 0xffff) + (int32_t)(int16_t)(w >> 16);
    }
}

__device__ __forceinline__ uint4 ld_chunk(const uint8_t *planes, long long U, int c, long long u) {
    return *reinterpret_cast<const uint4 *>(planes + ((long long)c * U + u) * 16);
}

// IQ2_S block integer sum (q8_k.rs:337-364).
__device__ __forceinline__ int32_t iq2s_unit(const uint8_t *planes, long long U, long long u, const ActIQ &a,
                                             const uint2 *grid, uint32_t &dbits) {
    const uint4 c0 = ld_chunk(planes, U, 0, u), c1 = ld_chunk(planes, U, 1, u);
    const uint4 c2 = ld_chunk(planes, U, 2, u), c3 = ld_chunk(planes, U, 3, u);
    const uint4 c4 = ld_chunk(planes, U, 4, u);
    dbits = *reinterpret_cast<const uint16_t *>(planes + 5 * U * 16 + u * 2);
    const uint32_t qs[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
    const uint32_t sg[8] = {c2.x, c2.y, c2.z, c2.w, c3.x, c3.y, c3.z, c3.w};
    int32_t bsum = 0;
#pragma unroll
    for (int g = 0; g < 8; ++g) {
        const uint32_t h = byte_of(g < 4 ? c4.x : c4.y, g & 3);
        const uint32_t sc = byte_of(g < 4 ? c4.z : c4.w, g & 3);
        int32_t part[2] = {0, 0};
#pragma unroll
        for (int lg = 0; lg < 4; ++lg) {
            const uint32_t idx = byte_of(qs[g], lg) | ((h << (8 - 2 * lg)) & 0x300u);
            const uint2 gv = grid[idx];
            const uint32_t s = byte_of(sg[g], lg);
            part[lg >> 1] = dot4(signed_mag(gv.x, s & 15u), a.q[8 * g + 2 * lg], part[lg >> 1]);
            part[lg >> 1] = dot4(signed_mag(gv.y, s >> 4), a.q[8 * g + 2 * lg + 1], part[lg >> 1]);
        }
        bsum += (int32_t)(1 + 2 * (sc & 15u)) * part[0] + (int32_t)(1 + 2 * (sc >> 4)) * part[1];
    }
    return bsum;
}

// IQ3_S block integer sum (q8_k.rs:380-428).
__device__ __forceinline__ int32_t iq3s_unit(const uint8_t *planes, long long U, long long u, const ActIQ &a,
                                             const uint32_t *grid, uint32_t &dbits) {
    uint32_t qs[16], sg[8];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const uint4 v = ld_chunk(planes, U, c, u);
        qs[4 * c] = v.x, qs[4 * c + 1] = v.y, qs[4 * c + 2] = v.z, qs[4 * c + 3] = v.w;
    }
#pragma unroll
    for (int c = 0; c < 2; ++c) {
        const uint4 v = ld_chunk(planes, U, 4 + c, u);
        sg[4 * c] = v.x, sg[4 * c + 1] = v.y, sg[4 * c + 2] = v.z, sg[4 * c + 3] = v.w;
    }
    const uint8_t *tail = planes + 6 * U * 16 + u * 12;
    const uint32_t qh0 = ld_u32(tail), qh1 = ld_u32(tail + 4), scl = ld_u32(tail + 8);
    dbits = *reinterpret_cast<const uint16_t *>(planes + 6 * U * 16 + 12 * U + u * 2);
    int32_t bsum = 0;
#pragma unroll
    for (int g = 0; g < 8; ++g) {
        const uint32_t h = byte_of(g < 4 ? qh0 : qh1, g & 3);
        const uint32_t ps = (byte_of(scl, g >> 1) >> (4 * (g & 1))) & 15u;
        int32_t gs = 0;
#pragma unroll
        for (int lg = 0; lg < 4; ++lg) {
            const uint32_t qq = qs[2 * g + (lg >> 1)];
            const int sh = 16 * (lg & 1);
            const uint32_t i1 = ((qq >> sh) & 0xffu) | ((h << (8 - 2 * lg)) & 0x100u);
            const uint32_t i2 = ((qq >> (sh + 8)) & 0xffu) | ((h << (7 - 2 * lg)) & 0x100u);
            const uint32_t s = byte_of(sg[g], lg);
            gs = dot4(signed_mag(grid[i1], s & 15u), a.q[8 * g + 2 * lg], gs);
            gs = dot4(signed_mag(grid[i2], s >> 4), a.q[8 * g + 2 * lg + 1], gs);
        }
        bsum += gs * (int32_t)(2 * ps + 1);
    }
    return bsum;
}

// scale_min (k_quants.rs:231-240) for all eight sub-blocks.
__device__ __forceinline__ void unpack_scale_min(uint32_t s0, uint32_t s1, uint32_t s2, int32_t sc[8], int32_t mn[8]) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        sc[j] = byte_of(s0, j) & 63;
        mn[j] = byte_of(s1, j) & 63;
        sc[j + 4] = (byte_of(s2, j) & 15) | ((byte_of(s0, j) >> 6) << 4);
        mn[j + 4] = (byte_of(s2, j) >> 4) | ((byte_of(s1, j) >> 6) << 4);
    }
}

// Q4_K / Q5_K integer stage (q8_k.rs:288-312): lane sums by residue + minimum_sum.
template <int TY>
__device__ __forceinline__ void kq_unit(const uint8_t *planes, long long U, long long u, const ActKQ &a,
                                        int32_t ls[8], int32_t &ms, uint32_t &dd) {
    const uint4 h = ld_chunk(planes, U, 0, u);
    dd = h.x;
    int32_t sc[8], mn[8];
    unpack_scale_min(h.y, h.z, h.w, sc, mn);
    ms = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) ms += mn[j] * a.bsp[j];
    uint32_t qh[8];
    constexpr int QS0 = TY == T_Q5_K ? 3 : 1;
    if (TY == T_Q5_K) {
        const uint4 v0 = ld_chunk(planes, U, 1, u), v1 = ld_chunk(planes, U, 2, u);
        qh[0] = v0.x, qh[1] = v0.y, qh[2] = v0.z, qh[3] = v0.w;
        qh[4] = v1.x, qh[5] = v1.y, qh[6] = v1.z, qh[7] = v1.w;
    }
#pragma unroll
    for (int t = 0; t < 8; ++t) ls[t] = 0;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        const uint4 v0 = ld_chunk(planes, U, QS0 + 2 * g, u), v1 = ld_chunk(planes, U, QS0 + 2 * g + 1, u);
        const uint32_t q[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            uint32_t lo = q[t] & 0x0f0f0f0fu;
            uint32_t hi = (q[t] >> 4) & 0x0f0f0f0fu;
            if (TY == T_Q5_K) {
                lo |= ((qh[t] >> (2 * g)) & 0x01010101u) << 4;
                hi |= ((qh[t] >> (2 * g + 1)) & 0x01010101u) << 4;
            }
            ls[t] += sc[2 * g] * dot4(lo, a.t[2 * g][t], 0);
            ls[t] += sc[2 * g + 1] * dot4(hi, a.t[2 * g + 1][t], 0);
        }
    }
}

__device__ __forceinline__ void store_y(const GemvArgs &p, int r, float v) {
    if (p.accumulate)
        p.y[r] = __fadd_rn(p.y[r], __fmul_rn(p.coef, v));
    else
        p.y[r] = v;
}

// One lane per (row, block) unit; a wave covers RPW = 64 / nb rows per step.
// Integer sums and per-block f32 terms are computed in parallel; the per-row
// f32 fold then runs in the reference's sequential block order out of LDS.
template <int TY>
__global__ void __launch_bounds__(256) k_gemv(GemvArgs p) {
    constexpr bool KQ = TY == T_Q4_K || TY == T_Q5_K;
    constexpr int CH = KQ ? 9 : 1;
    __shared__ uint2 s_grid2[TY == T_IQ2_S ? 1024 : 1];
    __shared__ uint32_t s_grid3[TY == T_IQ3_S ? 512 : 1];
    __shared__ float s_terms[4][CH][64];
    __shared__ float s_chain[4][KQ ? 64 : 1][9];

    if (TY == T_IQ2_S)
        for (int i = threadIdx.x; i < 1024; i += blockDim.x) {
            const uint64_t v = c_iq2s_grid[i];
            s_grid2[i] = make_uint2((uint32_t)v, (uint32_t)(v >> 32));
        }
    if (TY == T_IQ3_S)
        for (int i = threadIdx.x; i < 512; i += blockDim.x) s_grid3[i] = c_iq3s_grid[i];
    __syncthreads();
    if (status_set(p.status)) return;

    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    const int NB = p.m.nb, RPW = 64 / NB;
    const int slot = lane / NB, b = lane - slot * NB;
    const bool lane_on = slot < RPW;
    const long long U = p.m.units;

    typename std::conditional<KQ, ActKQ, ActIQ>::type act;
    load_act(p.q8 + (long long)b * 292, act);

    const int nwaves = gridDim.x * 4;
    for (int row0 = (blockIdx.x * 4 + wid) * RPW; row0 < p.m.rows; row0 += nwaves * RPW) {
        const int r = row0 + slot;
        const bool on = lane_on && r < p.m.rows;
        if (on) {
            const long long u = (long long)r * NB + b;
            if constexpr (KQ) {
                int32_t ls[8], ms;
                uint32_t dd;
                kq_unit<TY>(p.m.planes, U, u, act, ls, ms, dd);
                const float scale = __fmul_rn(f16_to_f32(dd & 0xffffu), act.d8);
                const float mscale = __fmul_rn(f16_to_f32(dd >> 16), act.d8);
#pragma unroll
                for (int t = 0; t < 8; ++t) s_terms[wid][t][lane] = __fmul_rn(scale, (float)ls[t]);
                s_terms[wid][8][lane] = __fmul_rn(mscale, (float)ms);
                if (p.block_sums) {
#pragma unroll
                    for (int t = 0; t < 8; ++t) p.block_sums[u * 9 + t] = ls[t];
                    p.block_sums[u * 9 + 8] = ms;
                }
            } else {
                uint32_t dbits;
                const int32_t bsum = TY == T_IQ2_S ? iq2s_unit(p.m.planes, U, u, act, s_grid2, dbits)
                                                   : iq3s_unit(p.m.planes, U, u, act, s_grid3, dbits);
                const float scale = __fmul_rn(f16_to_f32(dbits), act.d8);
                s_terms[wid][0][lane] = __fmul_rn(scale, (float)bsum);
                if (p.block_sums) p.block_sums[u] = bsum;
            }
        }
        wave_sync();
        if constexpr (KQ) {
            // Chains 0..7: sums[l] += term (q8_k.rs:316-318); chain 8: sum -= term (:319-320).
            for (int c = b; c < 9; c += NB) {
                if (on) {
                    float s = 0.0f;
                    for (int i = 0; i < NB; ++i) {
                        const float t = s_terms[wid][c][slot * NB + i];
                        s = c == 8 ? __fsub_rn(s, t) : __fadd_rn(s, t);
                    }
                    s_chain[wid][slot][c] = s;
                }
            }
            wave_sync();
            if (on && b == 0) {
                float s = s_chain[wid][slot][8];
#pragma unroll
                for (int l = 0; l < 8; ++l) s = __fadd_rn(s, s_chain[wid][slot][l]);  // q8_k.rs:323-325
                store_y(p, r, s);
            }
        } else {
            if (on && b == 0) {
                float s = 0.0f;
                for (int i = 0; i < NB; ++i) s = __fadd_rn(s, s_terms[wid][0][slot * NB + i]);
                if (TY == T_IQ2_S) s = __fmul_rn(0.125f, s);  // q8_k.rs:369
                store_y(p, r, s);
            }
        }
        wave_sync();
    }
}

// ---------------------------------------------------------------- launchers

static inline int cdiv(long long a, long long b) { return (int)((a + b - 1) / b); }

hipError_t launch_quantize_q8k(const float *x, uint8_t *out, long long nblocks, const DevStatus *st, hipStream_t s) {
    if (nblocks <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_quantize_q8k, dim3(cdiv(nblocks, 4)), dim3(256), 0, s, x, out, nblocks, st);
    return hipGetLastError();
}

hipError_t launch_find_nonfinite(const float *x, long long n, unsigned long long *first, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    int grid = cdiv(n, 256);
    grid = grid > 4096 ? 4096 : grid;
    hipLaunchKernelGGL(k_find_nonfinite, dim3(grid), dim3(256), 0, s, x, n, first);
    return hipGetLastError();
}

hipError_t launch_reset_status(DevStatus *st, hipStream_t s) {
    hipLaunchKernelGGL(k_reset_status, dim3(1), dim3(64), 0, s, st);
    return hipGetLastError();
}

hipError_t launch_gemv(const GemvArgs &a, hipStream_t s) {
    const int nb = a.m.nb;
    if (nb < 1 || nb > 64) return hipErrorInvalidValue;
    const int rpw = 64 / nb;
    const int waves = cdiv(a.m.rows, rpw);
    const int grid = cdiv(waves, 4);
    switch (a.m.type) {
    case T_IQ2_S: hipLaunchKernelGGL(k_gemv<T_IQ2_S>, dim3(grid), dim3(256), 0, s, a); break;
    case T_IQ3_S: hipLaunchKernelGGL(k_gemv<T_IQ3_S>, dim3(grid), dim3(256), 0, s, a); break;
    case T_Q4_K: hipLaunchKernelGGL(k_gemv<T_Q4_K>, dim3(grid), dim3(256), 0, s, a); break;
    case T_Q5_K: hipLaunchKernelGGL(k_gemv<T_Q5_K>, dim3(grid), dim3(256), 0, s, a); break;
    default: return hipErrorInvalidValue;
    }
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
