// lbh_dev.h — device building blocks shared by every kernel translation unit.
//
// Arithmetic contract (bit-identical to the reference CPU path,
// crates/bridge-quant-layout/src/q8_k.rs):
//   * integer block sums are exact int32 (v_dot4_i32_i8 on signed bytes);
//   * every f32 operation is a separately rounded IEEE op in the reference's
//     order (built with -ffp-contract=off; __fmul_rn/__fadd_rn where the order
//     matters), divides are correctly rounded, denormals are preserved.
//
// Work decomposition used by the matvec kernels: a "unit" is one
// (row, 256-element super-block) pair; LPU lanes ("parts") share a unit, each
// taking NG/LPU of its natural groups (8 groups of 32 for IQ2_S/IQ3_S, 4
// groups of 64 for Q4_K/Q5_K).  Lane l of a wave owns
//     part = l % LPU,  block b = (l / LPU) % NB,  row slot = l / (LPU * NB),
// so its K-range (block b, part p) is fixed for the whole kernel: the Q8_K
// activation bytes it needs live in registers while rows stream past.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "lbh_layout.h"

namespace lbh {

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

__device__ __forceinline__ uint32_t byte_of(uint32_t v, int i) { return (v >> (8 * i)) & 0xffu; }

// Byte-wise negation of grid magnitudes: every grid byte m is in 1..63, and
// 0x01010100 = sum over bytes i of 256 << 8i (mod 2^32), so byte i of the
// difference is 256 - m_i, i.e. -m_i, with no borrow between bytes.
__host__ __device__ constexpr uint32_t neg_bytes(uint32_t g) { return 0x01010100u - g; }

// v_perm selector applying four sign bits to a dword of magnitudes: byte i
// takes the negated magnitude (selector 4 + i, from the first source) when bit
// i of nib is set, else the magnitude (selector i, second source).
// nib * 0x810204 moves bit i to bit 8i+2 with no carries between terms.
__device__ __forceinline__ uint32_t sign_sel(uint32_t nib) {
    return ((nib * 0x810204u) & 0x04040404u) | 0x03020100u;
}

__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ uint32_t ld_u32(const uint8_t *p) { return *reinterpret_cast<const uint32_t *>(p); }
__device__ __forceinline__ uint32_t ld_u16(const uint8_t *p) { return *reinterpret_cast<const uint16_t *>(p); }
__device__ __forceinline__ uint2 ld_u64(const uint8_t *p) { return *reinterpret_cast<const uint2 *>(p); }
__device__ __forceinline__ uint4 ld_u128(const uint8_t *p) { return *reinterpret_cast<const uint4 *>(p); }

__device__ __forceinline__ uint4 ld_chunk(const uint8_t *planes, long long U, int c, long long u) {
    return *reinterpret_cast<const uint4 *>(planes + ((long long)c * U + u) * 16);
}

// Weight planes read through a raw buffer resource: SGPR base + 32-bit
// offsets, so a chunk load costs no VALU address arithmetic (the plane offset
// c * U * 16 is a scalar operand) and out-of-range offsets read zero.
// Matrices are limited to < 4 GiB of planes.  Word 3 = 0x00020000 is the
// raw-buffer configuration of the gfx9 family (gfx950 included).
struct Planes {
    __amdgpu_buffer_rsrc_t rsrc;
    uint32_t U16;   // units * 16: byte size of one chunk plane
    uint32_t U;     // units
};

__device__ __forceinline__ Planes make_planes(const uint8_t *base, long long units, long long bytes) {
    Planes p;
    p.rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(base), (short)0, (int)(uint32_t)bytes, 0x00020000);
    p.U16 = (uint32_t)(units * 16);
    p.U = (uint32_t)units;
    return p;
}

// Cache policy of the weight loads.  A matvec streams each weight byte once
// per launch: there the loads are nt (non-temporal, cache-policy bit 1 of the
// gfx950 buffer loads), which measured 12-16% faster on MI355X for every
// matvec shape (IQ2_S 1536x4096 5.48 -> 4.82 us, Q4_K 4096x4096 6.05 -> 5.17
// us, Q5_K 120832x4096 5.2 -> 5.6 TB/s).  A translation unit whose kernels
// read the same weights from several workgroups (the batched decode, where
// each chunk of an expert's tokens re-reads its rows) defines
// LBH_WEIGHT_CPOL 0 before including this header: there the nt policy
// measured 13% slower (450 -> 510 us per 64-token step).
#ifndef LBH_WEIGHT_CPOL
#define LBH_WEIGHT_CPOL 2
#endif
constexpr int WEIGHT_CPOL = LBH_WEIGHT_CPOL;
__device__ __forceinline__ uint4 bld128(const Planes &P, uint32_t voff, uint32_t soff) {
    return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(P.rsrc, voff, soff, WEIGHT_CPOL));
}
__device__ __forceinline__ uint2 bld64(const Planes &P, uint32_t voff, uint32_t soff) {
    return __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(P.rsrc, voff, soff, WEIGHT_CPOL));
}
__device__ __forceinline__ uint32_t bld32(const Planes &P, uint32_t voff, uint32_t soff) {
    return __builtin_amdgcn_raw_buffer_load_b32(P.rsrc, voff, soff, WEIGHT_CPOL);
}
__device__ __forceinline__ uint32_t bld16(const Planes &P, uint32_t voff, uint32_t soff) {
    return __builtin_amdgcn_raw_buffer_load_b16(P.rsrc, voff, soff, WEIGHT_CPOL);
}
__device__ __forceinline__ uint32_t bld8(const Planes &P, uint32_t voff, uint32_t soff) {
    return __builtin_amdgcn_raw_buffer_load_b8(P.rsrc, voff, soff, WEIGHT_CPOL);
}

// 24-bit signed multiply (full rate): every integer product in the dots has
// operands well inside +-2^23.
__device__ __forceinline__ int32_t mul24(int32_t a, int32_t b) { return __mul24(a, b); }

// ------------------------------------------------------------ Q8_K quantize

// nearest_int (q8_k.rs:224-228): magic-number rounding, ties to even.
__device__ __forceinline__ int32_t nearest_int(float v) {
    const float s = __fadd_rn(v, 12582912.0f);
    const int32_t b = __float_as_int(s);
    return (b & 0x007fffff) - 0x00400000;
}

// One wave quantizes up to four consecutive 256-element blocks, 16 lanes per
// block and 16 elements per lane: quantize_row_q8_k_into (q8_k.rs:35-73).
// Block first + (lane / 16) reads x + 256 * block and writes 292 bytes at
// out + 292 * block (global memory or LDS).  Every lane of the wave must call
// it; blocks at or beyond `nblocks` are skipped.
//
// The arg-max keeps the first index of the largest |x| (q8_k.rs:43-49): each
// lane scans its 16 elements in order with a strict compare, the row of 16
// lanes reduces the maximum, and the lowest lane holding it (a ballot) owns
// the first index, since lane order is element order.  bsums[g] covers
// exactly the 16 elements of lane g.
//
// Split in two so a kernel can issue these loads before its weight loads
// (vector loads complete in order for waiting purposes: inputs requested
// after a burst of weight loads would wait for the whole burst).
struct QuantIn {
    float v[16];
    long long blk;
    bool valid;
};

__device__ __forceinline__ QuantIn quantize_load(const float *__restrict__ x, long long first, long long nblocks) {
    QuantIn q;
    const int li = threadIdx.x & 15;
    q.blk = first + ((threadIdx.x & 63) >> 4);
    q.valid = q.blk < nblocks;
    if (q.valid) {
        const float4 *src = reinterpret_cast<const float4 *>(x + q.blk * 256 + 16 * li);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float4 f = src[i];
            q.v[4 * i] = f.x, q.v[4 * i + 1] = f.y, q.v[4 * i + 2] = f.z, q.v[4 * i + 3] = f.w;
        }
    } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) q.v[i] = 0.0f;
    }
    return q;
}

// Row (16-lane) reductions through DPP, every lane of the row receiving the
// result: quad butterflies, then the half-row and row mirrors.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_row(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, CTRL, 0xf, 0xf, false);
}
__device__ __forceinline__ uint32_t row16_max(uint32_t v) {
    uint32_t o = dpp_row<0xB1>(v);   // quad_perm [1, 0, 3, 2]
    v = o > v ? o : v;
    o = dpp_row<0x4E>(v);            // quad_perm [2, 3, 0, 1]
    v = o > v ? o : v;
    o = dpp_row<0x141>(v);           // row_half_mirror
    v = o > v ? o : v;
    o = dpp_row<0x140>(v);           // row_mirror
    return o > v ? o : v;
}
__device__ __forceinline__ uint32_t row16_or(uint32_t v) {
    v |= dpp_row<0xB1>(v);
    v |= dpp_row<0x4E>(v);
    v |= dpp_row<0x141>(v);
    return v | dpp_row<0x140>(v);
}

// out_r (optional): a residue-major copy of the block's quants for the
// K-quant dots, 256 bytes per block at out_r + RES_STRIDE * block (the 16
// bytes of padding keep the 16-byte reads of consecutive blocks by
// consecutive lanes in distinct LDS banks): dword t of
// 32-byte group j holds the quants 32j + t + 8k, k = 0..3 (the ActKQ layout).
// Lane li holds group li / 2's quants 16 (li & 1) .. + 15, i.e. bytes k = 2
// (li & 1) and 2 (li & 1) + 1 of each of the group's eight dwords.
// out_q (optional): the block's 256 quants alone, at out_q + RES_STRIDE *
// block, 16-byte aligned for the ActIQL reads.
constexpr int RES_STRIDE = 272;
__device__ __forceinline__ void quantize_store(const QuantIn &q, uint8_t *out, uint8_t *out_r = nullptr,
                                               uint8_t *out_q = nullptr) {
    const int lane = threadIdx.x & 63;
    const int li = lane & 15;
    const float *v = q.v;
    // The lane's largest |x| and the value at its first index: a pairwise
    // tree whose strict compare keeps the lower index on ties.
    uint32_t a[16];
    float mv[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) a[i] = __float_as_uint(fabsf(v[i])), mv[i] = v[i];
#pragma unroll
    for (int st = 1; st < 16; st *= 2) {
#pragma unroll
        for (int i = 0; i < 16; i += 2 * st) {
            if (a[i + st] > a[i]) a[i] = a[i + st], mv[i] = mv[i + st];
        }
    }
    const uint32_t amax_l = a[0];
    const uint32_t amax = row16_max(amax_l);
    // The lowest lane of the row holding the row maximum owns the first index
    // (lane order is element order); its value reaches the row by an OR of
    // the owner's bits with zeros.
    const unsigned long long hit = __ballot(amax_l == amax);
    const int row0 = lane & 48;
    const int owner = row0 + __builtin_ctzll((hit >> row0) & 0xffffull);
    const float maxv = __uint_as_float(row16_or(lane == owner ? __float_as_uint(mv[0]) : 0u));
    uint32_t packed[4] = {0, 0, 0, 0};
    int32_t qsum = 0;
    float d = 0.0f;
    if (amax != 0) {
        const float iscale = -127.0f / maxv;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            int32_t qv = nearest_int(__fmul_rn(iscale, v[i]));
            qv = qv < 127 ? qv : 127;
            packed[i >> 2] |= (uint32_t)(uint8_t)(int8_t)qv << (8 * (i & 3));
            qsum += (int8_t)qv;
        }
        d = 1.0f / iscale;
    }
    // bsums pair: this lane's sum and the next lane's (row_shl:1; only even
    // lanes of a row use it, so the source stays inside the row).
    const int32_t next = __builtin_amdgcn_update_dpp(0, qsum, 0x101, 0xf, 0xf, false);
    if (q.valid) {
        uint8_t *ob = out + q.blk * 292;
        uint32_t *qs = reinterpret_cast<uint32_t *>(ob + 4 + 16 * li);
#pragma unroll
        for (int i = 0; i < 4; ++i) qs[i] = packed[i];
        if ((li & 1) == 0)
            *reinterpret_cast<uint32_t *>(ob + 260 + 2 * li) =
                (uint32_t)(uint16_t)(int16_t)qsum | ((uint32_t)(uint16_t)(int16_t)next << 16);
        if (li == 0) *reinterpret_cast<uint32_t *>(ob) = __float_as_uint(d);
        if (out_q)
            *reinterpret_cast<uint4 *>(out_q + q.blk * RES_STRIDE + 16 * li) =
                make_uint4(packed[0], packed[1], packed[2], packed[3]);
        if (out_r) {
            // half-dword t = quants t and t + 8 of this lane's 16
            const uint32_t h01 = perm(packed[2], packed[0], 0x05010400u);   // t = 0, 1
            const uint32_t h23 = perm(packed[2], packed[0], 0x07030602u);   // t = 2, 3
            const uint32_t h45 = perm(packed[3], packed[1], 0x05010400u);   // t = 4, 5
            const uint32_t h67 = perm(packed[3], packed[1], 0x07030602u);   // t = 6, 7
            uint16_t *o = reinterpret_cast<uint16_t *>(out_r + q.blk * RES_STRIDE + 32 * (li >> 1) + 2 * (li & 1));
            o[0] = (uint16_t)h01, o[2] = (uint16_t)(h01 >> 16);
            o[4] = (uint16_t)h23, o[6] = (uint16_t)(h23 >> 16);
            o[8] = (uint16_t)h45, o[10] = (uint16_t)(h45 >> 16);
            o[12] = (uint16_t)h67, o[14] = (uint16_t)(h67 >> 16);
        }
    }
}

__device__ __forceinline__ void quantize_blocks_wave(const float *__restrict__ x, uint8_t *out, long long first,
                                                     long long nblocks, uint8_t *out_r = nullptr,
                                                     uint8_t *out_q = nullptr) {
    quantize_store(quantize_load(x, first, nblocks), out, out_r, out_q);
}

// ------------------------------------------------------------ type traits

template <int TY>
struct Traits;
template <>
struct Traits<T_IQ2_S> {
    static constexpr int NG = 8;      // natural groups per block
    static constexpr int NCH = 1;     // f32 chains of the fold
    static constexpr bool KQ = false;
};
template <>
struct Traits<T_IQ3_S> {
    static constexpr int NG = 8;
    static constexpr int NCH = 1;
    static constexpr bool KQ = false;
};
template <>
struct Traits<T_Q4_K> {
    static constexpr int NG = 4;
    static constexpr int NCH = 9;     // lane sums 0..7 + minimum sum
    static constexpr bool KQ = true;
};
template <>
struct Traits<T_Q5_K> {
    static constexpr int NG = 4;
    static constexpr int NCH = 9;
    static constexpr bool KQ = true;
};

// ---------------------------------------------------------- activations

// IQ activation slice: the 32*G quants of groups [G*p, G*p + G) as dwords.
template <int G>
struct ActIQ {
    uint32_t q[8 * G];
    float d8;
};

// K-quant activation slice for groups [G*p, G*p + G): sub-blocks j = 2g, 2g+1;
// t[j][r] holds the four bytes 32j + r + 8k (k = 0..3) so one dot4 per
// residue r reproduces the reference's lane split (q8_k.rs:301-312);
// bsp[j] = bsums[2j] + bsums[2j+1].
template <int G>
struct ActKQ {
    uint32_t t[2 * G][8];
    int32_t bsp[2 * G];
    float d8;
};

template <int TY, int LPU>
using ActOf = typename std::conditional<Traits<TY>::KQ, ActKQ<Traits<TY>::NG / LPU>,
                                        ActIQ<Traits<TY>::NG / LPU>>::type;

// IQ activation slice left in LDS: `q` addresses the lane's 256 quants in a
// 16-byte aligned copy (quantize_store's out_q), read one group of 32 at a
// time.  Holds 2 VGPRs where ActIQ<8> holds 65, for kernels whose occupancy
// the register file limits.
struct ActIQL {
    const uint8_t *q;
    float d8;
};

// The 32 quants (8 dwords) of group g of an activation slice.
template <int G>
__device__ __forceinline__ void act_group(const ActIQ<G> &a, int g, uint32_t (&q)[8]) {
#pragma unroll
    for (int i = 0; i < 8; ++i) q[i] = a.q[8 * g + i];
}
__device__ __forceinline__ void act_group(const ActIQL &a, int g, uint32_t (&q)[8]) {
    const uint4 *p = reinterpret_cast<const uint4 *>(a.q + 32 * g);
    const uint4 v0 = p[0], v1 = p[1];
    q[0] = v0.x, q[1] = v0.y, q[2] = v0.z, q[3] = v0.w;
    q[4] = v1.x, q[5] = v1.y, q[6] = v1.z, q[7] = v1.w;
}

// `blk` is a 292-byte Q8_K block (global or LDS); part p of LPU.
template <int G>
__device__ __forceinline__ void load_act(const uint8_t *blk, int p, ActIQ<G> &a) {
    a.d8 = __uint_as_float(ld_u32(blk));
    const uint8_t *q = blk + 4 + 32 * G * p;
#pragma unroll
    for (int i = 0; i < 8 * G; ++i) a.q[i] = ld_u32(q + 4 * i);
}

template <int G>
__device__ __forceinline__ void load_act(const uint8_t *blk, int p, ActKQ<G> &a) {
    a.d8 = __uint_as_float(ld_u32(blk));
    const uint8_t *q = blk + 4 + 64 * G * p;
#pragma unroll
    for (int j = 0; j < 2 * G; ++j) {
        uint32_t n[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) n[i] = ld_u32(q + 32 * j + 4 * i);
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            uint32_t v = 0;
#pragma unroll
            for (int k = 0; k < 4; ++k) v |= byte_of(n[2 * k + t / 4], t % 4) << (8 * k);
            a.t[j][t] = v;
        }
    }
    const uint8_t *bs = blk + 260 + 8 * G * p;
#pragma unroll
    for (int j = 0; j < 2 * G; ++j) {
        const uint32_t w = ld_u32(bs + 4 * j);
        a.bsp[j] = (int32_t)(int16_t)(w & 0xffff) + (int32_t)(int16_t)(w >> 16);
    }
}

// The same K-quant slice from a residue-major copy of the block's quants
// (quantize_store's out_r): `res` is the block's 256 bytes, `blk` its Q8_K
// block (scale and bsums).
template <int G>
__device__ __forceinline__ void load_act_res(const uint8_t *blk, const uint8_t *res, int p, ActKQ<G> &a) {
    a.d8 = __uint_as_float(ld_u32(blk));
    const uint4 *q = reinterpret_cast<const uint4 *>(res + 64 * G * p);
#pragma unroll
    for (int j = 0; j < 2 * G; ++j) {
        const uint4 v0 = q[2 * j], v1 = q[2 * j + 1];
        a.t[j][0] = v0.x, a.t[j][1] = v0.y, a.t[j][2] = v0.z, a.t[j][3] = v0.w;
        a.t[j][4] = v1.x, a.t[j][5] = v1.y, a.t[j][6] = v1.z, a.t[j][7] = v1.w;
    }
    const uint8_t *bs = blk + 260 + 8 * G * p;
#pragma unroll
    for (int j = 0; j < 2 * G; ++j) {
        const uint32_t w = ld_u32(bs + 4 * j);
        a.bsp[j] = (int32_t)(int16_t)(w & 0xffff) + (int32_t)(int16_t)(w >> 16);
    }
}

// ----------------------------------------------------------- grid tables
//
// LDS copies of the IQ codebooks, laid out so a signed grid dword is one v_perm:
//   IQ2S: uint2 x 1024 (8 KiB) of byte codes 0/1/2 for the magnitudes 8/25/43
//         (the only values in the codebook), entry q | h << 8 at byte address
//         iq2s_code_addr(q, h) (the address the encoded qs and qh bytes give,
//         lbh_layout.h); v_perm with selector code + 4*sign picks from the
//         constant dwords {8,25,43} / {-8,-25,-43}.
//   IQ3S: uint32 x 512 (2 KiB) magnitude words; the negation is one VALU
//         subtraction (neg_bytes), cheaper than the 4 more LDS bytes per
//         lookup a stored (magnitude, negation) pair costs.

// Each translation unit holds its own copy (no relocatable device code).
#include "lbh_iq_grids.inc"
static __constant__ uint64_t c_iq2s_grid[1024] = {LBH_IQ2S_GRID_VALUES};
static __constant__ uint32_t c_iq3s_grid[512] = {LBH_IQ3S_GRID_VALUES};

// IQ3S: 512 (magnitude, negation) pairs of 8 bytes at iq3_pair_offset, then
// the 256 sign-byte entries (iq3_sign_entry) at IQ3_SIGN_OFF.  The pair order
// makes a lookup's LDS address one v_perm of the qs bytes (iq3_group_addrs):
// stored magnitudes and negations cost 4 more LDS bytes per lookup than a
// magnitude table, but LDS bandwidth is not what bounds these decodes, VALU
// issue is.
// Table tag of the signed IQ3S table below (a layout tag, not a GGML type).
constexpr int T_IQ3S_SGN = 0x100 | T_IQ3_S;

template <int TY>
struct GridLDS {
    static constexpr int MAIN = TY == T_IQ2_S ? 1024 * 8 : TY == T_IQ3_S ? 512 * 8 : 0;
    static constexpr int BYTES = TY == T_IQ3S_SGN ? 8192 * 4 : TY == T_IQ3_S ? MAIN + 256 * 8 : MAIN;
};

// Byte address of IQ2S code entry q | h << 8 (q: 8 bits, h: 2 bits).
__host__ __device__ constexpr uint32_t iq2s_code_addr(uint32_t q, uint32_t h) {
    return 256u * ((q >> 5) | (h << 3)) + 8u * (q & 31u);
}

// One IQ2S group of four lookups in the device encoding (lbh_layout.h): its
// rotated qs dword q, the qh dword hw holding its high bits at bits 2k, 2k + 1
// of each byte, and its sign dword s.  addr(j) is lookup j's code address,
// sel(t) the v_perm sign bits of its weights 4t .. 4t + 3 (t = 2j, 2j + 1).
struct Iq2sGroup {
    uint32_t x, y, s;
    // k: the group's field in hw (a compile-time constant after unrolling)
    __device__ __forceinline__ static Iq2sGroup make(uint32_t q, uint32_t hw, int k, uint32_t s) {
        const uint32_t hs = (k < 2 ? hw << (3 - 2 * k) : hw >> (2 * k - 3)) & 0x18181818u;
        return Iq2sGroup{q & 0xf8f8f8f8u, (q & 0x07070707u) | hs, s};
    }
    __device__ __forceinline__ uint32_t addr(int j) const {
        return __builtin_amdgcn_perm(y, x, 0x0c0c0000u | ((4u + (uint32_t)j) << 8) | (uint32_t)j);
    }
    __device__ __forceinline__ uint32_t sel(int t) const { return (t >= 2 ? s >> (t - 2) : s << (2 - t)) & 0x04040404u; }
};
constexpr int IQ3_SIGN_OFF = 512 * 8;

// Signed IQ3S table (32 KiB): the signed grid dword of every 9-bit index
// q | h << 8 and four sign bits s4 (bit i negates byte i), at byte offset
// 256 * ((q & 3) | h << 2 | s4 << 3) + (q & 0xfc).  One LDS word per four
// weights replaces the (magnitude, negation) pair, the sign selectors and the
// v_perm that applies them.
__host__ __device__ constexpr uint32_t iq3_signed_offset(uint32_t q, uint32_t h, uint32_t s4) {
    return 256u * ((q & 3u) | (h << 2) | (s4 << 3)) + (q & 0xfcu);
}

// The eight signed-table offsets of one IQ3S group: qs bytes j = 0..7 (q0 =
// bytes 0-3, q1 = bytes 4-7), high bit j of the qh byte h, sign nibble j of
// the group's sign word s (q8_k.rs:397-420).  Per qs dword the offset is
// x_j + 256 y_j, one v_perm: x = q & 0xfc, y = (q & 3) | h << 2 | s4 << 3.
__device__ __forceinline__ void iq3_group_soffs(uint32_t q0, uint32_t q1, uint32_t h, uint32_t s, uint32_t (&a)[8]) {
    // bit j of a nibble to bit 0 of byte j (see iq3_group_addrs)
    const uint32_t b0 = __umul24(h & 15u, 0x204081u) & 0x01010101u;
    const uint32_t b1 = __umul24((h >> 4) & 15u, 0x204081u) & 0x01010101u;
    // sign nibbles j = 0..7 to bytes: lo holds nibbles 0, 2, 4, 6 and hi 1, 3, 5, 7
    const uint32_t lo = s & 0x0f0f0f0fu, hi = (s >> 4) & 0x0f0f0f0fu;
    const uint32_t n0 = perm(hi, lo, 0x05010400u), n1 = perm(hi, lo, 0x07030602u);
    const uint32_t y0 = (q0 & 0x03030303u) | (b0 << 2) | (n0 << 3), x0 = q0 & 0xfcfcfcfcu;
    const uint32_t y1 = (q1 & 0x03030303u) | (b1 << 2) | (n1 << 3), x1 = q1 & 0xfcfcfcfcu;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t sel = 0x0c0c0000u | ((4u + j) << 8) | (uint32_t)j;
        a[j] = perm(y0, x0, sel);
        a[4 + j] = perm(y1, x1, sel);
    }
}

// A lane's view of the signed IQ3S table.
struct Iq3SignedRef {
    const uint8_t *g;
    __device__ __forceinline__ explicit Iq3SignedRef(const void *p) : g(static_cast<const uint8_t *>(p)) {}
    __device__ __forceinline__ uint32_t word(uint32_t o) const { return *reinterpret_cast<const uint32_t *>(g + o); }
};

// Byte offset of the IQ3S pair of 9-bit index q | h << 8: (q & 15) * 256 +
// (q & 0xf0) + 8 h, a bijection onto the 8-byte slots of 4 KiB.
__host__ __device__ constexpr uint32_t iq3_pair_offset(uint32_t q, uint32_t h) {
    return (q & 15u) * 256u + (q & 0xf0u) + 8u * h;
}

// The eight pair offsets of one IQ3S group: qs bytes j = 0..7 (q0 = bytes
// 0-3, q1 = bytes 4-7) with high bit j of the group's qh byte h
// (q8_k.rs:397-420).  Per qs dword: y = low nibbles, x = high nibbles with the
// high bit at bit 3 of each byte, and offset j = x_j + 256 y_j, one v_perm.
__device__ __forceinline__ void iq3_group_addrs(uint32_t q0, uint32_t q1, uint32_t h, uint32_t (&a)[8]) {
    // bit j of a nibble to bit 0 of byte j: n * 0x204081 places bit j at
    // 8j + (7 (j' - j)) only for j' = j inside the mask, with no carries.
    const uint32_t b0 = __umul24(h & 15u, 0x204081u) & 0x01010101u;
    const uint32_t b1 = __umul24((h >> 4) & 15u, 0x204081u) & 0x01010101u;
    const uint32_t x0 = (q0 & 0xf0f0f0f0u) | (b0 << 3), y0 = q0 & 0x0f0f0f0fu;
    const uint32_t x1 = (q1 & 0xf0f0f0f0u) | (b1 << 3), y1 = q1 & 0x0f0f0f0fu;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        // byte 0 <- x byte j (selector j), byte 1 <- y byte j (4 + j), bytes 2-3 <- 0
        const uint32_t sel = 0x0c0c0000u | ((4u + j) << 8) | (uint32_t)j;
        a[j] = perm(y0, x0, sel);
        a[4 + j] = perm(y1, x1, sel);
    }
}

// A lane's view of a codebook in LDS.  VSEL computes the IQ3S sign selectors
// in VALU (three ops per nibble) instead of reading the sign table: one LDS
// read fewer per eight weights, for kernels whose LDS issue, not VALU, is
// short.
template <int TY, bool VSEL = false>
struct GridRef {
    const uint8_t *g;
    __device__ __forceinline__ explicit GridRef(const void *p) : g(static_cast<const uint8_t *>(p)) {}
    // IQ2S code entry at byte address a (iq2s_code_addr); IQ3S pair at byte
    // offset o (iq3_pair_offset); IQ3S selectors of sign byte sb
    // (iq3_sign_entry).
    __device__ __forceinline__ uint2 code_at(uint32_t a) const { return *reinterpret_cast<const uint2 *>(g + a); }
    __device__ __forceinline__ uint2 pair(uint32_t o) const { return *reinterpret_cast<const uint2 *>(g + o); }
    __device__ __forceinline__ uint2 sel(uint32_t sb) const {
        if constexpr (VSEL) {
            constexpr uint32_t o = TY == T_IQ3_S ? 0x03020100u : 0u;
            return make_uint2((__umul24(sb & 15u, 0x810204u) & 0x04040404u) | o,
                              (__umul24((sb >> 4) & 15u, 0x810204u) & 0x04040404u) | o);
        } else {
            return reinterpret_cast<const uint2 *>(g + GridLDS<TY>::MAIN)[sb];
        }
    }
};

// Sign-byte table appended to the IQ3S entries: entry s = the full v_perm
// selectors applying the low and the high nibble of s to a (magnitude,
// negation) pair, so each group of four signs costs one LDS read instead of
// the selector arithmetic.
__device__ __forceinline__ uint2 iq3_sign_entry(uint32_t s) { return make_uint2(sign_sel(s & 15u), sign_sel(s >> 4)); }

// The signed IQ3S grid dword of a (magnitude, negation) pair and its sign
// selector (q8_k.rs:397-420).
__device__ __forceinline__ uint32_t iq3_signed(uint2 pr, uint32_t sel) { return perm(pr.y, pr.x, sel); }

// The LDS images of both tables (GridLDS layout), built at compile time from
// the codebooks: a workgroup's fill is a plain copy with 16-byte loads.
struct GridImages {
    uint32_t iq2s[2 * 1024];
    uint32_t iq3s[2 * (512 + 256)];
    constexpr GridImages() : iq2s{}, iq3s{} {
        const uint64_t g2[1024] = {LBH_IQ2S_GRID_VALUES};
        for (int i = 0; i < 1024; ++i) {
            uint32_t c[2] = {0, 0};
            for (int e = 0; e < 8; ++e) {
                const uint32_t m = (uint32_t)(g2[i] >> (8 * e)) & 0xffu;
                c[e >> 2] |= (m == 8 ? 0u : m == 25 ? 1u : 2u) << (8 * (e & 3));
            }
            const uint32_t a = iq2s_code_addr((uint32_t)i & 255u, (uint32_t)i >> 8) / 4;
            iq2s[a] = c[0], iq2s[a + 1] = c[1];
        }
        const uint32_t g3[512] = {LBH_IQ3S_GRID_VALUES};
        for (uint32_t i = 0; i < 512; ++i) {
            const uint32_t o = iq3_pair_offset(i & 255u, i >> 8) / 4;
            iq3s[o] = g3[i], iq3s[o + 1] = neg_bytes(g3[i]);
        }
        // iq3_sign_entry: sign_sel of each nibble.
        for (uint32_t sb = 0; sb < 256; ++sb) {
            iq3s[1024 + 2 * sb] = (((sb & 15u) * 0x810204u) & 0x04040404u) | 0x03020100u;
            iq3s[1024 + 2 * sb + 1] = (((sb >> 4) * 0x810204u) & 0x04040404u) | 0x03020100u;
        }
    }
};
static __constant__ GridImages c_grid_images = GridImages();

// The signed IQ3S table image (iq3_signed_offset layout).
struct Iq3SignedImage {
    uint32_t w[8192];
    constexpr Iq3SignedImage() : w{} {
        const uint32_t g3[512] = {LBH_IQ3S_GRID_VALUES};
        for (uint32_t i = 0; i < 512; ++i)
            for (uint32_t s4 = 0; s4 < 16; ++s4) {
                uint32_t v = 0;
                for (int b = 0; b < 4; ++b) {
                    const uint32_t m = (g3[i] >> (8 * b)) & 0xffu;
                    v |= (((s4 >> b) & 1u) ? (256u - m) & 0xffu : m) << (8 * b);
                }
                w[iq3_signed_offset(i & 255u, i >> 8, s4) / 4] = v;
            }
    }
};
static __constant__ Iq3SignedImage c_iq3s_signed = Iq3SignedImage();

template <int TY>
__device__ __forceinline__ const uint4 *grid_image() {
    if constexpr (TY == T_IQ3S_SGN) return reinterpret_cast<const uint4 *>(c_iq3s_signed.w);
    return reinterpret_cast<const uint4 *>(TY == T_IQ2_S ? c_grid_images.iq2s : c_grid_images.iq3s);
}

// Fills the grid for TY into `lds` (cooperatively, the first NT threads of
// the block); the caller synchronises afterwards.  grid_load / grid_store
// split it so the table reads can be issued ahead of a kernel's weight loads
// (at NT = 256: three IQ2S or two IQ3S 16-byte pieces per thread).
template <int TY, int NT = 256>
struct GridIn {
    static constexpr int PIECES = GridLDS<TY>::BYTES / 16;
    static constexpr int N = PIECES == 0 ? 1 : (PIECES + NT - 1) / NT;
    uint4 e[N];
};

template <int TY, int NT = 256>
__device__ __forceinline__ GridIn<TY, NT> grid_load() {
    GridIn<TY, NT> g;
    if constexpr (GridIn<TY, NT>::PIECES > 0) {
        const uint4 *img = grid_image<TY>();
#pragma unroll
        for (int k = 0; k < GridIn<TY, NT>::N; ++k) {
            const int i = threadIdx.x + NT * k;
            g.e[k] = threadIdx.x < NT && i < GridIn<TY, NT>::PIECES ? img[i] : make_uint4(0u, 0u, 0u, 0u);
        }
    }
    return g;
}

template <int TY, int NT = 256>
__device__ __forceinline__ void grid_store(const GridIn<TY, NT> &g, void *lds) {
    if constexpr (GridIn<TY, NT>::PIECES > 0) {
        if (threadIdx.x >= NT) return;
        uint4 *out = reinterpret_cast<uint4 *>(lds);
#pragma unroll
        for (int k = 0; k < GridIn<TY, NT>::N; ++k) {
            const int i = threadIdx.x + NT * k;
            if (i < GridIn<TY, NT>::PIECES) out[i] = g.e[k];
        }
    }
}

template <int TY>
__device__ __forceinline__ void fill_grid(void *lds) {
    if constexpr (GridIn<TY>::PIECES > 0) {
        const uint4 *img = grid_image<TY>();
        uint4 *out = reinterpret_cast<uint4 *>(lds);
        for (int i = threadIdx.x; i < GridIn<TY>::PIECES; i += blockDim.x) out[i] = img[i];
    }
}

// The LDS codebook of TY as a static array of the kernel that inlines this:
// its address is fixed when the kernel is compiled, so every lookup folds it
// into the ds_read offset field (a table in dynamic LDS costs an address add
// per lookup).  Kernels that also use dynamic LDS get it after this array.
template <int TY>
__device__ __forceinline__ uint8_t *static_grid() {
    __shared__ __align__(16) uint8_t g[GridLDS<TY>::BYTES > 0 ? GridLDS<TY>::BYTES : 16];
    return g;
}

// ------------------------------------------------------------ weight slices
//
// The bytes one lane needs from its unit, loaded from the device layout
// (lbh_layout.h).  Load and compute are separate so a caller can keep the
// loads of the next unit in flight while computing the current one.

template <int TY, int LPU>
struct WSlice;

// IQ2_S: G = 8 / LPU groups; qs[4G], signs[4G], qh[G], scales[G] bytes.
template <int LPU>
struct WSlice<T_IQ2_S, LPU> {
    static constexpr int G = 8 / LPU;
    uint32_t qs[G], sg[G];
    uint32_t qh, sc;   // G bytes each (G <= 4), or the low 4 when G == 8 (see hq, hs)
    uint32_t qh2, sc2; // G == 8: groups 4..7
    uint32_t d;
};

// Per-lane constant part of a slice's load offsets (the lane's part p never
// changes), added to u * 16 each step.
template <int TY, int LPU>
__device__ __forceinline__ uint32_t part_offset(const Planes &P, int p) {
    if constexpr (TY == T_IQ2_S && LPU == 4) return (uint32_t)(p >> 1) * P.U16 + 8u * (uint32_t)(p & 1);
    else if constexpr (TY == T_IQ2_S && LPU == 2) return (uint32_t)p * P.U16;
    else if constexpr (TY == T_IQ3_S && LPU == 4) return (uint32_t)p * P.U16;
    else if constexpr (TY == T_IQ3_S && LPU == 2) return (uint32_t)(2 * p) * P.U16;
    else if constexpr ((TY == T_Q4_K || TY == T_Q5_K) && LPU < 4) return (uint32_t)(2 * (4 / LPU) * p) * P.U16;
    else if constexpr (TY == T_Q4_K || TY == T_Q5_K) return (uint32_t)(2 * p) * P.U16;
    else return 0u;
}

template <int LPU>
__device__ __forceinline__ void load_slice(const Planes &P, uint32_t u, uint32_t po, int p, WSlice<T_IQ2_S, LPU> &w) {
    constexpr int G = 8 / LPU;
    const uint32_t u16 = u * 16;
    w.d = bld16(P, u * 2, 5 * P.U16);
    if constexpr (G == 8) {
        const uint4 a = bld128(P, u16, 0), b = bld128(P, u16, P.U16);
        const uint4 c = bld128(P, u16, 2 * P.U16), d = bld128(P, u16, 3 * P.U16);
        const uint4 e = bld128(P, u16, 4 * P.U16);
        w.qs[0] = a.x, w.qs[1] = a.y, w.qs[2] = a.z, w.qs[3] = a.w;
        w.qs[4] = b.x, w.qs[5] = b.y, w.qs[6] = b.z, w.qs[7] = b.w;
        w.sg[0] = c.x, w.sg[1] = c.y, w.sg[2] = c.z, w.sg[3] = c.w;
        w.sg[4] = d.x, w.sg[5] = d.y, w.sg[6] = d.z, w.sg[7] = d.w;
        w.qh = e.x, w.qh2 = e.y, w.sc = e.z, w.sc2 = e.w;
    } else if constexpr (G == 4) {
        const uint4 a = bld128(P, u16 + po, 0), c = bld128(P, u16 + po, 2 * P.U16);
        w.qs[0] = a.x, w.qs[1] = a.y, w.qs[2] = a.z, w.qs[3] = a.w;
        w.sg[0] = c.x, w.sg[1] = c.y, w.sg[2] = c.z, w.sg[3] = c.w;
        const uint32_t e = u16 + 4u * (uint32_t)p;
        w.qh = bld32(P, e, 4 * P.U16);
        w.sc = bld32(P, e + 8, 4 * P.U16);
        w.qh2 = w.sc2 = 0;
    } else {  // G == 2
        const uint2 a = bld64(P, u16 + po, 0);
        const uint2 c = bld64(P, u16 + po, 2 * P.U16);
        w.qs[0] = a.x, w.qs[1] = a.y;
        w.sg[0] = c.x, w.sg[1] = c.y;
        const uint32_t e = u16 + 2u * (uint32_t)p;
        // the qh dword of groups 4 (p / 2) .. + 3, shifted so that this part's
        // groups 2p, 2p + 1 hold fields 0 and 1
        w.qh = bld32(P, u16 + 4u * (uint32_t)(p >> 1), 4 * P.U16) >> (4 * (p & 1));
        w.sc = bld16(P, e + 8, 4 * P.U16);
        w.qh2 = w.sc2 = 0;
    }
}

// IQ2_S magnitudes {8, 25, 43} and their negations as v_perm sources.
constexpr uint32_t IQ2S_POS = 0x002b1908u;
constexpr uint32_t IQ2S_NEG = 0x00d5e7f8u;

// IQ2_S integer block sum over the slice's groups (q8_k.rs:337-364), from the
// device encoding (lbh_layout.h): per group one v_perm per lookup for its
// code address and one shift-and-mask per four weights for their signs.  With
// GB > 0 the codebook reads of GB groups at a time are issued before any of
// them is used (one LDS round trip per GB groups instead of one per lookup,
// at the cost of the registers that hold them: a latency-bound matvec with one
// wave per SIMD gains, kernels that rely on occupancy keep GB = 0, the
// compiler's interleaved schedule).
template <int LPU>
__device__ __forceinline__ Iq2sGroup iq2s_group(const WSlice<T_IQ2_S, LPU> &w, int g) {
    constexpr int G = 8 / LPU;
    return Iq2sGroup::make(w.qs[g], G == 8 && g >= 4 ? w.qh2 : w.qh, g & 3, w.sg[g]);
}

template <int LPU, int GB = 0, class A, bool VS>
__device__ __forceinline__ int32_t slice_sum(const WSlice<T_IQ2_S, LPU> &w, const A &a, const GridRef<T_IQ2_S, VS> &grid) {
    constexpr int G = 8 / LPU;
    constexpr int GC = GB == 0 ? 1 : G < GB ? G : GB;
    int32_t bsum = 0;
#pragma unroll
    for (int g0 = 0; g0 < G; g0 += GC) {
        uint2 code[GC][4];
        if constexpr (GB > 0) {
#pragma unroll
            for (int k = 0; k < GC; ++k) {
                const Iq2sGroup q = iq2s_group(w, g0 + k);
#pragma unroll
                for (int lg = 0; lg < 4; ++lg) code[k][lg] = grid.code_at(q.addr(lg));
            }
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int k = 0; k < GC; ++k) {
            const int g = g0 + k;
            const Iq2sGroup q = iq2s_group(w, g);
            const uint32_t sc = byte_of(g < 4 ? w.sc : w.sc2, g & 3);
            uint32_t aq[8];
            act_group(a, g, aq);
            int32_t part[2] = {0, 0};
#pragma unroll
            for (int lg = 0; lg < 4; ++lg) {
                const uint2 c = GB > 0 ? code[k][lg] : grid.code_at(q.addr(lg));
                // byte i takes the negated source (selector 4 + code) when its sign is set
                const uint32_t sel_lo = q.sel(2 * lg) | c.x;
                const uint32_t sel_hi = q.sel(2 * lg + 1) | c.y;
                part[lg >> 1] = dot4(perm(IQ2S_NEG, IQ2S_POS, sel_lo), aq[2 * lg], part[lg >> 1]);
                part[lg >> 1] = dot4(perm(IQ2S_NEG, IQ2S_POS, sel_hi), aq[2 * lg + 1], part[lg >> 1]);
            }
            bsum += mul24((int32_t)(1 + 2 * (sc & 15u)), part[0]) + mul24((int32_t)(1 + 2 * (sc >> 4)), part[1]);
        }
    }
    return bsum;
}

// IQ3_S: G = 8 / LPU groups; qs[8G], signs[4G], qh[G], scale nibbles[G].
template <int LPU>
struct WSlice<T_IQ3_S, LPU> {
    static constexpr int G = 8 / LPU;
    uint32_t qs[2 * G], sg[G];
    uint32_t qh, qh2, sc;
    uint32_t d;
};

template <int LPU>
__device__ __forceinline__ void load_slice(const Planes &P, uint32_t u, uint32_t po, int p, WSlice<T_IQ3_S, LPU> &w) {
    constexpr int G = 8 / LPU;
    const uint32_t u16 = u * 16, tail = u * 12, tail_base = 6 * P.U16;
    w.d = bld16(P, u * 2, 6 * P.U16 + 12 * P.U);
    if constexpr (G == 8) {
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const uint4 v = bld128(P, u16, c * P.U16);
            w.qs[4 * c] = v.x, w.qs[4 * c + 1] = v.y, w.qs[4 * c + 2] = v.z, w.qs[4 * c + 3] = v.w;
        }
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            const uint4 v = bld128(P, u16, (4 + c) * P.U16);
            w.sg[4 * c] = v.x, w.sg[4 * c + 1] = v.y, w.sg[4 * c + 2] = v.z, w.sg[4 * c + 3] = v.w;
        }
        w.qh = bld32(P, tail, tail_base), w.qh2 = bld32(P, tail + 4, tail_base), w.sc = bld32(P, tail + 8, tail_base);
    } else if constexpr (G == 4) {
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            const uint4 v = bld128(P, u16 + po, c * P.U16);
            w.qs[4 * c] = v.x, w.qs[4 * c + 1] = v.y, w.qs[4 * c + 2] = v.z, w.qs[4 * c + 3] = v.w;
        }
        const uint4 sv = bld128(P, u16 + (uint32_t)p * P.U16, 4 * P.U16);
        w.sg[0] = sv.x, w.sg[1] = sv.y, w.sg[2] = sv.z, w.sg[3] = sv.w;
        w.qh = bld32(P, tail + 4u * (uint32_t)p, tail_base);
        w.sc = bld16(P, tail + 8u + 2u * (uint32_t)p, tail_base);
        w.qh2 = 0;
    } else {  // G == 2
        const uint4 v = bld128(P, u16 + po, 0);
        w.qs[0] = v.x, w.qs[1] = v.y, w.qs[2] = v.z, w.qs[3] = v.w;
        const uint2 sv = bld64(P, u16 + (uint32_t)(p >> 1) * P.U16 + 8u * (uint32_t)(p & 1), 4 * P.U16);
        w.sg[0] = sv.x, w.sg[1] = sv.y;
        w.qh = bld16(P, tail + 2u * (uint32_t)p, tail_base);
        w.sc = bld8(P, tail + 8u + (uint32_t)p, tail_base);
        w.qh2 = 0;
    }
}

// IQ3_S integer block sum over the slice's groups (q8_k.rs:380-428).  GB > 0
// issues the LDS reads of GB groups before any of them is used (as for
// IQ2_S).  Local group g is global group G*p + g; its scale nibble is nibble
// g of w.sc (G <= 4: the lane's scale bits; G == 8: all four scale bytes).
template <int LPU, int GB = 0, class A, bool VS>
__device__ __forceinline__ int32_t slice_sum(const WSlice<T_IQ3_S, LPU> &w, const A &a, const GridRef<T_IQ3_S, VS> &grid) {
    constexpr int G = 8 / LPU;
    constexpr int GC = GB == 0 ? 1 : G < GB ? G : GB;
    int32_t bsum = 0;
#pragma unroll
    for (int g0 = 0; g0 < G; g0 += GC) {
        uint2 pr[GC][8], sm[GC][4];
#pragma unroll
        for (int k = 0; k < GC; ++k) {
            const int g = g0 + k;
            uint32_t ad[8];
            iq3_group_addrs(w.qs[2 * g], w.qs[2 * g + 1], byte_of(g < 4 ? w.qh : w.qh2, g & 3), ad);
#pragma unroll
            for (int j = 0; j < 8; ++j) pr[k][j] = grid.pair(ad[j]);
#pragma unroll
            for (int lg = 0; lg < 4; ++lg) sm[k][lg] = grid.sel(byte_of(w.sg[g], lg));
        }
        if constexpr (GB > 0) __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int k = 0; k < GC; ++k) {
            const int g = g0 + k;
            const uint32_t ps = (w.sc >> (4 * g)) & 15u;
            uint32_t aq[8];
            act_group(a, g, aq);
            int32_t gs = 0;
#pragma unroll
            for (int lg = 0; lg < 4; ++lg) {
                gs = dot4(iq3_signed(pr[k][2 * lg], sm[k][lg].x), aq[2 * lg], gs);
                gs = dot4(iq3_signed(pr[k][2 * lg + 1], sm[k][lg].y), aq[2 * lg + 1], gs);
            }
            bsum += mul24(gs, (int32_t)(2 * ps + 1));
        }
    }
    return bsum;
}

// IQ3_S integer block sum read from the signed table (same sums as above).
template <int LPU, int GB = 0, class A>
__device__ __forceinline__ int32_t slice_sum(const WSlice<T_IQ3_S, LPU> &w, const A &a, const Iq3SignedRef &grid) {
    constexpr int G = 8 / LPU;
    int32_t bsum = 0;
#pragma unroll
    for (int g = 0; g < G; ++g) {
        uint32_t ad[8], sw[8];
        iq3_group_soffs(w.qs[2 * g], w.qs[2 * g + 1], byte_of(g < 4 ? w.qh : w.qh2, g & 3), w.sg[g], ad);
#pragma unroll
        for (int j = 0; j < 8; ++j) sw[j] = grid.word(ad[j]);
        const uint32_t ps = (w.sc >> (4 * g)) & 15u;
        uint32_t aq[8];
        act_group(a, g, aq);
        int32_t gs = 0;
#pragma unroll
        for (int j = 0; j < 8; ++j) gs = dot4(sw[j], aq[j], gs);
        bsum += mul24(gs, (int32_t)(2 * ps + 1));
    }
    return bsum;
}

// Q4_K / Q5_K: G = 4 / LPU groups of 64 (sub-blocks 2g, 2g+1).
template <int TY, int LPU>
struct WSliceKQ {
    static constexpr int G = 4 / LPU;
    uint4 hdr;                     // d|dmin, scales[12]
    uint32_t q[G][8];              // residue-major qs of each group
    uint32_t qh[TY == T_Q5_K ? 8 : 1];
};
template <int LPU>
struct WSlice<T_Q4_K, LPU> : WSliceKQ<T_Q4_K, LPU> {};
template <int LPU>
struct WSlice<T_Q5_K, LPU> : WSliceKQ<T_Q5_K, LPU> {};

template <int TY, int LPU>
__device__ __forceinline__ void load_slice(const Planes &P, uint32_t u, uint32_t po, int p, WSliceKQ<TY, LPU> &w) {
    constexpr int G = 4 / LPU;
    constexpr int QS0 = TY == T_Q5_K ? 3 : 1;
    const uint32_t u16 = u * 16;
    w.hdr = bld128(P, u16, 0);
    if constexpr (TY == T_Q5_K) {
        const uint4 v0 = bld128(P, u16, P.U16), v1 = bld128(P, u16, 2 * P.U16);
        w.qh[0] = v0.x, w.qh[1] = v0.y, w.qh[2] = v0.z, w.qh[3] = v0.w;
        w.qh[4] = v1.x, w.qh[5] = v1.y, w.qh[6] = v1.z, w.qh[7] = v1.w;
    }
    // chunks QS0 + 2 * (G * p + g) and the one after it; po = 2 * G * p * U16
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const uint4 v0 = bld128(P, u16 + po, (QS0 + 2 * g) * P.U16);
        const uint4 v1 = bld128(P, u16 + po, (QS0 + 2 * g + 1) * P.U16);
        w.q[g][0] = v0.x, w.q[g][1] = v0.y, w.q[g][2] = v0.z, w.q[g][3] = v0.w;
        w.q[g][4] = v1.x, w.q[g][5] = v1.y, w.q[g][6] = v1.z, w.q[g][7] = v1.w;
    }
}

// scale_min (k_quants.rs:231-240) of sub-block j from the 12 packed bytes
// (s0 = bytes 0-3, s1 = 4-7, s2 = 8-11).
__device__ __forceinline__ void scale_min_of(uint32_t s0, uint32_t s1, uint32_t s2, int j, int32_t &sc, int32_t &mn) {
    if (j < 4) {
        sc = byte_of(s0, j) & 63;
        mn = byte_of(s1, j) & 63;
    } else {
        sc = (byte_of(s2, j - 4) & 15) | ((byte_of(s0, j - 4) >> 6) << 4);
        mn = (byte_of(s2, j - 4) >> 4) | ((byte_of(s1, j - 4) >> 6) << 4);
    }
}

// Q4_K / Q5_K integer stage over the slice (q8_k.rs:288-312): lane sums by
// residue and the slice's share of minimum_sum.  Sub-block index j is global
// (2 * (G*p + g) + h); p is the lane's part.
template <int TY, int LPU>
__device__ __forceinline__ void slice_sums(const WSliceKQ<TY, LPU> &w, const ActKQ<4 / LPU> &a, int p,
                                           int32_t ls[8], int32_t &ms) {
    constexpr int G = 4 / LPU;
    ms = 0;
#pragma unroll
    for (int t = 0; t < 8; ++t) ls[t] = 0;
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const int gg = G * p + g;
        int32_t sc0, mn0, sc1, mn1;
        scale_min_of(w.hdr.y, w.hdr.z, w.hdr.w, 2 * gg, sc0, mn0);
        scale_min_of(w.hdr.y, w.hdr.z, w.hdr.w, 2 * gg + 1, sc1, mn1);
        ms += mul24(mn0, a.bsp[2 * g]) + mul24(mn1, a.bsp[2 * g + 1]);
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            uint32_t lo = w.q[g][t] & 0x0f0f0f0fu;
            uint32_t hi = (w.q[g][t] >> 4) & 0x0f0f0f0fu;
            if constexpr (TY == T_Q5_K) {
                lo |= ((w.qh[t] >> (2 * gg)) & 0x01010101u) << 4;
                hi |= ((w.qh[t] >> (2 * gg + 1)) & 0x01010101u) << 4;
            }
            ls[t] += mul24(sc0, dot4(lo, a.t[2 * g][t], 0));
            ls[t] += mul24(sc1, dot4(hi, a.t[2 * g + 1][t], 0));
        }
    }
}

// Sum an int32 over the LPU lanes of a unit (exact; the result is valid in every lane).
template <int LPU>
__device__ __forceinline__ int32_t unit_reduce(int32_t v) {
    if constexpr (LPU >= 2) v += __shfl_xor(v, 1, 64);
    if constexpr (LPU >= 4) v += __shfl_xor(v, 2, 64);
    if constexpr (LPU >= 8) v += __shfl_xor(v, 4, 64);
    return v;
}

}  // namespace lbh
