// lbh_gemm.hip — Q4_K / Q5_K x Q8_K for a batch of tokens on the f16 matrix
// cores (v_mfma_f32_32x32x16_f16), bit-identical to the reference's per-row
// dot (dot_q4_or_q5_k, crates/bridge-quant-layout/src/q8_k.rs:247-327) for
// every (row, token):
//
//   lane_sums[l] = sum_j sc_j * sum_{k<4} q[32j + 8k + l] * a[32j + 8k + l]
//   minimum_sum  = sum_j mn_j * (bsums[2j] + bsums[2j + 1])
//   per block:  sums[l] += (d * d8) * lane_sums[l];  sum -= (dmin * d8) * minimum_sum
//   result = sum + sums[0] + ... + sums[7]
//
// The integer stage runs on the matrix cores, the f32 chains on the VALU in
// the reference's block order.  Exactness: the A operand holds the weight
// pre-scaled by its sub-block scale, w = sc * q <= 63 * 31 = 1953, and the B
// operand the Q8_K byte, both integers an f16 holds exactly; every product
// and every partial sum of one lane sum is an integer below 2^24
// (32 * 1953 * 128 < 2^23), so the f32 accumulation inside the instruction
// is exact in any order and the result equals lane_sums[l] converted to f32
// (which the reference's `as f32` also does exactly).  Each lane sum (the 32
// elements of residue l) is two K = 16 instructions, the second accumulating
// onto the first.  The minimum sum is a 17th instruction on the 6-bit mins
// against the pair sums of bsums split as 128 * bh + bl: A holds
// (128 mn_j, mn_j), B holds (bh_j, bl_j), |partial sums| < 8 * 63 * 8128.
//
// Layouts (built once per matrix by k_prep_a, per call by k_prep_b):
//   A tile (32 rows, block b): 17 operands x 64 lanes x 16 B, operand o at
//     position op_pos(o) (0-3, 16, 4-15: the order the three-pass schedule
//     reads them in), then the 32 rows' d, -dmin, d, d as f32 (a pass of the
//     three-pass schedule stages rows 0-1 or 2-3: chain 2's scale row 1 is
//     then -dmin in pass 0 and d after it, at a fixed address).
//     Operand 2l + p, lane j: row j % 32, the 8 f16 of sub-blocks
//     4p + 2 (j / 32) + e / 4, element 8 (e % 4) + l.
//     Operand 16, lane j: sub-blocks 4 (j / 32) + e / 2, (128 mn, mn).
//   B tile (32 tokens, block b): the same operands for token j % 32 (Q8_K
//     bytes; operand 16 = (bh, bl)), then the 32 tokens' d8.
//   A and B use the same slot <-> element convention, so the contraction
//   pairs identical elements whatever the instruction's internal k order.
#include "lbh_internal.h"
#include "lbh_rows.h"

namespace lbh {

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int OPS = 17;                          // 8 residues x 2 halves + the minimum
constexpr int OP_BYTES = 1024;                   // 64 lanes x 8 f16
constexpr int A_TILE = OPS * OP_BYTES + 32 * 16; // + the rows' scales: d, -dmin, d, d (32 f32 each)
constexpr int B_TILE = OPS * OP_BYTES + 32 * 4;  // + d8 of the tile's tokens
constexpr int PIECES = OPS + 1;                  // 1 KiB staging units per tile (the last one partial)

// Position of operand o in a tile: residue operands 0-3, the minimum operand,
// residue operands 4-15.
__host__ __device__ constexpr int op_pos(int o) { return o < 4 ? o : o == 16 ? 4 : o + 1; }

__device__ __forceinline__ uint32_t pack_f16(_Float16 lo, _Float16 hi) {
    return (uint32_t)__builtin_bit_cast(uint16_t, lo) | ((uint32_t)__builtin_bit_cast(uint16_t, hi) << 16);
}

// ------------------------------------------------------------ A preparation
//
// One wave per (row tile, block).  Reads the block from the chunk-major
// device layout (lbh_layout.h): Q4_K chunk 0 header, chunks 1-8 residue-major
// qs; Q5_K chunk 0 header, 1-2 residue-major qh, 3-10 residue-major qs.
template <int TY>
__global__ void __launch_bounds__(64) k_prep_a(MatView m, uint8_t *a_out) {
    const int lane = threadIdx.x;
    const int nb = m.nb;
    const int tile = blockIdx.x / nb, b = blockIdx.x - tile * nb;
    const int h = lane >> 5;
    const int row = tile * 32 + (lane & 31);
    const bool valid = row < m.rows;
    const long long U = m.units, u = (long long)row * nb + b;
    constexpr int QS0 = TY == T_Q5_K ? 3 : 1;
    constexpr int NCH = TY == T_Q5_K ? 11 : 9;
    uint8_t blk[NCH * 16];
    for (int c = 0; c < NCH; ++c) {
        uint4 v = make_uint4(0, 0, 0, 0);
        if (valid) v = *reinterpret_cast<const uint4 *>(m.planes + ((long long)c * U + u) * 16);
        *reinterpret_cast<uint4 *>(blk + 16 * c) = v;
    }
    int sc[8], mn[8];
    {
        const uint32_t s0 = *reinterpret_cast<const uint32_t *>(blk + 4);
        const uint32_t s1 = *reinterpret_cast<const uint32_t *>(blk + 8);
        const uint32_t s2 = *reinterpret_cast<const uint32_t *>(blk + 12);
        for (int j = 0; j < 8; ++j) scale_min_of(s0, s1, s2, j, sc[j], mn[j]);
    }
    uint8_t *tile_base = a_out + ((long long)tile * nb + b) * A_TILE;
    uint8_t *dst = tile_base + lane * 16;
    for (int l = 0; l < 8; ++l) {
        for (int p = 0; p < 2; ++p) {
            uint32_t o[4];
            for (int e = 0; e < 8; e += 2) {
                int w[2];
                for (int f = 0; f < 2; ++f) {
                    const int jj = 4 * p + 2 * h + ((e + f) >> 2), k = (e + f) & 3;
                    // residue-major: dword l of qs group jj / 2 holds elements l + 8k
                    const int pos = 4 * l + k;
                    const uint8_t qb = blk[16 * (QS0 + 2 * (jj >> 1)) + pos];
                    int v = (jj & 1) ? (qb >> 4) : (qb & 15);
                    if (TY == T_Q5_K) v += ((blk[16 + pos] >> jj) & 1) << 4;
                    w[f] = sc[jj] * v;
                }
                o[e >> 1] = pack_f16((_Float16)w[0], (_Float16)w[1]);
            }
            *reinterpret_cast<uint4 *>(dst + op_pos(2 * l + p) * OP_BYTES) = make_uint4(o[0], o[1], o[2], o[3]);
        }
    }
    {
        uint32_t o[4];
        for (int e = 0; e < 8; e += 2) {
            const int jj = 4 * h + (e >> 1);
            o[e >> 1] = pack_f16((_Float16)(128 * mn[jj]), (_Float16)mn[jj]);
        }
        *reinterpret_cast<uint4 *>(dst + op_pos(16) * OP_BYTES) = make_uint4(o[0], o[1], o[2], o[3]);
    }
    if (lane < 32) {
        float2 v = make_float2(0.0f, 0.0f);
        if (valid) {
            const uint32_t hdr = *reinterpret_cast<const uint32_t *>(blk);
            v = make_float2(f16_to_f32(hdr & 0xffffu), f16_to_f32(hdr >> 16));
        }
        // -dmin: the minimum term is added, sum + (-dmin * d8) * minimum_sum,
        // the same f32 value as the reference's sum - (dmin * d8) * minimum_sum
        // (x - y is x + (-y), and (-a) * b is -(a * b) under round to nearest).
        float *dm = reinterpret_cast<float *>(tile_base + OPS * OP_BYTES);
        dm[lane] = v.x;
        dm[32 + lane] = -v.y;
        dm[64 + lane] = v.x;
        dm[96 + lane] = v.x;
    }
}

// ------------------------------------------------------------ B preparation
//
// One wave per (token tile, block) from GGML Q8_K bytes (d @0, qs @4,
// bsums @260; block (t, b) at q8 + (t * nb + b) * 292).  Lane j needs the
// four sub-blocks 2 (j / 32) + {0, 1, 4, 5} of token j % 32.
__global__ void __launch_bounds__(64) k_prep_b(const uint8_t *q8, int n_tokens, int nb, uint8_t *b_out) {
    const int lane = threadIdx.x;
    const int tile = blockIdx.x / nb, b = blockIdx.x - tile * nb;
    const int h = lane >> 5;
    const int t = tile * 32 + (lane & 31);
    const bool valid = t < n_tokens;
    const uint8_t *blk = q8 + ((long long)(valid ? t : 0) * nb + b) * 292;
    uint8_t *tile_base = b_out + ((long long)tile * nb + b) * B_TILE;
    uint8_t *dst = tile_base + lane * 16;
    // qs of sub-blocks 2h, 2h + 1 (p = 0) and 4 + 2h, 5 + 2h (p = 1): 64 bytes each
    uint32_t q[2][16];
#pragma unroll
    for (int p = 0; p < 2; ++p)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            uint4 v = make_uint4(0, 0, 0, 0);
            if (valid) v = *reinterpret_cast<const uint4 *>(blk + 4 + 32 * (4 * p + 2 * h) + 16 * i);
            q[p][4 * i] = v.x, q[p][4 * i + 1] = v.y, q[p][4 * i + 2] = v.z, q[p][4 * i + 3] = v.w;
        }
#pragma unroll
    for (int l = 0; l < 8; ++l) {
#pragma unroll
        for (int p = 0; p < 2; ++p) {
            uint32_t o[4];
#pragma unroll
            for (int e = 0; e < 8; e += 2) {
                _Float16 x[2];
#pragma unroll
                for (int f = 0; f < 2; ++f) {
                    // element 8k + l of sub-block 4p + 2h + (e + f) / 4: byte 32 * ((e + f) / 4) + 8k + l
                    const int k = (e + f) & 3, byte = 32 * ((e + f) >> 2) + 8 * k + l;
                    x[f] = (_Float16)(int)(int8_t)(q[p][byte >> 2] >> (8 * (byte & 3)));
                }
                o[e >> 1] = pack_f16(x[0], x[1]);
            }
            *reinterpret_cast<uint4 *>(dst + op_pos(2 * l + p) * OP_BYTES) = make_uint4(o[0], o[1], o[2], o[3]);
        }
    }
    {
        uint32_t o[4];
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
            const int jj = 4 * h + (e >> 1);
            int bsp = 0;
            if (valid)
                bsp = (int)*reinterpret_cast<const int16_t *>(blk + 260 + 4 * jj) +
                      (int)*reinterpret_cast<const int16_t *>(blk + 262 + 4 * jj);
            o[e >> 1] = pack_f16((_Float16)(bsp >> 7), (_Float16)(bsp & 127));
        }
        *reinterpret_cast<uint4 *>(dst + op_pos(16) * OP_BYTES) = make_uint4(o[0], o[1], o[2], o[3]);
    }
    if (lane < 32)
        reinterpret_cast<float *>(tile_base + OPS * OP_BYTES)[lane] = valid ? *reinterpret_cast<const float *>(blk) : 0.0f;
}

// ------------------------------------------------------------------ GEMM
//
// Workgroup: 2 x 2 tiles of 32 rows x 32 tokens, two waves per tile: wave
// half 0 runs residues 0-3 and the minimum, half 1 residues 4-7 (the eight
// lane-sum chains are independent until the final sum), so a wave keeps 16
// (row, token) pairs x 4 or 5 f32 chains in registers and two waves share
// each SIMD.  Per block the workgroup stages its two A tiles and two B tiles
// (70 KiB) in LDS, double-buffered.  Two ways to fill the buffers (`mode`):
//   0  global -> registers -> LDS, two blocks ahead: block b + 2 is loaded
//      into one register set while block b is computed, and the set loaded
//      during block b - 1 is written to LDS after it (140 KiB in flight per
//      CU; the loads are latency-bound, so depth is what buys bandwidth);
//   1  direct buffer-to-LDS loads one block ahead (no staging registers).
constexpr int RG = 2, TG = 2;                 // row tiles, token tiles per workgroup
constexpr int NW = 2 * RG * TG;               // waves
constexpr int UNITS = (RG + TG) * PIECES;     // 1 KiB staging units per block
constexpr int UPW = UNITS / NW;               // units per wave (9)
static_assert(UNITS % NW == 0, "every wave stages the same number of units");

// LDS tiles are PIECES whole KiB: the partial last piece is staged with all
// 64 lanes (no divergent loads or stores, so the compiler's wait counts stay
// exact); the bytes past the tile's data are never read.
constexpr int LDS_TILE = PIECES * OP_BYTES;
struct GemmLDS {
    uint8_t a[2][RG][LDS_TILE];
    uint8_t b[2][TG][LDS_TILE];
};

typedef __attribute__((address_space(3))) void lds_void;

// Where staging unit k of wave `wid` lives: unit u = wid + NW k is piece
// u % PIECES of tile u / PIECES (A tiles first).  Tiles past the matrix or
// the batch are clamped to the last one (their results are not stored).
struct Unit {
    bool is_a;
    int tile, piece;
};
__device__ __forceinline__ Unit unit_of(int wid, int k) {
    const int u = wid + NW * k;
    Unit x;
    x.tile = u / PIECES;
    x.piece = u - x.tile * PIECES;
    x.is_a = x.tile < RG;
    if (!x.is_a) x.tile -= RG;
    return x;
}

struct StageSrc {
    __amdgpu_buffer_rsrc_t ra, rb;   // this workgroup's A tiles / B tiles (all blocks)
    int last_a, last_b;              // last valid tile, relative to the workgroup's first
};

// Byte offset of unit x of block b in its descriptor (all operands uniform,
// so the offset is a scalar operand of the load).
__device__ __forceinline__ uint32_t unit_offset(const StageSrc &src, const Unit &x, int nb, int b) {
    if (x.is_a) {
        const int t = x.tile < src.last_a ? x.tile : src.last_a;
        return (uint32_t)((t * nb + b) * A_TILE + x.piece * OP_BYTES);
    }
    const int t = x.tile < src.last_b ? x.tile : src.last_b;
    return (uint32_t)((t * nb + b) * B_TILE + x.piece * OP_BYTES);
}
__device__ __forceinline__ uint8_t *unit_dst(GemmLDS &S, const Unit &x, int buf) {
    return (x.is_a ? S.a[buf][x.tile] : S.b[buf][x.tile]) + x.piece * OP_BYTES;
}

// Loads block b's units of this wave into R; for b >= nb the lane offset is
// pushed past the descriptors' ranges (< 2^31 bytes), so the loads return
// zeros and read no memory.
__device__ __forceinline__ void stage_regs(const StageSrc &src, uint4 (&R)[UPW], int nb, int b, int wid, int lane) {
    const uint32_t vo = (uint32_t)lane * 16 + (b < nb ? 0u : 0x80000000u);
    const int bc = b < nb ? b : nb - 1;
#pragma unroll
    for (int k = 0; k < UPW; ++k) {
        const Unit x = unit_of(wid, k);
        R[k] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(x.is_a ? src.ra : src.rb, vo,
                                                                               unit_offset(src, x, nb, bc), 0));
    }
}
__device__ __forceinline__ void store_regs(GemmLDS &S, const uint4 (&R)[UPW], int buf, int wid, int lane) {
#pragma unroll
    for (int k = 0; k < UPW; ++k) {
        const Unit x = unit_of(wid, k);
        reinterpret_cast<uint4 *>(unit_dst(S, x, buf))[lane] = R[k];
    }
}
__device__ __forceinline__ void stage_dma(const StageSrc &src, GemmLDS &S, int nb, int b, int buf, int wid, int lane) {
#pragma unroll
    for (int k = 0; k < UPW; ++k) {
        const Unit x = unit_of(wid, k);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(x.is_a ? src.ra : src.rb, (lds_void *)unit_dst(S, x, buf), 16,
                                                 lane * 16, unit_offset(src, x, nb, b), 0, 0);
    }
}
__device__ __forceinline__ void wait_dma() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Both MFMAs of residue l (operands 2l, 2l + 1), or the minimum (l = 8).
__device__ __forceinline__ v16f residue_mfma(const v8h *Av, const v8h *Bv, int l) {
    const v16f zero = {};
    if (l == 8) {
        v8h a = Av[op_pos(16) * 64], b = Bv[op_pos(16) * 64];
        asm volatile("" : "+v"(a), "+v"(b));
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, zero, 0, 0, 0);
    }
    const int p0 = op_pos(2 * l), p1 = op_pos(2 * l + 1);
    v8h a0 = Av[p0 * 64], b0 = Bv[p0 * 64], a1 = Av[p1 * 64], b1 = Bv[p1 * 64];
    asm volatile("" : "+v"(a0), "+v"(b0), "+v"(a1), "+v"(b1));
    const v16f c = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0, b0, zero, 0, 0, 0);
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a1, b1, c, 0, 0, 0);
}

// The f32 chains of one wave.  The lane's pair i (0..15) is row
// 8 (i / 4) + 4 (lane / 32) + i % 4 of the tile, token lane % 32.
template <int HV>
struct Chains {
    float c[16][4];   // residues 4 HV + r
    float msum[16];   // the minimum chain (HV 0)
};

// One block of one wave: HV 0 folds residues 0-3 and the minimum, HV 1
// residues 4-7, each in the reference's order within its chain.
template <int HV>
__device__ __forceinline__ void fold_block(Chains<HV> &ch, const uint8_t *At, const uint8_t *Bt, int lane) {
    const int h = lane >> 5;
    const v8h *Av = reinterpret_cast<const v8h *>(At) + lane;
    const v8h *Bv = reinterpret_cast<const v8h *>(Bt) + lane;
    const float d8 = reinterpret_cast<const float *>(Bt + OPS * OP_BYTES)[lane & 31];
    // d of rows 8q + 4h + 0..3 (the lane's pairs 4q..4q + 3): one 16-byte read per q
    const float4 *dv = reinterpret_cast<const float4 *>(At + OPS * OP_BYTES);
    float sc[16];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const float4 d = dv[2 * q + h];
        sc[4 * q] = __fmul_rn(d.x, d8);
        sc[4 * q + 1] = __fmul_rn(d.y, d8);
        sc[4 * q + 2] = __fmul_rn(d.z, d8);
        sc[4 * q + 3] = __fmul_rn(d.w, d8);
    }
    // The MFMAs of step r + 1 go out before step r is folded; the empty asm
    // statements (no instructions) keep the compiler from hoisting every
    // step's MFMAs (16 result registers each) above the folds.
    v16f cn = residue_mfma(Av, Bv, 4 * HV);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const v16f c = cn;
        if (r < 3) cn = residue_mfma(Av, Bv, 4 * HV + r + 1);
        else if (HV == 0) cn = residue_mfma(Av, Bv, 8);
#pragma unroll
        for (int i = 0; i < 16; ++i) ch.c[i][r] = __fadd_rn(ch.c[i][r], __fmul_rn(sc[i], c[i]));
        asm volatile("" : "+v"(ch.c[0][r]), "+v"(ch.c[1][r]), "+v"(ch.c[2][r]), "+v"(ch.c[3][r]),
                     "+v"(ch.c[4][r]), "+v"(ch.c[5][r]), "+v"(ch.c[6][r]), "+v"(ch.c[7][r]),
                     "+v"(ch.c[8][r]), "+v"(ch.c[9][r]), "+v"(ch.c[10][r]), "+v"(ch.c[11][r]),
                     "+v"(ch.c[12][r]), "+v"(ch.c[13][r]), "+v"(ch.c[14][r]), "+v"(ch.c[15][r]));
    }
    if (HV == 0) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float4 m = dv[8 + 2 * q + h];   // -dmin
            const float ms[4] = {__fmul_rn(m.x, d8), __fmul_rn(m.y, d8), __fmul_rn(m.z, d8), __fmul_rn(m.w, d8)};
#pragma unroll
            for (int e = 0; e < 4; ++e)
                ch.msum[4 * q + e] = __fadd_rn(ch.msum[4 * q + e], __fmul_rn(ms[e], cn[4 * q + e]));
        }
    }
}

template <int MODE, int HV>
__device__ __forceinline__ void gemm_tile(const GemmArgs &g, const MatGemm &M, GemmLDS &S, const StageSrc &src,
                                          int rg, int tg, int tw, int wid, int lane, int rt0, int tt0) {
    const int nb = g.nb;
    Chains<HV> ch;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        ch.msum[i] = 0.0f;
#pragma unroll
        for (int r = 0; r < 4; ++r) ch.c[i][r] = 0.0f;
    }
    if (MODE == 0) {
        // Block j: loaded into R[j % 2] during block j - 2, written to LDS
        // buffer j % 2 after block j - 1, computed as block j.  Every load
        // is unconditional, so the compiler's wait before each LDS store
        // leaves the younger set's loads in flight; loads past the last
        // block are sent out of the descriptor's range (they return zeros
        // without touching memory).
        uint4 R0[UPW], R1[UPW];
        stage_regs(src, R0, nb, 0, wid, lane);
        stage_regs(src, R1, nb, 1, wid, lane);
        store_regs(S, R0, 0, wid, lane);
        __syncthreads();
        for (int b = 0; b < nb; b += 2) {
            stage_regs(src, R0, nb, b + 2, wid, lane);
            fold_block<HV>(ch, S.a[0][rg], S.b[0][tg], lane);
            if (b + 1 < nb) store_regs(S, R1, 1, wid, lane);
            __syncthreads();
            if (b + 1 >= nb) break;
            stage_regs(src, R1, nb, b + 3, wid, lane);
            fold_block<HV>(ch, S.a[1][rg], S.b[1][tg], lane);
            if (b + 2 < nb) store_regs(S, R0, 0, wid, lane);
            __syncthreads();
        }
    } else {
        stage_dma(src, S, nb, 0, 0, wid, lane);
        wait_dma();
        __syncthreads();
        for (int b = 0; b < nb; ++b) {
            const int buf = b & 1;
            if (b + 1 < nb) stage_dma(src, S, nb, b + 1, buf ^ 1, wid, lane);
            fold_block<HV>(ch, S.a[buf][rg], S.b[buf][tg], lane);
            wait_dma();
            __syncthreads();
        }
    }

    // result = minimum chain + sums[0] + ... + sums[7]: half 0 adds its four
    // chains onto the minimum chain and hands the partial to half 1 through
    // LDS (the staging buffers are free after the last barrier).
    const int h = lane >> 5;
    float *xch = reinterpret_cast<float *>(&S) + tw * 16 * 64;
    if (HV == 0) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            float v = ch.msum[i];
#pragma unroll
            for (int r = 0; r < 4; ++r) v = __fadd_rn(v, ch.c[i][r]);
            xch[i * 64 + lane] = v;
        }
    }
    __syncthreads();
    if (HV == 1) {
        const int t = (tt0 + tg) * 32 + (lane & 31);
        if (t >= g.n_tokens) return;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int row = (rt0 + rg) * 32 + 8 * (i >> 2) + 4 * h + (i & 3);
            float v = xch[i * 64 + lane];
#pragma unroll
            for (int r = 0; r < 4; ++r) v = __fadd_rn(v, ch.c[i][r]);
            if (row < M.rows) M.y[(long long)t * M.ldy + row] = v;
        }
    }
}

template <int MODE>
__global__ void __launch_bounds__(64 * NW) k_kq_gemm(GemmArgs g) {
    extern __shared__ __align__(16) uint8_t smem[];
    GemmLDS &S = *reinterpret_cast<GemmLDS *>(smem);
    const int lane = threadIdx.x & 63;
    const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // waves w and w + RG * TG (the two halves of one tile) land on the same SIMD
    const int tw = wid % (RG * TG), hv = wid / (RG * TG);
    const int rg = tw % RG, tg = tw / RG;
    const MatGemm &M = g.mat[blockIdx.y];   // which matrix of the launch
    const int n_rt = (M.rows + 31) / 32, n_tt = (g.n_tokens + 31) / 32;
    const int row_wgs = (n_rt + RG - 1) / RG, tok_wgs = (n_tt + TG - 1) / TG;
    // XCD-aware order: workgroups are dealt to the eight XCDs round robin;
    // consecutive workgroups of one XCD share a row tile, so each A tile is
    // fetched into that XCD's L2 once for all of its token tiles.  Within an
    // XCD's range the token tiles are taken in two phases (the first half of
    // the token workgroups over all of the XCD's row bands, then the second
    // half): half the activation tiles are live in the XCD's 4 MB L2 at a
    // time, for every A band read twice (measured 2-4% faster than one phase).
    const int nwg = row_wgs * tok_wgs;
    const int id = (int)blockIdx.x;
    if (id >= nwg) return;
    const int nfull = nwg & ~7;
    int lin = id < nfull ? (id % 8) * (nfull / 8) + id / 8 : id;   // a bijection of [0, nwg)
    {
        constexpr int PHASES = 2;
        const int per = nfull / 8;
        if (id < nfull && tok_wgs % PHASES == 0 && per % tok_wgs == 0) {
            const int x = lin / per, i = lin - x * per;
            const int tq = tok_wgs / PHASES, bands = per / tok_wgs;
            const int ph = i / (bands * tq), rem = i - ph * bands * tq;
            lin = x * per + (rem / tq) * tok_wgs + ph * tq + rem % tq;   // still a bijection of the XCD's range
        }
    }
    const int wrt = lin / tok_wgs, wtt = lin - wrt * tok_wgs;
    const int rt0 = wrt * RG, tt0 = wtt * TG;

    // The descriptors span only the workgroup's valid tiles: the partial last
    // staging piece of the last tile then reads zeros past it, never memory
    // past the allocation.
    StageSrc src;
    src.last_a = n_rt - 1 - rt0 < RG - 1 ? n_rt - 1 - rt0 : RG - 1;
    src.last_b = n_tt - 1 - tt0 < TG - 1 ? n_tt - 1 - tt0 : TG - 1;
    src.ra = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(M.a + (long long)rt0 * g.nb * A_TILE), (short)0,
                                               (src.last_a + 1) * g.nb * A_TILE, 0x00020000);
    src.rb = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(g.b + (long long)tt0 * g.nb * B_TILE), (short)0,
                                               (src.last_b + 1) * g.nb * B_TILE, 0x00020000);

    if (hv == 0)
        gemm_tile<MODE, 0>(g, M, S, src, rg, tg, tw, wid, lane, rt0, tt0);
    else
        gemm_tile<MODE, 1>(g, M, S, src, rg, tg, tw, wid, lane, rt0, tt0);
}

// ------------------------------------------------------- three-pass GEMM
//
// The nine chains of a (row, token) pair are independent until the final sum
// result = ((sum_min + s_0) + s_1) + ... + s_7, so they can run as three
// passes over K in the reference's order, the running result kept in
// registers between them:
//   pass 0: lane chains 0, 1 and the minimum chain (tile positions 0-4)
//   pass 1: lane chains 2, 3, 4 (positions 5-10)
//   pass 2: lane chains 5, 6, 7 (positions 11-16)
// A pass stages only its own operands (six slots: pass p's positions
// 6p - (p > 0) + 0..5, pass 0's sixth slot zeros), plus the tile's scales,
// so one workgroup covers RG x TG = 12 tiles of 32 x 32 with one wave per
// tile and three chains per wave (3 waves per SIMD), and each staged tile
// serves TG (A) or RG (B) tiles: about 60% of the 2 x 2 schedule's staged
// bytes per output.  Chain c of a pass is the MFMA pair on slots 2c, 2c + 1;
// pass 0's minimum chain pairs its operand with the zero slot (the second
// instruction adds exact zeros).  A stage is (RG + TG) tiles x 7 KiB (six
// operand slots, then the 1 KiB piece holding d/-dmin or d8), triple-buffered
// in LDS by direct buffer-to-LDS loads two stages ahead.
constexpr int P3_WAVES = 12;
constexpr int P3_SLOTS = 7;                                   // 6 operands + the scale piece
constexpr int P3_TILE = P3_SLOTS * OP_BYTES;
constexpr int P3_MAX_TILES = 7;                               // RG + TG
constexpr int P3_PAD = P3_MAX_TILES * P3_TILE;                // target of the padding loads
constexpr int P3_BUF = P3_PAD + OP_BYTES;
static_assert(op_pos(16) == 4 && op_pos(4) == 5, "pass windows: 0-4 (+ zeros), 5-10, 11-16");

// The three stage buffers are distinct LDS arrays, each addressed statically
// (the stage loop is unrolled by three): the compiler's wait before an LDS
// read then covers only the buffer-to-LDS loads into that array, not the
// prefetches into the other two, which stay in flight.
__shared__ __align__(16) uint8_t p3_lds0[P3_BUF];
__shared__ __align__(16) uint8_t p3_lds1[P3_BUF];
__shared__ __align__(16) uint8_t p3_lds2[P3_BUF];

template <int BUF>
__device__ __forceinline__ uint8_t *p3_buffer() {
    return BUF == 0 ? p3_lds0 : BUF == 1 ? p3_lds1 : p3_lds2;
}

template <int RG_, int TG_>
struct P3 {
    static_assert(RG_ * TG_ == P3_WAVES, "one wave per tile");
    static_assert(RG_ + TG_ <= P3_MAX_TILES, "stages fit the LDS buffers");
    static constexpr int RG = RG_, TG = TG_;
    static constexpr int UA = (RG * P3_SLOTS + P3_WAVES - 1) / P3_WAVES;   // A loads per wave per stage
    static constexpr int UB = (TG * P3_SLOTS + P3_WAVES - 1) / P3_WAVES;   // B loads per wave per stage
    static constexpr int UPW = UA + UB;
};

// This wave's share of a stage's loads, fixed for the whole K loop: load k of
// the A side is unit u = wid + 12 k of the RG x 7 A units (slot u % 7 of A
// tile u / 7), likewise for the TG x 7 B units; units past a side's count
// are padding.  Per unit: its LDS offset in a stage buffer, the byte offset
// in the side's descriptor of its piece in block 0 of pass 0 (the scale
// piece: the same in every pass), and three masks: pad (0x80000000 for a
// unit past the stage), zero (all ones for pass 0's sixth slot), win (all
// ones unless the scale piece, which ignores the pass window).
struct P3Unit {
    int lds, off;
    uint32_t pad, zero, win;
};
template <int SIDE_TILES, int TILE_BYTES>
__device__ __forceinline__ P3Unit p3_unit(int u, int lds_tile0, int last, int nb) {
    P3Unit x;
    const int ti = u / P3_SLOTS, slot = u - ti * P3_SLOTS;
    const bool in_stage = u < SIDE_TILES * P3_SLOTS;
    x.pad = in_stage ? 0u : 0x80000000u;
    x.zero = slot == 5 ? ~0u : 0u;
    x.win = slot == 6 ? 0u : ~0u;
    x.lds = in_stage ? (lds_tile0 + ti) * P3_TILE + slot * OP_BYTES : P3_PAD;
    x.off = (ti < last ? ti : last) * nb * TILE_BYTES + (slot == 6 ? OPS : slot) * OP_BYTES;
    return x;
}

// Issues this wave's loads of the stage at (poff, bA, bB) into buffer BUF:
// poff = the pass's window start in bytes, bA / bB = the block's offset in a
// tile row of the A / B side, dead = 0x80000000 for a stage past the end (all
// its loads padding), z0 = 0x80000000 in pass 0 (its sixth slot is zeros),
// soff = where the A scale piece starts (0 in pass 0, 256 after).
// A padding load reads from beyond the descriptor range (zeros, no memory
// traffic): units past the stage into the buffer's padding piece, pass 0's
// sixth slot into that slot.  Every wave issues UPW loads per stage, with no
// branch between them, so one wait count serves all and the compiler's own
// waits before the LDS reads stay exact.
template <class S, int BUF>
__device__ __forceinline__ void p3_issue(const StageSrc &src, const P3Unit (&ua)[S::UA], const P3Unit (&ub)[S::UB],
                                         int poff, int bA, int bB, uint32_t dead, uint32_t z0, uint32_t soff,
                                         uint32_t lane16) {
    uint8_t *buf = p3_buffer<BUF>();
#pragma unroll
    for (int k = 0; k < S::UA + S::UB; ++k) {
        const bool is_a = k < S::UA;
        const P3Unit &x = is_a ? ua[k] : ub[k - S::UA];
        const uint32_t vo = lane16 | (x.pad | dead | (z0 & x.zero));
        uint32_t off = (uint32_t)(x.off + (is_a ? bA : bB)) + ((uint32_t)poff & x.win);
        if (is_a) off += soff & ~x.win;   // A scale piece: rows 0-1 in pass 0, rows 2-3 after
        __builtin_amdgcn_raw_ptr_buffer_load_lds(is_a ? src.ra : src.rb, (lds_void *)(buf + x.lds), 16, vo, off, 0, 0);
    }
}

// One block of the wave's tile (At, Bt: its A and B tiles in the stage
// buffer): chain c += (scale * d8) * integer sum, in the reference's order
// (q8_k.rs:314-326), with scale = staged row 0 (d) for chains 0 and 1, and
// for chain 2 row 1 in pass 0 (-dmin: the minimum chain) and d after it.
// The operands of chain c + 1 are read from LDS while chain c's MFMAs run
// and its fold issues.
__device__ __forceinline__ void p3_block(float (&ch)[3][16], const uint8_t *At, const uint8_t *Bt, int lane,
                                         bool first_pass) {
    const int h = lane >> 5;
    const v8h *Av = reinterpret_cast<const v8h *>(At) + lane;
    const v8h *Bv = reinterpret_cast<const v8h *>(Bt) + lane;
    const float d8 = reinterpret_cast<const float *>(Bt + 6 * OP_BYTES)[lane & 31];
    const float4 *dv = reinterpret_cast<const float4 *>(At + 6 * OP_BYTES);
    v8h a0 = Av[0], b0 = Bv[0], a1 = Av[64], b1 = Bv[64];
    float sc[16];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const float4 d = dv[2 * q + h];
        sc[4 * q] = __fmul_rn(d.x, d8);
        sc[4 * q + 1] = __fmul_rn(d.y, d8);
        sc[4 * q + 2] = __fmul_rn(d.z, d8);
        sc[4 * q + 3] = __fmul_rn(d.w, d8);
    }
#pragma unroll
    for (int c = 0; c < 3; ++c) {
        const v16f zero = {};
        asm volatile("" : "+v"(a0), "+v"(b0), "+v"(a1), "+v"(b1));
        const v16f x = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0, b0, zero, 0, 0, 0);
        const v16f cur = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1, b1, x, 0, 0, 0);
        if (c < 2) {
            a0 = Av[2 * (c + 1) * 64], b0 = Bv[2 * (c + 1) * 64];
            a1 = Av[(2 * c + 3) * 64], b1 = Bv[(2 * c + 3) * 64];
        }
        __builtin_amdgcn_sched_barrier(0);   // the reads go out before this chain's fold
        if (c < 2 || !first_pass) {
#pragma unroll
            for (int i = 0; i < 16; ++i) ch[c][i] = __fadd_rn(ch[c][i], __fmul_rn(sc[i], cur[i]));
        } else {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float4 e = dv[8 + 2 * q + h];
                const float ms[4] = {__fmul_rn(e.x, d8), __fmul_rn(e.y, d8), __fmul_rn(e.z, d8), __fmul_rn(e.w, d8)};
#pragma unroll
                for (int k = 0; k < 4; ++k) ch[2][4 * q + k] = __fadd_rn(ch[2][4 * q + k], __fmul_rn(ms[k], cur[4 * q + k]));
            }
        }
        asm volatile("" : "+v"(ch[c][0]), "+v"(ch[c][1]), "+v"(ch[c][2]), "+v"(ch[c][3]), "+v"(ch[c][4]),
                     "+v"(ch[c][5]), "+v"(ch[c][6]), "+v"(ch[c][7]), "+v"(ch[c][8]), "+v"(ch[c][9]),
                     "+v"(ch[c][10]), "+v"(ch[c][11]), "+v"(ch[c][12]), "+v"(ch[c][13]), "+v"(ch[c][14]),
                     "+v"(ch[c][15]));
    }
}

// Stage position: pass p, block b of the stage computed (cp, cb) and of the
// stage issued two ahead (ip, ib), advanced without divisions; ipoff, ibA,
// ibB the issued stage's pass window and block offsets.
struct P3Pos {
    int cp, cb, ip, ib, ipoff, ibA, ibB;
};
__device__ __forceinline__ void p3_next_issue(P3Pos &ps, int nb) {
    ps.ibA += A_TILE, ps.ibB += B_TILE;
    if (++ps.ib == nb) {
        ps.ib = 0, ps.ibA = 0, ps.ibB = 0, ++ps.ip;
        ps.ipoff = (6 * ps.ip - 1) * OP_BYTES;
    }
}
// The issued stage's masks for p3_issue, made opaque to the compiler (an empty
// asm statement) so it cannot specialise the loads on the pass.
template <class S, int BUF>
__device__ __forceinline__ void p3_issue_at(const StageSrc &src, const P3Unit (&ua)[S::UA],
                                            const P3Unit (&ub)[S::UB], const P3Pos &ps, uint32_t lane16) {
    uint32_t dead = (uint32_t)(2 - ps.ip) & 0x80000000u;   // ip == 3: past the end
    uint32_t z0 = (uint32_t)(ps.ip - 1) & 0x80000000u;     // ip == 0
    uint32_t soff = ~z0 >> 23 & 256u;                      // 0 in pass 0, 256 after
    asm volatile("" : "+s"(dead), "+s"(z0), "+s"(soff));
    p3_issue<S, BUF>(src, ua, ub, ps.ipoff, ps.ibA, ps.ibB, dead, z0, soff, lane16);
}

// Stage s of the K loop in buffer BUF = s % 3: wait for this wave's loads of
// stage s (stage s + 1's stay in flight), barrier (every wave's loads of
// stage s have landed and every wave has finished stage s - 1, whose buffer
// is refilled next), issue stage s + 2 (padding past the end: the control
// flow is the same in every stage, which keeps the compiler's own wait before
// each LDS read down to the loads into that buffer), then the block's MFMAs
// and folds for pass cp.  At a pass's last block the pass's chains go onto
// the running result v in the reference's order (pass 0: minimum chain, then
// lane chains 0, 1) and restart.
template <class S, int BUF>
__device__ __forceinline__ void p3_stage(float (&ch)[3][16], float (&v)[16], const StageSrc &src,
                                         const P3Unit (&ua)[S::UA], const P3Unit (&ub)[S::UB], P3Pos &ps, int nb,
                                         int lane, int rt, int tt) {
    static_assert(S::UPW == 5, "the wait count below is one stage's loads");
    asm volatile("s_waitcnt vmcnt(5)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    p3_issue_at<S, (BUF + 2) % 3>(src, ua, ub, ps, (uint32_t)lane * 16);
    p3_next_issue(ps, nb);
    // The lane index goes through an empty asm statement per stage, so the
    // lane addresses into this buffer are formed here, not kept in registers
    // across the loop for all three buffers.
    int ln = lane;
    asm volatile("" : "+v"(ln));
    const uint8_t *buf = p3_buffer<BUF>();
    const int p = ps.cp;
    p3_block(ch, buf + rt * P3_TILE, buf + (S::RG + tt) * P3_TILE, ln, p == 0);
    if (ps.cb == nb - 1) {
        if (p == 0) {
#pragma unroll
            for (int i = 0; i < 16; ++i) v[i] = __fadd_rn(__fadd_rn(ch[2][i], ch[0][i]), ch[1][i]);
        } else {
#pragma unroll
            for (int i = 0; i < 16; ++i) v[i] = __fadd_rn(__fadd_rn(__fadd_rn(v[i], ch[0][i]), ch[1][i]), ch[2][i]);
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) ch[0][i] = ch[1][i] = ch[2][i] = 0.0f;
    }
    if (++ps.cb == nb) ps.cb = 0, ++ps.cp;
}

template <int RG_, int TG_>
__global__ void __launch_bounds__(64 * P3_WAVES) k_kq_gemm3(GemmArgs g) {
    using S = P3<RG_, TG_>;
    const int lane = threadIdx.x & 63;
    const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int rt = wid % S::RG, tt = wid / S::RG;
    const MatGemm &M = g.mat[blockIdx.y];
    const int nb = g.nb;
    const int n_rt = (M.rows + 31) / 32, n_tt = (g.n_tokens + 31) / 32;
    const int row_wgs = (n_rt + S::RG - 1) / S::RG, tok_wgs = (n_tt + S::TG - 1) / S::TG;
    // XCD-aware order: workgroups are dealt to the eight XCDs round robin;
    // each XCD takes a contiguous run of row groups with all their token
    // groups, so the token groups of a row group run together on one XCD and
    // its A tiles are fetched into that XCD's L2 once.
    const int nwg = row_wgs * tok_wgs;
    const int id = (int)blockIdx.x;
    if (id >= nwg) return;
    const int nfull = nwg & ~7;
    const int lin = id < nfull ? (id % 8) * (nfull / 8) + id / 8 : id;   // a bijection of [0, nwg)
    const int wrt = lin / tok_wgs, wtt = lin - wrt * tok_wgs;
    const int rt0 = wrt * S::RG, tt0 = wtt * S::TG;

    // The descriptors span only the workgroup's valid tiles (the scale piece
    // of the last one reads zeros past it, never memory past the allocation).
    StageSrc src;
    src.last_a = n_rt - 1 - rt0 < S::RG - 1 ? n_rt - 1 - rt0 : S::RG - 1;
    src.last_b = n_tt - 1 - tt0 < S::TG - 1 ? n_tt - 1 - tt0 : S::TG - 1;
    src.ra = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(M.a + (long long)rt0 * nb * A_TILE), (short)0,
                                               (src.last_a + 1) * nb * A_TILE, 0x00020000);
    src.rb = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(g.b + (long long)tt0 * nb * B_TILE), (short)0,
                                               (src.last_b + 1) * nb * B_TILE, 0x00020000);

    P3Unit ua[S::UA], ub[S::UB];
#pragma unroll
    for (int k = 0; k < S::UA; ++k) ua[k] = p3_unit<S::RG, A_TILE>(wid + P3_WAVES * k, 0, src.last_a, nb);
#pragma unroll
    for (int k = 0; k < S::UB; ++k) ub[k] = p3_unit<S::TG, B_TILE>(wid + P3_WAVES * k, S::RG, src.last_b, nb);

    const int total = 3 * nb;   // stages: (pass, block), a multiple of three
    P3Pos ps{0, 0, 0, 0, 0, 0, 0};
    p3_issue_at<S, 0>(src, ua, ub, ps, (uint32_t)lane * 16);
    p3_next_issue(ps, nb);
    p3_issue_at<S, 1>(src, ua, ub, ps, (uint32_t)lane * 16);
    p3_next_issue(ps, nb);
    float ch[3][16], v[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) ch[0][i] = ch[1][i] = ch[2][i] = v[i] = 0.0f;
    for (int s = 0; s < total; s += 3) {
        p3_stage<S, 0>(ch, v, src, ua, ub, ps, nb, lane, rt, tt);
        p3_stage<S, 1>(ch, v, src, ua, ub, ps, nb, lane, rt, tt);
        p3_stage<S, 2>(ch, v, src, ua, ub, ps, nb, lane, rt, tt);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // the padding loads land before the LDS is released

    const int h = lane >> 5;
    const int t = (tt0 + tt) * 32 + (lane & 31);
    if (t >= g.n_tokens) return;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int row = (rt0 + rt) * 32 + 8 * (i >> 2) + 4 * h + (i & 3);
        if (row < M.rows) M.y[(long long)t * M.ldy + row] = v[i];
    }
}

// ---------------------------------------------------------------- launchers

static inline int cdiv(long long a, long long b) { return (int)((a + b - 1) / b); }

size_t gemm_a_bytes(int rows, int nb) { return (size_t)cdiv(rows, 32) * nb * A_TILE; }
size_t gemm_b_bytes(int n_tokens, int nb) { return (size_t)cdiv(n_tokens, 32) * nb * B_TILE; }

hipError_t launch_prep_a(const MatView &m, uint8_t *a, hipStream_t s) {
    const int grid = cdiv(m.rows, 32) * m.nb;
    if (m.type == T_Q4_K)
        hipLaunchKernelGGL(k_prep_a<T_Q4_K>, dim3(grid), dim3(64), 0, s, m, a);
    else if (m.type == T_Q5_K)
        hipLaunchKernelGGL(k_prep_a<T_Q5_K>, dim3(grid), dim3(64), 0, s, m, a);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_prep_b(const uint8_t *q8, int n_tokens, int nb, uint8_t *b, hipStream_t s) {
    hipLaunchKernelGGL(k_prep_b, dim3(cdiv(n_tokens, 32) * nb), dim3(64), 0, s, q8, n_tokens, nb, b);
    return hipGetLastError();
}

template <int MODE>
static hipError_t gemm_mode(const GemmArgs &g, hipStream_t s) {
    const int lds = (int)sizeof(GemmLDS);
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(k_kq_gemm<MODE>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    if (e != hipSuccess) return e;
    int rows = 0;
    for (int i = 0; i < g.n_mat; ++i) rows = g.mat[i].rows > rows ? g.mat[i].rows : rows;
    const int grid = cdiv(cdiv(rows, 32), RG) * cdiv(cdiv(g.n_tokens, 32), TG);
    hipLaunchKernelGGL((k_kq_gemm<MODE>), dim3(grid, g.n_mat), dim3(64 * NW), lds, s, g);
    return hipGetLastError();
}

template <int RG_, int TG_>
static hipError_t gemm_p3(const GemmArgs &g, hipStream_t s) {
    using S = P3<RG_, TG_>;
    int rows = 0;
    for (int i = 0; i < g.n_mat; ++i) rows = g.mat[i].rows > rows ? g.mat[i].rows : rows;
    const int grid = cdiv(cdiv(rows, 32), S::RG) * cdiv(cdiv(g.n_tokens, 32), S::TG);
    hipLaunchKernelGGL((k_kq_gemm3<RG_, TG_>), dim3(grid, g.n_mat), dim3(64 * P3_WAVES), 0, s, g);
    return hipGetLastError();
}

// shape: 0 default (three passes from 97 tokens: four token tiles per
// workgroup; the 2 x 2 schedule staged through registers below), 1 the 2 x 2
// schedule with direct buffer-to-LDS staging, 2 the 2 x 2 schedule staged
// through registers, 3 three passes.
hipError_t launch_kq_gemm(const GemmArgs &g, hipStream_t s) {
    if (g.n_mat < 1 || g.n_mat > GEMM_MAX_MATS || g.n_tokens < 1 || g.nb < 1 || g.nb > 64) return hipErrorInvalidValue;
    switch (g.shape) {
    case 1: return gemm_mode<1>(g, s);
    case 2: return gemm_mode<0>(g, s);
    case 3: return gemm_p3<3, 4>(g, s);
    default: return g.n_tokens > 96 ? gemm_p3<3, 4>(g, s) : gemm_mode<0>(g, s);
    }
}

}  // namespace lbh
