// lbh_gemm.hip — Q4_K / Q5_K x Q8_K for a batch of tokens on the i8 matrix
// cores (v_mfma_i32_32x32x32_i8), bit-identical to the reference's per-row
// dot (dot_q4_or_q5_k, crates/bridge-quant-layout/src/q8_k.rs:247-327) for
// every (row, token):
//
//   lane_sums[l] = sum_j sc_j * sum_{k<4} q[32j + 8k + l] * a[32j + 8k + l]
//   minimum_sum  = sum_j mn_j * (bsums[2j] + bsums[2j + 1])
//   per block:  sums[l] += (d * d8) * lane_sums[l];  sum -= (dmin * d8) * minimum_sum
//   result = sum + sums[0] + ... + sums[7]
//
// The integer stage runs on MFMA; the f32 chains run on the VALU in the
// reference's block order.  Exactness: every lane sum has its own MFMA
// (K = the 32 elements of residue l), the sub-block scale is folded into the
// weight (w = sc * q <= 63 * 31, split w = 64 * hi + lo into two int8 rows of
// the A operand, interleaved so one lane holds both), and the minimum sum is a
// ninth MFMA on the 6-bit mins and the pair sums of bsums split as
// 128 * bh + bl.  All integer sums are exact in int32.
//
// Layouts (built once per matrix by k_prep_a, per call by k_prep_b):
//   A tile (16 rows, block b): 9 MFMA operands x 64 lanes x 16 B; lane j
//     feeds A row m = j % 32 (real row m / 2, hi when m is even, lo when odd)
//     with the 16 K-bytes of half j / 32: sub-blocks 4 (j / 32) + q / 4,
//     k = q % 4 (q = byte).  Operand 8 is the minimum MFMA.
//   B tile (32 tokens, block b): the same shape; lane j feeds token j % 32.
//   A and B use the same byte <-> k convention, so the contraction pairs
//   identical elements whatever the instruction's internal k order.
#include "lbh_internal.h"
#include "lbh_rows.h"

namespace lbh {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int OPS = 9;                 // MFMA operands per (tile, block): 8 residues + minimum
constexpr int TILE_BYTES = OPS * 1024; // 64 lanes x 16 B per operand

// ------------------------------------------------------------ A preparation
//
// One wave per (row tile, block).  Reads the block from the chunk-major
// device layout (lbh_layout.h): Q4_K chunk 0 header, chunks 1-8 residue-major
// qs; Q5_K chunk 0 header, 1-2 residue-major qh, 3-10 residue-major qs.
template <int TY>
__global__ void __launch_bounds__(64) k_prep_a(MatView m, uint8_t *a_out, float2 *dm_out) {
    const int lane = threadIdx.x;
    const int nb = m.nb;
    const int tile = blockIdx.x / nb, b = blockIdx.x - tile * nb;
    const int mrow = lane & 31, hl = mrow & 1, h = lane >> 5;
    const int row = tile * 16 + (mrow >> 1);
    const bool valid = row < m.rows;
    const long long U = m.units, u = (long long)row * nb + b;
    constexpr int QS0 = TY == T_Q5_K ? 3 : 1;
    uint8_t blk[176];
    if (valid) {
        const int nch = TY == T_Q5_K ? 11 : 9;
        for (int c = 0; c < nch; ++c) {
            const uint4 v = *reinterpret_cast<const uint4 *>(m.planes + ((long long)c * U + u) * 16);
            *reinterpret_cast<uint4 *>(blk + 16 * c) = v;
        }
    } else {
        for (int i = 0; i < 176; ++i) blk[i] = 0;
    }
    int sc[8], mn[8];
    {
        const uint32_t s0 = *reinterpret_cast<const uint32_t *>(blk + 4);
        const uint32_t s1 = *reinterpret_cast<const uint32_t *>(blk + 8);
        const uint32_t s2 = *reinterpret_cast<const uint32_t *>(blk + 12);
        for (int j = 0; j < 8; ++j) scale_min_of(s0, s1, s2, j, sc[j], mn[j]);
    }
    uint8_t *dst = a_out + ((long long)tile * nb + b) * TILE_BYTES + lane * 16;
    for (int l = 0; l < 8; ++l) {
        uint8_t o[16];
        for (int q = 0; q < 16; ++q) {
            const int jj = 4 * h + q / 4, kk = q % 4;
            const int g = jj >> 1;
            // residue-major: dword l of group g holds elements l + 8k of the group's 32 bytes
            const int pos = 4 * l + kk;
            const uint8_t qb = blk[16 * (QS0 + 2 * g) + pos];
            int v = (jj & 1) ? (qb >> 4) : (qb & 15);
            if (TY == T_Q5_K) {
                const uint8_t hb = blk[16 + pos];
                v += ((hb >> jj) & 1) * 16;
            }
            const int w = sc[jj] * v;
            o[q] = (uint8_t)(hl ? (w & 63) : (w >> 6));
        }
        for (int q = 0; q < 16; ++q) dst[l * 1024 + q] = o[q];
    }
    {
        uint8_t o[16];
        for (int q = 0; q < 16; ++q) {
            int v = 0;
            if (h == 0) v = q < 8 ? (hl == 0 ? mn[q] : 0) : (hl == 1 ? mn[q - 8] : 0);
            o[q] = (uint8_t)v;
        }
        for (int q = 0; q < 16; ++q) dst[8 * 1024 + q] = o[q];
    }
    if (lane < 16) {
        const int r = tile * 16 + lane;
        float2 v = make_float2(0.0f, 0.0f);
        if (r < m.rows) {
            const uint32_t hdr = *reinterpret_cast<const uint32_t *>(m.planes + ((long long)r * nb + b) * 16);
            v = make_float2(f16_to_f32(hdr & 0xffffu), f16_to_f32(hdr >> 16));
        }
        dm_out[(long long)r * nb + b] = v;
    }
}

// ------------------------------------------------------------ B preparation
//
// One wave per (token tile, block) from GGML Q8_K bytes (d @0, qs @4,
// bsums @260; block (t, b) at q8 + (t * nb + b) * 292).
__global__ void __launch_bounds__(64) k_prep_b(const uint8_t *q8, int n_tokens, int nb, uint8_t *b_out, float *d8_out) {
    const int lane = threadIdx.x;
    const int tile = blockIdx.x / nb, b = blockIdx.x - tile * nb;
    const int n = lane & 31, h = lane >> 5;
    const int t = tile * 32 + n;
    const bool valid = t < n_tokens;
    const uint8_t *blk = q8 + ((long long)(valid ? t : 0) * nb + b) * 292;
    uint8_t *dst = b_out + ((long long)tile * nb + b) * TILE_BYTES + lane * 16;
    for (int l = 0; l < 8; ++l) {
        uint32_t w[4];
        for (int i = 0; i < 4; ++i) {
            uint32_t v = 0;
            for (int kk = 0; kk < 4; ++kk) {
                const int jj = 4 * h + i;
                const uint32_t byte = valid ? blk[4 + 32 * jj + 8 * kk + l] : 0u;
                v |= byte << (8 * kk);
            }
            w[i] = v;
        }
        *reinterpret_cast<uint4 *>(dst + l * 1024) = make_uint4(w[0], w[1], w[2], w[3]);
    }
    uint8_t o[16];
    for (int q = 0; q < 16; ++q) {
        int v = 0;
        if (valid && h == 0) {
            const int j = q & 7;
            const int bsp = (int)*reinterpret_cast<const int16_t *>(blk + 260 + 4 * j) +
                            (int)*reinterpret_cast<const int16_t *>(blk + 262 + 4 * j);
            v = q < 8 ? (bsp >> 7) : (bsp & 127);
        }
        o[q] = (uint8_t)(int8_t)v;
    }
    for (int q = 0; q < 16; ++q) dst[8 * 1024 + q] = o[q];
    if (lane < 32) d8_out[((long long)tile * nb + b) * 32 + lane] = valid ? *reinterpret_cast<const float *>(blk) : 0.0f;
}

// ------------------------------------------------------------------ GEMM
//
// Workgroup: RG x TG waves; wave (rg, tg) owns 16 rows x 32 tokens and keeps
// the nine f32 chains of its 8 (row, token) pairs per lane in registers.
// Per block the workgroup stages its A tiles (RG x 9 KiB), B tiles
// (TG x 9 KiB), d/dmin and d8 in LDS (double-buffered: the next block's
// global loads are in flight while the current block is computed).
template <int RG, int TG>
struct GemmLDS {
    uint8_t a[2][RG][TILE_BYTES];
    uint8_t b[2][TG][TILE_BYTES];
    float2 dm[2][RG * 16];
    float d8[2][TG * 32];
};

template <int RG, int TG>
__global__ void __launch_bounds__(64 * RG * TG) k_kq_gemm(GemmArgs g) {
    constexpr int NT = 64 * RG * TG;
    extern __shared__ __align__(16) uint8_t smem[];
    GemmLDS<RG, TG> &S = *reinterpret_cast<GemmLDS<RG, TG> *>(smem);
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int rg = wid % RG, tg = wid / RG;
    const int nb = g.nb;
    const int m_sel = blockIdx.y;   // which matrix of the launch
    const MatGemm &M = g.mat[m_sel];
    const int row_tiles_wg = (M.rows + 16 * RG - 1) / (16 * RG);
    const int tok_tiles_wg = (g.n_tokens + 32 * TG - 1) / (32 * TG);
    // XCD-aware order: workgroups are dealt to the eight XCDs round robin;
    // consecutive workgroups of one XCD share a row tile, so each A tile is
    // fetched into that XCD's L2 once for all of its token tiles.
    const int nwg = row_tiles_wg * tok_tiles_wg;
    const int id = (int)blockIdx.x;
    if (id >= nwg) return;
    const int nfull = nwg & ~7;
    const int lin = id < nfull ? (id % 8) * (nfull / 8) + id / 8 : id;   // a bijection of [0, nwg)
    const int wrt = lin / tok_tiles_wg, wtt = lin - wrt * tok_tiles_wg;
    const int rtile0 = wrt * RG, ttile0 = wtt * TG;

    // staging: per block, RG A tiles + TG B tiles as 16-byte units, then dm/d8
    constexpr int UNITS = (RG + TG) * TILE_BYTES / 16;
    constexpr int PER = (UNITS + NT - 1) / NT;
    uint4 st[PER];
    float2 st_dm;
    float st_d8;
    const int n_rtiles = (M.rows + 15) / 16;
    const int n_ttiles = (g.n_tokens + 31) / 32;
    auto load_stage = [&](int b) {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int uidx = tid + i * NT;
            st[i] = make_uint4(0, 0, 0, 0);
            if (uidx < UNITS) {
                const int which = uidx / (TILE_BYTES / 16), off = uidx - which * (TILE_BYTES / 16);
                if (which < RG) {
                    const int rt = rtile0 + which;
                    if (rt < n_rtiles)
                        st[i] = reinterpret_cast<const uint4 *>(M.a + ((long long)rt * nb + b) * TILE_BYTES)[off];
                } else {
                    const int tt = ttile0 + which - RG;
                    if (tt < n_ttiles)
                        st[i] = reinterpret_cast<const uint4 *>(g.b + ((long long)tt * nb + b) * TILE_BYTES)[off];
                }
            }
        }
        st_dm = make_float2(0.0f, 0.0f);
        if (tid < RG * 16) {
            const int r = rtile0 * 16 + tid;
            if (r < M.rows) st_dm = M.dm[(long long)r * nb + b];
        }
        st_d8 = 0.0f;
        if (tid < TG * 32) {
            const int tt = ttile0 + tid / 32;
            if (tt < n_ttiles) st_d8 = g.d8[((long long)tt * nb + b) * 32 + (tid & 31)];
        }
    };
    auto store_stage = [&](int buf) {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int uidx = tid + i * NT;
            if (uidx < UNITS) {
                const int which = uidx / (TILE_BYTES / 16), off = uidx - which * (TILE_BYTES / 16);
                uint4 *dst = which < RG ? reinterpret_cast<uint4 *>(S.a[buf][which])
                                        : reinterpret_cast<uint4 *>(S.b[buf][which - RG]);
                dst[off] = st[i];
            }
        }
        if (tid < RG * 16) S.dm[buf][tid] = st_dm;
        if (tid < TG * 32) S.d8[buf][tid] = st_d8;
    };

    // The lane's rows: register pair (r, r + 1), r = 4 (s / 2) + 2 (s % 2),
    // holds (hi, lo) of real row 4 (s / 2) + 2 (lane / 32) + s % 2 of the tile.
    const int hsel = lane >> 5;
    float chain[8][8];
    float msum[8];
#pragma unroll
    for (int s = 0; s < 8; ++s) {
        msum[s] = 0.0f;
#pragma unroll
        for (int l = 0; l < 8; ++l) chain[s][l] = 0.0f;
    }

    load_stage(0);
    store_stage(0);
    __syncthreads();
    for (int b = 0; b < nb; ++b) {
        const int buf = b & 1;
        if (b + 1 < nb) load_stage(b + 1);
        const uint8_t *A = S.a[buf][rg];
        const uint8_t *B = S.b[buf][tg];
        const float d8 = S.d8[buf][tg * 32 + (lane & 31)];
        float sc[8], ms[8];
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            const float2 dm = S.dm[buf][rg * 16 + 4 * (s >> 1) + 2 * hsel + (s & 1)];
            sc[s] = __fmul_rn(dm.x, d8);
            ms[s] = __fmul_rn(dm.y, d8);
        }
        // Two accumulators in flight: the MFMA of operand l + 1 is issued
        // before operand l is folded.  The empty asm statements (no
        // instructions) order "operands of l + 1 ready" after "fold of l - 1
        // done", so the compiler cannot hoist every MFMA of the block (nine
        // 16-register results) ahead of the folds.
        const v4i *Av = reinterpret_cast<const v4i *>(A) + lane;
        const v4i *Bv = reinterpret_cast<const v4i *>(B) + lane;
        const v16i zero = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
        v4i a0 = Av[0], b0 = Bv[0];
        asm volatile("" : "+v"(a0), "+v"(b0));
        v16i cn = __builtin_amdgcn_mfma_i32_32x32x32_i8(a0, b0, zero, 0, 0, 0);
#pragma unroll
        for (int l = 0; l < OPS; ++l) {
            const v16i c = cn;
            if (l + 1 < OPS) {
                v4i an = Av[(l + 1) * 64], bn = Bv[(l + 1) * 64];
                asm volatile("" : "+v"(an), "+v"(bn));
                cn = __builtin_amdgcn_mfma_i32_32x32x32_i8(an, bn, zero, 0, 0, 0);
            }
            if (l < 8) {
#pragma unroll
                for (int s = 0; s < 8; ++s) {
                    const int r = 4 * (s >> 1) + 2 * (s & 1);
                    const int v = (c[r] << 6) + c[r + 1];
                    chain[s][l] = __fadd_rn(chain[s][l], __fmul_rn(sc[s], (float)v));
                }
                asm volatile("" : "+v"(chain[0][l]), "+v"(chain[1][l]), "+v"(chain[2][l]), "+v"(chain[3][l]),
                             "+v"(chain[4][l]), "+v"(chain[5][l]), "+v"(chain[6][l]), "+v"(chain[7][l]));
            } else {
#pragma unroll
                for (int s = 0; s < 8; ++s) {
                    const int r = 4 * (s >> 1) + 2 * (s & 1);
                    const int v = (c[r] << 7) + c[r + 1];
                    msum[s] = __fsub_rn(msum[s], __fmul_rn(ms[s], (float)v));
                }
                asm volatile("" : "+v"(msum[0]), "+v"(msum[1]), "+v"(msum[2]), "+v"(msum[3]), "+v"(msum[4]),
                             "+v"(msum[5]), "+v"(msum[6]), "+v"(msum[7]));
            }
        }
        if (b + 1 < nb) store_stage(buf ^ 1);
        __syncthreads();
    }

    const int t = (ttile0 + tg) * 32 + (lane & 31);
    if (t >= g.n_tokens) return;
#pragma unroll
    for (int s = 0; s < 8; ++s) {
        const int r = (rtile0 + rg) * 16 + 4 * (s >> 1) + 2 * hsel + (s & 1);
        if (r >= M.rows) continue;
        float v = msum[s];
#pragma unroll
        for (int l = 0; l < 8; ++l) v = __fadd_rn(v, chain[s][l]);
        M.y[(long long)t * M.ldy + r] = v;
    }
}

// ---------------------------------------------------------------- launchers

static inline int cdiv(long long a, long long b) { return (int)((a + b - 1) / b); }

size_t gemm_a_bytes(int rows, int nb) { return (size_t)cdiv(rows, 16) * nb * TILE_BYTES; }
size_t gemm_dm_bytes(int rows, int nb) { return (size_t)cdiv(rows, 16) * 16 * nb * sizeof(float2); }
size_t gemm_b_bytes(int n_tokens, int nb) {
    return (size_t)cdiv(n_tokens, 32) * nb * (TILE_BYTES + 32 * sizeof(float));
}

hipError_t launch_prep_a(const MatView &m, uint8_t *a, float2 *dm, hipStream_t s) {
    const int grid = cdiv(m.rows, 16) * m.nb;
    if (m.type == T_Q4_K)
        hipLaunchKernelGGL(k_prep_a<T_Q4_K>, dim3(grid), dim3(64), 0, s, m, a, dm);
    else if (m.type == T_Q5_K)
        hipLaunchKernelGGL(k_prep_a<T_Q5_K>, dim3(grid), dim3(64), 0, s, m, a, dm);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_prep_b(const uint8_t *q8, int n_tokens, int nb, uint8_t *b, float *d8, hipStream_t s) {
    hipLaunchKernelGGL(k_prep_b, dim3(cdiv(n_tokens, 32) * nb), dim3(64), 0, s, q8, n_tokens, nb, b, d8);
    return hipGetLastError();
}

template <int RG, int TG>
static hipError_t gemm_shape(const GemmArgs &g, hipStream_t s) {
    const int lds = (int)sizeof(GemmLDS<RG, TG>);
    if (lds > 64 * 1024) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(k_kq_gemm<RG, TG>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, lds);
        if (e != hipSuccess) return e;
    }
    int rows = 0;
    for (int i = 0; i < g.n_mat; ++i) rows = g.mat[i].rows > rows ? g.mat[i].rows : rows;
    const int grid = cdiv(rows, 16 * RG) * cdiv(g.n_tokens, 32 * TG);
    hipLaunchKernelGGL((k_kq_gemm<RG, TG>), dim3(grid, g.n_mat), dim3(64 * RG * TG), lds, s, g);
    return hipGetLastError();
}

hipError_t launch_kq_gemm(const GemmArgs &g, hipStream_t s) {
    if (g.n_mat < 1 || g.n_mat > GEMM_MAX_MATS || g.n_tokens < 1 || g.nb < 1) return hipErrorInvalidValue;
    switch (g.shape) {
    case 0: return gemm_shape<2, 4>(g, s);
    case 1: return gemm_shape<2, 2>(g, s);
    case 2: return gemm_shape<4, 2>(g, s);
    default: return gemm_shape<1, 4>(g, s);
    }
}

}  // namespace lbh
