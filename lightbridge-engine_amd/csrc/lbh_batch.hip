// lbh_batch.hip — batched decode of a batch of tokens through the MoE layer.
//
// Per token the result is bit-identical to moe_routed_by_id_into
// (crates/bridge-kernels-reference/src/moe.rs:64-147), which the reference
// runs one token at a time (crates/bridge-runtime/src/hy3_scalar.rs:504-650).
// Here the batch's (token, routed expert) pairs are sorted by expert, so each
// selected expert's weights stream from HBM once per chunk of its tokens and
// are decoded once into registers for all of them:
//
//   k_mb_prep     counting sort of the pairs by expert (ascending token order
//                 inside an expert) into a chunk table; Q8_K of every token;
//   k_mb_gate_up  per (chunk, row tile): the chunk's Q8_K activations staged
//                 in LDS, gate and up rows decoded once, integer dots against
//                 every staged token, per-(row, token) folds in the
//                 reference's block order, SwiGLU -> h;
//   k_mb_quant_h  Q8_K of every h row (the down projections' inputs,
//                 gemv.rs:161-163);
//   k_mb_down     per (chunk, row tile): the down rows against every staged h;
//   k_mb_combine  per token and output row, in the reference's order:
//                 y = ((0 + c_0 d_0) + c_1 d_1) + ... + 1.0 * d_shared.
//
// The shared expert is one more "expert" that every token selects.
//
// Several workgroups read the same expert rows (one per chunk of its tokens),
// so the weight loads keep the default cache policy here.
#define LBH_WEIGHT_CPOL 0
#include "lbh_internal.h"
#include "lbh_math.h"
#include "lbh_router.h"
#include "lbh_rows.h"

namespace lbh {

constexpr int MB_THREADS = 256;
constexpr int MB_WAVES = MB_THREADS / 64;

// A staged Q8_K block in LDS: d at 0, qs at 16, bsums at 272 (16-byte aligned
// quants so a lane's slice is a run of 16-byte reads).
constexpr int Q8L = 304;

// Matrix-core operand copy of Q8_K rows, written beside the GGML bytes by the
// quantize kernels: block k's 256 quants XOR 0x80 (as unsigned bytes, q + 128)
// at q + 256 k, its scale at d[k].
struct MxRows {
    uint8_t *q;
    float *d;
};

__host__ __device__ constexpr int al16(int v) { return (v + 15) & ~15; }

// ------------------------------------------------------------ activations

template <int G>
__device__ __forceinline__ void load_act_lds(const uint8_t *blk, int p, ActIQ<G> &a) {
    a.d8 = __uint_as_float(*reinterpret_cast<const uint32_t *>(blk));
    const uint4 *q = reinterpret_cast<const uint4 *>(blk + 16 + 32 * G * p);
#pragma unroll
    for (int i = 0; i < 2 * G; ++i) {
        const uint4 v = q[i];
        a.q[4 * i] = v.x, a.q[4 * i + 1] = v.y, a.q[4 * i + 2] = v.z, a.q[4 * i + 3] = v.w;
    }
}

// K-quant consumers read residue-major qs (dword t of a 32-byte group holds
// bytes t, t + 8, t + 16, t + 24): the ActKQ layout, so no transpose here.
template <int G>
__device__ __forceinline__ void load_act_lds(const uint8_t *blk, int p, ActKQ<G> &a) {
    a.d8 = __uint_as_float(*reinterpret_cast<const uint32_t *>(blk));
    const uint4 *q = reinterpret_cast<const uint4 *>(blk + 16 + 64 * G * p);
#pragma unroll
    for (int j = 0; j < 2 * G; ++j) {
        const uint4 v0 = q[2 * j], v1 = q[2 * j + 1];
        a.t[j][0] = v0.x, a.t[j][1] = v0.y, a.t[j][2] = v0.z, a.t[j][3] = v0.w;
        a.t[j][4] = v1.x, a.t[j][5] = v1.y, a.t[j][6] = v1.z, a.t[j][7] = v1.w;
    }
    const uint32_t *bs = reinterpret_cast<const uint32_t *>(blk + 272 + 8 * G * p);
#pragma unroll
    for (int j = 0; j < 2 * G; ++j) {
        const uint32_t w = bs[j];
        a.bsp[j] = (int32_t)(int16_t)(w & 0xffff) + (int32_t)(int16_t)(w >> 16);
    }
}

// ------------------------------------------------------- decoded weights
//
// IQ2_S / IQ3_S: the slice's signed int8 weights and the integer scale of
// each 16-element half group (IQ2_S: 1 + 2 * nibble per half, q8_k.rs:355-362;
// IQ3_S: 2 * nibble + 1 for the whole group, q8_k.rs:389-427), so the block
// sum is sum over halves of scale * dot(16 weights, 16 quants): the same
// integer as the reference's (integer addition is exact in any order).
template <int LPU>
struct DecIQ {
    static constexpr int G = 8 / LPU;
    uint32_t w[8 * G];
    int32_t s[2 * G];
    float d;
};

// Q4_K / Q5_K: unsigned quants of each sub-block j in residue-major dwords,
// sub-block scale and min (scale_min, k_quants.rs:231-240), d and dmin.
template <int LPU>
struct DecKQ {
    static constexpr int G = 4 / LPU;
    uint32_t q[2 * G][8];
    int32_t sc[2 * G], mn[2 * G];
    float d, dmin;
};

template <int TY, int LPU>
using DecOf = typename std::conditional<Traits<TY>::KQ, DecKQ<LPU>, DecIQ<LPU>>::type;

template <int LPU>
__device__ __forceinline__ void decode(const WSlice<T_IQ2_S, LPU> &w, const void *gridp, int, DecIQ<LPU> &o) {
    constexpr int G = 8 / LPU;
    const GridRef<T_IQ2_S> grid(gridp);
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const Iq2sGroup q = iq2s_group(w, g);
        const uint32_t sc = byte_of(g < 4 ? w.sc : w.sc2, g & 3);
#pragma unroll
        for (int lg = 0; lg < 4; ++lg) {
            const uint2 code = grid.code_at(q.addr(lg));
            const uint32_t sel_lo = q.sel(2 * lg) | code.x;
            const uint32_t sel_hi = q.sel(2 * lg + 1) | code.y;
            o.w[8 * g + 2 * lg] = perm(IQ2S_NEG, IQ2S_POS, sel_lo);
            o.w[8 * g + 2 * lg + 1] = perm(IQ2S_NEG, IQ2S_POS, sel_hi);
        }
        o.s[2 * g] = (int32_t)(1 + 2 * (sc & 15u));
        o.s[2 * g + 1] = (int32_t)(1 + 2 * (sc >> 4));
    }
    o.d = f16_to_f32(w.d);
}

template <int LPU>
__device__ __forceinline__ void decode(const WSlice<T_IQ3_S, LPU> &w, const void *gridp, int, DecIQ<LPU> &o) {
    constexpr int G = 8 / LPU;
    const GridRef<T_IQ3_S> grid(gridp);
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const int32_t sc = (int32_t)(2 * ((w.sc >> (4 * g)) & 15u) + 1);
        uint32_t ad[8];
        iq3_group_addrs(w.qs[2 * g], w.qs[2 * g + 1], byte_of(g < 4 ? w.qh : w.qh2, g & 3), ad);
#pragma unroll
        for (int lg = 0; lg < 4; ++lg) {
            const uint2 sm = grid.sel(byte_of(w.sg[g], lg));
            o.w[8 * g + 2 * lg] = iq3_signed(grid.pair(ad[2 * lg]), sm.x);
            o.w[8 * g + 2 * lg + 1] = iq3_signed(grid.pair(ad[2 * lg + 1]), sm.y);
        }
        o.s[2 * g] = sc;
        o.s[2 * g + 1] = sc;
    }
    o.d = f16_to_f32(w.d);
}

template <int TY, int LPU>
__device__ __forceinline__ void decode(const WSliceKQ<TY, LPU> &w, const void *, int p, DecKQ<LPU> &o) {
    constexpr int G = 4 / LPU;
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const int gg = G * p + g;
        int32_t sc0, mn0, sc1, mn1;
        scale_min_of(w.hdr.y, w.hdr.z, w.hdr.w, 2 * gg, sc0, mn0);
        scale_min_of(w.hdr.y, w.hdr.z, w.hdr.w, 2 * gg + 1, sc1, mn1);
        o.sc[2 * g] = sc0, o.mn[2 * g] = mn0, o.sc[2 * g + 1] = sc1, o.mn[2 * g + 1] = mn1;
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            uint32_t lo = w.q[g][t] & 0x0f0f0f0fu;
            uint32_t hi = (w.q[g][t] >> 4) & 0x0f0f0f0fu;
            if constexpr (TY == T_Q5_K) {
                lo |= ((w.qh[t] >> (2 * gg)) & 0x01010101u) << 4;
                hi |= ((w.qh[t] >> (2 * gg + 1)) & 0x01010101u) << 4;
            }
            o.q[2 * g][t] = lo;
            o.q[2 * g + 1][t] = hi;
        }
    }
    o.d = f16_to_f32(w.hdr.x & 0xffffu);
    o.dmin = f16_to_f32(w.hdr.x >> 16);
}

// Integer stage of one token against a decoded slice: IQ -> v[0] = the
// slice's share of the block sum; K-quants -> v[0..7] lane sums, v[8] the
// minimum sum (q8_k.rs:288-312, :337-364, :380-428).
template <int LPU>
__device__ __forceinline__ void token_ints(const DecIQ<LPU> &o, const ActIQ<8 / LPU> &a, int32_t *v) {
    constexpr int G = 8 / LPU;
    int32_t bs = 0;
#pragma unroll
    for (int g = 0; g < G; ++g) {
        int32_t p0 = 0, p1 = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) p0 = dot4(o.w[8 * g + k], a.q[8 * g + k], p0);
#pragma unroll
        for (int k = 4; k < 8; ++k) p1 = dot4(o.w[8 * g + k], a.q[8 * g + k], p1);
        bs = mul24(o.s[2 * g], p0) + bs;
        bs = mul24(o.s[2 * g + 1], p1) + bs;
    }
    v[0] = bs;
}

template <int LPU>
__device__ __forceinline__ void token_ints(const DecKQ<LPU> &o, const ActKQ<4 / LPU> &a, int32_t *v) {
    constexpr int G = 4 / LPU;
    int32_t ms = 0;
#pragma unroll
    for (int t = 0; t < 8; ++t) v[t] = 0;
#pragma unroll
    for (int j = 0; j < 2 * G; ++j) {
#pragma unroll
        for (int t = 0; t < 8; ++t) v[t] = mul24(o.sc[j], dot4(o.q[j][t], a.t[j][t], 0)) + v[t];
        ms = mul24(o.mn[j], a.bsp[j]) + ms;
    }
    v[8] = ms;
}

// ------------------------------------------------------------ one wave step
//
// The decoded rows of NM matrices (rpw rows, one per slot) against n staged
// tokens.  Tokens go in fold batches of FB: the integer stage of every token
// of a batch writes its per-block f32 terms to the wave's LDS table, then the
// wave's lanes fold the (matrix, token, row, chain) chains in parallel, each
// chain in the reference's sequential block order (lbh_rows.h fold_terms),
// and lanes (token, row) combine the chains (K-quants: sum = minimum chain,
// then += lane chains 0..7, q8_k.rs:314-326; IQ2_S: x 0.125, q8_k.rs:369) and
// call out(token, slot, values[NM]).  Every lane of the wave must call it.
template <int TY, int LPU, int NM, int FB, class Out>
__device__ __forceinline__ void batch_step(const DecOf<TY, LPU> (&dec)[NM], bool on, const LaneMap<LPU> &L, int nb,
                                           const uint8_t *s_act, int n, float *terms, float *chains, Out out) {
    using Tr = Traits<TY>;
    constexpr int NCH = Tr::NCH;
    const int tstr = nb + 1;
    const int lane = threadIdx.x & 63;
    const int rpw = L.rpw;
    for (int i0 = 0; i0 < n; i0 += FB) {
        const int nf = n - i0 < FB ? n - i0 : FB;
        for (int f = 0; f < nf; ++f) {
            ActOf<TY, LPU> act;
            load_act_lds(s_act + ((i0 + f) * nb + L.b) * Q8L, L.part, act);
#pragma unroll
            for (int m = 0; m < NM; ++m) {
                int32_t v[NCH];
                token_ints(dec[m], act, v);
#pragma unroll
                for (int c = 0; c < NCH; ++c) v[c] = unit_reduce<LPU>(v[c]);
                if (on && L.part == 0) {
                    float *t = terms + (((m * FB + f) * rpw + L.slot) * NCH) * tstr + L.b;
                    if constexpr (Tr::KQ) {
                        const float s = __fmul_rn(dec[m].d, act.d8);
                        const float ms = __fmul_rn(dec[m].dmin, act.d8);
#pragma unroll
                        for (int c = 0; c < 8; ++c) t[c * tstr] = __fmul_rn(s, (float)v[c]);
                        t[8 * tstr] = __fmul_rn(ms, (float)v[8]);
                    } else {
                        t[0] = __fmul_rn(__fmul_rn(dec[m].d, act.d8), (float)v[0]);
                    }
                }
            }
        }
        wave_sync();
        const int tasks = NM * nf * rpw * NCH;
        for (int k = lane; k < tasks; k += 64) {
            const int c = k % NCH;
            int r = k / NCH;
            const int slot = r % rpw;
            r /= rpw;
            const int f = r % nf, m = r / nf;
            const int idx = ((m * FB + f) * rpw + slot) * NCH + c;
            chains[idx] = fold_terms(terms + idx * tstr, nb, Tr::KQ && c == 8);
        }
        wave_sync();
        for (int k = lane; k < nf * rpw; k += 64) {
            const int f = k % nf, slot = k / nf;
            float res[NM];
#pragma unroll
            for (int m = 0; m < NM; ++m) {
                const float *ch = chains + ((m * FB + f) * rpw + slot) * NCH;
                float s;
                if constexpr (Tr::KQ) {
                    s = ch[8];
#pragma unroll
                    for (int l = 0; l < 8; ++l) s = __fadd_rn(s, ch[l]);
                } else {
                    s = ch[0];
                    if (TY == T_IQ2_S) s = __fmul_rn(0.125f, s);
                }
                res[m] = s;
            }
            out(i0 + f, slot, res);
        }
        wave_sync();
    }
}

// Fold batch per type: IQ chains are short work per token, so their folds
// wait for up to eight tokens; K-quants carry nine chains per row and fold
// after every token (a small term table).
template <int TY>
constexpr int fold_batch() {
    return Traits<TY>::KQ ? 1 : 8;
}

// LDS floats of one wave's term table and chain results.
template <int TY, int NM>
__host__ __device__ constexpr int wave_fold_floats(int rpw, int nb) {
    return NM * fold_batch<TY>() * rpw * Traits<TY>::NCH * (nb + 2);
}

__host__ __device__ constexpr int rows_per_step(int lpu, int nb) { return (64 / lpu) / nb; }

// Rows [r0, r1) of NM matrices against the n tokens staged in s_act.  The
// wave's first weight loads are issued before `prologue` (codebook fill and
// activation staging, ended by a workgroup barrier), so their latency
// overlaps it; then a software pipeline keeps the next step's loads in flight.
// FUSED (chunks of one token): each row is the matvec's row dot (lbh_rows.h
// row_dot, the same terms and block-order fold as batch_step) on the staged
// token, with no decoded copy of the slice held for reuse, which a single
// token never needs; the wave's fold table holds its FoldLDS.
template <int TY, int LPU, int NM, bool FUSED = false, class Prologue, class Out>
__device__ __forceinline__ void batch_rows(const MatView (&mv)[NM], int r0, int r1, const uint8_t *s_act, int n,
                                           const void *grid, float *fold_lds, Prologue prologue, Out out) {
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    const int nb = mv[0].nb;
    const LaneMap<LPU> L(lane, nb);
    using W = WOf<TY, LPU>;
    Planes P[NM];
    uint32_t po[NM];
#pragma unroll
    for (int m = 0; m < NM; ++m) {
        P[m] = make_planes(mv[m].planes, mv[m].units, mv[m].bytes);
        po[m] = part_offset<TY, LPU>(P[m], L.part);
    }
    const int rpw = L.rpw;
    float *terms = fold_lds + wid * wave_fold_floats<TY, NM>(rpw, nb);
    float *chains = terms + NM * fold_batch<TY>() * rpw * Traits<TY>::NCH * (nb + 1);
    const int steps = (r1 - r0 + rpw - 1) / rpw;
    // Lanes past the tile (or past the wave's last whole row) load and decode
    // the tile's last row: every register is defined, and `on` gates the writes.
    // The loads are unconditional (a step past the end reloads the tile's last
    // row, never used), so the wait before a step's use leaves the next step's
    // loads in flight.
    auto issue = [&](int j, W (&w)[NM]) {
        int r = r0 + j * rpw + L.slot;
        r = L.lane_on && r < r1 ? r : r1 - 1;
#pragma unroll
        for (int m = 0; m < NM; ++m) load_slice(P[m], (uint32_t)(r * nb + L.b), po[m], L.part, w[m]);
    };
    ActOf<TY, LPU> act1;   // FUSED: the staged token
    auto process = [&](int j, const W (&w)[NM]) {
        const int r = r0 + j * rpw + L.slot;
        const bool on = L.lane_on && r < r1;
        if constexpr (FUSED) {
            FoldLDS<TY> &fl = *reinterpret_cast<FoldLDS<TY> *>(terms);
            float res[NM];
#pragma unroll
            for (int m = 0; m < NM; ++m) res[m] = row_dot<TY, LPU>(w[m], act1, on, L, grid, fl, nullptr, 0);
            if (on && L.leader()) out(0, r, res);
            return;
        }
        DecOf<TY, LPU> dec[NM];
#pragma unroll
        for (int m = 0; m < NM; ++m) decode(w[m], grid, L.part, dec[m]);
        batch_step<TY, LPU, NM, fold_batch<TY>()>(dec, on, L, nb, s_act, n, terms, chains,
                                                  [&](int i, int slot, const float *res) {
                                                      const int rr = r0 + j * rpw + slot;
                                                      if (rr < r1) out(i, rr, res);
                                                  });
    };
    int j = wid;
    W wa[NM], wb[NM];
    issue(j, wa);
    prologue();
    if constexpr (FUSED) load_act_lds(s_act + L.b * Q8L, L.part, act1);
    while (j < steps) {
        issue(j + MB_WAVES, wb);
        process(j, wa);
        j += MB_WAVES;
        if (j >= steps) break;
        issue(j + MB_WAVES, wa);
        process(j, wb);
        j += MB_WAVES;
    }
}

// Copies n x nb GGML Q8_K blocks (block (i, b) at src_of(i) + 292 * b) into
// the padded LDS layout, all threads of the workgroup.
template <class Src>
__device__ __forceinline__ void stage_q8(uint8_t *s_act, int n, int nb, Src src_of) {
    const int total = n * nb * 73;
    for (int k = threadIdx.x; k < total; k += blockDim.x) {
        const int blk = k / 73, w = k - blk * 73;
        const int i = blk / nb, b = blk - i * nb;
        const uint32_t v = *reinterpret_cast<const uint32_t *>(src_of(i) + b * 292 + 4 * w);
        const int off = w == 0 ? 0 : w <= 64 ? 16 + 4 * (w - 1) : 272 + 4 * (w - 65);
        *reinterpret_cast<uint32_t *>(s_act + blk * Q8L + off) = v;
    }
}

// LDS of a stream workgroup: the codebook (a static array, static_grid), then,
// dynamic, [staged activations][fold tables].
template <int TY, int NM>
__host__ __device__ constexpr int stream_lds(int tc, int nb, int lpu) {
    return al16(tc * nb * Q8L) + al16(GridLDS<TY>::BYTES) + MB_WAVES * 4 * wave_fold_floats<TY, NM>(rows_per_step(lpu, nb), nb);
}

template <int TY>
constexpr int mb_lpu() {
    return 2;
}

// ------------------------------------------------------------------ kernels

// Sort of the batch's pairs by expert (workgroup 0) and Q8_K of every token
// (the other workgroups, four blocks per wave).
__device__ __forceinline__ void quantize_rows_out(const float *x, long long nblocks, long long first, uint8_t *plain,
                                                  uint8_t *rm, uint8_t *lds_wave, MxRows mx = MxRows{}) {
    // Blocks [first, first + 4) (x points at block `first`) into the wave's
    // LDS, then out to global memory: the GGML bytes, (rm != NULL) the copy
    // with residue-major qs, and (mx.q != NULL) the matrix-core operand copy.
    const int lane = threadIdx.x & 63;
    const long long cnt = nblocks - first < 4 ? nblocks - first : 4;
    quantize_blocks_wave(x, lds_wave, 0, cnt);
    wave_sync();
    if (mx.q) {
        for (int k = lane; k < (int)cnt * 64; k += 64) {
            const int blk = k >> 6, w = k & 63;
            const uint32_t v = *reinterpret_cast<const uint32_t *>(lds_wave + blk * 292 + 4 + 4 * w);
            reinterpret_cast<uint32_t *>(mx.q)[(first + blk) * 64 + w] = v ^ 0x80808080u;
        }
        if (lane < cnt) mx.d[first + lane] = *reinterpret_cast<const float *>(lds_wave + lane * 292);
    }
    const int dw = (int)cnt * 73;
    for (int k = lane; k < dw; k += 64) {
        const int blk = k / 73, w = k - blk * 73;
        const uint8_t *sb = lds_wave + blk * 292;
        const uint32_t v = *reinterpret_cast<const uint32_t *>(sb + 4 * w);
        if (plain) *reinterpret_cast<uint32_t *>(plain + (first + blk) * 292 + 4 * w) = v;
        if (rm) {
            uint32_t r = v;
            if (w >= 1 && w <= 64) {
                const int q = w - 1, g = q >> 3, t = q & 7;
                const uint8_t *src = sb + 4 + 32 * g + t;
                r = (uint32_t)src[0] | ((uint32_t)src[8] << 8) | ((uint32_t)src[16] << 16) | ((uint32_t)src[24] << 24);
            }
            *reinterpret_cast<uint32_t *>(rm + (first + blk) * 292 + 4 * w) = r;
        }
    }
    wave_sync();
}

__global__ void __launch_bounds__(MB_THREADS) k_mb_prep(BatchArgs a) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int tid = threadIdx.x;
    if (blockIdx.x > 0) {
        const int nb = a.hidden / 256;
        const long long nblocks = (long long)a.n_tokens * nb;
        const long long first = ((long long)(blockIdx.x - 1) * MB_WAVES + (tid >> 6)) * 4;
        const bool rm = a.has_shared && !a.shared_gemm && (a.shared.gate.type == T_Q4_K || a.shared.gate.type == T_Q5_K);
        if (first < nblocks)
            quantize_rows_out(a.x + first * 256, nblocks, first, a.q8x, rm ? a.q8x_rm : nullptr,
                              smem + (tid >> 6) * 4 * 292, MxRows{a.mx ? a.xq_mx : nullptr, a.xd_mx});
        return;
    }
    const int NE = a.n_experts, T = a.n_tokens, K = a.top_k, TC = a.tc;
    const int W = (T + 31) / 32;
    uint32_t *bm = reinterpret_cast<uint32_t *>(smem);              // [NE][W] token bitmaps
    int32_t *cnt = reinterpret_cast<int32_t *>(bm + NE * W);       // [NE]
    int32_t *off = cnt + NE;                                       // [NE] first sorted pair
    int32_t *coff = off + NE;                                      // [NE] first chunk
    int32_t *part = coff + NE;                                     // [2][MB_THREADS] scan partials
    int32_t *flags = part + 2 * MB_THREADS;
    for (int i = tid; i < NE * W; i += MB_THREADS) bm[i] = 0;
    if (tid == 0) flags[0] = 0;
    __syncthreads();
    for (int p = tid; p < T * K; p += MB_THREADS) {
        const int t = p / K;
        const uint32_t e = a.ids[p];
        if (e >= (uint32_t)NE) {
            atomicOr(&flags[0], 1);
            continue;
        }
        const uint32_t bit = 1u << (t & 31);
        const uint32_t old = atomicOr(&bm[e * W + (t >> 5)], bit);
        if (old & bit) atomicOr(&flags[0], 2);
    }
    __syncthreads();
    // Per-expert counts and chunk counts; each thread owns a run of experts.
    const int per = (NE + MB_THREADS - 1) / MB_THREADS;
    const int e0 = tid * per, e1 = e0 + per < NE ? e0 + per : NE;
    int sc = 0, sk = 0;
    for (int e = e0; e < e1; ++e) {
        int c = 0;
        for (int w = 0; w < W; ++w) c += __popc(bm[e * W + w]);
        cnt[e] = c;
        sc += c;
        sk += (c + TC - 1) / TC;
    }
    part[tid] = sc;
    part[MB_THREADS + tid] = sk;
    __syncthreads();
    // Inclusive scan of the partials (Hillis-Steele), then exclusive offsets.
    for (int d = 1; d < MB_THREADS; d <<= 1) {
        const int v0 = tid >= d ? part[tid - d] : 0;
        const int v1 = tid >= d ? part[MB_THREADS + tid - d] : 0;
        __syncthreads();
        part[tid] += v0;
        part[MB_THREADS + tid] += v1;
        __syncthreads();
    }
    {
        int o = part[tid] - sc, ko = part[MB_THREADS + tid] - sk;
        for (int e = e0; e < e1; ++e) {
            off[e] = o;
            coff[e] = ko;
            o += cnt[e];
            ko += (cnt[e] + TC - 1) / TC;
        }
    }
    __syncthreads();
    const bool bad = flags[0] != 0;
    if (!bad) {
        for (int p = tid; p < T * K; p += MB_THREADS) {
            const int t = p / K;
            const uint32_t e = a.ids[p];
            int rank = __popc(bm[e * W + (t >> 5)] & ((1u << (t & 31)) - 1u));
            for (int w = 0; w < (t >> 5); ++w) rank += __popc(bm[e * W + w]);
            const int pos = off[e] + rank;
            a.pair_token[pos] = t;
            a.pair_of[p] = pos;
        }
        for (int e = e0; e < e1; ++e) {
            const int c = cnt[e];
            for (int j = 0; j * TC < c; ++j) {
                const int ch = coff[e] + j;
                a.chunk_expert[ch] = e;
                a.chunk_p0[ch] = off[e] + j * TC;
                a.chunk_n[ch] = c - j * TC < TC ? c - j * TC : TC;
            }
        }
    }
    if (tid == 0) {
        a.plan[0] = bad ? 0 : part[2 * MB_THREADS - 1];
        a.plan[1] = flags[0];
    }
}

// A chunk of n tokens of a TY stream belongs to the matrix-core kernels.
template <int TY>
__device__ __forceinline__ bool mx_takes(const BatchArgs &a, int n) {
    return (TY == T_IQ2_S || TY == T_IQ3_S) && a.mx && n >= a.mx_min;
}

// Tokens a VALU stream of type ty stages at most: the chunks the matrix cores
// leave to it (IQ types with mx on), else whole chunks.
__host__ __device__ inline int valu_cap(const BatchArgs &a, int ty) {
    return a.mx && (ty == T_IQ2_S || ty == T_IQ3_S) ? a.vc : a.tc;
}

// Gate/up, SwiGLU (activation.rs:170-178) -> h, one launch per stream:
// SHARED: workgroup (token chunk, row tile) of the shared expert; else
// workgroup (routed chunk, row tile), idle past the sort's chunk count.
// PART (routed IQ streams beside the matrix cores): 0 every VALU chunk, 1
// the chunks of one token (the FUSED rows of batch_rows: 116 instead of 170
// VGPRs, four waves per SIMD instead of two), 2 the other VALU chunks.
template <int TY, bool SHARED, int PART = 0>
__global__ void __launch_bounds__(MB_THREADS) k_mb_gate_up(BatchArgs a) {
    extern __shared__ __align__(16) uint8_t smem[];
    if (a.plan[1]) return;
    const int nb = a.hidden / 256;
    constexpr int LPU = mb_lpu<TY>();
    uint8_t *s_act = smem;
    uint8_t *grid = static_grid<TY>();
    float *fold = reinterpret_cast<float *>(smem + al16(valu_cap(a, TY) * nb * Q8L));
    if constexpr (SHARED) {
        const int tiles = (a.ffn_s + a.rt_gu_s - 1) / a.rt_gu_s;
        const int c = blockIdx.x / tiles, tile = blockIdx.x - c * tiles;
        const int t0 = c * a.tc;
        const int n = a.n_tokens - t0 < a.tc ? a.n_tokens - t0 : a.tc;
        if (mx_takes<TY>(a, n)) return;
        const int r0 = tile * a.rt_gu_s, r1 = r0 + a.rt_gu_s < a.ffn_s ? r0 + a.rt_gu_s : a.ffn_s;
        const uint8_t *src = Traits<TY>::KQ ? a.q8x_rm : a.q8x;
        const MatView mv[2] = {a.shared.gate, a.shared.up};
        batch_rows<TY, LPU, 2>(
            mv, r0, r1, s_act, n, grid, fold,
            [&]() {
                fill_grid<TY>(grid);
                stage_q8(s_act, n, nb, [&](int i) { return src + (long long)(t0 + i) * nb * 292; });
                __syncthreads();
            },
            [&](int i, int r, const float *res) {
                const long long o = (long long)(t0 + i) * a.ffn_s + r;
                a.g_s[o] = res[0];
                a.u_s[o] = res[1];
            });
    } else {
        const int tiles = (a.ffn_r + a.rt_gu_r - 1) / a.rt_gu_r;
        const int c = blockIdx.x / tiles, tile = blockIdx.x - c * tiles;
        if (c >= a.plan[0]) return;
        const int e = a.chunk_expert[c], p0 = a.chunk_p0[c], n = a.chunk_n[c];
        if (mx_takes<TY>(a, n)) return;
        if ((PART == 1 && n != 1) || (PART == 2 && n == 1)) return;
        const int r0 = tile * a.rt_gu_r, r1 = r0 + a.rt_gu_r < a.ffn_r ? r0 + a.rt_gu_r : a.ffn_r;
        const MatView mv[2] = {a.experts[e].gate, a.experts[e].up};
        batch_rows<TY, LPU, 2, PART == 1>(
            mv, r0, r1, s_act, n, grid, fold,
            [&]() {
                fill_grid<TY>(grid);
                stage_q8(s_act, n, nb, [&](int i) { return a.q8x + (long long)a.pair_token[p0 + i] * nb * 292; });
                __syncthreads();
            },
            [&](int i, int r, const float *res) {
                const long long o = (long long)(p0 + i) * a.ffn_r + r;
                a.g_r[o] = res[0];
                a.u_r[o] = res[1];
            });
    }
}

// h = SwiGLU(gate, up) (activation.rs:170-178) and its Q8_K (quantize_row_q8_k_into
// of each down projection's input, gemv.rs:161-163) for every routed pair row
// [0, pairs), then the shared rows.  The gate/up streams leave gate and up
// apart, so no exp runs inside their weight loops (its table load would wait
// for every weight load in flight).  shared_mode 0: the shared copy is GGML
// bytes plus the matrix-core operand copy (IQ down); 1: residue-major qs only
// (VALU K-quant down); 2: GGML bytes (K-quant GEMM down).
__global__ void __launch_bounds__(MB_THREADS) k_mb_quant_h(BatchArgs a, int shared_mode) {
    __shared__ __align__(16) uint8_t lds[MB_WAVES * 4 * 292];
    __shared__ __align__(16) float hbuf[MB_WAVES][4 * 256];
    if (a.plan[1]) return;
    const int nbr = a.ffn_r / 256, nbs = a.ffn_s / 256;
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    const long long br = (long long)a.n_tokens * a.top_k * nbr;
    const long long brp = (br + 3) & ~3ll;   // chunks of four never straddle the two ranges
    const long long bs = a.has_shared ? (long long)a.n_tokens * nbs : 0;
    const long long chunk = ((long long)blockIdx.x * MB_WAVES + wid) * 4;
    uint8_t *lw = lds + wid * 4 * 292;
    // Lane (block first + lane / 16, elements 16 (lane % 16) ..) forms the
    // sixteen values it quantizes below.
    auto swiglu_blocks = [&](const float *g, const float *u, long long first, long long nblocks) {
        const long long blk = first + (lane >> 4);
        if (blk < nblocks) {
            const long long base = blk * 256 + 16 * (lane & 15);
            float *hb = &hbuf[wid][(lane >> 4) * 256 + 16 * (lane & 15)];
#pragma unroll
            for (int i = 0; i < 16; ++i) hb[i] = swiglu_ref(g[base + i], u[base + i]);
        }
        wave_sync();
    };
    if (chunk < br) {
        swiglu_blocks(a.g_r, a.u_r, chunk, br);
        quantize_rows_out(&hbuf[wid][0], br, chunk, a.q8h_r, nullptr, lw, MxRows{a.mx ? a.hq_mx_r : nullptr, a.hd_mx_r});
    } else if (chunk >= brp && chunk - brp < bs) {
        const long long f = chunk - brp;
        swiglu_blocks(a.g_s, a.u_s, f, bs);
        quantize_rows_out(&hbuf[wid][0], bs, f, shared_mode == 1 ? nullptr : a.q8h_s, shared_mode == 1 ? a.q8h_s : nullptr,
                          lw, MxRows{a.mx && shared_mode == 0 ? a.hq_mx_s : nullptr, a.hd_mx_s});
    }
}

// Down rows -> d, one launch per stream (as k_mb_gate_up; PART 1: every
// chunk has one token, the FUSED rows of batch_rows).
template <int TY, bool SHARED, int PART = 0>
__global__ void __launch_bounds__(MB_THREADS) k_mb_down(BatchArgs a) {
    extern __shared__ __align__(16) uint8_t smem[];
    if (a.plan[1]) return;
    constexpr int LPU = mb_lpu<TY>();
    uint8_t *s_act = smem;
    if constexpr (SHARED) {
        const int nb = a.ffn_s / 256;
        const int tiles = (a.hidden + a.rt_d_s - 1) / a.rt_d_s;
        const int c = blockIdx.x / tiles, tile = blockIdx.x - c * tiles;
        const int t0 = c * a.tc;
        const int n = a.n_tokens - t0 < a.tc ? a.n_tokens - t0 : a.tc;
        if (mx_takes<TY>(a, n)) return;
        const int r0 = tile * a.rt_d_s, r1 = r0 + a.rt_d_s < a.hidden ? r0 + a.rt_d_s : a.hidden;
        uint8_t *grid = static_grid<TY>();
        float *fold = reinterpret_cast<float *>(smem + al16(valu_cap(a, TY) * nb * Q8L));
        const MatView mv[1] = {a.shared.down};
        batch_rows<TY, LPU, 1>(
            mv, r0, r1, s_act, n, grid, fold,
            [&]() {
                fill_grid<TY>(grid);
                stage_q8(s_act, n, nb, [&](int i) { return a.q8h_s + (long long)(t0 + i) * nb * 292; });
                __syncthreads();
            },
            [&](int i, int r, const float *res) { a.d_s[(long long)(t0 + i) * a.hidden + r] = res[0]; });
    } else {
        const int nb = a.ffn_r / 256;
        const int tiles = (a.hidden + a.rt_d_r - 1) / a.rt_d_r;
        const int c = blockIdx.x / tiles, tile = blockIdx.x - c * tiles;
        if (c >= a.plan[0]) return;
        const int e = a.chunk_expert[c], p0 = a.chunk_p0[c], n = a.chunk_n[c];
        if (mx_takes<TY>(a, n)) return;
        const int r0 = tile * a.rt_d_r, r1 = r0 + a.rt_d_r < a.hidden ? r0 + a.rt_d_r : a.hidden;
        uint8_t *grid = static_grid<TY>();
        float *fold = reinterpret_cast<float *>(smem + al16(valu_cap(a, TY) * nb * Q8L));
        const MatView mv[1] = {a.experts[e].down};
        batch_rows<TY, LPU, 1, PART == 1>(
            mv, r0, r1, s_act, n, grid, fold,
            [&]() {
                fill_grid<TY>(grid);
                stage_q8(s_act, n, nb, [&](int i) { return a.q8h_r + (long long)(p0 + i) * nb * 292; });
                __syncthreads();
            },
            [&](int i, int r, const float *res) { a.d_r[(long long)(p0 + i) * a.hidden + r] = res[0]; });
    }
}

// ==================================================== IQ streams on the matrix cores
//
// The IQ2_S / IQ3_S gate/up and down streams as f16 matrix-core products
// (v_mfma_f32_16x16x32_f16), bit-identical to the dot4 streams above: per
// (row, token, block) the integer block sum is formed exactly and folded in
// the reference's order.
//
// Wave tile: 16 rows x the chunk's tokens (up to 16) per block.  Lane l holds
// row l % 16 of the A operand and token l % 16 of the B operand, both for the
// block's elements 64 (l / 16) + 8 m .. + 7 in instruction m (m = 0..7): A and
// B use the same (lane, slot) -> element map, so each instruction contracts 32
// elements of the block whatever its internal k order.  The lane's slice of
// its row is the four-lane part l / 16 of the unit (load_slice<TY, 4>).
//   A: one codebook entry (IQ2_S: one 8-element grid entry; IQ3_S: two
//      4-element entries) from LDS tables of f16 magnitudes, the eight sign
//      bits applied by XOR with an f16 sign-mask table entry, times the
//      entry's integer scale (IQ2_S 1 + 2 nibble per 16 elements, IQ3_S
//      2 nibble + 1 per 32): |A| <= 43 * 31 = 1333 (IQ2_S), 15 * 31 = 465
//      (IQ3_S), integers an f16 holds exactly.
//   B: the Q8_K quants (|B| <= 128) from the operand copy of q + 128 as
//      unsigned bytes: 0x6400 | (q + 128) is the f16 1024 + q + 128, and one
//      packed f16 subtraction of 1152 leaves q exactly.
// Every product is an integer below 2^18 and every partial sum of a chain of
// instructions stays below 2^24 (IQ2_S: chains of three instructions, 96
// elements, 96 * 1333 * 128 < 2^24; IQ3_S: the whole block, 256 * 465 * 128 <
// 2^24), so the f32 accumulation is exact in any order; each chain converted
// to int32 and summed gives the reference's integer block sum (q8_k.rs:337-364,
// :380-428, integer additions, exact in any order).  The fold is the one of
// lbh_rows.h: term = (d * d8) * (float)bsum, chain += term in block order,
// IQ2_S result = 0.125 * chain.

typedef _Float16 mx_h8 __attribute__((ext_vector_type(8)));
typedef _Float16 mx_h2 __attribute__((ext_vector_type(2)));
typedef float mx_f4 __attribute__((ext_vector_type(4)));
typedef uint32_t mx_u4 __attribute__((ext_vector_type(4)));

constexpr int MX_THREADS = 256;
constexpr int MX_WAVES = MX_THREADS / 64;


// LDS tables: the f16 magnitudes of every codebook entry (IQ2_S 1024 x 8, the
// entry of index q | h << 8 at byte 2 * iq2s_code_addr(q, h); IQ3_S 512 x 4),
// then for IQ3_S 256 sign masks of eight f16 (bit 15 of element i is bit i of
// the sign byte); built at compile time, copied to LDS per workgroup.
template <int TY>
struct MxTab {
    static constexpr int ENTRY = TY == T_IQ2_S ? 16 : 8;
    static constexpr int GRID = (TY == T_IQ2_S ? 1024 : 512) * ENTRY;
    static constexpr int SIGNS = TY == T_IQ3_S ? 256 * 16 : 0;
    static constexpr int BYTES = GRID + SIGNS;
};

// f16 bits of a non-negative integer below 2048 (exact).
constexpr uint32_t f16_bits_of(uint32_t v) {
    if (v == 0) return 0;
    int e = 0;
    while ((v >> (e + 1)) != 0) ++e;
    return ((uint32_t)(e + 15) << 10) | ((v << (10 - e)) & 0x3ffu);
}

constexpr uint64_t k_iq2s_vals[1024] = {LBH_IQ2S_GRID_VALUES};
constexpr uint32_t k_iq3s_vals[512] = {LBH_IQ3S_GRID_VALUES};

struct MxTables {
    uint32_t iq2[1024][4];
    uint32_t iq3[512][2];
    uint32_t sign[256][4];
};

constexpr uint32_t f16_pair_of(uint32_t lo, uint32_t hi) { return f16_bits_of(lo) | (f16_bits_of(hi) << 16); }

constexpr MxTables make_mx_tables() {
    MxTables t{};
    for (int i = 0; i < 1024; ++i)
        for (int k = 0; k < 4; ++k)
            t.iq2[iq2s_code_addr((uint32_t)i & 255u, (uint32_t)i >> 8) / 8][k] =
                f16_pair_of((uint32_t)(k_iq2s_vals[i] >> (16 * k)) & 0xffu,
                            (uint32_t)(k_iq2s_vals[i] >> (16 * k + 8)) & 0xffu);
    for (int i = 0; i < 512; ++i)
        for (int k = 0; k < 2; ++k)
            t.iq3[i][k] = f16_pair_of((k_iq3s_vals[i] >> (16 * k)) & 0xffu, (k_iq3s_vals[i] >> (16 * k + 8)) & 0xffu);
    for (uint32_t v = 0; v < 256; ++v)
        for (int k = 0; k < 4; ++k)
            t.sign[v][k] = (((v >> (2 * k)) & 1u) << 15) | (((v >> (2 * k + 1)) & 1u) << 31);
    return t;
}

static __constant__ MxTables c_mx_tab = make_mx_tables();

__device__ __forceinline__ uint32_t mx_bits(mx_h2 v) { return __builtin_bit_cast(uint32_t, v); }
__device__ __forceinline__ mx_h2 mx_pair(uint32_t v) { return __builtin_bit_cast(mx_h2, v); }

// Copies TY's tables into LDS (all threads; the caller synchronises).
template <int TY>
__device__ __forceinline__ void mx_fill(uint8_t *tab) {
    const uint4 *g = reinterpret_cast<const uint4 *>(TY == T_IQ2_S ? &c_mx_tab.iq2[0][0] : &c_mx_tab.iq3[0][0]);
    const uint4 *sg = reinterpret_cast<const uint4 *>(&c_mx_tab.sign[0][0]);
    uint4 *o = reinterpret_cast<uint4 *>(tab);
    for (int i = threadIdx.x; i < MxTab<TY>::GRID / 16; i += MX_THREADS) o[i] = g[i];
    if constexpr (MxTab<TY>::SIGNS > 0)
        for (int i = threadIdx.x; i < 256; i += MX_THREADS) o[MxTab<TY>::GRID / 16 + i] = sg[i];
}

// Eight f16 magnitudes with their signs applied, times the integer scale ls.
__device__ __forceinline__ mx_h8 mx_signed_scaled(uint4 mag, uint4 sgn, uint32_t ls) {
    const _Float16 f = (_Float16)(float)ls;
    const mx_h2 s = {f, f};
    const mx_u4 r = {mx_bits(mx_pair(mag.x ^ sgn.x) * s), mx_bits(mx_pair(mag.y ^ sgn.y) * s),
                     mx_bits(mx_pair(mag.z ^ sgn.z) * s), mx_bits(mx_pair(mag.w ^ sgn.w) * s)};
    return __builtin_bit_cast(mx_h8, r);
}

// A operand of instruction m: the lane's slice holds sub-blocks 2p, 2p + 1;
// m covers entry m % 4 of sub-block m / 4 (q8_k.rs:337-364 index, sign and
// scale layout, read from the device encoding as slice_sum in lbh_dev.h).
// The sign of weight 4t + i sits at bit t of byte i of the group's sign dword:
// (b0, b0, b1, b1) << (7 - t) puts those of weights 4t, 4t + 1 at bits 15 and
// 31, the sign bits of the f16 pair (b2, b2, b3, b3: weights 4t + 2, 4t + 3).
__device__ __forceinline__ mx_h8 mx_a(const WSlice<T_IQ2_S, 4> &w, const uint8_t *tab, int m) {
    const int g = m >> 2, lg = m & 3;
    const Iq2sGroup q = iq2s_group(w, g);
    const uint4 mag = *reinterpret_cast<const uint4 *>(tab + 2 * q.addr(lg));
    const uint32_t p01 = perm(q.s, q.s, 0x01010000u), p23 = perm(q.s, q.s, 0x03030202u);
    const int t0 = 2 * lg, t1 = 2 * lg + 1;
    const uint4 sgn = make_uint4((p01 << (7 - t0)) & 0x80008000u, (p23 << (7 - t0)) & 0x80008000u,
                                 (p01 << (7 - t1)) & 0x80008000u, (p23 << (7 - t1)) & 0x80008000u);
    const uint32_t ls = 1u + 2u * ((byte_of(w.sc, g) >> (4 * (lg >> 1))) & 15u);
    return mx_signed_scaled(mag, sgn, ls);
}

// IQ3_S (q8_k.rs:380-428): instruction m covers the two 4-element entries of
// eighth m % 4 of sub-block m / 4, the sign byte's low nibble on the first.
__device__ __forceinline__ mx_h8 mx_a(const WSlice<T_IQ3_S, 4> &w, const uint8_t *tab, int m) {
    const int g = m >> 2, lg = m & 3;
    const uint32_t h = byte_of(w.qh, g);
    const uint32_t qq = w.qs[2 * g + (lg >> 1)];
    const int sh = 16 * (lg & 1);
    const uint32_t i1 = ((qq >> sh) & 0xffu) | ((h << (8 - 2 * lg)) & 0x100u);
    const uint32_t i2 = ((qq >> (sh + 8)) & 0xffu) | ((h << (7 - 2 * lg)) & 0x100u);
    const uint2 m1 = reinterpret_cast<const uint2 *>(tab)[i1], m2 = reinterpret_cast<const uint2 *>(tab)[i2];
    const uint4 sgn = reinterpret_cast<const uint4 *>(tab + MxTab<T_IQ3_S>::GRID)[byte_of(w.sg[g], lg)];
    const uint32_t ls = 2u * ((w.sc >> (4 * g)) & 15u) + 1u;
    return mx_signed_scaled(make_uint4(m1.x, m1.y, m2.x, m2.y), sgn, ls);
}

// B operand: eight biased quants (two dwords) as f16.
__device__ __forceinline__ mx_h8 mx_b(uint32_t x0, uint32_t x1) {
    const mx_h2 off = {(_Float16)-1152.0f, (_Float16)-1152.0f};
    const mx_u4 r = {mx_bits(mx_pair(perm(0x64646464u, x0, 0x04010400u)) + off),
                     mx_bits(mx_pair(perm(0x64646464u, x0, 0x04030402u)) + off),
                     mx_bits(mx_pair(perm(0x64646464u, x1, 0x04010400u)) + off),
                     mx_bits(mx_pair(perm(0x64646464u, x1, 0x04030402u)) + off)};
    return __builtin_bit_cast(mx_h8, r);
}

template <int TY>
constexpr int mx_chain() {
    return TY == T_IQ2_S ? 3 : 8;   // instructions per exact f32 chain
}

// One wave step's inputs: the lane's slices of NM matrices and the block of
// its token from the operand copy.
template <int TY, int NM>
struct MxStep {
    WSlice<TY, 4> w[NM];
    uint4 bq[4];
    float d8;
};

// LDS of a matrix-core stream workgroup: the tables, then (split > 1) per
// tile the per-block f32 terms [matrix][block][token][row].
__host__ __device__ constexpr int mx_lds_bytes(int ty, int nm, int split, int nb) {
    return (ty == T_IQ2_S ? MxTab<T_IQ2_S>::BYTES : MxTab<T_IQ3_S>::BYTES) +
           (split > 1 ? (MX_WAVES / split) * nm * nb * 256 * 4 : 0);
}

// Rows [r0, r1) (r1 - r0 <= 16 * MX_WAVES / S) of NM matrices (K = 256 nb)
// against the chunk's tokens.  The workgroup holds MX_WAVES / S tiles of 16
// rows; the S waves of a tile take its blocks j, j + S, ...: together they
// read S consecutive blocks of each row (adjacent 16-byte pieces of the same
// lines) per step.  With S > 1 each wave writes the f32 term
// (d * d8) * (float)bsum of each (row, token, block) it computes to LDS;
// after a workgroup barrier one thread per (tile, token, row) folds its terms
// in block order (lbh_rows.h: chain = 0 + t_0 + t_1 + ...; IQ2_S result =
// 0.125 * chain) and calls out(token column, row, values).  With S = 1 the
// wave computes every block of its tile in order and each lane keeps the
// chains of its four (row, token) results in registers (no term table, so
// the workgroup's LDS is the tables alone).  Lane l's token column holds the
// operand row bq / bd.  The first step's loads are issued before `prologue`
// (table fill, ended by a workgroup barrier); then each step's loads are in
// flight while the one before is computed.
template <int TY, int NM, int S, class Prologue, class Out>
__device__ __forceinline__ void mx_tiles(const MatView (&mv)[NM], int r0, int r1, int nb, const uint8_t *bq,
                                         const float *bd, const uint8_t *tab, float *terms, Prologue prologue, Out out) {
    const int lane = threadIdx.x & 63;
    const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int c = lane & 15, q = lane >> 4;
    const int tl = wid / S, j = wid - tl * S;
    const int rt0 = r0 + 16 * tl;
    const int steps = rt0 < r1 && j < nb ? (nb - j + S - 1) / S : 0;
    Planes P[NM];
    uint32_t po[NM];
    int32_t order[NM];   // wave-uniform: a tile copy (MAT_TILE16) or the row-major matrix
#pragma unroll
    for (int t = 0; t < NM; ++t) {
        P[t] = make_planes(mv[t].planes, mv[t].units, mv[t].bytes);
        po[t] = part_offset<TY, 4>(P[t], q);
        order[t] = __builtin_amdgcn_readfirstlane(mv[t].order);
    }
    // Rows past r1 load the last row (every register defined; never output).
    int r = rt0 + c;
    r = r < r1 ? r : r1 - 1;
    // The loads are unconditional: a step past the wave's last one reloads a
    // block of the row (in bounds, never used), so the compiler's wait before
    // a step's use counts exactly the younger step's loads.
    auto issue = [&](int s, MxStep<TY, NM> &st) {
        int b = j + S * (s < steps ? s : steps - 1);
        b = b < 0 ? 0 : b < nb ? b : nb - 1;
#pragma unroll
        for (int t = 0; t < NM; ++t) load_slice(P[t], unit_index(order[t], r, b, nb), po[t], q, st.w[t]);
        const uint4 *src = reinterpret_cast<const uint4 *>(bq + b * 256 + 64 * q);
#pragma unroll
        for (int k = 0; k < 4; ++k) st.bq[k] = src[k];
        st.d8 = bd[b];
    };
    float *tt = S > 1 ? terms + tl * NM * nb * 256 : terms;   // S == 1: no term table
    float chain[NM][4];   // S == 1: result i of the lane is (row 4q + i, token c)
#pragma unroll
    for (int t = 0; t < NM; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) chain[t][i] = 0.0f;
    auto process = [&](int s, const MxStep<TY, NM> &st) {
        constexpr int CH = mx_chain<TY>();
        const int b = j + S * s;
        int32_t bs[NM][4];
        mx_f4 acc[NM];
#pragma unroll
        for (int t = 0; t < NM; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i) bs[t][i] = 0;
#pragma unroll
        for (int m = 0; m < 8; ++m) {
            const uint4 v = st.bq[m >> 1];
            const mx_h8 bo = (m & 1) ? mx_b(v.z, v.w) : mx_b(v.x, v.y);
#pragma unroll
            for (int t = 0; t < NM; ++t) {
                const mx_h8 ao = mx_a(st.w[t], tab, m);
                const mx_f4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
                acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ao, bo, m % CH == 0 ? zero : acc[t], 0, 0, 0);
                if (m % CH == CH - 1 || m == 7) {
#pragma unroll
                    for (int i = 0; i < 4; ++i) bs[t][i] += (int32_t)acc[t][i];
                }
            }
        }
        // Result i of the lane is (row 4q + i, token c); row 4q + i's d is in lane 4q + i.
#pragma unroll
        for (int t = 0; t < NM; ++t) {
            const float da = f16_to_f32(st.w[t].d);
            float *o = tt + ((t * nb + b) * 16 + c) * 16 + 4 * q;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float dr = __shfl(da, 4 * q + i, 64);
                const float term = __fmul_rn(__fmul_rn(dr, st.d8), (float)bs[t][i]);
                if constexpr (S == 1)
                    chain[t][i] = __fadd_rn(chain[t][i], term);   // blocks in order
                else
                    o[i] = term;
            }
        }
    };
    MxStep<TY, NM> sa, sb;
    issue(0, sa);
    prologue();
    for (int s = 0; s < steps; s += 2) {
        issue(s + 1, sb);
        process(s, sa);
        if (s + 1 >= steps) break;
        issue(s + 2, sa);
        process(s + 1, sb);
    }
    if constexpr (S == 1) {
        if (rt0 >= r1) return;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float res[NM];
#pragma unroll
            for (int t = 0; t < NM; ++t) res[t] = TY == T_IQ2_S ? __fmul_rn(0.125f, chain[t][i]) : chain[t][i];  // q8_k.rs:369
            out(c, rt0 + 4 * q + i, res);
        }
        return;
    }
    __syncthreads();
    for (int p = threadIdx.x; p < (MX_WAVES / S) * 256; p += MX_THREADS) {
        const int ptl = p >> 8, cc = (p >> 4) & 15, row = p & 15;
        const float *src = terms + ptl * NM * nb * 256 + cc * 16 + row;
        float res[NM];
#pragma unroll
        for (int t = 0; t < NM; ++t) {
            float ch = 0.0f;
            for (int b = 0; b < nb; ++b) ch = __fadd_rn(ch, src[(t * nb + b) * 256]);
            res[t] = TY == T_IQ2_S ? __fmul_rn(0.125f, ch) : ch;  // q8_k.rs:369
        }
        out(cc, r0 + 16 * ptl + row, res);
    }
}

// Gate/up + SwiGLU on the matrix cores (as k_mb_gate_up): workgroup (chunk, row tile).
template <int TY, bool SHARED, int S>
__global__ void __launch_bounds__(MX_THREADS) k_mx_gate_up(BatchArgs a) {
    extern __shared__ __align__(16) uint8_t smem[];
    uint8_t *tab = smem;
    float *terms = reinterpret_cast<float *>(smem + MxTab<TY>::BYTES);
    if (a.plan[1]) return;
    const int nb = a.hidden / 256;
    const int ffn = SHARED ? a.ffn_s : a.ffn_r, rt = 16 * MX_WAVES / S;
    const int tiles = (ffn + rt - 1) / rt;
    const int ci = blockIdx.x / tiles, tile = blockIdx.x - ci * tiles;
    const int r0 = tile * rt, r1 = r0 + rt < ffn ? r0 + rt : ffn;
    int p0, n;
    MatView mv[2];
    if constexpr (SHARED) {
        p0 = ci * a.tc;
        n = a.n_tokens - p0 < a.tc ? a.n_tokens - p0 : a.tc;
        mv[0] = a.shared.gate, mv[1] = a.shared.up;
    } else {
        if (ci >= a.plan[0]) return;
        p0 = a.chunk_p0[ci], n = a.chunk_n[ci];
        const ExpertDev &E = a.experts_mx[a.chunk_expert[ci]];
        mv[0] = E.gate, mv[1] = E.up;
    }
    if (n < a.mx_min) return;
    const int c = (int)(threadIdx.x & 15) < n ? (int)(threadIdx.x & 15) : n - 1;
    const long long tok = SHARED ? (long long)(p0 + c) : (long long)a.pair_token[p0 + c];
    float *g = SHARED ? a.g_s : a.g_r, *u = SHARED ? a.u_s : a.u_r;
    mx_tiles<TY, 2, S>(
        mv, r0, r1, nb, a.xq_mx + tok * nb * 256, a.xd_mx + tok * nb, tab, terms,
        [&]() {
            mx_fill<TY>(tab);
            __syncthreads();
        },
        [&](int i, int r, const float *res) {
            if (i < n && r < r1) {
                const long long o = (long long)(p0 + i) * ffn + r;
                g[o] = res[0];
                u[o] = res[1];
            }
        });
}

// Down on the matrix cores (as k_mb_down).
template <int TY, bool SHARED, int S>
__global__ void __launch_bounds__(MX_THREADS) k_mx_down(BatchArgs a) {
    extern __shared__ __align__(16) uint8_t smem[];
    uint8_t *tab = smem;
    float *terms = reinterpret_cast<float *>(smem + MxTab<TY>::BYTES);
    if (a.plan[1]) return;
    const int nb = (SHARED ? a.ffn_s : a.ffn_r) / 256;
    const int rt = 16 * MX_WAVES / S;
    const int tiles = (a.hidden + rt - 1) / rt;
    const int ci = blockIdx.x / tiles, tile = blockIdx.x - ci * tiles;
    const int r0 = tile * rt, r1 = r0 + rt < a.hidden ? r0 + rt : a.hidden;
    int p0, n;
    MatView mv[1];
    if constexpr (SHARED) {
        p0 = ci * a.tc;
        n = a.n_tokens - p0 < a.tc ? a.n_tokens - p0 : a.tc;
        mv[0] = a.shared.down;
    } else {
        if (ci >= a.plan[0]) return;
        p0 = a.chunk_p0[ci], n = a.chunk_n[ci];
        mv[0] = a.experts_mx[a.chunk_expert[ci]].down;
    }
    if (n < a.mx_min) return;
    const int c = (int)(threadIdx.x & 15) < n ? (int)(threadIdx.x & 15) : n - 1;
    const long long row = p0 + c;
    const uint8_t *bq = (SHARED ? a.hq_mx_s : a.hq_mx_r) + row * nb * 256;
    const float *bd = (SHARED ? a.hd_mx_s : a.hd_mx_r) + row * nb;
    float *d = SHARED ? a.d_s : a.d_r;
    mx_tiles<TY, 1, S>(
        mv, r0, r1, nb, bq, bd, tab, terms,
        [&]() {
            mx_fill<TY>(tab);
            __syncthreads();
        },
        [&](int i, int r, const float *res) {
            if (i < n && r < r1) d[(long long)(p0 + i) * a.hidden + r] = res[0];
        });
}

// Ordered combine of one token's routed outputs in its slot (ascending id)
// order, then the shared expert at 1.0 (moe.rs:141-146).
__global__ void __launch_bounds__(MB_THREADS) k_mb_combine(BatchArgs a) {
    if (a.plan[1]) return;
    const long long total = (long long)a.n_tokens * a.hidden;
    for (long long k = (long long)blockIdx.x * MB_THREADS + threadIdx.x; k < total;
         k += (long long)gridDim.x * MB_THREADS) {
        const int t = (int)(k / a.hidden), r = (int)(k - (long long)t * a.hidden);
        float acc = 0.0f;
        for (int s = 0; s < a.top_k; ++s) {
            const int p = a.pair_of[t * a.top_k + s];
            acc = __fadd_rn(acc, __fmul_rn(a.coefs[t * a.top_k + s], a.d_r[(long long)p * a.hidden + r]));
        }
        if (a.has_shared) acc = __fadd_rn(acc, __fmul_rn(1.0f, a.d_s[(long long)t * a.hidden + r]));
        a.y[k] = a.residual ? __fadd_rn(a.y[k], acc) : acc;
    }
}

// Top-k selection of every token of a batch from finished logits, one wave per token.
__global__ void __launch_bounds__(64) k_route_batch(RouteBatchArgs a) {
    const int t = blockIdx.x;
    RouterArgs r = a.r;
    r.logits = const_cast<float *>(a.logits) + (long long)t * r.n_experts;
    MoeRoute out;
    unsigned long long bad;
    select_route(r, out, bad);
    // out is the same in every lane: lane s writes slot s.
#pragma unroll
    for (int s = 0; s < MOE_MAX_ROUTED; ++s) {
        if (s < r.top_k && (int)threadIdx.x == s) {
            a.ids[(long long)t * r.top_k + s] = out.ids[s];
            a.coefs[(long long)t * r.top_k + s] = out.coefs[s];
        }
    }
    if (threadIdx.x == 0 && a.status && bad != ~0ull) atomicMin(a.status, ((unsigned long long)t << 32) | bad);
}

// ---------------------------------------------------------------- launchers

static inline int cdiv(long long a, long long b) { return (int)((a + b - 1) / b); }

// LDS bytes of a stream launch of type ty (nm matrices, nb blocks per row).
static int stream_lds_of(int ty, int nm, int tc, int nb) {
    switch (ty) {
    case T_IQ2_S: return nm == 2 ? stream_lds<T_IQ2_S, 2>(tc, nb, 2) : stream_lds<T_IQ2_S, 1>(tc, nb, 2);
    case T_IQ3_S: return nm == 2 ? stream_lds<T_IQ3_S, 2>(tc, nb, 2) : stream_lds<T_IQ3_S, 1>(tc, nb, 2);
    case T_Q4_K: return nm == 2 ? stream_lds<T_Q4_K, 2>(tc, nb, 2) : stream_lds<T_Q4_K, 1>(tc, nb, 2);
    case T_Q5_K: return nm == 2 ? stream_lds<T_Q5_K, 2>(tc, nb, 2) : stream_lds<T_Q5_K, 1>(tc, nb, 2);
    default: return 1 << 30;
    }
}

// LDS of the launches of one stream: the VALU kernel's, and the matrix-core
// kernel's when it runs that type.
static int stream_max(const BatchArgs &a, int ty, int nm, int nb, int split) {
    const int v = stream_lds_of(ty, nm, valu_cap(a, ty), nb);
    if (!a.mx || (ty != T_IQ2_S && ty != T_IQ3_S)) return v;
    const int m = mx_lds_bytes(ty, nm, split < 1 ? 1 : split, nb);
    return v > m ? v : m;
}

// stage 0: sort + quantize; 1/2: routed / shared gate-up; 3/4: routed / shared down.
int batch_lds_bytes(const BatchArgs &a, int stage) {
    const int nbh = a.hidden / 256, nbr = a.ffn_r / 256, nbs = a.ffn_s / 256;
    switch (stage) {
    case 0: {
        const int W = (a.n_tokens + 31) / 32;
        const int sort = (a.n_experts * W + 3 * a.n_experts + 2 * MB_THREADS + 4) * 4;
        return sort > MB_WAVES * 4 * 292 ? sort : MB_WAVES * 4 * 292;
    }
    case 1: return stream_max(a, a.type_gate_r, 2, nbh, a.mx_split_gu);
    case 2: return a.has_shared ? stream_max(a, a.shared.gate.type, 2, nbh, a.mx_split_gu) : 0;
    case 3: return stream_max(a, a.type_down_r, 1, nbr, a.mx_split_d);
    default: return a.has_shared ? stream_max(a, a.shared.down.type, 1, nbs, a.mx_split_d) : 0;
    }
}

template <class K>
static hipError_t allow_lds(K kernel, int lds) {
    if (lds <= 64 * 1024) return hipSuccess;
    return hipFuncSetAttribute(reinterpret_cast<const void *>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize, lds);
}

// lds: the stage's LDS footprint; the VALU kernels hold the codebook
// statically, the rest is dynamic.
template <int TY, bool SHARED>
static hipError_t gate_up_typed(const BatchArgs &a, int lds, hipStream_t s) {
    lds -= al16(GridLDS<TY>::BYTES);
    const int grid = SHARED ? cdiv(a.n_tokens, a.tc) * cdiv(a.ffn_s, a.rt_gu_s) : a.max_chunks * cdiv(a.ffn_r, a.rt_gu_r);
    // Routed IQ chunks left to the VALU beside the matrix cores: one-token
    // chunks in their own launch, then the rest (measured on MI355X at the
    // configs[3] shapes: 378.7 -> 369.8 us per step; the fused rows for
    // two-token chunks too measured slower, 405 us).
    if constexpr (!SHARED && (TY == T_IQ2_S || TY == T_IQ3_S)) {
        if (a.mx) {
            hipError_t e = allow_lds(k_mb_gate_up<TY, SHARED, 1>, lds);
            if (e == hipSuccess) e = allow_lds(k_mb_gate_up<TY, SHARED, 2>, lds);
            if (e != hipSuccess) return e;
            hipLaunchKernelGGL((k_mb_gate_up<TY, SHARED, 1>), dim3(grid), dim3(MB_THREADS), lds, s, a);
            if ((e = hipGetLastError()) != hipSuccess || a.mx_min <= 2) return e;   // no chunk of 2+ left
            hipLaunchKernelGGL((k_mb_gate_up<TY, SHARED, 2>), dim3(grid), dim3(MB_THREADS), lds, s, a);
            return hipGetLastError();
        }
    }
    hipError_t e = allow_lds(k_mb_gate_up<TY, SHARED>, lds);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((k_mb_gate_up<TY, SHARED>), dim3(grid), dim3(MB_THREADS), lds, s, a);
    return hipGetLastError();
}

template <int TY, bool SHARED>
static hipError_t down_typed(const BatchArgs &a, int lds, hipStream_t s) {
    lds -= al16(GridLDS<TY>::BYTES);
    const int grid = SHARED ? cdiv(a.n_tokens, a.tc) * cdiv(a.hidden, a.rt_d_s) : a.max_chunks * cdiv(a.hidden, a.rt_d_r);
    // Routed IQ downs beside the matrix cores taking every chunk of 2+ tokens:
    // the VALU chunks all hold one token and run the fused rows (measured on
    // MI355X at the configs[3] shapes: 365.5 -> 359-362 us per step; with
    // 2-token chunks also left to the VALU, a second launch for them made the
    // split slower, 382 against 370 us).
    if constexpr (!SHARED && (TY == T_IQ2_S || TY == T_IQ3_S)) {
        if (a.mx && a.mx_min <= 2) {
            const hipError_t e = allow_lds(k_mb_down<TY, SHARED, 1>, lds);
            if (e != hipSuccess) return e;
            hipLaunchKernelGGL((k_mb_down<TY, SHARED, 1>), dim3(grid), dim3(MB_THREADS), lds, s, a);
            return hipGetLastError();
        }
    }
    hipError_t e = allow_lds(k_mb_down<TY, SHARED>, lds);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((k_mb_down<TY, SHARED>), dim3(grid), dim3(MB_THREADS), lds, s, a);
    return hipGetLastError();
}

// An IQ stream with the matrix cores on: the matrix-core launch when some
// chunk can reach mx_min tokens, then the VALU launch when some chunk can stay
// below it (each kernel returns early on the other's chunks).
template <int TY, bool SHARED, int S>
static hipError_t mx_gate_up_split(const BatchArgs &a, hipStream_t s) {
    const int nb = a.hidden / 256;
    const int lds = mx_lds_bytes(TY, 2, S, nb);
    hipError_t e = allow_lds(k_mx_gate_up<TY, SHARED, S>, lds);
    if (e != hipSuccess) return e;
    const int grid = (SHARED ? cdiv(a.n_tokens, a.tc) : a.max_chunks) * cdiv(SHARED ? a.ffn_s : a.ffn_r, 16 * MX_WAVES / S);
    hipLaunchKernelGGL((k_mx_gate_up<TY, SHARED, S>), dim3(grid), dim3(MX_THREADS), lds, s, a);
    return hipGetLastError();
}

template <int TY, bool SHARED, int S>
static hipError_t mx_down_split(const BatchArgs &a, hipStream_t s) {
    const int nb = (SHARED ? a.ffn_s : a.ffn_r) / 256;
    const int lds = mx_lds_bytes(TY, 1, S, nb);
    hipError_t e = allow_lds(k_mx_down<TY, SHARED, S>, lds);
    if (e != hipSuccess) return e;
    const int grid = (SHARED ? cdiv(a.n_tokens, a.tc) : a.max_chunks) * cdiv(a.hidden, 16 * MX_WAVES / S);
    hipLaunchKernelGGL((k_mx_down<TY, SHARED, S>), dim3(grid), dim3(MX_THREADS), lds, s, a);
    return hipGetLastError();
}

// An IQ stream with the matrix cores on: the matrix-core launch when some
// chunk can reach mx_min tokens, then the VALU launch when some chunk can stay
// below it (each kernel returns early on the other's chunks).  mx_split_* is
// the number of waves that share a 16-row tile (1, 2 or 4).
template <int TY, bool SHARED>
static hipError_t mx_gate_up_typed(const BatchArgs &a, int lds, hipStream_t s_mx, hipStream_t s_valu) {
    if (a.mx_min <= a.tc) {
        const hipError_t e = a.mx_split_gu == 4   ? mx_gate_up_split<TY, SHARED, 4>(a, s_mx)
                             : a.mx_split_gu == 2 ? mx_gate_up_split<TY, SHARED, 2>(a, s_mx)
                                                  : mx_gate_up_split<TY, SHARED, 1>(a, s_mx);
        if (e != hipSuccess) return e;
    }
    return a.mx_min > 1 ? gate_up_typed<TY, SHARED>(a, lds, s_valu) : hipSuccess;
}

template <int TY, bool SHARED>
static hipError_t mx_down_typed(const BatchArgs &a, int lds, hipStream_t s_mx, hipStream_t s_valu) {
    if (a.mx_min <= a.tc) {
        const hipError_t e = a.mx_split_d == 4   ? mx_down_split<TY, SHARED, 4>(a, s_mx)
                             : a.mx_split_d == 2 ? mx_down_split<TY, SHARED, 2>(a, s_mx)
                                                 : mx_down_split<TY, SHARED, 1>(a, s_mx);
        if (e != hipSuccess) return e;
    }
    return a.mx_min > 1 ? down_typed<TY, SHARED>(a, lds, s_valu) : hipSuccess;
}

// The matrix-core part of an IQ stream goes to s_mx, its VALU part to s_valu.
template <bool SHARED>
static hipError_t gate_up_any(int ty, const BatchArgs &a, int lds, hipStream_t s_mx, hipStream_t s_valu) {
    const hipStream_t s = s_valu;
    switch (ty) {
    case T_IQ2_S:
        return a.mx ? mx_gate_up_typed<T_IQ2_S, SHARED>(a, lds, s_mx, s_valu) : gate_up_typed<T_IQ2_S, SHARED>(a, lds, s);
    case T_Q4_K: return gate_up_typed<T_Q4_K, SHARED>(a, lds, s);
    default: return hipErrorInvalidValue;
    }
}

template <bool SHARED>
static hipError_t down_any(int ty, const BatchArgs &a, int lds, hipStream_t s_mx, hipStream_t s_valu) {
    const hipStream_t s = s_valu;
    switch (ty) {
    case T_IQ2_S: return a.mx ? mx_down_typed<T_IQ2_S, SHARED>(a, lds, s_mx, s_valu) : down_typed<T_IQ2_S, SHARED>(a, lds, s);
    case T_IQ3_S: return a.mx ? mx_down_typed<T_IQ3_S, SHARED>(a, lds, s_mx, s_valu) : down_typed<T_IQ3_S, SHARED>(a, lds, s);
    case T_Q5_K: return down_typed<T_Q5_K, SHARED>(a, lds, s);
    default: return hipErrorInvalidValue;
    }
}

bool batch_types_supported(int gate_r, int down_r, int gate_s, int down_s) {
    return gate_r == T_IQ2_S && (down_r == T_IQ3_S || down_r == T_IQ2_S) && (gate_s == T_IQ2_S || gate_s == T_Q4_K) &&
           (down_s == T_IQ2_S || down_s == T_IQ3_S || down_s == T_Q5_K);
}

hipError_t launch_moe_batch(const BatchArgs &a, hipStream_t s, const BatchStreams *streams) {
    if (a.n_tokens < 1 || a.n_tokens > BATCH_MAX_TOKENS || a.top_k < 1 || a.top_k > MOE_MAX_ROUTED ||
        a.n_experts < 1 || a.n_experts > BATCH_MAX_EXPERTS || a.tc < 1 || a.tc > BATCH_MAX_TC)
        return hipErrorInvalidValue;
    const int tsg = a.has_shared ? a.shared.gate.type : T_IQ2_S;
    const int tsd = a.has_shared ? a.shared.down.type : T_IQ3_S;
    if (!batch_types_supported(a.type_gate_r, a.type_down_r, tsg, tsd)) return hipErrorInvalidValue;
    int lds[5];
    for (int i = 0; i < 5; ++i) {
        lds[i] = batch_lds_bytes(a, i);
        if (lds[i] > 160 * 1024) return hipErrorInvalidValue;
    }
    const int nbh = a.hidden / 256;
    hipError_t e = allow_lds(k_mb_prep, lds[0]);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_mb_prep, dim3(1 + cdiv((long long)a.n_tokens * nbh, 4 * MB_WAVES)), dim3(MB_THREADS), lds[0],
                       s, a);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    // Stage 1 (gate/up) and stage 2 (down) each fork the side stream after the
    // main stream's last dependency and join it before the next dependent launch.
    const bool two = streams && streams->side;
    const hipStream_t s2 = two ? streams->side : s;
    auto fork = [&](int i) -> hipError_t {
        if (!two) return hipSuccess;
        hipError_t r = hipEventRecord(streams->fork[i], s);
        return r == hipSuccess ? hipStreamWaitEvent(s2, streams->fork[i], 0) : r;
    };
    auto join = [&](int i) -> hipError_t {
        if (!two) return hipSuccess;
        hipError_t r = hipEventRecord(streams->join[i], s2);
        return r == hipSuccess ? hipStreamWaitEvent(s, streams->join[i], 0) : r;
    };
    if ((e = fork(0)) != hipSuccess) return e;
    if (a.has_shared && a.shared_gemm) {
        // shared gate/up on the matrix cores: they only need Q8_K(x)
        GemmArgs gm{};
        gm.b = a.bx;
        gm.nb = nbh;
        gm.n_tokens = a.n_tokens;
        gm.shape = a.gemm_shape;
        gm.n_mat = 2;
        gm.mat[0] = a.sg;
        gm.mat[1] = a.su;
        if ((e = launch_prep_b(a.q8x, a.n_tokens, nbh, a.bx, s2)) != hipSuccess) return e;
        if ((e = launch_kq_gemm(gm, s2)) != hipSuccess) return e;
    } else if (a.has_shared && (e = gate_up_any<true>(tsg, a, lds[2], s2, s2)) != hipSuccess) {
        return e;
    }
    if ((e = gate_up_any<false>(a.type_gate_r, a, lds[1], s2, s)) != hipSuccess) return e;
    if ((e = join(0)) != hipSuccess) return e;

    const bool rm = tsd == T_Q4_K || tsd == T_Q5_K;
    const int mode = !a.has_shared ? 0 : a.shared_gemm ? 2 : rm ? 1 : 0;
    const long long br = (long long)a.n_tokens * a.top_k * (a.ffn_r / 256);
    const long long bs = a.has_shared ? (long long)a.n_tokens * (a.ffn_s / 256) : 0;
    hipLaunchKernelGGL(k_mb_quant_h, dim3(cdiv(((br + 3) & ~3ll) + bs, 4 * MB_WAVES)), dim3(MB_THREADS), 0, s, a, mode);
    if ((e = hipGetLastError()) != hipSuccess) return e;

    if ((e = fork(1)) != hipSuccess) return e;
    if (a.has_shared && a.shared_gemm) {
        const int nbs = a.ffn_s / 256;
        GemmArgs gm{};
        gm.b = a.bh;
        gm.nb = nbs;
        gm.n_tokens = a.n_tokens;
        gm.shape = a.gemm_shape;
        gm.n_mat = 1;
        gm.mat[0] = a.sd;
        if ((e = launch_prep_b(a.q8h_s, a.n_tokens, nbs, a.bh, s2)) != hipSuccess) return e;
        if ((e = launch_kq_gemm(gm, s2)) != hipSuccess) return e;
    } else if (a.has_shared && (e = down_any<true>(tsd, a, lds[4], s2, s2)) != hipSuccess) {
        return e;
    }
    if ((e = down_any<false>(a.type_down_r, a, lds[3], s2, s)) != hipSuccess) return e;
    if ((e = join(1)) != hipSuccess) return e;

    const long long total = (long long)a.n_tokens * a.hidden;
    int g = cdiv(total, MB_THREADS);
    g = g > 4096 ? 4096 : g;
    hipLaunchKernelGGL(k_mb_combine, dim3(g), dim3(MB_THREADS), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_route_batch(const RouteBatchArgs &a, hipStream_t s) {
    if (a.n_tokens < 1 || a.r.n_experts < 1 || a.r.n_experts > 256 || a.r.top_k < 1 || a.r.top_k > MOE_MAX_ROUTED ||
        a.r.top_k > a.r.n_experts)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_route_batch, dim3(a.n_tokens), dim3(64), 0, s, a);
    return hipGetLastError();
}

}  // namespace lbh
