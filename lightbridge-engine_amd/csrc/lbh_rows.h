// lbh_rows.h — one wave step of row dots: the integer stage of RPW rows of a
// packed matrix against a register-resident Q8_K slice, and the f32 fold of
// each row in the reference's order.  Shared by the matvec, MoE and batched
// kernels.
#pragma once
#include "lbh_dev.h"

namespace lbh {

// Row stride of a wave's term table: 65 floats keeps the chains of one row in
// distinct LDS banks while the fold lanes read them together.
constexpr int TERM_STRIDE = 65;

// Per-wave LDS scratch of the fold.
template <int TY>
struct FoldLDS {
    float terms[Traits<TY>::NCH][TERM_STRIDE];
    float chain[Traits<TY>::KQ ? 64 : 1][9];
};

// Chain of n <= W terms with every read issued first (clamped in-bounds
// index), padded to W with +0.0 terms, which leave every partial sum
// unchanged: a chain that starts at +0.0 never holds -0.0, and s - 0.0 == s
// for all s.
template <int W>
__device__ __forceinline__ float fold_padded(const float *t, int n, bool subtract) {
    float v[W], s = 0.0f;
#pragma unroll
    for (int i = 0; i < W; ++i) {
        const float x = t[i < n ? i : 0];
        v[i] = i < n ? x : 0.0f;
    }
    if (subtract) {
#pragma unroll
        for (int i = 0; i < W; ++i) s = __fsub_rn(s, v[i]);
    } else {
#pragma unroll
        for (int i = 0; i < W; ++i) s = __fadd_rn(s, v[i]);
    }
    return s;
}

// Sequential f32 fold of n per-block terms, s = ((0 + t0) + t1) + ... (or
// 0 - t0 - t1 ... for the minimum chain): the reference's block loop order.
// Rows of up to 16 blocks use a padded chain; with FW = 8 rows of up to 8
// blocks (K = 1536 rows have 6) take a chain of 8 (a shorter dependent-add
// chain, at the registers of a second unrolled copy: kernels whose
// occupancy sits at a register limit keep FW = 16).
template <int FW = 16>
__device__ __forceinline__ float fold_terms(const float *t, int n, bool subtract) {
    if (FW == 8 && n <= 8) return fold_padded<8>(t, n, subtract);
    if (n <= 16) return fold_padded<16>(t, n, subtract);
    float s = 0.0f;
    for (int i = 0; i < n; ++i) s = subtract ? __fsub_rn(s, t[i]) : __fadd_rn(s, t[i]);
    return s;
}

// A lane's place in a wave step (see lbh_dev.h): part of its unit, block b of
// the row, row slot; RPW rows per step.
template <int LPU>
struct LaneMap {
    int part, ui, b, slot, rpw, nb;
    bool lane_on;
    __device__ __forceinline__ LaneMap(int lane, int nb_) {
        nb = nb_;
        part = lane % LPU;
        ui = lane / LPU;
        b = ui % nb;
        slot = ui / nb;
        rpw = (64 / LPU) / nb;
        lane_on = slot < rpw;
    }
    __device__ __forceinline__ bool leader() const { return part == 0 && b == 0; }
};

template <int TY, int LPU>
using WOf = typename std::conditional<Traits<TY>::KQ, WSliceKQ<TY, LPU>, WSlice<TY, LPU>>::type;

// Integer stage + fold of one wave step.  `on` marks lanes whose row exists;
// the row value is returned in the row's leader lane (part 0, block 0).
// block_sums (optional) receives the integer stage of unit u.  GB: codebook
// lookups gathered per GB groups (slice_sum); FW: fold_terms.  Contains wave
// barriers: every lane of the wave must call it.  GR: the codebook accessor
// (GridRef, or Iq3SignedRef over the signed IQ3S table).
template <int TY, int LPU, int GB = 0, int FW = 16, class A = ActOf<TY, LPU>, class GR = GridRef<TY>>
__device__ __forceinline__ float row_dot(const WOf<TY, LPU> &w, const A &act, bool on,
                                         const LaneMap<LPU> &L, const void *grid, FoldLDS<TY> &f,
                                         int32_t *block_sums, long long u) {
    using Tr = Traits<TY>;
    float result = 0.0f;
    if constexpr (Tr::KQ) {
        int32_t ls[8], ms = 0;
        uint32_t dd = 0;
#pragma unroll
        for (int t = 0; t < 8; ++t) ls[t] = 0;
        if (on) {
            slice_sums(w, act, L.part, ls, ms);
            dd = w.hdr.x;
        }
#pragma unroll
        for (int t = 0; t < 8; ++t) ls[t] = unit_reduce<LPU>(ls[t]);
        ms = unit_reduce<LPU>(ms);
        if (on && L.part == 0) {
            const float scale = __fmul_rn(f16_to_f32(dd & 0xffffu), act.d8);
            const float mscale = __fmul_rn(f16_to_f32(dd >> 16), act.d8);
#pragma unroll
            for (int t = 0; t < 8; ++t) f.terms[t][L.ui] = __fmul_rn(scale, (float)ls[t]);
            f.terms[8][L.ui] = __fmul_rn(mscale, (float)ms);
            if (block_sums) {
#pragma unroll
                for (int t = 0; t < 8; ++t) block_sums[u * 9 + t] = ls[t];
                block_sums[u * 9 + 8] = ms;
            }
        }
        wave_sync();
        // Chains 0..7: sums[l] += term (q8_k.rs:316-318); chain 8: sum -= term (:319-320).
        if (on && L.part == 0)
            for (int c = L.b; c < 9; c += L.nb) f.chain[L.slot][c] = fold_terms<FW>(&f.terms[c][L.slot * L.nb], L.nb, c == 8);
        wave_sync();
        if (on && L.leader()) {
            float s = f.chain[L.slot][8];
#pragma unroll
            for (int l = 0; l < 8; ++l) s = __fadd_rn(s, f.chain[L.slot][l]);  // q8_k.rs:323-325
            result = s;
        }
    } else {
        int32_t bs = 0;
        uint32_t dbits = 0;
        if (on) {
            bs = slice_sum<LPU, GB>(w, act, GR(grid));
            dbits = w.d;
        }
        bs = unit_reduce<LPU>(bs);
        if (on && L.part == 0) {
            f.terms[0][L.ui] = __fmul_rn(__fmul_rn(f16_to_f32(dbits), act.d8), (float)bs);
            if (block_sums) block_sums[u] = bs;
        }
        wave_sync();
        if (on && L.leader()) {
            float s = fold_terms<FW>(&f.terms[0][L.slot * L.nb], L.nb, false);
            if (TY == T_IQ2_S) s = __fmul_rn(0.125f, s);  // q8_k.rs:369
            result = s;
        }
    }
    wave_sync();
    return result;
}

}  // namespace lbh
