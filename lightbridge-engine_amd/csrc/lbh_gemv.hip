// lbh_gemv.hip — {IQ2_S, IQ3_S, Q4_K, Q5_K} x Q8_K matvec for gfx950.
//
// y[r] = vec_dot_q8_k(row r, q8)  (crates/bridge-quant-layout/src/q8_k.rs:80-89,
// row loop of crates/bridge-kernels-reference/src/gemv.rs:56-70), or
// y[r] += coef * dot (gemv.rs:161-171).
//
// Decode matvecs are HBM-bound: every weight byte is read once with 16-byte
// loads from the chunk-major device layout (lbh_layout.h), the IQ codebooks
// sit in LDS next to their negations, the integer block sums use v_dot4, and
// the per-row f32 fold runs in the reference's sequential block order out of
// LDS.  With FUSEQ the kernel also performs the Q8_K quantization of the f32
// input itself (each workgroup quantizes into LDS; workgroup 0 publishes the
// bytes), which removes a launch from every gemv_into.
#include <atomic>

#include "lbh_internal.h"
#include "lbh_rows.h"

namespace lbh {

// Workgroups of 256 threads, or 512 for matrices large enough to give every
// CU several such workgroups' worth of wave steps: every workgroup pays the
// prologue (codebook and activation staging), so fewer, larger workgroups
// pay it fewer times.
constexpr int GEMV_THREADS = 256;
constexpr int GEMV_THREADS_LARGE = 512;
constexpr int GEMV_THREADS_XL = 1024;
constexpr int MAX_NB = 64;

#ifdef LBH_WAVE_TIMELINE
// Per-wave timeline of the matvec (a profiling build only: make timeline):
// s_memrealtime (100 MHz) at the kernel's start, the end of the prologue, the
// barrier, the first step's weights landed, that step folded, and the end;
// then the wave's step count and workgroup.
constexpr int TL_WAVES = 16384;
__device__ unsigned long long g_wave_timeline[TL_WAVES * 8];
__device__ __forceinline__ unsigned long long tl_now() { return __builtin_amdgcn_s_memrealtime(); }
#endif

__device__ __forceinline__ bool status_set(const DevStatus *st) {
    return st && (st->first_bad_input != ~0ull || st->first_bad_dest != ~0ull);
}

__device__ __forceinline__ void store_y(const GemvArgs &p, int r, float v) {
    if (!p.y) return;   // integer-stage export only (lbh_gemv_block_sums)
    if (p.accumulate)
        p.y[r] = __fadd_rn(p.y[r], __fmul_rn(p.coef, v));
    else
        p.y[r] = v;
}

template <int TY, int LPU, bool FUSEQ, int D, int NT>
__global__ void __launch_bounds__(NT) k_gemv(GemvArgs p) {
    constexpr int GEMV_WAVES = NT / 64;
    // Large IQ3_S instances read the signed table (one LDS word per four
    // weights, no sign work; 32 KiB to fill per workgroup), 256-thread ones
    // the 6 KiB pair table, whose fill costs their short prologue less
    // (measured on MI355X: IQ3_S 4096x1536 3.86 vs 3.93 us, 4096x13312 11.1 vs
    // 11.3 us).
    constexpr bool SGN = TY == T_IQ3_S && NT >= GEMV_THREADS_LARGE;
    constexpr int GT = SGN ? T_IQ3S_SGN : TY;
    constexpr int GB = GridLDS<GT>::BYTES > 0 ? GridLDS<GT>::BYTES : 16;
    __shared__ __align__(16) uint8_t s_grid[GB];
    __shared__ __align__(16) uint8_t s_q8[FUSEQ ? MAX_NB * 292 : 16];
    // K-quant dots read the quants residue-major: quantized once per workgroup
    // into that layout too, instead of a byte transpose in every lane.
    constexpr bool RES = FUSEQ && Traits<TY>::KQ;
    __shared__ __align__(16) uint8_t s_q8r[RES ? MAX_NB * RES_STRIDE : 16];
    // 1024-thread IQ instances read the activations from LDS one group at a
    // time (ActIQL) instead of holding a whole block in registers, which is
    // what fits four waves per SIMD.
    constexpr bool AL = LPU == 1 && !Traits<TY>::KQ && NT == GEMV_THREADS_XL;
    __shared__ __align__(16) uint8_t s_q8q[AL ? MAX_NB * RES_STRIDE : 16];
    __shared__ FoldLDS<TY> s_fold[GEMV_WAVES];

    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    const int NB = p.m.nb;
    const LaneMap<LPU> L(lane, NB);
    const int rows = p.m.rows;
    const Planes P = make_planes(p.m.planes, p.m.units, p.m.bytes);
    const uint32_t po = part_offset<TY, LPU>(P, L.part);
    const int items = (rows + L.rpw - 1) / L.rpw;
    const int nw = gridDim.x * GEMV_WAVES;
    using W = WOf<TY, LPU>;

    auto issue = [&](int it, W &w) {
        const int r = it * L.rpw + L.slot;
        if (it < items && L.lane_on && r < rows) load_slice(P, (uint32_t)(r * NB + L.b), po, L.part, w);
    };

    // Prologue loads first (codebook, this wave's first chunk of x), then the
    // first step's weight loads, then the prologue's LDS stores and barrier:
    // the small prologue loads do not wait behind the weight burst, and the
    // weights' HBM latency overlaps the prologue.  The first weight load is
    // unconditional (row clamped into the matrix; lanes without a row load a
    // row another lane loads) so the wait before the stores counts exactly the
    // weight loads issued after the prologue's; the other D - 1 steps go out
    // after the barrier.
#ifdef LBH_WAVE_TIMELINE
    unsigned long long tl[6] = {tl_now(), 0, 0, 0, 0, 0};
    int tl_steps = 0;
#endif
    int it = blockIdx.x * GEMV_WAVES + wid;
    const GridIn<GT, NT> gin = grid_load<GT, NT>();
    // The input blocks of the first QP quantize passes are loaded here, ahead
    // of the weights: a pass whose loads went out after the weight loads
    // would wait for the whole weight burst to land before the barrier.
    constexpr int QP = FUSEQ ? (MAX_NB / (4 * GEMV_WAVES) < 2 ? MAX_NB / (4 * GEMV_WAVES) : 2) : 1;
    QuantIn qin[QP];
    if constexpr (FUSEQ) {
#pragma unroll
        for (int q = 0; q < QP; ++q) qin[q] = quantize_load(p.x, 4 * wid + 4 * GEMV_WAVES * q, NB);
    }
    // Caller-quantized activations of an AL instance: their quants copied to
    // the aligned LDS copy (NB * 64 dwords, at most four per thread).
    constexpr int CP = !FUSEQ && AL ? MAX_NB * 64 / NT : 1;
    uint32_t cp[CP];
    if constexpr (!FUSEQ && AL) {
#pragma unroll
        for (int c = 0; c < CP; ++c) {
            const int i = threadIdx.x + NT * c;
            cp[c] = i < NB * 64 ? ld_u32(p.q8 + (i >> 6) * 292 + 4 + 4 * (i & 63)) : 0u;
        }
    }
    W w[D];
    // 512-thread IQ3_S instances: every wave's prologue loads go out before
    // any wave's weight loads (a plain s_barrier, no memory wait), so the
    // activation and table reads do not queue behind the weight burst
    // (measured on MI355X: IQ3_S 4096x8192 7.4 -> 7.0 us; the IQ2_S instances
    // measured slower with it).  1024-thread IQ3_S instances, whose one step
    // per wave requests the whole matrix at once, issue it after the prologue
    // barrier instead: the prologue then ends at about 2.5 us instead of 4 us,
    // and the decode overlaps the rest of the stream (IQ3_S 4096x13312 10.7 ->
    // 10.2 us; the IQ2_S instance gains nothing from it).
    constexpr bool LATE = TY == T_IQ3_S && NT == GEMV_THREADS_XL;
    if constexpr (TY == T_IQ3_S && NT == GEMV_THREADS_LARGE) __builtin_amdgcn_s_barrier();
    if constexpr (!LATE) {
        int r = it * L.rpw + (L.lane_on ? L.slot : L.rpw - 1);
        r = r < rows ? r : rows - 1;
        load_slice(P, (uint32_t)(r * NB + L.b), po, L.part, w[0]);
    }

    grid_store<GT, NT>(gin, s_grid);
    if constexpr (FUSEQ) {
#pragma unroll
        for (int q = 0; q < QP; ++q)
            if (4 * wid + 4 * GEMV_WAVES * q < NB)
                quantize_store(qin[q], s_q8, RES ? s_q8r : nullptr, AL ? s_q8q : nullptr);
        for (int b0 = 4 * wid + 4 * GEMV_WAVES * QP; b0 < NB; b0 += 4 * GEMV_WAVES)
            quantize_blocks_wave(p.x, s_q8, b0, NB, RES ? s_q8r : nullptr, AL ? s_q8q : nullptr);
    } else if constexpr (AL) {
#pragma unroll
        for (int c = 0; c < CP; ++c) {
            const int i = threadIdx.x + NT * c;
            if (i < NB * 64) *reinterpret_cast<uint32_t *>(s_q8q + (i >> 6) * RES_STRIDE + 4 * (i & 63)) = cp[c];
        }
    }
#ifdef LBH_WAVE_TIMELINE
    tl[1] = tl_now();
#endif
    __syncthreads();
#ifdef LBH_WAVE_TIMELINE
    tl[2] = tl_now();
#endif
    if constexpr (LATE) {
        int r = it * L.rpw + (L.lane_on ? L.slot : L.rpw - 1);
        r = r < rows ? r : rows - 1;
        load_slice(P, (uint32_t)(r * NB + L.b), po, L.part, w[0]);
    }
#pragma unroll
    for (int d = 1; d < D; ++d) issue(it + d * nw, w[d]);
    if (status_set(p.status)) return;
    if constexpr (FUSEQ) {
        if (p.q8_out && blockIdx.x == 0)
            for (int i = threadIdx.x; i < NB * 73; i += NT)
                reinterpret_cast<uint32_t *>(p.q8_out)[i] = reinterpret_cast<const uint32_t *>(s_q8)[i];
    }

    using A = typename std::conditional<AL, ActIQL, ActOf<TY, LPU>>::type;
    using GR = typename std::conditional<SGN, Iq3SignedRef, GridRef<TY>>::type;
    A act;
    if constexpr (AL) {
        act.q = s_q8q + L.b * RES_STRIDE;
        act.d8 = __uint_as_float(ld_u32(FUSEQ ? s_q8 + L.b * 292 : p.q8 + (long long)L.b * 292));
    } else if constexpr (RES) {
        load_act_res(s_q8 + L.b * 292, s_q8r + L.b * RES_STRIDE, L.part, act);
    } else {
        load_act(FUSEQ ? s_q8 + L.b * 292 : p.q8 + (long long)L.b * 292, L.part, act);
    }

    auto process = [&](int it, const W &w) {
#ifdef LBH_WAVE_TIMELINE
        if (tl_steps == 0) {
            __builtin_amdgcn_s_waitcnt(0);
            tl[3] = tl_now();
        }
#endif
        const int r = it * L.rpw + L.slot;
        const bool on = L.lane_on && r < rows;
        // One wave per SIMD (every instance but the 1024-thread ones): the
        // codebook reads are gathered (the latency of a single wave's LDS round
        // trips is the dot's critical path).
        constexpr int GB = NT == GEMV_THREADS_XL ? 0 : TY == T_IQ2_S ? 4 : TY == T_IQ3_S ? 2 : 0;
        const float v =
            row_dot<TY, LPU, GB, Traits<TY>::KQ ? 16 : 8, A, GR>(w, act, on, L, s_grid, s_fold[wid],
                                                                 p.block_sums, (long long)r * NB + L.b);
        if (on && L.leader()) store_y(p, r, v);
#ifdef LBH_WAVE_TIMELINE
        if (tl_steps++ == 0) tl[4] = tl_now();
#endif
    };

    // Software pipeline over a ring of D register buffers, unrolled D times so
    // the buffers rotate without copies: the loads of the wave's next D - 1
    // steps are in flight while the current step is computed, and the buffer
    // just consumed is refilled with the step D ahead.
    while (it < items) {
#pragma unroll
        for (int d = 0; d < D; ++d) {
            if (it >= items) break;
            process(it, w[d]);
            issue(it + D * nw, w[d]);
            it += nw;
        }
    }
#ifdef LBH_WAVE_TIMELINE
    tl[5] = tl_now();
    const int gw = blockIdx.x * GEMV_WAVES + wid;
    if (lane == 0 && gw < TL_WAVES) {
        unsigned long long *o = g_wave_timeline + (long long)gw * 8;
#pragma unroll
        for (int i = 0; i < 6; ++i) o[i] = tl[i];
        o[6] = (unsigned long long)tl_steps;
        o[7] = blockIdx.x;
    }
#endif
}

static inline int cdiv(long long a, long long b) { return (int)((a + b - 1) / b); }

// Workgroups of one kernel instance that fit on a CU at once (register and LDS
// limited), queried once per instance.
template <int TY, int LPU, bool FUSEQ, int D, int NT>
static int resident_per_cu() {
    static std::atomic<int> cached{0};
    int n = cached.load(std::memory_order_relaxed);
    if (n == 0) {
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, k_gemv<TY, LPU, FUSEQ, D, NT>, NT, 0) != hipSuccess || n < 1)
            n = 1;
        cached.store(n, std::memory_order_relaxed);
    }
    return n;
}

// Grid: one workgroup per NT / 64 wave steps, capped at `max_blocks`, or,
// when that is 0, at the workgroups resident on the device at once: a
// persistent grid pays the prologue (codebook and activation staging) once per
// resident workgroup instead of once per later wave of workgroups.
template <int TY, int LPU, bool FUSEQ, int D, int NT>
static hipError_t launch_nt(const GemvArgs &a, const GemvTuning &t, hipStream_t s) {
    const int rpw = (64 / LPU) / a.m.nb;
    const int items = cdiv(a.m.rows, rpw);
    int grid = cdiv(items, NT / 64);
    const int cap = t.max_blocks > 0 ? t.max_blocks : resident_per_cu<TY, LPU, FUSEQ, D, NT>() * t.cu_count;
    if (cap > 0 && grid > cap) grid = cap;
    hipLaunchKernelGGL((k_gemv<TY, LPU, FUSEQ, D, NT>), dim3(grid), dim3(NT), 0, s, a);
    return hipGetLastError();
}

// 512-thread workgroups for one lane per unit once the matrix has at least
// 2 * 64 * 4 units per CU (measured on MI355X: IQ2_S 8192x4096 7.2 -> 6.0 us,
// IQ3_S 4096x13312 14.5 -> 12.7 us; Q4_K 4096x4096 stays faster at 256).
template <int TY, int LPU, bool FUSEQ, int D>
static hipError_t launch_inst(const GemvArgs &a, const GemvTuning &t, hipStream_t s) {
    if constexpr (LPU == 1 && D == 1 && !Traits<TY>::KQ) return launch_nt<TY, LPU, FUSEQ, D, GEMV_THREADS_XL>(a, t, s);
    if constexpr (LPU == 1) {
        const long long units = (long long)a.m.rows * a.m.nb;
        if (units >= 2LL * 64 * 4 * (t.cu_count > 0 ? t.cu_count : 256))
            return launch_nt<TY, LPU, FUSEQ, D, GEMV_THREADS_LARGE>(a, t, s);
    }
    return launch_nt<TY, LPU, FUSEQ, D, GEMV_THREADS>(a, t, s);
}

template <int TY, int LPU, int D>
static hipError_t launch_depth(const GemvArgs &a, const GemvTuning &t, hipStream_t s) {
    return a.x ? launch_inst<TY, LPU, true, D>(a, t, s) : launch_inst<TY, LPU, false, D>(a, t, s);
}

template <int TY, int LPU>
static hipError_t launch_typed(const GemvArgs &a, const GemvTuning &t, int depth, hipStream_t s) {
    switch (depth) {
    case 4: return launch_depth<TY, LPU, 4>(a, t, s);
    case 3: return launch_depth<TY, LPU, 3>(a, t, s);
    case 1: return launch_depth<TY, LPU, 1>(a, t, s);
    default: return launch_depth<TY, LPU, 2>(a, t, s);
    }
}

template <int TY>
static hipError_t launch_lpu(const GemvArgs &a, const GemvTuning &t, int lpu, int depth, hipStream_t s) {
    switch (lpu) {
    case 4: return launch_typed<TY, 4>(a, t, depth, s);
    case 2: return launch_typed<TY, 2>(a, t, depth, s);
    default: return launch_typed<TY, 1>(a, t, depth, s);
    }
}

// Built-in lanes-per-unit choice.  One lane per (row, block) unit reads each
// block once with the fewest instructions, but holds a whole block of
// activations in registers; it is the faster choice once the matrix gives
// every CU at least four such waves.  Smaller matrices are latency-bound and
// gain from the shorter per-lane work of more lanes per unit (measured on
// MI355X: Q4_K 4096x4096 4.5 vs 5.5 us at one and two lanes; IQ2_S 1536x4096
// 4.6 vs 5.2 us at two and one; IQ2_S 1024x4096 4.3 vs 4.6 us at four and
// two).
static int default_lpu(const GemvArgs &a, int cu_count) {
    const long long units = (long long)a.m.rows * a.m.nb;
    const long long cus = cu_count > 0 ? cu_count : 256;
    return units >= 64LL * 4 * cus ? 1 : units >= 80LL * cus ? 2 : 4;
}

// Built-in depth: one row step per wave in 1024-thread workgroups (activations
// read from LDS, four waves per SIMD) for one-lane IQ matvecs with at least 12
// wave steps per CU (measured on MI355X, fused Q8_K: IQ2_S 13312x4096 8.9 ->
// 8.0 us, IQ3_S 4096x13312 12.3 -> 11.3 us; IQ3_S 4096x8192, 8 steps per CU,
// 7.7 vs 9.1 us stays at two).  Matrices whose row steps fit one wave per SIMD
// also take one buffer: the second would never be filled, and the smaller
// register footprint is faster (IQ2_S 1536x4096 4.02 -> 3.96 us, IQ3_S
// 4096x1536 3.86 -> 3.83 us, Q4_K 4096x4096 4.58 -> 4.48 us; IQ2_S 1024x4096
// at four lanes per unit stays at two, 3.72 vs 3.75 us).  Two steps in
// flight otherwise.
static int default_depth(const GemvArgs &a, int lpu, int cu_count) {
    const bool iq = a.m.type == T_IQ2_S || a.m.type == T_IQ3_S;
    const long long steps = (long long)a.m.rows * a.m.nb / 64;
    const long long cus = cu_count > 0 ? cu_count : 256;
    if (iq && lpu == 1 && steps >= 12LL * cus) return 1;
    const int rpw = (64 / lpu) / a.m.nb;
    const long long items = (a.m.rows + rpw - 1) / rpw;
    return items <= 4 * cus && (lpu <= 2 || !iq) ? 1 : 2;
}

hipError_t launch_gemv(const GemvArgs &a, const GemvTuning &t, hipStream_t s) {
    const int nb = a.m.nb;
    if (nb < 1 || nb > MAX_NB || a.m.rows < 1) return hipErrorInvalidValue;
    if (!a.q8 && !a.x) return hipErrorInvalidValue;
    int lpu = t.lpu > 0 ? t.lpu : default_lpu(a, t.cu_count);
    lpu = lpu >= 4 ? 4 : lpu >= 2 ? 2 : 1;
    // A wave step must hold at least one whole row: NB * LPU <= 64.
    while (lpu > 1 && nb * lpu > 64) lpu >>= 1;
    const int depth = t.depth > 0 ? t.depth : default_depth(a, lpu, t.cu_count);
    switch (a.m.type) {
    case T_IQ2_S: return launch_lpu<T_IQ2_S>(a, t, lpu, depth, s);
    case T_IQ3_S: return launch_lpu<T_IQ3_S>(a, t, lpu, depth, s);
    case T_Q4_K: return launch_lpu<T_Q4_K>(a, t, lpu, depth, s);
    case T_Q5_K: return launch_lpu<T_Q5_K>(a, t, lpu, depth, s);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace lbh

#ifdef LBH_WAVE_TIMELINE
// The per-wave timeline of the last matvec launches (8 words per wave, wave
// index = workgroup * waves per workgroup + wave): read and clear.
extern "C" int lbh_wave_timeline_read(void *host, size_t bytes) {
    return (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(lbh::g_wave_timeline), bytes, 0, hipMemcpyDeviceToHost);
}
extern "C" int lbh_wave_timeline_clear() {
    static unsigned long long zeros[lbh::TL_WAVES * 8];
    return (int)hipMemcpyToSymbol(HIP_SYMBOL(lbh::g_wave_timeline), zeros, sizeof(zeros), 0, hipMemcpyHostToDevice);
}
#endif
