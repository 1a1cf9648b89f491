// lbh_moe.hip — the routed + shared SwiGLU expert FFN of one token
// (moe_routed_by_id_into, crates/bridge-kernels-reference/src/moe.rs:64-147)
// in two launches:
//
//   k_moe_gate_up  one workgroup per (expert, tile of hidden rows): Q8_K(x) into
//                  LDS, gate and up row dots of the tile, SwiGLU with the
//                  libm-exact expf (activation.rs:170-178), h to scratch; the
//                  last workgroup to finish a 256-row block of h quantizes it
//                  to Q8_K (release/acquire on a self-resetting arrival count).
//   k_moe_down     one workgroup per tile of output rows: the down row dots of
//                  every routed expert and of the shared expert, then each row
//                  is combined in the reference order
//                      y = ((0 + c_0 d_0) + c_1 d_1) + ... + 1.0 * d_shared
//                  (gemv_accumulate_scaled_into, gemv.rs:161-171, moe.rs:141-146).
//
// The result is bit-identical to the reference: the same Q8_K bytes, integer
// block sums, per-row folds, SwiGLU and accumulation order.
#include "lbh_internal.h"
#include "lbh_math.h"
#include "lbh_rows.h"

namespace lbh {

constexpr int MOE_THREADS = 256;
constexpr int MOE_WAVES = MOE_THREADS / 64;

__host__ __device__ constexpr int align16(int v) { return (v + 15) & ~15; }

__device__ __forceinline__ int route_n(const MoeArgs &a) { return a.route_dev ? a.route_dev->n : a.route.n; }
__device__ __forceinline__ uint32_t route_id(const MoeArgs &a, int s) {
    return a.route_dev ? a.route_dev->ids[s] : a.route.ids[s];
}
__device__ __forceinline__ float route_coef(const MoeArgs &a, int s) {
    return a.route_dev ? a.route_dev->coefs[s] : a.route.coefs[s];
}

// LDS bytes of one gate/up tile body.
template <int TY>
__host__ __device__ constexpr int gate_up_lds(int nb) {
    return align16(GridLDS<TY>::BYTES) + align16(nb * 292) + MOE_WAVES * (int)sizeof(FoldLDS<TY>) + 16;
}

// Gate and up rows [r0, r1) of one expert, SwiGLU into h (slot), then the
// last-arriving tile of each 256-row block quantizes it to Q8_K.
template <int TY, int LPU>
__device__ __forceinline__ void gate_up_tile(const MoeArgs &a, const MatView &G, const MatView &Uv, int rows_total,
                                             int tile, int r0, int r1, int slot, int order, uint8_t *smem) {
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    const int NB = a.hidden / 256;
    uint8_t *s_grid = smem;
    uint8_t *s_q8 = smem + align16(GridLDS<TY>::BYTES);
    FoldLDS<TY> *s_fold = reinterpret_cast<FoldLDS<TY> *>(s_q8 + align16(NB * 292));
    int *s_flag = reinterpret_cast<int *>(s_fold + MOE_WAVES);

    const LaneMap<LPU> L(lane, NB);
    const Planes PG = make_planes(G.planes, G.units, G.bytes);
    const Planes PU = make_planes(Uv.planes, Uv.units, Uv.bytes);
    const uint32_t po = part_offset<TY, LPU>(PG, L.part);   // gate and up share the shape
    const int items = (r1 - r0 + L.rpw - 1) / L.rpw;
    using W = WOf<TY, LPU>;
    auto issue = [&](int it, W &wg, W &wu) {
        const int r = r0 + it * L.rpw + L.slot;
        if (it < items && L.lane_on && r < r1) {
            const uint32_t u = (uint32_t)(r * NB + L.b);
            load_slice(PG, u, po, L.part, wg);
            load_slice(PU, u, po, L.part, wu);
        }
    };
    int it = wid;
    W ga, ua, gb, ub;
    issue(it, ga, ua);

    fill_grid<TY>(s_grid);
    for (int b0 = 4 * wid; b0 < NB; b0 += 4 * MOE_WAVES) quantize_blocks_wave(a.x, s_q8, b0, NB);
    __syncthreads();
    ActOf<TY, LPU> act;
    load_act(s_q8 + L.b * 292, L.part, act);

    float *h = a.h + (long long)slot * a.h_stride;
    auto process = [&](int it, const W &wg, const W &wu) {
        const int r = r0 + it * L.rpw + L.slot;
        const bool on = L.lane_on && r < r1;
        const float gv = row_dot<TY, LPU>(wg, act, on, L, s_grid, s_fold[wid], nullptr, 0);
        const float uv = row_dot<TY, LPU>(wu, act, on, L, s_grid, s_fold[wid], nullptr, 0);
        if (on && L.leader()) {
            const float hv = swiglu_ref(gv, uv);
            h[r] = hv;
            if (a.check && !isfinite(hv))
                atomicMin(&a.status->first_bad_swiglu, ((unsigned long long)order << 32) | (unsigned)r);
        }
    };
    while (it < items) {
        issue(it + MOE_WAVES, gb, ub);
        process(it, ga, ua);
        it += MOE_WAVES;
        if (it >= items) break;
        issue(it + MOE_WAVES, ga, ua);
        process(it, gb, ub);
        it += MOE_WAVES;
    }

    // Publish this tile's h rows; the tile that completes a 256-row block
    // quantizes it (the count resets itself for the next call).
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) {
        const int b_first = r0 / 256, b_last = (r1 - 1) / 256;
        for (int blk = b_first, i = 0; i < 2; ++blk, ++i) {
            s_flag[i] = -1;
            if (blk > b_last) continue;
            const int t_first = (blk * 256) / tile;
            const int t_last = ((blk + 1) * 256 < rows_total ? (blk + 1) * 256 : rows_total) - 1;
            const unsigned need = (unsigned)(t_last / tile - t_first + 1);
            uint32_t *c = a.counters + (long long)slot * a.cnt_stride + blk;
            const unsigned old = __hip_atomic_fetch_add(c, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
            if (old + 1 == need) {
                s_flag[i] = blk;
                __hip_atomic_store(c, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
    }
    __syncthreads();
    if (wid < 2 && s_flag[wid] >= 0) {
        __threadfence();
        quantize_blocks_wave(h, a.q8h + (long long)slot * a.q8_stride, s_flag[wid], s_flag[wid] + 1);
    }
}

template <int TYR, int LPUR, int TYS, int LPUS>
__global__ void __launch_bounds__(MOE_THREADS) k_moe_gate_up(MoeArgs a) {
    extern __shared__ __align__(16) uint8_t smem[];
    if (a.status && a.status->first_bad_input != ~0ull) return;
    const int n = route_n(a);
    int bid = blockIdx.x;
    const int ts = a.has_shared ? a.tiles_s : 0;
    if (bid < ts) {
        const int r0 = bid * a.tile_s, r1 = r0 + a.tile_s < a.ffn_s ? r0 + a.tile_s : a.ffn_s;
        gate_up_tile<TYS, LPUS>(a, a.shared.gate, a.shared.up, a.ffn_s, a.tile_s, r0, r1, MOE_SHARED_SLOT, n, smem);
        return;
    }
    bid -= ts;
    const int s = bid / a.tiles_r, t = bid - s * a.tiles_r;
    const ExpertDev &E = a.experts[route_id(a, s)];
    const int r0 = t * a.tile_r, r1 = r0 + a.tile_r < a.ffn_r ? r0 + a.tile_r : a.ffn_r;
    gate_up_tile<TYR, LPUR>(a, E.gate, E.up, a.ffn_r, a.tile_r, r0, r1, s, s, smem);
}

// Down row dots of `count` matrices of one type for rows [r0, r1): matrix m
// reads its Q8_K input from s_q8 + m * in_stride and writes s_y[m][row - r0].
template <int TY, int LPU, class GetView>
__device__ __forceinline__ void down_rows(const GetView &view_of, int count, int nb, const uint8_t *s_q8, int in_stride,
                                          int r0, int r1, const void *s_grid, FoldLDS<TY> &fold, float *s_y, int y_stride,
                                          int m_base) {
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    const LaneMap<LPU> L(lane, nb);
    const int per = (r1 - r0 + L.rpw - 1) / L.rpw;
    const int total = count * per;
    for (int i = wid; i < total; i += MOE_WAVES) {
        const int m = i / per, j = i - m * per;
        const MatView V = view_of(m);
        const Planes P = make_planes(V.planes, V.units, V.bytes);
        const int r = r0 + j * L.rpw + L.slot;
        const bool on = L.lane_on && r < r1;
        WOf<TY, LPU> w;
        if (on) load_slice(P, (uint32_t)(r * nb + L.b), part_offset<TY, LPU>(P, L.part), L.part, w);
        ActOf<TY, LPU> act;
        load_act(s_q8 + m * in_stride + L.b * 292, L.part, act);
        const float v = row_dot<TY, LPU>(w, act, on, L, s_grid, fold, nullptr, 0);
        if (on && L.leader()) s_y[(m_base + m) * y_stride + (r - r0)] = v;
    }
}

template <int TYR, int TYS>
__host__ __device__ constexpr int down_fold_bytes() {
    return (int)sizeof(FoldLDS<TYR>) > (int)sizeof(FoldLDS<TYS>) ? (int)sizeof(FoldLDS<TYR>) : (int)sizeof(FoldLDS<TYS>);
}

template <int TYR, int LPUR, int TYS, int LPUS>
__global__ void __launch_bounds__(MOE_THREADS) k_moe_down(MoeArgs a) {
    extern __shared__ __align__(16) uint8_t smem[];
    if (a.status && (a.status->first_bad_input != ~0ull || a.status->first_bad_swiglu != ~0ull)) return;
    const int wid = threadIdx.x >> 6;
    const int n = route_n(a);
    const int nbr = a.ffn_r / 256, nbs = a.ffn_s / 256;
    const int r0 = blockIdx.x * a.tile_d;
    const int r1 = r0 + a.tile_d < a.hidden ? r0 + a.tile_d : a.hidden;
    constexpr int GB = GridLDS<TYR>::BYTES > GridLDS<TYS>::BYTES ? GridLDS<TYR>::BYTES : GridLDS<TYS>::BYTES;
    uint8_t *s_grid_r = smem;
    uint8_t *s_grid_s = smem + align16(GridLDS<TYR>::BYTES);
    uint8_t *s_q8 = smem + align16(GridLDS<TYR>::BYTES) + align16(TYS == TYR ? 0 : GridLDS<TYS>::BYTES);
    const int q8_bytes = align16((n * nbr + (a.has_shared ? nbs : 0)) * 292);
    uint8_t *s_foldp = s_q8 + q8_bytes;
    float *s_y = reinterpret_cast<float *>(s_foldp + MOE_WAVES * down_fold_bytes<TYR, TYS>());
    (void)GB;

    // Stage the Q8_K inputs: routed slots 0..n-1, then the shared slot.
    const int rbytes = nbr * 292;
    for (int m = 0; m < n; ++m)
        for (int i = threadIdx.x; i < rbytes / 4; i += MOE_THREADS)
            reinterpret_cast<uint32_t *>(s_q8 + m * rbytes)[i] =
                reinterpret_cast<const uint32_t *>(a.q8h + (long long)m * a.q8_stride)[i];
    if (a.has_shared)
        for (int i = threadIdx.x; i < nbs * 73; i += MOE_THREADS)
            reinterpret_cast<uint32_t *>(s_q8 + n * rbytes)[i] =
                reinterpret_cast<const uint32_t *>(a.q8h + (long long)MOE_SHARED_SLOT * a.q8_stride)[i];
    fill_grid<TYR>(s_grid_r);
    if (TYS != TYR) fill_grid<TYS>(s_grid_s);
    __syncthreads();

    const int ystride = a.tile_d;
    auto routed_view = [&](int m) { return a.experts[route_id(a, m)].down; };
    down_rows<TYR, LPUR>(routed_view, n, nbr, s_q8, rbytes, r0, r1, s_grid_r,
                         *reinterpret_cast<FoldLDS<TYR> *>(s_foldp + wid * down_fold_bytes<TYR, TYS>()), s_y, ystride, 0);
    if (a.has_shared) {
        auto shared_view = [&](int) { return a.shared.down; };
        down_rows<TYS, LPUS>(shared_view, 1, nbs, s_q8 + n * rbytes, 0, r0, r1, TYS == TYR ? s_grid_r : s_grid_s,
                             *reinterpret_cast<FoldLDS<TYS> *>(s_foldp + wid * down_fold_bytes<TYR, TYS>()), s_y, ystride,
                             n);
    }
    __syncthreads();

    // Ordered combine: output.fill(0), then dest += coef * dot per expert in
    // ascending id order, then the shared expert at 1.0 (moe.rs:141-146).
    const int last = a.has_shared ? n : n - 1;
    for (int t = threadIdx.x; t < r1 - r0; t += MOE_THREADS) {
        float acc = 0.0f;
        int bad = -1;
        for (int s = 0; s < n && s <= a.stop_step; ++s) {
            acc = __fadd_rn(acc, __fmul_rn(route_coef(a, s), s_y[s * ystride + t]));
            if (bad < 0 && !isfinite(acc)) bad = s;
        }
        if (a.has_shared && n <= a.stop_step) acc = __fadd_rn(acc, __fmul_rn(1.0f, s_y[n * ystride + t]));
        a.y[r0 + t] = acc;
        // A later accumulation call rejects a non-finite destination
        // (gemv.rs:126-127): record the step after which it first appeared.
        if (a.check && bad >= 0 && bad < last)
            atomicMin(&a.status->first_bad_fold, ((unsigned long long)bad << 32) | (unsigned)(r0 + t));
    }
}

__global__ void k_moe_reset_status(MoeStatus *st) {
    if (threadIdx.x == 0) {
        st->first_bad_swiglu = ~0ull;
        st->first_bad_fold = ~0ull;
        st->first_bad_input = ~0ull;
        st->pad = 0;
    }
}

// Diagnostics: the device expf (swiglu == 0) or SwiGLU element (swiglu != 0).
__global__ void k_expf(const float *in, float *out, long long n, int swiglu, const float *up) {
    for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long long)gridDim.x * blockDim.x)
        out[i] = swiglu ? swiglu_ref(in[i], up[i]) : expf_libm(in[i]);
}

// ---------------------------------------------------------------- launchers

static inline int cdiv(long long a, long long b) { return (int)((a + b - 1) / b); }

// Type combinations with a fused instantiation: routed gate/up IQ2_S with a
// Q4_K or IQ2_S shared expert; routed down IQ3_S or IQ2_S with a Q5_K, IQ3_S
// or IQ2_S shared down.  Lanes per unit: 2 for IQ types, 4 for K-quants.
template <int TY>
constexpr int moe_lpu() {
    return Traits<TY>::KQ ? 4 : 2;
}

template <int TYR, int TYS>
static hipError_t gate_up_typed(const MoeArgs &a, hipStream_t s) {
    const int nb = a.hidden / 256;
    const int lds = gate_up_lds<TYR>(nb) > gate_up_lds<TYS>(nb) ? gate_up_lds<TYR>(nb) : gate_up_lds<TYS>(nb);
    const int grid = (a.has_shared ? a.tiles_s : 0) + a.n_launch * a.tiles_r;
    if (grid <= 0) return hipSuccess;
    hipLaunchKernelGGL((k_moe_gate_up<TYR, moe_lpu<TYR>(), TYS, moe_lpu<TYS>()>), dim3(grid), dim3(MOE_THREADS), lds, s,
                       a);
    return hipGetLastError();
}

template <int TYR, int TYS>
static hipError_t down_typed(const MoeArgs &a, hipStream_t s) {
    const int n = a.route_dev ? MOE_MAX_ROUTED : a.route.n;
    const int nbr = a.ffn_r / 256, nbs = a.ffn_s / 256;
    const int lds = align16(GridLDS<TYR>::BYTES) + align16(TYS == TYR ? 0 : GridLDS<TYS>::BYTES) +
                    align16((n * nbr + (a.has_shared ? nbs : 0)) * 292) + MOE_WAVES * down_fold_bytes<TYR, TYS>() +
                    (MOE_MAX_ROUTED + 1) * a.tile_d * 4;
    hipLaunchKernelGGL((k_moe_down<TYR, moe_lpu<TYR>(), TYS, moe_lpu<TYS>()>), dim3(cdiv(a.hidden, a.tile_d)),
                       dim3(MOE_THREADS), lds, s, a);
    return hipGetLastError();
}

hipError_t launch_moe_gate_up(const MoeArgs &a, hipStream_t s) {
    const int tyr = a.type_gate_r;
    const int ts = a.has_shared ? a.shared.gate.type : tyr;
    if (tyr == T_IQ2_S && ts == T_Q4_K) return gate_up_typed<T_IQ2_S, T_Q4_K>(a, s);
    if (tyr == T_IQ2_S && ts == T_IQ2_S) return gate_up_typed<T_IQ2_S, T_IQ2_S>(a, s);
    return hipErrorInvalidValue;
}

hipError_t launch_moe_down(const MoeArgs &a, hipStream_t s) {
    const int tyr = a.type_down_r;
    const int ts = a.has_shared ? a.shared.down.type : tyr;
    if (tyr == T_IQ3_S && ts == T_Q5_K) return down_typed<T_IQ3_S, T_Q5_K>(a, s);
    if (tyr == T_IQ3_S && ts == T_IQ3_S) return down_typed<T_IQ3_S, T_IQ3_S>(a, s);
    if (tyr == T_IQ2_S && ts == T_IQ2_S) return down_typed<T_IQ2_S, T_IQ2_S>(a, s);
    if (tyr == T_IQ2_S && ts == T_IQ3_S) return down_typed<T_IQ2_S, T_IQ3_S>(a, s);
    return hipErrorInvalidValue;
}

hipError_t launch_moe_reset_status(MoeStatus *st, hipStream_t s) {
    hipLaunchKernelGGL(k_moe_reset_status, dim3(1), dim3(64), 0, s, st);
    return hipGetLastError();
}

hipError_t launch_expf(const float *in, float *out, long long n, int swiglu, const float *up, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    int grid = cdiv(n, 256);
    grid = grid > 8192 ? 8192 : grid;
    hipLaunchKernelGGL(k_expf, dim3(grid), dim3(256), 0, s, in, out, n, swiglu, up);
    return hipGetLastError();
}

}  // namespace lbh
