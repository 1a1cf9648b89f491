// lbh_moe.hip — the routed + shared SwiGLU expert FFN of one token
// (moe_routed_by_id_into, crates/bridge-kernels-reference/src/moe.rs:64-147)
// in two launches:
//
//   k_moe_gate_up  one workgroup per (expert, tile of hidden rows): Q8_K(x) into
//                  LDS, gate and up row dots of the tile, SwiGLU with the
//                  libm-exact expf (activation.rs:170-178), h to scratch;
//   k_moe_down     one workgroup per tile of output rows: Q8_K of every
//                  expert's h into LDS, the down row dots of
//                  every routed expert and of the shared expert, then each row
//                  is combined in the reference order
//                      y = ((0 + c_0 d_0) + c_1 d_1) + ... + 1.0 * d_shared
//                  (gemv_accumulate_scaled_into, gemv.rs:161-171, moe.rs:141-146).
//
// The result is bit-identical to the reference: the same Q8_K bytes, integer
// block sums, per-row folds, SwiGLU and accumulation order.  Data moves
// between workgroups only across kernel boundaries: an agent-scope fence
// inside a kernel writes back and invalidates the whole L2 of the XCD, which
// measured slower than an extra launch.
#include "lbh_internal.h"
#include "lbh_math.h"
#include "lbh_rows.h"
#include "lbh_router.h"

namespace lbh {

constexpr int MOE_THREADS = 256;
constexpr int MOE_WAVES = MOE_THREADS / 64;

__host__ __device__ constexpr int align16(int v) { return (v + 15) & ~15; }

__device__ __forceinline__ int route_n(const MoeArgs &a) { return a.route_dev ? a.route_dev->n : a.route.n; }
// A wave-uniform read of memory that no wave of the running kernel writes,
// through the constant address space: a scalar load.  (Through a generic
// pointer it is a vector load, and the wait for it drains every load the
// wave has in flight.)
template <class T>
__device__ __forceinline__ T scalar_read(const T *p) {
    static_assert(sizeof(T) % 4 == 0, "whole words");
    T v;
    uint32_t *d = reinterpret_cast<uint32_t *>(&v);
    const __attribute__((address_space(4))) uint32_t *w = (const __attribute__((address_space(4))) uint32_t *)p;
#pragma unroll
    for (int i = 0; i < (int)(sizeof(T) / 4); ++i) d[i] = w[i];
    return v;
}
// Stands in for absent status words (no non-finite value recorded).
__device__ const unsigned long long k_no_status[2] = {~0ull, ~0ull};
__device__ __forceinline__ uint32_t route_id(const MoeArgs &a, int s) {
    return a.route_dev ? a.route_dev->ids[s] : a.route.ids[s];
}
// A matrix view the compiler may treat as divergent (read from LDS or
// indexed by a wave-dependent slot) but that is the same in every lane of
// the wave: take lane 0's copy, so the buffer descriptor built from it lives
// in SGPRs (a divergent descriptor turns every load into a readfirstlane
// loop).
// (readfirstlane returns a signed int: each half goes through uint32_t so
// the low half does not sign-extend into the high one.)
__device__ __forceinline__ uint64_t uniform_u64(uint64_t v) {
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(v >> 32));
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)v);
    return ((uint64_t)hi << 32) | (uint64_t)lo;
}
__device__ __forceinline__ MatView uniform_view(const MatView &v) {
    MatView u;
    u.planes = reinterpret_cast<const uint8_t *>(uniform_u64(reinterpret_cast<uint64_t>(v.planes)));
    u.type = __builtin_amdgcn_readfirstlane(v.type);
    u.nb = __builtin_amdgcn_readfirstlane(v.nb);
    u.rows = __builtin_amdgcn_readfirstlane(v.rows);
    u.order = MAT_ROW_MAJOR;
    u.units = (long long)uniform_u64((uint64_t)v.units);
    u.bytes = (long long)uniform_u64((uint64_t)v.bytes);
    return u;
}

// Views of the routed expert in routing slot s (wave-uniform): from the
// arguments when the host gave the routing (scalar loads of the argument
// segment), else from the device table.
__device__ __forceinline__ ExpertDev routed_view(const MoeArgs &a, int s) {
    const int su = __builtin_amdgcn_readfirstlane(s);
    if (!a.routed_given) {
        // Device route (read only by launches that do not write it) and the
        // expert table: scalar loads.
        const uint32_t id = a.route_dev ? scalar_read(&a.route_dev->ids[su]) : a.route.ids[su];
        return scalar_read(&a.experts[__builtin_amdgcn_readfirstlane((int)id)]);
    }
    // The shape and the slot's plane pointers are read from the
    // kernel-argument segment through its own pointer (MoeArgs is the
    // launch's only argument, at offset 0): a copy of the by-value argument's
    // shape, then modified, made the compiler keep a private copy of it, and
    // a kernel that declares a private segment has its workgroups' launch
    // limited by the scratch allocation.
    using KBytes = const __attribute__((address_space(4))) uint8_t *;
    using KPtr = const __attribute__((address_space(4))) uint64_t *;
    const KBytes args = (KBytes)__builtin_amdgcn_kernarg_segment_ptr();
    const KPtr rp = (KPtr)(args + __builtin_offsetof(MoeArgs, routed_planes)) + 3 * su;
    ExpertDev v = scalar_read((const ExpertDev *)(args + __builtin_offsetof(MoeArgs, routed_shape)));
    v.gate.planes = reinterpret_cast<const uint8_t *>(rp[0]);
    v.up.planes = reinterpret_cast<const uint8_t *>(rp[1]);
    v.down.planes = reinterpret_cast<const uint8_t *>(rp[2]);
    return v;
}
__device__ __forceinline__ float route_coef(const MoeArgs &a, int s) {
    return a.route_dev ? a.route_dev->coefs[s] : a.route.coefs[s];
}

// Rows whose gate and up dots a wave has finished, waiting for SwiGLU: the
// exponential runs once per 64 rows with every lane busy instead of once per
// row step in the step's few leader lanes.
constexpr int SWIGLU_BATCH = 64;
struct PendingRows {
    float g[SWIGLU_BATCH], u[SWIGLU_BATCH];
    int32_t row[SWIGLU_BATCH];
    int32_t tag[SWIGLU_BATCH];   // scratch slot | (expert order << 8)
};

// Dynamic LDS bytes of one gate/up workgroup of type TY (the codebook is a
// static array, static_grid).
template <int TY>
__host__ __device__ constexpr int gate_up_lds(int nb) {
    return align16(nb * 292) + MOE_WAVES * (int)sizeof(FoldLDS<TY>) + MOE_WAVES * (int)sizeof(PendingRows);
}

// h = SwiGLU(gate, up) (activation.rs:170-178) of a wave's n pending rows, one
// lane per row; a non-finite h is recorded (first by expert order, then lane).
__device__ __forceinline__ void flush_swiglu(const MoeArgs &a, PendingRows &pr, int n) {
    wave_sync();
    const int lane = threadIdx.x & 63;
    if (lane < n && pr.row[lane] >= 0) {
        const int tag = pr.tag[lane], r = pr.row[lane];
        const float hv = swiglu_ref(pr.g[lane], pr.u[lane]);
        a.h[(long long)(tag & 0xff) * a.h_stride + r] = hv;
        if (a.check && !isfinite(hv))
            atomicMin(&a.status->first_bad_swiglu, ((unsigned long long)(tag >> 8) << 32) | (unsigned)r);
    }
    wave_sync();
}

// Gate and up rows of `count` experts of one type, SwiGLU into h.  The
// workgroup's waves walk the flattened (slot, row step) items of all of them
// with a stride of `nwaves`: Q8_K(x) stays in registers (the same input for
// every expert), the codebook is filled once per workgroup, and the next
// item's weights are loaded while the current item is computed.
template <int TY, int LPU, class SlotOf>
__device__ __forceinline__ void gate_up_stream(const MoeArgs &a, const SlotOf &slot_of, int count, int rows,
                                               int first_wave, int nwaves, uint8_t *smem) {
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    const int NB = a.hidden / 256;
    uint8_t *s_grid = static_grid<TY>();
    uint8_t *s_q8 = smem;
    FoldLDS<TY> *s_fold = reinterpret_cast<FoldLDS<TY> *>(s_q8 + align16(NB * 292));
    PendingRows &pend = reinterpret_cast<PendingRows *>(s_fold + MOE_WAVES)[wid];

    const LaneMap<LPU> L(lane, NB);
    const int per = (rows + L.rpw - 1) / L.rpw;
    const int items = count * per;
    using W = WOf<TY, LPU>;
    // Items walk with a stride of nwaves: (m, j) = (it / per, it % per) is
    // advanced by adding the stride's quotient and remainder (no division per item).
    const int dq = nwaves / per, dr = nwaves - dq * per;
    auto advance = [&](int &m, int &j) {
        m += dq, j += dr;
        if (j >= per) j -= per, m += 1;
    };
    // item (m, j) -> (slot index, expert views, row)
    auto issue = [&](int it, int m, int j, W &wg, W &wu) {
        if (it >= items) return;
        const int r = j * L.rpw + L.slot;
        if (!(L.lane_on && r < rows)) return;
        const MatView VG = uniform_view(slot_of(m).gate), VU = uniform_view(slot_of(m).up);
        const Planes PG = make_planes(VG.planes, VG.units, VG.bytes);
        const Planes PU = make_planes(VU.planes, VU.units, VU.bytes);
        const uint32_t po = part_offset<TY, LPU>(PG, L.part);
        const uint32_t u = (uint32_t)(r * NB + L.b);
        load_slice(PG, u, po, L.part, wg);
        load_slice(PU, u, po, L.part, wu);
    };
    // Prologue loads (codebook, this wave's first chunk of x) go out before
    // the first weight loads, so they do not wait behind the weight burst.
    // The first weight load is unconditional (item and row clamped into
    // range) so the wait before the prologue's stores counts exactly the
    // weight loads issued after it.
    int it = first_wave + wid;
    int im = it / per, ij = it - im * per;   // the wave's current item as (m, j)
    const GridIn<TY> gin = grid_load<TY>();
    const QuantIn qin = quantize_load(a.x, 4 * wid, NB);
    W ga, ua, gb, ub;
    {
        const int itc = it < items ? it : items - 1;
        const int m = itc / per, j = itc - m * per;
        int r = j * L.rpw + (L.lane_on ? L.slot : L.rpw - 1);
        r = r < rows ? r : rows - 1;
        const MatView VG = uniform_view(slot_of(m).gate), VU = uniform_view(slot_of(m).up);
        const Planes PG = make_planes(VG.planes, VG.units, VG.bytes);
        const Planes PU = make_planes(VU.planes, VU.units, VU.bytes);
        const uint32_t po = part_offset<TY, LPU>(PG, L.part);
        const uint32_t u = (uint32_t)(r * NB + L.b);
        load_slice(PG, u, po, L.part, ga);
        load_slice(PU, u, po, L.part, ua);
    }

    grid_store<TY>(gin, s_grid);
    quantize_store(qin, s_q8);
    for (int b0 = 4 * wid + 4 * MOE_WAVES; b0 < NB; b0 += 4 * MOE_WAVES) quantize_blocks_wave(a.x, s_q8, b0, NB);
    __syncthreads();
    ActOf<TY, LPU> act;
    load_act(s_q8 + L.b * 292, L.part, act);

    int npend = 0;   // wave-uniform count of pending rows
    auto process = [&](int m, int j, const W &wg, const W &wu) {
        const int r = j * L.rpw + L.slot;
        const bool on = L.lane_on && r < rows;
        const float gv = row_dot<TY, LPU>(wg, act, on, L, s_grid, s_fold[wid], nullptr, 0);
        const float uv = row_dot<TY, LPU>(wu, act, on, L, s_grid, s_fold[wid], nullptr, 0);
        if (npend + L.rpw > SWIGLU_BATCH) {
            flush_swiglu(a, pend, npend);
            npend = 0;
        }
        if (L.lane_on && L.leader()) {
            const int k = npend + L.slot;
            pend.g[k] = gv, pend.u[k] = uv;
            pend.row[k] = on ? r : -1;   // -1: a row past the matrix, nothing to store
            pend.tag[k] = slot_of.slot(m) | (slot_of.order(m) << 8);
        }
        npend += L.rpw;
    };
    while (it < items) {
        int m2 = im, j2 = ij;
        advance(m2, j2);
        issue(it + nwaves, m2, j2, gb, ub);
        process(im, ij, ga, ua);
        it += nwaves, im = m2, ij = j2;
        if (it >= items) break;
        advance(m2, j2);
        issue(it + nwaves, m2, j2, ga, ua);
        process(im, ij, gb, ub);
        it += nwaves, im = m2, ij = j2;
    }
    if (npend > 0) flush_swiglu(a, pend, npend);
}

// Routed experts of one launch: their gate/up views staged in LDS by the
// workgroup prologue (a per-item lookup through the device table would put
// dependent scalar loads in front of every item's weight loads).
struct RoutedSlots {
    const ExpertDev *views;   // LDS: [n] (gate, up) views; down unused here
    __device__ const ExpertDev &operator()(int m) const { return views[m]; }
    __device__ int slot(int m) const { return m; }
    __device__ int order(int m) const { return m; }
};
// Host-given routing: the views come from the arguments per item (slot m is
// wave-uniform), with no staging of ids or views in the prologue.
struct GivenSlots {
    const MoeArgs &a;
    __device__ ExpertDev operator()(int m) const { return routed_view(a, m); }
    __device__ int slot(int m) const { return m; }
    __device__ int order(int m) const { return m; }
};
struct SharedSlot {
    const MoeArgs &a;
    int n;
    __device__ const ExpertDev &operator()(int) const { return a.shared; }
    __device__ int slot(int) const { return MOE_SHARED_SLOT; }
    __device__ int order(int) const { return n; }
};

// Records a rejected selection for lbh_router_take_status: the count, and the
// first rejection's code and its logit and bias bits.
__device__ __forceinline__ void note_rejection(const RouterArgs &r, unsigned long long bad) {
    if (atomicAdd(r.reject, 1ull) == 0) {
        const int e = (int)(bad >> 2);
        const unsigned long long lb = __float_as_uint(r.logits[e]);
        const unsigned long long bb = r.mode == 1 ? __float_as_uint(r.bias[e]) : 0u;
        r.reject[1] = bad;
        r.reject[2] = lb | (bb << 32);
    }
}

// Workgroups [0, wg_s) stream the shared expert, the rest the routed experts.
template <int TYR, int LPUR, int TYS, int LPUS>
__global__ void __launch_bounds__(MOE_THREADS) k_moe_gate_up(MoeArgs a) {
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ uint32_t s_ids[MOE_MAX_ROUTED];
    __shared__ ExpertDev s_views[MOE_MAX_ROUTED];
    if (a.status && a.status->first_bad_input != ~0ull) return;
    const int wg_s = a.has_shared && !a.skip_shared_gate_up && a.gate_part != 1 ? a.tiles_s : 0;
    if ((int)blockIdx.x < wg_s) {
        const int n = a.route_dev && !a.select_in_kernel ? a.route_dev->n : a.route.n;
        gate_up_stream<TYS, LPUS>(a, SharedSlot{a, n}, 1, a.ffn_s, blockIdx.x * MOE_WAVES, wg_s * MOE_WAVES, smem);
        return;
    }
    const int wg_r = gridDim.x - wg_s;
    if (a.routed_given) {
        gate_up_stream<TYR, LPUR>(a, GivenSlots{a}, a.n_launch, a.ffn_r, (blockIdx.x - wg_s) * MOE_WAVES,
                                  wg_r * MOE_WAVES, smem);
        return;
    }
    if (a.select_in_kernel) {
        // Every workgroup selects the same route from the finished logits;
        // workgroup wg_s publishes it for the down kernel.
        // A non-finite logit (or a router chain that gave up) makes the route
        // invalid: it is published with n = -1, nothing is computed and the
        // down kernel leaves y unchanged.
        __shared__ int s_invalid;
        if (threadIdx.x < 64) {
            MoeRoute r;
            unsigned long long bad;
            select_route(a.router, r, bad);
            if (bad != ~0ull) r.n = -1;
            if (threadIdx.x == 0) {
#pragma unroll
                for (int q = 0; q < MOE_MAX_ROUTED; ++q) s_ids[q] = r.ids[q];
                s_invalid = bad != ~0ull;
                if ((int)blockIdx.x == wg_s) {
                    *const_cast<MoeRoute *>(a.route_dev) = r;
                    if (bad != ~0ull && a.router.reject) note_rejection(a.router, bad);
                }
            }
        }
        __syncthreads();
        if (s_invalid) return;
    } else if (threadIdx.x < MOE_MAX_ROUTED) {
        s_ids[threadIdx.x] = route_id(a, threadIdx.x < route_n(a) ? threadIdx.x : 0);
    }
    __syncthreads();
    if (threadIdx.x < a.n_launch) s_views[threadIdx.x] = a.experts[s_ids[threadIdx.x]];
    __syncthreads();
    gate_up_stream<TYR, LPUR>(a, RoutedSlots{s_views}, a.n_launch, a.ffn_r, (blockIdx.x - wg_s) * MOE_WAVES,
                              wg_r * MOE_WAVES, smem);
}

// Block decode, first launch: router chains (RT_EXPERTS experts per
// workgroup, in the first workgroups) beside the shared expert's gate/up
// stream, which does not depend on the routing.
template <int TYS, int LPUS>
__global__ void __launch_bounds__(MOE_THREADS) k_moe_router_shared(MoeArgs a) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int rw = (a.router.n_experts + RT_EXPERTS - 1) / RT_EXPERTS;
    if ((int)blockIdx.x < rw) {
        router_chain_wg(a.router, blockIdx.x * RT_EXPERTS, smem);
        return;
    }
    gate_up_stream<TYS, LPUS>(a, SharedSlot{a, a.route.n}, 1, a.ffn_s, (blockIdx.x - rw) * MOE_WAVES,
                              a.tiles_s * MOE_WAVES, smem);
}

// Down projections and the ordered combine for output rows [r0, r0 + tile_d).
// Waves 0..n-1 take routed expert m = wave (its Q8_K(h) slice in registers),
// waves n.. share the shared expert's rows; the row dots meet in LDS and one
// lane per row accumulates them in the reference order
//     y = ((0 + c_0 d_0) + c_1 d_1) + ... + 1.0 * d_shared   (moe.rs:141-146).
template <int TY, int LPU>
struct DownStream {
    using W = WOf<TY, LPU>;
    Planes P;
    int nb, r0, r1, it, stride;
    W wa, wb;

    __device__ __forceinline__ void issue(const LaneMap<LPU> &L, uint32_t po, int items, int i, W &w) const {
        const int r = r0 + i * L.rpw + L.slot;
        if (i < items && L.lane_on && r < r1) load_slice(P, (uint32_t)(r * nb + L.b), po, L.part, w);
    }
    // The stream's views and its first step's weight loads: callable before
    // the workgroup's prologue, so that HBM round trip overlaps it.
    __device__ __forceinline__ void start(const MatView &Vd, int nb_, int r0_, int r1_, int first, int stride_) {
        nb = nb_, r0 = r0_, r1 = r1_, it = first, stride = stride_;
        const MatView V = uniform_view(Vd);
        P = make_planes(V.planes, V.units, V.bytes);
        const LaneMap<LPU> L(threadIdx.x & 63, nb);
        issue(L, part_offset<TY, LPU>(P, L.part), (r1 - r0 + L.rpw - 1) / L.rpw, it, wa);
    }
    __device__ __forceinline__ void run(const uint8_t *q8, const void *s_grid, FoldLDS<TY> &fold, float *s_y) {
        const LaneMap<LPU> L(threadIdx.x & 63, nb);
        const uint32_t po = part_offset<TY, LPU>(P, L.part);
        const int items = (r1 - r0 + L.rpw - 1) / L.rpw;
        ActOf<TY, LPU> act;
        load_act(q8 + L.b * 292, L.part, act);
        auto process = [&](int i, const W &w) {
            const int r = r0 + i * L.rpw + L.slot;
            const bool on = L.lane_on && r < r1;
            const float v = row_dot<TY, LPU, 0, Traits<TY>::KQ ? 16 : 8>(w, act, on, L, s_grid, fold, nullptr, 0);
            if (on && L.leader()) s_y[r - r0] = v;
        };
        while (it < items) {
            issue(L, po, items, it + stride, wb);
            process(it, wa);
            it += stride;
            if (it >= items) break;
            issue(L, po, items, it + stride, wa);
            process(it, wb);
            it += stride;
        }
    }
};

template <int TY, int LPU>
__device__ __forceinline__ void down_wave(const MatView &Vd, const uint8_t *q8, int nb, int r0, int r1, int first,
                                          int stride, const void *s_grid, FoldLDS<TY> &fold, float *s_y) {
    DownStream<TY, LPU> d;
    d.start(Vd, nb, r0, r1, first, stride);
    d.run(q8, s_grid, fold, s_y);
}

template <int TYR, int TYS>
__host__ __device__ constexpr int down_fold_bytes() {
    return (int)sizeof(FoldLDS<TYR>) > (int)sizeof(FoldLDS<TYS>) ? (int)sizeof(FoldLDS<TYR>) : (int)sizeof(FoldLDS<TYS>);
}

constexpr int DOWN_SHARED_WAVES = 4;

constexpr int DOWN_MAX_WAVES = 12;

template <int TYR, int LPUR, int TYS, int LPUS>
__global__ void __launch_bounds__(64 * DOWN_MAX_WAVES) k_moe_down(MoeArgs a) {
    extern __shared__ __align__(16) uint8_t smem[];
    // The device route count is a scalar read (an unconditional load from a
    // selected address: a load inside a branch is waited for inside it); the
    // status words are read once the prologue's loads are out and acted on
    // after it (a non-finite input or SwiGLU, or an invalid device route,
    // leaves y unchanged), so no wait for them holds back a prologue load.
    const int route_count = a.route_dev ? scalar_read(&a.route_dev->n) : a.route.n;
    // Wave index and route count through readfirstlane: the task choice below
    // (and every descriptor derived from it) is wave-uniform.
    const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n = a.down_part == 2 || route_count < 0 ? 0 : __builtin_amdgcn_readfirstlane(route_count);
    // The shared expert's down runs here unless another launch writes it to d_shared (part 1).
    const bool shared_here = a.has_shared && a.down_part != 1;
    const int nbr = a.ffn_r / 256, nbs = a.ffn_s / 256;
    const int r0 = blockIdx.x * a.tile_d;
    const int r1 = r0 + a.tile_d < a.hidden ? r0 + a.tile_d : a.hidden;
    uint8_t *s_grid_r = static_grid<TYR>();
    uint8_t *s_grid_s = static_grid<TYS>();
    uint8_t *s_foldp = smem;
    const int nw = blockDim.x >> 6;
    float *s_y = reinterpret_cast<float *>(s_foldp + nw * down_fold_bytes<TYR, TYS>());
    uint8_t *s_q8 = reinterpret_cast<uint8_t *>(s_y + (MOE_MAX_ROUTED + 1) * a.tile_d);   // [n * nbr + nbs] blocks

    // Q8_K of every expert's h into LDS (quantize_row_q8_k_into of the down
    // projection's input, gemv.rs:161-163): chunks of up to four blocks of one
    // slot.  Order: the codebooks and the h of the wave's first two chunks,
    // a wait for them, the first weight step of the wave's first task
    // (routed expert `wid`, or its part of the shared expert), then the LDS
    // stores and the quantization, which overlap that step's HBM round trip.
    // A wave's first two chunks (wid, wid + nw) are straight-line code, their
    // indices clamped (an in-range reload), so no wait separates their loads;
    // chunks past 2 nw (more than eight routed experts) follow one at a time.
    const int tasks = n + (shared_here ? DOWN_SHARED_WAVES : 0);
    const bool first_routed = wid < n, first_shared = !first_routed && wid < tasks;
    DownStream<TYR, LPUR> d_r;
    DownStream<TYS, LPUS> d_s;
    unsigned long long bad_input, bad_swiglu;
    {
        const GridIn<TYR> gin_r = grid_load<TYR>();
        const GridIn<TYS> gin_s = grid_load<TYS>();
        const int cr = (nbr + 3) / 4, cs = (nbs + 3) / 4;
        const int chunks = n * cr + (shared_here ? cs : 0);
        auto chunk = [&](int c, const float *&x, uint8_t *&out, int &b0, int &nbl) {
            if (c < n * cr) {
                const int m = c / cr;
                b0 = 4 * (c - m * cr);
                x = a.h + (long long)m * a.h_stride;
                out = s_q8 + m * nbr * 292;
                nbl = nbr;
            } else {
                b0 = 4 * (c - n * cr);
                x = a.h + (long long)MOE_SHARED_SLOT * a.h_stride;
                out = s_q8 + n * nbr * 292;
                nbl = nbs;
            }
        };
        const int last = chunks > 0 ? chunks - 1 : 0;
        const float *x0, *x1;
        uint8_t *o0, *o1;
        int b0, b1, n0, n1;
        chunk(wid < last ? wid : last, x0, o0, b0, n0);
        chunk(wid + nw < last ? wid + nw : last, x1, o1, b1, n1);
        const QuantIn q0 = quantize_load(x0, b0, chunks > 0 ? n0 : 0);
        const QuantIn q1 = quantize_load(x1, b1, chunks > 0 ? n1 : 0);
        // vmcnt(0): the codebook and h land before the first weight step goes
        // out.  The weight loads differ by wave role, so a store that waited
        // for an older load behind them would wait for all of them; this way
        // the quantization runs while the weights are in flight.
        __builtin_amdgcn_s_waitcnt(0x0F70);
        if (first_routed)
            d_r.start(routed_view(a, wid).down, nbr, r0, r1, 0, 1);
        else if (first_shared)
            d_s.start(a.shared.down, nbs, r0, r1, wid - n, DOWN_SHARED_WAVES);
        bad_input = scalar_read(a.status ? &a.status->first_bad_input : &k_no_status[0]);
        bad_swiglu = scalar_read(a.status ? &a.status->first_bad_swiglu : &k_no_status[1]);
        grid_store<TYR>(gin_r, s_grid_r);
        if (TYS != TYR) grid_store<TYS>(gin_s, s_grid_s);
        if (wid < chunks) quantize_store(q0, o0);
        if (wid + nw < chunks) quantize_store(q1, o1);
        for (int c = wid + 2 * nw; c < chunks; c += nw) {
            const float *x;
            uint8_t *o;
            int b, nbl;
            chunk(c, x, o, b, nbl);
            quantize_store(quantize_load(x, b, nbl), o);
        }
    }
    __syncthreads();
    if (bad_input != ~0ull || bad_swiglu != ~0ull || (a.route_dev && route_count < 0)) return;

    // Tasks: routed experts 0..n-1, then DOWN_SHARED_WAVES interleaved parts of
    // the shared expert; wave w takes tasks w, w + nw, ... (the first one
    // started before the prologue).
    const int ystride = a.tile_d;
    FoldLDS<TYR> &fold_r = *reinterpret_cast<FoldLDS<TYR> *>(s_foldp + wid * down_fold_bytes<TYR, TYS>());
    FoldLDS<TYS> &fold_s = *reinterpret_cast<FoldLDS<TYS> *>(s_foldp + wid * down_fold_bytes<TYR, TYS>());
    if (first_routed)
        d_r.run(s_q8 + wid * nbr * 292, s_grid_r, fold_r, s_y + wid * ystride);
    else if (first_shared)
        d_s.run(s_q8 + n * nbr * 292, TYS == TYR ? s_grid_r : s_grid_s, fold_s, s_y + n * ystride);
    for (int t = wid + nw; t < tasks; t += nw) {
        if (t < n) {
            down_wave<TYR, LPUR>(routed_view(a, t).down, s_q8 + t * nbr * 292, nbr, r0, r1, 0, 1,
                                 s_grid_r,
                                 *reinterpret_cast<FoldLDS<TYR> *>(s_foldp + wid * down_fold_bytes<TYR, TYS>()),
                                 s_y + t * ystride);
        } else {
            down_wave<TYS, LPUS>(a.shared.down, s_q8 + n * nbr * 292, nbs, r0, r1, t - n,
                                 DOWN_SHARED_WAVES, TYS == TYR ? s_grid_r : s_grid_s,
                                 *reinterpret_cast<FoldLDS<TYS> *>(s_foldp + wid * down_fold_bytes<TYR, TYS>()),
                                 s_y + n * ystride);
        }
    }
    __syncthreads();

    // The shared expert's raw down rows for the combine of another launch.
    if (a.down_part == 2) {
        for (int t = threadIdx.x; t < r1 - r0; t += blockDim.x) a.d_shared[r0 + t] = s_y[t];
        return;
    }
    // Ordered combine: output.fill(0), then dest += coef * dot per expert in
    // ascending id order, then the shared expert at 1.0 (moe.rs:141-146).
    const int last = a.has_shared ? n : n - 1;
    for (int t = threadIdx.x; t < r1 - r0; t += blockDim.x) {
        float acc = 0.0f;
        int bad = -1;
        for (int s = 0; s < n && s <= a.stop_step; ++s) {
            acc = __fadd_rn(acc, __fmul_rn(route_coef(a, s), s_y[s * ystride + t]));
            if (bad < 0 && !isfinite(acc)) bad = s;
        }
        if (a.has_shared && n <= a.stop_step)
            acc = __fadd_rn(acc, __fmul_rn(1.0f, shared_here ? s_y[n * ystride + t] : a.d_shared[r0 + t]));
        a.y[r0 + t] = a.residual ? __fadd_rn(a.y[r0 + t], acc) : acc;
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
// or IQ2_S shared down.  Two lanes per (row, block) unit.
template <int TY>
constexpr int moe_lpu() {
    return TY == T_Q5_K ? 4 : 2;
}

template <int TYR, int TYS>
static hipError_t gate_up_typed(const MoeArgs &a, hipStream_t s) {
    const int nb = a.hidden / 256;
    const int lds = gate_up_lds<TYR>(nb) > gate_up_lds<TYS>(nb) ? gate_up_lds<TYR>(nb) : gate_up_lds<TYS>(nb);
    // tiles_s / tiles_r: workgroups of the shared / routed streams; when the
    // shared expert already ran (block decode) the routed stream takes both.
    const bool shared_here = a.has_shared && !a.skip_shared_gate_up && a.gate_part != 1;
    const bool routed_here = a.n_launch > 0 && a.gate_part != 2;
    const int grid = (shared_here ? a.tiles_s : 0) +
                     (routed_here ? a.tiles_r + (a.skip_shared_gate_up ? a.tiles_s : 0) : 0);
    if (grid <= 0) return hipSuccess;
    hipLaunchKernelGGL((k_moe_gate_up<TYR, moe_lpu<TYR>(), TYS, moe_lpu<TYS>()>), dim3(grid), dim3(MOE_THREADS), lds, s,
                       a);
    return hipGetLastError();
}

// Static LDS of a down launch: the codebooks (static_grid).
template <int TYR, int TYS>
constexpr int down_grid_lds() {
    return align16(GridLDS<TYR>::BYTES) + align16(TYS == TYR ? 0 : GridLDS<TYS>::BYTES);
}

// Waves of a down workgroup: one per routed expert, DOWN_SHARED_WAVES for the
// shared expert when its down runs in the launch, at most DOWN_MAX_WAVES and
// at least four, because grid_load spreads a codebook over the first 256
// threads of the workgroup (waves past the task count take part in the
// prologue only).
static int down_waves(int n, int has_shared) {
    const int waves = n + (has_shared ? DOWN_SHARED_WAVES : 0);
    return waves < 4 ? 4 : waves > DOWN_MAX_WAVES ? DOWN_MAX_WAVES : waves;
}

// LDS of a down launch over n routed experts: the codebooks (static), then,
// dynamic, one fold table per wave, the per-row down outputs of every expert
// and the Q8_K of every expert's h.
template <int TYR, int TYS>
static int down_lds(int n, int has_shared, int ffn_r, int ffn_s, int tile_d) {
    // (has_shared: the shared expert's down runs in this launch)
    const int nw = down_waves(n, has_shared);
    const int q8 = (n * (ffn_r / 256) + (has_shared ? ffn_s / 256 : 0)) * 292;
    return down_grid_lds<TYR, TYS>() + nw * down_fold_bytes<TYR, TYS>() + (MOE_MAX_ROUTED + 1) * tile_d * 4 + align16(q8);
}

template <int TYR, int TYS>
static hipError_t down_typed(const MoeArgs &a, hipStream_t s) {
    const int n = a.down_part == 2 ? 0 : a.route_dev ? a.n_launch : a.route.n;
    const int shared_here = a.has_shared && a.down_part != 1;
    const int nw = down_waves(n, shared_here);
    const int lds = down_lds<TYR, TYS>(n, shared_here, a.ffn_r, a.ffn_s, a.tile_d);
    if (lds > MOE_MAX_LDS) return hipErrorInvalidValue;
    const int dyn = lds - down_grid_lds<TYR, TYS>();
    auto kernel = k_moe_down<TYR, moe_lpu<TYR>(), TYS, moe_lpu<TYS>()>;
    if (dyn > 64 * 1024) {
        const hipError_t e =
            hipFuncSetAttribute(reinterpret_cast<const void *>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize, dyn);
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(kernel, dim3(cdiv(a.hidden, a.tile_d)), dim3(64 * nw), dyn, s, a);
    return hipGetLastError();
}

int moe_down_lds_bytes(int type_down_r, int type_down_s, int n_routed, int has_shared, int ffn_r, int ffn_s,
                       int tile_d) {
    const int tyr = type_down_r, ts = has_shared ? type_down_s : type_down_r;
    if (tyr == T_IQ3_S && ts == T_Q5_K) return down_lds<T_IQ3_S, T_Q5_K>(n_routed, has_shared, ffn_r, ffn_s, tile_d);
    if (tyr == T_IQ3_S && ts == T_IQ3_S) return down_lds<T_IQ3_S, T_IQ3_S>(n_routed, has_shared, ffn_r, ffn_s, tile_d);
    if (tyr == T_IQ2_S && ts == T_IQ2_S) return down_lds<T_IQ2_S, T_IQ2_S>(n_routed, has_shared, ffn_r, ffn_s, tile_d);
    if (tyr == T_IQ2_S && ts == T_IQ3_S) return down_lds<T_IQ2_S, T_IQ3_S>(n_routed, has_shared, ffn_r, ffn_s, tile_d);
    return 0x7fffffff;
}

template <int TYR, int TYS>
static int gate_up_resident(int hidden) {
    const int nb = hidden / 256;
    const int lds = gate_up_lds<TYR>(nb) > gate_up_lds<TYS>(nb) ? gate_up_lds<TYR>(nb) : gate_up_lds<TYS>(nb);
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &n, k_moe_gate_up<TYR, moe_lpu<TYR>(), TYS, moe_lpu<TYS>()>, MOE_THREADS, lds) != hipSuccess || n < 1)
        n = 1;
    return n;
}

int moe_gate_up_resident_per_cu(int type_gate_r, int type_gate_s, int hidden) {
    if (type_gate_r == T_IQ2_S && type_gate_s == T_Q4_K) return gate_up_resident<T_IQ2_S, T_Q4_K>(hidden);
    if (type_gate_r == T_IQ2_S && type_gate_s == T_IQ2_S) return gate_up_resident<T_IQ2_S, T_IQ2_S>(hidden);
    return 1;
}

hipError_t launch_moe_router_shared(const MoeArgs &a, hipStream_t s) {
    const int nb = a.hidden / 256;
    const int rw = (a.router.n_experts + RT_EXPERTS - 1) / RT_EXPERTS;
    const int ts = a.shared.gate.type;
    const int grid = rw + a.tiles_s;
    const int lq = gate_up_lds<T_Q4_K>(nb) > RT_LDS ? gate_up_lds<T_Q4_K>(nb) : RT_LDS;
    const int li = gate_up_lds<T_IQ2_S>(nb) > RT_LDS ? gate_up_lds<T_IQ2_S>(nb) : RT_LDS;
    if (ts == T_Q4_K) {
        hipLaunchKernelGGL((k_moe_router_shared<T_Q4_K, moe_lpu<T_Q4_K>()>), dim3(grid), dim3(MOE_THREADS), lq, s, a);
    } else if (ts == T_IQ2_S) {
        hipLaunchKernelGGL((k_moe_router_shared<T_IQ2_S, moe_lpu<T_IQ2_S>()>), dim3(grid), dim3(MOE_THREADS), li, s, a);
    } else {
        return hipErrorInvalidValue;
    }
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
