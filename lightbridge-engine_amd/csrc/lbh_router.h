// lbh_router.h — top-k selection of one token from finished router logits,
// shared by the router kernels and the MoE gate/up prologue.
#pragma once
#include "lbh_internal.h"
#include "lbh_math.h"

namespace lbh {

__device__ __forceinline__ float sigmoid_ref(float v) { return 1.0f / (1.0f + expf_libm(-v)); }  // routing.rs:109-111

// Total order of selection keys: larger score first, then smaller id.
// Scores are finite (checked) floats; +0.0 and -0.0 compare equal as in f32.
__device__ __forceinline__ unsigned long long sel_key(float score, uint32_t id) {
    const float s = score == 0.0f ? 0.0f : score;        // -0.0 == +0.0
    uint32_t b = __float_as_uint(s);
    b = (b & 0x80000000u) ? ~b : (b | 0x80000000u);     // monotone float -> uint
    return ((unsigned long long)b << 32) | (0xffffffffu - id);
}

// Router chains of RT_EXPERTS experts [e0, e0 + RT_EXPERTS) by one
// 256-thread workgroup.  Wave 0 runs the chains (lane = expert); waves 1-3
// stream the weights into a ring of RT_SLOTS chunks in LDS (RT_STEPS steps of
// four inputs each), producer wave w owning the chunks congruent to w - 1
// mod 3.  Slots change hands through workgroup-scope release/acquire flags:
// ready[slot] = index of the chunk it holds, done = last chunk consumed.
// Each wait is bounded, so no wave can wait forever.  A wave whose wait gives
// up reports it: the consumer stores NaN logits (which the selection rejects
// as non-finite, routing.rs:72-77) and marks done as past every chunk so the
// producers stop waiting; a producer stops producing (the consumer's wait for
// its chunk then gives up too).  Either sets the sticky *timeout word.
constexpr int RT_EXPERTS = 8;
constexpr int RT_STEPS = 64;
constexpr int RT_SLOTS = 4;
constexpr int RT_LDS = RT_SLOTS * RT_STEPS * RT_EXPERTS * 16 + 64;

__device__ __forceinline__ int lds_acquire(const int *p) {
    return __hip_atomic_load(p, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ void lds_release(int *p, int v) {
    __hip_atomic_store(p, v, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
}

__device__ __forceinline__ void router_chain_wg(const RouterArgs &a, int e0, uint8_t *lds) {
    float4 *ring = reinterpret_cast<float4 *>(lds);
    int *ready = reinterpret_cast<int *>(lds + RT_SLOTS * RT_STEPS * RT_EXPERTS * 16);
    int *done = ready + RT_SLOTS;
    const int tid = threadIdx.x, wid = tid >> 6, lane = tid & 63;
    const int n = a.n_experts;
    const int nch = a.hidden / (4 * RT_STEPS);   // hidden is a multiple of 256
    // spin_limit < 0 forces every wait to give up (a deterministic test of that path).
    const bool force = a.spin_limit < 0;
    const long long SPIN = a.spin_limit > 0 ? a.spin_limit : force ? 0 : (1ll << 22);
    auto gave_up = [&]() {
        if (lane == 0 && a.timeout) __hip_atomic_store(a.timeout, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    };
    if (tid < RT_SLOTS) ready[tid] = -1;
    if (tid == 0) *done = -1;
    __syncthreads();

    // The chains are a latency floor of `hidden` dependent adds: their waves
    // take issue priority over whatever else shares the CU (the shared
    // expert's stream runs beside them), the chain above its producers.
    if (wid >= 1 && wid <= 3) {
        __builtin_amdgcn_s_setprio(2);
        const float4 *wt = reinterpret_cast<const float4 *>(a.w);
        const float4 *x4 = reinterpret_cast<const float4 *>(a.x);
        constexpr int PER = RT_STEPS * RT_EXPERTS / 64;
        struct ChunkRegs {
            float4 v[PER], xv[PER];
        };
        auto load = [&](int c, ChunkRegs &r) {
#pragma unroll
            for (int k = 0; k < PER; ++k) {
                const int idx = lane + 64 * k;
                const int step = idx / RT_EXPERTS, e = e0 + idx % RT_EXPERTS;
                r.v[k] = e < n ? wt[(long long)(c * RT_STEPS + step) * n + e] : make_float4(0.f, 0.f, 0.f, 0.f);
                r.xv[k] = x4[c * RT_STEPS + step];
            }
        };
        // Chunk c waits for its ring slot, then its products go to LDS.  The
        // wave's next chunk is loaded before that wait, so two chunks per
        // producer are in flight (the loads' latency, not the adds, set the
        // pace with one).  false: the wait gave up.
        auto publish = [&](int c, const ChunkRegs &r) {
            for (long long k = 0; k < SPIN && lds_acquire(done) < c - RT_SLOTS; ++k) __builtin_amdgcn_s_sleep(1);
            if (force || lds_acquire(done) < c - RT_SLOTS) {
                gave_up();
                return false;
            }
            // The ring holds the products w[i] * x[i] (each rounded once, as the
            // reference's `weight * input_value`), so the chain only adds.
            float4 *slot = ring + (c % RT_SLOTS) * RT_STEPS * RT_EXPERTS;
#pragma unroll
            for (int k = 0; k < PER; ++k) {
                float4 p;
                p.x = __fmul_rn(r.v[k].x, r.xv[k].x), p.y = __fmul_rn(r.v[k].y, r.xv[k].y);
                p.z = __fmul_rn(r.v[k].z, r.xv[k].z), p.w = __fmul_rn(r.v[k].w, r.xv[k].w);
                slot[lane + 64 * k] = p;
            }
            if (lane == 0) lds_release(&ready[c % RT_SLOTS], c);
            return true;
        };
        ChunkRegs ra, rb;
        int c = wid - 1;
        if (c < nch) load(c, ra);
        while (c < nch) {
            if (c + 3 < nch) load(c + 3, rb);
            if (!publish(c, ra)) break;
            c += 3;
            if (c >= nch) break;
            if (c + 3 < nch) load(c + 3, ra);
            if (!publish(c, rb)) break;
            c += 3;
        }
    } else if (wid == 0) {
        __builtin_amdgcn_s_setprio(3);
        const int l = lane < RT_EXPERTS ? lane : 0;
        float sum = 0.0f;
        // Chunk c's slot holds it once ready[c % RT_SLOTS] == c.  false: the wait gave up.
        auto wait_ready = [&](int c) {
            for (long long k = 0; k < SPIN && lds_acquire(&ready[c % RT_SLOTS]) != c; ++k) __builtin_amdgcn_s_sleep(1);
            if (force || lds_acquire(&ready[c % RT_SLOTS]) != c) {
                gave_up();
                if (lane == 0) lds_release(done, 0x7fffffff);
                return false;
            }
            return true;
        };
        // The chain reads the ring in batches of B steps, double-buffered: the
        // reads of batch g + 1 are issued before the adds of batch g, and one
        // explicit wait for all but the newest B reads (LDS reads complete in
        // order) covers the whole batch, so the adds run back to back.  The
        // next chunk's slot is awaited before its first batch is issued.  The
        // empty asm statement closing each batch keeps its adds ahead of the
        // next issue (the compiler would otherwise sink them past it, and past
        // the wait for the next chunk).  Only the expert lanes run the chain.
        constexpr int B = 8, NB = RT_STEPS / B;
        float4 bufs[2][B];
        auto issue = [&](float4 (&dst)[B], const float4 *src) {
#pragma unroll
            for (int k = 0; k < B; ++k) dst[k] = src[k * RT_EXPERTS + l];
        };
        auto adds = [&](const float4 (&src)[B]) {
#pragma unroll
            for (int k = 0; k < B; ++k) {
                sum = __fadd_rn(sum, src[k].x);
                sum = __fadd_rn(sum, src[k].y);
                sum = __fadd_rn(sum, src[k].z);
                sum = __fadd_rn(sum, src[k].w);
            }
            asm volatile("" : "+v"(sum)::"memory");
        };
        // s_waitcnt lgkmcnt(B) (vmcnt and expcnt left at their maxima), fenced
        // by scheduling barriers so that the reads just issued stay ahead of it.
        constexpr int WAIT_NEWEST_B = 0xC07F | (B << 8);
        auto wait_lds = [](auto cnt) {
            __builtin_amdgcn_sched_barrier(0);
            __builtin_amdgcn_s_waitcnt(decltype(cnt)::value);
            __builtin_amdgcn_sched_barrier(0);
        };
        bool ok = nch > 0;
        if (lane < RT_EXPERTS) {
            ok = ok && wait_ready(0);
            if (ok) issue(bufs[0], ring);
            for (int c = 0; ok && c < nch; ++c) {
                const float4 *cur = ring + (c % RT_SLOTS) * RT_STEPS * RT_EXPERTS;
                const float4 *nxt = ring + ((c + 1) % RT_SLOTS) * RT_STEPS * RT_EXPERTS;
#pragma unroll
                for (int b = 0; b < NB - 1; ++b) {
                    issue(bufs[(b + 1) & 1], cur + (b + 1) * B * RT_EXPERTS);
                    wait_lds(std::integral_constant<int, WAIT_NEWEST_B>());
                    adds(bufs[b & 1]);
                }
                const bool more = c + 1 < nch;
                if (more && !wait_ready(c + 1)) ok = false;
                if (ok && more) {
                    issue(bufs[0], nxt);
                    wait_lds(std::integral_constant<int, WAIT_NEWEST_B>());
                } else {
                    wait_lds(std::integral_constant<int, 0xC07F>());
                }
                adds(bufs[(NB - 1) & 1]);
                if (ok && lane == 0) lds_release(done, c);
            }
        }
        if (!ok) sum = __int_as_float(0x7fc00000);
        const bool skip = a.skip_if && (a.skip_if->first_bad_input != ~0ull || a.skip_if->first_bad_dest != ~0ull ||
                                        a.skip_if->first_bad_scale != ~0ull);
        if (lane < RT_EXPERTS && e0 + lane < n && !skip) {
            float *o = a.logits + e0 + lane;
            *o = a.accumulate ? __fadd_rn(*o, __fmul_rn(a.coef, sum)) : sum;   // gemv.rs:161-171
        }
    }
}

// Maximum of a 32-bit value over the wave, returned in every lane (uniform):
// DPP steps (quad butterflies, half-row and row mirrors, then the row 15 and
// row 31 broadcasts) leave the maximum in lane 63, read back as a scalar.
template <int CTRL, int ROWS>
__device__ __forceinline__ uint32_t dpp_max_step(uint32_t v) {
    const uint32_t o = (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, CTRL, ROWS, 0xf, false);
    return o > v ? o : v;
}
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    v = dpp_max_step<0xB1, 0xf>(v);    // quad_perm [1, 0, 3, 2]
    v = dpp_max_step<0x4E, 0xf>(v);    // quad_perm [2, 3, 0, 1]
    v = dpp_max_step<0x141, 0xf>(v);   // row_half_mirror
    v = dpp_max_step<0x140, 0xf>(v);   // row_mirror
    v = dpp_max_step<0x142, 0xa>(v);   // row_bcast:15 into rows 1 and 3
    v = dpp_max_step<0x143, 0xc>(v);   // row_bcast:31 into rows 2 and 3
    return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}
// The 64-bit key maximum as two 32-bit passes: the high words, then the low
// words of the lanes that hold that high word.
__device__ __forceinline__ unsigned long long wave_max_u64(unsigned long long v) {
    const uint32_t hi = wave_max_u32((uint32_t)(v >> 32));
    const uint32_t lo = wave_max_u32((uint32_t)(v >> 32) == hi ? (uint32_t)v : 0u);
    return ((unsigned long long)hi << 32) | lo;
}

// Called by all 64 lanes of one wave; every lane returns the same route.
// bad: ~0 when valid, else (first invalid expert << 2) | field
// (0 logit, 1 bias, 2 selection score: the checks of routing.rs:72-77).
__device__ __forceinline__ void select_route(const RouterArgs &a, MoeRoute &out, unsigned long long &bad) {
    const int lane = threadIdx.x & 63;
    constexpr int SLOTS = 4;   // up to 256 experts
    unsigned long long key[SLOTS];
    float weight[SLOTS], logit[SLOTS], bias[SLOTS];
    bad = ~0ull;
    // Every load first (row clamped into the table), so they share one round
    // trip instead of one per slot behind the slot's branches.
#pragma unroll
    for (int k = 0; k < SLOTS; ++k) {
        const int e = lane + 64 * k;
        const int ec = e < a.n_experts ? e : a.n_experts - 1;
        logit[k] = a.logits[ec];
        bias[k] = a.mode == 1 ? a.bias[ec] : 0.0f;
    }
#pragma unroll
    for (int k = 0; k < SLOTS; ++k) {
        const int e = lane + 64 * k;
        key[k] = 0;
        weight[k] = 0.0f;
        if (e < a.n_experts) {
            const float l = logit[k];
            float score = l;
            if (a.mode == 1) {
                const float b = bias[k];
                const float w = sigmoid_ref(l);
                score = __fadd_rn(w, b);
                weight[k] = w;
                const unsigned long long code = !isfinite(l) ? 0ull : !isfinite(b) ? 1ull : !isfinite(score) ? 2ull : 3ull;
                if (code < 3) bad = min(bad, ((unsigned long long)e << 2) | code);
            } else if (!isfinite(l)) {
                bad = min(bad, (unsigned long long)e << 2);
            }
            key[k] = sel_key(score, (uint32_t)e);   // never 0: 0 marks empty / taken
        }
    }
    for (int off = 32; off >= 1; off >>= 1) {
        const unsigned long long o = __shfl_xor(bad, off, 64);
        bad = o < bad ? o : bad;
    }

    // top_k rounds of a wave arg-max; winners come out in rank order.
    uint32_t win_id[MOE_MAX_ROUTED];
    float win_score[MOE_MAX_ROUTED], win_w[MOE_MAX_ROUTED];
#pragma unroll
    for (int r = 0; r < MOE_MAX_ROUTED; ++r) {
        win_id[r] = 0, win_score[r] = 0.0f, win_w[r] = 0.0f;
        if (r >= a.top_k) continue;
        unsigned long long best = key[0];
#pragma unroll
        for (int k = 1; k < SLOTS; ++k)
            if (key[k] > best) best = key[k];
        const unsigned long long m = wave_max_u64(best);   // uniform
        const uint32_t id = 0xffffffffu - (uint32_t)(m & 0xffffffffull);
        const int owner = (int)(id & 63);
        const int slot = (int)(id >> 6);
        // the winner's weight and logit, read from its owner lane
        float wsel = weight[0], lsel = logit[0];
#pragma unroll
        for (int k = 1; k < SLOTS; ++k)
            if (k == slot) wsel = weight[k], lsel = logit[k];
        win_id[r] = id;
        win_w[r] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wsel), owner));
        win_score[r] = a.mode == 1 ? 0.0f : __int_as_float(__builtin_amdgcn_readlane(__float_as_int(lsel), owner));
        if (lane == owner) {
#pragma unroll
            for (int k = 0; k < SLOTS; ++k)
                if (k == slot) key[k] = 0;
        }
    }
    float coef[MOE_MAX_ROUTED];
    if (a.mode == 1) {
        float wsum = 0.0f;
#pragma unroll
        for (int r = 0; r < MOE_MAX_ROUTED; ++r)
            if (r < a.top_k) wsum = __fadd_rn(wsum, win_w[r]);
        const float floor_ = 0.000061035156f;   // 2^-14, routing.rs:5
        if (!(wsum >= floor_)) wsum = floor_;
#pragma unroll
        for (int r = 0; r < MOE_MAX_ROUTED; ++r) coef[r] = __fmul_rn(__fdiv_rn(win_w[r], wsum), a.weight_scale);
    } else {
        // Lane r evaluates the exponential of winner r (the values are uniform,
        // so one call per lane in parallel instead of sixteen dependent table
        // reads in one lane), then the sum runs in rank order as before.
        const float mx = win_score[0];
        float in = 0.0f;
#pragma unroll
        for (int r = 0; r < MOE_MAX_ROUTED; ++r)
            if (lane == r) in = __fsub_rn(win_score[r], mx);
        const float ev_lane = expf_libm(in);
        float ev[MOE_MAX_ROUTED];
        float s = 0.0f;
#pragma unroll
        for (int r = 0; r < MOE_MAX_ROUTED; ++r) {
            ev[r] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ev_lane), r));
            if (r < a.top_k) s = __fadd_rn(s, ev[r]);
        }
        const float coef_lane = __fdiv_rn(ev_lane, s);
#pragma unroll
        for (int r = 0; r < MOE_MAX_ROUTED; ++r)
            coef[r] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(coef_lane), r));
    }
    // Output ascending by id (routing.rs:105): position = winners with a
    // smaller id.  Lane r holds winner r and counts its position; position q
    // is then read from the lane that holds it.
    out.n = a.top_k;
    out.pad = 0;
    uint32_t my_id = 0;
    float my_coef = 0.0f;
#pragma unroll
    for (int r = 0; r < MOE_MAX_ROUTED; ++r)
        if (lane == r) my_id = win_id[r], my_coef = coef[r];
    int pos = 0;
#pragma unroll
    for (int q = 0; q < MOE_MAX_ROUTED; ++q) pos += (q < a.top_k && win_id[q] < my_id) ? 1 : 0;
    const bool holds = lane < a.top_k;
#pragma unroll
    for (int q = 0; q < MOE_MAX_ROUTED; ++q) {
        out.ids[q] = 0;
        out.coefs[q] = 0.0f;
        if (q >= a.top_k) continue;
        const unsigned long long m = __ballot(holds && pos == q);
        const int src = (int)__builtin_ctzll(m);
        out.ids[q] = (uint32_t)__builtin_amdgcn_readlane((int)my_id, src);
        out.coefs[q] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(my_coef), src));
    }
}

}  // namespace lbh
