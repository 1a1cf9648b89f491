// lbh_router.hip — MoE router of one token on the GPU.
//
// logits[e] = dot_f32_row(router row e, x) (crates/bridge-kernels-reference/
// src/gemv.rs:286-303): the reference sums w[i] * x[i] strictly in order, each
// product and sum separately rounded, so each logit is one sequential chain.
// Workgroups of EPW experts first form all products in LDS (the 3 MiB of
// router weights spread over many CUs), then one lane per expert runs its chain
// with the LDS reads issued ahead of the adds.  The last workgroup to finish
// (self-resetting arrival count) selects the top k and writes the MoeRoute the
// MoE kernels read:
//   mode 0  softmax over the top k by (logit desc, id asc), renormalised
//           (the benchmark configuration's router);
//   mode 1  route_experts_into (crates/bridge-model-hy3/src/routing.rs:25-107):
//           sigmoid(logit) + bias selects, sigmoid / max(sum, 2^-14) * scale
//           weights, output ascending by id.
#include "lbh_internal.h"
#include "lbh_math.h"

namespace lbh {

constexpr int ROUTER_THREADS = 256;

__device__ __forceinline__ float sigmoid_ref(float v) { return 1.0f / (1.0f + expf_libm(-v)); }  // routing.rs:109-111

// Total order of selection keys: larger score first, then smaller id.
// Scores are finite (checked) floats; +0.0 and -0.0 compare equal as in f32.
__device__ __forceinline__ unsigned long long sel_key(float score, uint32_t id) {
    const float s = score == 0.0f ? 0.0f : score;        // -0.0 == +0.0
    uint32_t b = __float_as_uint(s);
    b = (b & 0x80000000u) ? ~b : (b | 0x80000000u);     // monotone float -> uint
    return ((unsigned long long)b << 32) | (0xffffffffu - id);
}

__global__ void __launch_bounds__(ROUTER_THREADS) k_router(RouterArgs a) {
    extern __shared__ __align__(16) float s_p[];   // [epw][hidden + 4]
    const int tid = threadIdx.x;
    const int stride = a.hidden + 4;                // +4 floats: chains start in different banks
    const int e0 = blockIdx.x * a.epw;
    const int ne = min(a.epw, a.n_experts - e0);

    // Products w[e][i] * x[i] for the workgroup's experts.
    const float4 *x4 = reinterpret_cast<const float4 *>(a.x);
    for (int i4 = tid; i4 < a.hidden / 4; i4 += ROUTER_THREADS) {
        const float4 xv = x4[i4];
        for (int e = 0; e < ne; ++e) {
            const float4 wv = reinterpret_cast<const float4 *>(a.w + (long long)(e0 + e) * a.hidden)[i4];
            float4 p;
            p.x = __fmul_rn(wv.x, xv.x), p.y = __fmul_rn(wv.y, xv.y);
            p.z = __fmul_rn(wv.z, xv.z), p.w = __fmul_rn(wv.w, xv.w);
            *reinterpret_cast<float4 *>(&s_p[e * stride + 4 * i4]) = p;
        }
    }
    __syncthreads();

    // One lane per expert: sum = ((0 + p0) + p1) + ...  Sixteen products are
    // read ahead while the previous sixteen are added.
    if (tid < ne) {
        const float4 *row = reinterpret_cast<const float4 *>(&s_p[tid * stride]);
        const int n4 = a.hidden / 4;   // hidden is a multiple of 256
        float sum = 0.0f;
        float4 cur[4], nxt[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) cur[k] = row[k];
        for (int j = 4; j <= n4; j += 4) {
            if (j < n4) {
#pragma unroll
                for (int k = 0; k < 4; ++k) nxt[k] = row[j + k];
            }
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                sum = __fadd_rn(sum, cur[k].x);
                sum = __fadd_rn(sum, cur[k].y);
                sum = __fadd_rn(sum, cur[k].z);
                sum = __fadd_rn(sum, cur[k].w);
            }
#pragma unroll
            for (int k = 0; k < 4; ++k) cur[k] = nxt[k];
        }
        a.logits[e0 + tid] = sum;
    }

    // The last workgroup selects.
    __threadfence();
    __syncthreads();
    __shared__ int s_last;
    if (tid == 0) {
        const unsigned old = __hip_atomic_fetch_add(a.counter, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
        s_last = old + 1 == gridDim.x;
        if (s_last) __hip_atomic_store(a.counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!s_last || tid >= 64) return;
    __threadfence();

    const int lane = tid;
    constexpr int SLOTS = 4;   // up to 256 experts
    unsigned long long key[SLOTS];
    float weight[SLOTS];
    unsigned long long bad = ~0ull;
#pragma unroll
    for (int k = 0; k < SLOTS; ++k) {
        const int e = lane + 64 * k;
        key[k] = 0;
        weight[k] = 0.0f;
        if (e < a.n_experts) {
            const float l = a.logits[e];
            float score = l;
            if (a.mode == 1) {
                const float b = a.bias[e];
                const float w = sigmoid_ref(l);
                score = __fadd_rn(w, b);
                weight[k] = w;
                // routing.rs:72-77: logits, then bias, then score, first bad index wins
                const unsigned long long code = !isfinite(l) ? 0ull : !isfinite(b) ? 1ull : !isfinite(score) ? 2ull : 3ull;
                if (code < 3) bad = min(bad, ((unsigned long long)e << 2) | code);
            } else {
                if (!isfinite(l)) bad = min(bad, (unsigned long long)e << 2);
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
        int bk = 0;
#pragma unroll
        for (int k = 1; k < SLOTS; ++k)
            if (key[k] > best) best = key[k], bk = k;
        unsigned long long m = best;
        for (int off = 32; off >= 1; off >>= 1) {
            const unsigned long long o = __shfl_xor(m, off, 64);
            m = o > m ? o : m;
        }
        const uint32_t id = 0xffffffffu - (uint32_t)(m & 0xffffffffull);
        const int owner = (int)(id & 63);
        const int slot = (int)(id >> 6);
        const float wv = __shfl(weight[bk], owner, 64);
        win_id[r] = id;
        win_w[r] = wv;
        win_score[r] = a.mode == 1 ? 0.0f : a.logits[id];
        if (lane == owner) {
#pragma unroll
            for (int k = 0; k < SLOTS; ++k)
                if (k == slot) key[k] = 0;
        }
    }
    if (lane != 0) return;
    if (a.status) {
        if (bad != ~0ull) {
            a.status[0] = bad;
            return;
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
        const float mx = win_score[0];
        float ev[MOE_MAX_ROUTED];
        float s = 0.0f;
#pragma unroll
        for (int r = 0; r < MOE_MAX_ROUTED; ++r) {
            ev[r] = expf_libm(__fsub_rn(win_score[r], mx));
            if (r < a.top_k) s = __fadd_rn(s, ev[r]);
        }
#pragma unroll
        for (int r = 0; r < MOE_MAX_ROUTED; ++r) coef[r] = __fdiv_rn(ev[r], s);
    }
    // Output ascending by id (routing.rs:105): position = number of winners
    // with a smaller id.
    a.route->n = a.top_k;
#pragma unroll
    for (int r = 0; r < MOE_MAX_ROUTED; ++r) {
        if (r >= a.top_k) continue;
        int pos = 0;
#pragma unroll
        for (int q = 0; q < MOE_MAX_ROUTED; ++q) pos += (q < a.top_k && win_id[q] < win_id[r]) ? 1 : 0;
        a.route->ids[pos] = win_id[r];
        a.route->coefs[pos] = coef[r];
    }
}

hipError_t launch_router(const RouterArgs &a, hipStream_t s) {
    if (a.n_experts < 1 || a.n_experts > 256 || a.top_k < 1 || a.top_k > MOE_MAX_ROUTED || a.top_k > a.n_experts ||
        a.hidden % 256 || a.epw < 1)
        return hipErrorInvalidValue;
    const int grid = (a.n_experts + a.epw - 1) / a.epw;
    const size_t lds = (size_t)a.epw * (a.hidden + 4) * sizeof(float);
    hipLaunchKernelGGL(k_router, dim3(grid), dim3(ROUTER_THREADS), lds, s, a);
    return hipGetLastError();
}

}  // namespace lbh
