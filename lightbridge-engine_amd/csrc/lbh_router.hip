// lbh_router.hip — MoE router of one token on the GPU.
//
// logits[e] = dot_f32_row(router row e, x) (crates/bridge-kernels-reference/
// src/gemv.rs:286-303): the reference sums w[i] * x[i] strictly in order, each
// product and sum separately rounded, so each logit is one sequential chain of
// `hidden` dependent adds.  One lane owns one expert: the weights are stored
// transposed and interleaved by four (wt[j][e][0..3] = w[e][4j..4j+3]); per
// workgroup one wave runs eight experts' chains out of an LDS ring that three
// producer waves keep filled (lbh_router.h), the products formed off the add
// chain.  Selection
// (select_route) is a device function shared by the standalone router kernel
// and the MoE gate/up kernel's prologue:
//   mode 0  softmax over the top k by (logit desc, id asc), renormalised
//           (the benchmark configuration's router);
//   mode 1  route_experts_into (crates/bridge-model-hy3/src/routing.rs:25-107):
//           sigmoid(logit) + bias selects, sigmoid / max(sum, 2^-14) * scale
//           weights, output ascending by id.
#include "lbh_internal.h"
#include "lbh_router.h"

namespace lbh {

__global__ void __launch_bounds__(256) k_router_logits(RouterArgs a) {
    __shared__ __align__(16) uint8_t lds[RT_LDS];
    router_chain_wg(a, blockIdx.x * RT_EXPERTS, lds);
}

// Selection of one token from the finished logits, by wave 0 of the block;
// lane 0 writes the result (and the first invalid lane to *bad_out).
__global__ void __launch_bounds__(64) k_router_select(RouterArgs a) {
    MoeRoute r;
    unsigned long long bad;
    select_route(a, r, bad);
    if (threadIdx.x == 0) {
        if (a.status) a.status[0] = bad;
        if (bad == ~0ull || !a.status) *a.route = r;
    }
}

hipError_t launch_router_logits(const RouterArgs &a, hipStream_t s) {
    if (a.n_experts < 1 || a.n_experts > 256 || a.hidden % 256) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_router_logits, dim3((a.n_experts + RT_EXPERTS - 1) / RT_EXPERTS), dim3(256), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_f32_chains(const RouterArgs &a, hipStream_t s) {
    if (a.n_experts < 1 || a.n_experts > 0x7ffffff0 || a.hidden < 256 || a.hidden % 256) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_router_logits, dim3((a.n_experts + RT_EXPERTS - 1) / RT_EXPERTS), dim3(256), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_router(const RouterArgs &a, hipStream_t s) {
    if (a.n_experts < 1 || a.n_experts > 256 || a.top_k < 1 || a.top_k > MOE_MAX_ROUTED || a.top_k > a.n_experts ||
        a.hidden % 256)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_router_logits, dim3((a.n_experts + RT_EXPERTS - 1) / RT_EXPERTS), dim3(256), 0, s, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_router_select, dim3(1), dim3(64), 0, s, a);
    return hipGetLastError();
}

}  // namespace lbh
