// lbh_math.h — f32 exp with the exact results of the host C library's expf.
//
// The reference's SwiGLU and router call Rust's f32::exp, i.e. the platform
// libm expf (crates/bridge-kernels-reference/src/activation.rs:172,
// crates/bridge-model-hy3/src/routing.rs:109-111); on Linux that is glibc,
// whose expf implements the published table-driven method of ARM's
// optimized-routines (math/expf.c): with N = 32,
//     x * N / ln2 = k + r,  |r| <= 1/2,
//     exp(x) = 2^(k/N) * 2^(r/N),   2^(r/N) ~= 1 + C2 r + C1 r^2 + C0 r^3,
// evaluated in double and rounded once to float.  The polynomial
// coefficients are that method's published minimax values; the table holds
// bits(2^(i/N)) - (i << 47), computed here from the definition.  glibc's x86-64
// build contracts the polynomial and the reduction into fused multiply-adds;
// this restatement uses the same fma steps and reproduces that expf bit for
// bit on every non-NaN input (checked exhaustively against the host library).
#pragma once
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

namespace lbh {

#define LBH_EXPF_TABLE \
  0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull, \
  0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull, \
  0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull, \
  0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull, \
  0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull, \
  0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull, \
  0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull, \
  0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull

// Device copy in constant memory (a dynamically indexed local table would be
// placed in scratch); host copy for the host-side build of the same function.
static __constant__ uint64_t c_expf_tab[32] = {LBH_EXPF_TABLE};
static const uint64_t h_expf_tab[32] = {LBH_EXPF_TABLE};

__host__ __device__ inline float expf_libm(float x) {
    constexpr double N = 32.0;
    constexpr double INV_LN2_N = 0x1.71547652b82fep+0 * N;
    constexpr double SHIFT = 0x1.8p+52;
    constexpr double C0 = 0x1.c6af84b912394p-5 / N / N / N;
    constexpr double C1 = 0x1.ebfce50fac4f3p-3 / N / N;
    constexpr double C2 = 0x1.62e42ff0c52d6p-1 / N;
    const uint32_t ux = __builtin_bit_cast(uint32_t, x);
    const uint32_t abstop = (ux >> 20) & 0x7ffu;
    if (abstop >= 0x42bu) {                          // |x| >= 88, inf or NaN
        if (ux == 0xff800000u) return 0.0f;           // -inf
        if (abstop >= 0x7f8u) return x + x;           // +inf, NaN
        if (x > 0x1.62e42ep6f) return __builtin_inff();   // overflow
        if (x < -0x1.9fe368p6f) return 0.0f;              // underflow
    }
    const double xd = (double)x;
    double kd = fma(INV_LN2_N, xd, SHIFT);
    const uint64_t ki = __builtin_bit_cast(uint64_t, kd);
    kd -= SHIFT;
    const double r = fma(INV_LN2_N, xd, -kd);
#ifdef __HIP_DEVICE_COMPILE__
    const uint64_t t = c_expf_tab[ki % 32] + (ki << 47);
#else
    const uint64_t t = h_expf_tab[ki % 32] + (ki << 47);
#endif
    const double s = __builtin_bit_cast(double, t);
    const double z = fma(C0, r, C1);
    const double r2 = r * r;
    double y = fma(C2, r, 1.0);
    y = fma(z, r2, y);
    y = y * s;
    return (float)y;
}

// apply_swiglu's element (activation.rs:170-178): gate / (1 + exp(-gate)) * up,
// each step separately rounded.
__host__ __device__ inline float swiglu_ref(float gate, float up) {
    const float e = expf_libm(-gate);
    const float act = gate / (1.0f + e);
    return act * up;
}

}  // namespace lbh
