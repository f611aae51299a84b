// exp for fp32 arguments with the fp32 results of the x86 reference build, usable on the
// host and on gfx950.
//
// The reference's x86 build takes its softmax and SwiGLU exponentials from the platform
// libm (`f32::exp`, real_llm.rs:9595 and 9803).  On x86-64 Linux that is glibc's expf
// (glibc 2.27 and later), whose method is Szabolcs Nagy's expf from Arm Optimized Routines
// (2017): in double precision, x * 32/ln2 = k + r with k the nearest integer, 2^(k/32)
// from a 32-entry table of 2^(i/32) with the integer part of k/32 added to the exponent
// bits, and 2^(r/32) by the published degree-3 polynomial.  glibc's x86-64 build selects
// an FMA-compiled copy on CPUs with FMA, where the compiler fuses the reduction and the
// polynomial's multiply-adds; this routine is written with those fused operations.
//
// The table holds the round-to-nearest double of 2^(i/32) for i = 0 .. 31, stored minus
// i << 47 (the exponent increment that the integer k adds back).  Every operation is an
// IEEE double operation (fma correctly rounded on both sides), so the host and the device
// compute the same bits.  Compared with glibc's expf over all 2^32 fp32 inputs (a CPU
// test), every result is identical, NaN payloads and the overflow / underflow limits
// included.
#pragma once
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

namespace k2t {

__host__ __device__ inline float expf_rn(float x) {
    static constexpr uint64_t kTab[32] = {
        0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
        0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
        0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
        0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
        0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
        0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
        0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
        0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
    };
    if (x != x) return x + x;
    if (x > 0x1.62e42ep6f) return INFINITY;   // exp(x) rounds above FLT_MAX
    if (x < -0x1.9fe368p6f) return 0.0f;      // below half the smallest subnormal
    const double kInvLn2N = 0x1.71547652b82fep+0 * 32.0;
    const double kShift = 0x1.8p+52;  // adding it rounds to an integer (ties to even)
    const double kC0 = 0x1.c6af84b912394p-5 / (32.0 * 32.0 * 32.0);
    const double kC1 = 0x1.ebfce50fac4f3p-3 / (32.0 * 32.0);
    const double kC2 = 0x1.62e42ff0c52d6p-1 / 32.0;
    const double xd = (double)x;
    double kd = fma(kInvLn2N, xd, kShift);
    const uint64_t ki = (uint64_t)__builtin_bit_cast(uint64_t, kd);
    kd -= kShift;
    const double r = fma(kInvLn2N, xd, -kd);
    const double s = __builtin_bit_cast(double, kTab[ki % 32] + (ki << 47));
    const double z = fma(kC0, r, kC1);
    const double r2 = r * r;
    double y = fma(kC2, r, 1.0);
    y = fma(z, r2, y);
    return (float)(y * s);
}

}  // namespace k2t
