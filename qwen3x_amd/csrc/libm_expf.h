// libm_expf.h -- float exp with the host libm's arithmetic, so that the
// router's softmax on the GPU equals the reference's CPU softmax bit for bit.
//
// The reference router takes std::exp of a float (engine.cpp:383-386).  On
// x86-64, glibc (2.28 and later) implements it with the ARM Optimized
// Routines expf (Szabolcs Nagy, 2017: math/expf.c, math/exp2f_data.c), in
// double precision:
//   z = x * 32/ln2 = k + r with k an integer and |r| <= 1/2,
//   2^(k/32) = 2^(k div 32) * 2^((k mod 32)/32), the second factor from a
//   32-entry table of 2^(i/32),
//   2^(r/32) ~= C0 r^3 + C1 r^2 + C2 r + 1 (a minimax cubic),
// and one rounding of the double product to float.  glibc selects a build
// compiled with FMA on hosts that have it, where the compiler fuses every
// product into the add that follows it; the fusions are written here as
// explicit fma, so the device computes exactly what the host computes.
// Checked against the host expf on every float in [-110, 0] and on [0, 88)
// (tests/test_libm_expf.py); the GPU router is checked against the reference
// router with exact ids and weights.
//
// Domain: x < 88 (the router calls it on logit - max <= 0).  Below
// ln(2^-150) the result is +0, as in libm; NaN propagates.
//
// The table of 2^(i/32) and the cubic's coefficients below are those of the
// ARM Optimized Routines expf, whose upstream notice is:
//
//   Copyright (c) 2017-2018, Arm Limited.
//   SPDX-License-Identifier: MIT OR Apache-2.0 WITH LLVM-exception
//
// Under the MIT option:  Permission is hereby granted, free of charge, to any
// person obtaining a copy of this software and associated documentation files
// (the "Software"), to deal in the Software without restriction, including
// without limitation the rights to use, copy, modify, merge, publish,
// distribute, sublicense, and/or sell copies of the Software, and to permit
// persons to whom the Software is furnished to do so, subject to the
// following conditions: The above copyright notice and this permission
// notice shall be included in all copies or substantial portions of the
// Software.  THE SOFTWARE IS PROVIDED "AS IS", WITHOUT WARRANTY OF ANY KIND,
// EXPRESS OR IMPLIED, INCLUDING BUT NOT LIMITED TO THE WARRANTIES OF
// MERCHANTABILITY, FITNESS FOR A PARTICULAR PURPOSE AND NONINFRINGEMENT.  IN
// NO EVENT SHALL THE AUTHORS OR COPYRIGHT HOLDERS BE LIABLE FOR ANY CLAIM,
// DAMAGES OR OTHER LIABILITY, WHETHER IN AN ACTION OF CONTRACT, TORT OR
// OTHERWISE, ARISING FROM, OUT OF OR IN CONNECTION WITH THE SOFTWARE OR THE
// USE OR OTHER DEALINGS IN THE SOFTWARE.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace q3x {

// Bits of 2^(i/32) rounded to the nearest double, minus i << 47 so that
// adding k << 47 (k the full table index) sets the exponent of 2^(k/32).
__host__ __device__ inline uint64_t libm_exp2_table(int i) {
    constexpr uint64_t kTable[32] = {
        0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
        0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
        0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
        0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
        0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
        0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
        0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
        0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
    };
    return kTable[i];
}

__host__ __device__ inline double libm_as_double(uint64_t u) {
    double d;
    __builtin_memcpy(&d, &u, sizeof(d));
    return d;
}

__host__ __device__ inline uint64_t libm_as_u64(double d) {
    uint64_t u;
    __builtin_memcpy(&u, &d, sizeof(u));
    return u;
}

__host__ __device__ inline float libm_expf(float x) {
    if (!(x >= -0x1.9fe368p6f)) return x != x ? x + x : 0.0f;  // NaN, or below ln(2^-150): +0
    constexpr double kInvLn2N = 0x1.71547652b82fep+0 * 32;    // 32 / ln 2
    constexpr double kShift = 0x1.8p+52;                      // rounds to an integer in the last place
    constexpr double C0 = 0x1.c6af84b912394p-5 / (32.0 * 32.0 * 32.0);
    constexpr double C1 = 0x1.ebfce50fac4f3p-3 / (32.0 * 32.0);
    constexpr double C2 = 0x1.62e42ff0c52d6p-1 / 32.0;
    const double xd = static_cast<double>(x);
    double kd = fma(kInvLn2N, xd, kShift);   // k + shift, k = round(x * 32/ln2)
    const uint64_t ki = libm_as_u64(kd);      // k in the low bits
    kd -= kShift;
    const double r = fma(kInvLn2N, xd, -kd);  // x * 32/ln2 - k
    const uint64_t t = libm_exp2_table(static_cast<int>(ki % 32)) + (ki << 47);
    const double s = libm_as_double(t);       // 2^(k/32)
    const double c = fma(C0, r, C1);
    const double r2 = r * r;
    double y = fma(C2, r, 1.0);
    y = fma(c, r2, y);
    y = y * s;
    return static_cast<float>(y);
}

}  // namespace q3x
