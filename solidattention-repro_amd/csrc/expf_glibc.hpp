// expf_glibc.hpp — expf(x) by the method of glibc 2.35's expf
// (sysdeps/ieee754/flt-32/e_expf.c, e_exp2f_data.c), which is what the
// reference's std::exp(float) runs (cpp/src/selection.cpp:53), restated so
// that the device builders' softmax probabilities equal the reference's bit
// for bit.  The including translation unit is compiled with
// -ffp-contract=off: the double steps fuse exactly where written, as in
// glibc's x86-64 FMA build.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sa {
namespace {

// 2^(i/32) correctly rounded to double, minus i << 47 in the bit pattern
// (adding k << 47 to entry k mod 32 then scales it by 2^(k div 32)).
__constant__ uint64_t kExpfTab[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
};

// expf(x) by glibc 2.35's method: z = x * 32/ln2 in double; k = z rounded to
// the nearest integer by adding and subtracting 1.5 * 2^52 (k sits in the low
// bits of the shifted double); r = fma(32/ln2, x, -k); 2^(k/32) from the
// table; 2^(r/32) ~ 1 + c2 r + c1 r^2 + c0 r^3 as fma(fma(c0, r, c1), r^2,
// fma(c2, r, 1)); the double result rounded to float.  The special inputs
// (NaN, overflow, underflow) are selected after the main path, which runs for
// every x (its table index k mod 32 is always in range), so a caller's
// several exponentials issue their table reads together instead of one
// branch at a time.
__device__ inline float expf_glibc(float x) {
  constexpr double kInvLn2N = 0x1.71547652b82fep+0 * 32;
  constexpr double kShift = 0x1.8p+52;
  constexpr double kC0 = 0x1.c6af84b912394p-5 / (32.0 * 32.0 * 32.0);
  constexpr double kC1 = 0x1.ebfce50fac4f3p-3 / (32.0 * 32.0);
  constexpr double kC2 = 0x1.62e42ff0c52d6p-1 / 32.0;
  const double xd = static_cast<double>(x);
  const double z = kInvLn2N * xd;
  const double kd_shifted = z + kShift;
  const uint64_t ki = __builtin_bit_cast(uint64_t, kd_shifted);
  const double kd = kd_shifted - kShift;
  const double r = __builtin_fma(kInvLn2N, xd, -kd);
  const double s = __builtin_bit_cast(double, kExpfTab[ki % 32] + (ki << 47));
  const double p = __builtin_fma(kC0, r, kC1);
  const double r2 = r * r;
  double y = __builtin_fma(kC2, r, 1.0);
  y = __builtin_fma(p, r2, y);
  y = y * s;
  float out = static_cast<float>(y);
  out = x < -0x1.9fe368p6f ? 0.0f : out;                  // below log(2^-150)
  out = x > 0x1.62e42ep6f ? __builtin_huge_valf() : out;  // above log(2^128)
  return x != x ? x + x : out;
}

}  // namespace
}  // namespace sa
