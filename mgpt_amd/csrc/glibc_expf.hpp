// glibc_expf.hpp -- expf with the same bits as the host glibc's expf.
//
// The reference's softmax calls std::exp(float) = glibc expf
// (/root/reference/src/main/utils/Tensor.cpp:873).  Routing must be
// bit-exact, so the GPU evaluates the same published algorithm that glibc
// (2.27+) uses on x86-64 CPUs with FMA: the table-driven exp2 scheme of
// ARM's optimized-routines (Szabolcs Nagy, 2017),
//   exp(x) = 2^(k/N) * 2^(r/N),  N = 32,  k = round(x N / ln 2),
//   2^(r/N) ~= 1 + c2 r + c1 r^2 + c0 r^3   (|r| <= 1/2, evaluated in double),
// with the table entries 2^(i/32) correctly rounded to double and the
// fused multiply-adds at the places glibc's FMA build contracts them.
// The table below was computed from its definition with exact integer
// arithmetic (floor of the 32nd root of 2^(52*32+i+32*64), rounded), which
// tests/test_expf.py repeats.  Exhaustive
// agreement with the host expf over every float in [-104, 0] (the only
// range softmax passes it, x = l - max(l) <= 0) is checked by
// tests/test_expf.py; outside that range only the special cases below are
// needed (x < -103.97 underflows to 0, NaN propagates).
#pragma once

#include <stdint.h>

#ifdef __HIPCC__
#define MGPT_HD __host__ __device__ __forceinline__
#else
#define MGPT_HD static inline
#include <math.h>
#include <string.h>
#endif

namespace mgpt_expf {

// Polynomial of 2^(r/32) for |r| <= 1/2 (minimax cubic; coefficients of
// the published algorithm, already divided by 32^3, 32^2, 32).
#define MGPT_EXPF_C0 (0x1.c6af84b912394p-5 / 32 / 32 / 32)
#define MGPT_EXPF_C1 (0x1.ebfce50fac4f3p-3 / 32 / 32)
#define MGPT_EXPF_C2 (0x1.62e42ff0c52d6p-1 / 32)
#define MGPT_EXPF_INVLN2N (0x1.71547652b82fep+0 * 32)
#define MGPT_EXPF_SHIFT 0x1.8p+52

// MGPT_EXP2_TABLE_INIT[i] = bits(2^(i/32) rounded to double) - (i << 47).
#define MGPT_EXP2_TABLE_INIT                                                 \
  {0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full,      \
   0x3fef9301d0125b51ull, 0x3fef72b83c7d517bull, 0x3fef54873168b9aaull,      \
   0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull, 0x3fef06fe0a31b715ull,      \
   0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,      \
   0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull,      \
   0x3feea47eb03a5585ull, 0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull,      \
   0x3feea11473eb0187ull, 0x3feea589994cce13ull, 0x3feeace5422aa0dbull,      \
   0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,      \
   0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull,      \
   0x3fef3720dcef9069ull, 0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full,      \
   0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull}

MGPT_HD uint64_t as_u64(double d) {
#ifdef __HIP_DEVICE_COMPILE__
  return (uint64_t)__double_as_longlong(d);
#else
  uint64_t u;
  __builtin_memcpy(&u, &d, 8);
  return u;
#endif
}
MGPT_HD double as_f64(uint64_t u) {
#ifdef __HIP_DEVICE_COMPILE__
  return __longlong_as_double((long long)u);
#else
  double d;
  __builtin_memcpy(&d, &u, 8);
  return d;
#endif
}
MGPT_HD uint32_t as_u32(float f) {
#ifdef __HIP_DEVICE_COMPILE__
  return __float_as_uint(f);
#else
  uint32_t u;
  __builtin_memcpy(&u, &f, 4);
  return u;
#endif
}

// expf(x) given T = MGPT_EXP2_TABLE_INIT (in device-visible memory on the GPU).  x must be <= 88 (softmax only passes x <= 0).
MGPT_HD float expf_glibc(float x, const uint64_t* T) {
  const uint32_t abstop = (as_u32(x) >> 20) & 0x7ff;
  if (abstop >= 0x42b) {                 // |x| >= 88 (top 12 bits of 88.0f), or NaN/Inf
    if (as_u32(x) == 0xff800000u) return 0.0f;        // -inf
    if (abstop >= 0x7f8) return x + x;                 // NaN (or +inf)
    if (x < -0x1.9fe368p6f) return 0.0f;               // below log(2^-150): underflow
  }
  const double xd = (double)x;
  double kd = __builtin_fma(MGPT_EXPF_INVLN2N, xd, MGPT_EXPF_SHIFT);
  const uint64_t ki = as_u64(kd);
  kd -= MGPT_EXPF_SHIFT;
  const double r = __builtin_fma(MGPT_EXPF_INVLN2N, xd, -kd);
  uint64_t t = T[ki % 32];
  t += ki << (52 - 5);
  const double s = as_f64(t);
  const double z = __builtin_fma(MGPT_EXPF_C0, r, MGPT_EXPF_C1);
  const double r2 = r * r;
  double y = __builtin_fma(MGPT_EXPF_C2, r, 1.0);
  y = __builtin_fma(z, r2, y);
  y = y * s;
  return (float)y;
}

}  // namespace mgpt_expf
