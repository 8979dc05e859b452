// Scalar math shared by the HIP kernels (and usable on the host for self-checks).
//
// Every function here reproduces one reference elementwise operation bit for bit, given the same
// inputs.  Translation units that include this header are compiled with -ffp-contract=off, so
// each float/double operation written below is one IEEE round-to-nearest operation, as in the
// reference x86-64 build (g++ -O2, no FMA, hls/build_host_wrappers.sh:32).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "qwen_layout.h"

namespace qwen {

#define QWEN_HD __host__ __device__ __forceinline__

QWEN_HD uint32_t f32_bits(float f) { return __builtin_bit_cast(uint32_t, f); }
QWEN_HD float bits_f32(uint32_t u) { return __builtin_bit_cast(float, u); }
QWEN_HD uint64_t f64_bits(double d) { return __builtin_bit_cast(uint64_t, d); }
QWEN_HD double bits_f64(uint64_t u) { return __builtin_bit_cast(double, u); }

// ---- glibc-compatible expf -------------------------------------------------------------------
// The decode path calls the host expf (softmax qwen_decode_attention_kernel.cpp:149, SiLU
// qwen_decode_mlp_kernel.cpp:80).  glibc >= 2.27 implements expf with the published
// ARM Optimized Routines method (Szabolcs Nagy, 2017): x*32/ln2 = k + r, exp(x) = 2^(k/32) *
// P(r) with a 32-entry table of 2^(i/32) and a cubic P evaluated in double; on FMA-capable x86-64
// the FMA build of that routine is selected.  This is that method written with explicit fma, so
// it agrees with the host expf for every float input (checked exhaustively on the CPU against
// glibc 2.35's expf over all 2^32 inputs: 0 mismatches; the GPU test re-checks device vs host).
// kExp2Tab[i] = bits(double(2^(i/32))) - (i << 47), the stored form used by that method.
__device__ __constant__ static const uint64_t kExp2Tab[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
};

// `tab` is kExp2Tab or a copy of it (e.g. in LDS, so that a kernel epilogue does not wait on a
// memory load per call); the result does not depend on where the table is read from.
__device__ __forceinline__ float glibc_expf(float x, const uint64_t* tab = kExp2Tab) {
  // Special cases for |x| >= 88 (inf, nan, overflow, underflow), as in the published routine.
  const uint32_t ux = f32_bits(x);
  const uint32_t abstop = (ux >> 20) & 0x7ffu;
  if (abstop >= 0x42bu) {  // top12(88.0f)
    if (ux == 0xff800000u) return 0.0f;          // -inf
    if (abstop >= 0x7f8u) return x + x;          // inf or nan
    if (x > 0x1.62e42ep6f) return __builtin_huge_valf();
    if (x < -0x1.9fe368p6f) return 0.0f;
  }
  const double kInvLn2N = 0x1.71547652b82fep+0 * 32.0;
  const double kShift = 0x1.8p+52;
  const double c0 = 0x1.c6af84b912394p-5 / 32.0 / 32.0 / 32.0;
  const double c1 = 0x1.ebfce50fac4f3p-3 / 32.0 / 32.0;
  const double c2 = 0x1.62e42ff0c52d6p-1 / 32.0;
  const double xd = (double)x;
  double kd = __builtin_fma(kInvLn2N, xd, kShift);
  const uint64_t ki = f64_bits(kd);
  kd -= kShift;
  const double r = __builtin_fma(kInvLn2N, xd, -kd);
  uint64_t t = tab[ki % 32u];
  t += ki << 47;
  const double s = bits_f64(t);
  const double z = __builtin_fma(c0, r, c1);
  const double r2 = r * r;
  double y = __builtin_fma(c2, r, 1.0);
  y = __builtin_fma(z, r2, y);
  y = y * s;
  return (float)y;
}

// ---- prefill approximations (qwen_prefill_attention_kernel.cpp:47-110) ----------------------
QWEN_HD float approx_sqrt(float v) {  // :47-57
  if (v <= 0.0f) return 0.0f;
  float g = v > 1.0f ? v : 1.0f;
#pragma unroll
  for (int it = 0; it < 6; ++it) g = 0.5f * (g + v / g);
  return g;
}

QWEN_HD float wrap_angle(float a) {  // :59-67
  const float kPi = 3.14159265358979323846f;
  const float kTwoPi = 6.28318530717958647692f;
  while (a > kPi) a -= kTwoPi;
  while (a < -kPi) a += kTwoPi;
  return a;
}

QWEN_HD void approx_sincos(float a, float* s, float* c) {  // :69-85
  const float kPi = 3.14159265358979323846f;
  const float kHalfPi = 1.57079632679489661923f;
  float r = wrap_angle(a);
  float cs = 1.0f;
  if (r > kHalfPi) {
    r = kPi - r;
    cs = -1.0f;
  } else if (r < -kHalfPi) {
    r = -kPi - r;
    cs = -1.0f;
  }
  const float x2 = r * r;
  *s = r * (1.0f + x2 * (-1.0f / 6.0f + x2 * (1.0f / 120.0f + x2 * (-1.0f / 5040.0f))));
  *c = cs * (1.0f + x2 * (-0.5f + x2 * (1.0f / 24.0f + x2 * (-1.0f / 720.0f))));
}

QWEN_HD float approx_exp(float v) {  // :87-110; `term *= s / deg` divides first
  if (v <= -16.0f) return 0.0f;
  int halves = 0;
  float s = v;
  while (s < -1.0f) {
    s *= 0.5f;
    ++halves;
  }
  float term = 1.0f, series = 1.0f;
#pragma unroll
  for (int deg = 1; deg <= 6; ++deg) {
    term *= s / (float)deg;
    series += term;
  }
  for (int k = 0; k < halves; ++k) series *= series;
  return series > 0.0f ? series : 0.0f;
}

__device__ __forceinline__ float silu_decode(float v, const uint64_t* tab = kExp2Tab) {  // mlp :79-81
  return v / (1.0f + glibc_expf(-v, tab));
}
QWEN_HD float silu_prefill(float v) { return v / (1.0f + approx_exp(-v)); }                   // mlp :256-258

// Signed INT4 nibble of byte b: low nibble for even flat index (qwen_decode_attention_kernel.cpp:44-48).
QWEN_HD int nibble_lo(uint32_t b) { return (int)((b & 0xFu) ^ 8u) - 8; }
QWEN_HD int nibble_hi(uint32_t b) { return (int)(((b >> 4) & 0xFu) ^ 8u) - 8; }

// bf16 rounding of the driver (verification/reference_wrapper_backend.py:40-46), uint32 wrap-around.
QWEN_HD float round_bf16(float x) {
  uint32_t b = f32_bits(x);
  b += 0x7FFFu + ((b >> 16) & 1u);
  b &= 0xFFFF0000u;
  return bits_f32(b);
}

}  // namespace qwen
