// px_math.h -- the framework's float32 elementary functions on the device.
//
// exp, log, tanh, sin and cos follow the Cephes single-precision algorithms
// (S. L. Moshier, Cephes Math Library: expf.c, logf.c, tanhf.c, sinf.c): Cody-Waite
// range reduction and the published minimax polynomials. They are evaluated
// with plain float32 +, -, *, / (the library is built with
// -ffp-contract=off), so every result is a fixed sequence of correctly
// rounded IEEE operations and is reproducible bit for bit by any conforming
// implementation of the same steps. Accuracy is within 2 ulp of the exact
// function over the float32 range.
#pragma once

#ifndef __HIPCC_RTC__
#include <hip/hip_runtime.h>
#include <stdint.h>
#endif

namespace px {

__device__ __forceinline__ float pow2i(int n) {
  return __uint_as_float(static_cast<uint32_t>(n + 127) << 23);
}

__device__ __forceinline__ float expf_(float x) {
  if (x != x) return x;
  if (x > 88.72283935546875f) return __builtin_huge_valf();
  if (x < -103.97208404541015625f) return 0.0f;
  float fn = floorf(x * 1.44269502162933349609375f + 0.5f);
  int n = static_cast<int>(fn);
  // ln 2 split in two: 0.693359375 has 9 significant bits, so fn * C1 is exact.
  float r = x - fn * 0.693359375f;
  r = r - fn * -2.12194440e-4f;
  float z = r * r;
  float p = 1.9875691500e-4f;
  p = p * r + 1.3981999507e-3f;
  p = p * r + 8.3334519073e-3f;
  p = p * r + 4.1665795894e-2f;
  p = p * r + 1.6666665459e-1f;
  p = p * r + 5.0000001201e-1f;
  p = p * z + r;
  p = p + 1.0f;
  if (n > 127) return (p * pow2i(127)) * pow2i(n - 127);
  if (n < -126) return (p * pow2i(n + 64)) * pow2i(-64);
  return p * pow2i(n);
}

__device__ __forceinline__ float logf_(float x) {
  if (x != x) return x;
  if (x < 0.0f) return __builtin_nanf("");
  if (x == 0.0f) return -__builtin_huge_valf();
  if (x == __builtin_huge_valf()) return x;
  int e = 0;
  uint32_t b = __float_as_uint(x);
  if ((b >> 23) == 0u) {  // subnormal input: bring it into the normal range
    x = x * 33554432.0f;
    b = __float_as_uint(x);
    e = -25;
  }
  e += static_cast<int>((b >> 23) & 0xFFu) - 126;
  float m = __uint_as_float((b & 0x007FFFFFu) | 0x3F000000u);  // [0.5, 1)
  if (m < 0.707106781186547524f) {
    e -= 1;
    m = m + m - 1.0f;
  } else {
    m = m - 1.0f;
  }
  float z = m * m;
  float y = 7.0376836292e-2f;
  y = y * m - 1.1514610310e-1f;
  y = y * m + 1.1676998740e-1f;
  y = y * m - 1.2420140846e-1f;
  y = y * m + 1.4249322787e-1f;
  y = y * m - 1.6668057665e-1f;
  y = y * m + 2.0000714765e-1f;
  y = y * m - 2.4999993993e-1f;
  y = y * m + 3.3333331174e-1f;
  y = y * m;
  y = y * z;
  float fe = static_cast<float>(e);
  if (e != 0) y = y + -2.12194440e-4f * fe;
  y = y + -0.5f * z;
  float r = m + y;
  if (e != 0) r = r + 0.693359375f * fe;
  return r;
}

__device__ __forceinline__ float tanhf_(float x) {
  float z = fabsf(x);
  if (z > 44.36141967773437500f) return x > 0.0f ? 1.0f : -1.0f;
  if (z >= 0.625f) {
    float s = expf_(z + z);
    float t = 1.0f - 2.0f / (s + 1.0f);
    return x < 0.0f ? -t : t;
  }
  if (x == 0.0f) return x;
  float y = x * x;
  float p = -5.70498872745e-3f;
  p = p * y + 2.06390887954e-2f;
  p = p * y - 5.37397155531e-2f;
  p = p * y + 1.33314422036e-1f;
  p = p * y - 3.33332819422e-1f;
  p = p * y;
  p = p * x;
  return p + x;
}

__device__ __forceinline__ float sigmoidf_(float x) { return 1.0f / (1.0f + expf_(-x)); }

// log1p and expm1 by Kahan's method (D. Goldberg, "What Every Computer
// Scientist Should Know About Floating-Point Arithmetic", ACM Computing
// Surveys 23(1), 1991, Theorem 4): with u = fl(1 + x), the rounding error of
// the sum cancels in x * (log(u) / (u - 1)); likewise expm1 from u = exp(x)
// as (u - 1) * (x / log(u)). Exact for u == 1; infinities pass through.
__device__ __forceinline__ float log1pf_(float x) {
  const float u = 1.0f + x;
  if (u == 1.0f) return x;
  if (u == __builtin_huge_valf()) return u;
  return x * (logf_(u) / (u - 1.0f));
}

__device__ __forceinline__ float expm1f_(float x) {
  const float u = expf_(x);
  if (u == 1.0f) return x;
  if (u == __builtin_huge_valf()) return u;
  const float um1 = u - 1.0f;
  if (um1 == -1.0f) return -1.0f;
  return um1 * (x / logf_(u));
}

// sin and cos follow Cephes sinf.c / cosf.c (Moshier): |x| is reduced
// modulo pi/4 by the octant j = trunc(|x| * 4/pi), rounded up to even, and
// r = |x| - j * pi/4 with pi/4 split in three (DP1 and DP2 have few
// significant bits, so j * DP1 and j * DP2 are exact while |x| <= 8192);
// the sine or cosine minimax polynomial of r on [-pi/4, pi/4] is chosen by
// octant. Past 8192 the reduction loses precision (Cephes' PLOSS), past
// 2^24 - 1 the result is 0 (TLOSS); infinities and NaN give NaN.
__device__ __forceinline__ float sincos_reduce_(float x, int j) {
  if (x > 8192.0f)
    x = x - static_cast<float>(j) * 0.7853981633974483096f;
  else
    x = ((x - static_cast<float>(j) * 0.78515625f) - static_cast<float>(j) * 2.4187564849853515625e-4f) -
        static_cast<float>(j) * 3.77489497744594108e-8f;
  return x;
}

__device__ __forceinline__ float sin_poly_(float x, float z) {
  float r = ((-1.9515295891e-4f * z + 8.3321608736e-3f) * z - 1.6666654611e-1f) * z * x;
  return r + x;
}

__device__ __forceinline__ float cos_poly_(float z) {
  float r = ((2.443315711809948e-5f * z - 1.388731625493765e-3f) * z + 4.166664568298827e-2f) * z * z;
  r = r - 0.5f * z;
  return r + 1.0f;
}

__device__ __forceinline__ float cosf_(float xx) {
  if (xx != xx) return xx;
  const float x = fabsf(xx);
  if (x == __builtin_huge_valf()) return __builtin_nanf("");
  if (x > 16777215.0f) return 0.0f;
  int j = static_cast<int>(1.27323954473516f * x);
  int y = j;
  if (j & 1) {
    j += 1;
    y += 1;
  }
  j &= 7;
  bool neg = false;
  if (j > 3) {
    j -= 4;
    neg = true;
  }
  if (j > 1) neg = !neg;
  const float r = sincos_reduce_(x, y);
  const float z = r * r;
  const float v = (j == 1 || j == 2) ? sin_poly_(r, z) : cos_poly_(z);
  return neg ? -v : v;
}

__device__ __forceinline__ float sinf_(float xx) {
  if (xx != xx) return xx;
  bool neg = (__float_as_uint(xx) >> 31) != 0u;  // sin(-0) = -0
  const float x = fabsf(xx);
  if (x == __builtin_huge_valf()) return __builtin_nanf("");
  if (x > 16777215.0f) return 0.0f;
  int j = static_cast<int>(1.27323954473516f * x);
  int y = j;
  if (j & 1) {
    j += 1;
    y += 1;
  }
  j &= 7;
  if (j > 3) {
    neg = !neg;
    j -= 4;
  }
  const float r = sincos_reduce_(x, y);
  const float z = r * r;
  const float v = (j == 1 || j == 2) ? cos_poly_(z) : sin_poly_(r, z);
  return neg ? -v : v;
}

// jnp.maximum / jnp.minimum: NaN in either operand propagates.
__device__ __forceinline__ float fmax_nan(float a, float b) {
  if (a != a) return a;
  if (b != b) return b;
  return a > b ? a : b;
}
__device__ __forceinline__ float fmin_nan(float a, float b) {
  if (a != a) return a;
  if (b != b) return b;
  return a < b ? a : b;
}

// float32(b) ** float32(t) for Adam's bias correction: an integer-valued t in
// [0, 2^24] is raised by binary exponentiation in float64 and rounded once
// (each double product is correctly rounded, so the bits are fixed); any other
// t falls back to the device powf.
__device__ __forceinline__ float pow_step(float b, float t) {
  if (t >= 0.0f && t <= 16777216.0f && floorf(t) == t) {
    uint32_t n = static_cast<uint32_t>(t);
    double base = static_cast<double>(b), acc = 1.0;
    while (n) {
      if (n & 1u) acc *= base;
      base *= base;
      n >>= 1;
    }
    return static_cast<float>(acc);
  }
  return powf(b, t);
}

}  // namespace px
