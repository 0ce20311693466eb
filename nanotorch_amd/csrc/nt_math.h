// Device math shared by the forward and backward elementwise kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cmath>
#include <limits>

namespace nt {

// pow(x, e) for a run-time scalar exponent.  The generic path calls the
// device library's powf / pow (about 150 instructions per element, which
// makes the pow kernels compute-bound).  Small integer and half-integer
// exponents, |e| <= 4.5, take a short exact-operation path instead:
//   e = n      : x^|n| from x*x (<= 2 roundings), 1/r if n < 0
//   e = n + .5 : |x^n * sqrt(x)| (fp32: hardware sqrt, 1 ulp), 1/r if e < 0
// Both stay within 4 ulp of the correctly rounded power while every step is
// a normal number.  Any other case -- a zero, subnormal, infinite or NaN
// intermediate or result, which covers x = +-0, +-inf, NaN, x < 0 with a
// half-integer exponent, overflow and underflow -- is recomputed with the
// library pow, so pow's special values and its subnormal results are kept.
// x^0 = 1 for every x, NaN included, as pow defines it.
struct PowPlan {
  int mode = 0; // 0 generic, 1 integer, 2 half-integer
  int n = 0;    // |integer part|
  bool neg = false;
};

inline PowPlan make_pow_plan(double e) {
  PowPlan p;
  const double a = std::fabs(e);
  if (a <= 4.5 && std::floor(e) == e) {
    p.mode = 1;
    p.n = int(a);
    p.neg = e < 0;
  } else if (a <= 4.5 && std::floor(2 * e) == 2 * e) {
    p.mode = 2;
    p.n = int(std::floor(a));
    p.neg = e < 0;
  }
  return p;
}

// Square root for the pow fast path.  fp32: the hardware v_sqrt_f32 (1 ulp,
// one instruction; the correctly rounded sqrtf is a ~40-instruction
// refinement, most of the fast path's cost).  Callers pass normal inputs only.
// fp64: the correctly rounded sqrt.
__device__ __forceinline__ float dev_sqrt(float a) {
  return __builtin_amdgcn_sqrtf(a);
}
__device__ __forceinline__ double dev_sqrt(double a) { return sqrt(a); }
__device__ __forceinline__ float dev_pow(float a, float e) { return powf(a, e); }
__device__ __forceinline__ double dev_pow(double a, double e) {
  return pow(a, e);
}

// The library pow for pow_planned's rare cases, out of line: inlined at every
// unrolled element it made the pow kernels 3x larger, and the transposed
// ones 10-20% slower (measured on the [4096, 4096] sweep).
template <class T> __device__ __noinline__ T pow_fallback(T x, T e) {
  return dev_pow(x, e);
}

template <class T> __device__ __forceinline__ bool is_normal_num(T v) {
  const T a = std::fabs(v);
  return a >= std::numeric_limits<T>::min() &&
         a <= std::numeric_limits<T>::max();
}

// x^n for 0 <= n <= 4 with straight-line code (n is uniform across the
// launch): x*x, (x*x)*x, (x*x)*(x*x) -- at most two roundings.
template <class T> __device__ __forceinline__ T ipow4(T x, int n) {
  const T x2 = x * x;
  const T lo = n == 0 ? T(1) : x;
  const T hi = n == 2 ? x2 : (n == 3 ? x2 * x : x2 * x2);
  return n < 2 ? lo : hi;
}

template <class T>
__device__ __forceinline__ T pow_planned(T x, T e, const PowPlan &p) {
  if (p.mode == 1 && p.n == 0)
    return T(1); // pow(x, +-0) = 1 for every x, NaN included
  if (p.mode != 0) {
    T r = ipow4(x, p.n);
    if (p.mode == 2) // x must be normal for dev_sqrt (else r becomes NaN)
      r = is_normal_num(x) ? std::fabs(r * dev_sqrt(x))
                           : std::numeric_limits<T>::quiet_NaN();
    T res = r;
    if (p.neg) {
      // A uniform branch: the empty volatile asm keeps the compiler from
      // evaluating the (correctly rounded, ~10-instruction) division for
      // positive exponents too.
      asm volatile("" ::: "memory");
      res = T(1) / r;
    }
    // A zero, subnormal, infinite or NaN intermediate or result (x = 0,
    // inf, NaN, x < 0 under a square root, overflow, underflow) takes the
    // library pow below.
    // (Marked unlikely so that the library call's code is laid out after
    // the kernel's hot path instead of between its unrolled elements.)
    if (__builtin_expect(is_normal_num(r) && is_normal_num(res), 1))
      return res;
  }
  return pow_fallback(x, e);
}

} // namespace nt
