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
//   e = n      : x^|n| by square-and-multiply (<= 3 roundings), 1/r if n < 0
//   e = n + .5 : |x^n * sqrt(x)| (sqrt correctly rounded), 1/r if e < 0
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

__device__ __forceinline__ float dev_sqrt(float a) { return sqrtf(a); }
__device__ __forceinline__ double dev_sqrt(double a) { return sqrt(a); }
__device__ __forceinline__ float dev_pow(float a, float e) { return powf(a, e); }
__device__ __forceinline__ double dev_pow(double a, double e) {
  return pow(a, e);
}

template <class T> __device__ __forceinline__ T ipow_small(T x, int n) {
  T r = T(1);
  T b = x;
  while (n > 0) {
    if (n & 1)
      r = r * b;
    n >>= 1;
    if (n)
      b = b * b;
  }
  return r;
}

template <class T> __device__ __forceinline__ bool is_normal_num(T v) {
  const T a = std::fabs(v);
  return a >= std::numeric_limits<T>::min() &&
         a <= std::numeric_limits<T>::max();
}

template <class T>
__device__ __forceinline__ T pow_planned(T x, T e, const PowPlan &p) {
  if (p.mode != 0) {
    if (p.n == 0 && p.mode == 1)
      return T(1);
    T r = ipow_small(x, p.n);
    if (p.mode == 2)
      r = std::fabs(r * dev_sqrt(x));
    const T res = p.neg ? T(1) / r : r;
    if (is_normal_num(x) && is_normal_num(r) && is_normal_num(res))
      return res;
  }
  return dev_pow(x, e);
}

} // namespace nt
