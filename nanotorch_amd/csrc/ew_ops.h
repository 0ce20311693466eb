// Elementwise functors: the per-element arithmetic of the forward ops
// (elementwise.hip) and of the fused backward kernels (backward.hip), kept
// in one header so that every kernel built on ew_engine.h evaluates the same
// rounding chains.
//
// Forward arithmetic follows the reference's functors exactly:
//   src/cpp/ops/unary_ops.cu:40-58 (int_pow / PowOp), :101-107 (unary)
//   src/cpp/ops/binary_ops.cu:107-113 (binary and comparisons)
//   src/cpp/storage.cpp:55-61 (casts: bool is s != 0, else static_cast)
// Backward chains (the reference's Python compositions, one fp32/fp64
// rounding per step; accumulate mode adds `old + term` with one rounding,
// src/cpp/ops/inplace_ops.cu:75):
//   neg      g * -1                               ops_unary.py:32-33
//   exp      g * y                                ops_unary.py:69-70
//   log      g * pow(x, -1)      = g * (1 / x)    ops_unary.py:105-106
//   sqrt     (g * 0.5) * pow(y, -1)               ops_unary.py:142-144
//   tanh     g * (1 - pow(y, 2)) = g * (1 - y*y)  ops_unary.py:180-182
//   sigmoid  (g * y) * (1 - y)                    ops_unary.py:218-220
//   relu     g * float(y > 0)                     ops_unary.py:287-289
//   pow      (g * e) * pow(x, e - 1)              ops_unary.py:264-266
//   add      (g, g)                               ops_binary.py:49-50
//   sub      (g, g * -1)                          ops_binary.py:95-100
//   mul      (b * g, a * g)                       ops_binary.py:145-150
//   div      (g / b, ((-a) / pow(b, 2)) * g)      ops_binary.py:197-202
// pow(v, -1) and pow(v, 2) are evaluated as 1 / v and v * v (correctly
// rounded); see backward.hip for how that relates to the reference's powf.
// fp32 division and square root are correctly rounded
// (-fhip-fp32-correctly-rounded-divide-sqrt) and nothing is contracted into
// FMA (-ffp-contract=off), so +,-,*,/,sqrt match the host bit for bit.
#pragma once

#include "ew_engine.h"
#include "nt_math.h"

namespace nt {

// --------------------------------------------------------- device math

__device__ __forceinline__ float d_exp(float a) { return expf(a); }
__device__ __forceinline__ double d_exp(double a) { return exp(a); }
__device__ __forceinline__ float d_log(float a) { return logf(a); }
__device__ __forceinline__ double d_log(double a) { return log(a); }
__device__ __forceinline__ float d_sqrt(float a) { return sqrtf(a); }
__device__ __forceinline__ double d_sqrt(double a) { return sqrt(a); }
__device__ __forceinline__ float d_tanh(float a) { return tanhf(a); }
__device__ __forceinline__ double d_tanh(double a) { return tanh(a); }

// Square-and-multiply for integer dtypes (reference: int_pow,
// src/cpp/ops/unary_ops.cu:40-49).
template <class T> __device__ __forceinline__ T int_pow(T a, T n) {
  T r = 1;
  while (n > 0) {
    if (n & 1)
      r *= a;
    a *= a;
    n >>= 1;
  }
  return r;
}

// ------------------------------------------------------------ functors

template <int OP, class T> struct UnaryFwd {
  T e; // exponent for NT_POW, as the reference's value.item<T>()
  PowPlan plan;
  static constexpr bool heavy = OP == NT_TANH || OP == NT_SIGMOID;
  __device__ __forceinline__ void operator()(const T (&x)[1], T (&y)[1]) const {
    const T a = x[0];
    if constexpr (OP == NT_EXP)
      y[0] = d_exp(a);
    else if constexpr (OP == NT_LOG)
      y[0] = d_log(a);
    else if constexpr (OP == NT_NEG)
      y[0] = -a;
    else if constexpr (OP == NT_RELU)
      y[0] = (a >= 0) ? a : T(0);
    else if constexpr (OP == NT_SQRT)
      y[0] = d_sqrt(a);
    else if constexpr (OP == NT_TANH)
      y[0] = d_tanh(a);
    else if constexpr (OP == NT_SIGMOID)
      y[0] = T(1) / (T(1) + d_exp(-a));
    else if constexpr (OP == NT_POW) {
      if constexpr (std::is_integral_v<T>)
        y[0] = int_pow(a, e);
      else
        y[0] = pow_planned(a, e, plan);
    }
  }
};

template <int OP, class T> struct BinaryFwd {
  __device__ __forceinline__ void operator()(const T (&x)[2], T (&y)[1]) const {
    const T a = x[0], b = x[1];
    if constexpr (OP == NT_ADD)
      y[0] = a + b;
    else if constexpr (OP == NT_SUB)
      y[0] = a - b;
    else if constexpr (OP == NT_MUL)
      y[0] = a * b;
    else if constexpr (OP == NT_DIV)
      y[0] = a / b;
  }
};

template <int OP, class T> struct CompareFwd {
  __device__ __forceinline__ void operator()(const T (&x)[2],
                                             bool (&y)[1]) const {
    if constexpr (OP == NT_EQ)
      y[0] = x[0] == x[1];
    else if constexpr (OP == NT_GT)
      y[0] = x[0] > x[1];
    else
      y[0] = x[0] >= x[1];
  }
};

template <class TI, class TO> struct CastOp {
  __device__ __forceinline__ void operator()(const TI (&x)[1],
                                             TO (&y)[1]) const {
    if constexpr (std::is_same_v<TO, bool>)
      y[0] = (x[0] != TI(0));
    else
      y[0] = static_cast<TO>(x[0]);
  }
};

template <int OP> constexpr bool unary_uses_saved() { return OP != NT_NEG; }

template <int OP, class T, bool ACC> struct UnaryBwd {
  T e;   // pow exponent (already rounded as the reference's fp32 tensor)
  T em1; // e - 1 formed in fp32
  PowPlan plan; // evaluation plan for pow(x, em1)
  // pow's backward evaluates a general power (x^1.5 for the config's 2.5):
  // heavy (ew_heavy), so a transposed first-write backward keeps 64 x 128
  // tiles (39.5 us against 48 us in 128 x 128 on [4096, 4096]).
  static constexpr bool heavy = OP == NT_POW;
  static constexpr bool S = unary_uses_saved<OP>();
  static constexpr int NI = 1 + (S ? 1 : 0) + (ACC ? 1 : 0);
  __device__ __forceinline__ void operator()(const T (&x)[NI],
                                             T (&y)[1]) const {
    const T g = x[0];
    const T s = S ? x[1] : T(0);
    T t;
    if constexpr (OP == NT_NEG)
      t = g * T(-1);
    else if constexpr (OP == NT_EXP)
      t = g * s;
    else if constexpr (OP == NT_LOG)
      t = g * (T(1) / s);
    else if constexpr (OP == NT_SQRT)
      t = (g * T(0.5)) * (T(1) / s);
    else if constexpr (OP == NT_TANH)
      t = g * (T(1) - s * s);
    else if constexpr (OP == NT_SIGMOID)
      t = (g * s) * (T(1) - s);
    else if constexpr (OP == NT_RELU)
      t = g * (s > T(0) ? T(1) : T(0));
    else
      t = (g * e) * pow_planned(s, em1, plan);
    if constexpr (ACC)
      y[0] = x[NI - 1] + t;
    else
      y[0] = t;
  }
};

// Gradients of a binary op.  NA / NB: which gradients are produced; AA / AB:
// accumulate into them.  Inputs, in order: g, a (if read), b (if read),
// ga_old (if NA && AA), gb_old (if NB && AB).
template <int OP, class T, bool NA, bool NB, bool AA, bool AB>
struct BinaryBwd {
  static constexpr bool UA = (OP == NT_MUL || OP == NT_DIV) && NB;
  static constexpr bool UB =
      (OP == NT_MUL && NA) || (OP == NT_DIV && (NA || NB));
  static constexpr int IA = 1;
  static constexpr int IB = 1 + (UA ? 1 : 0);
  static constexpr int IGA = IB + (UB ? 1 : 0);
  static constexpr int IGB = IGA + ((NA && AA) ? 1 : 0);
  static constexpr int NI = IGB + ((NB && AB) ? 1 : 0);
  static constexpr int NO = (NA ? 1 : 0) + (NB ? 1 : 0);
  __device__ __forceinline__ void operator()(const T (&x)[NI],
                                             T (&y)[NO]) const {
    const T g = x[0];
    const T a = UA ? x[IA] : T(0);
    const T b = UB ? x[IB] : T(0);
    T ta = T(0), tb = T(0);
    if constexpr (OP == NT_ADD) {
      ta = g;
      tb = g;
    } else if constexpr (OP == NT_SUB) {
      ta = g;
      tb = g * T(-1);
    } else if constexpr (OP == NT_MUL) {
      ta = b * g;
      tb = a * g;
    } else {
      if constexpr (NA)
        ta = g / b;
      if constexpr (NB)
        tb = ((-a) / (b * b)) * g;
    }
    int o = 0;
    if constexpr (NA) {
      if constexpr (AA)
        y[o] = x[IGA] + ta;
      else
        y[o] = ta;
      ++o;
    }
    if constexpr (NB) {
      if constexpr (AB)
        y[o] = x[IGB] + tb;
      else
        y[o] = tb;
    }
  }
};

} // namespace nt
