// Fused backward kernels for the elementwise family.
//
// The reference computes every gradient as a Python composition of forward
// kernels, then adds it into the existing gradient with a separate in-place
// kernel (src/nanotorch/autograd/ops_unary.py, ops_binary.py;
// src/nanotorch/core.py:865-871).  Here one pass reads the upstream gradient,
// the saved tensors and (in accumulate mode) the old gradient, and writes the
// new gradient, evaluating the same fp32/fp64 rounding chain:
//
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
//
// pow(v, -1) and pow(v, 2) are evaluated as 1 / v and v * v, the correctly
// rounded values.  The reference calls the host powf there; glibc's powf
// is one ulp off correct rounding for a fraction of a percent of inputs, so
// those chains (log, sqrt, tanh, the b-gradient of div) agree with the
// reference to within that ulp; the others are bit-identical.
// pow(x, e - 1) for a general e stays a pow call; e - 1 is formed in fp32
// as the reference does with its fp32 exponent tensor.  Accumulate mode is
// `old + term` with one rounding, the reference's add_inplace
// (src/cpp/ops/inplace_ops.cu:75).
#include "ew_ops.h"

namespace nt {

namespace {

template <int OP, class T, bool ACC>
void run_unary_bwd(const nt_view *g, const nt_view *s, double scalar,
                   const nt_view *gx) {
  using F = UnaryBwd<OP, T, ACC>;
  const float ef = float(scalar);
  const T em1 = T(ef - 1.0f);
  F f{T(scalar), em1, make_pow_plan(double(em1))};
  const nt_view *ins[F::NI];
  int k = 0;
  ins[k++] = g;
  if (F::S)
    ins[k++] = s;
  if (ACC)
    ins[k++] = gx;
  const nt_view *outs[1] = {gx};
  launch_elementwise<T, T, F::NI, 1>(ins, outs, f);
}

template <int OP, class T>
void unary_bwd_acc(const nt_view *g, const nt_view *s, double scalar,
                   const nt_view *gx, bool acc) {
  if (acc)
    run_unary_bwd<OP, T, true>(g, s, scalar, gx);
  else
    run_unary_bwd<OP, T, false>(g, s, scalar, gx);
}

// p - (g * lr): the multiply kernel's rounding, then sub_inplace's (no
// contraction: the build passes -ffp-contract=off).
struct SgdStep {
  float lr;
  __device__ __forceinline__ void operator()(const float (&x)[2],
                                             float (&y)[1]) const {
    const float t = x[1] * lr;
    y[0] = x[0] - t;
  }
};

} // namespace
} // namespace nt

using namespace nt;

extern "C" {

int nt_unary_bwd(int32_t op, const nt_view *g, const nt_view *saved,
                 double scalar, const nt_view *gx, int32_t accumulate) {
  return guard_ew([&] {
    check_view(g, "unary_bwd");
    check_view(gx, "unary_bwd");
    require_same_shape(g, gx, "unary_bwd");
    require_same_dtype(g, gx, "unary_bwd");
    if (op != NT_NEG) {
      check_view(saved, "unary_bwd");
      require_same_shape(g, saved, "unary_bwd");
      require_same_dtype(g, saved, "unary_bwd");
    }
    const bool acc = accumulate != 0;
    dispatch_float(g->dtype, [&]<class T>() {
      switch (op) {
      case NT_NEG:
        return unary_bwd_acc<NT_NEG, T>(g, saved, scalar, gx, acc);
      case NT_EXP:
        return unary_bwd_acc<NT_EXP, T>(g, saved, scalar, gx, acc);
      case NT_LOG:
        return unary_bwd_acc<NT_LOG, T>(g, saved, scalar, gx, acc);
      case NT_SQRT:
        return unary_bwd_acc<NT_SQRT, T>(g, saved, scalar, gx, acc);
      case NT_TANH:
        return unary_bwd_acc<NT_TANH, T>(g, saved, scalar, gx, acc);
      case NT_SIGMOID:
        return unary_bwd_acc<NT_SIGMOID, T>(g, saved, scalar, gx, acc);
      case NT_RELU:
        return unary_bwd_acc<NT_RELU, T>(g, saved, scalar, gx, acc);
      case NT_POW:
        return unary_bwd_acc<NT_POW, T>(g, saved, scalar, gx, acc);
      }
      fail(NT_ERR_VALUE, "unary_bwd: unknown op");
    });
  });
}

int nt_sgd_step(const nt_view *p, const nt_view *g, double lr) {
  return guard_ew([&] {
    check_view(p, "sgd_step");
    check_view(g, "sgd_step");
    require_same_shape(p, g, "sgd_step");
    require_same_dtype(p, g, "sgd_step");
    if (p->dtype != NT_FLOAT32)
      fail(NT_ERR_VALUE, "sgd_step: float32 parameters only");
    const float lr32 = float(lr);
    if (double(lr32) != lr)
      fail(NT_ERR_VALUE, "sgd_step: lr must be a float32 value");
    const nt_view *ins[2] = {p, g};
    const nt_view *outs[1] = {p};
    launch_elementwise<float, float, 2, 1>(ins, outs, SgdStep{lr32});
  });
}

} // extern "C"
