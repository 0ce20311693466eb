// Fused backward of the binary elementwise ops (add / sub / mul / div):
// one pass reads the upstream gradient, the saved operands the op needs
// and, in accumulate mode, the old gradients, and writes the gradients of
// both operands (the BinaryBwd functor of ew_ops.h has the rounding
// chains and their reference citations).  Split from backward.hip so the
// two translation units compile in parallel.
#include "ew_ops.h"

namespace nt {

namespace {

template <int OP, class T, bool NA, bool NB, bool AA, bool AB>
void run_binary_bwd(const nt_view *g, const nt_view *a, const nt_view *b,
                    const nt_view *ga, const nt_view *gb) {
  using F = BinaryBwd<OP, T, NA, NB, AA, AB>;
  const nt_view *ins[F::NI];
  int k = 0;
  ins[k++] = g;
  if (F::UA)
    ins[k++] = a;
  if (F::UB)
    ins[k++] = b;
  if (NA && AA)
    ins[k++] = ga;
  if (NB && AB)
    ins[k++] = gb;
  const nt_view *outs[F::NO > 0 ? F::NO : 1];
  int m = 0;
  if (NA)
    outs[m++] = ga;
  if (NB)
    outs[m++] = gb;
  launch_elementwise<T, T, F::NI, F::NO>(ins, outs, F{});
}

template <int OP, class T>
void binary_bwd_t(const nt_view *g, const nt_view *a, const nt_view *b,
                  const nt_view *ga, bool aa, const nt_view *gb, bool ab) {
  const bool na = ga != nullptr, nb = gb != nullptr;
  if (na && nb) {
    if (aa && ab)
      run_binary_bwd<OP, T, true, true, true, true>(g, a, b, ga, gb);
    else if (aa)
      run_binary_bwd<OP, T, true, true, true, false>(g, a, b, ga, gb);
    else if (ab)
      run_binary_bwd<OP, T, true, true, false, true>(g, a, b, ga, gb);
    else
      run_binary_bwd<OP, T, true, true, false, false>(g, a, b, ga, gb);
  } else if (na) {
    if (aa)
      run_binary_bwd<OP, T, true, false, true, false>(g, a, b, ga, gb);
    else
      run_binary_bwd<OP, T, true, false, false, false>(g, a, b, ga, gb);
  } else if (nb) {
    if (ab)
      run_binary_bwd<OP, T, false, true, false, true>(g, a, b, ga, gb);
    else
      run_binary_bwd<OP, T, false, true, false, false>(g, a, b, ga, gb);
  }
}

} // namespace
} // namespace nt

using namespace nt;

extern "C" {

int nt_binary_bwd(int32_t op, const nt_view *g, const nt_view *a,
                  const nt_view *b, const nt_view *ga, int32_t acc_a,
                  const nt_view *gb, int32_t acc_b) {
  return guard_ew([&] {
    check_view(g, "binary_bwd");
    if (!ga && !gb)
      return;
    const bool reads_ab = (op == NT_MUL || op == NT_DIV);
    if (reads_ab) {
      check_view(a, "binary_bwd");
      check_view(b, "binary_bwd");
      require_same_shape(g, a, "binary_bwd");
      require_same_shape(g, b, "binary_bwd");
      require_same_dtype(g, a, "binary_bwd");
      require_same_dtype(g, b, "binary_bwd");
    }
    for (const nt_view *v : {ga, gb})
      if (v) {
        check_view(v, "binary_bwd");
        require_same_shape(g, v, "binary_bwd");
        require_same_dtype(g, v, "binary_bwd");
      }
    dispatch_float(g->dtype, [&]<class T>() {
      switch (op) {
      case NT_ADD:
        return binary_bwd_t<NT_ADD, T>(g, a, b, ga, acc_a, gb, acc_b);
      case NT_SUB:
        return binary_bwd_t<NT_SUB, T>(g, a, b, ga, acc_a, gb, acc_b);
      case NT_MUL:
        return binary_bwd_t<NT_MUL, T>(g, a, b, ga, acc_a, gb, acc_b);
      case NT_DIV:
        return binary_bwd_t<NT_DIV, T>(g, a, b, ga, acc_a, gb, acc_b);
      }
      fail(NT_ERR_VALUE, "binary_bwd: unknown op");
    });
  });
}

} // extern "C"
