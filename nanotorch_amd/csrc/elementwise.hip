// Forward elementwise ops: unary (exp/log/neg/relu/sqrt/tanh/sigmoid/pow),
// binary (add/sub/mul/div and the ==, >, >= comparisons), in-place updates,
// casts/strided copies and whole-tensor equality.  All run through the
// elementwise engine (ew_engine.h).
//
// Arithmetic follows the reference's functors exactly:
//   src/cpp/ops/unary_ops.cu:40-58 (int_pow / PowOp), :101-107 (unary)
//   src/cpp/ops/binary_ops.cu:107-113 (binary and comparisons)
//   src/cpp/ops/inplace_ops.cu:75-79 (in-place)
//   src/cpp/storage.cpp:55-61 (casts: bool is s != 0, else static_cast)
// fp32 division and square root are correctly rounded
// (-fhip-fp32-correctly-rounded-divide-sqrt) and nothing is contracted into
// FMA (-ffp-contract=off), so +,-,*,/,sqrt match the host bit for bit.
#include "ew_ops.h"

namespace nt {

// ------------------------------------------------------------ host side

namespace {

template <int OP, class T> void run_unary(const nt_view *x, double scalar,
                                          const nt_view *out) {
  const T e = static_cast<T>(scalar);
  UnaryFwd<OP, T> f{e, make_pow_plan(double(e))};
  const nt_view *ins[1] = {x};
  const nt_view *outs[1] = {out};
  launch_elementwise<T, T, 1, 1>(ins, outs, f);
}

template <int OP> void unary_float(const nt_view *x, double s,
                                   const nt_view *out) {
  dispatch_float(x->dtype, [&]<class T>() { run_unary<OP, T>(x, s, out); });
}

template <int OP> void unary_arith(const nt_view *x, double s,
                                   const nt_view *out) {
  dispatch_arith(x->dtype, [&]<class T>() { run_unary<OP, T>(x, s, out); });
}

template <int OP> void binary_all(const nt_view *a, const nt_view *b,
                                  const nt_view *out) {
  dispatch_all(a->dtype, [&]<class T>() {
    const nt_view *ins[2] = {a, b};
    const nt_view *outs[1] = {out};
    launch_elementwise<T, T, 2, 1>(ins, outs, BinaryFwd<OP, T>{});
  });
}

template <int OP> void binary_arith(const nt_view *a, const nt_view *b,
                                    const nt_view *out) {
  dispatch_arith(a->dtype, [&]<class T>() {
    const nt_view *ins[2] = {a, b};
    const nt_view *outs[1] = {out};
    launch_elementwise<T, T, 2, 1>(ins, outs, BinaryFwd<OP, T>{});
  });
}

template <int OP> void compare_all(const nt_view *a, const nt_view *b,
                                   const nt_view *out) {
  dispatch_all(a->dtype, [&]<class T>() {
    const nt_view *ins[2] = {a, b};
    const nt_view *outs[1] = {out};
    launch_elementwise<T, bool, 2, 1>(ins, outs, CompareFwd<OP, T>{});
  });
}

void binary_dispatch(int op, const nt_view *a, const nt_view *b,
                     const nt_view *out, const char *fname) {
  check_view(a, fname);
  check_view(b, fname);
  check_view(out, fname);
  require_same_shape(a, b, fname);
  require_same_shape(a, out, fname);
  require_same_dtype(a, b, fname);
  const bool cmp = (op == NT_EQ || op == NT_GT || op == NT_GE);
  if (cmp ? out->dtype != NT_BOOL : out->dtype != a->dtype)
    fail(NT_ERR_RUNTIME, std::string(fname) + ": output dtype mismatch");
  switch (op) {
  case NT_ADD:
    return binary_all<NT_ADD>(a, b, out);
  case NT_SUB:
    return binary_all<NT_SUB>(a, b, out);
  case NT_MUL:
    return binary_all<NT_MUL>(a, b, out);
  case NT_DIV:
    return binary_arith<NT_DIV>(a, b, out);
  case NT_EQ:
    return compare_all<NT_EQ>(a, b, out);
  case NT_GT:
    return compare_all<NT_GT>(a, b, out);
  case NT_GE:
    return compare_all<NT_GE>(a, b, out);
  }
  fail(NT_ERR_VALUE, std::string(fname) + ": unknown op");
}

template <class T> struct NotEqualFlag {
  __device__ __forceinline__ void operator()(const T (&x)[2],
                                             bool (&y)[1]) const {
    y[0] = !(x[0] == x[1]);
  }
};

__global__ void any_true_kernel(const bool *v, int64_t n, int *flag) {
  const int64_t stride = int64_t(gridDim.x) * blockDim.x;
  bool any = false;
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += stride)
    any |= v[i];
  if (any)
    atomicOr(flag, 1);
}

} // namespace
} // namespace nt

using namespace nt;

extern "C" {

int nt_copy(const nt_view *src, const nt_view *dst) {
  return guard_ew([&] {
    check_view(src, "copy");
    check_view(dst, "copy");
    require_same_shape(src, dst, "copy");
    dispatch_all(src->dtype, [&]<class TI>() {
      dispatch_all(dst->dtype, [&]<class TO>() {
        const nt_view *ins[1] = {src};
        const nt_view *outs[1] = {dst};
        launch_elementwise<TI, TO, 1, 1>(ins, outs, CastOp<TI, TO>{});
      });
    });
  });
}

int nt_unary(int32_t op, const nt_view *x, double scalar, const nt_view *out) {
  return guard_ew([&] {
    check_view(x, "unary");
    check_view(out, "unary");
    require_same_shape(x, out, "unary");
    require_same_dtype(x, out, "unary");
    switch (op) {
    case NT_EXP:
      return unary_float<NT_EXP>(x, scalar, out);
    case NT_LOG:
      return unary_float<NT_LOG>(x, scalar, out);
    case NT_NEG:
      return unary_arith<NT_NEG>(x, scalar, out);
    case NT_RELU:
      return unary_arith<NT_RELU>(x, scalar, out);
    case NT_SQRT:
      return unary_float<NT_SQRT>(x, scalar, out);
    case NT_TANH:
      return unary_float<NT_TANH>(x, scalar, out);
    case NT_SIGMOID:
      return unary_float<NT_SIGMOID>(x, scalar, out);
    case NT_POW:
      return unary_arith<NT_POW>(x, scalar, out);
    }
    fail(NT_ERR_VALUE, "unary: unknown op");
  });
}

int nt_binary(int32_t op, const nt_view *a, const nt_view *b,
              const nt_view *out) {
  return guard_ew([&] { binary_dispatch(op, a, b, out, "_dispatch_binary"); });
}

int nt_inplace(int32_t op, const nt_view *out, const nt_view *other) {
  return guard_ew([&] {
    check_view(out, "_dispatch_inplace_apply");
    check_view(other, "_dispatch_inplace_apply");
    require_same_dtype(out, other, "_dispatch_inplace_apply");
    require_same_shape(out, other, "_dispatch_inplace_apply");
    if (op == NT_COPY) {
      dispatch_all(out->dtype, [&]<class T>() {
        const nt_view *ins[1] = {other};
        const nt_view *outs[1] = {out};
        launch_elementwise<T, T, 1, 1>(ins, outs, CastOp<T, T>{});
      });
      return;
    }
    if (op != NT_ADD && op != NT_SUB && op != NT_MUL && op != NT_DIV)
      fail(NT_ERR_VALUE, "inplace: unknown op");
    binary_dispatch(op, out, other, out, "_dispatch_inplace_apply");
  });
}

int nt_equals(const nt_view *a, const nt_view *b, int32_t *result) {
  return guard([&] {
    check_view(a, "equals");
    check_view(b, "equals");
    require_same_shape(a, b, "equals");
    require_same_dtype(a, b, "equals");
    const int64_t n = numel(a);
    if (n == 0) {
      *result = 1;
      return;
    }
    // Materialise a != b as a bool mask, then OR-reduce it into a flag.
    DeviceScratch mask_buf{size_t(n)}, flag_buf{sizeof(int)};
    void *mask = mask_buf.get();
    void *flag = flag_buf.get();
    nt_view mv{};
    mv.data = mask;
    mv.dtype = NT_BOOL;
    mv.ndim = a->ndim;
    int64_t st = 1;
    for (int d = a->ndim - 1; d >= 0; --d) {
      mv.shape[d] = a->shape[d];
      mv.strides[d] = st;
      st *= a->shape[d];
    }
    dispatch_all(a->dtype, [&]<class T>() {
      const nt_view *ins[2] = {a, b};
      const nt_view *outs[1] = {&mv};
      launch_elementwise<T, bool, 2, 1>(ins, outs, NotEqualFlag<T>{});
    });
    if (nt_fill(flag, NT_INT32, 1, 0.0) != NT_OK)
      fail(NT_ERR_RUNTIME, nt_last_error());
    const int64_t blocks = std::min<int64_t>((n + 255) / 256, 4096);
    any_true_kernel<<<dim3(unsigned(blocks)), 256, 0, stream()>>>(
        static_cast<const bool *>(mask), n, static_cast<int *>(flag));
    NT_LAUNCH_CHECK();
    int host_flag = 0;
    NT_HIP_CHECK(hipMemcpyAsync(&host_flag, flag, sizeof(int),
                                hipMemcpyDeviceToHost, stream()));
    NT_HIP_CHECK(hipStreamSynchronize(stream()));
    *result = host_flag ? 0 : 1;
  });
}

} // extern "C"
