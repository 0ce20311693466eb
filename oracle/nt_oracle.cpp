// nt_oracle -- CPU restatement of the reference's CPU kernels.  TEST
// INFRASTRUCTURE ONLY: used by tests/, by __graft_entry__.smoke() and by the
// cpu_baseline leg of bench.py as the checker and the CPU baseline.  Nothing
// in the nanotorch_amd package loads it.
//
// Every loop follows the reference's CPU code path element for element:
//   unary     src/cpp/ops/unary_ops.cu:6-17 (loop), :40-58 (int_pow/PowOp),
//             :101-107 (ops: exp, log, neg, relu, sqrt, tanh, sigmoid)
//   binary    src/cpp/ops/binary_ops.cu:6-20 (loop), :107-113 (ops)
//   in-place  src/cpp/ops/inplace_ops.cu:6-16 (loop), :75-79 (ops)
//   cast      src/cpp/storage.cpp:47-65 (bool: s ? 1 : 0, else static_cast)
//   reduce    src/cpp/ops/reduction_ops.cu:8-76 (MatItem, combine ops,
//             sequential loop), :183-233 (keep/drop views)
//   matmul    src/cpp/ops/matmul.cu:21-57 (sequential k dot product)
//   unravel   src/cpp/tensor_view.cuh:42-52
//   uniform   src/cpp/factory.cu:73-83 with src/cpp/random.h:5-13: one
//             std::mt19937_64 drawn through std::uniform_real_distribution<T>
//             element by element (the standard library of this compiler,
//             libstdc++, is the reference's dependency for this path)
// The logical index walks row-major order; outputs are contiguous.
// Built with -O3 -ffp-contract=off and no fast-math, so each + - * / is one
// IEEE rounding as in the reference, and the std:: math calls resolve to the
// host libm exactly as the reference's CPU path does.
//
// or_matmul_omp computes each output with the same sequential k loop as
// or_matmul -- acc = 0, then acc = acc + a_k * b_k for k = 0, 1, ..., K-1,
// one rounding per * and per + -- but in a cache-blocked i-k-j order spread
// over OpenMP threads: the k order of every output is unchanged, so the result
// is bit-identical to or_matmul (vector width changes nothing either: each
// lane is one output).
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <limits>
#include <random>
#include <stdexcept>
#include <string>
#include <type_traits>
#include <vector>

#ifdef _OPENMP
#include <omp.h>
#endif
#include <immintrin.h>

extern "C" {
typedef struct or_view {
  void *data;
  int64_t offset;
  int32_t dtype; // 0 bool, 1 int32, 2 int64, 3 float32, 4 float64
  int32_t ndim;
  int64_t shape[8];
  int64_t strides[8];
} or_view;
}

namespace {

thread_local std::string g_err;

template <class F> int guard(F &&f) {
  try {
    f();
    return 0;
  } catch (const std::invalid_argument &e) {
    g_err = e.what();
    return 2;
  } catch (const std::exception &e) {
    g_err = e.what();
    return 1;
  }
}

template <class F> void dispatch_all(int dt, F &&f) {
  switch (dt) {
  case 0:
    return f.template operator()<bool>();
  case 1:
    return f.template operator()<int32_t>();
  case 2:
    return f.template operator()<int64_t>();
  case 3:
    return f.template operator()<float>();
  case 4:
    return f.template operator()<double>();
  }
  throw std::invalid_argument("Unknown dtype.");
}
template <class F> void dispatch_float(int dt, F &&f) {
  if (dt == 3)
    return f.template operator()<float>();
  if (dt == 4)
    return f.template operator()<double>();
  throw std::invalid_argument("Invalid dtype.");
}
template <class F> void dispatch_arith(int dt, F &&f) {
  switch (dt) {
  case 1:
    return f.template operator()<int32_t>();
  case 2:
    return f.template operator()<int64_t>();
  case 3:
    return f.template operator()<float>();
  case 4:
    return f.template operator()<double>();
  }
  throw std::invalid_argument("Invalid dtype.");
}

int64_t numel(const or_view &v) {
  int64_t n = 1;
  for (int i = 0; i < v.ndim; ++i)
    n *= v.shape[i];
  return n;
}

// tensor_view.cuh:42-52
int64_t unravel(int64_t i, const or_view &v) {
  int64_t idx = v.offset;
  for (int64_t j = v.ndim - 1; j >= 0; --j) {
    int64_t coord = i % v.shape[j];
    i /= v.shape[j];
    idx += coord * v.strides[j];
  }
  return idx;
}

void same_shape(const or_view &a, const or_view &b) {
  if (a.ndim != b.ndim)
    throw std::runtime_error("shape mismatch");
  for (int i = 0; i < a.ndim; ++i)
    if (a.shape[i] != b.shape[i])
      throw std::runtime_error("shape mismatch");
}

template <class T> T int_pow(T a, T n) {
  T r = 1;
  while (n > 0) {
    if (n & 1)
      r *= a;
    a *= a;
    n >>= 1;
  }
  return r;
}

template <class T> T unary_apply(int op, T a, T e) {
  switch (op) {
  case 0:
    if constexpr (std::is_floating_point_v<T>)
      return std::exp(a);
    break;
  case 1:
    if constexpr (std::is_floating_point_v<T>)
      return std::log(a);
    break;
  case 2:
    return -a;
  case 3:
    return (a >= 0) ? a : 0;
  case 4:
    if constexpr (std::is_floating_point_v<T>)
      return std::sqrt(a);
    break;
  case 5:
    if constexpr (std::is_floating_point_v<T>)
      return std::tanh(a);
    break;
  case 6:
    if constexpr (std::is_floating_point_v<T>)
      return T(1) / (T(1) + std::exp(-a));
    break;
  case 7:
    if constexpr (std::is_integral_v<T>)
      return int_pow(a, e);
    else
      return std::pow(a, e);
  }
  throw std::invalid_argument("Invalid dtype.");
}

template <class T> T binary_apply(int op, T a, T b) {
  switch (op) {
  case 0:
    return a + b;
  case 1:
    return a - b;
  case 2:
    return a * b;
  case 3:
    return a / b;
  }
  throw std::invalid_argument("unknown op");
}

// reduction_ops.cu:8-50
template <class O> struct MatItem {
  int64_t idx;
  O value;
};

template <class O> MatItem<O> combine(int op, MatItem<O> a, MatItem<O> b) {
  if (op == 0)
    return MatItem<O>{-1, static_cast<O>(a.value + b.value)};
  if (op == 1 || op == 3) // max / argmax
    return (a.value > b.value || (a.value == b.value && a.idx < b.idx)) ? a : b;
  return (a.value < b.value || (a.value == b.value && a.idx < b.idx)) ? a : b;
}

template <class O> MatItem<O> neutral(int op) {
  if (op == 0)
    return MatItem<O>{-1, O(0)};
  if (op == 1 || op == 3)
    return MatItem<O>{std::numeric_limits<int64_t>::max(),
                      std::numeric_limits<O>::lowest()};
  return MatItem<O>{std::numeric_limits<int64_t>::max(),
                    std::numeric_limits<O>::max()};
}

} // namespace

// ----------------------------------------------------- blocked product
// C[M,N] = A[M,K] . B[K,N] on packed row-major operands.  C is zeroed first,
// then every C[i][j] receives C[i][j] + A[i][k] * B[k][j] for k = 0, 1, ...
// in increasing order (k blocks in order, k increasing inside a block): the
// per-output operation sequence of the reference's loop (matmul.cu:33-45).
namespace {

constexpr int64_t MB_I = 64, MB_J = 256, MB_K = 256;

// 4 x 64 register tile of C over k in [k0, k1): AVX-512, separate multiply
// and add (no FMA), one output per lane.
__attribute__((target("avx512f"))) void mm_tile4x64_avx512(
    const float *A, const float *B, float *C, int64_t K, int64_t N, int64_t i,
    int64_t j, int64_t k0, int64_t k1) {
  __m512 c[4][4];
  for (int r = 0; r < 4; ++r)
    for (int v = 0; v < 4; ++v)
      c[r][v] = _mm512_loadu_ps(C + (i + r) * N + j + 16 * v);
  for (int64_t k = k0; k < k1; ++k) {
    const float *b = B + k * N + j;
    __m512 b0 = _mm512_loadu_ps(b), b1 = _mm512_loadu_ps(b + 16),
           b2 = _mm512_loadu_ps(b + 32), b3 = _mm512_loadu_ps(b + 48);
    for (int r = 0; r < 4; ++r) {
      __m512 a = _mm512_set1_ps(A[(i + r) * K + k]);
      c[r][0] = _mm512_add_ps(c[r][0], _mm512_mul_ps(a, b0));
      c[r][1] = _mm512_add_ps(c[r][1], _mm512_mul_ps(a, b1));
      c[r][2] = _mm512_add_ps(c[r][2], _mm512_mul_ps(a, b2));
      c[r][3] = _mm512_add_ps(c[r][3], _mm512_mul_ps(a, b3));
    }
  }
  for (int r = 0; r < 4; ++r)
    for (int v = 0; v < 4; ++v)
      _mm512_storeu_ps(C + (i + r) * N + j + 16 * v, c[r][v]);
}

template <class T>
void mm_block_scalar(const T *A, const T *B, T *C, int64_t K, int64_t N,
                     int64_t i0, int64_t i1, int64_t j0, int64_t j1, int64_t k0,
                     int64_t k1) {
  for (int64_t i = i0; i < i1; ++i)
    for (int64_t k = k0; k < k1; ++k) {
      const T a = A[i * K + k];
      const T *b = B + k * N;
      T *c = C + i * N;
      for (int64_t j = j0; j < j1; ++j)
        c[j] += a * b[j];
    }
}

template <class T>
void mm_blocked(const T *A, const T *B, T *C, int64_t M, int64_t K,
                int64_t N) {
  for (int64_t x = 0; x < M * N; ++x)
    C[x] = static_cast<T>(0.0);
  bool wide = false;
  if constexpr (std::is_same_v<T, float>)
    wide = __builtin_cpu_supports("avx512f");
  const int64_t nbi = (M + MB_I - 1) / MB_I, nbj = (N + MB_J - 1) / MB_J;
#pragma omp parallel for schedule(dynamic)
  for (int64_t t = 0; t < nbi * nbj; ++t) {
    const int64_t i0 = (t / nbj) * MB_I, j0 = (t % nbj) * MB_J;
    const int64_t i1 = std::min(M, i0 + MB_I), j1 = std::min(N, j0 + MB_J);
    for (int64_t k0 = 0; k0 < K; k0 += MB_K) {
      const int64_t k1 = std::min(K, k0 + MB_K);
      int64_t iv = i0, jv = j0;
      if constexpr (std::is_same_v<T, float>) {
        if (wide) {
          iv = i0 + (i1 - i0) / 4 * 4;
          jv = j0 + (j1 - j0) / 64 * 64;
          for (int64_t i = i0; i < iv; i += 4)
            for (int64_t j = j0; j < jv; j += 64)
              mm_tile4x64_avx512(A, B, C, K, N, i, j, k0, k1);
        }
      }
      // the rest of the block: columns right of the vector tiles, rows below
      mm_block_scalar(A, B, C, K, N, i0, iv, jv, j1, k0, k1);
      mm_block_scalar(A, B, C, K, N, iv, i1, j0, j1, k0, k1);
    }
  }
}

} // namespace

extern "C" {

const char *or_last_error(void) { return g_err.c_str(); }

int or_has_openmp(void) {
#ifdef _OPENMP
  return 1;
#else
  return 0;
#endif
}

int or_max_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

// out: contiguous, same dtype as x.
int or_unary(int32_t op, const or_view *x, double scalar, void *out) {
  return guard([&] {
    auto run = [&]<class T>() {
      const T *in = static_cast<const T *>(x->data);
      T *o = static_cast<T *>(out);
      const T e = static_cast<T>(scalar);
      const int64_t n = numel(*x);
      for (int64_t i = 0; i < n; ++i)
        o[i] = unary_apply<T>(op, in[unravel(i, *x)], e);
    };
    if (op == 2 || op == 3 || op == 7)
      dispatch_arith(x->dtype, run);
    else
      dispatch_float(x->dtype, run);
  });
}

// op 0..3 arithmetic (out dtype = a dtype), 4 ==, 5 >, 6 >= (out bool).
int or_binary(int32_t op, const or_view *a, const or_view *b, void *out) {
  return guard([&] {
    same_shape(*a, *b);
    if (a->dtype != b->dtype)
      throw std::runtime_error("dtype mismatch");
    const int64_t n = numel(*a);
    auto run = [&]<class T>() {
      const T *pa = static_cast<const T *>(a->data);
      const T *pb = static_cast<const T *>(b->data);
      if (op >= 4) {
        bool *o = static_cast<bool *>(out);
        for (int64_t i = 0; i < n; ++i) {
          const T x = pa[unravel(i, *a)], y = pb[unravel(i, *b)];
          o[i] = op == 4 ? (x == y) : op == 5 ? (x > y) : (x >= y);
        }
      } else {
        T *o = static_cast<T *>(out);
        for (int64_t i = 0; i < n; ++i)
          o[i] = static_cast<T>(
              binary_apply<T>(op, pa[unravel(i, *a)], pb[unravel(i, *b)]));
      }
    };
    if (op == 3)
      dispatch_arith(a->dtype, run);
    else
      dispatch_all(a->dtype, run);
  });
}

// out = out (op) other in place; op 0..3, 7 = copy.
int or_inplace(int32_t op, const or_view *out, const or_view *other) {
  return guard([&] {
    same_shape(*out, *other);
    if (out->dtype != other->dtype)
      throw std::runtime_error("dtype mismatch");
    const int64_t n = numel(*out);
    auto run = [&]<class T>() {
      T *po = static_cast<T *>(out->data);
      const T *px = static_cast<const T *>(other->data);
      for (int64_t i = 0; i < n; ++i) {
        const int64_t io = unravel(i, *out);
        const T b = px[unravel(i, *other)];
        po[io] = op == 7 ? b : static_cast<T>(binary_apply<T>(op, po[io], b));
      }
    };
    if (op == 3)
      dispatch_arith(out->dtype, run);
    else
      dispatch_all(out->dtype, run);
  });
}

// dst (contiguous, dtype dst_dtype) = cast(src view).
int or_cast(const or_view *src, int32_t dst_dtype, void *dst) {
  return guard([&] {
    const int64_t n = numel(*src);
    dispatch_all(src->dtype, [&]<class S>() {
      dispatch_all(dst_dtype, [&]<class D>() {
        const S *s = static_cast<const S *>(src->data);
        D *d = static_cast<D *>(dst);
        for (int64_t i = 0; i < n; ++i) {
          const S v = s[unravel(i, *src)];
          if constexpr (std::is_same_v<D, bool>)
            d[i] = v ? D{1} : D{0};
          else
            d[i] = static_cast<D>(v);
        }
      });
    });
  });
}

// op 0 sum (accumulation dtype out_dtype), 1 max, 2 min (out dtype = x),
// 3 argmax, 4 argmin (int64).  out contiguous over the kept axes.
int or_reduce(int32_t op, const or_view *x, const int64_t *axes, int32_t naxes,
              int32_t out_dtype, void *out) {
  return guard([&] {
    std::vector<bool> drop(x->ndim, false);
    or_view keep{}, dv{};
    keep.offset = x->offset;
    for (int i = 0; i < naxes; ++i) {
      if (axes[i] < 0 || axes[i] >= x->ndim || drop[axes[i]])
        throw std::runtime_error("bad axes");
      drop[axes[i]] = true;
      dv.shape[dv.ndim] = x->shape[axes[i]];
      dv.strides[dv.ndim] = x->strides[axes[i]];
      dv.ndim++;
    }
    for (int d = 0; d < x->ndim; ++d)
      if (!drop[d]) {
        keep.shape[keep.ndim] = x->shape[d];
        keep.strides[keep.ndim] = x->strides[d];
        keep.ndim++;
      }
    const int64_t nk = numel(keep), nd = numel(dv);
    if (op == 1 || op == 2)
      out_dtype = x->dtype;
    dispatch_all(x->dtype, [&]<class T>() {
      const T *in = static_cast<const T *>(x->data);
      auto body = [&]<class O>() {
        for (int64_t i = 0; i < nk; ++i) {
          const int64_t base = unravel(i, keep);
          MatItem<O> acc = neutral<O>(op);
          for (int64_t j = 0; j < nd; ++j)
            acc = combine<O>(
                op, acc,
                MatItem<O>{j, static_cast<O>(in[base + unravel(j, dv)])});
          if (op >= 3)
            static_cast<int64_t *>(out)[i] = acc.idx;
          else
            static_cast<O *>(out)[i] = acc.value;
        }
      };
      if (op == 0)
        dispatch_arith(out_dtype, body);
      else
        body.template operator()<T>();
    });
  });
}

static int matmul_impl(const or_view *a, const or_view *b, void *out,
                       bool parallel) {
  return guard([&] {
    if (a->dtype != b->dtype || a->ndim != b->ndim || a->ndim < 2)
      throw std::invalid_argument("matmul: bad operands");
    const int nd = a->ndim;
    for (int d = 0; d < nd - 2; ++d)
      if (a->shape[d] != b->shape[d])
        throw std::invalid_argument("Invalid broacast shapes.");
    const int64_t M = a->shape[nd - 2], K = a->shape[nd - 1],
                  N = b->shape[nd - 1];
    if (b->shape[nd - 2] != K)
      throw std::invalid_argument("Invalid matmul shape.");
    std::vector<int64_t> oshape(a->shape, a->shape + nd);
    oshape[nd - 1] = N;
    int64_t total = 1;
    for (auto s : oshape)
      total *= s;
    dispatch_arith(a->dtype, [&]<class T>() {
      const T *A = static_cast<const T *>(a->data);
      const T *B = static_cast<const T *>(b->data);
      T *C = static_cast<T *>(out);
      if (parallel) {
        // Per batch index: pack both operands row-major (a copy, exact),
        // then the blocked product.
        const int64_t nbatch = (M * N) ? total / (M * N) : 0;
        std::vector<T> pa(size_t(M * K)), pb(size_t(K * N));
        for (int64_t bi = 0; bi < nbatch; ++bi) {
          int64_t oa = a->offset, ob = b->offset, r = bi;
          for (int d = nd - 3; d >= 0; --d) {
            const int64_t l = r % oshape[d];
            r /= oshape[d];
            oa += l * a->strides[d];
            ob += l * b->strides[d];
          }
#pragma omp parallel for schedule(static)
          for (int64_t i = 0; i < M; ++i)
            for (int64_t c = 0; c < K; ++c)
              pa[size_t(i * K + c)] =
                  A[oa + i * a->strides[nd - 2] + c * a->strides[nd - 1]];
#pragma omp parallel for schedule(static)
          for (int64_t c = 0; c < K; ++c)
            for (int64_t j = 0; j < N; ++j)
              pb[size_t(c * N + j)] =
                  B[ob + c * b->strides[nd - 2] + j * b->strides[nd - 1]];
          mm_blocked(pa.data(), pb.data(), C + bi * M * N, M, K, N);
        }
        return;
      }
      for (int64_t idx = 0; idx < total; ++idx) {
        // loc = row-major coordinates of output idx (matmul.cu:31-56)
        int64_t loc[8];
        int64_t r = idx;
        for (int d = nd - 1; d >= 0; --d) {
          loc[d] = r % oshape[d];
          r /= oshape[d];
        }
        T acc = static_cast<T>(0.0);
        for (int64_t c = 0; c < K; ++c) {
          int64_t i1 = a->offset + c * a->strides[nd - 1] +
                       loc[nd - 2] * a->strides[nd - 2];
          int64_t i2 = b->offset + c * b->strides[nd - 2] +
                       loc[nd - 1] * b->strides[nd - 1];
          for (int d = 0; d < nd - 2; ++d) {
            i1 += a->strides[d] * loc[d];
            i2 += b->strides[d] * loc[d];
          }
          acc += A[i1] * B[i2];
        }
        C[idx] = acc;
      }
    });
  });
}

int or_matmul(const or_view *a, const or_view *b, void *out) {
  return matmul_impl(a, b, out, false);
}

int or_matmul_omp(const or_view *a, const or_view *b, void *out) {
  return matmul_impl(a, b, out, true);
}

// n draws of uniform_real_distribution<T>(low, high) from a std::mt19937_64
// seeded with `seed`, after dropping the first `skip` engine outputs (one
// draw consumes one output for float and double).
int or_uniform(uint64_t seed, int64_t skip, int64_t n, int32_t dtype,
               double low, double high, void *out) {
  return guard([&] {
    std::mt19937_64 eng(seed);
    eng.discard((unsigned long long)skip);
    if (dtype == 3) {
      std::uniform_real_distribution<float> dist{float(low), float(high)};
      for (int64_t i = 0; i < n; ++i)
        static_cast<float *>(out)[i] = dist(eng);
    } else if (dtype == 4) {
      std::uniform_real_distribution<double> dist{low, high};
      for (int64_t i = 0; i < n; ++i)
        static_cast<double *>(out)[i] = dist(eng);
    } else {
      throw std::invalid_argument("or_uniform: float dtype required");
    }
  });
}

// The k-th (1-based) raw output of std::mt19937_64 seeded with `seed`.
uint64_t or_mt64_output(uint64_t seed, int64_t k) {
  std::mt19937_64 eng(seed);
  if (k > 1)
    eng.discard((unsigned long long)(k - 1));
  return eng();
}

} // extern "C"
