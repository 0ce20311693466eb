/*
 * nt.h -- C ABI of libnt, the MI355X (gfx950) compute library behind the
 * nanotorch_amd Tensor/autograd API.
 *
 * Every entry point replaces one binding of the reference's pybind11 module
 * `nanotorch._C` (src/cpp/_C.cpp:12-24, typed in src/nanotorch/_C.pyi).  The
 * citation above each declaration names the reference interface it stands in
 * for.  Conventions:
 *
 *  - All tensors are described by `nt_view`: a base pointer to device memory,
 *    an element offset, a dtype and up to NT_MAX_DIMS (shape, element-stride)
 *    pairs.  This is the reference's TensorView (src/cpp/tensor_view.cuh:10-15)
 *    with the storage replaced by a raw pointer.  Strides are in elements and
 *    may be 0 (broadcast) or any positive value.
 *  - The caller allocates and owns every buffer, outputs included.  The
 *    library never keeps a pointer after a call returns.
 *  - Every function returns an nt_status.  On failure a message is kept in
 *    thread-local storage and returned by nt_last_error().  The Python layer
 *    maps NT_ERR_RUNTIME to RuntimeError and NT_ERR_VALUE to ValueError, the
 *    exception types the reference's C++ raises (std::runtime_error and
 *    std::invalid_argument through pybind11).
 *  - All device work is ordered on one HIP stream owned by the library.
 *    Calls return once work is queued; nt_sync() and the device-to-host copy
 *    wait for it.
 *  - Any host thread may call any entry point.  Calls are serialised by one
 *    library-wide (recursive) lock, and the caching allocator has a lock of
 *    its own, so concurrent callers queue their work on the stream one call
 *    at a time.  This is the guarantee the reference's binding gets from the
 *    Python GIL.
 */
#ifndef NT_H_
#define NT_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NT_MAX_DIMS 8

/* Dtype codes; the order is the reference's promotion order
 * (src/cpp/dtype.h:21, `enum class Dtype { Bool, Int32, Int64, Float32,
 * Float64 }`). */
enum nt_dtype {
  NT_BOOL = 0,
  NT_INT32 = 1,
  NT_INT64 = 2,
  NT_FLOAT32 = 3,
  NT_FLOAT64 = 4
};

enum nt_status {
  NT_OK = 0,
  NT_ERR_RUNTIME = 1, /* shape/device/dtype mismatch, HIP errors */
  NT_ERR_VALUE = 2,   /* unsupported dtype for the op, bad matmul shapes */
  NT_ERR_INDEX = 3,
  NT_ERR_OOM = 4
};

/* Unary ops (src/cpp/ops/unary_ops.cu:101-107 and pow :40-73). */
enum nt_unary_op {
  NT_EXP = 0,
  NT_LOG = 1,
  NT_NEG = 2,
  NT_RELU = 3,
  NT_SQRT = 4,
  NT_TANH = 5,
  NT_SIGMOID = 6,
  NT_POW = 7
};

/* Binary ops (src/cpp/ops/binary_ops.cu:107-113); NT_COPY only for
 * nt_inplace (src/cpp/ops/inplace_ops.cu:79). */
enum nt_binary_op {
  NT_ADD = 0,
  NT_SUB = 1,
  NT_MUL = 2,
  NT_DIV = 3,
  NT_EQ = 4,
  NT_GT = 5,
  NT_GE = 6,
  NT_COPY = 7
};

/* Reductions (src/cpp/ops/reduction_ops.cu:13-50); NT_MEAN only for
 * nt_reduce_bwd. */
enum nt_reduce_op {
  NT_SUM = 0,
  NT_MAX = 1,
  NT_MIN = 2,
  NT_ARGMAX = 3,
  NT_ARGMIN = 4,
  NT_MEAN = 5
};

typedef struct nt_view {
  void *data;     /* base of the device allocation */
  int64_t offset; /* element offset of the first element */
  int32_t dtype;  /* enum nt_dtype */
  int32_t ndim;   /* 0 .. NT_MAX_DIMS */
  int64_t shape[NT_MAX_DIMS];
  int64_t strides[NT_MAX_DIMS]; /* element strides */
} nt_view;

/* ---------------------------------------------------------------- runtime */

/* Selects device 0 and creates the library stream.  Called implicitly by
 * every other entry point; safe to call repeatedly. */
int nt_init(void);

/* Replaces `is_cuda_available()` (src/cpp/cuda.h:20-22, cuda.cpp:3-5).
 * Writes 1 if a HIP device can be used, else 0.  Never fails. */
int nt_is_available(int *available);

/* Replaces `cuda_sync()` (src/cpp/cuda.h:24-26, cuda.cpp:6).  Also returns
 * (once) NT_ERR_INDEX when an earlier gather/scatter met an out-of-range
 * index; nt_memcpy_d2h does the same. */
int nt_sync(void);

/* Message of the last failing call on this thread ("" if none). */
const char *nt_last_error(void);

/* Replaces `Storage::allocate` on the CUDA device and the caching allocator
 * behind it (src/cpp/storage.cpp:4-11, src/cpp/allocator.cpp:16-36).  Freed
 * blocks are cached and reused; nt_empty_cache returns them to HIP. */
int nt_malloc(void **ptr, size_t nbytes);
int nt_free(void *ptr);
int nt_empty_cache(void);
int nt_memory_stats(size_t *bytes_in_use, size_t *bytes_cached);

/* Replaces `Storage::to` and `Storage::clone` (src/cpp/storage.cpp:25-45).
 * nt_memcpy_d2h waits for all queued work before copying. */
int nt_memcpy_h2d(void *dst, const void *src, size_t nbytes);
int nt_memcpy_d2h(void *dst, const void *src, size_t nbytes);
int nt_memcpy_d2d(void *dst, const void *src, size_t nbytes);

/* Replaces `zeros/ones/full` on the CUDA device (src/cpp/factory.cu:5-49).
 * Fills n elements of dtype at data with value (cast as static_cast<T>,
 * bool as value != 0). */
int nt_fill(void *data, int32_t dtype, int64_t n, double value);

/* ------------------------------------------------------------ elementwise */

/* Replaces `cast` (src/cpp/storage.cpp:47-65, which round-trips through host
 * memory on CUDA) and `copy_view` / `clone_contiguous_view_from`
 * (src/cpp/ops/copy_ops.cu:187-217).  dst[i] = cast(src[i]) for every logical
 * index i; src and dst have the same shape and any strides and dtypes.  Casts
 * to bool give s != 0, every other cast is static_cast. */
int nt_copy(const nt_view *src, const nt_view *dst);

/* Replaces `exp, log, neg, relu, sqrt, tanh, sigmoid, pow`
 * (src/cpp/ops/unary_ops.cu:59-128).  out[i] = f(x[i]); out has x's shape and
 * dtype and any strides (normally a fresh contiguous buffer).  scalar is the
 * exponent of NT_POW (the reference's `Scalar` argument) and is ignored
 * otherwise.  exp/log/sqrt/tanh/sigmoid need a float dtype, neg/relu/pow an
 * arithmetic dtype (NT_ERR_VALUE otherwise, as DispatchFloat /
 * DispatchArithmetic raise in src/cpp/dtype.h:52,72). */
int nt_unary(int32_t op, const nt_view *x, double scalar, const nt_view *out);

/* Replaces `add, subtract, multiply, divide, pw_equal, pw_greater,
 * pw_greater_eq` (src/cpp/ops/binary_ops.cu:68-113,178-196).  a and b have
 * the same shape and dtype (broadcast operands arrive as stride-0 views);
 * out has that shape and a's dtype, or NT_BOOL for the comparisons.  out may
 * be the same view as a (each element is read before it is written). */
int nt_binary(int32_t op, const nt_view *a, const nt_view *b,
              const nt_view *out);

/* Replaces `add_inplace, sub_inplace, mul_inplace, div_inplace,
 * copy_inplace` (src/cpp/ops/inplace_ops.cu:39-91): out = out (op) other.
 * The storage version bump of the reference (:60) is kept by the caller. */
int nt_inplace(int32_t op, const nt_view *out, const nt_view *other);

/* Replaces `equals` (src/cpp/ops/binary_ops.cu:117-176).  Writes 1 if every
 * element compares equal, else 0. */
int nt_equals(const nt_view *a, const nt_view *b, int32_t *result);

/* ----------------------------------------------------- fused backward ops */

/* Fused backward of one unary op.  The reference has no such kernel: each
 * Op.backward is a Python composition of forward kernels
 * (src/nanotorch/autograd/ops_unary.py:32,69,105,142-144,180-182,218-220,
 * 264-266,287-289) followed by the engine's `x._grad += grad`
 * (src/nanotorch/core.py:865-871).  This computes the same fp32/fp64
 * rounding chain in one pass:
 *   neg:     gx = g * -1
 *   exp:     gx = g * y                      (saved = output y)
 *   log:     gx = g * (1 / x)                (saved = input x)
 *   sqrt:    gx = (g * 0.5) * (1 / y)        (saved = output y)
 *   tanh:    gx = g * (1 - y*y)              (saved = output y)
 *   sigmoid: gx = (g * y) * (1 - y)          (saved = output y)
 *   relu:    gx = g * (y > 0 ? 1 : 0)        (saved = output y)
 *   pow:     gx = (g * e) * pow(x, e - 1)    (saved = input x, scalar = e)
 * With accumulate != 0, gx = gx_old + (that), one rounding, in place.
 * g, saved and gx share one shape and float dtype; saved is ignored for neg. */
int nt_unary_bwd(int32_t op, const nt_view *g, const nt_view *saved,
                 double scalar, const nt_view *gx, int32_t accumulate);

/* Fused backward of one binary op (src/nanotorch/autograd/ops_binary.py:
 * 49-50, 95-100, 145-150, 197-202):
 *   add: ga = g,          gb = g
 *   sub: ga = g,          gb = g * -1
 *   mul: ga = b * g,      gb = a * g
 *   div: ga = g / b,      gb = ((-a) / (b*b)) * g
 * ga or gb may be NULL (that gradient is not needed).  acc_a / acc_b select
 * gx = gx_old + term (in place) instead of gx = term.  All views share one
 * shape (no broadcasting here) and one float dtype. */
int nt_binary_bwd(int32_t op, const nt_view *g, const nt_view *a,
                  const nt_view *b, const nt_view *ga, int32_t acc_a,
                  const nt_view *gb, int32_t acc_b);

/* Fused SGD update of one parameter, in place: p = p - (g * lr).  The
 * reference has no such kernel: `GradientDescent.step` runs
 * `p -= p.grad * lr` under no_grad (src/nanotorch/nn/optimizers.py:45-51),
 * a multiply kernel into a temporary (binary_ops.cu:109) and then
 * `sub_inplace` (src/cpp/ops/inplace_ops.cu:63-79).  This keeps both fp32
 * roundings (the product, then the difference) in one pass and no
 * temporary.  p and g share one shape and the float32 dtype; lr is the
 * float32 value of the step size (the reference's 0-d scalar tensor).  The
 * storage version bump stays with the caller. */
int nt_sgd_step(const nt_view *p, const nt_view *g, double lr);

/* ------------------------------------------------------------- reductions */

/* Replaces `sum, min, max, argmin, argmax` (src/cpp/ops/reduction_ops.cu:
 * 183-276).  axes (naxes >= 1, distinct, in range) are the reduced axes in
 * the caller's order; the reduced index j of an element is its row-major
 * position over those axes in that order, as in the reference (:187-217).
 * out is contiguous with the kept axes' numel:
 *   NT_SUM:           out dtype is the accumulation dtype (any arithmetic)
 *   NT_MAX / NT_MIN:  out dtype = x dtype; first extremum on ties
 *   NT_ARGMAX/ARGMIN: out dtype NT_INT64, the first extremum's j
 * For NT_MAX / NT_MIN, idx (NT_INT64) and count (NT_INT32) may be non-NULL:
 * they receive j of the selected element and how many elements of the slice
 * equal the extremum, which is what nt_reduce_bwd needs. */
int nt_reduce(int32_t op, const nt_view *x, const int64_t *axes, int32_t naxes,
              const nt_view *out, const nt_view *idx, const nt_view *count);

/* Bytes of the static device scratch array of the allocation-free entry
 * points (one array per GPU, held until the process ends). */
#define NT_NOALLOC_SCRATCH_BYTES (16u << 20)

/* nt_reduce without any allocation.  No counterpart in the reference: it is
 * for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Same
 * arguments, results and errors as nt_reduce; the partial results of
 * multi-pass reductions go to the library's static scratch array of
 * NT_NOALLOC_SCRATCH_BYTES instead of the caching allocator, and a
 * reduction that would need more is rejected (NT_ERR_VALUE) -- every plan
 * nt_reduce makes today fits (its largest partial set, max/min along axis 0
 * of a wide tensor, is 8 MiB for fp32).  The library must be initialised
 * first (nt_init or any other call): initialisation allocates, this entry
 * point refuses to do it (NT_ERR_RUNTIME).  Calls that overlap on one GPU
 * share the array and race; host-serialised calls on the library stream
 * (the library's own ordering) do not. */
int nt_reduce_noalloc(int32_t op, const nt_view *x, const int64_t *axes,
                      int32_t naxes, const nt_view *out, const nt_view *idx,
                      const nt_view *count);

/* Backward of the reductions (src/nanotorch/autograd/ops_reduction.py:67-74,
 * 129-138, 201-212, 275-286), fused with the engine's accumulation:
 *   NT_SUM:  gx = g_s                        (broadcast over reduced axes)
 *   NT_MEAN: gx = g_s / scale                (scale = float(n_in / n_out))
 *   NT_MAX / NT_MIN:
 *            gx = g_s * (j == idx_s && count_s == 1 ? 1 : 0)
 *     which is what the reference's mask chain computes: `1 / mask.sum()` is
 *     an int64 division, so slices whose extremum is tied route 0 everywhere.
 * g is contiguous over the kept axes; idx/count as written by nt_reduce.
 * With accumulate != 0: gx = gx_old + term, in place. */
int nt_reduce_bwd(int32_t op, const nt_view *g, double scale, const nt_view *idx,
                  const nt_view *count, const int64_t *axes, int32_t naxes,
                  const nt_view *gx, int32_t accumulate);

/* ----------------------------------------------------------------- matmul */

/* Replaces `matmul` (src/cpp/ops/matmul.cu:207-279): c[..., i, j] =
 * sum_k a[..., i, k] * b[..., k, j] over equal batch dims (broadcast batch
 * dims arrive as stride-0 views).  Operand orientation is read from the
 * strides, so the backward products dA = dG.B^T and dB = A^T.dG
 * (src/nanotorch/autograd/ops_binary.py:253-267) are this call on transposed
 * views, read in place.  fp32 runs on the gfx950 fp32 MFMA units.  With
 * accumulate != 0, c = c_old + (a.b), one rounding after the full sum. */
int nt_matmul(const nt_view *a, const nt_view *b, const nt_view *c,
              int32_t accumulate);

/* No single counterpart in the reference: its Linear layer computes
 * `x @ W + b` as MatmulOp then AddOp, two kernels (src/nanotorch/nn/
 * module.py:73-75 over matmul.cu:207-279 and binary_ops.cu:178).  This is
 * that pair in one call: c[..., i, j] = fl(sum_k a[..., i, k] b[..., k, j])
 * + bias[j], the bias added in the product's epilogue with the same two
 * fp32 roundings (the product's, then the add's).  float32 only
 * (NT_ERR_VALUE otherwise); bias is 1-D with one value per column of c. */
int nt_matmul_bias(const nt_view *a, const nt_view *b, const nt_view *bias,
                   const nt_view *c);

/* --------------------------------------------------------------- indexing */

/* Replaces `gather_from_axes` (src/cpp/ops/copy_ops.cu:93-160, host only in
 * the reference): out (any strides, x's dtype) = x indexed along the view
 * axes fancy_dims_in_src[q] by the int64 arrays index_arrays[q], which all
 * have one shape (the broadcast index shape, any strides).  Output axis i
 * walks index axis out_axis_target[i] when out_axis_is_fancy[i], else view
 * axis out_axis_target[i] -- the plan of the reference's _FancyAxes
 * (src/nanotorch/core.py:667-774).  Indices must already be normalised to
 * [0, axis length).  The call only queues work.  An index outside its axis
 * is caught on the device: its element is not read (out gets 0 there), and
 * the next nt_sync() or nt_memcpy_d2h() returns NT_ERR_INDEX. */
int nt_gather_axes(const nt_view *x, const nt_view *out, int32_t nfancy,
                   const int32_t *fancy_dims_in_src,
                   const nt_view *index_arrays,
                   const int32_t *out_axis_is_fancy,
                   const int32_t *out_axis_target);

/* Replaces `scatter_to_axes` (src/cpp/ops/copy_ops.cu:7-91): out indexed as
 * in nt_gather_axes = src, src having the plan's output shape (any strides,
 * stride 0 for broadcast values).  out is the indexed view itself (the
 * reference passes the whole tensor, which is only right when no basic
 * selector moved the view).  keep, when not NULL, is a bool array of the
 * index shape: positions with keep = 0 are skipped, which the caller uses to
 * keep only the last occurrence of a repeated index tuple (the reference's
 * sequential last-write-wins).  An index outside its axis is skipped and
 * reported as in nt_gather_axes. */
int nt_scatter_axes(const nt_view *src, const nt_view *out, int32_t nfancy,
                    const int32_t *fancy_dims_in_src,
                    const nt_view *index_arrays,
                    const int32_t *out_axis_is_fancy,
                    const int32_t *out_axis_target, const nt_view *keep);

/* ------------------------------------------------------------- host utils */

/* Replaces `manual_seed` / `uniform` (src/cpp/random.h:5-13,
 * src/cpp/factory.cu:73-83): the reference's one global std::mt19937_64
 * (seeded from std::random_device until nt_manual_seed) drawn through
 * libstdc++'s uniform_real_distribution<T>(low, high), T = float32 or
 * float64.  nt_host_uniform writes n draws into HOST memory (no device is
 * needed unless earlier draws ran there).  nt_device_uniform writes the same
 * n draws -- the same stream, bit for bit -- into DEVICE memory, generated on
 * the device and queued on the library stream; draws from either continue
 * the one stream in call order.  The first device draw of a process builds
 * the generator's jump tables on the host (a few hundred milliseconds). */
int nt_manual_seed(uint64_t seed);
int nt_host_uniform(void *host_out, int32_t dtype, int64_t n, double low,
                    double high);
int nt_device_uniform(void *device_out, int32_t dtype, int64_t n, double low,
                      double high);
/* No counterpart in the reference: builds the host-side jump tables that
 * nt_device_uniform otherwise builds at its first call (about 0.2 s, host
 * only, no device needed), and checks them against stepping the generator
 * directly (NT_ERR_RUNTIME if that check fails).  For callers that want the
 * cost out of a timed region. */
int nt_rng_prepare(void);

/* Timing events on the library stream (no reference counterpart; used by the
 * benchmark to time kernels on the stream they run on).  Timing-only events:
 * recording one orders nothing for the host or other devices. */
int nt_event_create(void **ev);
int nt_event_record(void *ev);
int nt_event_elapsed_ms(void *start, void *end, float *ms);
int nt_event_destroy(void *ev);

/* No counterpart in the reference (the reference launches every kernel in
 * stream order): counts, since the library initialised, of elementwise
 * kernels queued without the stream barrier (hipExtAnyOrderLaunch; allowed
 * only between kernels that touch no common bytes, see launch_window.h),
 * elementwise kernels queued with it, and the empty barrier kernels queued
 * before other stream work while such kernels could still be running.  A
 * diagnostic for tests and benchmarks; any pointer may be NULL. */
int nt_launch_stats(uint64_t *unordered, uint64_t *ordered, uint64_t *fences);

#ifdef __cplusplus
}
#endif

#endif /* NT_H_ */
