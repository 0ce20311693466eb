// Internal helpers shared by the libnt translation units: error handling,
// dtype dispatch, host-side view analysis and the device-side index helpers.
#pragma once

#include <hip/hip_runtime.h>

#include <array>
#include <cstdint>
#include <cstring>
#include <mutex>
#include <stdexcept>
#include <string>
#include <vector>

#include "launch_window.h"
#include "nt.h"

namespace nt {

// ------------------------------------------------------------------ errors

struct Error : std::exception {
  int code;
  std::string msg;
  Error(int c, std::string m) : code(c), msg(std::move(m)) {}
  const char *what() const noexcept override { return msg.c_str(); }
};

[[noreturn]] inline void fail(int code, const std::string &msg) {
  throw Error(code, msg);
}

void set_last_error(const std::string &msg);
void ensure_init();
bool runtime_initialised();
// Device address of the current GPU's static scratch array (bytes:
// NT_NOALLOC_SCRATCH_BYTES), resolved when the library initialised.
void *noalloc_scratch();
hipStream_t stream();
// Device pointer to the deferred-error word: a kernel that finds an invalid
// argument it cannot report synchronously stores an nt_status there (plain
// store; any writer's value wins).  nt_sync and the device-to-host copy,
// which synchronise anyway, raise it once and clear it.
int *deferred_error_word();
void raise_deferred_error();
int device_cu_count();
// Library-internal scratch allocations through the caching allocator.
void *device_alloc(size_t nbytes);
void device_free(void *p);

// Scoped scratch buffer, returned to the caching allocator when the scope
// ends -- also when a check throws.  All work runs on the library stream and
// the allocator hands a freed block only to later work on that stream, so
// freeing while a queued kernel still uses the buffer is safe.
class DeviceScratch {
public:
  explicit DeviceScratch(size_t nbytes)
      : p_(nbytes ? device_alloc(nbytes) : nullptr) {}
  ~DeviceScratch() {
    if (p_)
      device_free(p_);
  }
  DeviceScratch(const DeviceScratch &) = delete;
  DeviceScratch &operator=(const DeviceScratch &) = delete;
  template <class T = void> T *get() const { return static_cast<T *>(p_); }

private:
  void *p_;
};

#define NT_HIP_CHECK(expr)                                                     \
  do {                                                                         \
    hipError_t e_ = (expr);                                                    \
    if (e_ != hipSuccess)                                                      \
      ::nt::fail(e_ == hipErrorOutOfMemory ? NT_ERR_OOM : NT_ERR_RUNTIME,      \
                 std::string(#expr) + ": " + hipGetErrorString(e_));           \
  } while (0)

// Checks the launch that was just queued.
#define NT_LAUNCH_CHECK() NT_HIP_CHECK(hipGetLastError())

// One lock for the library's process-wide state (initialisation, the
// stream, the generator, cached work buffers): every entry point holds it for
// its whole body, so calls from several host threads run one at a time, as
// the reference's binding serialises them under the GIL.  The allocator has
// its own lock as well (caching_allocator.h).
std::recursive_mutex &api_mutex();

// Launch flags for an elementwise-engine kernel that reads `reads` and
// writes `writes` (byte ranges): hipExtAnyOrderLaunch when the launch
// window (launch_window.h) admits it, i.e. the calling entry point is an
// elementwise one (WindowScope) and the kernel has no hazard with the
// kernels queued since the last barrier launch; else 0.  NT_OVERLAP=0 turns
// the overlap off.
uint32_t ew_launch_flags(const ByteRange *reads, int nr,
                         const ByteRange *writes, int nw);
// Closes the launch window: when a kernel of it went without the barrier,
// queues an empty barrier kernel, so that whatever is queued next (a copy,
// an event, a synchronisation, any other kernel) starts after every earlier
// kernel has finished.
void stream_fence();

// Measurement knobs of the transposed-tile kernels (fp32), read once from
// the environment: NT_TILE_SHAPE=<rows>x<cols> forces one of the compiled
// shapes (64x64, 64x128, 128x128, 32x256; 0 = the shape rule), and
// NT_TILE_ORIENT=keep|swap forces the orientation (0 = the cost rule).
// Results do not depend on them; they exist so that each shape can be
// profiled inside the full sweep.
struct TileOverride {
  int tr = 0, tc = 0;
  int orient = 0; // 0 rule, 1 keep, 2 swap
};
const TileOverride &tile_override();

// Entry-point scope for the launch window.
//  * Elementwise: every device launch of the entry point goes through the
//    elementwise engine; its kernels may skip the barrier.
//  * NoStream: the entry point queues no stream work (allocation, queries);
//    the window is left as it is, so elementwise kernels on either side of
//    an output allocation can still overlap.  (The allocator's one stream
//    operation, the synchronisation before it returns cached blocks to HIP,
//    closes the window itself.)
//  * Other: closes the window first (stream_fence) and runs with the
//    overlap off; on the way out it leaves the window empty, so the next
//    elementwise kernel takes the barrier and so starts after whatever the
//    entry point queued.
// Nested entry points never open the window wider than the outer one.
enum class StreamUse { Other, Elementwise, NoStream };
class WindowScope {
public:
  explicit WindowScope(StreamUse use);
  ~WindowScope();
  WindowScope(const WindowScope &) = delete;
  WindowScope &operator=(const WindowScope &) = delete;

private:
  StreamUse use_;
  bool prev_;
};

// Runs f, converting exceptions into a status code plus a thread-local
// message.  Every extern "C" entry point is a guard() (or guard_ew()) around
// its body.
template <StreamUse USE, class F> int guard_scoped(F &&f) {
  std::lock_guard<std::recursive_mutex> lock(api_mutex());
  try {
    ensure_init();
    WindowScope scope(USE);
    f();
    return NT_OK;
  } catch (const Error &e) {
    set_last_error(e.msg);
    return e.code;
  } catch (const std::bad_alloc &) {
    set_last_error("host allocation failed");
    return NT_ERR_OOM;
  } catch (const std::exception &e) {
    set_last_error(e.what());
    return NT_ERR_RUNTIME;
  }
}

template <class F> int guard(F &&f) {
  return guard_scoped<StreamUse::Other>(std::forward<F>(f));
}

// guard() for the entry points whose device work is elementwise-engine
// kernels only: they may skip the stream barrier (WindowScope).
template <class F> int guard_ew(F &&f) {
  return guard_scoped<StreamUse::Elementwise>(std::forward<F>(f));
}

// guard() for the entry points that queue no stream work.
template <class F> int guard_nostream(F &&f) {
  return guard_scoped<StreamUse::NoStream>(std::forward<F>(f));
}

// guard() for the allocation-free entry points: the library must already be
// initialised (initialisation creates the stream and allocates), so this
// variant refuses to run instead of initialising.
template <class F> int guard_initialised(F &&f) {
  std::lock_guard<std::recursive_mutex> lock(api_mutex());
  if (!runtime_initialised()) {
    set_last_error("the library is not initialised: call nt_init() first "
                   "(initialisation allocates; this entry point does not)");
    return NT_ERR_RUNTIME;
  }
  return guard(std::forward<F>(f));
}

// ------------------------------------------------------------------ dtypes

inline size_t dtype_size(int dt) {
  switch (dt) {
  case NT_BOOL:
    return 1;
  case NT_INT32:
  case NT_FLOAT32:
    return 4;
  case NT_INT64:
  case NT_FLOAT64:
    return 8;
  }
  fail(NT_ERR_VALUE, "Unknown dtype.");
}

inline const char *dtype_name(int dt) {
  switch (dt) {
  case NT_BOOL:
    return "bool";
  case NT_INT32:
    return "int32";
  case NT_INT64:
    return "int64";
  case NT_FLOAT32:
    return "float32";
  case NT_FLOAT64:
    return "float64";
  }
  return "?";
}

// Dispatch families mirror the reference's DispatchAll / DispatchFloat /
// DispatchArithmetic (src/cpp/dtype.h:23-79): a dtype outside the family is
// a ValueError.
template <class F> void dispatch_all(int dt, F &&f) {
  switch (dt) {
  case NT_BOOL:
    return f.template operator()<bool>();
  case NT_INT32:
    return f.template operator()<int32_t>();
  case NT_INT64:
    return f.template operator()<int64_t>();
  case NT_FLOAT32:
    return f.template operator()<float>();
  case NT_FLOAT64:
    return f.template operator()<double>();
  }
  fail(NT_ERR_VALUE, "Unknown dtype.");
}

template <class F> void dispatch_float(int dt, F &&f) {
  switch (dt) {
  case NT_FLOAT32:
    return f.template operator()<float>();
  case NT_FLOAT64:
    return f.template operator()<double>();
  }
  fail(NT_ERR_VALUE, "Invalid dtype.");
}

template <class F> void dispatch_arith(int dt, F &&f) {
  switch (dt) {
  case NT_INT32:
    return f.template operator()<int32_t>();
  case NT_INT64:
    return f.template operator()<int64_t>();
  case NT_FLOAT32:
    return f.template operator()<float>();
  case NT_FLOAT64:
    return f.template operator()<double>();
  }
  fail(NT_ERR_VALUE, "Invalid dtype.");
}

// ------------------------------------------------------------------- views

inline void check_view(const nt_view *v, const char *what) {
  if (v == nullptr)
    fail(NT_ERR_RUNTIME, std::string(what) + ": null view");
  if (v->ndim < 0 || v->ndim > NT_MAX_DIMS)
    fail(NT_ERR_RUNTIME, std::string(what) + ": ndim out of range (max 8)");
  for (int i = 0; i < v->ndim; ++i)
    if (v->shape[i] < 0 || v->strides[i] < 0)
      fail(NT_ERR_RUNTIME,
           std::string(what) + ": negative shape or stride not supported");
  if (v->offset < 0)
    fail(NT_ERR_RUNTIME, std::string(what) + ": negative offset");
  dtype_size(v->dtype);
}

inline int64_t numel(const nt_view *v) {
  int64_t n = 1;
  for (int i = 0; i < v->ndim; ++i)
    n *= v->shape[i];
  return n;
}

inline bool same_shape(const nt_view *a, const nt_view *b) {
  if (a->ndim != b->ndim)
    return false;
  for (int i = 0; i < a->ndim; ++i)
    if (a->shape[i] != b->shape[i])
      return false;
  return true;
}

inline void require_same_shape(const nt_view *a, const nt_view *b,
                               const char *fname) {
  if (!same_shape(a, b))
    fail(NT_ERR_RUNTIME,
         std::string(fname) + ": Expected two views of the same shape.");
}

inline void require_same_dtype(const nt_view *a, const nt_view *b,
                               const char *fname) {
  if (a->dtype != b->dtype)
    fail(NT_ERR_RUNTIME, std::string(fname) + ": dtype mismatch (" +
                             dtype_name(a->dtype) + " vs " +
                             dtype_name(b->dtype) + ")");
}

// Row-major contiguity over the logical shape (reference: is_contiguous,
// src/cpp/tensor_view.cuh:31-41).  Size-1 dims do not constrain strides.
inline bool is_contiguous(const nt_view *v) {
  int64_t expect = 1;
  for (int i = v->ndim - 1; i >= 0; --i) {
    if (v->shape[i] != 1 && v->strides[i] != expect)
      return false;
    expect *= v->shape[i];
  }
  return true;
}

template <class T> inline T *typed_ptr(const nt_view *v) {
  return static_cast<T *>(v->data) + v->offset;
}

// Joint layout of several same-shape operands after dropping size-1 dims
// and merging dims that are adjacent in memory for every operand.  The
// merged shape is what the elementwise and reduction kernels iterate over.
struct JointLayout {
  int ndim = 0;
  int64_t shape[NT_MAX_DIMS];
  std::vector<std::array<int64_t, NT_MAX_DIMS>> strides; // per operand
};

JointLayout coalesce(const nt_view *const *ops, int nops);

// ------------------------------------------------- device index helpers

// Unsigned 32-bit division by a run-time constant through a multiply-high
// (Granlund & Montgomery, "Division by invariant integers using
// multiplication", PLDI 1994, round-up variant).  Exact for all n < 2^32.
struct FastDivU32 {
  uint32_t d, m, s;
  FastDivU32() : d(1), m(0), s(0) {}
  explicit FastDivU32(uint32_t dd) : d(dd) {
    s = 0;
    while ((uint64_t(1) << s) < dd)
      ++s;
    m = uint32_t(((uint64_t(1) << 32) * ((uint64_t(1) << s) - dd)) / dd + 1);
  }
  __host__ __device__ __forceinline__ uint32_t div(uint32_t n) const {
    uint32_t t = uint32_t((uint64_t(n) * m) >> 32);
    return uint32_t((uint64_t(t) + n) >> s);
  }
};

} // namespace nt
