// Device runtime of libnt: initialisation, the library stream, the caching
// allocator, host<->device copies, fills and timing events.
//
// Reference counterparts: src/cpp/cuda.{h,cpp} (availability, sync, error
// checks), src/cpp/allocator.{h,cpp} (caching allocator), src/cpp/storage.cpp
// (allocate/to/clone) and src/cpp/factory.cu (fills).
#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>

#include <hip/hip_ext.h>

#include "caching_allocator.h"
#include "ew_engine.h"

namespace nt {

namespace {

thread_local std::string g_last_error;

// Scratch of the allocation-free entry points (nt_reduce_noalloc): one
// static device array per GPU, held until the process ends.  Host code never
// passes `scratch` itself to a kernel (on the host the name is a stand-in,
// not a device address): set-up resolves its device address with
// hipGetSymbolAddress, once per device, and every use goes through that
// pointer.  Calls that overlap on one GPU share the array and race; the
// reductions' partial results are written in full before they are read, so
// nothing in it needs clearing between calls.
static __device__ __align__(256) unsigned char scratch[NT_NOALLOC_SCRATCH_BYTES];

constexpr int MAX_DEVICES = 64;

struct Runtime {
  bool initialised = false;
  void *scratch_ptr[MAX_DEVICES] = {};
  bool available = false;
  int cu_count = 0;
  hipStream_t stream = nullptr;
  // Deferred device-side error word: pinned, coherent host memory that
  // kernels may store an nt_status into; read after stream syncs.
  volatile int *deferred_host = nullptr;
  int *deferred_dev = nullptr;
  // Elementwise kernels queued since the last barrier launch, and whether
  // the entry point running now may skip the barrier (WindowScope).
  LaunchWindow window;
  bool window_open = false;
  int scope_depth = 0;
  uint64_t n_unordered = 0, n_ordered = 0, n_fences = 0;
};

Runtime &rt() {
  static Runtime r;
  return r;
}

// ---------------------------------------------------------------- allocator

struct HipBackend {
  static void *raw_alloc(size_t n, bool *oom) {
    void *p = nullptr;
    const hipError_t e = hipMalloc(&p, n);
    if (e == hipSuccess)
      return p;
    (void)hipGetLastError();
    *oom = (e == hipErrorOutOfMemory);
    return nullptr;
  }
  static void raw_free(void *p) { NT_HIP_CHECK(hipFree(p)); }
  static void sync() {
    // nt_malloc and nt_free leave the launch window open: close it first.
    stream_fence();
    NT_HIP_CHECK(hipStreamSynchronize(rt().stream));
  }
  [[noreturn]] static void fail_oom(const std::string &msg) {
    fail(NT_ERR_OOM, msg);
  }
  [[noreturn]] static void fail_bad_free(const std::string &msg) {
    fail(NT_ERR_RUNTIME, msg);
  }
};

CachingAllocator<HipBackend> &allocator() {
  static CachingAllocator<HipBackend> a;
  return a;
}

__global__ void fill_kernel_bytes(uint8_t *p, int64_t nbytes_pattern_units,
                                  uint64_t pattern, int unit) {
  // Generic fill for element sizes 1, 4 and 8 bytes: unit = element size.
  int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  int64_t stride = int64_t(gridDim.x) * blockDim.x;
  for (; i < nbytes_pattern_units; i += stride) {
    if (unit == 1)
      p[i] = uint8_t(pattern);
    else if (unit == 4)
      reinterpret_cast<uint32_t *>(p)[i] = uint32_t(pattern);
    else
      reinterpret_cast<uint64_t *>(p)[i] = pattern;
  }
}

// 16-byte stores for the aligned bulk of a fill.
__global__ void fill_kernel_x4(uint4 *p, int64_t n16, uint4 v) {
  int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  int64_t stride = int64_t(gridDim.x) * blockDim.x;
  for (; i < n16; i += stride)
    p[i] = v;
}

} // namespace

void set_last_error(const std::string &msg) { g_last_error = msg; }

std::recursive_mutex &api_mutex() {
  static std::recursive_mutex m;
  return m;
}

void ensure_init() {
  Runtime &r = rt();
  if (r.initialised)
    return;
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess || n == 0) {
    (void)hipGetLastError();
    fail(NT_ERR_RUNTIME, "no HIP device available");
  }
  NT_HIP_CHECK(hipSetDevice(0));
  // The static scratch array's address on this device (it may load the
  // library's code object, so it is done here, not in the entry point).
  void *sp = nullptr;
  NT_HIP_CHECK(hipGetSymbolAddress(&sp, HIP_SYMBOL(scratch)));
  if (sp == nullptr)
    fail(NT_ERR_RUNTIME, "no device address for the static scratch array");
  r.scratch_ptr[0] = sp;
  hipDeviceProp_t prop;
  NT_HIP_CHECK(hipGetDeviceProperties(&prop, 0));
  r.cu_count = prop.multiProcessorCount;
  // Default priority, non-blocking w.r.t. the legacy null stream.
  NT_HIP_CHECK(hipStreamCreateWithFlags(&r.stream, hipStreamNonBlocking));
  void *word = nullptr;
  NT_HIP_CHECK(hipHostMalloc(&word, sizeof(int), hipHostMallocCoherent));
  *static_cast<volatile int *>(word) = 0;
  void *dword = nullptr;
  NT_HIP_CHECK(hipHostGetDevicePointer(&dword, word, 0));
  r.deferred_host = static_cast<volatile int *>(word);
  r.deferred_dev = static_cast<int *>(dword);
  // Kernels per launch window (launch_window.h); NT_OVERLAP_WINDOW overrides.
  if (const char *w = std::getenv("NT_OVERLAP_WINDOW"))
    r.window.set_limit(std::atoi(w));
  r.available = true;
  r.initialised = true;
}

// The barrier kernel of stream_fence: no work; its dispatch packet carries
// the barrier bit, so it starts after every earlier kernel has finished, and
// work queued after it is ordered after it as usual.
__global__ void stream_fence_kernel() {}

namespace {
bool overlap_enabled() {
  static const bool on = [] {
    const char *e = std::getenv("NT_OVERLAP");
    return !(e && e[0] == '0');
  }();
  return on;
}
} // namespace

uint32_t ew_launch_flags(const ByteRange *reads, int nr,
                         const ByteRange *writes, int nw) {
  Runtime &r = rt();
  const bool allowed = r.window_open && overlap_enabled();
  if (r.window.admit(reads, nr, writes, nw, allowed)) {
    ++r.n_unordered;
    return uint32_t(hipExtAnyOrderLaunch);
  }
  ++r.n_ordered;
  return 0u;
}

void stream_fence() {
  Runtime &r = rt();
  if (r.window.close()) {
    stream_fence_kernel<<<dim3(1), dim3(64), 0, r.stream>>>();
    NT_LAUNCH_CHECK();
    ++r.n_fences;
  }
}

WindowScope::WindowScope(StreamUse use) : use_(use), prev_(rt().window_open) {
  Runtime &r = rt();
  if (use == StreamUse::Other)
    stream_fence(); // may throw: nothing else has changed yet
  r.window_open = use == StreamUse::Elementwise && (r.scope_depth == 0 || prev_);
  ++r.scope_depth;
}

WindowScope::~WindowScope() {
  Runtime &r = rt();
  --r.scope_depth;
  r.window_open = prev_;
  if (use_ == StreamUse::Other) {
    // The entry point's own launches were all barrier launches (the window
    // was off), but it may have queued kernels the window does not know
    // about: the next elementwise kernel must take the barrier.  Nothing in
    // the window went without it, so no fence is needed.
    r.window.close();
  }
}

const TileOverride &tile_override() {
  static const TileOverride o = [] {
    TileOverride t;
    if (const char *e = std::getenv("NT_TILE_SHAPE")) {
      int a = 0, b = 0;
      if (std::sscanf(e, "%dx%d", &a, &b) == 2 &&
          ((a == 64 && (b == 64 || b == 128)) || (a == 128 && b == 128) ||
           (a == 32 && b == 256))) {
        t.tr = a;
        t.tc = b;
      }
    }
    if (const char *e = std::getenv("NT_TILE_ORIENT"))
      t.orient = std::strcmp(e, "keep") == 0 ? 1 : (std::strcmp(e, "swap") == 0 ? 2 : 0);
    return t;
  }();
  return o;
}

bool ew_nontemporal() {
  static const bool on = [] {
    const char *e = std::getenv("NT_NONTEMPORAL");
    return !(e && e[0] == '0');
  }();
  return on;
}

hipStream_t stream() { return rt().stream; }
bool runtime_initialised() { return rt().initialised; }

void *noalloc_scratch() {
  int dev = 0;
  NT_HIP_CHECK(hipGetDevice(&dev));
  void *p = (dev >= 0 && dev < MAX_DEVICES) ? rt().scratch_ptr[dev] : nullptr;
  if (p == nullptr)
    fail(NT_ERR_RUNTIME, "static scratch not set up on the current device");
  return p;
}
int *deferred_error_word() { return rt().deferred_dev; }

void raise_deferred_error() {
  volatile int *w = rt().deferred_host;
  if (w == nullptr || *w == NT_OK)
    return;
  const int code = *w;
  *w = NT_OK;
  fail(code, "an earlier gather/scatter call met an index outside its axis "
             "(found by the device-side check; those elements were skipped)");
}
int device_cu_count() { return rt().cu_count; }
void *device_alloc(size_t nbytes) { return allocator().alloc(nbytes); }
void device_free(void *p) { allocator().free(p); }

JointLayout coalesce(const nt_view *const *ops, int nops) {
  JointLayout L;
  L.strides.resize(nops);
  const nt_view *ref = ops[0];
  // Keep dims of size != 1 (a size-1 dim never moves the index).
  int nd = 0;
  for (int d = 0; d < ref->ndim; ++d) {
    if (ref->shape[d] == 1)
      continue;
    L.shape[nd] = ref->shape[d];
    for (int k = 0; k < nops; ++k)
      L.strides[k][nd] = ops[k]->strides[d];
    ++nd;
  }
  // Merge dim d into d-1 when, for every operand, stepping the outer dim is
  // the same as running off the end of the inner one.
  int out = 0;
  for (int d = 0; d < nd; ++d) {
    if (out > 0) {
      bool mergeable = true;
      for (int k = 0; k < nops; ++k)
        if (L.strides[k][out - 1] != L.strides[k][d] * L.shape[d]) {
          mergeable = false;
          break;
        }
      if (mergeable) {
        L.shape[out - 1] *= L.shape[d];
        for (int k = 0; k < nops; ++k)
          L.strides[k][out - 1] = L.strides[k][d];
        continue;
      }
    }
    L.shape[out] = L.shape[d];
    for (int k = 0; k < nops; ++k)
      L.strides[k][out] = L.strides[k][d];
    ++out;
  }
  L.ndim = out;
  return L;
}

} // namespace nt

using namespace nt;

extern "C" {

int nt_init(void) {
  return guard([] {});
}

int nt_is_available(int *available) {
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess)
    (void)hipGetLastError();
  if (available)
    *available = (e == hipSuccess && n > 0) ? 1 : 0;
  return NT_OK;
}

int nt_sync(void) {
  return guard([] {
    NT_HIP_CHECK(hipStreamSynchronize(stream()));
    raise_deferred_error();
  });
}

const char *nt_last_error(void) { return g_last_error.c_str(); }

int nt_malloc(void **ptr, size_t nbytes) {
  return guard_nostream([&] {
    if (!ptr)
      fail(NT_ERR_RUNTIME, "nt_malloc: null out pointer");
    *ptr = allocator().alloc(nbytes);
  });
}

int nt_free(void *ptr) {
  return guard_nostream([&] {
    if (ptr)
      allocator().free(ptr);
  });
}

int nt_empty_cache(void) {
  return guard([] { allocator().release_cache(); });
}

int nt_memory_stats(size_t *bytes_in_use, size_t *bytes_cached) {
  return guard_nostream([&] { allocator().stats(bytes_in_use, bytes_cached); });
}

int nt_memcpy_h2d(void *dst, const void *src, size_t nbytes) {
  return guard([&] {
    if (nbytes == 0)
      return;
    NT_HIP_CHECK(
        hipMemcpyAsync(dst, src, nbytes, hipMemcpyHostToDevice, stream()));
    // The source is pageable caller memory that may be reused on return.
    NT_HIP_CHECK(hipStreamSynchronize(stream()));
  });
}

int nt_memcpy_d2h(void *dst, const void *src, size_t nbytes) {
  return guard([&] {
    if (nbytes == 0)
      return;
    NT_HIP_CHECK(
        hipMemcpyAsync(dst, src, nbytes, hipMemcpyDeviceToHost, stream()));
    NT_HIP_CHECK(hipStreamSynchronize(stream()));
    raise_deferred_error();
  });
}

int nt_memcpy_d2d(void *dst, const void *src, size_t nbytes) {
  return guard([&] {
    if (nbytes == 0)
      return;
    NT_HIP_CHECK(
        hipMemcpyAsync(dst, src, nbytes, hipMemcpyDeviceToDevice, stream()));
  });
}

int nt_fill(void *data, int32_t dtype, int64_t n, double value) {
  return guard([&] {
    if (n < 0)
      fail(NT_ERR_RUNTIME, "nt_fill: negative size");
    if (n == 0)
      return;
    uint64_t pattern = 0;
    size_t es = dtype_size(dtype);
    dispatch_all(dtype, [&]<class T>() {
      T v;
      if constexpr (std::is_same_v<T, bool>)
        v = (value != 0.0);
      else
        v = static_cast<T>(value);
      std::memcpy(&pattern, &v, sizeof(T));
    });
    // Replicate the element into a 16-byte word for the bulk of the fill.
    uint8_t word[16];
    for (int i = 0; i < 16; ++i)
      word[i] = reinterpret_cast<uint8_t *>(&pattern)[i % es];
    uint4 v4;
    std::memcpy(&v4, word, 16);
    uint8_t *p = static_cast<uint8_t *>(data);
    if (reinterpret_cast<uintptr_t>(p) % es != 0)
      fail(NT_ERR_RUNTIME, "nt_fill: pointer not aligned to the element size");
    int64_t nbytes = n * int64_t(es);
    int64_t head = 0;
    uintptr_t addr = reinterpret_cast<uintptr_t>(p);
    if (addr % 16 != 0)
      head = std::min<int64_t>(nbytes, (16 - addr % 16));
    head -= head % int64_t(es); // element aligned (allocations are aligned)
    int64_t n16 = (nbytes - head) / 16;
    int64_t tail_start = head + n16 * 16;
    int threads = 256;
    if (head > 0) {
      fill_kernel_bytes<<<1, threads, 0, stream()>>>(p, head / int64_t(es),
                                                     pattern, int(es));
      NT_LAUNCH_CHECK();
    }
    if (n16 > 0) {
      // one work-item per 16 bytes: a one-shot grid writes faster than a
      // grid-stride loop over a few workgroups per CU; past 2^30 work-items
      // (16 GiB) the kernel's grid-stride loop takes the rest, since a
      // dispatch holds fewer than 2^32 work-items
      const int64_t blocks = std::min<int64_t>((n16 + threads - 1) / threads,
                                               (int64_t(1) << 30) / threads);
      fill_kernel_x4<<<dim3(unsigned(blocks)), threads, 0, stream()>>>(
          reinterpret_cast<uint4 *>(p + head), n16, v4);
      NT_LAUNCH_CHECK();
    }
    if (tail_start < nbytes) {
      fill_kernel_bytes<<<1, threads, 0, stream()>>>(
          p + tail_start, (nbytes - tail_start) / int64_t(es), pattern,
          int(es));
      NT_LAUNCH_CHECK();
    }
  });
}

int nt_event_create(void **ev) {
  return guard_nostream([&] {
    hipEvent_t e;
    // Timing only: no system-scope release at record time, so a bracket
    // around one launch does not add an L2 write-back to what it measures.
    NT_HIP_CHECK(hipEventCreateWithFlags(&e, hipEventDisableSystemFence));
    *ev = reinterpret_cast<void *>(e);
  });
}

int nt_event_record(void *ev) {
  return guard([&] {
    NT_HIP_CHECK(hipEventRecord(reinterpret_cast<hipEvent_t>(ev), stream()));
  });
}

int nt_event_elapsed_ms(void *start, void *end, float *ms) {
  return guard([&] {
    NT_HIP_CHECK(hipEventSynchronize(reinterpret_cast<hipEvent_t>(end)));
    NT_HIP_CHECK(hipEventElapsedTime(ms, reinterpret_cast<hipEvent_t>(start),
                                     reinterpret_cast<hipEvent_t>(end)));
  });
}

int nt_launch_stats(uint64_t *unordered, uint64_t *ordered, uint64_t *fences) {
  return guard_nostream([&] {
    const Runtime &r = rt();
    if (unordered)
      *unordered = r.n_unordered;
    if (ordered)
      *ordered = r.n_ordered;
    if (fences)
      *fences = r.n_fences;
  });
}

int nt_event_destroy(void *ev) {
  return guard_nostream([&] {
    NT_HIP_CHECK(hipEventDestroy(reinterpret_cast<hipEvent_t>(ev)));
  });
}

} // extern "C"
