// Launch window: which elementwise kernels may be queued without the
// barrier that orders a HIP stream.
//
// Every kernel of the library is queued on one stream.  By default each
// dispatch packet carries the barrier bit, so a kernel starts only when the
// one before it has finished, and every launch pays the GPU's ramp-up and
// drain (~2-3 us of a 20-80 us elementwise kernel at 2^24 elements).
// Launched with hipExtAnyOrderLaunch, a packet has no barrier bit: the
// command processor still dispatches packets in queue order, but starts a
// kernel's workgroups while the previous kernels are still draining.
// That is safe only between kernels that touch no common memory (or only
// read it).  The window holds the byte ranges of the kernels queued since
// the last barrier launch -- the only kernels that may still be running
// unordered with respect to a new one, since everything before a barrier
// kernel finished before it started -- and admits a kernel without a barrier
// when
//   * it writes nothing that a window kernel reads or writes, and reads
//     nothing that a window kernel writes;
//   * the window holds at least one and fewer than limit() kernels.
// Otherwise the kernel is launched with the barrier and starts a new window.
//
// Host-only code (no HIP header), so a CPU test exercises it directly.
#pragma once

#include <cstddef>
#include <cstdint>

namespace nt {

struct ByteRange {
  uintptr_t lo = 0, hi = 0; // [lo, hi); empty when lo == hi
  bool overlaps(const ByteRange &o) const {
    return lo < hi && o.lo < o.hi && lo < o.hi && o.lo < hi;
  }
};

class LaunchWindow {
public:
  // At most MAX_KERNELS kernels per window (a barrier launch at least every
  // limit() kernels); the limit is set at run time up to that.
  static constexpr int MAX_KERNELS = 16;
  static constexpr int DEFAULT_LIMIT = 12;
  static constexpr int MAX_RANGES = 16; // operands per kernel

  void set_limit(int k) {
    limit_ = k < 1 ? 1 : (k > MAX_KERNELS ? MAX_KERNELS : k);
  }
  int limit() const { return limit_; }

  // Records a kernel reading `reads` and writing `writes`; true when it may
  // be launched without the barrier.  More than MAX_RANGES ranges of either
  // kind, or `allowed` false, always take the barrier.
  bool admit(const ByteRange *reads, int nr, const ByteRange *writes, int nw,
             bool allowed) {
    const bool fits = nr <= MAX_RANGES && nw <= MAX_RANGES;
    bool free_of_hazards = allowed && fits && n_ > 0 && n_ < limit_;
    for (int k = 0; k < n_ && free_of_hazards; ++k) {
      const Entry &e = win_[k];
      for (int i = 0; i < nw && free_of_hazards; ++i) {
        for (int j = 0; j < e.nr; ++j)
          if (writes[i].overlaps(e.r[j]))
            free_of_hazards = false;
        for (int j = 0; j < e.nw; ++j)
          if (writes[i].overlaps(e.w[j]))
            free_of_hazards = false;
      }
      for (int i = 0; i < nr && free_of_hazards; ++i)
        for (int j = 0; j < e.nw; ++j)
          if (reads[i].overlaps(e.w[j]))
            free_of_hazards = false;
    }
    if (!free_of_hazards) {
      n_ = 0;
      unordered_ = false;
    }
    if (!fits) // cannot be tracked: nothing may skip the barrier after it
      return false;
    Entry &e = win_[n_++];
    e.nr = nr;
    e.nw = nw;
    for (int i = 0; i < nr; ++i)
      e.r[i] = reads[i];
    for (int i = 0; i < nw; ++i)
      e.w[i] = writes[i];
    unordered_ = unordered_ || free_of_hazards;
    return free_of_hazards;
  }

  // Another kind of stream work follows (a kernel outside the window's
  // bookkeeping, a copy, an event, a synchronisation).  Returns true when a
  // kernel of the window was launched without the barrier, i.e. the caller
  // must first queue a barrier kernel so that work queued next starts after
  // every window kernel has finished.  The window is empty afterwards.
  bool close() {
    const bool need_fence = unordered_;
    n_ = 0;
    unordered_ = false;
    return need_fence;
  }

  int size() const { return n_; }
  bool unordered() const { return unordered_; }

private:
  struct Entry {
    int nr = 0, nw = 0;
    ByteRange r[MAX_RANGES], w[MAX_RANGES];
  };
  Entry win_[MAX_KERNELS];
  int limit_ = DEFAULT_LIMIT;
  int n_ = 0;
  bool unordered_ = false;
};

} // namespace nt
