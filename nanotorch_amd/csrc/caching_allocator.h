// Stream-ordered caching allocator of libnt, host-only code (no HIP header):
// the device backend is a template parameter, so the same class is built
// into libnt over hipMalloc and into a CPU test over malloc.
//
// Every kernel and copy of the library runs on one stream, so a block freed
// by the host can be handed to the next request immediately: any later use
// is queued after the last use of the previous owner.  Requests are rounded
// up to 512 B (small) or 2 MiB (large) so that the free lists see a handful
// of distinct sizes per workload.  On an out-of-memory error the cache is
// returned to the backend and the request retried once.  The reference's
// allocator buckets by 256 B and never frees (src/cpp/allocator.cpp:16-36).
//
// Thread safety: every public member takes one mutex, so callers on several
// threads (a garbage collector freeing on another thread, a multi-threaded
// host) cannot hand one block to two owners or corrupt the maps.
//
// Backend requirements (static members):
//   void *raw_alloc(size_t n, bool *oom)  -- nullptr on failure; *oom tells
//                                            an out-of-memory failure apart
//   void raw_free(void *p)
//   void sync()                           -- waits for queued device work
//   [[noreturn]] void fail_oom(const std::string &msg)
//   [[noreturn]] void fail_bad_free(const std::string &msg)
#pragma once

#include <cstddef>
#include <map>
#include <mutex>
#include <string>

namespace nt {

template <class Backend> class CachingAllocator {
public:
  static size_t round_size(size_t n) {
    if (n == 0)
      n = 1;
    const size_t small = 512, large = size_t(2) << 20;
    if (n < large)
      return (n + small - 1) / small * small;
    return (n + large - 1) / large * large;
  }

  void *alloc(size_t nbytes) {
    std::lock_guard<std::mutex> lock(m_);
    const size_t sz = round_size(nbytes);
    // Best fit among cached blocks no more than 25% larger than asked.
    auto it = free_blocks_.lower_bound(sz);
    if (it != free_blocks_.end() && it->first <= sz + sz / 4) {
      void *p = it->second;
      const size_t bsz = it->first;
      free_blocks_.erase(it);
      bytes_cached_ -= bsz;
      live_[p] = bsz;
      bytes_in_use_ += bsz;
      return p;
    }
    bool oom = false;
    void *p = Backend::raw_alloc(sz, &oom);
    if (p == nullptr && oom) {
      release_cache_locked();
      p = Backend::raw_alloc(sz, &oom);
    }
    if (p == nullptr)
      Backend::fail_oom("device allocation of " + std::to_string(sz) +
                        " bytes failed");
    live_[p] = sz;
    bytes_in_use_ += sz;
    return p;
  }

  void free(void *p) {
    std::lock_guard<std::mutex> lock(m_);
    auto it = live_.find(p);
    if (it == live_.end())
      Backend::fail_bad_free("nt_free: pointer not allocated by nt_malloc");
    free_blocks_.emplace(it->second, p);
    bytes_cached_ += it->second;
    bytes_in_use_ -= it->second;
    live_.erase(it);
  }

  void release_cache() {
    std::lock_guard<std::mutex> lock(m_);
    release_cache_locked();
  }

  void stats(size_t *in_use, size_t *cached) {
    std::lock_guard<std::mutex> lock(m_);
    if (in_use)
      *in_use = bytes_in_use_;
    if (cached)
      *cached = bytes_cached_;
  }

private:
  void release_cache_locked() {
    if (free_blocks_.empty())
      return;
    // Blocks may still be read by queued work of their previous owner.
    Backend::sync();
    for (auto &kv : free_blocks_)
      Backend::raw_free(kv.second);
    free_blocks_.clear();
    bytes_cached_ = 0;
  }

  std::mutex m_;
  std::multimap<size_t, void *> free_blocks_; // size -> ptr
  std::map<void *, size_t> live_;             // ptr -> size
  size_t bytes_in_use_ = 0;
  size_t bytes_cached_ = 0;
};

} // namespace nt
