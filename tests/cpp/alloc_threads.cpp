// Host-only stress test of libnt's caching allocator (caching_allocator.h)
// over a malloc backend: 8 threads allocate, write, verify and free blocks
// of mixed sizes, one thread keeps releasing the cache, and every block must
// be owned by one thread at a time.  Built with -fsanitize=thread by
// tests/test_allocator_threads.py; exits 0 when every check holds.
#include <atomic>
#include <chrono>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <stdexcept>
#include <string>
#include <thread>
#include <vector>

#include "caching_allocator.h"

namespace {

std::atomic<int64_t> g_raw_live{0};

struct MallocBackend {
  static void *raw_alloc(size_t n, bool *oom) {
    void *p = std::malloc(n);
    if (!p)
      *oom = true;
    else
      g_raw_live.fetch_add(1);
    return p;
  }
  static void raw_free(void *p) {
    g_raw_live.fetch_sub(1);
    std::free(p);
  }
  static void sync() {}
  [[noreturn]] static void fail_oom(const std::string &m) {
    throw std::runtime_error(m);
  }
  [[noreturn]] static void fail_bad_free(const std::string &m) {
    throw std::runtime_error(m);
  }
};

nt::CachingAllocator<MallocBackend> g_alloc;
std::atomic<int> g_errors{0};

void worker(int id, int iters) {
  std::mt19937_64 r(1234 + id);
  const size_t sizes[] = {1, 100, 512, 513, 4096, 70000, (size_t(2) << 20) + 1};
  std::vector<std::pair<uint8_t *, size_t>> held;
  for (int i = 0; i < iters; ++i) {
    if (held.size() < 8 && (r() & 1)) {
      const size_t n = sizes[r() % 7];
      auto *p = static_cast<uint8_t *>(g_alloc.alloc(n));
      // stamp the whole block with this thread's id: a block handed to two
      // owners at once shows up as a foreign stamp below
      std::memset(p, id + 1, n);
      held.push_back({p, n});
    } else if (!held.empty()) {
      const size_t k = r() % held.size();
      auto [p, n] = held[k];
      for (size_t j = 0; j < n; j += 61)
        if (p[j] != uint8_t(id + 1)) {
          g_errors.fetch_add(1);
          break;
        }
      g_alloc.free(p);
      held.erase(held.begin() + long(k));
    }
  }
  for (auto [p, n] : held)
    g_alloc.free(p);
}

} // namespace

int main() {
  std::vector<std::thread> ts;
  std::atomic<bool> stop{false};
  std::thread releaser([&] {
    while (!stop.load()) {
      g_alloc.release_cache();
      std::this_thread::sleep_for(std::chrono::microseconds(20));
    }
  });
  for (int i = 0; i < 8; ++i)
    ts.emplace_back(worker, i, 3000);
  for (auto &t : ts)
    t.join();
  stop.store(true);
  releaser.join();
  size_t in_use = 1, cached = 1;
  g_alloc.stats(&in_use, &cached);
  // a pointer the allocator never gave out is rejected
  int x = 0;
  bool rejected = false;
  try {
    g_alloc.free(&x);
  } catch (const std::runtime_error &) {
    rejected = true;
  }
  g_alloc.release_cache();
  std::printf("errors=%d in_use=%zu raw_live=%lld rejected=%d\n",
              g_errors.load(), in_use, (long long)g_raw_live.load(),
              int(rejected));
  return (g_errors.load() == 0 && in_use == 0 && g_raw_live.load() == 0 &&
          rejected)
             ? 0
             : 1;
}
