// Host-only check of libnt's launch window (launch_window.h): a random
// stream of kernels with random read / write byte ranges, interleaved with
// closes (copies, events, other kernels), is fed to LaunchWindow, and the
// stream's ordering is modelled the way the command processor orders it: a
// barrier launch starts after every earlier kernel has finished, a kernel
// launched without the barrier may run alongside every kernel back to the
// last barrier launch.  Every such concurrent pair must be free of
// read-after-write, write-after-read and write-after-write overlaps, and
// each barrier the window asked for must have had a reason (a hazard, a
// full window, an empty window, an untracked kernel or a refusal).  Exits 0
// when every check holds; prints the share of launches without a barrier.
#include <cstdint>
#include <cstdio>
#include <random>
#include <vector>

#include "launch_window.h"

using nt::ByteRange;
using nt::LaunchWindow;

namespace {

struct K {
  std::vector<ByteRange> r, w;
  bool barrier = true;
};

bool hazard(const K &a, const K &b) {
  for (const auto &x : a.w) {
    for (const auto &y : b.r)
      if (x.overlaps(y))
        return true;
    for (const auto &y : b.w)
      if (x.overlaps(y))
        return true;
  }
  for (const auto &x : a.r)
    for (const auto &y : b.w)
      if (x.overlaps(y))
        return true;
  return false;
}

ByteRange rnd_range(std::mt19937_64 &g, uintptr_t space) {
  std::uniform_int_distribution<uintptr_t> d(0, space - 1);
  const uintptr_t a = d(g), len = 1 + d(g) % (space / 8);
  ByteRange r;
  r.lo = 4096 + a;
  r.hi = r.lo + ((g() % 16 == 0) ? 0 : len); // some empty ranges
  return r;
}

} // namespace

int main() {
  int errors = 0;
  long admitted = 0, launched = 0, fences = 0;
  for (int trial = 0; trial < 400; ++trial) {
    std::mt19937_64 g(1000 + trial);
    const uintptr_t space = (trial % 4 == 0) ? 64 : ((trial % 4 == 1) ? 4096 : (1u << 20));
    LaunchWindow win;
    win.set_limit(1 + trial % LaunchWindow::MAX_KERNELS);
    std::vector<K> ks;
    int last_barrier = -1;
    for (int step = 0; step < 500; ++step) {
      const int what = int(g() % 20);
      if (what == 0) { // a copy / event / other kernel: close, fence if asked
        if (win.close()) {
          ++fences;
          K f; // the fence: a barrier kernel touching nothing
          ks.push_back(f);
          last_barrier = int(ks.size()) - 1;
        }
        // the work itself is ordered after everything before it
        K other;
        other.r.push_back(rnd_range(g, space));
        other.w.push_back(rnd_range(g, space));
        ks.push_back(other);
        last_barrier = int(ks.size()) - 1;
        continue;
      }
      K k;
      const int nr = int(g() % 6), nw = 1 + int(g() % 2);
      for (int i = 0; i < nr; ++i)
        k.r.push_back(rnd_range(g, space));
      for (int i = 0; i < nw; ++i)
        k.w.push_back(rnd_range(g, space));
      if (g() % 8 == 0) // in-place: an output is also read
        k.r.push_back(k.w[0]);
      const bool allowed = g() % 10 != 0;
      const int before = win.size();
      const bool free_ = win.admit(k.r.data(), int(k.r.size()), k.w.data(), int(k.w.size()), allowed);
      k.barrier = !free_;
      ++launched;
      if (free_) {
        ++admitted;
        if (!allowed || before == 0 || before >= win.limit()) {
          std::printf("admitted against the rules (trial %d step %d)\n", trial, step);
          ++errors;
        }
      }
      ks.push_back(k);
      const int j = int(ks.size()) - 1;
      if (k.barrier)
        last_barrier = j;
      // every kernel since the last barrier launch may run alongside this one
      for (int i = std::max(last_barrier, 0); i < j; ++i)
        if (!k.barrier && hazard(ks[i], k)) {
          std::printf("hazard between kernels %d and %d (trial %d)\n", i, j, trial);
          ++errors;
        }
      // a barrier asked for with room in the window, permission and no
      // hazard against the window would be a missed overlap (not unsafe,
      // but the window must do what it says)
      if (k.barrier && allowed && before > 0 && before < win.limit()) {
        bool any = false;
        for (int i = j - before; i < j; ++i)
          any = any || hazard(ks[i], k);
        if (!any) {
          std::printf("barrier without a reason (trial %d step %d)\n", trial, step);
          ++errors;
        }
      }
    }
  }
  // more ranges than the window tracks: the kernel takes the barrier and
  // the next one too
  {
    LaunchWindow win;
    ByteRange a{100, 200}, many[LaunchWindow::MAX_RANGES + 1];
    for (auto &m : many)
      m = ByteRange{1000, 1001};
    win.admit(&a, 1, &a, 1, true);
    if (win.admit(many, LaunchWindow::MAX_RANGES + 1, &a, 0, true) || win.size() != 0) {
      std::printf("untracked kernel admitted\n");
      ++errors;
    }
    ByteRange b{5000, 6000};
    if (win.admit(&b, 1, &b, 1, true)) {
      std::printf("kernel after an untracked one admitted\n");
      ++errors;
    }
  }
  std::printf("errors=%d launched=%ld admitted=%ld fences=%ld\n", errors, launched, admitted, fences);
  return errors == 0 && admitted > launched / 20 ? 0 : 1;
}
