// Randomised allocate/release sequences against the device pool with a host
// policy that hands out disjoint address ranges of a bounded "device": no
// two live blocks overlap, freed segments merge back whole, the counters add
// up, and running short of memory recycles the cache instead of failing.
#include <stdio.h>
#include <stdlib.h>

#include <algorithm>
#include <random>
#include <stdexcept>
#include <unordered_map>
#include <vector>

#include "../../easyfhe-llama3-8b_amd/csrc/device_pool.hpp"

namespace {

struct HostDevice {
  static size_t capacity, used;
  static std::unordered_map<void *, size_t> allocs;
  static char *next;
  static bool alloc(void **p, size_t bytes) {
    if (used + bytes > capacity) return false;
    *p = next;  // addresses only: the pool never touches the memory
    next += (bytes + 4095) / 4096 * 4096 + 4096;
    allocs[*p] = bytes;
    used += bytes;
    return true;
  }
  static void release(void *p) {
    auto it = allocs.find(p);
    if (it == allocs.end()) {
      fprintf(stderr, "release of an address the device did not hand out\n");
      abort();
    }
    used -= it->second;
    allocs.erase(it);
  }
  static size_t free_bytes() { return capacity - used; }
  static void synchronize() {}
};
size_t HostDevice::capacity = 0, HostDevice::used = 0;
std::unordered_map<void *, size_t> HostDevice::allocs;
char *HostDevice::next = (char *)(uintptr_t)0x100000000ull;

using TestPool = ckks::BasicPool<HostDevice>;

int fail(const char *what, long it) {
  fprintf(stderr, "FAIL %s at step %ld\n", what, it);
  return 1;
}

int run(size_t capacity, long steps, uint64_t seed, size_t max_live) {
  HostDevice::capacity = capacity;
  TestPool pool;
  std::mt19937_64 rng(seed);
  struct Live {
    char *p;
    size_t n;
  };
  std::vector<Live> live;
  size_t live_bytes = 0;
  long exhausted = 0;
  for (long it = 0; it < steps; it++) {
    const bool grow = live.empty() || (rng() % 100 < 52 && live_bytes < max_live);
    if (grow) {
      size_t n;
      const int r = (int)(rng() % 10);
      if (r < 3)
        n = 1 + rng() % (1u << 20);  // small classes
      else if (r < 9)
        n = ((size_t)(1 + rng() % 80) << 20) + rng() % 4096;  // limb-sized blocks
      else
        n = ((size_t)(1 + rng() % 3) << 30) + rng() % 4096;  // above one segment
      char *p = nullptr;
      try {
        p = (char *)pool.alloc(n);
      } catch (const std::runtime_error &) {
        // only when the device is short and the pool holds nothing it could
        // give back: no small cache, no segment without a live block
        if (HostDevice::free_bytes() >= n) return fail("exhausted with room left", it);
        for (auto &kv : pool.free_)
          if (!kv.second.empty()) return fail("exhausted while holding small blocks", it);
        for (auto &sg : pool.segments_) {
          auto *b = pool.blocks_.at(sg.first);
          if (b->free && b->size == sg.second) return fail("exhausted while holding an empty segment", it);
        }
        exhausted++;
        continue;
      }
      for (auto &l : live)
        if (!(p + n <= l.p || l.p + l.n <= p)) return fail("overlap", it);
      live.push_back({p, n});
      live_bytes += n;
    } else {
      const size_t k = rng() % live.size();
      pool.release(live[k].p, live[k].n);
      live_bytes -= live[k].n;
      live[k] = live.back();
      live.pop_back();
    }
    if (pool.live < live_bytes) return fail("live counter below the bytes handed out", it);
  }
  for (auto &l : live) pool.release(l.p, l.n);
  if (pool.live != 0) return fail("live counter after releasing everything", steps);
  if (pool.blocks_.size() != pool.segments_.size()) return fail("free neighbours not merged", steps);
  size_t binned = 0;
  for (auto &kv : pool.bins_) binned += kv.first;
  for (auto &kv : pool.huge_) binned += kv.first;
  if (binned != pool.segment_bytes) return fail("segments not whole", steps);
  pool.trim();
  if (!pool.segments_.empty() || HostDevice::used != 0 || pool.cached != 0)
    return fail("trim left memory behind", steps);
  pool.release_all();
  printf("ok capacity %.0f GiB, %ld steps, peak live %.1f GiB, device allocations %llu, "
         "requests beyond the device %ld\n",
         capacity / 1073741824.0, steps, pool.peak / 1073741824.0,
         (unsigned long long)pool.device_allocs, exhausted);
  return 0;
}

}  // namespace

int main() {
  // roomy device: segments of 1 GiB; tight device: recycling the cache and
  // giving up the runtime reserve under pressure
  if (run((size_t)64 << 30, 200000, 1, (size_t)24 << 30)) return 1;
  if (run((size_t)20 << 30, 100000, 2, (size_t)12 << 30)) return 1;
  return 0;
}
