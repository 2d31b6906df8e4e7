// device_pool.hpp -- the device memory pool of one context.
//
// Blocks up to 1 MiB come from exact-size free lists; larger ones up to
// 1 GiB are carved best-fit out of 1 GiB segments, split on allocation and
// merged with free neighbours on release, so that buffers of every modulus
// level share one cache instead of one cache per size.  A block above 1 GiB
// gets a segment of its own, which is reused whole (by a request of at least
// two thirds of its size) and never split, so that it can always go back to
// the device when memory runs short.  All work of a context is ordered on
// one stream, so a block released here can be handed to the next kernel on
// that stream without a synchronisation.
//
// The pool is written against a device policy `Dev` with
//   static bool   alloc(void **p, size_t bytes);  // false when out of memory
//   static void   release(void *p);
//   static size_t free_bytes();                   // device memory free now
//   static void   synchronize();                  // wait for the device
// so that the same code runs on the GPU and, over host memory, in tests.
#pragma once

#include <stddef.h>
#include <stdint.h>

#include <map>
#include <stdexcept>
#include <unordered_map>
#include <utility>
#include <vector>

namespace ckks {

template <class Dev>
struct BasicPool {
  static constexpr size_t kSmallMax = (size_t)1 << 20;     // exact classes up to here
  static constexpr size_t kLargeGrain = (size_t)64 << 10;  // large blocks: 64 KiB units
  static constexpr size_t kSegment = (size_t)1 << 30;      // large blocks come from 1 GiB
  // Device memory the pool leaves free for the runtime: hardware queues and
  // the private segment it sizes for a kernel when that kernel is dispatched.
  static constexpr size_t kRuntimeReserve = (size_t)2 << 30;

  struct Block {
    char *base;
    size_t size;
    bool free;
    Block *prev, *next;  // address neighbours inside the segment
    typename std::multimap<size_t, Block *>::iterator slot;  // entry in `bins_`/`huge_` while free
  };

  std::unordered_map<size_t, std::vector<void *>> free_;  // small classes
  std::unordered_map<void *, size_t> live_;               // small blocks handed out
  std::multimap<size_t, Block *> bins_;                   // free large blocks by size
  std::multimap<size_t, Block *> huge_;                   // free own-segment blocks by size
  std::unordered_map<void *, Block *> blocks_;            // every large block by base
  std::vector<std::pair<char *, size_t>> segments_;
  size_t live = 0, cached = 0, peak = 0, segment_bytes = 0;
  uint64_t device_allocs = 0;

  BasicPool() = default;
  // host records only: device memory goes back through release_all
  ~BasicPool() {
    for (auto &kv : blocks_) delete kv.second;
  }
  BasicPool(const BasicPool &) = delete;
  BasicPool &operator=(const BasicPool &) = delete;

  static size_t round_up(size_t v, size_t g) { return (v + g - 1) / g * g; }

  void *alloc(size_t bytes) {
    void *p = nullptr;
    if (bytes > kSmallMax) {
      p = alloc_large(bytes);
    } else {
      bytes = round_up(bytes, 256);
      auto it = free_.find(bytes);
      if (it != free_.end() && !it->second.empty()) {
        p = it->second.back();
        it->second.pop_back();
        cached -= bytes;
      } else {
        p = raw_alloc(bytes);
      }
      live_[p] = bytes;
      live += bytes;
    }
    if (live > peak) peak = live;
    return p;
  }

  void release(void *p, size_t bytes) {
    if (!p) return;
    if (bytes > kSmallMax) {
      release_large(p);
      return;
    }
    bytes = round_up(bytes, 256);
    live_.erase(p);
    free_[bytes].push_back(p);
    live -= bytes;
    cached += bytes;
  }

  // Device memory for long-lived objects (keys, tensors), after giving back
  // what the cache holds when the device is short of it.
  void *raw_alloc(size_t bytes) {
    void *p = nullptr;
    if (Dev::free_bytes() < bytes + kRuntimeReserve) make_room(bytes);
    if (!Dev::alloc(&p, bytes)) {
      make_room(bytes);
      if (!Dev::alloc(&p, bytes)) throw std::runtime_error("device memory exhausted");
    }
    device_allocs++;
    return p;
  }

  // Everything cached goes back to the device; live blocks stay.
  void trim() {
    Dev::synchronize();
    for (auto &kv : free_)
      for (void *p : kv.second) Dev::release(p);
    free_.clear();
    free_segments();
    cached = 0;
    for (auto &kv : bins_) cached += kv.first;
    for (auto &kv : huge_) cached += kv.first;
  }

  // Every block, live or not, goes back to the device (context teardown).
  void release_all() {
    trim();
    for (auto &kv : live_) Dev::release(kv.first);
    live_.clear();
    for (auto &s : segments_) Dev::release(s.first);
    segments_.clear();
    for (auto &kv : blocks_) delete kv.second;
    blocks_.clear();
    bins_.clear();
    huge_.clear();
    live = cached = segment_bytes = 0;
  }

 private:
  void *alloc_large(size_t bytes) {
    bytes = round_up(bytes, kLargeGrain);
    if (bytes > kSegment) return alloc_huge(bytes);
    auto it = bins_.lower_bound(bytes);
    if (it == bins_.end()) {
      if (!grow(bytes)) throw std::runtime_error("device memory exhausted");
      it = bins_.lower_bound(bytes);
    }
    Block *b = it->second;
    bins_.erase(it);
    b->free = false;
    if (b->size > bytes) {  // split: the tail stays free
      Block *t = new Block{b->base + bytes, b->size - bytes, true, b, b->next, {}};
      if (b->next) b->next->prev = t;
      b->next = t;
      b->size = bytes;
      t->slot = bins_.emplace(t->size, t);
      blocks_[t->base] = t;
    }
    cached -= bytes;
    live += bytes;
    return b->base;
  }

  // A block above one segment: a cached own segment of at most 1.5 times
  // the size, else a new one.
  void *alloc_huge(size_t bytes) {
    auto it = huge_.lower_bound(bytes);
    Block *b = nullptr;
    if (it != huge_.end() && 2 * it->first <= 3 * bytes) {
      b = it->second;
      huge_.erase(it);
    } else {
      if (Dev::free_bytes() < bytes + kRuntimeReserve) make_room(bytes);
      char *d = nullptr;
      if (!Dev::alloc((void **)&d, bytes)) {
        make_room(bytes);
        if (!Dev::alloc((void **)&d, bytes)) throw std::runtime_error("device memory exhausted");
      }
      device_allocs++;
      segments_.push_back({d, bytes});
      segment_bytes += bytes;
      b = new Block{d, bytes, true, nullptr, nullptr, {}};
      blocks_[d] = b;
      cached += bytes;
    }
    b->free = false;
    cached -= b->size;
    live += b->size;
    return b->base;
  }

  void release_large(void *p) {
    auto it = blocks_.find(p);
    if (it == blocks_.end() || it->second->free)
      throw std::runtime_error("release of a block the pool did not hand out");
    Block *b = it->second;
    live -= b->size;
    cached += b->size;
    b->free = true;
    if (b->size > kSegment) {  // an own segment: kept whole
      b->slot = huge_.emplace(b->size, b);
      return;
    }
    if (b->next && b->next->free) {  // merge the following free block
      Block *n = b->next;
      bins_.erase(n->slot);
      blocks_.erase(n->base);
      b->size += n->size;
      b->next = n->next;
      if (n->next) n->next->prev = b;
      delete n;
    }
    if (b->prev && b->prev->free) {  // merge into the preceding free block
      Block *q = b->prev;
      bins_.erase(q->slot);
      blocks_.erase(b->base);
      q->size += b->size;
      q->next = b->next;
      if (b->next) b->next->prev = q;
      delete b;
      b = q;
    }
    b->slot = bins_.emplace(b->size, b);
  }

  // A new segment of at least `bytes`: 1 GiB where the device has room for
  // it beside the runtime reserve, else exactly `bytes` after handing back
  // what the cache holds.
  bool grow(size_t bytes) {
    size_t want = bytes > kSegment ? bytes : kSegment;
    if (Dev::free_bytes() < want + kRuntimeReserve) {
      want = bytes;
      if (!make_room(bytes)) return false;
    }
    char *d = nullptr;
    if (!Dev::alloc((void **)&d, want)) return false;
    device_allocs++;
    segments_.push_back({d, want});
    segment_bytes += want;
    Block *b = new Block{d, want, true, nullptr, nullptr, {}};
    b->slot = bins_.emplace(want, b);
    blocks_[d] = b;
    cached += want;
    return true;
  }

  // Segments with nothing live in them go back to the device.
  size_t free_segments() {
    size_t freed = 0;
    for (size_t i = 0; i < segments_.size();) {
      Block *b = blocks_.at(segments_[i].first);
      if (b->free && b->size == segments_[i].second) {
        (b->size > kSegment ? huge_ : bins_).erase(b->slot);
        blocks_.erase(b->base);
        Dev::release(b->base);
        cached -= b->size;
        segment_bytes -= b->size;
        freed += b->size;
        delete b;
        segments_[i] = segments_.back();
        segments_.pop_back();
      } else {
        i++;
      }
    }
    return freed;
  }

  // Make `bytes` (plus the runtime reserve) free on the device: first the
  // small classes and the empty segments, then give up the reserve.
  // Whole free segments go back first; the small cached blocks (at most
  // 1 MiB each, each its own device allocation) only when that is not
  // enough: they free little and cost one device allocation each when they
  // are needed again (a layer of the prefill reallocated about 550 of them,
  // over a second, each time they went).
  bool make_room(size_t bytes) {
    if (Dev::free_bytes() >= bytes + kRuntimeReserve) return true;
    Dev::synchronize();
    free_segments();
    if (Dev::free_bytes() >= bytes + kRuntimeReserve) return true;
    for (auto &kv : free_) {
      for (void *q : kv.second) Dev::release(q);
      cached -= kv.first * kv.second.size();
      kv.second.clear();
    }
    return Dev::free_bytes() >= bytes;
  }
};

}  // namespace ckks
