// The execution layer's pooled allocator: the policy of the reference's
// GpuBufferAllocator (src/runtime/allocator.ts:168-388), with the device
// calls left to a Backend so the policy runs without a GPU as well:
//   static bool Backend::create(uint64_t bytes, void** out);
//   static void Backend::destroy(void* buffer);
// Plain C++ (no HIP), single-threaded per pool; the tally shared by every
// pool on a device carries its own lock.
#pragma once

#include <algorithm>
#include <cstdint>
#include <list>
#include <map>
#include <mutex>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

namespace afhip {

// Requests of at least this size take whole mebibytes (POOL_GRANULARITY_BYTES,
// allocator.ts:41-48).
constexpr uint64_t kPoolGranularity = 1ull << 20;
// An idle buffer untouched for this many submitted boundaries is freed
// (POOL_IDLE_GENERATIONS, allocator.ts:32-39).
constexpr uint64_t kIdleGenerations = 4;
// The idle pool's default cap (COMPACT_GPU_POOL_BYTES, allocator.ts:27-30).
constexpr uint64_t kDefaultMaxPooled = 864ull << 20;

// Resident bytes of every pool on a device and the budget that caps them
// (deviceTally, setGpuMemoryBudget, allocator.ts:50-71).
struct MemoryTally {
  std::mutex mutex;
  uint64_t resident = 0;
  uint64_t budget = UINT64_MAX;
};

// Labels differing only by a trailing index share one group (allocationGroup,
// allocator.ts:110: the label with /-?\d+$/ removed; "" reads "unlabelled").
inline std::string allocation_group(const char* label) {
  std::string s = (label && *label) ? label : "unlabelled";
  size_t end = s.size();
  while (end > 0 && s[end - 1] >= '0' && s[end - 1] <= '9') end--;
  if (end < s.size()) {
    if (end > 0 && s[end - 1] == '-') end--;
    s.resize(end);
  }
  return s;
}

enum class PoolStatus { ok, over_budget, device_refused, invalid_size };

template <typename Backend> class BufferPool {
 public:
  struct Share {
    std::string label;
    uint64_t bytes;
    uint64_t count;
  };

  BufferPool(MemoryTally& tally, uint64_t max_pooled) : tally_(tally), max_pooled_(max_pooled) {}
  BufferPool(const BufferPool&) = delete;
  BufferPool& operator=(const BufferPool&) = delete;

  // allocate (allocator.ts:197-269): the request rounded up to 4 bytes, and
  // to whole mebibytes from 1 MiB; the smallest idle buffer that covers it and
  // is at most twice its size is reused, else a new one is created within
  // the budget. *physical receives the buffer's size (the bytes a budget
  // refusal asked for).
  PoolStatus allocate(const char* label, uint64_t requested, void** out, uint64_t* physical) {
    if (requested == 0) return PoolStatus::invalid_size;
    const uint64_t bytes = (requested + 3) / 4 * 4;
    const uint64_t want =
        bytes >= kPoolGranularity ? (bytes + kPoolGranularity - 1) / kPoolGranularity * kPoolGranularity : bytes;
    auto best = idle_.end();
    for (auto it = idle_.begin(); it != idle_.end(); ++it) {
      if (it->bytes < want || it->bytes > 2 * want) continue;
      if (best == idle_.end() || it->bytes < best->bytes) best = it;
    }
    void* buffer = nullptr;
    uint64_t size = want;
    if (best != idle_.end()) {
      buffer = best->buffer;
      size = best->bytes;
      pooled_ -= best->bytes;
      idle_.erase(best);
    } else {
      {
        std::lock_guard<std::mutex> lock(tally_.mutex);
        if (tally_.budget != UINT64_MAX && tally_.resident + want > tally_.budget) {
          *physical = want;
          return PoolStatus::over_budget;
        }
        tally_.resident += want;
      }
      if (!Backend::create(want, &buffer)) {
        std::lock_guard<std::mutex> lock(tally_.mutex);
        tally_.resident -= want;
        *physical = want;
        return PoolStatus::device_refused;
      }
      resident_ += want;
      peak_resident_ = std::max(peak_resident_, resident_);
      buffer_count_++;
    }
    Live l{bytes, size, allocation_group(label)};
    current_ += bytes;
    auto& g = live_by_group_[l.group];
    g.first += bytes;
    g.second += 1;
    if (current_ > peak_) {
      peak_ = current_;
      peak_composition_.clear();
      for (const auto& e : live_by_group_) peak_composition_.push_back({e.first, e.second.first, e.second.second});
      std::stable_sort(peak_composition_.begin(), peak_composition_.end(),
                       [](const Share& a, const Share& b) { return a.bytes > b.bytes; });
    }
    live_[buffer] = std::move(l);
    allocation_count_++;
    *out = buffer;
    *physical = size;
    return PoolStatus::ok;
  }

  // noteRelease (allocator.ts:287-321): the buffer joins the idle pool, the
  // newest at the back; false when `buffer` is not a live allocation.
  bool release(void* buffer) {
    auto it = live_.find(buffer);
    if (it == live_.end()) return false;
    current_ -= it->second.bytes;
    auto g = live_by_group_.find(it->second.group);
    if (g != live_by_group_.end()) {
      g->second.first -= it->second.bytes;
      if (--g->second.second == 0) live_by_group_.erase(g);
    }
    idle_.push_back({buffer, it->second.physical, generation_});
    pooled_ += it->second.physical;
    live_.erase(it);
    return true;
  }

  bool is_live(void* buffer) const { return live_.count(buffer) != 0; }

  // trimPooled (allocator.ts:323-325): the oldest idle buffers are freed
  // until the pool is within its cap.
  void trim() {
    while (pooled_ > max_pooled_ && !idle_.empty()) evict(idle_.begin());
  }

  // noteSubmitted (allocator.ts:332-341).
  void note_submitted() {
    generation_++;
    while (!idle_.empty() && idle_.front().generation + kIdleGenerations <= generation_) evict(idle_.begin());
    trim();
  }

  // destroyPooled (allocator.ts:362-374).
  void destroy_pooled() {
    while (!idle_.empty()) evict(idle_.begin());
  }

  uint64_t current_bytes() const { return current_; }
  uint64_t peak_bytes() const { return peak_; }
  const std::vector<Share>& peak_composition() const { return peak_composition_; }
  uint64_t resident_bytes() const { return resident_; }
  uint64_t peak_resident_bytes() const { return peak_resident_; }
  uint64_t pooled_bytes() const { return pooled_; }
  uint64_t allocation_count() const { return allocation_count_; }
  uint64_t buffer_count() const { return buffer_count_; }

 private:
  struct Idle {
    void* buffer;
    uint64_t bytes;
    uint64_t generation;
  };
  struct Live {
    uint64_t bytes;     // requested, rounded up to 4
    uint64_t physical;  // the buffer's size
    std::string group;
  };

  void evict(typename std::list<Idle>::iterator it) {
    Backend::destroy(it->buffer);
    {
      std::lock_guard<std::mutex> lock(tally_.mutex);
      tally_.resident -= it->bytes;
    }
    resident_ -= it->bytes;
    pooled_ -= it->bytes;
    idle_.erase(it);
  }

  MemoryTally& tally_;
  uint64_t max_pooled_;
  std::list<Idle> idle_;  // retirement order, the oldest first
  std::unordered_map<void*, Live> live_;
  // Live bytes and count by group, ordered so the peak composition is
  // reproducible.
  std::map<std::string, std::pair<uint64_t, uint64_t>> live_by_group_;
  std::vector<Share> peak_composition_;
  uint64_t generation_ = 0;
  uint64_t current_ = 0, peak_ = 0, resident_ = 0, peak_resident_ = 0, pooled_ = 0;
  uint64_t allocation_count_ = 0, buffer_count_ = 0;
};

}  // namespace afhip
