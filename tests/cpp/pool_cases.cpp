// The execution layer's allocator policy (alphafold2-webgpu_amd/csrc/pool.h)
// against a mock device, in the scenarios of the reference's allocator tests
// (test/allocator.test.ts:5-165) plus the HIP-specific ones. Built and run by
// tests/test_execution_pool.py; prints "ok <checks>" or the failed checks.
#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

#include "pool.h"

using afhip::BufferPool;
using afhip::MemoryTally;
using afhip::PoolStatus;

namespace {

int g_checks = 0, g_failed = 0;
#define CHECK(cond)                                                   \
  do {                                                                \
    g_checks++;                                                       \
    if (!(cond)) {                                                    \
      g_failed++;                                                     \
      std::printf("FAILED %s:%d: %s\n", __FILE__, __LINE__, #cond);    \
    }                                                                 \
  } while (0)

// Fake buffers: distinct addresses, creations and destructions recorded.
struct Mock {
  static std::vector<uintptr_t> created;
  static std::vector<uintptr_t> destroyed;
  static bool create(uint64_t, void** out) {
    const uintptr_t p = 0x1000 * (created.size() + 1);
    created.push_back(p);
    *out = reinterpret_cast<void*>(p);
    return true;
  }
  static void destroy(void* b) { destroyed.push_back(reinterpret_cast<uintptr_t>(b)); }
  static void reset() {
    created.clear();
    destroyed.clear();
  }
  static void* buffer(size_t i) { return reinterpret_cast<void*>(created.at(i)); }
  static bool was_destroyed(size_t i) {
    for (uintptr_t d : destroyed)
      if (d == created.at(i)) return true;
    return false;
  }
};
std::vector<uintptr_t> Mock::created, Mock::destroyed;

using Pool = BufferPool<Mock>;

void* take(Pool& p, const char* label, uint64_t bytes) {
  void* out = nullptr;
  uint64_t physical = 0;
  const PoolStatus s = p.allocate(label, bytes, &out, &physical);
  CHECK(s == PoolStatus::ok);
  return out;
}

// allocator.test.ts:5-31
void defers_bounded_eviction_until_a_submitted_boundary() {
  Mock::reset();
  MemoryTally tally;
  Pool pool(tally, 12);
  void* first = take(pool, "first", 8);
  void* second = take(pool, "second", 8);
  pool.release(first);
  pool.release(second);
  CHECK(pool.current_bytes() == 0 && pool.resident_bytes() == 16 && pool.pooled_bytes() == 16);
  CHECK(pool.peak_resident_bytes() == 16);
  CHECK(Mock::destroyed.empty());
  pool.trim();
  CHECK(pool.resident_bytes() == 8 && pool.pooled_bytes() == 8 && pool.peak_resident_bytes() == 16);
  CHECK(Mock::was_destroyed(0) && !Mock::was_destroyed(1));
  void* reused = take(pool, "reused", 8);
  CHECK(Mock::created.size() == 2 && reused == Mock::buffer(1));
  CHECK(pool.pooled_bytes() == 0);
  pool.release(reused);
  pool.destroy_pooled();
  CHECK(pool.current_bytes() == 0 && pool.resident_bytes() == 0 && pool.pooled_bytes() == 0);
  CHECK(tally.resident == 0);
}

// allocator.test.ts:33-44
void does_not_retain_a_buffer_larger_than_the_cap() {
  Mock::reset();
  MemoryTally tally;
  Pool pool(tally, 4);
  pool.release(take(pool, "large", 8));
  CHECK(Mock::destroyed.empty());
  pool.trim();
  CHECK(Mock::was_destroyed(0));
  CHECK(pool.resident_bytes() == 0 && pool.pooled_bytes() == 0);
}

// allocator.test.ts:46-66
void smallest_compatible_allocation_for_a_smaller_tensor() {
  Mock::reset();
  MemoryTally tally;
  Pool pool(tally, 128);
  void* large = take(pool, "large", 32);
  void* best = take(pool, "best", 24);
  pool.release(large);
  pool.release(best);
  void* logical = take(pool, "logical", 16);
  CHECK(logical == Mock::buffer(1) && Mock::created.size() == 2);
  CHECK(pool.current_bytes() == 16 && pool.resident_bytes() == 56 && pool.pooled_bytes() == 32);
  CHECK(pool.buffer_count() == 2);
  pool.release(logical);
  CHECK(pool.current_bytes() == 0 && pool.resident_bytes() == 56 && pool.pooled_bytes() == 56);
  pool.destroy_pooled();
}

// allocator.test.ts:68-86, without usage flags (a HIP buffer has none): a
// retired buffer serves the next request of its size, before and after a
// submitted boundary.
void reuses_a_retired_buffer() {
  Mock::reset();
  MemoryTally tally;
  Pool pool(tally, afhip::kDefaultMaxPooled);
  pool.release(take(pool, "uploaded", 32));
  void* scratch = take(pool, "scratch", 32);
  CHECK(scratch == Mock::buffer(0) && Mock::created.size() == 1);
  pool.release(scratch);
  pool.note_submitted();
  CHECK(take(pool, "uploaded-again", 32) == Mock::buffer(0) && Mock::created.size() == 1);
}

// allocator.test.ts:107-127: two pools on one device share the budget. The
// second pool here pools too (every HIP execution does), so its release is
// followed by destroy_pooled to return the bytes.
void refuses_an_allocation_over_the_budget() {
  Mock::reset();
  MemoryTally tally;
  tally.budget = 64;
  Pool first(tally, afhip::kDefaultMaxPooled), second(tally, afhip::kDefaultMaxPooled);
  void* held = take(first, "trunk", 40);
  CHECK(tally.resident == 40);
  void* out = nullptr;
  uint64_t physical = 0;
  CHECK(second.allocate("structure", 32, &out, &physical) == PoolStatus::over_budget && physical == 32);
  CHECK(Mock::created.size() == 1);
  second.release(take(second, "structure", 24));
  second.destroy_pooled();
  CHECK(tally.resident == 40);
  first.release(held);
  first.destroy_pooled();
  CHECK(tally.resident == 0);
}

// allocator.test.ts:143-165
void reuses_the_smallest_idle_allocation_that_covers() {
  Mock::reset();
  MemoryTally tally;
  Pool pool(tally, afhip::kDefaultMaxPooled);
  void* large = take(pool, "large", 64);
  void* medium = take(pool, "medium", 32);
  pool.release(large);
  pool.release(medium);
  void* reused = take(pool, "small", 16);
  CHECK(reused == Mock::buffer(1) && Mock::created.size() == 2);
  pool.release(reused);
  CHECK(pool.current_bytes() == 0 && pool.resident_bytes() == 96 && pool.pooled_bytes() == 96);
  pool.destroy_pooled();
}

// Mebibyte granularity from 1 MiB (allocator.ts:41-48, :213-214), and the
// twice-the-request bound on reuse (:223-225).
void mebibyte_granularity_and_the_reuse_bound() {
  Mock::reset();
  MemoryTally tally;
  Pool pool(tally, afhip::kDefaultMaxPooled);
  const uint64_t MiB = 1 << 20;
  void* a = take(pool, "a", MiB + MiB / 2);
  CHECK(pool.resident_bytes() == 2 * MiB && pool.current_bytes() == MiB + MiB / 2);
  pool.release(a);
  CHECK(take(pool, "b", MiB + MiB / 10) == Mock::buffer(0));  // 1.1 MiB takes 2 MiB
  pool.release(Mock::buffer(0));
  void* c = take(pool, "c", 900 * 1024);  // under 1 MiB: exact, and 2 MiB is over twice that
  CHECK(c == Mock::buffer(1) && pool.resident_bytes() == 2 * MiB + 900 * 1024);
  uint64_t physical = 0;
  CHECK(pool.allocate("zero", 0, &c, &physical) == PoolStatus::invalid_size);
  pool.release(Mock::buffer(1));
  pool.destroy_pooled();
}

// POOL_IDLE_GENERATIONS (allocator.ts:32-39, :332-341): an idle buffer goes
// at the fourth submitted boundary after its release.
void idle_buffers_go_after_four_boundaries() {
  Mock::reset();
  MemoryTally tally;
  Pool pool(tally, afhip::kDefaultMaxPooled);
  pool.release(take(pool, "one-shot", 64));
  for (int i = 0; i < 3; i++) pool.note_submitted();
  CHECK(pool.pooled_bytes() == 64 && Mock::destroyed.empty());
  pool.note_submitted();
  CHECK(pool.pooled_bytes() == 0 && Mock::was_destroyed(0) && tally.resident == 0);
}

// allocationGroup (allocator.ts:110) and the peak composition (:255-262).
void label_groups_and_peak_composition() {
  CHECK(afhip::allocation_group("block-12") == "block");
  CHECK(afhip::allocation_group("recycle3") == "recycle");
  CHECK(afhip::allocation_group("") == "unlabelled");
  CHECK(afhip::allocation_group(nullptr) == "unlabelled");
  CHECK(afhip::allocation_group("x-") == "x-");
  CHECK(afhip::allocation_group("123").empty());
  Mock::reset();
  MemoryTally tally;
  Pool pool(tally, afhip::kDefaultMaxPooled);
  void* m1 = take(pool, "msa-1", 100);
  take(pool, "msa-2", 100);
  take(pool, "pair", 52);
  pool.release(m1);
  take(pool, "pair-7", 8);
  CHECK(pool.peak_bytes() == 252 && pool.current_bytes() == 160);
  const auto& comp = pool.peak_composition();
  CHECK(comp.size() == 2 && comp[0].label == "msa" && comp[0].bytes == 200 && comp[0].count == 2);
  CHECK(comp[1].label == "pair" && comp[1].bytes == 52 && comp[1].count == 1);
  CHECK(pool.allocation_count() == 4);
}

}  // namespace

int main() {
  defers_bounded_eviction_until_a_submitted_boundary();
  does_not_retain_a_buffer_larger_than_the_cap();
  smallest_compatible_allocation_for_a_smaller_tensor();
  reuses_a_retired_buffer();
  refuses_an_allocation_over_the_budget();
  reuses_the_smallest_idle_allocation_that_covers();
  mebibyte_granularity_and_the_reuse_bound();
  idle_buffers_go_after_four_boundaries();
  label_groups_and_peak_composition();
  if (g_failed) {
    std::printf("%d of %d checks failed\n", g_failed, g_checks);
    return 1;
  }
  std::printf("ok %d\n", g_checks);
  return 0;
}
