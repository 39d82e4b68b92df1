// The HIP execution layer: device-resident tensors that outlive one operator
// call, so a block's steps chain on the device with no host round trip. The
// counterpart of WebGpuExecution (src/runtime/execution.ts:153-555) and its
// GpuBufferAllocator (src/runtime/allocator.ts:168-388).
//
// Allocation follows the reference allocator's policy, restated for HIP:
//  - requests of 1 MiB and more are backed by whole mebibytes, so scratch
//    sized from byte budgets a few percent apart shares buffers
//    (POOL_GRANULARITY_BYTES, allocator.ts:41-48);
//  - a released tensor's buffer goes to an idle pool; a request takes the
//    smallest idle buffer that covers it and is at most twice its size
//    (allocator.ts:211-233);
//  - an idle buffer no request took within four submitted boundaries is
//    freed, and the pool is trimmed to a byte cap (864 MiB by default) at
//    each boundary (POOL_IDLE_GENERATIONS, COMPACT_GPU_POOL_BYTES,
//    allocator.ts:30-39, :323-341);
//  - one budget caps the resident bytes of every execution on the device
//    together, and a request past it fails naming the tensor
//    (setGpuMemoryBudget, GpuMemoryBudgetError, allocator.ts:56-100).
// What WebGPU needed and HIP does not: queue writes overtaking encoded
// commands (requireSubmitted, allocator.ts:102-109) cannot happen, since
// uploads and kernels share one stream and run in its order; bind-group
// caching and submission pacing have no counterpart, since a kernel launch
// binds plain pointers and a HIP stream has no command-buffer timeout.
//
// An execution is used from one host thread at a time, as the reference's is
// from the JS thread. Releasing a tensor while kernels that use it are still
// queued is safe: a later request reuses the buffer on the same stream, and
// freeing it (hipFree) waits for the device.
#include <algorithm>
#include <cstring>
#include <string>
#include <vector>

#include "internal.h"
#include "pool.h"

namespace afhip {
namespace {

struct HipBackend {
  static bool create(uint64_t bytes, void** out) {
    if (hipMalloc(out, bytes) == hipSuccess) return true;
    (void)hipGetLastError();
    return false;
  }
  static void destroy(void* buffer) { (void)hipFree(buffer); }
};

// The open device's tally: every execution's resident bytes and the budget.
MemoryTally g_tally;

double mib(uint64_t bytes) { return (double)bytes / (1024.0 * 1024.0); }

template <typename TB, typename TU>
__global__ void add_in_place_kernel(TB* __restrict__ base, const TU* __restrict__ update, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    base[i] = (TB)((float)base[i] + (float)update[i]);
}

}  // namespace
}  // namespace afhip

using namespace afhip;

struct afhip_execution {
  explicit afhip_execution(uint64_t max_pooled) : pool(g_tally, max_pooled) {}

  hipStream_t stream = nullptr;
  BufferPool<HipBackend> pool;
  // Every allocation in order, for checkpoints (WebGpuExecution.#allocations,
  // execution.ts:160); released ones stay until release_since drops them.
  std::vector<void*> records;

  int allocate(const char* label, uint64_t bytes, void** out) {
    uint64_t physical = 0;
    switch (pool.allocate(label, bytes, out, &physical)) {
      case PoolStatus::ok:
        records.push_back(*out);
        return AFHIP_OK;
      case PoolStatus::invalid_size:
        return set_error(AFHIP_ERR_INVALID_ARGUMENT, "invalid allocation size %llu for %s",
                         (unsigned long long)bytes, label ? label : "unlabelled");
      case PoolStatus::over_budget: {
        uint64_t resident, budget;
        {
          std::lock_guard<std::mutex> lock(g_tally.mutex);
          resident = g_tally.resident;
          budget = g_tally.budget;
        }
        return set_error(AFHIP_ERR_OUT_OF_MEMORY,
                         "GPU memory budget exceeded: allocating %.0f MiB for %s would bring resident GPU memory to "
                         "%.0f MiB, over the %.0f MiB budget. Reduce the MSA rows, the sequence length, or the "
                         "number of chains.",
                         mib(physical), label ? label : "unlabelled", mib(resident + physical), mib(budget));
      }
      default:
        return set_error(AFHIP_ERR_OUT_OF_MEMORY, "hipMalloc of %.0f MiB for %s failed", mib(physical),
                         label ? label : "unlabelled");
    }
  }
  int release_since(uint64_t checkpoint) {
    AFHIP_REQUIRE(checkpoint <= records.size(), "invalid GPU allocation checkpoint %llu",
                  (unsigned long long)checkpoint);
    // A released tensor's buffer may since have been handed out again; only
    // the newest record of a pointer can still be the live one.
    for (size_t i = records.size(); i-- > checkpoint;) {
      bool newest = true;
      for (size_t k = i + 1; k < records.size() && newest; k++) newest = records[k] != records[i];
      if (newest) pool.release(records[i]);
    }
    records.resize(checkpoint);
    pool.trim();
    return AFHIP_OK;
  }
};

namespace {

int require_execution(const afhip_execution* ex) {
  if (int s = require_open()) return s;
  AFHIP_REQUIRE(ex != nullptr, "NULL execution");
  return AFHIP_OK;
}

// The pair-stack steps share these: the workspace of one step comes from the
// execution's pool and goes back to it when the step has been queued.
template <typename SizeFn, typename RunFn>
int pooled_step(afhip_execution* ex, const char* label, SizeFn size, RunFn run) {
  size_t bytes = 0;
  if (int s = size(&bytes)) return s;
  const uint64_t mark = ex->records.size();
  void* ws = nullptr;
  if (bytes > 0)
    if (int s = ex->allocate(label, bytes, &ws)) return s;
  const int s = run(ws, bytes);
  ex->release_since(mark);
  return s;
}

}  // namespace

extern "C" {

int afhip_set_memory_budget(uint64_t bytes) {
  std::lock_guard<std::mutex> lock(g_tally.mutex);
  g_tally.budget = bytes == 0 ? UINT64_MAX : bytes;
  return AFHIP_OK;
}

int afhip_memory_resident(uint64_t* bytes) {
  AFHIP_REQUIRE(bytes != nullptr, "output is NULL");
  std::lock_guard<std::mutex> lock(g_tally.mutex);
  *bytes = g_tally.resident;
  return AFHIP_OK;
}

int afhip_execution_create(uint64_t max_pooled_bytes, void* stream, afhip_execution** out) {
  if (int s = require_open()) return s;
  AFHIP_REQUIRE(out != nullptr, "output is NULL");
  auto* ex = new (std::nothrow) afhip_execution(max_pooled_bytes == 0 ? kDefaultMaxPooled : max_pooled_bytes);
  if (!ex) return set_error(AFHIP_ERR_OUT_OF_MEMORY, "cannot allocate an execution");
  ex->stream = (hipStream_t)stream;
  *out = ex;
  return AFHIP_OK;
}

int afhip_execution_destroy(afhip_execution* ex) {
  if (!ex) return AFHIP_OK;
  ex->release_since(0);
  ex->pool.destroy_pooled();
  delete ex;
  return AFHIP_OK;
}

int afhip_execution_allocate(afhip_execution* ex, const char* label, uint64_t bytes, void** out) {
  if (int s = require_execution(ex)) return s;
  AFHIP_REQUIRE(out != nullptr, "output is NULL");
  return ex->allocate(label, bytes, out);
}

int afhip_execution_upload(afhip_execution* ex, const char* label, const void* host, uint64_t bytes, void** out) {
  if (int s = require_execution(ex)) return s;
  AFHIP_REQUIRE(host != nullptr && out != nullptr, "NULL argument");
  void* p = nullptr;
  if (int s = ex->allocate(label, bytes, &p)) return s;
  AFHIP_CHECK_HIP(hipMemcpyAsync(p, host, bytes, hipMemcpyHostToDevice, ex->stream));
  AFHIP_CHECK_HIP(hipStreamSynchronize(ex->stream));  // the host data may go away on return
  *out = p;
  return AFHIP_OK;
}

int afhip_execution_release(afhip_execution* ex, void* tensor) {
  if (int s = require_execution(ex)) return s;
  AFHIP_REQUIRE(ex->pool.release(tensor), "the pointer is not a live tensor of this execution");
  return AFHIP_OK;
}

int afhip_execution_checkpoint(const afhip_execution* ex, uint64_t* out) {
  AFHIP_REQUIRE(ex != nullptr && out != nullptr, "NULL argument");
  *out = ex->records.size();
  return AFHIP_OK;
}

int afhip_execution_release_since(afhip_execution* ex, uint64_t checkpoint) {
  if (int s = require_execution(ex)) return s;
  return ex->release_since(checkpoint);
}

int afhip_execution_note_submitted(afhip_execution* ex) {
  if (int s = require_execution(ex)) return s;
  ex->pool.note_submitted();
  return AFHIP_OK;
}

int afhip_execution_snapshot(const afhip_execution* ex, char* json, size_t capacity) {
  AFHIP_REQUIRE(ex != nullptr && json != nullptr && capacity > 0, "NULL argument");
  const auto& p = ex->pool;
  std::string s = "{\"currentBytes\":" + std::to_string(p.current_bytes()) +
                  ",\"peakBytes\":" + std::to_string(p.peak_bytes()) + ",\"peakComposition\":[";
  const auto& comp = p.peak_composition();
  for (size_t i = 0; i < comp.size(); i++) {
    std::string label;
    for (char c : comp[i].label) {
      if (c == '"' || c == '\\') label += '\\';
      if ((unsigned char)c >= 0x20) label += c;
    }
    s += (i ? "," : "") + std::string("{\"label\":\"") + label + "\",\"bytes\":" +
         std::to_string(comp[i].bytes) + ",\"count\":" + std::to_string(comp[i].count) + "}";
  }
  s += "],\"residentBytes\":" + std::to_string(p.resident_bytes()) +
       ",\"peakResidentBytes\":" + std::to_string(p.peak_resident_bytes()) +
       ",\"pooledBytes\":" + std::to_string(p.pooled_bytes()) +
       ",\"allocationCount\":" + std::to_string(p.allocation_count()) +
       ",\"bufferCount\":" + std::to_string(p.buffer_count()) + "}";
  AFHIP_REQUIRE(s.size() + 1 <= capacity, "snapshot needs %zu bytes", s.size() + 1);
  std::memcpy(json, s.c_str(), s.size() + 1);
  return AFHIP_OK;
}

int afhip_execution_add_in_place(afhip_execution* ex, void* base, int32_t base_dtype, const void* update,
                                 int32_t update_dtype, int64_t elements) {
  if (int s = require_execution(ex)) return s;
  AFHIP_REQUIRE(base && update, "NULL tensor");
  AFHIP_REQUIRE(elements > 0, "residual tensors must have a positive size");
  AFHIP_REQUIRE(valid_float_dtype(base_dtype) && valid_float_dtype(update_dtype), "residuals are f32 or f16");
  const int cus = device_cu_count() > 0 ? device_cu_count() : 256;
  const dim3 grid((unsigned)std::min<int64_t>(ceil_div(elements, 256), (int64_t)cus * 16));
  hipStream_t st = ex->stream;
  if (base_dtype == AFHIP_F32)
    return update_dtype == AFHIP_F32
               ? launch("execution.add_in_place", add_in_place_kernel<float, float>, grid, dim3(256), 0, st,
                        (float*)base, (const float*)update, elements)
               : launch("execution.add_in_place", add_in_place_kernel<float, half_t>, grid, dim3(256), 0, st,
                        (float*)base, (const half_t*)update, elements);
  return update_dtype == AFHIP_F32
             ? launch("execution.add_in_place", add_in_place_kernel<half_t, float>, grid, dim3(256), 0, st,
                      (half_t*)base, (const float*)update, elements)
             : launch("execution.add_in_place", add_in_place_kernel<half_t, half_t>, grid, dim3(256), 0, st,
                      (half_t*)base, (const half_t*)update, elements);
}

int afhip_execution_pair_stack(afhip_execution* ex, const afhip_pair_stack_desc* desc,
                               const afhip_pair_stack_weights* weights, const void* msa, const float* msa_mask,
                               void* pair, const float* pair_mask) {
  if (int s = require_execution(ex)) return s;
  AFHIP_REQUIRE(desc && weights && pair && pair_mask, "NULL argument");
  const afhip_pair_stack_desc& d = *desc;
  const int L = d.outgoing.length;
  AFHIP_REQUIRE(L > 0, "the pair stack needs a positive length");
  // Every step updates the pair in place: its own residual add, the pair as
  // both input and output. Each step reads a pair's values before writing
  // that pair, and the triangle projects all of z before any output block.
  afhip_triangle_desc out = d.outgoing, in = d.incoming;
  afhip_opm_desc opm = d.opm;
  afhip_transition_desc tr = d.transition;
  out.direction = AFHIP_TRIANGLE_OUTGOING;
  in.direction = AFHIP_TRIANGLE_INCOMING;
  out.residual = in.residual = opm.residual = tr.residual = 1;
  AFHIP_REQUIRE(in.length == L && in.c_z == out.c_z, "the two triangle steps disagree on the pair's shape");
  AFHIP_REQUIRE(out.pair_dtype == out.out_dtype && in.pair_dtype == in.out_dtype && in.pair_dtype == out.pair_dtype,
                "the pair stays in one dtype through the stack");
  const int pdt = out.pair_dtype;
  if (weights->opm) {
    AFHIP_REQUIRE(msa && msa_mask, "the outer-product mean needs the MSA and its mask");
    AFHIP_REQUIRE(opm.length == L && opm.c_z == out.c_z && opm.out_dtype == pdt,
                  "the outer-product mean's output does not match the pair");
    if (int s = pooled_step(
            ex, "pair-stack.outer-product-mean",
            [&](size_t* b) { return afhip_opm_workspace_size(&opm, b); },
            [&](void* ws, size_t b) {
              return afhip_opm_run(&opm, msa, msa_mask, weights->opm, pair, ws, b, ex->stream);
            }))
      return s;
  }
  if (weights->outgoing) {
    if (int s = pooled_step(
            ex, "pair-stack.triangle-outgoing", [&](size_t* b) { return afhip_triangle_workspace_size(&out, b); },
            [&](void* ws, size_t b) {
              return afhip_triangle_run(&out, pair, pair_mask, weights->outgoing, pair, ws, b, ex->stream);
            }))
      return s;
  }
  if (weights->incoming) {
    if (int s = pooled_step(
            ex, "pair-stack.triangle-incoming", [&](size_t* b) { return afhip_triangle_workspace_size(&in, b); },
            [&](void* ws, size_t b) {
              return afhip_triangle_run(&in, pair, pair_mask, weights->incoming, pair, ws, b, ex->stream);
            }))
      return s;
  }
  afhip_attention_desc att[2] = {d.attention_start, d.attention_end};
  const void* att_w[2] = {weights->attention_start, weights->attention_end};
  const char* att_label[2] = {"pair-stack.triangle-attention-starting", "pair-stack.triangle-attention-ending"};
  for (int i = 0; i < 2; i++) {
    if (!att_w[i]) continue;
    afhip_attention_desc& ad = att[i];
    ad.transpose = i;
    ad.pair_bias = AFHIP_PAIR_BIAS_NORMALIZED_INPUT;
    ad.residual = 1;
    AFHIP_REQUIRE(ad.batch == L && ad.queries == L && ad.channels == out.c_z && ad.in_dtype == pdt &&
                      ad.out_dtype == pdt,
                  "the triangle attention does not match the pair");
    if (int s = pooled_step(
            ex, att_label[i], [&](size_t* b) { return afhip_attention_workspace_size(&ad, b); },
            [&](void* ws, size_t b) {
              return afhip_attention_run(&ad, pair, pair_mask, nullptr, att_w[i], pair, ws, b, ex->stream);
            }))
      return s;
  }
  if (weights->transition) {
    AFHIP_REQUIRE(tr.rows == (int64_t)L * L && tr.channels == out.c_z && tr.in_dtype == pdt && tr.out_dtype == pdt,
                  "the pair transition does not match the pair");
    if (int s = pooled_step(
            ex, "pair-stack.transition", [&](size_t* b) { return afhip_transition_workspace_size(&tr, b); },
            [&](void* ws, size_t b) {
              return afhip_transition_run(&tr, pair, weights->transition, pair, ws, b, ex->stream);
            }))
      return s;
  }
  return AFHIP_OK;
}

int afhip_execution_evoformer_block(afhip_execution* ex, const afhip_evoformer_block_desc* desc,
                                    const afhip_evoformer_block_weights* weights, void* msa, const float* msa_mask,
                                    void* pair, const float* pair_mask) {
  if (int s = require_execution(ex)) return s;
  AFHIP_REQUIRE(desc && weights && msa && msa_mask && pair && pair_mask, "NULL argument");
  const afhip_evoformer_block_desc& d = *desc;
  const afhip_pair_stack_desc& ps = d.pair;
  const int L = ps.outgoing.length, S = ps.opm.sequences, cm = ps.opm.c_m, cz = ps.outgoing.c_z;
  const int dt = ps.outgoing.pair_dtype;
  AFHIP_REQUIRE(L > 0 && S > 0 && cm > 0, "the block needs positive sequences, length and MSA channels");
  afhip_attention_desc row = d.msa_row, col = d.msa_column;
  afhip_transition_desc mt = d.msa_transition;
  row.transpose = 0;
  row.pair_bias = AFHIP_PAIR_BIAS_SEPARATE;
  col.transpose = 1;
  col.pair_bias = AFHIP_PAIR_BIAS_NONE;
  row.residual = col.residual = mt.residual = 1;
  AFHIP_REQUIRE(row.batch == S && row.queries == L && row.channels == cm && row.pair_channels == cz &&
                    row.in_dtype == dt && row.out_dtype == dt,
                "the MSA row attention does not match the block");
  AFHIP_REQUIRE(col.batch == L && col.queries == S && col.channels == cm && col.in_dtype == dt && col.out_dtype == dt,
                "the MSA column attention does not match the block");
  AFHIP_REQUIRE(mt.rows == (int64_t)S * L && mt.channels == cm && mt.in_dtype == dt && mt.out_dtype == dt,
                "the MSA transition does not match the block");
  AFHIP_REQUIRE(ps.opm.msa_dtype == dt, "the MSA and the pair share one dtype");
  const afhip_pair_stack_weights& pw = weights->pair;
  const afhip_pair_stack_weights opm_only{pw.opm, nullptr, nullptr, nullptr, nullptr, nullptr};
  afhip_pair_stack_weights rest = pw;
  if (d.opm_first) {
    if (int s = afhip_execution_pair_stack(ex, &ps, &opm_only, msa, msa_mask, pair, pair_mask)) return s;
    rest.opm = nullptr;
  }
  if (weights->msa_row) {
    if (int s = pooled_step(
            ex, "evoformer.msa-row-attention", [&](size_t* b) { return afhip_attention_workspace_size(&row, b); },
            [&](void* ws, size_t b) {
              return afhip_attention_run(&row, msa, msa_mask, pair, weights->msa_row, msa, ws, b, ex->stream);
            }))
      return s;
  }
  if (weights->msa_column) {
    if (int s = pooled_step(
            ex, "evoformer.msa-column-attention", [&](size_t* b) { return afhip_attention_workspace_size(&col, b); },
            [&](void* ws, size_t b) {
              return afhip_attention_run(&col, msa, msa_mask, nullptr, weights->msa_column, msa, ws, b, ex->stream);
            }))
      return s;
  }
  if (weights->msa_transition) {
    if (int s = pooled_step(
            ex, "evoformer.msa-transition", [&](size_t* b) { return afhip_transition_workspace_size(&mt, b); },
            [&](void* ws, size_t b) {
              return afhip_transition_run(&mt, msa, weights->msa_transition, msa, ws, b, ex->stream);
            }))
      return s;
  }
  return afhip_execution_pair_stack(ex, &ps, &rest, msa, msa_mask, pair, pair_mask);
}

}  // extern "C"
