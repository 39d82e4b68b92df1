// afhip_gemm_run_static: afhip_gemm_run with the plan's workspace in a
// device array the library owns, for callers that cannot allocate device
// memory (code under HIP graph capture, tight serving loops, harnesses that
// forbid hipMalloc).
//
// The workspace a plan needs is the weight laid out k-contiguous for the
// kernels (a [K][N] weight transposed, and converted to the kernel's dtype).
// Here it goes into `scratch`, a file-scope device array of
// kStaticScratchBytes; each GPU the library runs on holds its own copy until
// the process ends. Host code never passes the array's name to a kernel (on
// the host it is only a stand-in symbol): afhip_open looks up the array's
// device address once per device, with that device current, and every use
// goes through that address.
//
// Every call on one GPU shares that GPU's array and leaves the last call's
// transposed weight in it. Nothing needs clearing: a run writes every
// element of the transposed weight it then reads. Calls that overlap on one
// GPU (two streams, two threads) race on the array; a caller serialises
// them.
#include <mutex>

#include "gemm.h"

namespace afhip {

// 8 MiB: a [K][N] weight with K * N up to 4,194,304 f16 (or int8) or
// 2,097,152 f32 elements per run, every batch's copy included. The model's
// projection weights are at most 1,024 x 1,024.
constexpr size_t kStaticScratchBytes = size_t(8) << 20;
constexpr int kMaxDevices = 64;

static __device__ __align__(256) unsigned char scratch[kStaticScratchBytes];

namespace {
std::mutex g_scratch_mutex;
void* g_scratch_address[kMaxDevices] = {};
}  // namespace

int static_scratch_init(int device) {
  AFHIP_REQUIRE(device >= 0 && device < kMaxDevices, "device ordinal %d is beyond the %d devices afhip tracks",
                device, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_address[device] != nullptr) return AFHIP_OK;
  void* address = nullptr;
  AFHIP_CHECK_HIP(hipGetSymbolAddress(&address, HIP_SYMBOL(scratch)));
  AFHIP_REQUIRE(address != nullptr, "the static GEMM scratch has no device address on device %d", device);
  g_scratch_address[device] = address;
  return AFHIP_OK;
}

}  // namespace afhip

using namespace afhip;

extern "C" {

int afhip_gemm_static_scratch_bytes(size_t* bytes) {
  AFHIP_REQUIRE(bytes != nullptr, "output is NULL");
  *bytes = kStaticScratchBytes;
  return AFHIP_OK;
}

int afhip_gemm_run_static(const afhip_gemm_plan* plan, const void* a, const void* w, const float* scale,
                          const float* bias, const void* residual, void* c, void* stream) {
  if (int s = require_open()) return s;
  AFHIP_REQUIRE(plan != nullptr, "plan is NULL");
  size_t need = 0;
  if (int s = afhip_gemm_workspace_size(plan, &need)) return s;
  AFHIP_REQUIRE(need <= kStaticScratchBytes,
                "this plan needs a %zu-byte workspace; the static scratch holds %zu bytes (use afhip_gemm_run "
                "with a workspace of your own)",
                need, kStaticScratchBytes);
  void* address = nullptr;
  {
    const int device = current_device();
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (device >= 0 && device < kMaxDevices) address = g_scratch_address[device];
  }
  if (address == nullptr)
    return set_error(AFHIP_ERR_NOT_OPEN, "the static GEMM scratch was not set up on this device");
  // Timing events are objects the runtime creates; none are made here.
  TimingOff no_events;
  return run_gemm_plan(plan, a, w, scale, bias, residual, c, need ? address : nullptr, need ? kStaticScratchBytes : 0,
                       stream);
}

}  // extern "C"
