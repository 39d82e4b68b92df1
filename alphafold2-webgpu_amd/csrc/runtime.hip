// Context, errors, buffers, device report and kernel timing.
#include <atomic>
#include <cstdarg>
#include <cstring>
#include <map>
#include <mutex>
#include <vector>

#include "internal.h"

namespace afhip {

namespace {
thread_local std::string g_last_error = "no error";
std::mutex g_mutex;
// Read without the lock by every entry point (require_open, the launch paths),
// possibly on other threads than the one that opens or closes the context
// (the Node addon runs operators on its worker threads).
std::atomic<int> g_device{-1};
std::atomic<int> g_cu_count{0};

struct TimingRecord {
  hipEvent_t start, stop;
  std::string label;
};
std::atomic<bool> g_timing{false};
thread_local int g_timing_off = 0;
std::mutex g_timing_mutex;  // guards g_pending and g_totals
std::vector<TimingRecord> g_pending;
std::map<std::string, std::pair<long, double>> g_totals;
}  // namespace

int set_error(int status, const char* fmt, ...) {
  char buffer[1024];
  va_list args;
  va_start(args, fmt);
  vsnprintf(buffer, sizeof(buffer), fmt, args);
  va_end(args);
  g_last_error = buffer;
  return status;
}

int hip_status(hipError_t err, const char* what) {
  if (err == hipErrorOutOfMemory) return set_error(AFHIP_ERR_OUT_OF_MEMORY, "%s: %s", what, hipGetErrorString(err));
  return set_error(AFHIP_ERR_HIP, "%s: %s", what, hipGetErrorString(err));
}

bool is_open() { return g_device.load(std::memory_order_relaxed) >= 0; }

int require_open() {
  if (g_device.load(std::memory_order_relaxed) < 0)
    return set_error(AFHIP_ERR_NOT_OPEN, "afhip_open has not been called");
  return AFHIP_OK;
}

int device_cu_count() { return g_cu_count.load(std::memory_order_relaxed); }

bool timing_enabled() { return g_timing && g_timing_off == 0; }

TimingOff::TimingOff() { g_timing_off++; }
TimingOff::~TimingOff() { g_timing_off--; }

int current_device() { return g_device.load(std::memory_order_relaxed); }

int allow_lds(const void* kernel, size_t bytes) {
  if (bytes <= 65536) return AFHIP_OK;
  static std::mutex mutex;
  static std::map<const void*, size_t> granted;
  std::lock_guard<std::mutex> lock(mutex);
  auto it = granted.find(kernel);
  if (it != granted.end() && it->second >= bytes) return AFHIP_OK;
  AFHIP_CHECK_HIP(hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes));
  granted[kernel] = bytes;
  return AFHIP_OK;
}

bool timing_events(hipEvent_t* start, hipEvent_t* stop) {
  if (hipEventCreate(start) != hipSuccess) return false;
  if (hipEventCreate(stop) != hipSuccess) {
    (void)hipEventDestroy(*start);
    return false;
  }
  return true;
}

void timing_record(const char* label, hipEvent_t start, hipEvent_t stop) {
  std::lock_guard<std::mutex> lock(g_timing_mutex);
  g_pending.push_back({start, stop, label});
}

// Callers hold g_timing_mutex.
static void timing_drain() {
  for (auto& r : g_pending) {
    (void)hipEventSynchronize(r.stop);
    float ms = 0.0f;
    (void)hipEventElapsedTime(&ms, r.start, r.stop);
    auto& t = g_totals[r.label];
    t.first += 1;
    t.second += ms;
    (void)hipEventDestroy(r.start);
    (void)hipEventDestroy(r.stop);
  }
  g_pending.clear();
}

}  // namespace afhip

using namespace afhip;

extern "C" {

const char* afhip_last_error(void) { return g_last_error.c_str(); }

int afhip_abi_version(void) { return AFHIP_ABI_VERSION; }

int afhip_open(int device_ordinal) {
  std::lock_guard<std::mutex> lock(g_mutex);
  int count = 0;
  hipError_t err = hipGetDeviceCount(&count);
  if (err != hipSuccess) return hip_status(err, "hipGetDeviceCount");
  AFHIP_REQUIRE(device_ordinal >= 0 && device_ordinal < count, "device ordinal %d out of range (0..%d)",
                device_ordinal, count - 1);
  AFHIP_CHECK_HIP(hipSetDevice(device_ordinal));
  hipDeviceProp_t prop;
  AFHIP_CHECK_HIP(hipGetDeviceProperties(&prop, device_ordinal));
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return set_error(AFHIP_ERR_UNSUPPORTED, "afhip is built for gfx950; device %d is %s", device_ordinal,
                     prop.gcnArchName);
  if (int s = static_scratch_init(device_ordinal)) return s;
  g_device = device_ordinal;
  g_cu_count = prop.multiProcessorCount;
  return AFHIP_OK;
}

int afhip_close(void) {
  std::lock_guard<std::mutex> lock(g_mutex);
  g_device = -1;
  return AFHIP_OK;
}

int afhip_device_report(char* json, size_t capacity) {
  if (int s = require_open()) return s;
  AFHIP_REQUIRE(json != nullptr && capacity > 0, "report buffer is empty");
  hipDeviceProp_t prop;
  AFHIP_CHECK_HIP(hipGetDeviceProperties(&prop, current_device()));
  int driver = 0, runtime = 0;
  (void)hipDriverGetVersion(&driver);
  (void)hipRuntimeGetVersion(&runtime);
  int n = snprintf(json, capacity,
                   "{\"name\":\"%s\",\"arch\":\"%s\",\"compute_units\":%d,\"clock_khz\":%d,"
                   "\"memory_clock_khz\":%d,\"lds_bytes_per_block\":%zu,\"hbm_bytes\":%zu,"
                   "\"l2_bytes\":%d,\"warp_size\":%d,\"driver_version\":%d,\"runtime_version\":%d}",
                   prop.name, prop.gcnArchName, prop.multiProcessorCount, prop.clockRate, prop.memoryClockRate,
                   (size_t)prop.sharedMemPerBlock, (size_t)prop.totalGlobalMem, prop.l2CacheSize, prop.warpSize,
                   driver, runtime);
  AFHIP_REQUIRE(n > 0 && (size_t)n < capacity, "report buffer of %zu bytes is too small", capacity);
  return AFHIP_OK;
}

int afhip_buffer_create(size_t bytes, void** out) {
  if (int s = require_open()) return s;
  AFHIP_REQUIRE(out != nullptr, "output pointer is NULL");
  AFHIP_REQUIRE(bytes > 0, "buffer size must be positive");
  AFHIP_CHECK_HIP(hipMalloc(out, bytes));
  return AFHIP_OK;
}

int afhip_buffer_destroy(void* buffer) {
  if (buffer == nullptr) return AFHIP_OK;
  AFHIP_CHECK_HIP(hipFree(buffer));
  return AFHIP_OK;
}

int afhip_buffer_write(void* buffer, size_t offset, const void* source, size_t bytes) {
  if (int s = require_open()) return s;
  AFHIP_REQUIRE(buffer != nullptr && (source != nullptr || bytes == 0), "NULL buffer or source");
  AFHIP_CHECK_HIP(hipMemcpy((char*)buffer + offset, source, bytes, hipMemcpyHostToDevice));
  return AFHIP_OK;
}

int afhip_buffer_read(const void* buffer, size_t offset, void* destination, size_t bytes) {
  if (int s = require_open()) return s;
  AFHIP_REQUIRE(buffer != nullptr && (destination != nullptr || bytes == 0), "NULL buffer or destination");
  AFHIP_CHECK_HIP(hipMemcpy(destination, (const char*)buffer + offset, bytes, hipMemcpyDeviceToHost));
  return AFHIP_OK;
}

int afhip_synchronize(void* stream) {
  if (int s = require_open()) return s;
  AFHIP_CHECK_HIP(hipStreamSynchronize((hipStream_t)stream));
  return AFHIP_OK;
}

int afhip_timing_enable(int enable) {
  std::lock_guard<std::mutex> lock(g_mutex);
  g_timing = enable != 0;
  return AFHIP_OK;
}

int afhip_timing_reset(void) {
  std::lock_guard<std::mutex> lock(g_timing_mutex);
  timing_drain();
  g_totals.clear();
  return AFHIP_OK;
}

int afhip_timing_report(char* json, size_t capacity) {
  std::lock_guard<std::mutex> lock(g_timing_mutex);
  AFHIP_REQUIRE(json != nullptr && capacity > 0, "report buffer is empty");
  timing_drain();
  std::string out = "{";
  bool first = true;
  for (auto& kv : g_totals) {
    char entry[256];
    snprintf(entry, sizeof(entry), "%s\"%s\":{\"count\":%ld,\"total_ms\":%.6f}", first ? "" : ",", kv.first.c_str(),
             kv.second.first, kv.second.second);
    out += entry;
    first = false;
  }
  out += "}";
  AFHIP_REQUIRE(out.size() < capacity, "report buffer of %zu bytes is too small", capacity);
  std::memcpy(json, out.c_str(), out.size() + 1);
  return AFHIP_OK;
}

}  // extern "C"
