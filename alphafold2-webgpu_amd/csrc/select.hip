// GEMM variant selection: the heuristic, per-device calibration and the
// persisted answer (src/runtime/gemm-selection.ts, calibration-store.ts).
//
// A variant is a tile shape for a precision the caller already chose. Every
// tile walks K in the same 32-deep steps, so all variants of a precision give
// bit-identical results and only speed separates them; the correctness check
// still runs first, against a plain f32 loop on the device, so a candidate
// that computes nothing cannot win (gemm-selection.ts:584-586). Candidates
// are timed round-robin, best of the repeats (:513-520), and a tie keeps the
// smaller tile (:592-595).
#include <algorithm>
#include <cmath>
#include <cstring>
#include <fstream>
#include <map>
#include <mutex>
#include <sstream>
#include <string>
#include <tuple>
#include <vector>

#include "gemm.h"

namespace afhip {

std::string shape_class(const GemmTypes& t, int64_t M, int64_t N, int64_t K, int batch);
void install_calibrated(const std::string& key, const afhip_variant& v);
std::map<std::string, afhip_variant> calibrated_snapshot();
void replace_calibrated(const std::map<std::string, afhip_variant>& m);
bool valid_variant(const afhip_variant& v);
void pin_variant(const afhip_variant* v);

// What identifies a device well enough to reuse an answer measured on it
// (calibrationKey, calibration-store.ts:104-117): name, arch, CU count and
// driver version, so a driver update measures again. Cached per device.
std::string device_key() {
  static std::mutex mutex;
  static std::map<int, std::string> cache;
  int dev = 0;
  (void)hipGetDevice(&dev);
  std::lock_guard<std::mutex> lock(mutex);
  auto it = cache.find(dev);
  if (it != cache.end()) return it->second;
  hipDeviceProp_t p;
  if (hipGetDeviceProperties(&p, dev) != hipSuccess) return "unknown";
  int driver = 0;
  (void)hipDriverGetVersion(&driver);
  char key[512];
  snprintf(key, sizeof(key), "v1|%s|%s|cu%d|drv%d", p.name, p.gcnArchName, p.multiProcessorCount, driver);
  cache[dev] = key;
  return key;
}

namespace {

constexpr double kCheckTolerance = 0.02;  // gemm-selection.ts:81-84
constexpr int kRepeats = 2;               // PROBE_REPEATS
constexpr double kBatchMs = 12.0;         // PROBE_BATCH_MILLISECONDS
constexpr int kMaxLaunches = 2000;        // PROBE_MAX_DISPATCHES
constexpr int kSchema = 1;


// Deterministic values in [-0.5, 0.5) (f32, f16) or [-127, 127] (int8).
template <typename T> __global__ void fill_kernel(T* p, int64_t n, uint32_t seed) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  uint32_t x = (uint32_t)i * 2654435761u ^ seed;
  x ^= x >> 13;
  x *= 0x5bd1e995u;
  x ^= x >> 15;
  if constexpr (sizeof(T) == 1) p[i] = (T)((int)(x % 255u) - 127);
  else p[i] = (T)((float)(x & 0xffffu) / 65536.0f - 0.5f);
}

// The plain loop the candidates are checked against: one lane per output of
// the sampled rows, f32 accumulation over A[b][m][k] * W[b][n][k]; sample r
// is row rows[r] of batch batches[r].
template <typename TA, typename TB>
__global__ void naive_kernel(const TA* a, const TB* b, float* c, const int* batches, const int* rows, int samples,
                             int M, int N, int K) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)samples * N) return;
  const int r = (int)(i / N), n = (int)(i % N);
  const int64_t bb = batches[r], m = rows[r];
  float s = 0.0f;
  for (int k = 0; k < K; k++)
    s += (float)a[(bb * M + m) * K + k] * (float)b[(bb * N + n) * K + k];
  c[i] = s;
}

template <typename T> int fill(void* p, int64_t n, uint32_t seed, hipStream_t s) {
  return launch("calibrate.fill", fill_kernel<T>, dim3((unsigned)ceil_div(n, 256)), dim3(256), 0, s, (T*)p, n, seed);
}

int fill_dtype(int dtype, void* p, int64_t n, uint32_t seed, hipStream_t s) {
  if (dtype == AFHIP_F32) return fill<float>(p, n, seed, s);
  if (dtype == AFHIP_F16) return fill<half_t>(p, n, seed, s);
  return fill<int8_t>(p, n, seed, s);
}

int naive(int ad, int bd, const void* a, const void* b, float* c, const int* batches, const int* rows, int samples,
          int M, int N, int K, hipStream_t s) {
  dim3 grid((unsigned)ceil_div((int64_t)samples * N, 256));
#define AFHIP_NAIVE(TA, TB)                                                                                        \
  return launch("calibrate.check", naive_kernel<TA, TB>, grid, dim3(256), 0, s, (const TA*)a, (const TB*)b, c,      \
                batches, rows, samples, M, N, K)
  if (ad == AFHIP_F32 && bd == AFHIP_F32) AFHIP_NAIVE(float, float);
  if (ad == AFHIP_F32 && bd == AFHIP_F16) AFHIP_NAIVE(float, half_t);
  if (ad == AFHIP_F32) AFHIP_NAIVE(float, int8_t);
  if (bd == AFHIP_F16) AFHIP_NAIVE(half_t, half_t);
  AFHIP_NAIVE(half_t, int8_t);
#undef AFHIP_NAIVE
}

// Faults a test forces on chosen candidates from the host
// (afhip_calibration_inject): the calibration's own failure handling is what
// is under test, so no kernel is made to fail.
std::mutex g_fault_mutex;
std::map<std::tuple<int, int, int>, int> g_faults;

int fault_of(const afhip_variant& v) {
  std::lock_guard<std::mutex> lock(g_fault_mutex);
  auto it = g_faults.find(std::make_tuple(v.kernel, v.tile_rows, v.tile_columns));
  return it == g_faults.end() ? AFHIP_CALIBRATION_FAULT_NONE : it->second;
}

struct DeviceBuffer {
  void* p = nullptr;
  ~DeviceBuffer() {
    if (p) (void)hipFree(p);
  }
  int alloc(size_t bytes) {
    hipError_t e = hipMalloc(&p, bytes < 256 ? 256 : bytes);
    return e == hipSuccess ? AFHIP_OK : hip_status(e, "hipMalloc (calibration)");
  }
};

struct Events {
  hipEvent_t a = nullptr, b = nullptr;
  ~Events() {
    if (a) (void)hipEventDestroy(a);
    if (b) (void)hipEventDestroy(b);
  }
};

// The candidate set for a shape class (gemmVariantCandidates,
// gemm-selection.ts:234-272): every register-staged tile, plus the LDS_DMA
// tiles where its operand contract holds.
std::vector<afhip_variant> candidates(int precision, bool dma, bool stream) {
  std::vector<afhip_variant> out;
  auto add = [&](int kernel, int rows, int cols) {
    afhip_variant v{};
    v.precision = precision;
    v.tile_rows = rows;
    v.tile_columns = cols;
    v.tile_inner = 32;
    v.vectorized = 1;
    v.source = 1;
    v.kernel = kernel;
    out.push_back(v);
  };
  const int shapes[4][2] = {{64, 64}, {64, 128}, {128, 64}, {128, 128}};
  for (auto& s : shapes) add(AFHIP_KERNEL_REGISTER_STAGED, s[0], s[1]);
  if (dma) {
    const int dshapes[4][2] = {{128, 128}, {192, 192}, {128, 256}, {256, 256}};
    for (auto& s : dshapes) add(AFHIP_KERNEL_LDS_DMA, s[0], s[1]);
  }
  if (stream) add(AFHIP_KERNEL_STREAM, 64, 512);
  return out;
}

// A minimal reader of the document afhip_calibration_save writes:
// {"schema": 1, "entries": {"<key>": {"precision": p, "tile_rows": r, ...}, ...}}.
bool read_int(const std::string& obj, const char* field, int& out) {
  std::string needle = std::string("\"") + field + "\"";
  size_t at = obj.find(needle);
  if (at == std::string::npos) return false;
  at = obj.find(':', at + needle.size());
  if (at == std::string::npos) return false;
  char* end = nullptr;
  long v = strtol(obj.c_str() + at + 1, &end, 10);
  if (end == obj.c_str() + at + 1) return false;
  out = (int)v;
  return true;
}

}  // namespace

}  // namespace afhip

using namespace afhip;

extern "C" {

int afhip_gemm_select(const afhip_gemm_desc* d, afhip_variant* out) {
  AFHIP_REQUIRE(d && out, "NULL descriptor or output");
  AFHIP_REQUIRE(d->rows > 0 && d->inner > 0 && d->columns > 0 && d->batch > 0, "GEMM dimensions must be positive");
  AFHIP_REQUIRE(valid_precision(d->precision), "unknown precision %d", d->precision);
  GemmTypes t{d->precision, d->a_dtype, d->w_dtype, d->out_dtype};
  *out = select_plan_variant(*d, t);
  return AFHIP_OK;
}

int afhip_gemm_force_variant(const afhip_variant* v) {
  if (v != nullptr) AFHIP_REQUIRE(valid_variant(*v), "not a variant this build runs");
  pin_variant(v);
  return AFHIP_OK;
}

int afhip_gemm_calibrate(const afhip_gemm_desc* d, afhip_variant* out) {
  if (int s = require_open()) return s;
  AFHIP_REQUIRE(d && out, "NULL descriptor or output");
  AFHIP_REQUIRE(d->rows > 0 && d->inner > 0 && d->columns > 0 && d->batch > 0, "GEMM dimensions must be positive");
  AFHIP_REQUIRE(valid_precision(d->precision), "unknown precision %d", d->precision);
  GemmTypes t{d->precision, d->a_dtype, d->w_dtype, d->out_dtype};
  if (t.precision == AFHIP_PRECISION_F16 && t.b_dtype == AFHIP_F32) t.b_dtype = AFHIP_F16;
  if (t.precision == AFHIP_PRECISION_F32) t.a_dtype = t.b_dtype = AFHIP_F32;
  AFHIP_REQUIRE(!(t.precision == AFHIP_PRECISION_F32 && d->w_dtype == AFHIP_I8), "int8 weights need f16 precision");
  const int M = d->rows, N = d->columns, K = d->inner, B = d->batch;
  const size_t ea = dtype_size(t.a_dtype), eb = dtype_size(t.b_dtype), ec = dtype_size(t.c_dtype);
  hipStream_t st = nullptr;
  DeviceBuffer a, b, c, ref;
  if (int s = a.alloc(ea * (size_t)M * K * B)) return s;
  if (int s = b.alloc(eb * (size_t)N * K * B)) return s;
  if (int s = c.alloc(ec * (size_t)M * N * B)) return s;
  if (int s = fill_dtype(t.a_dtype, a.p, (int64_t)M * K * B, 0x1234567u, st)) return s;
  if (int s = fill_dtype(t.b_dtype, b.p, (int64_t)N * K * B, 0x89abcdefu, st)) return s;

  GemmArgs g;
  g.a = a.p;
  g.b = b.p;
  g.c = c.p;
  g.M = M;
  g.N = N;
  g.K = K;
  g.lda = K;
  g.ldb = K;
  g.ldc = N;
  g.sa = (int64_t)M * K;
  g.sb = (int64_t)N * K;
  g.sc = (int64_t)M * N;
  g.batch = B;

  // Correctness first, on sampled rows spread over every batch (the first
  // and last rows of each batch among them), so a candidate that is wrong
  // only on later batches or rows cannot win: 256 rows, or one row of every
  // batch when there are more batches than that.
  const int samples = (int)std::min<int64_t>((int64_t)M * B, std::max<int64_t>(256, B));
  std::vector<int> sb(samples), sm(samples);
  for (int r = 0; r < samples; r++) {
    sb[r] = r % B;
    const int k = r / B, per = (samples + B - 1) / B;
    sm[r] = per <= 1 ? 0 : (int)((int64_t)k * (M - 1) / (per - 1));
  }
  DeviceBuffer rows_b, rows_m;
  if (int s = ref.alloc(4 * (size_t)samples * N)) return s;
  if (int s = rows_b.alloc(4 * (size_t)samples)) return s;
  if (int s = rows_m.alloc(4 * (size_t)samples)) return s;
  AFHIP_CHECK_HIP(hipMemcpy(rows_b.p, sb.data(), 4 * (size_t)samples, hipMemcpyHostToDevice));
  AFHIP_CHECK_HIP(hipMemcpy(rows_m.p, sm.data(), 4 * (size_t)samples, hipMemcpyHostToDevice));
  if (int s = naive(t.a_dtype, t.b_dtype, a.p, b.p, (float*)ref.p, (const int*)rows_b.p, (const int*)rows_m.p,
                    samples, M, N, K, st))
    return s;
  std::vector<float> expect((size_t)samples * N);
  AFHIP_CHECK_HIP(hipMemcpy(expect.data(), ref.p, 4 * expect.size(), hipMemcpyDeviceToHost));
  double scale = 0.0;
  for (float v : expect) scale = std::max(scale, (double)std::fabs(v));

  std::vector<afhip_variant> cands = candidates(t.precision, dma_eligible(g, t), stream_eligible(g, t));
  std::vector<afhip_variant> usable;
  std::vector<char> host((size_t)B * M * N * ec);
  for (auto& v : cands) {
    const int fault = fault_of(v);
    // A candidate that does not run is dropped, not allowed to end the
    // calibration (gemm-selection.ts:482-495).
    if (fault == AFHIP_CALIBRATION_FAULT_RUN) continue;
    if (run_gemm(g, t, v, "calibrate.candidate", st) != AFHIP_OK) continue;
    if (hipMemcpy(host.data(), c.p, host.size(), hipMemcpyDeviceToHost) != hipSuccess) continue;
    double worst = 0.0;
    for (int r = 0; r < samples; r++)
      for (int n = 0; n < N; n++) {
        const size_t at = ((size_t)sb[r] * M + sm[r]) * N + n;
        double got = t.c_dtype == AFHIP_F32 ? (double)reinterpret_cast<float*>(host.data())[at]
                                            : (double)(float)reinterpret_cast<_Float16*>(host.data())[at];
        if (fault == AFHIP_CALIBRATION_FAULT_RESULT || (fault == AFHIP_CALIBRATION_FAULT_LAST_BATCH && sb[r] == B - 1))
          got += 0.05 * scale;
        worst = std::max(worst, std::fabs(got - (double)expect[(size_t)r * N + n]));
      }
    double rel = scale == 0.0 ? INFINITY : worst / scale;
    if (rel <= kCheckTolerance) usable.push_back(v);  // :584-586
  }
  if (usable.empty()) {
    // Nothing reproduced the reference: the probe, not the arithmetic, is
    // suspect, so nothing is installed and the heuristic stays
    // (gemm-selection.ts:590-593, :653-656).
    *out = heuristic_variant(t, M, N, K, B);
    return AFHIP_OK;
  }

  Events ev;
  AFHIP_CHECK_HIP(hipEventCreate(&ev.a));
  AFHIP_CHECK_HIP(hipEventCreate(&ev.b));
  auto time_batch = [&](const afhip_variant& v, int launches, double& ms) -> int {
    AFHIP_CHECK_HIP(hipEventRecord(ev.a, st));
    for (int i = 0; i < launches; i++)
      if (int s = run_gemm(g, t, v, "calibrate.candidate", st)) return s;
    AFHIP_CHECK_HIP(hipEventRecord(ev.b, st));
    AFHIP_CHECK_HIP(hipEventSynchronize(ev.b));
    float f = 0.0f;
    AFHIP_CHECK_HIP(hipEventElapsedTime(&f, ev.a, ev.b));
    ms = f / launches;
    return AFHIP_OK;
  };
  std::vector<int> launches(usable.size(), 4);
  std::vector<double> best(usable.size(), INFINITY);
  for (size_t i = 0; i < usable.size(); i++) {  // rough pass sizes each batch
    double ms = 0;
    if (int s = time_batch(usable[i], 4, ms)) return s;
    launches[i] = (int)std::max(4.0, std::min((double)kMaxLaunches, std::ceil(kBatchMs / std::max(ms, 0.001))));
  }
  for (int r = 0; r < kRepeats; r++)
    for (size_t i = 0; i < usable.size(); i++) {
      double ms = 0;
      if (int s = time_batch(usable[i], launches[i], ms)) return s;
      best[i] = std::min(best[i], ms);
    }
  size_t win = 0;
  for (size_t i = 1; i < usable.size(); i++) {
    const double area_i = (double)usable[i].tile_rows * usable[i].tile_columns;
    const double area_w = (double)usable[win].tile_rows * usable[win].tile_columns;
    if (best[i] < best[win] || (best[i] == best[win] && area_i < area_w)) win = i;
  }
  afhip_variant v = usable[win];
  v.source = 1;
  install_calibrated(device_key() + "|" + shape_class(t, M, N, K, B), v);
  *out = v;
  return AFHIP_OK;
}

int afhip_calibration_inject(int32_t kernel, int32_t tile_rows, int32_t tile_columns, int32_t fault) {
  std::lock_guard<std::mutex> lock(g_fault_mutex);
  if (fault == AFHIP_CALIBRATION_FAULT_NONE && kernel < 0) {
    g_faults.clear();
    return AFHIP_OK;
  }
  AFHIP_REQUIRE(fault >= AFHIP_CALIBRATION_FAULT_NONE && fault <= AFHIP_CALIBRATION_FAULT_LAST_BATCH,
                "unknown calibration fault %d", fault);
  const auto key = std::make_tuple((int)kernel, (int)tile_rows, (int)tile_columns);
  if (fault == AFHIP_CALIBRATION_FAULT_NONE) g_faults.erase(key);
  else g_faults[key] = fault;
  return AFHIP_OK;
}

int afhip_calibration_clear(void) {
  replace_calibrated({});
  return AFHIP_OK;
}

int afhip_calibration_save(const char* path) {
  AFHIP_REQUIRE(path != nullptr, "path is NULL");
  auto m = calibrated_snapshot();
  std::ofstream f(path);
  if (!f) return set_error(AFHIP_ERR_INVALID_ARGUMENT, "cannot write %s", path);
  f << "{\"schema\": " << kSchema << ", \"entries\": {";
  bool first = true;
  for (auto& kv : m) {
    f << (first ? "\n  " : ",\n  ") << "\"" << kv.first << "\": {\"precision\": " << kv.second.precision
      << ", \"tile_rows\": " << kv.second.tile_rows << ", \"tile_columns\": " << kv.second.tile_columns
      << ", \"tile_inner\": " << kv.second.tile_inner << ", \"kernel\": " << kv.second.kernel << "}";
    first = false;
  }
  f << "\n}}\n";
  return AFHIP_OK;
}

int afhip_calibration_load(const char* path) {
  AFHIP_REQUIRE(path != nullptr, "path is NULL");
  std::ifstream f(path);
  if (!f) return set_error(AFHIP_ERR_INVALID_ARGUMENT, "cannot read %s", path);
  std::stringstream ss;
  ss << f.rdbuf();
  const std::string doc = ss.str();
  int schema = -1;
  if (!read_int(doc, "schema", schema) || schema != kSchema) return AFHIP_OK;  // not ours: measure again
  std::map<std::string, afhip_variant> m = calibrated_snapshot();
  size_t at = doc.find("\"entries\"");
  if (at == std::string::npos) return AFHIP_OK;
  at = doc.find('{', at);
  while (at != std::string::npos) {
    size_t k0 = doc.find('"', at + 1);
    if (k0 == std::string::npos) break;
    size_t k1 = doc.find('"', k0 + 1);
    size_t o0 = doc.find('{', k1);
    size_t o1 = doc.find('}', o0);
    if (k1 == std::string::npos || o0 == std::string::npos || o1 == std::string::npos) break;
    std::string key = doc.substr(k0 + 1, k1 - k0 - 1);
    std::string obj = doc.substr(o0, o1 - o0 + 1);
    afhip_variant v{};
    v.vectorized = 1;
    v.source = 1;
    // A remembered answer is validated, not trusted (gemm-selection.ts:543-558).
    if (!read_int(obj, "kernel", v.kernel)) v.kernel = AFHIP_KERNEL_REGISTER_STAGED;
    if (read_int(obj, "precision", v.precision) && read_int(obj, "tile_rows", v.tile_rows) &&
        read_int(obj, "tile_columns", v.tile_columns) && read_int(obj, "tile_inner", v.tile_inner) &&
        valid_variant(v))
      m[key] = v;
    at = o1;
    size_t next = doc.find(',', at);
    if (next == std::string::npos) break;
    at = next;
  }
  replace_calibrated(m);
  return AFHIP_OK;
}

}  // extern "C"
