// afhip.node: a thin Node-API addon over libafhip's C ABI (include/afhip.h),
// the HIP counterpart of the reference's native/wgpu-backend addon.
//
// Conventions, as the wgpu addon keeps them (native/wgpu-backend/src/lib.rs,
// device.rs):
//  - device memory is referred to by u32 handles from a registry owned by the
//    addon (lib.rs:24-730 hands out u32 handles for every wgpu object);
//    explicit destroy calls free them (lib.rs:706-730);
//  - host data crosses as TypedArrays, copied in and out;
//  - every call is synchronous on the JS thread except the operator runs,
//    which return Promises and do their device work on a libuv worker
//    thread (the reference's run() is async, src/triangle/webgpu.ts:56);
//  - failures become JS exceptions: RangeError for invalid arguments (the
//    reference's RangeError, src/triangle/types.ts:42-52), Error otherwise,
//    with libafhip's message.
// The operator entry points (triangleRun, opmRun, transitionRun,
// attentionRun) upload, run and read back in one job, as
// TriangleMultiplicationGpu.run does (src/triangle/webgpu.ts:56-201), and
// report the elapsed wall time from the first upload through the readback,
// as that method does (:189-196).
#include <node_api.h>

#include <chrono>
#include <climits>
#include <cstdint>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/afhip.h"

namespace {

// ---------------------------------------------------------------------------
// Error plumbing
// ---------------------------------------------------------------------------

struct JsError {
  bool range;
  std::string message;
};

void throw_js(napi_env env, const JsError& e) {
  if (e.range) napi_throw_range_error(env, nullptr, e.message.c_str());
  else napi_throw_error(env, nullptr, e.message.c_str());
}

// Status of a libafhip call -> exception (returns false when thrown).
bool check(napi_env env, int status, const char* what) {
  if (status == AFHIP_OK) return true;
  std::string msg = std::string(what) + ": " + afhip_last_error();
  throw_js(env, {status == AFHIP_ERR_INVALID_ARGUMENT, msg});
  return false;
}

#define NAPI_OK(expr)                                          \
  do {                                                         \
    if ((expr) != napi_ok) {                                   \
      napi_throw_error(env, nullptr, "Node-API call failed: " #expr); \
      return nullptr;                                          \
    }                                                          \
  } while (0)

struct Args {
  size_t argc = 8;
  napi_value argv[8];
  napi_value self;
};

bool get_args(napi_env env, napi_callback_info info, Args& a, size_t need) {
  if (napi_get_cb_info(env, info, &a.argc, a.argv, &a.self, nullptr) != napi_ok) return false;
  if (a.argc < need) {
    napi_throw_type_error(env, nullptr, "too few arguments");
    return false;
  }
  return true;
}

bool get_int64(napi_env env, napi_value v, int64_t* out) {
  napi_valuetype t;
  if (napi_typeof(env, v, &t) != napi_ok) return false;
  if (t == napi_bigint) {
    bool lossless;
    return napi_get_value_bigint_int64(env, v, out, &lossless) == napi_ok;
  }
  double d;
  if (t != napi_number || napi_get_value_double(env, v, &d) != napi_ok) {
    napi_throw_type_error(env, nullptr, "expected a number");
    return false;
  }
  *out = (int64_t)d;
  return true;
}

bool get_string(napi_env env, napi_value v, std::string* out) {
  size_t len = 0;
  if (napi_get_value_string_utf8(env, v, nullptr, 0, &len) != napi_ok) {
    napi_throw_type_error(env, nullptr, "expected a string");
    return false;
  }
  std::vector<char> buf(len + 1);
  napi_get_value_string_utf8(env, v, buf.data(), buf.size(), &len);
  out->assign(buf.data(), len);
  return true;
}

// Integer-valued property of a descriptor object (missing -> fallback).
bool prop_int(napi_env env, napi_value obj, const char* name, int64_t fallback, int64_t* out) {
  bool has = false;
  napi_has_named_property(env, obj, name, &has);
  if (!has) {
    *out = fallback;
    return true;
  }
  napi_value v;
  napi_get_named_property(env, obj, name, &v);
  napi_valuetype t;
  napi_typeof(env, v, &t);
  if (t == napi_undefined) {
    *out = fallback;
    return true;
  }
  return get_int64(env, v, out);
}

bool prop_double(napi_env env, napi_value obj, const char* name, double fallback, double* out) {
  bool has = false;
  napi_has_named_property(env, obj, name, &has);
  if (!has) {
    *out = fallback;
    return true;
  }
  napi_value v;
  napi_get_named_property(env, obj, name, &v);
  napi_valuetype t;
  napi_typeof(env, v, &t);
  if (t == napi_undefined) {
    *out = fallback;
    return true;
  }
  if (napi_get_value_double(env, v, out) != napi_ok) {
    napi_throw_type_error(env, nullptr, "expected a number");
    return false;
  }
  return true;
}

struct HostView {
  void* data = nullptr;
  size_t bytes = 0;
  napi_typedarray_type type = napi_uint8_array;
};

bool get_view(napi_env env, napi_value v, HostView* out) {
  bool is_typed = false;
  napi_is_typedarray(env, v, &is_typed);
  if (!is_typed) {
    napi_throw_type_error(env, nullptr, "expected a TypedArray");
    return false;
  }
  size_t length = 0, offset = 0;
  napi_value ab;
  if (napi_get_typedarray_info(env, v, &out->type, &length, &out->data, &ab, &offset) != napi_ok) return false;
  size_t es = 1;
  switch (out->type) {
    case napi_int16_array: case napi_uint16_array: es = 2; break;
    case napi_int32_array: case napi_uint32_array: case napi_float32_array: es = 4; break;
    case napi_float64_array: case napi_bigint64_array: case napi_biguint64_array: es = 8; break;
    default: es = 1;
  }
  out->bytes = length * es;
  return true;
}

napi_value make_float32(napi_env env, const std::vector<float>& v) {
  napi_value ab, arr;
  void* data = nullptr;
  if (napi_create_arraybuffer(env, v.size() * 4, &data, &ab) != napi_ok) return nullptr;
  if (!v.empty()) std::memcpy(data, v.data(), v.size() * 4);
  if (napi_create_typedarray(env, napi_float32_array, v.size(), ab, 0, &arr) != napi_ok) return nullptr;
  return arr;
}

size_t dtype_bytes(int64_t d) { return d == AFHIP_F16 ? 2 : d == AFHIP_I8 ? 1 : 4; }

napi_value make_number(napi_env env, double d) {
  napi_value v;
  napi_create_double(env, d, &v);
  return v;
}

// ---------------------------------------------------------------------------
// Device-memory registry (u32 handles), the wgpu addon's Registry
// (native/wgpu-backend/src/device.rs:60-95) for HIP buffers and plans.
// ---------------------------------------------------------------------------

struct ExecutionEntry {
  afhip_execution* ex = nullptr;
  // (allocation index in the execution, buffer handle) of each tensor this
  // addon handed out, so release_since can retire the handles it frees.
  std::vector<std::pair<uint64_t, uint32_t>> handles;
  // Operator runs queued on this execution whose completion has not run yet
  // (counted on the JS thread only). A destroy requested while some are
  // pending marks the entry released: no new work may name it, and the last
  // completion frees it, since its worker may still be using the memory.
  int pending = 0;
  bool released = false;
};

struct Registry {
  uint32_t next = 1;
  std::map<uint32_t, std::pair<void*, size_t>> buffers;
  std::map<uint32_t, afhip_gemm_plan*> plans;
  std::map<uint32_t, afhip_gemm_desc> plan_descs;  // what each plan's operands must hold
  std::map<uint32_t, std::string> prepared;        // buffer handle -> weight kind it was prepared as
  std::map<uint32_t, ExecutionEntry> executions;
  std::map<uint32_t, uint32_t> owner;  // buffer handle -> execution handle, for pooled tensors
};
Registry g_reg;

// RAII device allocation for the operator entry points.
struct DeviceBuf {
  void* p = nullptr;
  ~DeviceBuf() {
    if (p) afhip_buffer_destroy(p);
  }
  int alloc(size_t bytes) { return afhip_buffer_create(bytes ? bytes : 1, &p); }
};

double now_ms() {
  using namespace std::chrono;
  return duration<double, std::milli>(steady_clock::now().time_since_epoch()).count();
}

// ---------------------------------------------------------------------------
// Context
// ---------------------------------------------------------------------------

int g_ordinal = 0;  // the device Open selected; each worker thread selects it too
// Set by Close while operator runs are still queued: the context is closed by
// the last of their completions instead (a worker re-selects the device and
// uses the execution's memory until its job ends).
bool g_close_deferred = false;

napi_value Open(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 0)) return nullptr;
  int64_t ordinal = 0;
  if (a.argc > 0 && !get_int64(env, a.argv[0], &ordinal)) return nullptr;
  if (!check(env, afhip_open((int)ordinal), "open")) return nullptr;
  g_ordinal = (int)ordinal;
  g_close_deferred = false;  // opened again before the pending runs ended: stay open
  return nullptr;
}

bool runs_pending() {
  for (auto& kv : g_reg.executions)
    if (kv.second.pending > 0) return true;
  return false;
}

napi_value Close(napi_env env, napi_callback_info) {
  for (auto& kv : g_reg.buffers)
    if (!g_reg.owner.count(kv.first)) afhip_buffer_destroy(kv.second.first);
  for (auto it = g_reg.executions.begin(); it != g_reg.executions.end();) {
    if (it->second.pending > 0) {
      it->second.released = true;
      ++it;
    } else {
      afhip_execution_destroy(it->second.ex);
      it = g_reg.executions.erase(it);
    }
  }
  for (auto& kv : g_reg.plans) afhip_gemm_plan_destroy(kv.second);
  g_reg.buffers.clear();
  g_reg.plans.clear();
  g_reg.owner.clear();
  g_reg.prepared.clear();
  if (runs_pending()) {
    g_close_deferred = true;
    return nullptr;
  }
  if (!check(env, afhip_close(), "close")) return nullptr;
  return nullptr;
}

napi_value AbiVersion(napi_env env, napi_callback_info) { return make_number(env, afhip_abi_version()); }

napi_value DeviceReport(napi_env env, napi_callback_info) {
  std::vector<char> buf(4096);
  if (!check(env, afhip_device_report(buf.data(), buf.size()), "deviceReport")) return nullptr;
  napi_value s;
  NAPI_OK(napi_create_string_utf8(env, buf.data(), NAPI_AUTO_LENGTH, &s));
  return s;
}

// ---------------------------------------------------------------------------
// Buffers
// ---------------------------------------------------------------------------

napi_value BufferCreate(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 1)) return nullptr;
  int64_t bytes;
  if (!get_int64(env, a.argv[0], &bytes)) return nullptr;
  if (bytes <= 0) {
    throw_js(env, {true, "buffer size must be positive"});
    return nullptr;
  }
  void* p = nullptr;
  if (!check(env, afhip_buffer_create((size_t)bytes, &p), "bufferCreate")) return nullptr;
  const uint32_t h = g_reg.next++;
  g_reg.buffers[h] = {p, (size_t)bytes};
  return make_number(env, h);
}

bool lookup_buffer(napi_env env, napi_value v, void** p, size_t* bytes) {
  int64_t h;
  if (!get_int64(env, v, &h)) return false;
  auto it = g_reg.buffers.find((uint32_t)h);
  if (it == g_reg.buffers.end()) {
    throw_js(env, {true, "unknown buffer handle " + std::to_string(h)});
    return false;
  }
  *p = it->second.first;
  if (bytes) *bytes = it->second.second;
  return true;
}

napi_value BufferDestroy(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 1)) return nullptr;
  int64_t h;
  if (!get_int64(env, a.argv[0], &h)) return nullptr;
  auto it = g_reg.buffers.find((uint32_t)h);
  if (it == g_reg.buffers.end()) return nullptr;
  if (g_reg.owner.count((uint32_t)h)) {
    throw_js(env, {true, "the buffer belongs to an execution; release it there"});
    return nullptr;
  }
  afhip_buffer_destroy(it->second.first);
  g_reg.buffers.erase(it);
  return nullptr;
}

napi_value BufferWrite(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 3)) return nullptr;
  void* p;
  size_t cap;
  int64_t offset;
  HostView src;
  if (!lookup_buffer(env, a.argv[0], &p, &cap) || !get_int64(env, a.argv[1], &offset) || !get_view(env, a.argv[2], &src))
    return nullptr;
  if (offset < 0 || (size_t)offset + src.bytes > cap) {
    throw_js(env, {true, "write past the end of the buffer"});
    return nullptr;
  }
  if (!check(env, afhip_buffer_write(p, (size_t)offset, src.data, src.bytes), "bufferWrite")) return nullptr;
  return nullptr;
}

napi_value BufferRead(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 3)) return nullptr;
  void* p;
  size_t cap;
  int64_t offset;
  HostView dst;
  if (!lookup_buffer(env, a.argv[0], &p, &cap) || !get_int64(env, a.argv[1], &offset) || !get_view(env, a.argv[2], &dst))
    return nullptr;
  if (offset < 0 || (size_t)offset + dst.bytes > cap) {
    throw_js(env, {true, "read past the end of the buffer"});
    return nullptr;
  }
  if (!check(env, afhip_buffer_read(p, (size_t)offset, dst.data, dst.bytes), "bufferRead")) return nullptr;
  return nullptr;
}

napi_value Synchronize(napi_env env, napi_callback_info) {
  if (!check(env, afhip_synchronize(nullptr), "synchronize")) return nullptr;
  return nullptr;
}

// ---------------------------------------------------------------------------
// GEMM plan surface
// ---------------------------------------------------------------------------

bool read_gemm_desc(napi_env env, napi_value o, afhip_gemm_desc* d) {
  std::memset(d, 0, sizeof(*d));
  int64_t v;
#define FIELD(name, js, fallback)                                   \
  if (!prop_int(env, o, js, fallback, &v)) return false;            \
  d->name = (decltype(d->name))v;
  FIELD(rows, "rows", 0)
  FIELD(inner, "inner", 0)
  FIELD(columns, "columns", 0)
  FIELD(batch, "batch", 1)
  FIELD(precision, "precision", AFHIP_PRECISION_F32)
  FIELD(a_dtype, "aDtype", AFHIP_F32)
  FIELD(w_dtype, "wDtype", AFHIP_F32)
  FIELD(w_layout, "wLayout", AFHIP_WEIGHT_COLUMN_CONTIGUOUS)
  FIELD(out_dtype, "outDtype", AFHIP_F32)
  FIELD(epilogue, "epilogue", 0)
  FIELD(heads, "heads", 0)
  FIELD(head_dim, "headDim", 0)
  FIELD(lda, "lda", 0)
  FIELD(ldw, "ldw", 0)
  FIELD(ldc, "ldc", 0)
  FIELD(batch_stride_a, "batchStrideA", 0)
  FIELD(batch_stride_w, "batchStrideW", 0)
  FIELD(batch_stride_c, "batchStrideC", 0)
  FIELD(a_layout, "aLayout", AFHIP_SOURCE_K_CONTIGUOUS)
  FIELD(c_layout, "cLayout", AFHIP_OUTPUT_ROW_MAJOR)
#undef FIELD
  return true;
}

napi_value variant_object(napi_env env, const afhip_variant& v) {
  napi_value o;
  napi_create_object(env, &o);
  napi_set_named_property(env, o, "precision", make_number(env, v.precision));
  napi_set_named_property(env, o, "tileRows", make_number(env, v.tile_rows));
  napi_set_named_property(env, o, "tileColumns", make_number(env, v.tile_columns));
  napi_set_named_property(env, o, "tileInner", make_number(env, v.tile_inner));
  napi_set_named_property(env, o, "source", make_number(env, v.source));
  napi_set_named_property(env, o, "kernel", make_number(env, v.kernel));
  return o;
}

napi_value GemmGrid(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 2)) return nullptr;
  int64_t rows, cols, tc = 128, tr = 64;
  if (!get_int64(env, a.argv[0], &rows) || !get_int64(env, a.argv[1], &cols)) return nullptr;
  if (a.argc > 2 && !get_int64(env, a.argv[2], &tc)) return nullptr;
  if (a.argc > 3 && !get_int64(env, a.argv[3], &tr)) return nullptr;
  uint32_t xy[2];
  if (!check(env, afhip_gemm_grid(rows, cols, (int32_t)tc, (int32_t)tr, xy), "gemmGrid")) return nullptr;
  napi_value arr;
  napi_create_array_with_length(env, 2, &arr);
  napi_set_element(env, arr, 0, make_number(env, xy[0]));
  napi_set_element(env, arr, 1, make_number(env, xy[1]));
  return arr;
}

napi_value GemmSelect(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 1)) return nullptr;
  afhip_gemm_desc d;
  if (!read_gemm_desc(env, a.argv[0], &d)) return nullptr;
  afhip_variant v;
  if (!check(env, afhip_gemm_select(&d, &v), "gemmSelect")) return nullptr;
  return variant_object(env, v);
}

napi_value GemmCalibrate(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 1)) return nullptr;
  afhip_gemm_desc d;
  if (!read_gemm_desc(env, a.argv[0], &d)) return nullptr;
  afhip_variant v;
  if (!check(env, afhip_gemm_calibrate(&d, &v), "gemmCalibrate")) return nullptr;
  return variant_object(env, v);
}

napi_value GemmForceVariant(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 0)) return nullptr;
  napi_valuetype t = napi_undefined;
  if (a.argc > 0) napi_typeof(env, a.argv[0], &t);
  if (t == napi_undefined || t == napi_null) {
    if (!check(env, afhip_gemm_force_variant(nullptr), "gemmForceVariant")) return nullptr;
    return nullptr;
  }
  afhip_variant v{};
  int64_t x;
  if (!prop_int(env, a.argv[0], "precision", AFHIP_PRECISION_F16, &x)) return nullptr;
  v.precision = (int32_t)x;
  if (!prop_int(env, a.argv[0], "tileRows", 128, &x)) return nullptr;
  v.tile_rows = (int32_t)x;
  if (!prop_int(env, a.argv[0], "tileColumns", 128, &x)) return nullptr;
  v.tile_columns = (int32_t)x;
  if (!prop_int(env, a.argv[0], "tileInner", 32, &x)) return nullptr;
  v.tile_inner = (int32_t)x;
  if (!prop_int(env, a.argv[0], "kernel", AFHIP_KERNEL_REGISTER_STAGED, &x)) return nullptr;
  v.kernel = (int32_t)x;
  v.vectorized = 1;
  v.source = 2;
  if (!check(env, afhip_gemm_force_variant(&v), "gemmForceVariant")) return nullptr;
  return nullptr;
}

napi_value CalibrationLoad(napi_env env, napi_callback_info info) {
  Args a;
  std::string path;
  if (!get_args(env, info, a, 1) || !get_string(env, a.argv[0], &path)) return nullptr;
  if (!check(env, afhip_calibration_load(path.c_str()), "calibrationLoad")) return nullptr;
  return nullptr;
}

napi_value CalibrationClear(napi_env env, napi_callback_info) {
  check(env, afhip_calibration_clear(), "calibrationClear");
  return nullptr;
}

// calibrationInject(kernel, tileRows, tileColumns, fault): a fault forced on
// one calibration candidate, for tests of the calibration's failure handling.
napi_value CalibrationInject(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 4)) return nullptr;
  int64_t v[4];
  for (int i = 0; i < 4; i++)
    if (!get_int64(env, a.argv[i], &v[i])) return nullptr;
  check(env, afhip_calibration_inject((int32_t)v[0], (int32_t)v[1], (int32_t)v[2], (int32_t)v[3]),
        "calibrationInject");
  return nullptr;
}

napi_value CalibrationSave(napi_env env, napi_callback_info info) {
  Args a;
  std::string path;
  if (!get_args(env, info, a, 1) || !get_string(env, a.argv[0], &path)) return nullptr;
  if (!check(env, afhip_calibration_save(path.c_str()), "calibrationSave")) return nullptr;
  return nullptr;
}

napi_value GemmPlanCreate(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 1)) return nullptr;
  afhip_gemm_desc d;
  if (!read_gemm_desc(env, a.argv[0], &d)) return nullptr;
  afhip_gemm_plan* plan = nullptr;
  if (!check(env, afhip_gemm_plan_create(&d, &plan), "gemmPlanCreate")) return nullptr;
  const uint32_t h = g_reg.next++;
  g_reg.plans[h] = plan;
  g_reg.plan_descs[h] = d;
  return make_number(env, h);
}

napi_value GemmPlanDestroy(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 1)) return nullptr;
  int64_t h;
  if (!get_int64(env, a.argv[0], &h)) return nullptr;
  auto it = g_reg.plans.find((uint32_t)h);
  if (it != g_reg.plans.end()) {
    afhip_gemm_plan_destroy(it->second);
    g_reg.plans.erase(it);
    g_reg.plan_descs.erase((uint32_t)h);
  }
  return nullptr;
}

napi_value GemmWorkspaceSize(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 1)) return nullptr;
  int64_t h;
  if (!get_int64(env, a.argv[0], &h)) return nullptr;
  auto it = g_reg.plans.find((uint32_t)h);
  if (it == g_reg.plans.end()) {
    throw_js(env, {true, "unknown plan handle"});
    return nullptr;
  }
  size_t bytes = 0;
  if (!check(env, afhip_gemm_workspace_size(it->second, &bytes), "gemmWorkspaceSize")) return nullptr;
  return make_number(env, (double)bytes);
}

// gemmRun(plan, {a, w, scale?, bias?, residual?, c, workspace?}) with buffer handles.
napi_value GemmRun(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 2)) return nullptr;
  int64_t h;
  if (!get_int64(env, a.argv[0], &h)) return nullptr;
  auto it = g_reg.plans.find((uint32_t)h);
  if (it == g_reg.plans.end()) {
    throw_js(env, {true, "unknown plan handle"});
    return nullptr;
  }
  const char* names[7] = {"a", "w", "scale", "bias", "residual", "c", "workspace"};
  void* ptrs[7] = {};
  size_t sizes[7] = {};
  for (int i = 0; i < 7; i++) {
    bool has = false;
    napi_has_named_property(env, a.argv[1], names[i], &has);
    if (!has) continue;
    napi_value v;
    napi_get_named_property(env, a.argv[1], names[i], &v);
    napi_valuetype t;
    napi_typeof(env, v, &t);
    if (t == napi_undefined || t == napi_null) continue;
    if (!lookup_buffer(env, v, &ptrs[i], &sizes[i])) return nullptr;
  }
  // Every operand the plan reads or writes must lie inside its buffer, as
  // WebGPU validates a binding against its buffer's size.
  const afhip_gemm_desc& d = g_reg.plan_descs[(uint32_t)h];
  const int64_t M = d.rows, K = d.inner, N = d.columns, B = d.batch;
  const bool a_rows = d.a_layout == AFHIP_SOURCE_ROW_CONTIGUOUS, w_k = d.w_layout == AFHIP_WEIGHT_K_CONTIGUOUS,
             c_cols = d.c_layout == AFHIP_OUTPUT_COLUMN_MAJOR;
  const int64_t lda = d.lda ? d.lda : (a_rows ? M : K), ldw = d.ldw ? d.ldw : (w_k ? K : N),
                ldc = d.ldc ? d.ldc : (c_cols ? M : N);
  auto extent = [&](int64_t outer, int64_t ld, int64_t run, int64_t stride) {
    return (B - 1) * stride + (outer - 1) * ld + run;  // elements
  };
  const size_t need[6] = {
      (size_t)extent(a_rows ? K : M, lda, a_rows ? M : K, d.batch_stride_a) * dtype_bytes(d.a_dtype),
      (size_t)extent(w_k ? N : K, ldw, w_k ? K : N, d.batch_stride_w) * dtype_bytes(d.w_dtype),
      (d.epilogue & AFHIP_EPILOGUE_SCALE) ? (size_t)N * 4 : 0,
      (d.epilogue & AFHIP_EPILOGUE_BIAS) ? (size_t)N * 4 : 0,
      (d.epilogue & AFHIP_EPILOGUE_RESIDUAL)
          ? (size_t)extent(c_cols ? N : M, ldc, c_cols ? M : N, d.batch_stride_c) * dtype_bytes(d.out_dtype)
          : 0,
      (size_t)extent(c_cols ? N : M, ldc, c_cols ? M : N, d.batch_stride_c) * dtype_bytes(d.out_dtype)};
  for (int i = 0; i < 6; i++) {
    if (need[i] == 0) continue;
    if (ptrs[i] == nullptr) {
      throw_js(env, {true, std::string("gemmRun: the plan needs operand ") + names[i]});
      return nullptr;
    }
    if (sizes[i] < need[i]) {
      throw_js(env, {true, std::string("gemmRun: buffer ") + names[i] + " holds " + std::to_string(sizes[i]) +
                               " bytes; the plan reads or writes " + std::to_string(need[i])});
      return nullptr;
    }
  }
  if (!check(env,
             afhip_gemm_run(it->second, ptrs[0], ptrs[1], (const float*)ptrs[2], (const float*)ptrs[3], ptrs[4],
                            ptrs[5], ptrs[6], sizes[6], nullptr),
             "gemmRun"))
    return nullptr;
  return nullptr;
}

// packWeightQ8Block(codes, scales, block, start, rowsK, columnsN, dst, dtype)
// with buffer handles: the bundle's int8 codes and f16 scale bits in, the
// packed GEMM operand W[n][k] of dtype (DTYPE.f32 or DTYPE.f16) out
// (afhip_pack_weight_q8_block). The buffers' sizes bound every access.
napi_value PackWeightQ8Block(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 8)) return nullptr;
  void *codes, *scales, *dst;
  size_t codes_bytes, scales_bytes, dst_bytes;
  int64_t block, start, rows_k, columns_n, dtype;
  // The numbers first, so a block or shape that does not fit the C ABI's
  // 32-bit arguments is refused before anything is looked up or cast.
  if (!get_int64(env, a.argv[2], &block) || !get_int64(env, a.argv[3], &start) || !get_int64(env, a.argv[4], &rows_k) ||
      !get_int64(env, a.argv[5], &columns_n) || !get_int64(env, a.argv[7], &dtype))
    return nullptr;
  if (block <= 0 || block > INT32_MAX || start < 0 || rows_k <= 0 || columns_n <= 0 || rows_k > INT32_MAX ||
      columns_n > INT32_MAX || (dtype != AFHIP_F32 && dtype != AFHIP_F16)) {
    throw_js(env, {true, "packWeightQ8Block: invalid block, range, shape or dtype"});
    return nullptr;
  }
  if (!lookup_buffer(env, a.argv[0], &codes, &codes_bytes) || !lookup_buffer(env, a.argv[1], &scales, &scales_bytes) ||
      !lookup_buffer(env, a.argv[6], &dst, &dst_bytes))
    return nullptr;
  const int64_t count = rows_k * columns_n;
  if (start + count > (int64_t)codes_bytes) {
    throw_js(env, {true, "packWeightQ8Block: tensor range is out of bounds"});
    return nullptr;
  }
  if ((start + count - 1) / block >= (int64_t)(scales_bytes / 2)) {
    throw_js(env, {true, "packWeightQ8Block: int8 tensor has too few scales"});
    return nullptr;
  }
  if (count * (dtype == AFHIP_F16 ? 2 : 4) > (int64_t)dst_bytes) {
    throw_js(env, {true, "packWeightQ8Block: destination buffer is too small"});
    return nullptr;
  }
  if (!check(env,
             afhip_pack_weight_q8_block((const int8_t*)codes, (const uint16_t*)scales, (int32_t)block, start,
                                        (int32_t)rows_k, (int32_t)columns_n, dst, (int32_t)dtype, nullptr),
             "packWeightQ8Block"))
    return nullptr;
  return nullptr;
}

// ---------------------------------------------------------------------------
// Execution layer (afhip_execution_*): pooled device tensors as buffer
// handles, usable wherever a buffer handle is (gemmRun, packWeightQ8Block),
// and the pair stack chained on the device.
// ---------------------------------------------------------------------------

bool lookup_execution(napi_env env, napi_value v, uint32_t* handle, ExecutionEntry** out) {
  int64_t h;
  if (!get_int64(env, v, &h)) return false;
  auto it = g_reg.executions.find((uint32_t)h);
  if (it == g_reg.executions.end() || it->second.released) {
    throw_js(env, {true, "unknown execution handle " + std::to_string(h)});
    return false;
  }
  *handle = (uint32_t)h;
  *out = &it->second;
  return true;
}

void forget_buffer(uint32_t h) {
  g_reg.buffers.erase(h);
  g_reg.owner.erase(h);
  g_reg.prepared.erase(h);
}

// A prepared-weight handle for a chained step: it must have been prepared as
// `kind` and hold the bytes that step's prepared weights take.
bool lookup_prepared(napi_env env, napi_value v, const char* kind, size_t need, void** p) {
  size_t bytes = 0;
  if (!lookup_buffer(env, v, p, &bytes)) return false;
  int64_t h = 0;
  get_int64(env, v, &h);
  auto it = g_reg.prepared.find((uint32_t)h);
  if (it == g_reg.prepared.end() || it->second != kind) {
    throw_js(env, {true, std::string("weights for ") + kind + " must come from executionPrepareWeights(\"" + kind +
                             "\"); handle " + std::to_string(h) + " was prepared as " +
                             (it == g_reg.prepared.end() ? std::string("nothing") : "\"" + it->second + "\"")});
    return false;
  }
  if (bytes < need) {
    throw_js(env, {true, std::string("prepared weights for ") + kind + " hold " + std::to_string(bytes) +
                             " bytes; this shape needs " + std::to_string(need)});
    return false;
  }
  return true;
}

// Registers the execution's newest allocation (pointer p) as a buffer handle.
napi_value register_pooled(napi_env env, uint32_t exh, ExecutionEntry& e, void* p, size_t bytes) {
  uint64_t count = 0;
  afhip_execution_checkpoint(e.ex, &count);
  const uint32_t h = g_reg.next++;
  g_reg.buffers[h] = {p, bytes};
  g_reg.owner[h] = exh;
  e.handles.push_back({count - 1, h});
  return make_number(env, h);
}

// executionCreate(maxPooledBytes = 0) -> handle
napi_value ExecutionCreate(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 0)) return nullptr;
  int64_t cap = 0;
  if (a.argc > 0 && !get_int64(env, a.argv[0], &cap)) return nullptr;
  if (cap < 0) {
    throw_js(env, {true, "maxPooledBytes must not be negative"});
    return nullptr;
  }
  afhip_execution* ex = nullptr;
  if (!check(env, afhip_execution_create((uint64_t)cap, nullptr, &ex), "executionCreate")) return nullptr;
  const uint32_t h = g_reg.next++;
  g_reg.executions[h].ex = ex;
  return make_number(env, h);
}

napi_value ExecutionDestroy(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 1)) return nullptr;
  uint32_t exh;
  ExecutionEntry* e;
  if (!lookup_execution(env, a.argv[0], &exh, &e)) return nullptr;
  for (auto& ih : e->handles) forget_buffer(ih.second);
  e->handles.clear();
  if (e->pending > 0) {
    e->released = true;  // the last pending run's completion destroys it
    return nullptr;
  }
  afhip_execution_destroy(e->ex);
  g_reg.executions.erase(exh);
  return nullptr;
}

// executionAllocate(ex, label, bytes) -> buffer handle
napi_value ExecutionAllocate(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 3)) return nullptr;
  uint32_t exh;
  ExecutionEntry* e;
  std::string label;
  int64_t bytes;
  if (!lookup_execution(env, a.argv[0], &exh, &e) || !get_string(env, a.argv[1], &label) ||
      !get_int64(env, a.argv[2], &bytes))
    return nullptr;
  if (bytes <= 0) {
    throw_js(env, {true, "invalid allocation size " + std::to_string(bytes) + " for " + label});
    return nullptr;
  }
  void* p = nullptr;
  if (!check(env, afhip_execution_allocate(e->ex, label.c_str(), (uint64_t)bytes, &p), "executionAllocate"))
    return nullptr;
  return register_pooled(env, exh, *e, p, (size_t)bytes);
}

// executionUpload(ex, label, typedArray) -> buffer handle
napi_value ExecutionUpload(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 3)) return nullptr;
  uint32_t exh;
  ExecutionEntry* e;
  std::string label;
  HostView src;
  if (!lookup_execution(env, a.argv[0], &exh, &e) || !get_string(env, a.argv[1], &label) ||
      !get_view(env, a.argv[2], &src))
    return nullptr;
  void* p = nullptr;
  if (!check(env, afhip_execution_upload(e->ex, label.c_str(), src.data, src.bytes, &p), "executionUpload"))
    return nullptr;
  return register_pooled(env, exh, *e, p, src.bytes);
}

// executionRelease(ex, buffer)
napi_value ExecutionRelease(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 2)) return nullptr;
  uint32_t exh;
  ExecutionEntry* e;
  int64_t h;
  if (!lookup_execution(env, a.argv[0], &exh, &e) || !get_int64(env, a.argv[1], &h)) return nullptr;
  auto o = g_reg.owner.find((uint32_t)h);
  if (o == g_reg.owner.end() || o->second != exh) {
    throw_js(env, {true, "the buffer is not a tensor of this execution"});
    return nullptr;
  }
  if (!check(env, afhip_execution_release(e->ex, g_reg.buffers[(uint32_t)h].first), "executionRelease"))
    return nullptr;
  forget_buffer((uint32_t)h);
  for (auto it = e->handles.begin(); it != e->handles.end(); ++it)
    if (it->second == (uint32_t)h) {
      e->handles.erase(it);
      break;
    }
  return nullptr;
}

napi_value ExecutionCheckpoint(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 1)) return nullptr;
  uint32_t exh;
  ExecutionEntry* e;
  if (!lookup_execution(env, a.argv[0], &exh, &e)) return nullptr;
  uint64_t n = 0;
  if (!check(env, afhip_execution_checkpoint(e->ex, &n), "executionCheckpoint")) return nullptr;
  return make_number(env, (double)n);
}

napi_value ExecutionReleaseSince(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 2)) return nullptr;
  uint32_t exh;
  ExecutionEntry* e;
  int64_t mark;
  if (!lookup_execution(env, a.argv[0], &exh, &e) || !get_int64(env, a.argv[1], &mark)) return nullptr;
  if (mark < 0) {
    throw_js(env, {true, "invalid GPU allocation checkpoint " + std::to_string(mark)});
    return nullptr;
  }
  if (!check(env, afhip_execution_release_since(e->ex, (uint64_t)mark), "executionReleaseSince")) return nullptr;
  std::vector<std::pair<uint64_t, uint32_t>> kept;
  for (auto& ih : e->handles) {
    if (ih.first >= (uint64_t)mark) forget_buffer(ih.second);
    else kept.push_back(ih);
  }
  e->handles.swap(kept);
  return nullptr;
}

napi_value ExecutionNoteSubmitted(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 1)) return nullptr;
  uint32_t exh;
  ExecutionEntry* e;
  if (!lookup_execution(env, a.argv[0], &exh, &e)) return nullptr;
  check(env, afhip_execution_note_submitted(e->ex), "executionNoteSubmitted");
  return nullptr;
}

// executionSnapshot(ex) -> JSON text of the AllocationSnapshot
napi_value ExecutionSnapshot(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 1)) return nullptr;
  uint32_t exh;
  ExecutionEntry* e;
  if (!lookup_execution(env, a.argv[0], &exh, &e)) return nullptr;
  std::vector<char> buf(1 << 16);
  if (!check(env, afhip_execution_snapshot(e->ex, buf.data(), buf.size()), "executionSnapshot")) return nullptr;
  napi_value s;
  NAPI_OK(napi_create_string_utf8(env, buf.data(), NAPI_AUTO_LENGTH, &s));
  return s;
}


// executionAddInPlace(ex, base, baseDtype, update, updateDtype, elements)
napi_value ExecutionAddInPlace(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 6)) return nullptr;
  uint32_t exh;
  ExecutionEntry* e;
  void *base, *update;
  size_t nb, nu;
  int64_t bd, ud, n;
  if (!lookup_execution(env, a.argv[0], &exh, &e) || !lookup_buffer(env, a.argv[1], &base, &nb) ||
      !get_int64(env, a.argv[2], &bd) || !lookup_buffer(env, a.argv[3], &update, &nu) ||
      !get_int64(env, a.argv[4], &ud) || !get_int64(env, a.argv[5], &n))
    return nullptr;
  if (n <= 0 || (size_t)n * dtype_bytes(bd) > nb || (size_t)n * dtype_bytes(ud) > nu) {
    throw_js(env, {true, "residual tensors must hold the element count"});
    return nullptr;
  }
  check(env, afhip_execution_add_in_place(e->ex, base, (int32_t)bd, update, (int32_t)ud, n), "executionAddInPlace");
  return nullptr;
}

// The pair stack's shape from {length, sequences, cM, cZ = 128, cOuter = 32,
// cHidden = 128, transitionFactor = 4, precision = PRECISION.f16,
// pairDtype = DTYPE.f16, msaDtype = DTYPE.f16, opmRowBlock = 0,
// triangleBlockRows = 0, attentionHeads = 4}.
bool read_stack_desc(napi_env env, napi_value o, afhip_pair_stack_desc* d) {
  int64_t L, S, cm, cz, co, ch, tf, prec, pdt, mdt, rb, br, heads;
  if (!prop_int(env, o, "length", 0, &L) || !prop_int(env, o, "sequences", 0, &S) ||
      !prop_int(env, o, "cM", 0, &cm) || !prop_int(env, o, "cZ", 128, &cz) || !prop_int(env, o, "cOuter", 32, &co) ||
      !prop_int(env, o, "cHidden", 128, &ch) || !prop_int(env, o, "transitionFactor", 4, &tf) ||
      !prop_int(env, o, "precision", AFHIP_PRECISION_F16, &prec) || !prop_int(env, o, "pairDtype", AFHIP_F16, &pdt) ||
      !prop_int(env, o, "msaDtype", AFHIP_F16, &mdt) || !prop_int(env, o, "opmRowBlock", 0, &rb) ||
      !prop_int(env, o, "triangleBlockRows", 0, &br) || !prop_int(env, o, "attentionHeads", 4, &heads))
    return false;
  if (L <= 0 || L > 65535 || cz <= 0 || ch <= 0 || tf <= 0 || S < 0 || cm < 0 || co <= 0 || heads <= 0) {
    throw_js(env, {true, "pair stack dimensions must be positive"});
    return false;
  }
  std::memset(d, 0, sizeof(*d));
  d->opm = {(int32_t)S, (int32_t)L, (int32_t)cm, (int32_t)co, (int32_t)cz, (int32_t)prec, (int32_t)mdt, (int32_t)pdt,
            (int32_t)rb, 1, 1e-5f, 1e-3f};
  d->outgoing = {(int32_t)L, (int32_t)cz, (int32_t)ch, AFHIP_TRIANGLE_OUTGOING, (int32_t)prec, (int32_t)pdt,
                 (int32_t)pdt, (int32_t)br, 1, 1e-5f};
  d->incoming = d->outgoing;
  d->incoming.direction = AFHIP_TRIANGLE_INCOMING;
  d->attention_start = {(int32_t)L, (int32_t)L, (int32_t)cz, (int32_t)heads, 0, AFHIP_PAIR_BIAS_NORMALIZED_INPUT, 0,
                        (int32_t)prec, (int32_t)pdt, (int32_t)pdt, 1, 1e-5f};
  d->attention_end = d->attention_start;
  d->attention_end.transpose = 1;
  d->transition = {(int64_t)L * L, (int32_t)cz, (int32_t)(tf * cz), (int32_t)prec, (int32_t)pdt, (int32_t)pdt, 1,
                   1e-5f};
  return true;
}

// The block's shape: the pair stack's, plus msaHeads = 8,
// msaTransitionFactor = 4, opmFirst = false.
bool read_block_desc(napi_env env, napi_value o, afhip_evoformer_block_desc* d) {
  std::memset(d, 0, sizeof(*d));
  if (!read_stack_desc(env, o, &d->pair)) return false;
  int64_t mh, mf;
  bool opm_first = false;
  if (!prop_int(env, o, "msaHeads", 8, &mh) || !prop_int(env, o, "msaTransitionFactor", 4, &mf)) return false;
  bool has = false;
  napi_has_named_property(env, o, "opmFirst", &has);
  if (has) {
    napi_value v;
    napi_get_named_property(env, o, "opmFirst", &v);
    napi_get_value_bool(env, v, &opm_first);
  }
  if (mh <= 0 || mf <= 0) {
    throw_js(env, {true, "block dimensions must be positive"});
    return false;
  }
  const afhip_opm_desc& o_ = d->pair.opm;
  const int32_t S = o_.sequences, L = o_.length, cm = o_.c_m, cz = o_.c_z, prec = o_.precision,
                dt = d->pair.outgoing.pair_dtype;
  d->msa_row = {S, L, cm, (int32_t)mh, 0, AFHIP_PAIR_BIAS_SEPARATE, cz, prec, dt, dt, 1, 1e-5f};
  d->msa_column = {L, S, cm, (int32_t)mh, 1, AFHIP_PAIR_BIAS_NONE, 0, prec, dt, dt, 1, 1e-5f};
  d->msa_transition = {(int64_t)S * L, cm, (int32_t)(mf * cm), prec, dt, dt, 1, 1e-5f};
  d->opm_first = opm_first ? 1 : 0;
  return true;
}

// executionPrepareWeights(ex, kind, stackDesc, Float32Array packed) -> buffer
// handle of the prepared weights in the execution's pool; kind is
// "outerProductMean", "triangleOutgoing", "triangleIncoming",
// "triangleAttentionStarting", "triangleAttentionEnding" or "pairTransition",
// packed in that operator's reference order.
napi_value ExecutionPrepareWeights(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 4)) return nullptr;
  uint32_t exh;
  ExecutionEntry* e;
  std::string kind;
  afhip_evoformer_block_desc bd;
  HostView packed;
  if (!lookup_execution(env, a.argv[0], &exh, &e) || !get_string(env, a.argv[1], &kind) ||
      !read_block_desc(env, a.argv[2], &bd) || !get_view(env, a.argv[3], &packed))
    return nullptr;
  const afhip_pair_stack_desc& d = bd.pair;
  size_t bytes = 0;
  int st;
  if (kind == "outerProductMean") st = afhip_opm_weights_size(&d.opm, &bytes);
  else if (kind == "triangleOutgoing") st = afhip_triangle_weights_size(&d.outgoing, &bytes);
  else if (kind == "triangleIncoming") st = afhip_triangle_weights_size(&d.incoming, &bytes);
  else if (kind == "triangleAttentionStarting") st = afhip_attention_weights_size(&d.attention_start, &bytes);
  else if (kind == "triangleAttentionEnding") st = afhip_attention_weights_size(&d.attention_end, &bytes);
  else if (kind == "pairTransition") st = afhip_transition_weights_size(&d.transition, &bytes);
  else if (kind == "msaRowAttention") st = afhip_attention_weights_size(&bd.msa_row, &bytes);
  else if (kind == "msaColumnAttention") st = afhip_attention_weights_size(&bd.msa_column, &bytes);
  else if (kind == "msaTransition") st = afhip_transition_weights_size(&bd.msa_transition, &bytes);
  else {
    throw_js(env, {true, "unknown weight kind " + kind});
    return nullptr;
  }
  if (!check(env, st, "executionPrepareWeights")) return nullptr;
  void *src = nullptr, *dst = nullptr;
  const std::string label = "pair-stack." + kind;
  if (!check(env, afhip_execution_upload(e->ex, (label + ".weights-f32").c_str(), packed.data, packed.bytes, &src),
             "executionPrepareWeights"))
    return nullptr;
  if (!check(env, afhip_execution_allocate(e->ex, (label + ".weights").c_str(), bytes, &dst),
             "executionPrepareWeights")) {
    afhip_execution_release(e->ex, src);
    return nullptr;
  }
  napi_value handle = register_pooled(env, exh, *e, dst, bytes);
  {
    int64_t h = 0;
    get_int64(env, handle, &h);
    g_reg.prepared[(uint32_t)h] = kind;
  }
  const float* f = (const float*)src;
  if (kind == "outerProductMean") st = afhip_opm_prepare_weights(&d.opm, f, dst, nullptr);
  else if (kind == "triangleOutgoing") st = afhip_triangle_prepare_weights(&d.outgoing, f, dst, nullptr);
  else if (kind == "triangleIncoming") st = afhip_triangle_prepare_weights(&d.incoming, f, dst, nullptr);
  else if (kind == "triangleAttentionStarting") st = afhip_attention_prepare_weights(&d.attention_start, f, dst, nullptr);
  else if (kind == "triangleAttentionEnding") st = afhip_attention_prepare_weights(&d.attention_end, f, dst, nullptr);
  else if (kind == "msaRowAttention") st = afhip_attention_prepare_weights(&bd.msa_row, f, dst, nullptr);
  else if (kind == "msaColumnAttention") st = afhip_attention_prepare_weights(&bd.msa_column, f, dst, nullptr);
  else if (kind == "msaTransition") st = afhip_transition_prepare_weights(&bd.msa_transition, f, dst, nullptr);
  else st = afhip_transition_prepare_weights(&d.transition, f, dst, nullptr);
  if (st == AFHIP_OK) st = afhip_synchronize(nullptr);
  afhip_execution_release(e->ex, src);
  if (!check(env, st, "executionPrepareWeights")) return nullptr;
  return handle;
}

// executionPairStack(ex, stackDesc, {outerProductMean?, triangleOutgoing?,
// triangleIncoming?, triangleAttentionStarting?, triangleAttentionEnding?,
// pairTransition?}, pair, pairMask, msa?, msaMask?)
napi_value ExecutionPairStack(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 5)) return nullptr;
  uint32_t exh;
  ExecutionEntry* e;
  afhip_pair_stack_desc d;
  if (!lookup_execution(env, a.argv[0], &exh, &e) || !read_stack_desc(env, a.argv[1], &d)) return nullptr;
  const char* names[6] = {"outerProductMean", "triangleOutgoing", "triangleIncoming", "triangleAttentionStarting",
                          "triangleAttentionEnding", "pairTransition"};
  void* w[6] = {};
  size_t need[6] = {};
  afhip_opm_weights_size(&d.opm, &need[0]);
  afhip_triangle_weights_size(&d.outgoing, &need[1]);
  afhip_triangle_weights_size(&d.incoming, &need[2]);
  afhip_attention_weights_size(&d.attention_start, &need[3]);
  afhip_attention_weights_size(&d.attention_end, &need[4]);
  afhip_transition_weights_size(&d.transition, &need[5]);
  for (int i = 0; i < 6; i++) {
    bool has = false;
    napi_has_named_property(env, a.argv[2], names[i], &has);
    if (!has) continue;
    napi_value v;
    napi_get_named_property(env, a.argv[2], names[i], &v);
    napi_valuetype t;
    napi_typeof(env, v, &t);
    if (t == napi_undefined || t == napi_null) continue;
    if (!lookup_prepared(env, v, names[i], need[i], &w[i])) return nullptr;
  }
  void *pair, *pmask, *msa = nullptr, *mmask = nullptr;
  size_t np, npm, nm = 0, nmm = 0;
  if (!lookup_buffer(env, a.argv[3], &pair, &np) || !lookup_buffer(env, a.argv[4], &pmask, &npm)) return nullptr;
  if (a.argc > 6) {
    napi_valuetype t;
    napi_typeof(env, a.argv[5], &t);
    if (t != napi_undefined && t != napi_null) {
      if (!lookup_buffer(env, a.argv[5], &msa, &nm) || !lookup_buffer(env, a.argv[6], &mmask, &nmm)) return nullptr;
    }
  }
  const size_t pairs = (size_t)d.outgoing.length * d.outgoing.length;
  if (np < pairs * d.outgoing.c_z * dtype_bytes(d.outgoing.pair_dtype) || npm < pairs * 4) {
    throw_js(env, {true, "the pair or its mask buffer is too small"});
    return nullptr;
  }
  if (w[0]) {
    const size_t rows = (size_t)d.opm.sequences * d.opm.length;
    if (!msa || nm < rows * d.opm.c_m * dtype_bytes(d.opm.msa_dtype) || nmm < rows * 4) {
      throw_js(env, {true, "the outer-product mean needs the MSA and its mask buffers"});
      return nullptr;
    }
  }
  afhip_pair_stack_weights pw{w[0], w[1], w[2], w[3], w[4], w[5]};
  check(env, afhip_execution_pair_stack(e->ex, &d, &pw, msa, (const float*)mmask, pair, (const float*)pmask),
        "executionPairStack");
  return nullptr;
}

// executionEvoformerBlock(ex, blockDesc, {msaRowAttention?, msaColumnAttention?,
// msaTransition?, and the pair stack's}, msa, msaMask, pair, pairMask)
napi_value ExecutionEvoformerBlock(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 7)) return nullptr;
  uint32_t exh;
  ExecutionEntry* e;
  afhip_evoformer_block_desc d;
  if (!lookup_execution(env, a.argv[0], &exh, &e) || !read_block_desc(env, a.argv[1], &d)) return nullptr;
  const char* names[9] = {"msaRowAttention", "msaColumnAttention", "msaTransition", "outerProductMean",
                          "triangleOutgoing", "triangleIncoming", "triangleAttentionStarting",
                          "triangleAttentionEnding", "pairTransition"};
  void* w[9] = {};
  size_t need[9] = {};
  afhip_attention_weights_size(&d.msa_row, &need[0]);
  afhip_attention_weights_size(&d.msa_column, &need[1]);
  afhip_transition_weights_size(&d.msa_transition, &need[2]);
  afhip_opm_weights_size(&d.pair.opm, &need[3]);
  afhip_triangle_weights_size(&d.pair.outgoing, &need[4]);
  afhip_triangle_weights_size(&d.pair.incoming, &need[5]);
  afhip_attention_weights_size(&d.pair.attention_start, &need[6]);
  afhip_attention_weights_size(&d.pair.attention_end, &need[7]);
  afhip_transition_weights_size(&d.pair.transition, &need[8]);
  for (int i = 0; i < 9; i++) {
    bool has = false;
    napi_has_named_property(env, a.argv[2], names[i], &has);
    if (!has) continue;
    napi_value v;
    napi_get_named_property(env, a.argv[2], names[i], &v);
    napi_valuetype t;
    napi_typeof(env, v, &t);
    if (t == napi_undefined || t == napi_null) continue;
    if (!lookup_prepared(env, v, names[i], need[i], &w[i])) return nullptr;
  }
  void *msa, *mmask, *pair, *pmask;
  size_t nm, nmm, np, npm;
  if (!lookup_buffer(env, a.argv[3], &msa, &nm) || !lookup_buffer(env, a.argv[4], &mmask, &nmm) ||
      !lookup_buffer(env, a.argv[5], &pair, &np) || !lookup_buffer(env, a.argv[6], &pmask, &npm))
    return nullptr;
  const size_t rows = (size_t)d.pair.opm.sequences * d.pair.opm.length;
  const size_t pairs = (size_t)d.pair.outgoing.length * d.pair.outgoing.length;
  const size_t es = dtype_bytes(d.pair.outgoing.pair_dtype);
  if (nm < rows * d.pair.opm.c_m * es || nmm < rows * 4 || np < pairs * d.pair.outgoing.c_z * es || npm < pairs * 4) {
    throw_js(env, {true, "the MSA, the pair or a mask buffer is too small"});
    return nullptr;
  }
  afhip_evoformer_block_weights bw{w[0], w[1], w[2], {w[3], w[4], w[5], w[6], w[7], w[8]}};
  check(env, afhip_execution_evoformer_block(e->ex, &d, &bw, msa, (const float*)mmask, pair, (const float*)pmask),
        "executionEvoformerBlock");
  return nullptr;
}

// setMemoryBudget(bytes | null), memoryResident() -> bytes
napi_value SetMemoryBudget(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 1)) return nullptr;
  napi_valuetype t;
  napi_typeof(env, a.argv[0], &t);
  int64_t bytes = 0;
  if (t != napi_undefined && t != napi_null) {
    if (!get_int64(env, a.argv[0], &bytes)) return nullptr;
    if (bytes <= 0) {
      throw_js(env, {true, "GPU memory budget must be a positive safe integer"});
      return nullptr;
    }
  }
  check(env, afhip_set_memory_budget((uint64_t)bytes), "setMemoryBudget");
  return nullptr;
}

napi_value MemoryResident(napi_env env, napi_callback_info) {
  uint64_t bytes = 0;
  if (!check(env, afhip_memory_resident(&bytes), "memoryResident")) return nullptr;
  return make_number(env, (double)bytes);
}

// ---------------------------------------------------------------------------
// Operators with host arrays (upload, prepare, run, read back), as Promises
//
// The reference's run() is async (src/triangle/webgpu.ts:56,
// outer-product-mean.ts:549, transition.ts:264): it validates and queues
// synchronously, then awaits the GPU. Here the call copies its host arrays
// on the JS thread and returns a Promise; a libuv worker thread uploads
// through the operator's own execution (its allocator, allocator.ts:168-388,
// so repeated runs reuse pooled buffers), prepares the weights, runs, reads
// back and takes the execution's AllocationSnapshot while everything is
// still live, as the reference does before releasing (webgpu.ts:197-201).
// Runs on one execution take its lock in turn.
// ---------------------------------------------------------------------------

struct OperatorJob {
  napi_async_work work = nullptr;
  napi_deferred deferred = nullptr;
  afhip_execution* ex = nullptr;
  uint32_t exh = 0;  // the execution's handle, for its pending count
  std::mutex* lock = nullptr;
  std::vector<std::vector<char>> inputs;  // host copies, in the order the body uploads them
  int (*body)(OperatorJob&) = nullptr;
  afhip_triangle_desc tri{};
  afhip_opm_desc opm{};
  afhip_transition_desc tra{};
  afhip_attention_desc att{};
  int status = AFHIP_OK;
  std::string message;
  std::vector<float> output;
  double ms = 0.0;
  std::string memory;
};

// Uploads input i under `label`.
int job_upload(OperatorJob& j, size_t i, const char* label, void** out) {
  return afhip_execution_upload(j.ex, label, j.inputs[i].data(), j.inputs[i].size(), out);
}

// The common tail: wait, read the output back, snapshot the live allocation.
int job_finish(OperatorJob& j, const void* out, size_t out_bytes, double t0) {
  if (int s = afhip_synchronize(nullptr)) return s;
  j.output.resize(out_bytes / 4);
  if (int s = afhip_buffer_read(out, 0, j.output.data(), out_bytes)) return s;
  j.ms = now_ms() - t0;
  std::vector<char> json(1 << 16);
  if (int s = afhip_execution_snapshot(j.ex, json.data(), json.size())) return s;
  j.memory = json.data();
  return AFHIP_OK;
}

int triangle_body(OperatorJob& j) {
  const afhip_triangle_desc& d = j.tri;
  size_t wbytes = 0, wsbytes = 0;
  if (int s = afhip_triangle_weights_size(&d, &wbytes)) return s;
  if (int s = afhip_triangle_workspace_size(&d, &wsbytes)) return s;
  const size_t out_bytes = (size_t)d.length * d.length * d.c_z * 4;
  const double t0 = now_ms();
  void *z, *mask, *packed, *weights, *ws, *out;
  if (int s = job_upload(j, 0, "triangle.z", &z)) return s;
  if (int s = job_upload(j, 1, "triangle.mask", &mask)) return s;
  if (int s = job_upload(j, 2, "triangle.weights-f32", &packed)) return s;
  if (int s = afhip_execution_allocate(j.ex, "triangle.weights", wbytes, &weights)) return s;
  if (int s = afhip_execution_allocate(j.ex, "triangle.workspace", wsbytes ? wsbytes : 1, &ws)) return s;
  if (int s = afhip_execution_allocate(j.ex, "triangle.output", out_bytes, &out)) return s;
  if (int s = afhip_triangle_prepare_weights(&d, (const float*)packed, weights, nullptr)) return s;
  if (int s = afhip_triangle_run(&d, z, (const float*)mask, weights, out, ws, wsbytes, nullptr)) return s;
  return job_finish(j, out, out_bytes, t0);
}

int opm_body(OperatorJob& j) {
  const afhip_opm_desc& d = j.opm;
  size_t wbytes = 0, wsbytes = 0;
  if (int s = afhip_opm_weights_size(&d, &wbytes)) return s;
  if (int s = afhip_opm_workspace_size(&d, &wsbytes)) return s;
  const size_t out_bytes = (size_t)d.length * d.length * d.c_z * 4;
  const double t0 = now_ms();
  void *act, *mask, *packed, *weights, *ws, *out;
  if (int s = job_upload(j, 0, "outer-product-mean.activations", &act)) return s;
  if (int s = job_upload(j, 1, "outer-product-mean.mask", &mask)) return s;
  if (int s = job_upload(j, 2, "outer-product-mean.weights-f32", &packed)) return s;
  if (int s = afhip_execution_allocate(j.ex, "outer-product-mean.weights", wbytes, &weights)) return s;
  if (int s = afhip_execution_allocate(j.ex, "outer-product-mean.workspace", wsbytes ? wsbytes : 1, &ws)) return s;
  if (int s = afhip_execution_allocate(j.ex, "outer-product-mean.output", out_bytes, &out)) return s;
  if (int s = afhip_opm_prepare_weights(&d, (const float*)packed, weights, nullptr)) return s;
  if (int s = afhip_opm_run(&d, act, (const float*)mask, weights, out, ws, wsbytes, nullptr)) return s;
  return job_finish(j, out, out_bytes, t0);
}

int transition_body(OperatorJob& j) {
  const afhip_transition_desc& d = j.tra;
  size_t wbytes = 0, wsbytes = 0;
  if (int s = afhip_transition_weights_size(&d, &wbytes)) return s;
  if (int s = afhip_transition_workspace_size(&d, &wsbytes)) return s;
  const size_t out_bytes = (size_t)d.rows * d.channels * 4;
  const double t0 = now_ms();
  void *act, *packed, *weights, *ws, *out;
  if (int s = job_upload(j, 0, "transition.activations", &act)) return s;
  if (int s = job_upload(j, 1, "transition.weights-f32", &packed)) return s;
  if (int s = afhip_execution_allocate(j.ex, "transition.weights", wbytes, &weights)) return s;
  if (int s = afhip_execution_allocate(j.ex, "transition.workspace", wsbytes ? wsbytes : 1, &ws)) return s;
  if (int s = afhip_execution_allocate(j.ex, "transition.output", out_bytes, &out)) return s;
  if (int s = afhip_transition_prepare_weights(&d, (const float*)packed, weights, nullptr)) return s;
  if (int s = afhip_transition_run(&d, act, weights, out, ws, wsbytes, nullptr)) return s;
  return job_finish(j, out, out_bytes, t0);
}

int attention_body(OperatorJob& j) {
  const afhip_attention_desc& d = j.att;
  size_t wbytes = 0, wsbytes = 0;
  if (int s = afhip_attention_weights_size(&d, &wbytes)) return s;
  if (int s = afhip_attention_workspace_size(&d, &wsbytes)) return s;
  const size_t out_bytes = (size_t)d.batch * d.queries * d.channels * 4;
  const double t0 = now_ms();
  void *act, *mask, *pair = nullptr, *packed, *weights, *ws, *out;
  if (int s = job_upload(j, 0, "attention.activations", &act)) return s;
  if (int s = job_upload(j, 1, "attention.mask", &mask)) return s;
  if (int s = job_upload(j, 2, "attention.weights-f32", &packed)) return s;
  if (j.inputs.size() > 3)
    if (int s = job_upload(j, 3, "attention.pair-activations", &pair)) return s;
  if (int s = afhip_execution_allocate(j.ex, "attention.weights", wbytes, &weights)) return s;
  if (int s = afhip_execution_allocate(j.ex, "attention.workspace", wsbytes ? wsbytes : 1, &ws)) return s;
  if (int s = afhip_execution_allocate(j.ex, "attention.output", out_bytes, &out)) return s;
  if (int s = afhip_attention_prepare_weights(&d, (const float*)packed, weights, nullptr)) return s;
  if (int s = afhip_attention_run(&d, act, (const float*)mask, pair, weights, out, ws, wsbytes, nullptr)) return s;
  return job_finish(j, out, out_bytes, t0);
}

void job_execute(napi_env, void* data) {
  auto* j = static_cast<OperatorJob*>(data);
  std::lock_guard<std::mutex> guard(*j->lock);
  uint64_t mark = 0;
  // HIP's current device is a per-thread setting: select the opened device
  // on this worker before anything else.
  int s = afhip_open(g_ordinal);
  if (s == AFHIP_OK) s = afhip_execution_checkpoint(j->ex, &mark);
  if (s == AFHIP_OK) s = j->body(*j);
  if (s != AFHIP_OK) {
    j->message = afhip_last_error();
    (void)afhip_synchronize(nullptr);  // nothing queued may still use what is released below
  }
  (void)afhip_execution_release_since(j->ex, mark);
  (void)afhip_execution_note_submitted(j->ex);
  j->status = s;
  j->inputs.clear();
}

void job_complete(napi_env env, napi_status, void* data) {
  OperatorJob* j = static_cast<OperatorJob*>(data);
  if (j->status == AFHIP_OK) {
    napi_value o, mem;
    napi_create_object(env, &o);
    napi_value arr = make_float32(env, j->output);
    napi_set_named_property(env, o, "output", arr);
    napi_set_named_property(env, o, "elapsedMilliseconds", make_number(env, j->ms));
    napi_create_string_utf8(env, j->memory.c_str(), NAPI_AUTO_LENGTH, &mem);
    napi_set_named_property(env, o, "memoryJson", mem);
    napi_resolve_deferred(env, j->deferred, o);
  } else {
    napi_value msg, err;
    napi_create_string_utf8(env, j->message.c_str(), NAPI_AUTO_LENGTH, &msg);
    if (j->status == AFHIP_ERR_INVALID_ARGUMENT) napi_create_range_error(env, nullptr, msg, &err);
    else napi_create_error(env, nullptr, msg, &err);
    napi_reject_deferred(env, j->deferred, err);
  }
  napi_delete_async_work(env, j->work);
  // The worker is done with the execution: free it if a destroy (or Close)
  // came while this run was pending, and finish a deferred Close.
  auto it = g_reg.executions.find(j->exh);
  if (it != g_reg.executions.end() && --it->second.pending == 0 && it->second.released) {
    afhip_execution_destroy(it->second.ex);
    g_reg.executions.erase(it);
  }
  delete j;
  if (g_close_deferred && !runs_pending()) {
    g_close_deferred = false;
    (void)afhip_close();
  }
}

std::mutex& execution_lock(uint32_t handle) {
  static std::map<uint32_t, std::unique_ptr<std::mutex>> locks;
  auto& m = locks[handle];
  if (!m) m.reset(new std::mutex);
  return *m;
}

// Copies the TypedArray argument into the job's inputs.
bool job_input(napi_env env, napi_value v, OperatorJob& j, HostView* view = nullptr) {
  HostView h;
  if (!get_view(env, v, &h)) return false;
  const char* p = static_cast<const char*>(h.data);
  j.inputs.emplace_back(p, p + h.bytes);
  if (view) *view = h;
  return true;
}

napi_value queue_job(napi_env env, OperatorJob* j, uint32_t exh, const char* name) {
  j->lock = &execution_lock(exh);
  j->exh = exh;
  g_reg.executions[exh].pending++;
  napi_value promise, resource;
  napi_create_promise(env, &j->deferred, &promise);
  napi_create_string_utf8(env, name, NAPI_AUTO_LENGTH, &resource);
  napi_create_async_work(env, nullptr, resource, job_execute, job_complete, j, &j->work);
  napi_queue_async_work(env, j->work);
  return promise;
}

// triangleRun(execution, desc, z: Float32Array | Uint16Array (f16 bits),
// mask: Float32Array, packed: Float32Array) -> Promise<{output,
// elapsedMilliseconds, memoryJson}>
napi_value TriangleRun(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 5)) return nullptr;
  uint32_t exh;
  ExecutionEntry* e;
  if (!lookup_execution(env, a.argv[0], &exh, &e)) return nullptr;
  std::unique_ptr<OperatorJob> j(new OperatorJob);
  afhip_triangle_desc& d = j->tri;
  int64_t v;
  double eps;
  napi_value o = a.argv[1];
  if (!prop_int(env, o, "length", 0, &v)) return nullptr;
  d.length = (int32_t)v;
  if (!prop_int(env, o, "cZ", 0, &v)) return nullptr;
  d.c_z = (int32_t)v;
  if (!prop_int(env, o, "cHidden", 0, &v)) return nullptr;
  d.c_hidden = (int32_t)v;
  if (!prop_int(env, o, "direction", AFHIP_TRIANGLE_OUTGOING, &v)) return nullptr;
  d.direction = (int32_t)v;
  if (!prop_int(env, o, "precision", AFHIP_PRECISION_F32, &v)) return nullptr;
  d.precision = (int32_t)v;
  if (!prop_int(env, o, "blockRows", 0, &v)) return nullptr;
  d.block_rows = (int32_t)v;
  if (!prop_double(env, o, "epsilon", 1e-5, &eps)) return nullptr;
  d.epsilon = (float)eps;
  d.out_dtype = AFHIP_F32;
  d.residual = 0;
  HostView z, mask;
  if (!job_input(env, a.argv[2], *j, &z) || !job_input(env, a.argv[3], *j, &mask) || !job_input(env, a.argv[4], *j))
    return nullptr;
  d.pair_dtype = z.type == napi_uint16_array ? AFHIP_F16 : AFHIP_F32;
  size_t bytes = 0;
  if (!check(env, afhip_triangle_weights_size(&d, &bytes), "triangle")) return nullptr;
  const size_t pairs = (size_t)d.length * d.length;
  if (z.bytes != pairs * d.c_z * (d.pair_dtype == AFHIP_F16 ? 2 : 4) || mask.bytes != pairs * 4) {
    throw_js(env, {true, "z or mask does not match the descriptor's shape"});
    return nullptr;
  }
  j->ex = e->ex;
  j->body = triangle_body;
  return queue_job(env, j.release(), exh, "afhip.triangle");
}

// opmRun(execution, desc, activations: Float32Array, mask: Float32Array,
// packed: Float32Array) -> Promise<...>
napi_value OpmRun(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 5)) return nullptr;
  uint32_t exh;
  ExecutionEntry* e;
  if (!lookup_execution(env, a.argv[0], &exh, &e)) return nullptr;
  std::unique_ptr<OperatorJob> j(new OperatorJob);
  afhip_opm_desc& d = j->opm;
  int64_t v;
  double e1, e2;
  napi_value o = a.argv[1];
  if (!prop_int(env, o, "sequences", 0, &v)) return nullptr;
  d.sequences = (int32_t)v;
  if (!prop_int(env, o, "length", 0, &v)) return nullptr;
  d.length = (int32_t)v;
  if (!prop_int(env, o, "cM", 0, &v)) return nullptr;
  d.c_m = (int32_t)v;
  if (!prop_int(env, o, "cOuter", 0, &v)) return nullptr;
  d.c_outer = (int32_t)v;
  if (!prop_int(env, o, "cZ", 0, &v)) return nullptr;
  d.c_z = (int32_t)v;
  if (!prop_int(env, o, "precision", AFHIP_PRECISION_F32, &v)) return nullptr;
  d.precision = (int32_t)v;
  if (!prop_int(env, o, "rowBlockResidues", 0, &v)) return nullptr;
  d.row_block = (int32_t)v;
  if (!prop_double(env, o, "layerNormEpsilon", 1e-5, &e1) || !prop_double(env, o, "normalizationEpsilon", 1e-3, &e2))
    return nullptr;
  d.layer_norm_epsilon = (float)e1;
  d.normalization_epsilon = (float)e2;
  d.msa_dtype = AFHIP_F32;
  d.out_dtype = AFHIP_F32;
  HostView act, mask;
  if (!job_input(env, a.argv[2], *j, &act) || !job_input(env, a.argv[3], *j, &mask) || !job_input(env, a.argv[4], *j))
    return nullptr;
  size_t bytes = 0;
  if (!check(env, afhip_opm_weights_size(&d, &bytes), "outerProductMean")) return nullptr;
  const size_t rows = (size_t)d.sequences * d.length;
  if (act.bytes != rows * d.c_m * 4 || mask.bytes != rows * 4) {
    throw_js(env, {true, "activations or mask do not match the descriptor's shape"});
    return nullptr;
  }
  j->ex = e->ex;
  j->body = opm_body;
  return queue_job(env, j.release(), exh, "afhip.outerProductMean");
}

// transitionRun(execution, desc, activations: Float32Array, packed:
// Float32Array) -> Promise<...>
napi_value TransitionRun(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 4)) return nullptr;
  uint32_t exh;
  ExecutionEntry* e;
  if (!lookup_execution(env, a.argv[0], &exh, &e)) return nullptr;
  std::unique_ptr<OperatorJob> j(new OperatorJob);
  afhip_transition_desc& d = j->tra;
  int64_t v;
  double eps;
  napi_value o = a.argv[1];
  if (!prop_int(env, o, "rows", 0, &v)) return nullptr;
  d.rows = v;
  if (!prop_int(env, o, "channels", 0, &v)) return nullptr;
  d.channels = (int32_t)v;
  if (!prop_int(env, o, "hidden", 0, &v)) return nullptr;
  d.hidden = (int32_t)v;
  if (!prop_int(env, o, "precision", AFHIP_PRECISION_F32, &v)) return nullptr;
  d.precision = (int32_t)v;
  if (!prop_double(env, o, "epsilon", 1e-5, &eps)) return nullptr;
  d.epsilon = (float)eps;
  d.in_dtype = AFHIP_F32;
  d.out_dtype = AFHIP_F32;
  HostView act;
  if (!job_input(env, a.argv[2], *j, &act) || !job_input(env, a.argv[3], *j)) return nullptr;
  size_t bytes = 0;
  if (!check(env, afhip_transition_weights_size(&d, &bytes), "transition")) return nullptr;
  if (act.bytes != (size_t)d.rows * d.channels * 4) {
    throw_js(env, {true, "activations do not match the descriptor's shape"});
    return nullptr;
  }
  j->ex = e->ex;
  j->body = transition_body;
  return queue_job(env, j.release(), exh, "afhip.transition");
}

// attentionRun(execution, desc {batch, queries, channels, heads, transpose,
// pairBias (0 none, 1 normalized-input, 2 separate), pairChannels,
// precision, epsilon}, activations: Float32Array, mask: Float32Array,
// pairActivations: Float32Array | null, packed: Float32Array) ->
// Promise<...>: AttentionGpu.run (src/evoformer/attention.ts:1334-1452).
napi_value AttentionRun(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 6)) return nullptr;
  uint32_t exh;
  ExecutionEntry* e;
  if (!lookup_execution(env, a.argv[0], &exh, &e)) return nullptr;
  std::unique_ptr<OperatorJob> j(new OperatorJob);
  afhip_attention_desc& d = j->att;
  int64_t v[8];
  double eps;
  napi_value o = a.argv[1];
  const char* keys[8] = {"batch", "queries", "channels", "heads", "transpose", "pairBias", "pairChannels",
                         "precision"};
  const int64_t defaults[8] = {0, 0, 0, 0, 0, AFHIP_PAIR_BIAS_NONE, 0, AFHIP_PRECISION_F32};
  for (int i = 0; i < 8; i++)
    if (!prop_int(env, o, keys[i], defaults[i], &v[i])) return nullptr;
  if (!prop_double(env, o, "epsilon", 1e-5, &eps)) return nullptr;
  d = {(int32_t)v[0], (int32_t)v[1], (int32_t)v[2], (int32_t)v[3], (int32_t)v[4], (int32_t)v[5], (int32_t)v[6],
       (int32_t)v[7], AFHIP_F32, AFHIP_F32, 0, (float)eps};
  napi_valuetype pt;
  napi_typeof(env, a.argv[4], &pt);
  const bool has_pair = pt != napi_undefined && pt != napi_null;
  HostView act, mask, pair;
  if (!job_input(env, a.argv[2], *j, &act) || !job_input(env, a.argv[3], *j, &mask) || !job_input(env, a.argv[5], *j) ||
      (has_pair && !job_input(env, a.argv[4], *j, &pair)))
    return nullptr;
  size_t bytes = 0;
  if (!check(env, afhip_attention_weights_size(&d, &bytes), "attention")) return nullptr;
  const size_t rows = (size_t)d.batch * d.queries;
  if (act.bytes != rows * d.channels * 4 || mask.bytes != rows * 4) {
    throw_js(env, {true, "activations or mask do not match the descriptor's shape"});
    return nullptr;
  }
  if (d.pair_bias == AFHIP_PAIR_BIAS_SEPARATE &&
      (!has_pair || pair.bytes != (size_t)d.queries * d.queries * d.pair_channels * 4)) {
    throw_js(env, {true, "a separate pair bias needs pair activations [queries][queries][pairChannels]"});
    return nullptr;
  }
  j->ex = e->ex;
  j->body = attention_body;
  return queue_job(env, j.release(), exh, "afhip.attention");
}

// ---------------------------------------------------------------------------
// Kernel timing (WebGpuExecution's timestamp profile, execution.ts:329-345)
// ---------------------------------------------------------------------------

napi_value TimingEnable(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 1)) return nullptr;
  bool on = false;
  napi_get_value_bool(env, a.argv[0], &on);
  if (!check(env, afhip_timing_enable(on ? 1 : 0), "timingEnable")) return nullptr;
  return nullptr;
}

napi_value TimingReset(napi_env env, napi_callback_info) {
  if (!check(env, afhip_timing_reset(), "timingReset")) return nullptr;
  return nullptr;
}

napi_value TimingReport(napi_env env, napi_callback_info) {
  std::vector<char> buf(1 << 16);
  if (!check(env, afhip_timing_report(buf.data(), buf.size()), "timingReport")) return nullptr;
  napi_value s;
  NAPI_OK(napi_create_string_utf8(env, buf.data(), NAPI_AUTO_LENGTH, &s));
  return s;
}

napi_value Init(napi_env env, napi_value exports) {
  const struct {
    const char* name;
    napi_callback cb;
  } fns[] = {
      {"open", Open}, {"close", Close}, {"abiVersion", AbiVersion}, {"deviceReport", DeviceReport},
      {"bufferCreate", BufferCreate}, {"bufferDestroy", BufferDestroy}, {"bufferWrite", BufferWrite},
      {"bufferRead", BufferRead}, {"synchronize", Synchronize}, {"gemmGrid", GemmGrid}, {"gemmSelect", GemmSelect},
      {"gemmCalibrate", GemmCalibrate}, {"gemmForceVariant", GemmForceVariant}, {"calibrationLoad", CalibrationLoad},
      {"calibrationSave", CalibrationSave}, {"calibrationClear", CalibrationClear},
      {"calibrationInject", CalibrationInject}, {"gemmPlanCreate", GemmPlanCreate}, {"gemmPlanDestroy", GemmPlanDestroy},
      {"gemmWorkspaceSize", GemmWorkspaceSize}, {"gemmRun", GemmRun}, {"packWeightQ8Block", PackWeightQ8Block},
      {"executionCreate", ExecutionCreate}, {"executionDestroy", ExecutionDestroy},
      {"executionAllocate", ExecutionAllocate}, {"executionUpload", ExecutionUpload},
      {"executionRelease", ExecutionRelease}, {"executionCheckpoint", ExecutionCheckpoint},
      {"executionReleaseSince", ExecutionReleaseSince}, {"executionNoteSubmitted", ExecutionNoteSubmitted},
      {"executionSnapshot", ExecutionSnapshot}, {"executionAddInPlace", ExecutionAddInPlace},
      {"executionPrepareWeights", ExecutionPrepareWeights}, {"executionPairStack", ExecutionPairStack},
      {"executionEvoformerBlock", ExecutionEvoformerBlock},
      {"setMemoryBudget", SetMemoryBudget}, {"memoryResident", MemoryResident}, {"triangleRun", TriangleRun},
      {"opmRun", OpmRun}, {"transitionRun", TransitionRun}, {"attentionRun", AttentionRun}, {"timingEnable", TimingEnable},
      {"timingReset", TimingReset}, {"timingReport", TimingReport},
  };
  for (const auto& f : fns) {
    napi_value fn;
    if (napi_create_function(env, f.name, NAPI_AUTO_LENGTH, f.cb, nullptr, &fn) != napi_ok) return nullptr;
    if (napi_set_named_property(env, exports, f.name, fn) != napi_ok) return nullptr;
  }
  return exports;
}

}  // namespace

NAPI_MODULE(NODE_GYP_MODULE_NAME, Init)
