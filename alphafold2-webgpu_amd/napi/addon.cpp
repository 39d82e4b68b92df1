// afhip.node: a thin Node-API addon over libafhip's C ABI (include/afhip.h),
// the HIP counterpart of the reference's native/wgpu-backend addon.
//
// Conventions, as the wgpu addon keeps them (native/wgpu-backend/src/lib.rs,
// device.rs):
//  - device memory is referred to by u32 handles from a registry owned by the
//    addon (lib.rs:24-730 hands out u32 handles for every wgpu object);
//    explicit destroy calls free them (lib.rs:706-730);
//  - host data crosses as TypedArrays, copied in and out;
//  - every call is synchronous on the JS thread;
//  - failures become JS exceptions: RangeError for invalid arguments (the
//    reference's RangeError, src/triangle/types.ts:42-52), Error otherwise,
//    with libafhip's message.
// The operator entry points (triangleRun, opmRun, transitionRun) upload,
// run and read back in one call, as TriangleMultiplicationGpu.run does
// (src/triangle/webgpu.ts:56-201), and report the elapsed wall time from
// the first upload through the readback, as that method does (:189-196).
#include <node_api.h>

#include <chrono>
#include <climits>
#include <cstdint>
#include <cstring>
#include <map>
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
};

struct Registry {
  uint32_t next = 1;
  std::map<uint32_t, std::pair<void*, size_t>> buffers;
  std::map<uint32_t, afhip_gemm_plan*> plans;
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

napi_value Open(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 0)) return nullptr;
  int64_t ordinal = 0;
  if (a.argc > 0 && !get_int64(env, a.argv[0], &ordinal)) return nullptr;
  if (!check(env, afhip_open((int)ordinal), "open")) return nullptr;
  return nullptr;
}

napi_value Close(napi_env env, napi_callback_info) {
  for (auto& kv : g_reg.buffers)
    if (!g_reg.owner.count(kv.first)) afhip_buffer_destroy(kv.second.first);
  for (auto& kv : g_reg.executions) afhip_execution_destroy(kv.second.ex);
  for (auto& kv : g_reg.plans) afhip_gemm_plan_destroy(kv.second);
  g_reg.buffers.clear();
  g_reg.plans.clear();
  g_reg.executions.clear();
  g_reg.owner.clear();
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
  if (!lookup_buffer(env, a.argv[0], &codes, &codes_bytes) || !lookup_buffer(env, a.argv[1], &scales, &scales_bytes) ||
      !get_int64(env, a.argv[2], &block) || !get_int64(env, a.argv[3], &start) || !get_int64(env, a.argv[4], &rows_k) ||
      !get_int64(env, a.argv[5], &columns_n) || !lookup_buffer(env, a.argv[6], &dst, &dst_bytes) ||
      !get_int64(env, a.argv[7], &dtype))
    return nullptr;
  if (block <= 0 || start < 0 || rows_k <= 0 || columns_n <= 0 || rows_k > INT32_MAX || columns_n > INT32_MAX ||
      (dtype != AFHIP_F32 && dtype != AFHIP_F16)) {
    throw_js(env, {true, "packWeightQ8Block: invalid block, range, shape or dtype"});
    return nullptr;
  }
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
  if (it == g_reg.executions.end()) {
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

size_t dtype_bytes(int64_t d) { return d == AFHIP_F16 ? 2 : 4; }

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
  for (int i = 0; i < 6; i++) {
    bool has = false;
    napi_has_named_property(env, a.argv[2], names[i], &has);
    if (!has) continue;
    napi_value v;
    napi_get_named_property(env, a.argv[2], names[i], &v);
    napi_valuetype t;
    napi_typeof(env, v, &t);
    if (t == napi_undefined || t == napi_null) continue;
    if (!lookup_buffer(env, v, &w[i], nullptr)) return nullptr;
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
  for (int i = 0; i < 9; i++) {
    bool has = false;
    napi_has_named_property(env, a.argv[2], names[i], &has);
    if (!has) continue;
    napi_value v;
    napi_get_named_property(env, a.argv[2], names[i], &v);
    napi_valuetype t;
    napi_typeof(env, v, &t);
    if (t == napi_undefined || t == napi_null) continue;
    if (!lookup_buffer(env, v, &w[i], nullptr)) return nullptr;
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
// Operators with host arrays (upload, prepare, run, read back)
// ---------------------------------------------------------------------------

napi_value result_object(napi_env env, const std::vector<float>& out, double ms, size_t peak) {
  napi_value o, mem;
  napi_create_object(env, &o);
  napi_value arr = make_float32(env, out);
  if (!arr) return nullptr;
  napi_set_named_property(env, o, "output", arr);
  napi_set_named_property(env, o, "elapsedMilliseconds", make_number(env, ms));
  napi_create_object(env, &mem);
  napi_set_named_property(env, mem, "peakBytes", make_number(env, (double)peak));
  napi_set_named_property(env, o, "memory", mem);
  return o;
}

// triangleRun(desc, z: Float32Array | Uint16Array (f16 bits), mask: Float32Array, packed: Float32Array)
napi_value TriangleRun(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 4)) return nullptr;
  afhip_triangle_desc d{};
  int64_t v;
  double eps;
  napi_value o = a.argv[0];
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
  HostView z, mask, packed;
  if (!get_view(env, a.argv[1], &z) || !get_view(env, a.argv[2], &mask) || !get_view(env, a.argv[3], &packed))
    return nullptr;
  d.pair_dtype = z.type == napi_uint16_array ? AFHIP_F16 : AFHIP_F32;
  size_t wbytes = 0, wsbytes = 0;
  if (!check(env, afhip_triangle_weights_size(&d, &wbytes), "triangle") ||
      !check(env, afhip_triangle_workspace_size(&d, &wsbytes), "triangle"))
    return nullptr;
  const size_t pairs = (size_t)d.length * d.length;
  const size_t zbytes = pairs * d.c_z * (d.pair_dtype == AFHIP_F16 ? 2 : 4);
  if (z.bytes != zbytes || mask.bytes != pairs * 4) {
    throw_js(env, {true, "z or mask does not match the descriptor's shape"});
    return nullptr;
  }
  const double t0 = now_ms();
  DeviceBuf dz, dm, dp, dw, dws, dout;
  if (!check(env, dz.alloc(zbytes), "triangle") || !check(env, dm.alloc(mask.bytes), "triangle") ||
      !check(env, dp.alloc(packed.bytes), "triangle") || !check(env, dw.alloc(wbytes), "triangle") ||
      !check(env, dws.alloc(wsbytes), "triangle") || !check(env, dout.alloc(pairs * d.c_z * 4), "triangle"))
    return nullptr;
  if (!check(env, afhip_buffer_write(dz.p, 0, z.data, zbytes), "triangle") ||
      !check(env, afhip_buffer_write(dm.p, 0, mask.data, mask.bytes), "triangle") ||
      !check(env, afhip_buffer_write(dp.p, 0, packed.data, packed.bytes), "triangle") ||
      !check(env, afhip_triangle_prepare_weights(&d, (const float*)dp.p, dw.p, nullptr), "triangle") ||
      !check(env, afhip_triangle_run(&d, dz.p, (const float*)dm.p, dw.p, dout.p, dws.p, wsbytes, nullptr),
             "triangle"))
    return nullptr;
  std::vector<float> out(pairs * d.c_z);
  if (!check(env, afhip_buffer_read(dout.p, 0, out.data(), out.size() * 4), "triangle")) return nullptr;
  const double ms = now_ms() - t0;
  const size_t peak = zbytes + mask.bytes + packed.bytes + wbytes + wsbytes + out.size() * 4;
  return result_object(env, out, ms, peak);
}

// opmRun(desc, activations: Float32Array, mask: Float32Array, packed: Float32Array)
napi_value OpmRun(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 4)) return nullptr;
  afhip_opm_desc d{};
  int64_t v;
  double e1, e2;
  napi_value o = a.argv[0];
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
  HostView act, mask, packed;
  if (!get_view(env, a.argv[1], &act) || !get_view(env, a.argv[2], &mask) || !get_view(env, a.argv[3], &packed))
    return nullptr;
  size_t wbytes = 0, wsbytes = 0;
  if (!check(env, afhip_opm_weights_size(&d, &wbytes), "outerProductMean") ||
      !check(env, afhip_opm_workspace_size(&d, &wsbytes), "outerProductMean"))
    return nullptr;
  const size_t rows = (size_t)d.sequences * d.length;
  if (act.bytes != rows * d.c_m * 4 || mask.bytes != rows * 4) {
    throw_js(env, {true, "activations or mask do not match the descriptor's shape"});
    return nullptr;
  }
  const size_t obytes = (size_t)d.length * d.length * d.c_z * 4;
  const double t0 = now_ms();
  DeviceBuf da, dm, dp, dw, dws, dout;
  if (!check(env, da.alloc(act.bytes), "outerProductMean") || !check(env, dm.alloc(mask.bytes), "outerProductMean") ||
      !check(env, dp.alloc(packed.bytes), "outerProductMean") || !check(env, dw.alloc(wbytes), "outerProductMean") ||
      !check(env, dws.alloc(wsbytes), "outerProductMean") || !check(env, dout.alloc(obytes), "outerProductMean"))
    return nullptr;
  if (!check(env, afhip_buffer_write(da.p, 0, act.data, act.bytes), "outerProductMean") ||
      !check(env, afhip_buffer_write(dm.p, 0, mask.data, mask.bytes), "outerProductMean") ||
      !check(env, afhip_buffer_write(dp.p, 0, packed.data, packed.bytes), "outerProductMean") ||
      !check(env, afhip_opm_prepare_weights(&d, (const float*)dp.p, dw.p, nullptr), "outerProductMean") ||
      !check(env, afhip_opm_run(&d, da.p, (const float*)dm.p, dw.p, dout.p, dws.p, wsbytes, nullptr),
             "outerProductMean"))
    return nullptr;
  std::vector<float> out(obytes / 4);
  if (!check(env, afhip_buffer_read(dout.p, 0, out.data(), obytes), "outerProductMean")) return nullptr;
  const double ms = now_ms() - t0;
  return result_object(env, out, ms, act.bytes + mask.bytes + packed.bytes + wbytes + wsbytes + obytes);
}

// transitionRun(desc, activations: Float32Array, packed: Float32Array)
napi_value TransitionRun(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 3)) return nullptr;
  afhip_transition_desc d{};
  int64_t v;
  double eps;
  napi_value o = a.argv[0];
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
  HostView act, packed;
  if (!get_view(env, a.argv[1], &act) || !get_view(env, a.argv[2], &packed)) return nullptr;
  size_t wbytes = 0, wsbytes = 0;
  if (!check(env, afhip_transition_weights_size(&d, &wbytes), "transition") ||
      !check(env, afhip_transition_workspace_size(&d, &wsbytes), "transition"))
    return nullptr;
  if (act.bytes != (size_t)d.rows * d.channels * 4) {
    throw_js(env, {true, "activations do not match the descriptor's shape"});
    return nullptr;
  }
  const double t0 = now_ms();
  DeviceBuf da, dp, dw, dws, dout;
  if (!check(env, da.alloc(act.bytes), "transition") || !check(env, dp.alloc(packed.bytes), "transition") ||
      !check(env, dw.alloc(wbytes), "transition") || !check(env, dws.alloc(wsbytes), "transition") ||
      !check(env, dout.alloc(act.bytes), "transition"))
    return nullptr;
  if (!check(env, afhip_buffer_write(da.p, 0, act.data, act.bytes), "transition") ||
      !check(env, afhip_buffer_write(dp.p, 0, packed.data, packed.bytes), "transition") ||
      !check(env, afhip_transition_prepare_weights(&d, (const float*)dp.p, dw.p, nullptr), "transition") ||
      !check(env, afhip_transition_run(&d, da.p, dw.p, dout.p, dws.p, wsbytes, nullptr), "transition"))
    return nullptr;
  std::vector<float> out(act.bytes / 4);
  if (!check(env, afhip_buffer_read(dout.p, 0, out.data(), act.bytes), "transition")) return nullptr;
  const double ms = now_ms() - t0;
  return result_object(env, out, ms, act.bytes * 2 + packed.bytes + wbytes + wsbytes);
}

// attentionRun(desc {batch, queries, channels, heads, transpose, pairBias
// (0 none, 1 normalized-input, 2 separate), pairChannels, precision,
// epsilon}, activations: Float32Array, mask: Float32Array, pairActivations:
// Float32Array | null, packed: Float32Array) -- AttentionGpu.run
// (src/evoformer/attention.ts:1334-1452) over host arrays.
napi_value AttentionRun(napi_env env, napi_callback_info info) {
  Args a;
  if (!get_args(env, info, a, 5)) return nullptr;
  afhip_attention_desc d{};
  int64_t v[8];
  double eps;
  napi_value o = a.argv[0];
  const char* keys[8] = {"batch", "queries", "channels", "heads", "transpose", "pairBias", "pairChannels",
                         "precision"};
  const int64_t defaults[8] = {0, 0, 0, 0, 0, AFHIP_PAIR_BIAS_NONE, 0, AFHIP_PRECISION_F32};
  for (int i = 0; i < 8; i++)
    if (!prop_int(env, o, keys[i], defaults[i], &v[i])) return nullptr;
  if (!prop_double(env, o, "epsilon", 1e-5, &eps)) return nullptr;
  d = {(int32_t)v[0], (int32_t)v[1], (int32_t)v[2], (int32_t)v[3], (int32_t)v[4], (int32_t)v[5], (int32_t)v[6],
       (int32_t)v[7], AFHIP_F32, AFHIP_F32, 0, (float)eps};
  HostView act, mask, pair, packed;
  napi_valuetype pt;
  napi_typeof(env, a.argv[3], &pt);
  const bool has_pair = pt != napi_undefined && pt != napi_null;
  if (!get_view(env, a.argv[1], &act) || !get_view(env, a.argv[2], &mask) ||
      (has_pair && !get_view(env, a.argv[3], &pair)) || !get_view(env, a.argv[4], &packed))
    return nullptr;
  size_t wbytes = 0, wsbytes = 0;
  if (!check(env, afhip_attention_weights_size(&d, &wbytes), "attention") ||
      !check(env, afhip_attention_workspace_size(&d, &wsbytes), "attention"))
    return nullptr;
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
  const double t0 = now_ms();
  DeviceBuf da, dm, dpair, dp, dw, dws, dout;
  if (!check(env, da.alloc(act.bytes), "attention") || !check(env, dm.alloc(mask.bytes), "attention") ||
      !check(env, dp.alloc(packed.bytes), "attention") || !check(env, dw.alloc(wbytes), "attention") ||
      !check(env, dws.alloc(wsbytes), "attention") || !check(env, dout.alloc(act.bytes), "attention") ||
      (has_pair && !check(env, dpair.alloc(pair.bytes), "attention")))
    return nullptr;
  if (!check(env, afhip_buffer_write(da.p, 0, act.data, act.bytes), "attention") ||
      !check(env, afhip_buffer_write(dm.p, 0, mask.data, mask.bytes), "attention") ||
      (has_pair && !check(env, afhip_buffer_write(dpair.p, 0, pair.data, pair.bytes), "attention")) ||
      !check(env, afhip_buffer_write(dp.p, 0, packed.data, packed.bytes), "attention") ||
      !check(env, afhip_attention_prepare_weights(&d, (const float*)dp.p, dw.p, nullptr), "attention") ||
      !check(env, afhip_attention_run(&d, da.p, (const float*)dm.p, has_pair ? dpair.p : nullptr, dw.p, dout.p,
                                      dws.p, wsbytes, nullptr),
             "attention"))
    return nullptr;
  std::vector<float> out(act.bytes / 4);
  if (!check(env, afhip_buffer_read(dout.p, 0, out.data(), act.bytes), "attention")) return nullptr;
  const double ms = now_ms() - t0;
  return result_object(env, out, ms, act.bytes * 2 + mask.bytes + pair.bytes + packed.bytes + wbytes + wsbytes);
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
      {"calibrationSave", CalibrationSave}, {"gemmPlanCreate", GemmPlanCreate}, {"gemmPlanDestroy", GemmPlanDestroy},
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
