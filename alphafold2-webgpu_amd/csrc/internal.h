// Internal definitions shared by the afhip translation units (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>
#include <hip/hip_fp16.h>

#include <cstdint>
#include <cstdio>
#include <string>

#include "../../include/afhip.h"

namespace afhip {

// ---------------------------------------------------------------------------
// Errors: every entry point funnels failures through set_error and returns a
// status; no exception leaves the library.
// ---------------------------------------------------------------------------
int set_error(int status, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int hip_status(hipError_t err, const char* what);

#define AFHIP_CHECK_HIP(expr)                                   \
  do {                                                          \
    hipError_t err__ = (expr);                                  \
    if (err__ != hipSuccess) return ::afhip::hip_status(err__, #expr); \
  } while (0)

#define AFHIP_REQUIRE(cond, ...)                                          \
  do {                                                                    \
    if (!(cond)) return ::afhip::set_error(AFHIP_ERR_INVALID_ARGUMENT, __VA_ARGS__); \
  } while (0)

bool is_open();
int require_open();
int device_cu_count();
// The ordinal afhip_open selected (-1 when closed).
int current_device();

// The allocation-free GEMM entry point's device array (gemm_static.hip):
// records its address on `device`, which must be current; afhip_open calls
// it once per device.
int static_scratch_init(int device);

// ---------------------------------------------------------------------------
// Kernel timing: when enabled, each launch carries a start and a stop event
// on its own dispatch (hipExtLaunchKernelGGL), which time the kernel's
// execution as a kernel trace does, without event packets of their own
// between launches.
// ---------------------------------------------------------------------------
bool timing_enabled();
// While a TimingOff is alive on a thread, its launches create no events
// (an entry point that must not allocate anything runs under one).
struct TimingOff {
  TimingOff();
  ~TimingOff();
};
// Two fresh events for one launch labelled `label` (false: timing skipped).
bool timing_events(hipEvent_t* start, hipEvent_t* stop);
void timing_record(const char* label, hipEvent_t start, hipEvent_t stop);

// Raises a kernel's dynamic LDS ceiling to `bytes` (gfx950 grants up to
// 160 KiB a workgroup); once per kernel and size.
int allow_lds(const void* kernel, size_t bytes);

template <typename Kernel, typename... Args>
int launch(const char* label, Kernel kernel, dim3 grid, dim3 block, size_t shared, hipStream_t stream,
           Args... args) {
  if (grid.x == 0 || grid.y == 0 || grid.z == 0) return AFHIP_OK;
  hipEvent_t start = nullptr, stop = nullptr;
  if (timing_enabled() && timing_events(&start, &stop)) {
    hipExtLaunchKernelGGL(kernel, grid, block, shared, stream, start, stop, 0, args...);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return hip_status(err, label);
    timing_record(label, start, stop);
    return AFHIP_OK;
  }
  hipLaunchKernelGGL(kernel, grid, block, shared, stream, args...);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return hip_status(err, label);
  return AFHIP_OK;
}

inline size_t dtype_size(int dtype) { return dtype == AFHIP_F32 ? 4 : dtype == AFHIP_F16 ? 2 : 1; }
inline bool valid_float_dtype(int d) { return d == AFHIP_F32 || d == AFHIP_F16; }
inline bool valid_precision(int p) { return p == AFHIP_PRECISION_F32 || p == AFHIP_PRECISION_F16; }
__host__ __device__ inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }
__host__ __device__ inline int64_t round_up(int64_t a, int64_t b) { return ceil_div(a, b) * b; }

// ---------------------------------------------------------------------------
// Device-side vocabulary
// ---------------------------------------------------------------------------
typedef _Float16 half_t;
typedef half_t half8 __attribute__((ext_vector_type(8)));
typedef half_t half4 __attribute__((ext_vector_type(4)));
typedef half_t half2v __attribute__((ext_vector_type(2)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

// The MFMA tile every kernel here is written against: 32 x 32 output per
// wave64 instruction. Lane l owns output column (l % 32) and rows
//   8 * (v / 4) + 4 * (l / 32) + (v % 4),  v = 0..15.
// f16: A fragment = A[l % 32][8*(l/32) .. +8), B fragment = B[8*(l/32) .. +8][l % 32] (K = 16).
// f32: A fragment = A[l % 32][l / 32],         B fragment = B[l / 32][l % 32]          (K = 2).
__device__ __forceinline__ int mfma_row(int v, int lane) { return 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3); }

__device__ __forceinline__ floatx16 mfma_f16(half8 a, half8 b, floatx16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ floatx16 mfma_f32(float a, float b, floatx16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

template <int CTRL> __device__ __forceinline__ float dpp(float x) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), CTRL, 0xF, 0xF, true));
}

// Sum over a row of 16 lanes, every lane receiving it: DPP quad permutes,
// then the half-row and row mirrors, each fused into a v_add_f32_dpp (no LDS
// traffic, unlike a ds_bpermute shuffle).
__device__ __forceinline__ float row_sum16(float x) {
  x += dpp<0xB1>(x);   // quad_perm [1,0,3,2]
  x += dpp<0x4E>(x);   // quad_perm [2,3,0,1]
  x += dpp<0x141>(x);  // row_half_mirror: lane i <-> 7 - i
  x += dpp<0x140>(x);  // row_mirror: lane i <-> 15 - i
  return x;
}

// Sum over each aligned group of N lanes (N = 8, 16 or 32), every lane of the
// group receiving it: the 16-lane steps are DPP, the step across the two rows
// of a 32-lane group a swizzle.
template <int N> __device__ __forceinline__ float lane_sum(float x) {
  static_assert(N == 8 || N == 16 || N == 32, "lane group");
  x += dpp<0xB1>(x);
  x += dpp<0x4E>(x);
  x += dpp<0x141>(x);
  if constexpr (N >= 16) x += dpp<0x140>(x);
  if constexpr (N == 32) x += __shfl_xor(x, 16);
  return x;
}

// Hardware transcendentals (v_exp_f32, v_rcp_f32, v_rsq_f32; 1 ulp each):
// a correctly rounded division or square root expands to a dozen
// instructions, which in the per-element gates and LayerNorms costs more
// than the MFMA work around them.
__device__ __forceinline__ float fast_rcp(float x) { return __builtin_amdgcn_rcpf(x); }
__device__ __forceinline__ float fast_rsqrt(float x) { return __builtin_amdgcn_rsqf(x); }
// 1 / (1 + e^-x) = 1 / (1 + 2^(-x log2 e)); an infinite 2^(...) gives 0.
__device__ __forceinline__ float sigmoidf_(float x) {
  return fast_rcp(1.0f + __builtin_amdgcn_exp2f(-1.4426950408889634f * x));
}

// Vector-memory stores read their data VGPRs some time after they issue
// (under heavy memory traffic, long after), counting in EXP_CNT until they
// have; the compiler takes the data as read at issue and may hand the
// registers to the next instruction. A store whose data registers can be
// rewritten soon after (the next LDS read into the same registers, say) is
// followed by stores_read(data...), which waits for EXP_CNT to drain and
// keeps the registers live up to the wait.
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void stores_read(u32x4& a) { asm volatile("s_waitcnt expcnt(0)" : "+v"(a)); }
__device__ __forceinline__ void stores_read(u32x4& a, u32x4& b) {
  asm volatile("s_waitcnt expcnt(0)" : "+v"(a), "+v"(b));
}
__device__ __forceinline__ void stores_read(u32x4& a, u32x4& b, u32x4& c, u32x4& d) {
  asm volatile("s_waitcnt expcnt(0)" : "+v"(a), "+v"(b), "+v"(c), "+v"(d));
}

template <typename T> __device__ __forceinline__ float to_f32(T v) { return (float)v; }
template <typename T> __device__ __forceinline__ T from_f32(float v) { return (T)v; }

}  // namespace afhip
