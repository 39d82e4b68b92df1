// The shared tiled GEMM for gfx950, its plan API, weight packing and the
// int8 dequantisation kernels.
//
// One workgroup of 256 lanes (four wave64s in a 2 x 2 arrangement) covers a
// BM x BN output tile and walks K in steps of 32. Both operands are staged
// k-contiguous in LDS, double-buffered, with the next step's 16-byte global
// loads issued before the current step's MFMAs. f16 precision feeds
// v_mfma_f32_32x32x16_f16 (operands rounded to f16, f32 accumulation); f32
// precision feeds v_mfma_f32_32x32x2_f32 (exact f32 products). int8 weights
// are widened to f16 on their way into LDS, which is exact for |q| <= 127,
// and their per-column scale is applied to the f32 accumulator.
//
// Workgroups are numbered so that consecutive tiles land on one XCD: the
// hardware deals workgroup ids round-robin over the eight XCDs, so tile
// t = (id % 8) * per_xcd + id / 8 keeps a batch's tiles (which share
// operands) inside one XCD's L2.
#include <cmath>
#include <cstring>
#include <map>
#include <mutex>
#include <string>

#include "gemm_kernel.h"

namespace afhip {

namespace {

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace

static afhip_variant tile_variant(const GemmTypes& t, int64_t M, int64_t N, int64_t K, int batch);

int run_gemm(const GemmArgs& g, const GemmTypes& t, const afhip_variant& v, const char* label, hipStream_t stream) {
  AFHIP_REQUIRE(g.M > 0 && g.N > 0 && g.K > 0 && g.batch > 0, "GEMM dimensions must be positive (M=%d N=%d K=%d batch=%d)",
                g.M, g.N, g.K, g.batch);
  AFHIP_REQUIRE(g.a && g.b && g.c, "GEMM operand or output is NULL");
  AFHIP_REQUIRE(valid_precision(t.precision), "unknown precision %d", t.precision);
  AFHIP_REQUIRE(valid_float_dtype(t.a_dtype), "source dtype must be f32 or f16");
  AFHIP_REQUIRE(valid_float_dtype(t.b_dtype) || t.b_dtype == AFHIP_I8, "weight dtype must be f32, f16 or i8");
  AFHIP_REQUIRE(valid_float_dtype(t.c_dtype), "output dtype must be f32 or f16");
  AFHIP_REQUIRE(!(t.b_dtype == AFHIP_I8 && t.precision == AFHIP_PRECISION_F32),
                "int8 weights run with f16 precision (the widening to f16 is exact)");
  AFHIP_REQUIRE(!(g.flags & AFHIP_EPILOGUE_SCALE) || g.scale, "SCALE epilogue without a scale vector");
  AFHIP_REQUIRE(!(g.flags & AFHIP_EPILOGUE_BIAS) || g.bias, "BIAS epilogue without a bias vector");
  AFHIP_REQUIRE(!(g.flags & AFHIP_EPILOGUE_RESIDUAL) || g.residual, "RESIDUAL epilogue without a residual");
  AFHIP_REQUIRE(!(g.flags & AFHIP_EPILOGUE_ATTENTION) || (g.head_cols > 0 && g.N == 4 * g.head_cols),
                "ATTENTION epilogue needs columns == 4 * heads * head_dim");
  if (v.kernel == AFHIP_KERNEL_STREAM) {
    if (stream_eligible(g, t)) return run_gemm_stream(g, t, label, stream);
    // Operands STREAM cannot take run on the family the tile heuristic picks
    // for them without it.
    return run_gemm(g, t, tile_variant(t, g.M, g.N, g.K, g.batch), label, stream);
  }
  if (v.kernel == AFHIP_KERNEL_LDS_DMA) {
    if (dma_eligible(g, t) && dma_tile_supported(v.tile_rows, v.tile_columns))
      return run_gemm_dma(g, t, v.tile_rows, v.tile_columns, label, stream);
    // Operands the LDS_DMA family cannot take (alignment, K % 8, dtypes) run
    // on the register-staged kernel with its heuristic tile.
    return run_gemm(g, t, register_variant(t.precision, g.M, g.N, g.K, g.batch), label, stream);
  }
  AFHIP_REQUIRE(v.kernel == AFHIP_KERNEL_REGISTER_STAGED, "unknown kernel family %d", v.kernel);
  const int va = 16 / (int)dtype_size(t.a_dtype), vb = 16 / (int)dtype_size(t.b_dtype);
  // 16-byte operand loads run along k (or, for a row-contiguous A, along m,
  // where the loader guards a ragged last chunk itself).
  const bool vec_a = (g.a_row_contiguous || g.K % va == 0) && g.lda % va == 0 && g.sa % va == 0 && aligned16(g.a);
  bool vec = vec_a && g.K % vb == 0 && g.ldb % vb == 0 && g.sb % vb == 0 && aligned16(g.b);
  if (t.precision == AFHIP_PRECISION_F16) {
    AFHIP_REQUIRE(t.b_dtype != AFHIP_F32, "f16 precision takes f16 or int8 weights (prepare them first)");
    if (t.a_dtype == AFHIP_F32) return gemm_dispatch_f16_a32(g, t, v, vec, label, stream);
    return gemm_dispatch_f16_a16(g, t, v, vec, label, stream);
  }
  AFHIP_REQUIRE(t.a_dtype == AFHIP_F32 && t.b_dtype == AFHIP_F32, "f32 precision takes f32 operands");
  return gemm_dispatch_f32(g, t, v, vec, label, stream);
}

// The REGISTER_STAGED family's variant, the one every operand form runs on
// (and what a run falls back to when a faster family refuses its operands).
// Prefer the largest tile that still gives every CU two workgroups, or one
// when K is long enough for a tile's own k-loop to hide its latency
// (measured on the reference's opm-contract shape, 128 x 508 x 32000:
// 128 x 64 at 0.053 ms against 64 x 64 at 0.065 ms).
afhip_variant register_variant(int precision, int64_t M, int64_t N, int64_t K, int batch) {
  afhip_variant v{};
  v.precision = precision;
  v.tile_inner = gemm_detail::kBK;
  v.vectorized = 1;
  v.source = 0;
  v.kernel = AFHIP_KERNEL_REGISTER_STAGED;
  const int64_t cus = device_cu_count() > 0 ? device_cu_count() : 256;
  const int64_t target = K >= 384 ? cus : 2 * cus;
  const int shapes[4][2] = {{128, 128}, {128, 64}, {64, 128}, {64, 64}};
  for (auto& s : shapes) {
    int64_t tiles = ceil_div(M, s[0]) * ceil_div(N, s[1]) * batch;
    v.tile_rows = s[0];
    v.tile_columns = s[1];
    if (tiles >= target) return v;
  }
  return v;
}

// The heuristic among the tiled families (LDS_DMA, REGISTER_STAGED).
static afhip_variant tile_variant(const GemmTypes& t, int64_t M, int64_t N, int64_t K, int batch) {
  afhip_variant v = register_variant(t.precision, M, N, K, batch);
  // LDS_DMA takes f16 operands with an even K (16-byte loads when K is a
  // multiple of 8, 4-byte loads otherwise), an f32 A with K a multiple of 8
  // (rounded to f16 as its fragments are read), and int8 weights that a plan
  // widens to f16 first (exact); anything else is staged through registers.
  if (t.precision == AFHIP_PRECISION_F16 && ((t.a_dtype == AFHIP_F16 && K % 2 == 0) || (t.a_dtype == AFHIP_F32 && K % 8 == 0)) &&
      (t.b_dtype == AFHIP_F16 || t.b_dtype == AFHIP_I8)) {
    v.kernel = AFHIP_KERNEL_LDS_DMA;
    dma_heuristic_tile(M, N, K, batch, &v.tile_rows, &v.tile_columns);
    return v;
  }
  // f32 arithmetic with K a multiple of 4 takes LDS_DMA too, which runs it
  // on 64 x 64 tiles whatever the variant's tile (its nominal 128 x 128).
  // Measured on MI355X against the register-staged kernel's best tile (f32
  // out, bias + ReLU): 4096 x 128 x 512 10.6 / 12.5 us, 1024^3 26.3 / 32.9,
  // 128 x 384^3 142 / 158, 4096 x 1024 x 4096 317 / 331, 65536 x 128 x 512
  // 111 / 109.
  if (t.precision == AFHIP_PRECISION_F32 && t.a_dtype == AFHIP_F32 && t.b_dtype == AFHIP_F32 && K % 4 == 0) {
    v.kernel = AFHIP_KERNEL_LDS_DMA;
    v.tile_rows = v.tile_columns = 128;
    return v;
  }
  return v;
}

// Weight-stationary streaming for tall, bandwidth-bound projections (many
// rows against a short K and at least 448 columns, so a slice's eight waves
// are mostly busy); the tiled families otherwise. Measured on the
// reference's SHAPES (tools/gemm-candidates.ts:637-669): STREAM wins from
// ~16k rows (29,972 x 256 x 1,024: 0.026 ms against 0.028 for the best tile)
// and loses below (8,192 x 128 x 512: 0.0083 against 0.0071).
afhip_variant heuristic_variant(const GemmTypes& t, int64_t M, int64_t N, int64_t K, int batch) {
  if (stream_shape_ok(t, M, N, K, batch) && M >= 16384 && N >= 448) {
    afhip_variant v{};
    v.precision = t.precision;
    v.tile_rows = 64;
    v.tile_columns = 512;
    v.tile_inner = gemm_detail::kBK;
    v.vectorized = 1;
    v.kernel = AFHIP_KERNEL_STREAM;
    return v;
  }
  return tile_variant(t, M, N, K, batch);
}

// ---------------------------------------------------------------------------
// Packing and conversion kernels
// ---------------------------------------------------------------------------

namespace {

template <typename TS, typename TD>
__global__ void pack_transpose_kernel(const TS* __restrict__ src, int K, int N, int64_t ld_src, TD* __restrict__ dst,
                                      int64_t ld_dst) {
  __shared__ float tile[32][33];
  int k0 = blockIdx.y * 32, n0 = blockIdx.x * 32;
  int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 32 x 8
  for (int r = ty; r < 32; r += 8) {
    int k = k0 + r, n = n0 + tx;
    tile[r][tx] = (k < K && n < N) ? (float)src[(int64_t)k * ld_src + n] : 0.0f;
  }
  __syncthreads();
  for (int r = ty; r < 32; r += 8) {
    int n = n0 + r, k = k0 + tx;
    if (n < N && k < K) dst[(int64_t)n * ld_dst + k] = (TD)tile[tx][r];
  }
}

// int8 rows [rows][cols] (leading dimension ld_src) widened to f16 rows of
// cols halves; exact, |q| <= 127. Eight columns a lane (one 8-byte read, one
// 16-byte write where both are aligned), rows along y.
__global__ void widen_rows_kernel(const int8_t* __restrict__ src, int rows, int cols, int64_t ld_src,
                                  half_t* __restrict__ dst) {
  const int c = 8 * (blockIdx.x * blockDim.x + threadIdx.x);
  if (c >= cols) return;
  for (int r = blockIdx.y; r < rows; r += gridDim.y) {
    const int8_t* s = src + (int64_t)r * ld_src + c;
    half_t* d = dst + (int64_t)r * cols + c;
    if (c + 8 <= cols && (reinterpret_cast<uintptr_t>(s) & 7) == 0 && (reinterpret_cast<uintptr_t>(d) & 15) == 0) {
      const uint2 v = *reinterpret_cast<const uint2*>(s);
      half8 h;
#pragma unroll
      for (int e = 0; e < 4; e++) {
        h[e] = (half_t)(float)(int8_t)(v.x >> (8 * e));
        h[4 + e] = (half_t)(float)(int8_t)(v.y >> (8 * e));
      }
      *reinterpret_cast<half8*>(d) = h;
    } else {
      for (int e = 0; e < 8 && c + e < cols; e++) d[e] = (half_t)(float)s[e];
    }
  }
}

template <typename TD>
__global__ void convert_kernel(const float* __restrict__ src, int64_t count, TD* __restrict__ dst) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (; i < count; i += stride) dst[i] = (TD)src[i];
}

__global__ void dequant_channel_kernel(const int8_t* __restrict__ q, const float* __restrict__ scale, int K, int N,
                                       float* __restrict__ out) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  int64_t total = (int64_t)K * N;
  if (i >= total) return;
  int n = (int)(i % N);
  // One correctly rounded product; __fmul_rn keeps it from being contracted.
  out[i] = __fmul_rn((float)q[i], scale[n]);
}

__global__ void dequant_block_kernel(const int8_t* __restrict__ codes, const uint16_t* __restrict__ scales, int block,
                                     int64_t start, int64_t count, float* __restrict__ out) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= count) return;
  int64_t absolute = start + i;
  __half_raw raw;
  raw.x = scales[absolute / block];
  float s = __half2float(__half(raw));
  out[i] = __fmul_rn((float)codes[absolute], s);
}

// W[n][k] (k-contiguous, the GEMM's packed operand) from the reference
// bundle's mixed-q8 tensor [K][N], stored flat from element `start` of the
// bundle's int8 stream: w = f32(code[e]) * f32(scale_f16[e / block]),
// e = start + k N + n (src/reference/dtype.ts:66-99), one correctly rounded
// product as the host decode computes it, then converted to TD (round to
// nearest even for f16). A 32 x 32 tile passes through LDS so that both the
// code reads (along n) and the stores (along k) are contiguous.
template <typename TD>
__global__ void pack_q8_block_kernel(const int8_t* __restrict__ codes, const uint16_t* __restrict__ scales, int block,
                                     int64_t start, int K, int N, TD* __restrict__ dst) {
  __shared__ float tile[32][33];
  const int k0 = blockIdx.y * 32, n0 = blockIdx.x * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 32 x 8
  for (int r = ty; r < 32; r += 8) {
    const int k = k0 + r, n = n0 + tx;
    float v = 0.0f;
    if (k < K && n < N) {
      const int64_t e = start + (int64_t)k * N + n;
      __half_raw raw;
      raw.x = scales[e / block];
      v = __fmul_rn((float)codes[e], __half2float(__half(raw)));
    }
    tile[r][tx] = v;
  }
  __syncthreads();
  for (int r = ty; r < 32; r += 8) {
    const int n = n0 + r, k = k0 + tx;
    if (n < N && k < K) dst[(int64_t)n * K + k] = (TD)tile[tx][r];
  }
}

template <typename TS>
int pack_dispatch(const TS* src, int K, int N, int64_t ld_src, void* dst, int dst_dtype, int64_t ld_dst,
                  hipStream_t s) {
  dim3 grid((unsigned)ceil_div(N, 32), (unsigned)ceil_div(K, 32));
  if (dst_dtype == AFHIP_F32)
    return launch("pack_transpose", pack_transpose_kernel<TS, float>, grid, dim3(256), 0, s, src, K, N, ld_src,
                  (float*)dst, ld_dst);
  if (dst_dtype == AFHIP_F16)
    return launch("pack_transpose", pack_transpose_kernel<TS, half_t>, grid, dim3(256), 0, s, src, K, N, ld_src,
                  (half_t*)dst, ld_dst);
  return launch("pack_transpose", pack_transpose_kernel<TS, int8_t>, grid, dim3(256), 0, s, src, K, N, ld_src,
                (int8_t*)dst, ld_dst);
}

}  // namespace

int pack_transpose(const void* src, int src_dtype, int K, int N, int64_t ld_src, void* dst, int dst_dtype,
                   int64_t ld_dst, hipStream_t s) {
  AFHIP_REQUIRE(src && dst && K > 0 && N > 0, "invalid weight pack arguments");
  AFHIP_REQUIRE(src_dtype != AFHIP_I8 || dst_dtype == AFHIP_I8 || dst_dtype == AFHIP_F16,
                "int8 weights pack to int8 or (exactly) to f16");
  if (src_dtype == AFHIP_F32) return pack_dispatch((const float*)src, K, N, ld_src, dst, dst_dtype, ld_dst, s);
  if (src_dtype == AFHIP_F16) return pack_dispatch((const half_t*)src, K, N, ld_src, dst, dst_dtype, ld_dst, s);
  return pack_dispatch((const int8_t*)src, K, N, ld_src, dst, dst_dtype, ld_dst, s);
}

int convert_f32(const float* src, int64_t count, void* dst, int dst_dtype, hipStream_t s) {
  if (count <= 0) return AFHIP_OK;
  unsigned blocks = (unsigned)std::min<int64_t>(ceil_div(count, 256), 65536);
  if (dst_dtype == AFHIP_F32)
    return launch("convert", convert_kernel<float>, dim3(blocks), dim3(256), 0, s, src, count, (float*)dst);
  return launch("convert", convert_kernel<half_t>, dim3(blocks), dim3(256), 0, s, src, count, (half_t*)dst);
}

// ---------------------------------------------------------------------------
// Selection: pinned > calibrated > heuristic
// ---------------------------------------------------------------------------

namespace {
std::mutex g_select_mutex;
bool g_pinned = false;
afhip_variant g_pin{};
std::map<std::string, afhip_variant> g_calibrated;

int log2_bucket(int64_t v) {
  int b = 0;
  while (v > 1) { v >>= 1; b++; }
  return b;
}
}  // namespace

std::string device_key();

std::string shape_class(const GemmTypes& t, int64_t M, int64_t N, int64_t K, int batch) {
  char key[160];
  snprintf(key, sizeof(key), "p%d.a%d.w%d.c%d.m%d.n%d.k%d.b%d", t.precision, t.a_dtype, t.b_dtype, t.c_dtype,
           log2_bucket(M), log2_bucket(N), log2_bucket(K), log2_bucket(batch));
  return key;
}

afhip_variant select_variant(const GemmTypes& t, int64_t M, int64_t N, int64_t K, int batch) {
  std::lock_guard<std::mutex> lock(g_select_mutex);
  if (g_pinned) {
    afhip_variant v = g_pin;
    v.precision = t.precision;
    v.source = 2;
    // A pinned LDS_DMA or STREAM variant only applies where that family runs.
    if (v.kernel == AFHIP_KERNEL_STREAM) {
      if (stream_shape_ok(t, M, N, K, batch)) return v;
    } else if (v.kernel != AFHIP_KERNEL_LDS_DMA ||
               ((t.a_dtype == AFHIP_F16 || t.a_dtype == AFHIP_F32) && t.b_dtype == AFHIP_F16) ||
               (t.precision == AFHIP_PRECISION_F32 && t.a_dtype == AFHIP_F32 && t.b_dtype == AFHIP_F32)) {
      return v;
    }
  }
  if (!g_calibrated.empty()) {
    auto it = g_calibrated.find(device_key() + "|" + shape_class(t, M, N, K, batch));
    if (it != g_calibrated.end()) return it->second;
  }
  return heuristic_variant(t, M, N, K, batch);
}

void install_calibrated(const std::string& key, const afhip_variant& v) {
  std::lock_guard<std::mutex> lock(g_select_mutex);
  g_calibrated[key] = v;
}

std::map<std::string, afhip_variant> calibrated_snapshot() {
  std::lock_guard<std::mutex> lock(g_select_mutex);
  return g_calibrated;
}

void replace_calibrated(const std::map<std::string, afhip_variant>& m) {
  std::lock_guard<std::mutex> lock(g_select_mutex);
  g_calibrated = m;
}

bool valid_variant(const afhip_variant& v) {
  if (v.tile_inner != gemm_detail::kBK || !valid_precision(v.precision)) return false;
  if (v.kernel == AFHIP_KERNEL_LDS_DMA) return dma_tile_supported(v.tile_rows, v.tile_columns);
  if (v.kernel == AFHIP_KERNEL_STREAM)
    return v.precision == AFHIP_PRECISION_F16 && v.tile_rows == 64 && v.tile_columns == 512;
  return v.kernel == AFHIP_KERNEL_REGISTER_STAGED && (v.tile_rows == 64 || v.tile_rows == 128) &&
         (v.tile_columns == 64 || v.tile_columns == 128);
}

void pin_variant(const afhip_variant* v) {
  std::lock_guard<std::mutex> lock(g_select_mutex);
  g_pinned = v != nullptr;
  if (v) g_pin = *v;
}

// The GemmArgs a run of this description passes its kernels (run_gemm_plan),
// with 256-byte aligned stand-ins for the operand pointers, which nothing
// dereferences: what the description alone decides of a family's operand
// rules. `repacked`: the weight goes through the plan's workspace ([N][K],
// ldb = K).
static GemmArgs desc_args(const afhip_gemm_desc& d, bool repacked) {
  const char* const aligned = reinterpret_cast<const char*>(uintptr_t{256});
  GemmArgs g;
  g.a = g.b = g.residual = aligned;
  g.c = const_cast<char*>(aligned);
  g.M = d.rows;
  g.N = d.columns;
  g.K = d.inner;
  g.batch = d.batch;
  g.lda = d.lda ? d.lda : (d.a_layout == AFHIP_SOURCE_ROW_CONTIGUOUS ? d.rows : d.inner);
  g.ldb = repacked ? d.inner : (d.ldw ? d.ldw : (d.w_layout == AFHIP_WEIGHT_K_CONTIGUOUS ? d.inner : d.columns));
  g.ldc = d.ldc ? d.ldc : (d.c_layout == AFHIP_OUTPUT_COLUMN_MAJOR ? d.rows : d.columns);
  g.sa = d.batch_stride_a;
  g.sb = repacked ? (d.batch_stride_w == 0 ? 0 : (int64_t)d.inner * d.columns) : d.batch_stride_w;
  g.sc = d.batch_stride_c;
  g.a_row_contiguous = d.a_layout == AFHIP_SOURCE_ROW_CONTIGUOUS;
  g.c_column_major = d.c_layout == AFHIP_OUTPUT_COLUMN_MAJOR;
  g.flags = d.epilogue;
  if (d.epilogue & AFHIP_EPILOGUE_ATTENTION) g.head_cols = d.heads * d.head_dim;
  return g;
}

// The variant a description runs with: the selection for its shape class,
// except where the description itself rules that family out (a layout, a
// stride, K or M that STREAM or LDS_DMA does not take), where it is the
// variant the run would fall back to. So the variant names the family that
// runs, unless the operands' own addresses are misaligned, which only the
// run sees (and falls back the same way).
afhip_variant select_plan_variant(const afhip_gemm_desc& d, const GemmTypes& types) {
  // The weight dtype the kernels read: f16 under f16 arithmetic (a
  // column-contiguous weight is converted on its way into the workspace)
  // unless it is int8.
  GemmTypes kt = types;
  if (d.precision == AFHIP_PRECISION_F16 && d.w_dtype != AFHIP_I8) kt.b_dtype = AFHIP_F16;
  afhip_variant v = select_variant(kt, d.rows, d.columns, d.inner, d.batch);
  const int source = v.source;
  const bool column_w = d.w_layout == AFHIP_WEIGHT_COLUMN_CONTIGUOUS;
  if (v.kernel == AFHIP_KERNEL_STREAM && !stream_eligible(desc_args(d, column_w), kt))
    v = tile_variant(kt, d.rows, d.columns, d.inner, d.batch);
  if (v.kernel == AFHIP_KERNEL_LDS_DMA) {
    // LDS_DMA reads an int8 weight widened to f16 in the workspace.
    GemmTypes dt = kt;
    if (dt.b_dtype == AFHIP_I8) dt.b_dtype = AFHIP_F16;
    if (!dma_eligible(desc_args(d, column_w || d.w_dtype == AFHIP_I8), dt) ||
        !dma_tile_supported(v.tile_rows, v.tile_columns))
      v = register_variant(kt.precision, d.rows, d.columns, d.inner, d.batch);
  }
  v.source = source;
  return v;
}

}  // namespace afhip

// ---------------------------------------------------------------------------
// C ABI: plans
// ---------------------------------------------------------------------------

struct afhip_gemm_plan {
  afhip_gemm_desc desc;
  afhip::GemmTypes types;
  afhip_variant variant;
  int64_t lda, ldw, ldc;
};

using namespace afhip;

extern "C" {

int afhip_gemm_grid(int64_t rows, int64_t columns, int32_t tile_columns, int32_t tile_rows, uint32_t out_xy[2]) {
  AFHIP_REQUIRE(out_xy != nullptr, "output is NULL");
  AFHIP_REQUIRE(rows > 0 && columns > 0 && rows <= ((int64_t)1 << 53) && columns <= ((int64_t)1 << 53),
                "GEMM dispatch dimensions must be positive safe integers");
  AFHIP_REQUIRE(tile_columns > 0 && tile_rows > 0, "tile sizes must be positive");
  const int64_t limit = 65535;
  int64_t column_tiles = ceil_div(columns, tile_columns);
  int64_t row_tiles = ceil_div(rows, tile_rows);
  int64_t folds = ceil_div(row_tiles, limit);
  int64_t x = column_tiles * folds, y = row_tiles < limit ? row_tiles : limit;
  AFHIP_REQUIRE(x <= 0xffffffffll, "grid too large");
  out_xy[0] = (uint32_t)x;
  out_xy[1] = (uint32_t)y;
  return AFHIP_OK;
}

static int validate_desc(const afhip_gemm_desc* d) {
  AFHIP_REQUIRE(d != nullptr, "descriptor is NULL");
  AFHIP_REQUIRE(d->rows > 0 && d->inner > 0 && d->columns > 0 && d->batch > 0,
                "GEMM dimensions must be positive (rows=%d inner=%d columns=%d batch=%d)", d->rows, d->inner,
                d->columns, d->batch);
  AFHIP_REQUIRE(valid_precision(d->precision), "unknown precision %d", d->precision);
  AFHIP_REQUIRE(valid_float_dtype(d->a_dtype), "a_dtype must be F32 or F16");
  AFHIP_REQUIRE(valid_float_dtype(d->w_dtype) || d->w_dtype == AFHIP_I8, "w_dtype must be F32, F16 or I8");
  AFHIP_REQUIRE(valid_float_dtype(d->out_dtype), "out_dtype must be F32 or F16");
  AFHIP_REQUIRE(d->w_layout == AFHIP_WEIGHT_COLUMN_CONTIGUOUS || d->w_layout == AFHIP_WEIGHT_K_CONTIGUOUS,
                "unknown weight layout %d", d->w_layout);
  AFHIP_REQUIRE((d->epilogue & ~31u) == 0, "unknown epilogue flags 0x%x", d->epilogue);
  if (d->epilogue & AFHIP_EPILOGUE_ATTENTION)
    AFHIP_REQUIRE(d->heads > 0 && d->head_dim > 0 && d->columns == 4 * d->heads * d->head_dim,
                  "attention epilogue needs columns == 4 * heads * head_dim");
  AFHIP_REQUIRE(!(d->w_dtype == AFHIP_I8 && d->precision == AFHIP_PRECISION_F32),
                "int8 weights need f16 precision");
  AFHIP_REQUIRE(!(d->precision == AFHIP_PRECISION_F32 && d->a_dtype != AFHIP_F32),
                "f32 precision needs an f32 source");
  AFHIP_REQUIRE(!(d->w_layout == AFHIP_WEIGHT_K_CONTIGUOUS && d->w_dtype != AFHIP_I8 &&
                  d->w_dtype != (d->precision == AFHIP_PRECISION_F16 ? AFHIP_F16 : AFHIP_F32)),
                "k-contiguous weights must be given in the precision's dtype (f16 for f16, f32 for f32)");
  AFHIP_REQUIRE(d->a_layout == AFHIP_SOURCE_K_CONTIGUOUS || d->a_layout == AFHIP_SOURCE_ROW_CONTIGUOUS,
                "unknown source layout %d", d->a_layout);
  AFHIP_REQUIRE(d->c_layout == AFHIP_OUTPUT_ROW_MAJOR || d->c_layout == AFHIP_OUTPUT_COLUMN_MAJOR,
                "unknown output layout %d", d->c_layout);
  const int64_t a_run = d->a_layout == AFHIP_SOURCE_ROW_CONTIGUOUS ? d->rows : d->inner;
  const int64_t c_run = d->c_layout == AFHIP_OUTPUT_COLUMN_MAJOR ? d->rows : d->columns;
  int64_t lda = d->lda ? d->lda : a_run;
  int64_t ldw = d->ldw ? d->ldw : (d->w_layout == AFHIP_WEIGHT_K_CONTIGUOUS ? d->inner : d->columns);
  int64_t ldc = d->ldc ? d->ldc : c_run;
  AFHIP_REQUIRE(lda >= a_run, "lda %lld is shorter than a source run of %lld", (long long)lda, (long long)a_run);
  AFHIP_REQUIRE(ldw >= (d->w_layout == AFHIP_WEIGHT_K_CONTIGUOUS ? d->inner : d->columns), "ldw too small");
  AFHIP_REQUIRE(ldc >= c_run, "ldc %lld is shorter than an output run of %lld", (long long)ldc, (long long)c_run);
  if (d->batch > 1)
    AFHIP_REQUIRE(d->batch_stride_a >= 0 && d->batch_stride_w >= 0 && d->batch_stride_c > 0,
                  "batched GEMM needs batch strides");
  return AFHIP_OK;
}

int afhip_gemm_plan_create(const afhip_gemm_desc* desc, afhip_gemm_plan** out) {
  if (int s = validate_desc(desc)) return s;
  AFHIP_REQUIRE(out != nullptr, "output pointer is NULL");
  auto* p = new (std::nothrow) afhip_gemm_plan;
  if (!p) return set_error(AFHIP_ERR_OUT_OF_MEMORY, "plan allocation failed");
  p->desc = *desc;
  p->types = {desc->precision, desc->a_dtype, desc->w_dtype, desc->out_dtype};
  p->lda = desc->lda ? desc->lda : (desc->a_layout == AFHIP_SOURCE_ROW_CONTIGUOUS ? desc->rows : desc->inner);
  p->ldw = desc->ldw ? desc->ldw : (desc->w_layout == AFHIP_WEIGHT_K_CONTIGUOUS ? desc->inner : desc->columns);
  p->ldc = desc->ldc ? desc->ldc : (desc->c_layout == AFHIP_OUTPUT_COLUMN_MAJOR ? desc->rows : desc->columns);
  p->variant = select_plan_variant(*desc, p->types);
  *out = p;
  return AFHIP_OK;
}

int afhip_gemm_plan_destroy(afhip_gemm_plan* plan) {
  delete plan;
  return AFHIP_OK;
}

// The weight dtype the kernels read for a precision: f16 (or int8) under f16
// arithmetic, f32 under f32 arithmetic. An int8 weight stays int8 for the
// families that widen it themselves (STREAM, REGISTER_STAGED) and is widened
// to f16 (exactly) for LDS_DMA, whose stages take f16 rows; the per-column
// scale is applied to the f32 accumulator either way.
static int kernel_w_dtype(const afhip_gemm_plan& p) {
  const auto& d = p.desc;
  if (d.precision != AFHIP_PRECISION_F16) return AFHIP_F32;
  if (d.w_dtype != AFHIP_I8) return AFHIP_F16;
  return p.variant.kernel == AFHIP_KERNEL_LDS_DMA ? AFHIP_F16 : AFHIP_I8;
}

// A column-contiguous weight is rewritten per run (transposed, and converted
// to the kernel's dtype on the way); a k-contiguous one must already be in
// that dtype, which plan creation checks, except an int8 one widened for
// LDS_DMA.
static bool needs_weight_workspace(const afhip_gemm_plan& p) {
  return p.desc.w_layout == AFHIP_WEIGHT_COLUMN_CONTIGUOUS || kernel_w_dtype(p) != p.desc.w_dtype;
}

int afhip_gemm_workspace_size(const afhip_gemm_plan* plan, size_t* bytes) {
  AFHIP_REQUIRE(plan && bytes, "NULL plan or output");
  const auto& d = plan->desc;
  if (needs_weight_workspace(*plan)) {
    size_t one = (size_t)d.inner * d.columns * dtype_size(kernel_w_dtype(*plan));
    size_t n = d.batch_stride_w == 0 ? 1 : (size_t)d.batch;
    *bytes = round_up((int64_t)(one * n), 256);
  } else {
    *bytes = 0;
  }
  return AFHIP_OK;
}

int afhip_gemm_run(const afhip_gemm_plan* plan, const void* a, const void* w, const float* scale, const float* bias,
                   const void* residual, void* c, void* workspace, size_t workspace_bytes, void* stream) {
  if (int s = require_open()) return s;
  return afhip::run_gemm_plan(plan, a, w, scale, bias, residual, c, workspace, workspace_bytes, stream);
}

}  // extern "C"

// The body of afhip_gemm_run, shared with the entry point that brings its own
// workspace (gemm_static.hip).
int afhip::run_gemm_plan(const afhip_gemm_plan* plan, const void* a, const void* w, const float* scale,
                         const float* bias, const void* residual, void* c, void* workspace, size_t workspace_bytes,
                         void* stream) {
  AFHIP_REQUIRE(plan != nullptr, "plan is NULL");
  const auto& d = plan->desc;
  hipStream_t st = (hipStream_t)stream;
  GemmArgs g;
  g.a = a;
  g.b = w;
  g.c = c;
  g.residual = residual;
  g.scale = scale;
  g.bias = bias;
  g.M = d.rows;
  g.N = d.columns;
  g.K = d.inner;
  g.lda = plan->lda;
  g.ldb = plan->ldw;
  g.ldc = plan->ldc;
  g.sa = d.batch_stride_a;
  g.sb = d.batch_stride_w;
  g.sc = d.batch_stride_c;
  g.batch = d.batch;
  g.a_row_contiguous = d.a_layout == AFHIP_SOURCE_ROW_CONTIGUOUS;
  g.c_column_major = d.c_layout == AFHIP_OUTPUT_COLUMN_MAJOR;
  g.flags = d.epilogue;
  if (d.epilogue & AFHIP_EPILOGUE_ATTENTION) {
    g.head_cols = d.heads * d.head_dim;
    g.q_scale = (float)(1.0 / std::sqrt((double)d.head_dim));
  }
  GemmTypes types = plan->types;
  if (needs_weight_workspace(*plan)) {
    size_t need = 0;
    afhip_gemm_workspace_size(plan, &need);
    AFHIP_REQUIRE(workspace != nullptr && workspace_bytes >= need,
                  "these weights need a %zu-byte workspace to be laid out for the kernel", need);
    AFHIP_REQUIRE(w != nullptr, "weight is NULL");
    const int kd = kernel_w_dtype(*plan);
    int nb = d.batch_stride_w == 0 ? 1 : d.batch;
    size_t es = dtype_size(d.w_dtype), kes = dtype_size(kd);
    for (int b = 0; b < nb; b++) {
      const char* src = (const char*)w + (size_t)b * d.batch_stride_w * es;
      char* dst = (char*)workspace + (size_t)b * d.inner * d.columns * kes;
      if (d.w_layout == AFHIP_WEIGHT_COLUMN_CONTIGUOUS) {
        if (int s = pack_transpose(src, d.w_dtype, d.inner, d.columns, plan->ldw, dst, kd, d.inner, st)) return s;
      } else {
        // A k-contiguous int8 weight [N][K], widened in place of the layout.
        const dim3 grid((unsigned)ceil_div(d.inner, 8 * 256), (unsigned)std::min(d.columns, 65535));
        if (int s = launch("widen_int8", widen_rows_kernel, grid, dim3(256), 0, st, (const int8_t*)src, d.columns,
                           d.inner, plan->ldw, (half_t*)dst))
          return s;
      }
    }
    g.b = workspace;
    g.ldb = d.inner;
    g.sb = d.batch_stride_w == 0 ? 0 : (int64_t)d.inner * d.columns;
    types.b_dtype = kd;
  }
  return run_gemm(g, types, plan->variant, "gemm", st);
}

extern "C" {

int afhip_pack_weight(const void* src, int32_t src_dtype, int32_t rows_k, int32_t columns_n, void* dst,
                      int32_t dst_dtype, void* stream) {
  if (int s = require_open()) return s;
  return pack_transpose(src, src_dtype, rows_k, columns_n, columns_n, dst, dst_dtype, rows_k, (hipStream_t)stream);
}

int afhip_dequant_q8_channel(const int8_t* q, const float* scale, int32_t rows_k, int32_t columns_n, float* out,
                             void* stream) {
  if (int s = require_open()) return s;
  AFHIP_REQUIRE(q && scale && out && rows_k > 0 && columns_n > 0, "invalid dequantisation arguments");
  int64_t total = (int64_t)rows_k * columns_n;
  return launch("dequant_q8_channel", dequant_channel_kernel, dim3((unsigned)ceil_div(total, 256)), dim3(256), 0,
                (hipStream_t)stream, q, scale, rows_k, columns_n, out);
}

int afhip_dequant_q8_block(const int8_t* codes, const uint16_t* scales_f16, int32_t block, int64_t start, int64_t count,
                           float* out, void* stream) {
  if (int s = require_open()) return s;
  AFHIP_REQUIRE(codes && scales_f16 && out, "NULL argument");
  AFHIP_REQUIRE(block > 0, "int8 tensor has an invalid block size");
  AFHIP_REQUIRE(start >= 0 && count >= 0, "tensor range is out of bounds");
  if (count == 0) return AFHIP_OK;
  return launch("dequant_q8_block", dequant_block_kernel, dim3((unsigned)ceil_div(count, 256)), dim3(256), 0,
                (hipStream_t)stream, codes, scales_f16, block, start, count, out);
}

int afhip_pack_weight_q8_block(const int8_t* codes, const uint16_t* scales_f16, int32_t block, int64_t start,
                               int32_t rows_k, int32_t columns_n, void* dst, int32_t dst_dtype, void* stream) {
  if (int s = require_open()) return s;
  AFHIP_REQUIRE(codes && scales_f16 && dst, "NULL argument");
  AFHIP_REQUIRE(block > 0, "int8 tensor has an invalid block size");
  AFHIP_REQUIRE(start >= 0, "tensor range is out of bounds");
  AFHIP_REQUIRE(rows_k > 0 && columns_n > 0, "weight dimensions must be positive");
  AFHIP_REQUIRE(rows_k <= 65535 * 32, "weight has too many rows");
  AFHIP_REQUIRE(dst_dtype == AFHIP_F32 || dst_dtype == AFHIP_F16, "packed q8 weights decode to f32 or f16");
  const dim3 grid((unsigned)ceil_div(columns_n, 32), (unsigned)ceil_div(rows_k, 32));
  if (dst_dtype == AFHIP_F32)
    return launch("pack_q8_block", pack_q8_block_kernel<float>, grid, dim3(256), 0, (hipStream_t)stream, codes,
                  scales_f16, block, start, rows_k, columns_n, (float*)dst);
  return launch("pack_q8_block", pack_q8_block_kernel<half_t>, grid, dim3(256), 0, (hipStream_t)stream, codes,
                scales_f16, block, start, rows_k, columns_n, (half_t*)dst);
}

}  // extern "C"
