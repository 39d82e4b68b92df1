// The tiled GEMM kernel template, instantiated per operand type in the
// gemm_inst_*.hip translation units (so a parallel build compiles them
// side by side). See gemm.hip for the design.
#pragma once

#include <type_traits>

#include "gemm.h"

namespace afhip {
namespace gemm_detail {
constexpr int kThreads = 256;
constexpr int kBK = 32;

template <typename T> struct Vec16 { static constexpr int n = 16 / sizeof(T); };

struct KernelArgs {
  GemmArgs g;
  int tiles_m, tiles_n, total_tiles, per_xcd;
};

template <typename CT> struct LdsPitch;
template <> struct LdsPitch<half_t> { static constexpr int value = kBK + 8; };  // 80-byte rows, 16-byte aligned
template <> struct LdsPitch<float> { static constexpr int value = kBK + 1; };   // odd word pitch: conflict-free columns

// Loads `count` consecutive elements starting at (row, k) of a row-major
// operand into CT registers, zero-filling outside [0, rows) x [0, K).
template <typename T, typename CT, bool VEC>
__device__ __forceinline__ void load_chunk(const T* __restrict__ base, int64_t ld, int row, int k, int rows, int K,
                                           CT* out) {
  constexpr int n = Vec16<T>::n;
  if (VEC) {
    if (row < rows && k < K) {
      const T* p = base + (int64_t)row * ld + k;
      T tmp[n];
      *reinterpret_cast<uint4*>(tmp) = *reinterpret_cast<const uint4*>(p);
#pragma unroll
      for (int e = 0; e < n; e++) out[e] = (CT)(float)tmp[e];
    } else {
#pragma unroll
      for (int e = 0; e < n; e++) out[e] = (CT)0.0f;
    }
  } else {
#pragma unroll
    for (int e = 0; e < n; e++) {
      bool ok = row < rows && (k + e) < K;
      out[e] = ok ? (CT)(float)base[(int64_t)row * ld + k + e] : (CT)0.0f;
    }
  }
}

template <> __device__ __forceinline__ void load_chunk<int8_t, half_t, true>(const int8_t* __restrict__ base,
                                                                            int64_t ld, int row, int k, int rows,
                                                                            int K, half_t* out) {
  if (row < rows && k < K) {
    int8_t tmp[16];
    *reinterpret_cast<uint4*>(tmp) = *reinterpret_cast<const uint4*>(base + (int64_t)row * ld + k);
#pragma unroll
    for (int e = 0; e < 16; e++) out[e] = (half_t)(int)tmp[e];
  } else {
#pragma unroll
    for (int e = 0; e < 16; e++) out[e] = (half_t)0.0f;
  }
}

template <typename T, typename CT, int ROWS, bool VEC> struct TileLoader {
  static constexpr int n = Vec16<T>::n;
  static constexpr int per_row = kBK / n;
  static constexpr int chunks = ROWS * per_row;
  static constexpr int iters = (chunks + kThreads - 1) / kThreads;
  CT regs[iters][n];

  __device__ __forceinline__ void load(const T* __restrict__ base, int64_t ld, int row0, int k0, int rows, int K,
                                       int tid) {
#pragma unroll
    for (int it = 0; it < iters; it++) {
      int q = tid + it * kThreads;
      if (chunks % kThreads == 0 || q < chunks) {
        int r = q / per_row;
        int kc = (q % per_row) * n;
        load_chunk<T, CT, VEC>(base, ld, row0 + r, k0 + kc, rows, K, regs[it]);
      }
    }
  }

  __device__ __forceinline__ void store(CT* __restrict__ lds, int tid) {
    constexpr int pitch = LdsPitch<CT>::value;
#pragma unroll
    for (int it = 0; it < iters; it++) {
      int q = tid + it * kThreads;
      if (chunks % kThreads == 0 || q < chunks) {
        int r = q / per_row;
        int kc = (q % per_row) * n;
        CT* dst = lds + r * pitch + kc;
        if constexpr (sizeof(CT) == 2) {
#pragma unroll
          for (int e = 0; e < n; e += 8 < n ? 8 : n) {
            if constexpr (n >= 8) {
              *reinterpret_cast<half8*>(dst + e) = *reinterpret_cast<const half8*>(&regs[it][e]);
            } else {
              *reinterpret_cast<half4*>(dst + e) = *reinterpret_cast<const half4*>(&regs[it][e]);
            }
          }
        } else {
#pragma unroll
          for (int e = 0; e < n; e++) dst[e] = regs[it][e];
        }
      }
    }
  }
};

// The same LDS tile from an operand stored k-major, [k][row] at
// base + k * ld + row (the reference's sourceContiguous "row",
// GemmOperandArray.columnMajor, src/runtime/gemm.ts:321, :341-360). A lane
// takes `n` consecutive rows at two consecutive k: two 16-byte loads along
// the rows, then one LDS word (f16) or two (f32) per row holding the pair of
// k values, so the tile lands k-contiguous as TileLoader leaves it and the
// MFMA fragments read it the same way.
template <typename T, typename CT, bool VEC>
__device__ __forceinline__ void load_rows(const T* __restrict__ base, int64_t ld, int row, int k, int rows, int K,
                                          CT* out) {
  constexpr int n = Vec16<T>::n;
  if (k >= K) {
#pragma unroll
    for (int e = 0; e < n; e++) out[e] = (CT)0.0f;
    return;
  }
  const T* p = base + (int64_t)k * ld + row;
  if (VEC && row + n <= rows) {
    T tmp[n];
    *reinterpret_cast<uint4*>(tmp) = *reinterpret_cast<const uint4*>(p);
#pragma unroll
    for (int e = 0; e < n; e++) out[e] = (CT)(float)tmp[e];
  } else {
#pragma unroll
    for (int e = 0; e < n; e++) out[e] = row + e < rows ? (CT)(float)p[e] : (CT)0.0f;
  }
}

template <typename T, typename CT, int ROWS, bool VEC> struct TileLoaderKMajor {
  static constexpr int n = Vec16<T>::n;
  static constexpr int kpairs = kBK / 2;
  static constexpr int chunks = (ROWS / n) * kpairs;
  static constexpr int iters = (chunks + kThreads - 1) / kThreads;
  CT regs[iters][2][n];

  __device__ __forceinline__ void load(const T* __restrict__ base, int64_t ld, int row0, int k0, int rows, int K,
                                       int tid) {
#pragma unroll
    for (int it = 0; it < iters; it++) {
      const int q = tid + it * kThreads;
      if (chunks % kThreads == 0 || q < chunks) {
        const int kp = q % kpairs, rc = q / kpairs;
        load_rows<T, CT, VEC>(base, ld, row0 + rc * n, k0 + 2 * kp, rows, K, regs[it][0]);
        load_rows<T, CT, VEC>(base, ld, row0 + rc * n, k0 + 2 * kp + 1, rows, K, regs[it][1]);
      }
    }
  }

  __device__ __forceinline__ void store(CT* __restrict__ lds, int tid) {
    constexpr int pitch = LdsPitch<CT>::value;
#pragma unroll
    for (int it = 0; it < iters; it++) {
      const int q = tid + it * kThreads;
      if (chunks % kThreads == 0 || q < chunks) {
        const int kp = q % kpairs, rc = q / kpairs;
#pragma unroll
        for (int e = 0; e < n; e++) {
          CT* dst = lds + (rc * n + e) * pitch + 2 * kp;
          if constexpr (sizeof(CT) == 2) {
            half2v v;
            v[0] = regs[it][0][e];
            v[1] = regs[it][1][e];
            *reinterpret_cast<half2v*>(dst) = v;
          } else {
            dst[0] = regs[it][0][e];
            dst[1] = regs[it][1][e];
          }
        }
      }
    }
  }
};

template <typename TC>
__device__ __forceinline__ void epilogue_store(const GemmArgs& g, int b, int row, int col, float y) {
  // Every operation rounds on its own (no fused multiply-add), so each kernel
  // family applying these steps in this order gives the same bits.
#pragma clang fp contract(off)
  uint32_t flags = g.flags;
  if (flags & AFHIP_EPILOGUE_SCALE) y *= g.scale[col];
  if (flags & AFHIP_EPILOGUE_BIAS) y += g.bias[col];
  if (flags & EPILOGUE_OPM_OUTPUT) y += g.bias[col] / (g.opm_eps + g.opm_count[(int64_t)g.opm_row0 + row]);
  if (flags & AFHIP_EPILOGUE_ATTENTION) {
    int block = col / g.head_cols;
    if (block == 0) y *= g.q_scale;
    else if (block == 3) y = sigmoidf_(y);
  }
  if (flags & AFHIP_EPILOGUE_RELU) y = fmaxf(y, 0.0f);
  if (flags & EPILOGUE_OPM_CONTRACT) {
    // row = i_local * c_outer + a, col = j * c_outer + b
    int co = g.opm_outer;
    int il = row / co, a = row - il * co;
    int j = col / co, bb = col - j * co;
    int i = g.opm_row0 + il;
    y = y / (g.opm_eps + g.opm_count[(int64_t)i * g.opm_length + j]);
    int64_t at = (((int64_t)il * g.opm_length + j) * co + a) * co + bb;
    reinterpret_cast<TC*>(g.c)[at] = (TC)y;
    return;
  }
  const int64_t at = (int64_t)b * g.sc + (g.c_column_major ? (int64_t)col * g.ldc + row : (int64_t)row * g.ldc + col);
  if (flags & AFHIP_EPILOGUE_RESIDUAL) y += (float)reinterpret_cast<const TC*>(g.residual)[at];
  reinterpret_cast<TC*>(g.c)[at] = (TC)y;
}

// Epilogue flags that act on one output row elementwise (everything but
// ATTENTION, whose column blocks differ, and OPM_CONTRACT, which scatters).
constexpr uint32_t kRowwiseEpilogue = AFHIP_EPILOGUE_SCALE | AFHIP_EPILOGUE_BIAS | AFHIP_EPILOGUE_RELU |
                                      AFHIP_EPILOGUE_RESIDUAL | EPILOGUE_OPM_OUTPUT;

// epilogue_store for `n` (<= 4) consecutive columns of one row, the same
// steps in the same order with the same roundings, written with one vector
// access when `vec` (all four columns present, row start and ldc aligned to
// four elements).
template <typename TC>
__device__ __forceinline__ void epilogue_row4(const GemmArgs& g, int b, int row, int col, float* y, int n, bool vec) {
#pragma clang fp contract(off)
  const uint32_t flags = g.flags;
  float denom = 0.0f;
  if (flags & EPILOGUE_OPM_OUTPUT) denom = g.opm_eps + g.opm_count[(int64_t)g.opm_row0 + row];
#pragma unroll
  for (int e = 0; e < 4; e++) {
    if (e >= n) break;
    if (flags & AFHIP_EPILOGUE_SCALE) y[e] *= g.scale[col + e];
    if (flags & AFHIP_EPILOGUE_BIAS) y[e] += g.bias[col + e];
    if (flags & EPILOGUE_OPM_OUTPUT) y[e] += g.bias[col + e] / denom;
    if (flags & AFHIP_EPILOGUE_RELU) y[e] = fmaxf(y[e], 0.0f);
  }
  const int64_t at = (int64_t)b * g.sc + (int64_t)row * g.ldc + col;
  TC* c = reinterpret_cast<TC*>(g.c) + at;
  if (vec && n == 4) {
    typedef TC tc4 __attribute__((ext_vector_type(4)));
    tc4 v;
    if (flags & AFHIP_EPILOGUE_RESIDUAL) {
      const tc4 r = *reinterpret_cast<const tc4*>(reinterpret_cast<const TC*>(g.residual) + at);
#pragma unroll
      for (int e = 0; e < 4; e++) y[e] += (float)r[e];
    }
#pragma unroll
    for (int e = 0; e < 4; e++) v[e] = (TC)y[e];
    *reinterpret_cast<tc4*>(c) = v;
    return;
  }
  for (int e = 0; e < n; e++) {
    if (flags & AFHIP_EPILOGUE_RESIDUAL) y[e] += (float)reinterpret_cast<const TC*>(g.residual)[at + e];
    c[e] = (TC)y[e];
  }
}

template <int BM, int BN, bool F16MATH, typename TA, typename TB, typename TC, bool VEC, bool AKMAJOR>
__global__ __launch_bounds__(kThreads) void gemm_kernel(KernelArgs ka) {
  using CT = typename std::conditional<F16MATH, half_t, float>::type;
  constexpr int pitch = LdsPitch<CT>::value;
  constexpr int WTM = BM / 2, WTN = BN / 2;
  constexpr int TM = WTM / 32, TN = WTN / 32;
  __shared__ __attribute__((aligned(16))) CT As[2][BM * pitch];
  __shared__ __attribute__((aligned(16))) CT Bs[2][BN * pitch];

  const GemmArgs& g = ka.g;
  const int id = blockIdx.x;
  const int t = (id & 7) * ka.per_xcd + (id >> 3);
  if (t >= ka.total_tiles) return;
  const int per_batch = ka.tiles_m * ka.tiles_n;
  const int b = t / per_batch;
  const int r = t - b * per_batch;
  const int m0 = (r / ka.tiles_n) * BM;
  const int n0 = (r % ka.tiles_n) * BN;

  const TA* A = reinterpret_cast<const TA*>(g.a) + (int64_t)b * g.sa;
  const TB* B = reinterpret_cast<const TB*>(g.b) + (int64_t)b * g.sb;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = (wave >> 1) * WTM;
  const int wn = (wave & 1) * WTN;

  typename std::conditional<AKMAJOR, TileLoaderKMajor<TA, CT, BM, VEC>, TileLoader<TA, CT, BM, VEC>>::type la;
  TileLoader<TB, CT, BN, VEC> lb;

  floatx16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; i++)
#pragma unroll
    for (int j = 0; j < TN; j++)
#pragma unroll
      for (int v = 0; v < 16; v++) acc[i][j][v] = 0.0f;

  const int ksteps = (g.K + kBK - 1) / kBK;
  la.load(A, g.lda, m0, 0, g.M, g.K, tid);
  lb.load(B, g.ldb, n0, 0, g.N, g.K, tid);
  la.store(As[0], tid);
  lb.store(Bs[0], tid);
  __syncthreads();

  for (int ks = 0; ks < ksteps; ks++) {
    const int cur = ks & 1;
    const bool more = ks + 1 < ksteps;
    if (more) {
      la.load(A, g.lda, m0, (ks + 1) * kBK, g.M, g.K, tid);
      lb.load(B, g.ldb, n0, (ks + 1) * kBK, g.N, g.K, tid);
    }
    const CT* as = As[cur];
    const CT* bs = Bs[cur];
    if constexpr (F16MATH) {
#pragma unroll
      for (int kk = 0; kk < kBK / 16; kk++) {
        half8 af[TM], bf[TN];
        const int koff = kk * 16 + 8 * (lane >> 5);
#pragma unroll
        for (int i = 0; i < TM; i++)
          af[i] = *reinterpret_cast<const half8*>(as + (wm + 32 * i + (lane & 31)) * pitch + koff);
#pragma unroll
        for (int j = 0; j < TN; j++)
          bf[j] = *reinterpret_cast<const half8*>(bs + (wn + 32 * j + (lane & 31)) * pitch + koff);
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
          for (int j = 0; j < TN; j++) acc[i][j] = mfma_f16(af[i], bf[j], acc[i][j]);
      }
    } else {
#pragma unroll
      for (int kk = 0; kk < kBK / 2; kk++) {
        // MFMA kk of a step takes k = 16 (kk / 8) + kk % 8 from lanes 0-31
        // and that + 8 from lanes 32-63, so each lane's 8 consecutive k of a
        // half-step are one contiguous run, the order the LDS_DMA kernel's f32
        // stages read them in (the two families give the same bits).
        float af[TM], bf[TN];
        const int koff = 16 * (kk >> 3) + 8 * (lane >> 5) + (kk & 7);
#pragma unroll
        for (int i = 0; i < TM; i++) af[i] = as[(wm + 32 * i + (lane & 31)) * pitch + koff];
#pragma unroll
        for (int j = 0; j < TN; j++) bf[j] = bs[(wn + 32 * j + (lane & 31)) * pitch + koff];
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
          for (int j = 0; j < TN; j++) acc[i][j] = mfma_f32(af[i], bf[j], acc[i][j]);
      }
    }
    if (more) {
      la.store(As[cur ^ 1], tid);
      lb.store(Bs[cur ^ 1], tid);
    }
    __syncthreads();
  }

  if ((g.flags & ~(AFHIP_EPILOGUE_SCALE | AFHIP_EPILOGUE_BIAS | AFHIP_EPILOGUE_RELU | AFHIP_EPILOGUE_RESIDUAL)) == 0) {
    // Scale, bias, ReLU and residual only: epilogue_store's steps in its
    // order, with every global read issued before the stores it would
    // otherwise wait behind (the output may alias the residual and, as far
    // as the compiler knows, the scale and bias, so it keeps such a read
    // after any earlier store: one memory round trip per element). A lane's
    // column is fixed per 32 x 32 tile, so its scale and bias are read once;
    // the tile's residual values are read before its first store, and a
    // lane reads only the elements it later writes.
#pragma clang fp contract(off)
    const uint32_t flags = g.flags;
    float sc_[TN], bi_[TN];
#pragma unroll
    for (int j = 0; j < TN; j++) {
      const int col = n0 + wn + 32 * j + (lane & 31);
      sc_[j] = (flags & AFHIP_EPILOGUE_SCALE) && col < g.N ? g.scale[col] : 1.0f;
      bi_[j] = (flags & AFHIP_EPILOGUE_BIAS) && col < g.N ? g.bias[col] : 0.0f;
    }
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
      for (int j = 0; j < TN; j++) {
        const int col = n0 + wn + 32 * j + (lane & 31);
        if (col >= g.N) continue;
        auto at_of = [&](int row) {
          return (int64_t)b * g.sc + (g.c_column_major ? (int64_t)col * g.ldc + row : (int64_t)row * g.ldc + col);
        };
        float r[16];
        if (flags & AFHIP_EPILOGUE_RESIDUAL) {
#pragma unroll
          for (int v = 0; v < 16; v++) {
            const int row = m0 + wm + 32 * i + mfma_row(v, lane);
            r[v] = row < g.M ? (float)reinterpret_cast<const TC*>(g.residual)[at_of(row)] : 0.0f;
          }
        }
#pragma unroll
        for (int v = 0; v < 16; v++) {
          const int row = m0 + wm + 32 * i + mfma_row(v, lane);
          if (row >= g.M) continue;
          float y = acc[i][j][v];
          if (flags & AFHIP_EPILOGUE_SCALE) y *= sc_[j];
          if (flags & AFHIP_EPILOGUE_BIAS) y += bi_[j];
          if (flags & AFHIP_EPILOGUE_RELU) y = fmaxf(y, 0.0f);
          if (flags & AFHIP_EPILOGUE_RESIDUAL) y += r[v];
          reinterpret_cast<TC*>(g.c)[at_of(row)] = (TC)y;
        }
      }
    return;
  }
#pragma unroll
  for (int i = 0; i < TM; i++)
#pragma unroll
    for (int j = 0; j < TN; j++) {
      const int col = n0 + wn + 32 * j + (lane & 31);
      if (col >= g.N) continue;
#pragma unroll
      for (int v = 0; v < 16; v++) {
        const int row = m0 + wm + 32 * i + mfma_row(v, lane);
        if (row < g.M) epilogue_store<TC>(g, b, row, col, acc[i][j][v]);
      }
    }
}

template <int BM, int BN, bool F16MATH, typename TA, typename TB, typename TC>
int launch_tiles(const GemmArgs& g, bool vec, const char* label, hipStream_t stream) {
  KernelArgs ka;
  ka.g = g;
  ka.tiles_m = (int)ceil_div(g.M, BM);
  ka.tiles_n = (int)ceil_div(g.N, BN);
  int64_t total = (int64_t)ka.tiles_m * ka.tiles_n * g.batch;
  if (total > (int64_t)1 << 30) return set_error(AFHIP_ERR_INVALID_ARGUMENT, "GEMM has too many tiles");
  ka.total_tiles = (int)total;
  ka.per_xcd = (int)ceil_div(total, 8);
  dim3 grid((unsigned)(ka.per_xcd * 8));
  if (g.a_row_contiguous) {
    if (vec)
      return launch(label, gemm_kernel<BM, BN, F16MATH, TA, TB, TC, true, true>, grid, dim3(kThreads), 0, stream, ka);
    return launch(label, gemm_kernel<BM, BN, F16MATH, TA, TB, TC, false, true>, grid, dim3(kThreads), 0, stream, ka);
  }
  if (vec) return launch(label, gemm_kernel<BM, BN, F16MATH, TA, TB, TC, true, false>, grid, dim3(kThreads), 0, stream, ka);
  return launch(label, gemm_kernel<BM, BN, F16MATH, TA, TB, TC, false, false>, grid, dim3(kThreads), 0, stream, ka);
}

template <bool F16MATH, typename TA, typename TB, typename TC>
int launch_variant(const GemmArgs& g, const afhip_variant& v, bool vec, const char* label, hipStream_t stream) {
  if (v.tile_rows == 128 && v.tile_columns == 128) return launch_tiles<128, 128, F16MATH, TA, TB, TC>(g, vec, label, stream);
  if (v.tile_rows == 64 && v.tile_columns == 128) return launch_tiles<64, 128, F16MATH, TA, TB, TC>(g, vec, label, stream);
  if (v.tile_rows == 128 && v.tile_columns == 64) return launch_tiles<128, 64, F16MATH, TA, TB, TC>(g, vec, label, stream);
  if (v.tile_rows == 64 && v.tile_columns == 64) return launch_tiles<64, 64, F16MATH, TA, TB, TC>(g, vec, label, stream);
  return set_error(AFHIP_ERR_INVALID_ARGUMENT, "unsupported GEMM tile %dx%d", v.tile_rows, v.tile_columns);
}

template <bool F16MATH, typename TA, typename TB>
int dispatch_c(const GemmArgs& g, const GemmTypes& t, const afhip_variant& v, bool vec, const char* label,
               hipStream_t s) {
  if (t.c_dtype == AFHIP_F32) return launch_variant<F16MATH, TA, TB, float>(g, v, vec, label, s);
  return launch_variant<F16MATH, TA, TB, half_t>(g, v, vec, label, s);
}

template <typename TA>
int dispatch_b_f16(const GemmArgs& g, const GemmTypes& t, const afhip_variant& v, bool vec, const char* label,
                   hipStream_t s) {
  if (t.b_dtype == AFHIP_F16) return dispatch_c<true, TA, half_t>(g, t, v, vec, label, s);
  return dispatch_c<true, TA, int8_t>(g, t, v, vec, label, s);
}


}  // namespace gemm_detail

// Entry points of the instantiation units.
int gemm_dispatch_f16_a32(const GemmArgs& g, const GemmTypes& t, const afhip_variant& v, bool vec, const char* label,
                          hipStream_t s);
int gemm_dispatch_f16_a16(const GemmArgs& g, const GemmTypes& t, const afhip_variant& v, bool vec, const char* label,
                          hipStream_t s);
int gemm_dispatch_f32(const GemmArgs& g, const GemmTypes& t, const afhip_variant& v, bool vec, const char* label,
                      hipStream_t s);

}  // namespace afhip
