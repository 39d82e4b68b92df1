// The shared tiled GEMM, as the other translation units launch it.
#pragma once

#include "internal.h"

namespace afhip {

// One batched GEMM launch: C[b][m][n] = epilogue(sum_k A[b][m][k] * B[b][n][k]).
// A is row-major [M][K] (row stride lda), or [K][M] when a_row_contiguous
// (element (m, k) at k * lda + m); B is [N][K] (row stride ldb), the
// k-contiguous layout every kernel here consumes. C is [M][N] (row stride
// ldc), or [N][M] when c_column_major (element (m, n) at n * ldc + m).
struct GemmArgs {
  const void* a = nullptr;
  const void* b = nullptr;
  void* c = nullptr;
  const void* residual = nullptr;
  const float* scale = nullptr;
  const float* bias = nullptr;
  int M = 0, N = 0, K = 0;
  int64_t lda = 0, ldb = 0, ldc = 0;
  int64_t sa = 0, sb = 0, sc = 0;
  int batch = 1;
  bool a_row_contiguous = false;  // the REGISTER_STAGED and LDS_DMA kernels take it
  bool c_column_major = false;    // the REGISTER_STAGED and LDS_DMA kernels take it
  uint32_t flags = 0;
  int head_cols = 0;  // heads * head_dim, ATTENTION only
  float q_scale = 1.0f;
  // Outer-product-mean contraction epilogue: y /= (eps + count[i][j]) with
  // i = (row0 + m) / c_outer, j = n / c_outer; stored at the [i][j][a][b] layout.
  const float* opm_count = nullptr;
  int opm_outer = 0;
  int opm_length = 0;
  int opm_row0 = 0;
  float opm_eps = 0.0f;
  // The fused contraction + output projection (run_opm_fused) only: the
  // output weights in the order opm_fused_weight_index gives.
  const void* opm_w = nullptr;
};

// Epilogue flags private to the library (beyond the public AFHIP_EPILOGUE_*).
// OPM_CONTRACT: y /= (eps + count[i][j]), stored at [i_local][j][a][b].
// OPM_OUTPUT:   y += bias[col] / (eps + count[opm_row0 + row]) (bias scaled by
//               the pair's 1/(eps + count), outer-product-mean.ts:462-479).
constexpr uint32_t EPILOGUE_OPM_CONTRACT = 1u << 16;
constexpr uint32_t EPILOGUE_OPM_OUTPUT = 1u << 17;

struct GemmTypes {
  int precision;  // AFHIP_PRECISION_*
  int a_dtype;    // AFHIP_F32 | AFHIP_F16
  int b_dtype;    // AFHIP_F32 | AFHIP_F16 | AFHIP_I8
  int c_dtype;    // AFHIP_F32 | AFHIP_F16
};

// Runs one GEMM with the given variant (tile shape); the variant's
// vectorized flag is ignored and derived from alignment.
int run_gemm(const GemmArgs& args, const GemmTypes& types, const afhip_variant& variant, const char* label,
             hipStream_t stream);

// Heuristic kernel and tile choice for a problem of these types and size.
afhip_variant heuristic_variant(const GemmTypes& types, int64_t M, int64_t N, int64_t K, int batch);
// The REGISTER_STAGED variant for a shape: what takes every operand form.
afhip_variant register_variant(int precision, int64_t M, int64_t N, int64_t K, int batch);

// The LDS_DMA kernel family (gemm_dma.hip): f16 arithmetic on an f16 or f32
// A and an f16 B (k-contiguous), or f32 arithmetic on f32 operands.
bool dma_tile_supported(int tile_m, int tile_n);
bool dma_eligible(const GemmArgs& args, const GemmTypes& types);
void dma_heuristic_tile(int64_t M, int64_t N, int64_t K, int64_t batch, int* tile_m, int* tile_n);
int run_gemm_dma(const GemmArgs& args, const GemmTypes& types, int tile_m, int tile_n, const char* label,
                 hipStream_t stream);

// The outer-product mean's contraction and output projection in one launch
// (gemm_dma.hip), for f16 arithmetic with c_outer = 32 and c_z in (96, 128]:
// A = left [L * 32][K], B = right [L * 32][K] (rows i * 32 + a, k-contiguous,
// row stride lda = ldb), count [L][L], opm_w the permuted output weights,
// bias [128], out [L][L][c_z] (row stride ldc = c_z) of dtype c_dtype, plus
// the old contents when flags has AFHIP_EPILOGUE_RESIDUAL. Every pair (i, j)
// computes
//   outer[a][b] = f16(sum_s left[i * 32 + a][s] right[j * 32 + b][s] / (eps + count[i][j]))
//   out[i][j][z] = sum_(a, b) outer[a][b] W[a * 32 + b][z] + bias[z] / (eps + count[i][j]).
int run_opm_fused(const GemmArgs& args, int c_dtype, const char* label, hipStream_t stream);
// Where W[k][z] (k = a * 32 + b, z < 128) sits in the fused kernel's
// 128 x 1024 f16 weight array. The pair rows in LDS hold (a, b) at half
// k' = 128 (b / 4) + 4 a + b % 4; an MFMA step reads 16-byte chunk
// c = 8 Q + 4 h + t of a row (k' in [8 c, 8 c + 8)) in lane half h, so the
// array is stored in the order the lanes load it, [z / 32][Q][t][h][z % 32]
// [k' % 8]: every wave-level load of a step's B fragment is 1 KiB contiguous.
__host__ __device__ inline int64_t opm_fused_weight_index(int k, int z) {
  const int a = k >> 5, b = k & 31;
  const int kp = 128 * (b >> 2) + 4 * a + (b & 3);
  const int c = kp >> 3, Q = c >> 3, h = (c >> 2) & 1, t = c & 3;
  return (((((int64_t)(z >> 5) * 16 + Q) * 4 + t) * 2 + h) * 32 + (z & 31)) * 8 + (kp & 7);
}

// The STREAM kernel (gemm_stream.hip): f16 activations and output, f16 or
// int8 weights held in registers, K in {64, 128, 256}, N % 64 == 0.
bool stream_shape_ok(const GemmTypes& types, int64_t M, int64_t N, int64_t K, int batch);
bool stream_eligible(const GemmArgs& args, const GemmTypes& types);
// add_f16: out += f16(result) in f32 with one more rounding (the attention
// output's residual), after a plain bias epilogue, at K <= 128.
int run_gemm_stream(const GemmArgs& args, const GemmTypes& types, const char* label, hipStream_t stream,
                    bool add_f16 = false);

// The variant plans of this shape should use (pinned, calibrated or heuristic).
afhip_variant select_variant(const GemmTypes& types, int64_t M, int64_t N, int64_t K, int batch);
// select_variant for a whole description: its layouts, strides and the
// weight dtype the kernels read included (types as the description gives
// them).
afhip_variant select_plan_variant(const afhip_gemm_desc& desc, const GemmTypes& types);

// W[k][n] (src) -> W[n][k] (dst), with dtype conversion.
int pack_transpose(const void* src, int src_dtype, int rows_k, int cols_n, int64_t ld_src, void* dst,
                   int dst_dtype, int64_t ld_dst, hipStream_t stream);

// afhip_gemm_run after its open check: `workspace` holds the plan's
// afhip_gemm_workspace_size bytes (or more) when the plan needs any.
int run_gemm_plan(const afhip_gemm_plan* plan, const void* a, const void* w, const float* scale, const float* bias,
                  const void* residual, void* c, void* workspace, size_t workspace_bytes, void* stream);

// Elementwise f32 -> dst dtype conversion (dst may be F32: plain copy).
int convert_f32(const float* src, int64_t count, void* dst, int dst_dtype, hipStream_t stream);

}  // namespace afhip
