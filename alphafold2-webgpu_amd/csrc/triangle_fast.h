// The f16, c_z = c_hidden = 128 triangle kernels (triangle_fast.hip).
#pragma once

#include "internal.h"

namespace afhip {

// Folded weight matrices the fast path prepares: AP, AG, BP, BG, Z, G.
constexpr int kFoldMatrices = 6;

// The folded matrices (128 x 128, [out n][in k]) are stored in the order the
// kernels' MFMA fragments read them: matrix m, row block nb = n / 32, input
// step s = k / 16, then the 64 lanes of the fragment, 8 halves each, lane
// (n % 32) + 32 ((k / 8) % 2) holding inputs 16 s + 8 ((k / 8) % 2) ... So the
// eight waves' sixteen fragment loads each read one contiguous KiB.
__host__ __device__ inline size_t fold_index(int m, int n, int k) {
  const int lane = (n & 31) + 32 * ((k >> 3) & 1);
  return ((((size_t)m * 4 + (n >> 5)) * 8 + (k >> 4)) * 64 + lane) * 8 + (k & 7);
}
// The 16-byte fragment (nb, s) of lane `lane` of the matrix at `w`.
__device__ __forceinline__ half8 fold_fragment(const half_t* w, int nb, int s, int lane) {
  return reinterpret_cast<const half8*>(w)[(nb * 8 + s) * 64 + lane];
}

// Weights are the folded ones (fold_weights_kernel in triangle.hip): the
// LayerNorm affines are inside W and b, and the gates' rows carry -log2(e).
struct FastProjectArgs {
  const void* z;         // [P][128], f32 or f16
  const float* mask;     // [P]
  const half_t* w_proj;  // AP, AG, BP, BG, folded, in fragment order (fold_index)
  const float* b_proj;   // [4][128], folded
  half_t* out_a;         // [128][cstride]
  half_t* out_b;
  int64_t cstride;
  int L, P;
  int incoming;
  float eps;
};

struct FastOutputArgs {
  const half_t* contracted;  // [128][bstride]
  int64_t bstride;
  const void* z;             // [P][128]
  const half_t* w_z;         // folded with LayerNorm-out, fragment order
  const float* b_z;
  const half_t* w_g;         // folded with LayerNorm-in and -log2(e), fragment order
  const float* b_g;
  void* out;                 // [P][128]
  int pair0, pairs;
  int residual;
  float eps;
};

bool triangle_fast_eligible(const afhip_triangle_desc& d);
// The most output rows one block of the fast output kernels takes (their
// per-block buffer offsets stay below 2 GiB).
int triangle_fast_block_rows(const afhip_triangle_desc& d);
int launch_triangle_project_f16(const FastProjectArgs& a, int pair_dtype, hipStream_t s);
int launch_triangle_output_f16(const FastOutputArgs& a, int pair_dtype, int out_dtype, hipStream_t s);

}  // namespace afhip
