// The f16, c_z = c_hidden = 128 triangle kernels (triangle_fast.hip).
#pragma once

#include "internal.h"

namespace afhip {

// Folded weight matrices the fast path prepares: AP, AG, BP, BG, Z, G.
constexpr int kFoldMatrices = 6;

// Weights are the folded ones (fold_weights_kernel in triangle.hip): the
// LayerNorm affines are inside W and b, and the gates' rows carry -log2(e).
struct FastProjectArgs {
  const void* z;         // [P][128], f32 or f16
  const float* mask;     // [P]
  const half_t* w_proj;  // [4][128][128]: AP, AG, BP, BG, [out][in], folded
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
  const half_t* w_z;         // [128][128], folded with LayerNorm-out
  const float* b_z;
  const half_t* w_g;         // [128][128], folded with LayerNorm-in and -log2(e)
  const float* b_g;
  void* out;                 // [P][128]
  int pair0, pairs;
  int residual;
  float eps;
};

bool triangle_fast_eligible(const afhip_triangle_desc& d);
int launch_triangle_project_f16(const FastProjectArgs& a, int pair_dtype, hipStream_t s);
int launch_triangle_output_f16(const FastOutputArgs& a, int pair_dtype, int out_dtype, hipStream_t s);

}  // namespace afhip
