// The fused pair transition (transition_fused.hip): f16 precision at
// channels 128, hidden 512.
#pragma once

#include "internal.h"

namespace afhip {

struct FusedTransitionArgs {
  const void* x;       // [rows][128], f32 or f16
  void* out;           // [rows][128], f32 or f16; read too when residual
  int64_t rows;
  int residual;
  const float* scale;  // LayerNorm affine [128]
  const float* offset;
  float eps;
  const half_t* w1;    // [512][128]
  const float* b1;     // [512]
  const half_t* w2;    // [128][512]
  const float* b2;     // [128]
};

// The shape the fused kernel covers (it needs no workspace), and whether a
// call of that shape can take it (x and out 16-byte aligned).
bool transition_fused_shape(const afhip_transition_desc& d);
bool transition_fused_eligible(const afhip_transition_desc& d, const void* x, const void* out);
int launch_transition_fused(const FusedTransitionArgs& a, int in_dtype, int out_dtype, hipStream_t s);

}  // namespace afhip
