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

// The MSA transition fused (transition_msa.hip): f16 precision at channels
// 256, hidden 1024, f16 rows in, f32 or f16 out.
struct MsaTransitionArgs {
  const half_t* x;       // [rows][256]
  void* out;             // [rows][256]; read too when residual
  int64_t rows;
  int residual;
  float eps;
  const void* blocks;    // the folded weights in fragment order (prepare_transition_msa)
  const float* b1;       // folded first bias [1024]
  const float* b2;       // [256]
};
bool transition_msa_shape(const afhip_transition_desc& d);
bool transition_msa_eligible(const afhip_transition_desc& d, const void* x, const void* out);
// Bytes of the prepared region: the weight blocks, then b1' [1024] and b2 [256].
size_t transition_msa_weight_bytes();
int prepare_transition_msa(const float* packed, void* dst, hipStream_t s);
int launch_transition_msa(const MsaTransitionArgs& a, int out_dtype, hipStream_t s);

}  // namespace afhip
