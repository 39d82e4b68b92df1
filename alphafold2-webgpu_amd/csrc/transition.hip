// Transition for gfx950: LayerNorm, linear channels -> hidden + bias + ReLU,
// linear hidden -> channels + bias (src/evoformer/transition.ts:179-234,
// :264-361). At f16 precision with 128 channels and hidden 512 (the pair
// transition) one fused kernel does all three steps (transition_fused.hip);
// so does another at 256 channels and hidden 1024 (the MSA transition,
// transition_msa.hip), from its own folded copy of the weights.
// Otherwise the LayerNorm writes the normalised rows in the GEMM's operand
// dtype (rows spread over lane groups with 16-byte accesses for the f16 path
// at 64, 128 or 256 channels, one wave per row otherwise) and both linears run
// through the shared GEMM.
#include <algorithm>
#include <cmath>

#include "gemm.h"
#include "transition_fused.h"

namespace afhip {

namespace {

struct TransitionWeights {
  size_t scale, offset, w1, b1, w2, b2, msa, total;
};

TransitionWeights layout(const afhip_transition_desc& d) {
  TransitionWeights w{};
  size_t es = d.precision == AFHIP_PRECISION_F16 ? 2 : 4;
  size_t at = 0;
  auto take = [&](size_t bytes) {
    size_t here = at;
    at = round_up((int64_t)(at + bytes), 256);
    return here;
  };
  w.scale = take(4 * (size_t)d.channels);
  w.offset = take(4 * (size_t)d.channels);
  w.w1 = take(es * (size_t)d.hidden * d.channels);  // [H][C]
  w.b1 = take(4 * (size_t)d.hidden);
  w.w2 = take(es * (size_t)d.channels * d.hidden);  // [C][H]
  w.b2 = take(4 * (size_t)d.channels);
  w.msa = transition_msa_shape(d) ? take(transition_msa_weight_bytes()) : 0;
  w.total = at;
  return w;
}

// Rows processed per pass, bounding the workspace: the normalised rows and
// the hidden activation of one chunk (transitionChunkRows, transition.ts:60-85,
// bounds the same two tensors).
constexpr int64_t kChunkRows = 1 << 20;

struct TransitionWorkspace {
  size_t normalized, hidden, total;
  int64_t chunk;
};

TransitionWorkspace workspace(const afhip_transition_desc& d) {
  TransitionWorkspace w{};
  size_t es = d.precision == AFHIP_PRECISION_F16 ? 2 : 4;
  w.chunk = std::min<int64_t>(d.rows, kChunkRows);
  w.normalized = 0;
  w.hidden = round_up((int64_t)(es * (size_t)w.chunk * d.channels), 256);
  w.total = w.hidden + round_up((int64_t)(es * (size_t)w.chunk * d.hidden), 256);
  return w;
}

// One wave64 per row; lanes stride the channels.
template <typename IT, typename CT>
__global__ __launch_bounds__(256) void layer_norm_kernel(const IT* __restrict__ x, int64_t rows, int C,
                                                         const float* __restrict__ scale,
                                                         const float* __restrict__ offset, float eps,
                                                         CT* __restrict__ y) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const IT* xr = x + row * C;
  float s = 0.0f;
  for (int c = lane; c < C; c += 64) s += (float)xr[c];
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
  const float mean = s / (float)C;
  float v = 0.0f;
  for (int c = lane; c < C; c += 64) {
    float d = (float)xr[c] - mean;
    v += d * d;
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  const float rstd = fast_rsqrt(v / (float)C + eps);
  for (int c = lane; c < C; c += 64) y[row * C + c] = (CT)(((float)xr[c] - mean) * rstd * scale[c] + offset[c]);
}

template <typename CT>
__global__ void transition_prepare_kernel(const float* __restrict__ packed, int C, int H, float* __restrict__ scale,
                                          float* __restrict__ offset, CT* __restrict__ w1, float* __restrict__ b1,
                                          CT* __restrict__ w2, float* __restrict__ b2) {
  const float* s = packed;
  const float* o = s + C;
  const float* f = o + C;                // [C][H]
  const float* fb = f + (size_t)C * H;   // [H]
  const float* g = fb + H;               // [H][C]
  const float* gb = g + (size_t)H * C;   // [C]
  const int64_t n1 = (int64_t)H * C, total = 2 * n1 + 2 * C + H + C;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    if (i < n1) {  // w1 [H][C] <- first [C][H]
      int h = (int)(i / C), c = (int)(i % C);
      w1[i] = (CT)f[(size_t)c * H + h];
    } else if (i < 2 * n1) {  // w2 [C][H] <- second [H][C]
      int64_t j = i - n1;
      int c = (int)(j / H), h = (int)(j % H);
      w2[j] = (CT)g[(size_t)h * C + c];
    } else {
      int64_t j = i - 2 * n1;
      if (j < C) scale[j] = s[j];
      else if (j < 2 * C) offset[j - C] = o[j - C];
      else if (j < 2 * C + H) b1[j - 2 * C] = fb[j - 2 * C];
      else b2[j - 2 * C - H] = gb[j - 2 * C - H];
    }
  }
}

int validate(const afhip_transition_desc* d) {
  AFHIP_REQUIRE(d != nullptr, "descriptor is NULL");
  AFHIP_REQUIRE(d->rows > 0 && d->channels > 0 && d->hidden > 0, "transition dimensions must be positive safe integers");
  AFHIP_REQUIRE(d->rows <= ((int64_t)1 << 31) - 1, "too many rows");
  AFHIP_REQUIRE(valid_precision(d->precision), "unknown precision %d", d->precision);
  AFHIP_REQUIRE(valid_float_dtype(d->in_dtype) && valid_float_dtype(d->out_dtype), "dtypes must be f32 or f16");
  AFHIP_REQUIRE(d->epsilon > 0.0f && std::isfinite(d->epsilon), "epsilon must be finite and positive");
  return AFHIP_OK;
}

// f16 output, C = 8 LANES channels (64, 128 or 256): LANES consecutive lanes
// own a row, eight channels each (one 16-byte load of f16, two of f32), so
// the whole row is in registers after one pass and its sums are DPP
// reductions within the lane group; each lane carries four rows at a time to
// keep loads in flight. The same two-pass statistics and the same
// expression as layer_norm_kernel.
template <typename IT, int LANES>
__global__ __launch_bounds__(256) void layer_norm_rows_kernel(const IT* __restrict__ x, int64_t rows,
                                                              const float* __restrict__ scale,
                                                              const float* __restrict__ offset, float eps,
                                                              half_t* __restrict__ y) {
  constexpr int C = 8 * LANES;
  constexpr int RPW = 64 / LANES;  // rows a wave covers per load
  constexpr int U = 4;             // rows in flight per lane
  constexpr int LOADS = sizeof(IT) / 2;
  const int lane = threadIdx.x & 63, sub = lane / LANES, part = lane % LANES;
  float sc[8], of[8];
#pragma unroll
  for (int e = 0; e < 8; e++) {
    sc[e] = scale[8 * part + e];
    of[e] = offset[8 * part + e];
  }
  const int64_t wave = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  const int64_t waves = ((int64_t)gridDim.x * blockDim.x) >> 6;
  for (int64_t base = wave * RPW * U; base < rows; base += waves * RPW * U) {
    u32x4 raw[U][LOADS];
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int64_t row = base + u * RPW + sub;
#pragma unroll
      for (int l = 0; l < LOADS; l++)
        raw[u][l] = row < rows ? reinterpret_cast<const u32x4*>(x + row * C + 8 * part)[l] : u32x4{0u, 0u, 0u, 0u};
    }
    u32x4 out[U];
#pragma unroll
    for (int u = 0; u < U; u++) {
      float v[8];
      if constexpr (sizeof(IT) == 2) {
        const half8 h = __builtin_bit_cast(half8, raw[u][0]);
#pragma unroll
        for (int e = 0; e < 8; e++) v[e] = (float)h[e];
      } else {
#pragma unroll
        for (int l = 0; l < 2; l++) {
          const floatx4 f = __builtin_bit_cast(floatx4, raw[u][l]);
#pragma unroll
          for (int e = 0; e < 4; e++) v[4 * l + e] = f[e];
        }
      }
      float s = 0.0f;
#pragma unroll
      for (int e = 0; e < 8; e++) s += v[e];
      const float mean = lane_sum<LANES>(s) / (float)C;
      float d2 = 0.0f;
#pragma unroll
      for (int e = 0; e < 8; e++) {
        const float d = v[e] - mean;
        d2 += d * d;
      }
      const float rstd = fast_rsqrt(lane_sum<LANES>(d2) / (float)C + eps);
      half8 h;
#pragma unroll
      for (int e = 0; e < 8; e++) h[e] = (half_t)((v[e] - mean) * rstd * sc[e] + of[e]);
      out[u] = __builtin_bit_cast(u32x4, h);
      const int64_t row = base + u * RPW + sub;
      if (row < rows) *reinterpret_cast<u32x4*>(y + row * C + 8 * part) = out[u];
    }
    stores_read(out[0], out[1], out[2], out[3]);
  }
}

template <typename IT, typename CT>
int launch_ln(const void* x, int64_t rows, int C, const float* s, const float* o, float eps, void* y, hipStream_t st) {
  if constexpr (sizeof(CT) == 2) {
    const bool aligned = (reinterpret_cast<uintptr_t>(x) & 15) == 0 && (reinterpret_cast<uintptr_t>(y) & 15) == 0;
    if (aligned && (C == 64 || C == 128 || C == 256)) {
      const int cus = device_cu_count() > 0 ? device_cu_count() : 256;
      const int64_t rows_per_block = 4 * (64 / (C / 8)) * 4;  // four waves, four rows in flight per lane
      const unsigned grid = (unsigned)std::min<int64_t>(ceil_div(rows, rows_per_block), (int64_t)cus * 8);
      if (C == 64)
        return launch("transition.layer_norm", layer_norm_rows_kernel<IT, 8>, dim3(grid), dim3(256), 0, st,
                      (const IT*)x, rows, s, o, eps, (half_t*)y);
      if (C == 128)
        return launch("transition.layer_norm", layer_norm_rows_kernel<IT, 16>, dim3(grid), dim3(256), 0, st,
                      (const IT*)x, rows, s, o, eps, (half_t*)y);
      return launch("transition.layer_norm", layer_norm_rows_kernel<IT, 32>, dim3(grid), dim3(256), 0, st,
                    (const IT*)x, rows, s, o, eps, (half_t*)y);
    }
  }
  return launch("transition.layer_norm", layer_norm_kernel<IT, CT>, dim3((unsigned)ceil_div(rows, 4)), dim3(256), 0, st,
                (const IT*)x, rows, C, s, o, eps, (CT*)y);
}

}  // namespace

}  // namespace afhip

using namespace afhip;

extern "C" {

int afhip_transition_weights_size(const afhip_transition_desc* desc, size_t* bytes) {
  if (int s = validate(desc)) return s;
  AFHIP_REQUIRE(bytes != nullptr, "output is NULL");
  *bytes = layout(*desc).total;
  return AFHIP_OK;
}

int afhip_transition_workspace_size(const afhip_transition_desc* desc, size_t* bytes) {
  if (int s = validate(desc)) return s;
  AFHIP_REQUIRE(bytes != nullptr, "output is NULL");
  // The fused kernels keep the normalised rows and the hidden activation on chip.
  *bytes = transition_fused_shape(*desc) || transition_msa_shape(*desc) ? 0 : workspace(*desc).total;
  return AFHIP_OK;
}

int afhip_transition_prepare_weights(const afhip_transition_desc* desc, const float* packed, void* prepared,
                                     void* stream) {
  if (int s = require_open()) return s;
  if (int s = validate(desc)) return s;
  AFHIP_REQUIRE(packed && prepared, "NULL weights");
  const auto& d = *desc;
  const TransitionWeights w = layout(d);
  char* b = (char*)prepared;
  hipStream_t st = (hipStream_t)stream;
  if (d.precision == AFHIP_PRECISION_F16) {
    if (int s = launch("transition.prepare", transition_prepare_kernel<half_t>, dim3(1024), dim3(256), 0, st, packed,
                       d.channels, d.hidden, (float*)(b + w.scale), (float*)(b + w.offset), (half_t*)(b + w.w1),
                       (float*)(b + w.b1), (half_t*)(b + w.w2), (float*)(b + w.b2)))
      return s;
    if (transition_msa_shape(d)) return prepare_transition_msa(packed, b + w.msa, st);
    return AFHIP_OK;
  }
  return launch("transition.prepare", transition_prepare_kernel<float>, dim3(1024), dim3(256), 0, st, packed,
                d.channels, d.hidden, (float*)(b + w.scale), (float*)(b + w.offset), (float*)(b + w.w1),
                (float*)(b + w.b1), (float*)(b + w.w2), (float*)(b + w.b2));
}

int afhip_transition_run(const afhip_transition_desc* desc, const void* activations, const void* prepared, void* out,
                         void* workspace_ptr, size_t workspace_bytes, void* stream) {
  if (int s = require_open()) return s;
  if (int s = validate(desc)) return s;
  AFHIP_REQUIRE(activations && prepared && out, "NULL tensor");
  const auto& d = *desc;
  const TransitionWeights w = layout(d);
  const TransitionWorkspace ws = workspace(d);
  hipStream_t st = (hipStream_t)stream;
  const bool f16 = d.precision == AFHIP_PRECISION_F16;
  const int ct = f16 ? AFHIP_F16 : AFHIP_F32;
  const char* wb = (const char*)prepared;
  if (transition_fused_eligible(d, activations, out)) {
    FusedTransitionArgs f{};
    f.x = activations;
    f.out = out;
    f.rows = d.rows;
    f.residual = d.residual;
    f.scale = (const float*)(wb + w.scale);
    f.offset = (const float*)(wb + w.offset);
    f.eps = d.epsilon;
    f.w1 = (const half_t*)(wb + w.w1);
    f.b1 = (const float*)(wb + w.b1);
    f.w2 = (const half_t*)(wb + w.w2);
    f.b2 = (const float*)(wb + w.b2);
    return launch_transition_fused(f, d.in_dtype, d.out_dtype, st);
  }
  if (transition_msa_eligible(d, activations, out)) {
    MsaTransitionArgs m{};
    m.x = (const half_t*)activations;
    m.out = out;
    m.rows = d.rows;
    m.residual = d.residual;
    m.eps = d.epsilon;
    m.blocks = wb + w.msa;
    m.b1 = (const float*)(wb + w.msa + transition_msa_weight_bytes() - 4 * (size_t)(d.hidden + d.channels));
    m.b2 = m.b1 + d.hidden;
    return launch_transition_msa(m, d.out_dtype, st);
  }
  AFHIP_REQUIRE(!(transition_fused_shape(d) || transition_msa_shape(d)) || workspace_bytes >= ws.total,
                "this transition shape runs fused and needs activations and output 16-byte aligned");
  AFHIP_REQUIRE(workspace_ptr != nullptr && workspace_bytes >= ws.total, "workspace of %zu bytes is smaller than %zu",
                workspace_bytes, ws.total);
  char* normalized = (char*)workspace_ptr + ws.normalized;
  char* hidden = (char*)workspace_ptr + ws.hidden;
  const size_t ie = dtype_size(d.in_dtype), oe = dtype_size(d.out_dtype);
  for (int64_t r0 = 0; r0 < d.rows; r0 += ws.chunk) {
    const int64_t rows = std::min<int64_t>(ws.chunk, d.rows - r0);
    const char* x = (const char*)activations + ie * (size_t)r0 * d.channels;
    const float* sc = (const float*)(wb + w.scale);
    const float* of = (const float*)(wb + w.offset);
    int s;
    if (d.in_dtype == AFHIP_F32)
      s = f16 ? launch_ln<float, half_t>(x, rows, d.channels, sc, of, d.epsilon, normalized, st)
              : launch_ln<float, float>(x, rows, d.channels, sc, of, d.epsilon, normalized, st);
    else
      s = f16 ? launch_ln<half_t, half_t>(x, rows, d.channels, sc, of, d.epsilon, normalized, st)
              : launch_ln<half_t, float>(x, rows, d.channels, sc, of, d.epsilon, normalized, st);
    if (s) return s;
    GemmArgs g1;
    g1.a = normalized;
    g1.b = wb + w.w1;
    g1.c = hidden;
    g1.bias = (const float*)(wb + w.b1);
    g1.M = (int)rows;
    g1.N = d.hidden;
    g1.K = d.channels;
    g1.lda = d.channels;
    g1.ldb = d.channels;
    g1.ldc = d.hidden;
    g1.flags = AFHIP_EPILOGUE_BIAS | AFHIP_EPILOGUE_RELU;
    GemmTypes t1{d.precision, ct, ct, ct};
    if ((s = run_gemm(g1, t1, select_variant(t1, g1.M, g1.N, g1.K, 1), "transition.first", st))) return s;
    GemmArgs g2;
    g2.a = hidden;
    g2.b = wb + w.w2;
    g2.c = (char*)out + oe * (size_t)r0 * d.channels;
    g2.residual = g2.c;
    g2.bias = (const float*)(wb + w.b2);
    g2.M = (int)rows;
    g2.N = d.channels;
    g2.K = d.hidden;
    g2.lda = d.hidden;
    g2.ldb = d.hidden;
    g2.ldc = d.channels;
    g2.flags = AFHIP_EPILOGUE_BIAS | (d.residual ? AFHIP_EPILOGUE_RESIDUAL : 0u);
    GemmTypes t2{d.precision, ct, ct, d.out_dtype};
    if ((s = run_gemm(g2, t2, select_variant(t2, g2.M, g2.N, g2.K, 1), "transition.second", st))) return s;
  }
  return AFHIP_OK;
}

}  // extern "C"
