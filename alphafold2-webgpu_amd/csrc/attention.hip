// Gated multi-head attention with an optional pair bias, the Evoformer's
// row, column and triangle attention (src/evoformer/attention.ts:1321-1452,
// AttentionGpu.run; encodeAttention in src/evoformer/block.ts):
//
//   x_hat = LayerNorm(x) over the rows in attention order (entry (b, q) is
//           source row b Q + q, or q B + b when transposed);
//   q, k, v, g = x_hat [Wq | Wk | Wv | Wg], q scaled by 1/sqrt(d), g = sigmoid(. + bg)
//           (one GEMM with the ATTENTION epilogue, as attentionProjectShader);
//   bias[h][q][k] = y[q][k] . Wb[:, h], y the normalised input itself
//           (triangle attention) or a separate LayerNormed pair tensor (MSA
//           row attention);
//   o = softmax_k(clamp(q.k + 1e9 (mask[b][k] - 1) + bias, -1e8, 1e8)) v * g;
//   out = o Wo + bo (+ out), back in source order.
//
// Kernels: a row kernel (LayerNorm in attention order, the key bias, and the
// normalized-input pair bias from the same registers), the projection GEMM,
// a row kernel for a separate pair source, the flash kernel, the output GEMM.
//
// At f16 precision with a head dimension of 8, 16, 24 or 32 (heads padded to
// 32 channels with zeros) the flash kernel runs on the MFMA
// as S^T = K Q^T and O^T = V^T P^T: a lane then holds one query's scores for
// 16 keys and the same query's output for 16 channels, so the running maximum,
// sum and rescale stay inside the lane (one exchange with the lane 32 away),
// and the probabilities feed the second MFMA from the registers they were
// computed in. V stays in its natural [key][channel] layout: the V^T
// fragments come from gfx950's transposing LDS read (ds_read_b64_tr_b16),
// which hands each lane its channel's keys in the order of those registers.
// Its logits are kept in base-2 units (q, the key bias and the pair bias
// carry a factor log2(e)), which changes nothing but the rounding:
// exp2(log2(e) x) = exp(x). Any other head dimension, or f32 precision, runs
// a one-thread-per-query kernel in f32 on the natural units.
#include <algorithm>
#include <cmath>
#include <cstddef>
#include <utility>

#include "dma.h"
#include "gemm.h"

namespace afhip {

namespace {

constexpr float kLog2e = 1.4426950408889634f;

// The f16 MFMA flash kernel takes head dimensions 8, 16, 24 and 32 (heads
// padded to 32 channels with zeros).
bool fast_path(const afhip_attention_desc& d) {
  return d.precision == AFHIP_PRECISION_F16 && (d.channels / d.heads) % 8 == 0;
}

// Prepared weights: everything the kernels read, in their dtypes.
struct AttentionWeights {
  size_t ln_scale, ln_offset, w_proj, b_proj, w_out, b_out, pair_scale, pair_offset, w_bias, total;
};

AttentionWeights weights_layout(const afhip_attention_desc& d) {
  AttentionWeights w{};
  const size_t es = d.precision == AFHIP_PRECISION_F16 ? 2 : 4;
  const size_t C = d.channels;
  size_t at = 0;
  auto take = [&](size_t bytes) {
    size_t here = at;
    at = round_up((int64_t)(at + bytes), 256);
    return here;
  };
  w.ln_scale = take(4 * C);
  w.ln_offset = take(4 * C);
  w.w_proj = take(es * 4 * C * C);  // [4C][C]: rows q, k, v, g (k-contiguous)
  w.b_proj = take(4 * 4 * C);       // zeros, then the gating bias
  w.w_out = take(es * C * C);       // [C][C] (k-contiguous)
  w.b_out = take(4 * C);
  const size_t pc = d.pair_bias == AFHIP_PAIR_BIAS_SEPARATE ? (size_t)d.pair_channels : C;
  w.pair_scale = take(4 * pc);
  w.pair_offset = take(4 * pc);
  w.w_bias = take(4 * pc * d.heads);  // [channel][head]
  w.total = at;
  return w;
}

// Workspace. The key bias [B][stride] and the pair bias [H][Q][stride] rows
// are padded to a multiple of four keys, so the flash kernels read them as
// float4; the padding is never used as a live key. On the fast path the
// flash kernel reads whole blocks of 32 keys (its read-ahead stops at the
// last block), up to 31 keys past the last, so the tensors it reads end in
// at least that much padding.
struct AttentionWorkspace {
  size_t normalized, key_bias, key_mask, qkvg, bias, weighted, total;
  int stride, code_stride;
};

constexpr int kReadAhead = 64;  // keys

AttentionWorkspace workspace_layout(const afhip_attention_desc& d) {
  AttentionWorkspace w{};
  const size_t es = d.precision == AFHIP_PRECISION_F16 ? 2 : 4;
  const size_t rows = (size_t)d.batch * d.queries, C = d.channels;
  const bool fast = fast_path(d);
  size_t at = 0;
  auto take = [&](size_t bytes) {
    size_t here = at;
    at = round_up((int64_t)(at + bytes), 256);
    return here;
  };
  w.stride = (int)round_up(d.queries, 4);
  w.code_stride = (int)round_up(d.queries, 32);
  w.normalized = take(es * rows * C);
  w.key_bias = take(fast ? 0 : 4 * (size_t)d.batch * w.stride);
  // f16 key mask codes [B][code_stride] (fast path)
  w.key_mask = take(fast ? 2 * (size_t)d.batch * w.code_stride : 0);
  w.qkvg = take(es * (rows + (fast ? kReadAhead : 0)) * 4 * C);
  w.bias = take(d.pair_bias ? 4 * ((size_t)d.heads * d.queries * w.stride + (fast ? kReadAhead : 0)) : 0);
  w.weighted = take(es * rows * C);
  w.total = at;
  return w;
}

int validate(const afhip_attention_desc* dp) {
  AFHIP_REQUIRE(dp != nullptr, "NULL attention description");
  const auto& d = *dp;
  AFHIP_REQUIRE(d.batch > 0 && d.queries > 0 && d.channels > 0 && d.heads > 0,
                "attention dimensions must be positive safe integers");
  AFHIP_REQUIRE(d.channels % d.heads == 0 && d.channels / d.heads <= 32,
                "attention needs an integral head dimension no larger than 32");
  AFHIP_REQUIRE(d.pair_bias >= AFHIP_PAIR_BIAS_NONE && d.pair_bias <= AFHIP_PAIR_BIAS_SEPARATE,
                "unknown pair bias source %d", d.pair_bias);
  AFHIP_REQUIRE(d.pair_bias != AFHIP_PAIR_BIAS_NORMALIZED_INPUT || d.batch == d.queries,
                "a normalized-input pair bias needs batch == queries");
  AFHIP_REQUIRE(d.pair_bias != AFHIP_PAIR_BIAS_SEPARATE || d.pair_channels > 0,
                "a separate pair bias needs its pair channels");
  AFHIP_REQUIRE(d.transpose == 0 || d.transpose == 1, "transpose is 0 or 1");
  AFHIP_REQUIRE(std::isfinite(d.epsilon) && d.epsilon >= 0.0f, "epsilon must be a finite non-negative number");
  AFHIP_REQUIRE(valid_precision(d.precision), "unknown precision %d", d.precision);
  AFHIP_REQUIRE(valid_float_dtype(d.in_dtype) && valid_float_dtype(d.out_dtype), "attention dtypes are f32 or f16");
  AFHIP_REQUIRE((int64_t)d.batch * d.queries < ((int64_t)1 << 31), "attention has too many rows");
  AFHIP_REQUIRE((int64_t)d.heads * d.queries * round_up(d.queries, 4) < ((int64_t)1 << 31),
                "attention has too many queries");
  return AFHIP_OK;
}

// --------------------------------------------------------------------------
// Kernels
// --------------------------------------------------------------------------

template <typename T> __device__ __forceinline__ float ld(const T* p, int64_t i) { return (float)p[i]; }

// Weight preparation from the reference's packed f32 order
// (packAttentionWeights, attention.ts:179-201): the four projections
// [C][C] ([in][out]) transposed into [4C][C] k-contiguous rows, the gating
// bias after 3C zeros, the output projection transposed to [C][C].
template <typename CT>
__global__ void attention_prepare_kernel(const float* __restrict__ packed, int C, int H, int pc, int separate,
                                         int has_bias, float* __restrict__ ln_scale, float* __restrict__ ln_offset,
                                         CT* __restrict__ w_proj, float* __restrict__ b_proj, CT* __restrict__ w_out,
                                         float* __restrict__ b_out, float* __restrict__ pair_scale,
                                         float* __restrict__ pair_offset, float* __restrict__ w_bias) {
  const int64_t CC = (int64_t)C * C;
  // packed offsets: scale C, offset C, q CC, k CC, v CC, g CC, gb C, out CC, ob C, then the pair tensors
  const float* p_scale = packed;
  const float* p_offset = p_scale + C;
  const float* p_w[4] = {p_offset + C, p_offset + C + CC, p_offset + C + 2 * CC, p_offset + C + 3 * CC};
  const float* p_gb = p_offset + C + 4 * CC;
  const float* p_out = p_gb + C;
  const float* p_ob = p_out + CC;
  const float* p_pair = p_ob + C;
  // Index space, in order: w_proj 4CC, w_out CC, b_proj 4C, the per-channel
  // vectors C, the pair LayerNorm pc, w_bias pc H.
  const int64_t total = 5 * CC + 5 * (int64_t)C + pc + (int64_t)pc * H;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    int64_t j = i;
    if (j < 4 * CC) {  // w_proj[n][k] = W_{n / C}[k][n % C]
      const int64_t n = j / C, k = j % C;
      w_proj[j] = (CT)p_w[n / C][k * C + n % C];
      continue;
    }
    j -= 4 * CC;
    if (j < CC) {  // w_out[n][k] = out[k][n]
      const int64_t n = j / C, k = j % C;
      w_out[j] = (CT)p_out[k * C + n];
      continue;
    }
    j -= CC;
    if (j < 4 * C) {
      b_proj[j] = j < 3 * C ? 0.0f : p_gb[j - 3 * C];
      continue;
    }
    j -= 4 * C;
    if (j < C) {
      ln_scale[j] = p_scale[j];
      ln_offset[j] = p_offset[j];
      b_out[j] = p_ob[j];
      continue;
    }
    j -= C;
    if (j < pc) {
      if (has_bias && separate) {
        pair_scale[j] = p_pair[j];
        pair_offset[j] = p_pair[pc + j];
      }
      continue;
    }
    j -= pc;
    if (has_bias) w_bias[j] = p_pair[(separate ? 2 * (int64_t)pc : 0) + j];
  }
}

// One row pass over [rows][C]: LayerNorm (two-pass mean and biased variance,
// eps inside the root, attention.ts:312-324) and, as asked, the normalised
// row, the row's key bias key_scale (mask - 1) (:688-690), and the pair bias
// bias[h][r / Q][r % Q] = bias_scale (y . w[:, h]) (:631-661).
struct RowsArgs {
  const void* x;
  int64_t rows;
  int C, B, Q, transpose;  // row r = (b, q) = (r / Q, r % Q) reads source row q B + b when transposed
  const float* scale;
  const float* offset;
  float eps;
  void* out;                // [rows][C] in attention order, or null
  const float* mask;        // source order, or null (no key bias)
  float* key_bias;          // [B][stride] f32, or null
  float key_scale;
  half_t* key_mask;         // [B][code_stride] f16 codes (mask - 1) kMaskCode, or null
  const float* w;           // [C][H], or null (no pair bias)
  int H;
  float bias_scale;
  float* bias;              // [H][Q][stride]
  int stride;
  int code_stride;          // Q rounded up to 32: keys Q.. of a code row hold -inf
};

// The key mask code of the fast path: (mask - 1) 32768 in f16 (exact for a
// 0/1 mask). Times kMaskScale, the f16 nearest 1e9 log2(e) / 32768, it is the
// key bias 1e9 (mask - 1) in base-2 units to within 1.1e-4 relative.
constexpr float kMaskCode = 32768.0f;
constexpr float kMaskScale = 44032.0f;

// Key (b, q)'s bias or code. The last key of a code row also fills the row's
// padding with -inf codes: past the last key a key block's mask step then
// gives -inf logits.
__device__ __forceinline__ void key_bias_store(const RowsArgs& a, int64_t b, int64_t q, float mask) {
  if (a.key_bias) a.key_bias[b * a.stride + q] = a.key_scale * (mask - 1.0f);
  if (a.key_mask) {
    half_t* row = a.key_mask + b * a.code_stride;
    row[q] = (half_t)((mask - 1.0f) * kMaskCode);
    if (q == a.Q - 1)
      for (int k = a.Q; k < a.code_stride; k++) row[k] = (half_t)(-INFINITY);
  }
}

// Pair bias (h, query b, key q); the last key of a row also zeroes the row's
// padding up to the stride, which the fast kernels read as keys past the end.
__device__ __forceinline__ void pair_bias_store(const RowsArgs& a, int h, int64_t b, int64_t q, float v) {
  float* row = a.bias + ((int64_t)h * a.Q + b) * a.stride;
  row[q] = a.bias_scale * v;
  if (q == a.Q - 1)
    for (int k = a.Q; k < a.stride; k++) row[k] = 0.0f;
}

template <typename T> __device__ __forceinline__ void load8(const T* p, float (&v)[8]) {
  if constexpr (sizeof(T) == 2) {
    const half8 h = *reinterpret_cast<const half8*>(p);
#pragma unroll
    for (int e = 0; e < 8; e++) v[e] = (float)h[e];
  } else {
    const float4 a = *reinterpret_cast<const float4*>(p), b = *reinterpret_cast<const float4*>(p + 4);
    v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w, v[4] = b.x, v[5] = b.y, v[6] = b.z, v[7] = b.w;
  }
}

template <typename T> __device__ __forceinline__ void store8(T* p, const float (&v)[8]) {
  if constexpr (sizeof(T) == 2) {
    half8 h;
#pragma unroll
    for (int e = 0; e < 8; e++) h[e] = (half_t)v[e];
    *reinterpret_cast<half8*>(p) = h;
  } else {
    *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
    *reinterpret_cast<float4*>(p + 4) = make_float4(v[4], v[5], v[6], v[7]);
  }
}

// Vectorised rows: LANES lanes a row, eight channels a lane (C = 8 LANES);
// a workgroup walks 256 / LANES rows at a time through the tensor, the head
// weights (zero past H, H <= HB, HB 4 or 8) staged once in LDS. Rows are
// fewer than 2^24, so a row's (b, q) comes from an f32 reciprocal of Q and
// one correction instead of a 64-bit division.
template <typename IT, typename OT, int LANES, int HB>
__global__ __launch_bounds__(256) void attention_rows_kernel(RowsArgs a) {
  constexpr int C = 8 * LANES;
  constexpr int kRows = 256 / LANES;
  static_assert(HB == 4 || HB == 8, "head bound");
  __shared__ __attribute__((aligned(16))) float wl[C * HB];
  if (a.w) {
    // channel c = 8 j + e at [e][j][HB]: the lanes of a row read adjacent
    // 4 HB-byte pieces for each e
    for (int i = threadIdx.x; i < C * HB; i += 256) {
      const int c = i / HB, h = i % HB;
      wl[((c & 7) * LANES + (c >> 3)) * HB + h] = h < a.H ? a.w[c * a.H + h] : 0.0f;
    }
    __syncthreads();
  }
  const float inv_q = 1.0f / (float)a.Q;
  const int j = threadIdx.x % LANES;
  // The LayerNorm affine of this lane's channels, read once (inside the
  // loop each read would wait behind the previous row's stores, which the
  // compiler cannot prove do not alias it).
  float sc[8], of[8];
#pragma unroll
  for (int e = 0; e < 8; e++) {
    sc[e] = a.scale[8 * j + e];
    of[e] = a.offset[8 * j + e];
  }
  for (int64_t r0 = (int64_t)blockIdx.x * kRows; r0 < a.rows; r0 += (int64_t)gridDim.x * kRows) {
    const int64_t r = r0 + threadIdx.x / LANES;
    const bool live = r < a.rows;
    const int64_t rr = live ? r : a.rows - 1;  // past the end: recompute the last row, store nothing
    // floor(rr / Q) to within one from the f32 product (rr < 2^24 converts
    // exactly; the product is off by less than one), then corrected.
    int bi = (int)((float)(int)rr * inv_q);
    int qi = (int)rr - bi * a.Q;
    if (qi < 0) {
      bi -= 1;
      qi += a.Q;
    } else if (qi >= a.Q) {
      bi += 1;
      qi -= a.Q;
    }
    const int64_t b = bi, q = qi;
    const int64_t src = a.transpose ? q * a.B + b : rr;
    float v[8];
    load8(reinterpret_cast<const IT*>(a.x) + src * C + 8 * j, v);
    float s = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; e++) s += v[e];
    const float mean = lane_sum<LANES>(s) / (float)C;
    float var = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; e++) {
      const float dlt = v[e] - mean;
      var += dlt * dlt;
    }
    const float rstd = 1.0f / sqrtf(lane_sum<LANES>(var) / (float)C + a.eps);
#pragma unroll
    for (int e = 0; e < 8; e++) v[e] = (v[e] - mean) * rstd * sc[e] + of[e];
    if (a.out && live) store8(reinterpret_cast<OT*>(a.out) + rr * C + 8 * j, v);
    if (a.mask && live && j == 0) key_bias_store(a, b, q, a.mask[src]);
    if (a.w) {
      float acc[HB] = {};
#pragma unroll
      for (int e = 0; e < 8; e++) {
#pragma unroll
        for (int h4 = 0; h4 < HB; h4 += 4) {
          const float4 w4 = *reinterpret_cast<const float4*>(&wl[(e * LANES + j) * HB + h4]);
          acc[h4] += v[e] * w4.x, acc[h4 + 1] += v[e] * w4.y, acc[h4 + 2] += v[e] * w4.z, acc[h4 + 3] += v[e] * w4.w;
        }
      }
      float mine = 0.0f;
#pragma unroll
      for (int h = 0; h < HB; h++) {
        const float t = lane_sum<LANES>(acc[h]);
        if (h == j) mine = t;
      }
      if (live && j < a.H) pair_bias_store(a, j, b, q, mine);
    }
  }
}

// The same pass for any width: one wave a row.
template <typename IT, typename OT>
__global__ __launch_bounds__(256) void attention_rows_any_kernel(RowsArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= a.rows) return;  // the whole wave
  const int64_t b = r / a.Q, q = r % a.Q;
  const int64_t src = a.transpose ? q * a.B + b : r;
  const int C = a.C;
  const IT* xr = reinterpret_cast<const IT*>(a.x) + src * C;
  float s = 0.0f;
  for (int c = lane; c < C; c += 64) s += ld(xr, c);
  for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
  const float mean = s / (float)C;
  float var = 0.0f;
  for (int c = lane; c < C; c += 64) {
    const float dlt = ld(xr, c) - mean;
    var += dlt * dlt;
  }
  for (int o = 32; o > 0; o >>= 1) var += __shfl_xor(var, o);
  const float rstd = 1.0f / sqrtf(var / (float)C + a.eps);
  if (a.out)
    for (int c = lane; c < C; c += 64)
      reinterpret_cast<OT*>(a.out)[r * C + c] = (OT)((ld(xr, c) - mean) * rstd * a.scale[c] + a.offset[c]);
  if (a.mask && lane == 0) key_bias_store(a, b, q, a.mask[src]);
  if (a.w) {
    for (int h = 0; h < a.H; h++) {
      float acc = 0.0f;
      for (int c = lane; c < C; c += 64)
        acc += ((ld(xr, c) - mean) * rstd * a.scale[c] + a.offset[c]) * a.w[(int64_t)c * a.H + h];
      for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o);
      if (lane == 0) pair_bias_store(a, h, b, q, acc);
    }
  }
}

struct FlashArgs {
  const void* qkvg;       // [B Q][4C]: q (scaled), k, v, g (sigmoid)
  const float* key_bias;  // [B][stride] (general kernel)
  const half_t* key_mask; // [B][code_stride] codes (f16 kernels)
  const float* bias;      // [H][Q][stride] or null
  void* weighted;         // [B Q][C] in source order
  int B, Q, C, H, d, transpose, stride, code_stride;
  float clamp;
};

// One thread per (b, h, q), f32 arithmetic: the reference's recurrence
// (attention.ts:688-723) with the query and the accumulator in registers,
// one instance per head dimension D.
template <typename CT, int D>
__global__ __launch_bounds__(256) void attention_flash_generic_kernel(FlashArgs a) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = (int64_t)a.B * a.H * a.Q;
  if (t >= total) return;
  const int q = (int)(t % a.Q);
  const int h = (int)((t / a.Q) % a.H);
  const int64_t b = t / ((int64_t)a.Q * a.H);
  const CT* base = reinterpret_cast<const CT*>(a.qkvg);
  const int64_t ld4 = 4 * (int64_t)a.C;
  const CT* qr = base + (b * a.Q + q) * ld4 + h * D;
  float qv[D], acc[D];
#pragma unroll
  for (int e = 0; e < D; e++) {
    qv[e] = (float)qr[e];
    acc[e] = 0.0f;
  }
  float run_max = -1e30f, run_sum = 0.0f;
  for (int k = 0; k < a.Q; k++) {
    const CT* kr = base + (b * a.Q + k) * ld4 + a.C + h * D;
    float dot = 0.0f;
#pragma unroll
    for (int e = 0; e < D; e++) dot += qv[e] * (float)kr[e];
    float logit = dot + a.key_bias[b * a.stride + k];
    if (a.bias) logit += a.bias[((int64_t)h * a.Q + q) * a.stride + k];
    logit = fminf(fmaxf(logit, -a.clamp), a.clamp);
    const float new_max = fmaxf(run_max, logit);
    const float scale = expf(run_max - new_max), weight = expf(logit - new_max);
    run_sum = run_sum * scale + weight;
    run_max = new_max;
    const CT* vr = kr + a.C;
#pragma unroll
    for (int e = 0; e < D; e++) acc[e] = acc[e] * scale + weight * (float)vr[e];
  }
  const CT* gr = qr + 3 * a.C;
  const int64_t src = a.transpose ? (int64_t)q * a.B + b : b * a.Q + q;
  CT* out = reinterpret_cast<CT*>(a.weighted) + src * a.C + h * D;
#pragma unroll
  for (int e = 0; e < D; e++) out[e] = (CT)(acc[e] / run_sum * (float)gr[e]);
}

template <typename CT, int... Ds>
int launch_flash_generic(const FlashArgs& fa, hipStream_t st, std::integer_sequence<int, Ds...>) {
  using Kernel = void (*)(FlashArgs);
  static constexpr Kernel table[] = {attention_flash_generic_kernel<CT, Ds + 1>...};
  const int64_t threads = (int64_t)fa.B * fa.H * fa.Q;
  return launch("attention.flash", table[fa.d - 1], dim3((unsigned)ceil_div(threads, 256)), dim3(256), 0, st, fa);
}

// f16 operands, head_dim 32: one wave per 32 queries of one (b, h), keys in
// blocks of 32. S^T = K Q^T: A = K [key][d] straight from the projection
// output, B = Q^T (the wave's queries, held for the whole loop); the result
// gives lane l query l % 32 and keys 8 (v / 4) + 4 (l / 32) + v % 4. The
// probabilities, packed to f16 in that key order, are the B operand of
// O^T = V^T P^T, whose A operand holds V^T in the same key order.
//
// The MFMA does the per-logit additions: the accumulator starts from the pair
// bias (loaded in the accumulator's own layout), and a 32x32x8 step adds
// code[key] kMaskScale - m, with A = (code, 1) per key and B = (kMaskScale,
// -m) per query, m an f16 offset that stands in for the running maximum. m
// moves only when a block's logits exceed it by more than kSlack (and once,
// to the first block's maximum), so probabilities stay below 2^kSlack and
// the rescale of the accumulator is rare. The clamp is kept relative to m.
// On this path the clamp is +-kLogitBound (base 2; 20794 in natural units)
// rather than +-1e8: the same softmax wherever a row's largest logit lies
// within those bounds, and a row whose every key is masked still averages
// its values.
//
// A workgroup is two batch entries by 128 queries of one head: eight waves,
// wave (bi, qi) taking queries 32 qi.. of batch entry bi. Each key block's
// K and V tiles (shared by a batch entry's four query waves) and pair-bias
// tile (shared by both batch entries) pass through LDS, double-buffered:
// every lane holds its share of blocks j + 1 and j + 2 in registers while
// block j is computed, stores block j + 1 to LDS after, and after the
// block's one barrier loads its share of block j + 3. Keys past the end of
// the last block are masked.
constexpr int kFlashBatch = 2;
constexpr int kFlashQueryWaves = 4;
constexpr int kFlashThreads = 64 * kFlashBatch * kFlashQueryWaves;
constexpr float kLogitBound = 30000.0f;
constexpr float kSlack = 8.0f;
// Base-2 distance below the row maximum past which exp2 gives 0 in f32
// (below 2^-149) and therefore in f16.
constexpr float kClampReach = 160.0f;

typedef short short4v __attribute__((ext_vector_type(4)));
typedef short short8v __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) short4v lds_short4v;

struct FlashTile {
  half_t k[kFlashBatch][32][40];   // [bi][key][channel], rows padded to 80 bytes
  half_t v[kFlashBatch][32][32];   // [bi][key][channel], read transposed (ds_read_b64_tr_b16)
  float bias[32 * kFlashQueryWaves][36];  // [query][key], rows padded to 144 bytes
  half_t code[kFlashBatch * kFlashQueryWaves][32];  // [wave][key]: each wave's own copy of its keys' mask codes
};

template <bool BIAS>
__global__ __launch_bounds__(kFlashThreads) void attention_flash_f16_kernel(FlashArgs a) {
  __shared__ FlashTile tiles[2];
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int col = lane & 31, hi = lane >> 5;
  const int bi = wave / kFlashQueryWaves, qi = wave % kFlashQueryWaves;
  const int Q = a.Q;
  const int qblocks = (Q + 32 * kFlashQueryWaves - 1) / (32 * kFlashQueryWaves);
  const int qb = (int)(blockIdx.x % qblocks);
  const int h = (int)((blockIdx.x / qblocks) % a.H);
  const int64_t b0 = (int64_t)(blockIdx.x / qblocks / a.H) * kFlashBatch;
  const half_t* base = reinterpret_cast<const half_t*>(a.qkvg);
  const int64_t ld4 = 4 * (int64_t)a.C;
  const int qbase = qb * 32 * kFlashQueryWaves;

  // This lane's share of a block's loads, at key block 0; block k0 adds
  // uniform offsets: one 16-byte piece of a tile (lanes 0-127 and 128-255 the
  // K tiles of batch entries 0 and 1, lanes 256-383 and 384-511 their V
  // tiles; piece u of a tile holds key u / 4, channels 8 (u % 4)..) and two
  // of the bias tile (lane t: pieces t and t + 512, piece c holding row c / 8,
  // keys 4 (c % 8)..).
  const half_t* tile_src;
  int64_t tile_step;  // elements per key block
  uint32_t tile_dst;  // byte offset in tiles[0]; tiles[1] is sizeof(FlashTile) further
  {
    const int part = tid >> 7;
    const int u = tid & 127;
    const int e = part & 1;
    const int64_t be = min(b0 + e, (int64_t)a.B - 1);
    tile_src = base + (be * Q + (u >> 2)) * ld4 + (part < 2 ? 1 : 2) * a.C + h * a.d + 8 * (u & 3);
    tile_step = 32 * ld4;
    // K rows are padded to 80 bytes for the fragment reads; V rows are 64
    // bytes, which keeps the transposing reads free of bank conflicts.
    tile_dst = part < 2 ? (uint32_t)offsetof(FlashTile, k) + 2u * (uint32_t)((e * 32 + (u >> 2)) * 40 + 8 * (u & 3))
                        : (uint32_t)offsetof(FlashTile, v) + 2u * (uint32_t)((e * 32 + (u >> 2)) * 32 + 8 * (u & 3));
  }
  const float* bias_src[2] = {nullptr, nullptr};
  uint32_t bias_dst[2] = {};
  if (BIAS) {
    for (int i = 0; i < 2; i++) {
      const int c = tid + kFlashThreads * i;
      const int r = c >> 3;
      const int q = min(qbase + r, Q - 1);
      bias_src[i] = a.bias + ((int64_t)h * Q + q) * a.stride + 4 * (c & 7);
      bias_dst[i] = (uint32_t)offsetof(FlashTile, bias) + 4u * (uint32_t)(r * 36 + 4 * (c & 7));
    }
  }
  static_assert(2 * kFlashThreads * 4 == 32 * kFlashQueryWaves * 32, "two bias pieces a lane cover the tile");

  // This wave's batch entry and queries.
  const int64_t b = b0 + bi;
  const int q0 = qbase + 32 * qi;
  const bool active = b < a.B && q0 < Q;  // idle waves still load and meet every barrier
  const int64_t bc = active ? b : 0;
  const int64_t row0 = bc * Q;
  const int myq = q0 + col;
  const int qrow = myq < Q ? myq : Q - 1;
  half8 qf[2] = {};
  if (active) {
    const half_t* qr = base + (row0 + qrow) * ld4 + h * a.d + 8 * hi;
    if (8 * hi < a.d) qf[0] = *reinterpret_cast<const half8*>(qr);
    if (16 + 8 * hi < a.d) qf[1] = *reinterpret_cast<const half8*>(qr + 16);
  }
  const half_t* cp = a.key_mask + bc * a.code_stride + col;

  floatx16 o = {};       // O^T: lane holds query myq, channels 8 (v / 4) + 4 hi + v % 4
  float run_sum = 0.0f;  // over this lane's keys; the lane 32 away holds the rest
  float m = 0.0f;        // f16-representable, subtracted by the MFMA
  float lo = -kLogitBound, up = kLogitBound;  // clamp bounds relative to m
  half4 bm_frag = hi ? half4{} : half4{(half_t)kMaskScale, (half_t)0.0f, (half_t)0.0f, (half_t)0.0f};
  const half_t one = (half_t)1.0f;

  // V^T fragments of O^T = V^T P^T from the [key][channel] tile with the
  // transposing LDS read: within each 16-lane group, output lane i gets, as
  // its element j, element i % 4 of the 8 bytes lane 4 j + i / 4 addressed.
  // Lane 16 g + m addresses key 16 s + 4 (lane / 32) + m / 4 (+ 8 for the
  // second read), channels 16 (g % 2) + 4 (m % 4).., so lane (channel c, hi)
  // receives keys 16 s + 8 (e / 4) + 4 hi + e % 4 of channel c: the order the
  // probabilities take in the MFMA's other operand.
  const int tr_key = 4 * hi + ((lane & 15) >> 2), tr_ch = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
  auto step = [&](const FlashTile& tl, int k0, bool first) {
    const half_t code = tl.code[wave][col];
    floatx16 sc = {};
    if constexpr (BIAS) {
#pragma unroll
      for (int g = 0; g < 4; g++) {
        const float4 t = *reinterpret_cast<const float4*>(&tl.bias[32 * qi + col][8 * g + 4 * hi]);
        sc[4 * g] = t.x, sc[4 * g + 1] = t.y, sc[4 * g + 2] = t.z, sc[4 * g + 3] = t.w;
      }
    }
#pragma unroll
    for (int s = 0; s < 2; s++)
      sc = mfma_f16(*reinterpret_cast<const half8*>(&tl.k[bi][col][16 * s + 8 * hi]), qf[s], sc);
    const half4 am = hi ? half4{} : half4{code, one, (half_t)0.0f, (half_t)0.0f};
    sc = __builtin_amdgcn_mfma_f32_32x32x8f16(am, bm_frag, sc, 0, 0, 0);
    float x[16];
#pragma unroll
    for (int v = 0; v < 16; v++) x[v] = sc[v];
    const bool last = k0 + 32 > Q;
    auto drop_past_end = [&]() {  // the last block: keys past the end take no weight
#pragma unroll
      for (int g = 0; g < 4; g++)
#pragma unroll
        for (int i = 0; i < 4; i++)
          if (k0 + 8 * g + 4 * hi + i >= Q) x[4 * g + i] = -INFINITY;
    };
    if (last) drop_past_end();
    float bm = x[0];
#pragma unroll
    for (int v = 1; v < 16; v++) bm = fmaxf(bm, x[v]);
    // The clamp to [lo, up] changes a probability only where the block's
    // largest logit is above up or within kClampReach of lo: otherwise
    // every logit below lo, clamped or not, is more than kClampReach under
    // the row's maximum and its probability underflows to 0 in f32 and f16
    // alike. So it runs (exactly) only for such blocks.
    if (__builtin_amdgcn_ballot_w64(bm > up || bm < lo + kClampReach)) {
#pragma unroll
      for (int v = 0; v < 16; v++) x[v] = __builtin_amdgcn_fmed3f(x[v], lo, up);
      if (last) drop_past_end();
      bm = __builtin_amdgcn_fmed3f(bm, lo, up);
    }
    if (first || __builtin_amdgcn_ballot_w64(bm > kSlack)) {
      // Move m to the pair's maximum, rounded to the nearest f16: the first
      // block sets it, a later one only raises it. Within [-kLogitBound,
      // kLogitBound] the rounding is at most 8, so every probability stays
      // within [2^-8, 2^8] of the largest one's 1.
      const float pm = fmaxf(bm, __shfl_xor(bm, 32));
      const float want = first ? pm : m + fmaxf(pm, 0.0f);
      const float mn = (float)(half_t)want;
      const float delta = mn - m;
#pragma unroll
      for (int v = 0; v < 16; v++) x[v] -= delta;
      lo -= delta;
      up -= delta;
      if (!first) {
        const float f = __builtin_amdgcn_exp2f(-delta);
        run_sum *= f;
#pragma unroll
        for (int v = 0; v < 16; v++) o[v] *= f;
      }
      m = mn;
      if (!hi) bm_frag[1] = (half_t)(-mn);
    }
    half8 pf[2];
#pragma unroll
    for (int v = 0; v < 16; v += 2) {
      const half2v pp = half2v{(half_t)__builtin_amdgcn_exp2f(x[v]), (half_t)__builtin_amdgcn_exp2f(x[v + 1])};
      run_sum = __builtin_amdgcn_fdot2(pp, half2v{one, one}, run_sum, false);
      pf[v >> 3][v & 7] = pp[0];
      pf[v >> 3][(v & 7) + 1] = pp[1];
    }
#pragma unroll
    for (int s = 0; s < 2; s++) {
      const half_t* vp = &tl.v[bi][16 * s + tr_key][tr_ch];
      const short4v lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4v*)vp);
      const short4v up = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4v*)(vp + 8 * 32));
      o = mfma_f16(__builtin_bit_cast(half8, short8v{lo[0], lo[1], lo[2], lo[3], up[0], up[1], up[2], up[3]}), pf[s], o);
    }
  };

  // K and V channels past the head dimension are zero (their loads, kept
  // for a uniform count, read the row's next columns), and so are keys past
  // the last (whose loads read the next rows or the tensor's padding: a
  // probability of 0 times a non-finite value would not be 0). The zeros go
  // in at the LDS store, so no wait for the load sits at the fetch.
  const unsigned tile_keep = 8 * (tid & 3) >= a.d ? 0u : ~0u;
  const int tile_key = (tid & 127) >> 2;
  // A block's share of the loads, two sets in flight, each with the mask
  // code of the lane's key in that block. Blocks past the last one fetch the
  // last one again (and are never stored).
  const int last_k0 = ((Q - 1) >> 5) << 5;
  struct Staged {
    uint4 v[3];
    half_t code;
  };
  auto fetch = [&](int k0, Staged& st) {
    k0 = min(k0, last_k0);
    st.v[0] = *reinterpret_cast<const uint4*>(tile_src + (k0 >> 5) * tile_step);
    if (BIAS) {
      st.v[1] = *reinterpret_cast<const uint4*>(bias_src[0] + k0);
      st.v[2] = *reinterpret_cast<const uint4*>(bias_src[1] + k0);
    }
    st.code = cp[k0];
  };
  // Byte offsets into the __shared__ array (not generic pointers), so the
  // writes are LDS stores. The mask code goes through LDS too (the wave
  // reads back its own), so no register with a load in flight is live
  // across the loop's back edge, where a copy of it would wait for every
  // load.
  unsigned char* const lds_tiles = reinterpret_cast<unsigned char*>(tiles);
  const uint32_t code_dst = (uint32_t)offsetof(FlashTile, code) + 2u * (uint32_t)(wave * 32 + col);
  auto stash = [&](int t, const Staged& st, int k0) {
    unsigned char* const tb = lds_tiles + t * (uint32_t)sizeof(FlashTile);
    const uint4 tv = st.v[0];
    const unsigned keep = k0 + tile_key < Q ? tile_keep : 0u;
    *reinterpret_cast<uint4*>(tb + tile_dst) = uint4{tv.x & keep, tv.y & keep, tv.z & keep, tv.w & keep};
    if (BIAS) {
      *reinterpret_cast<uint4*>(tb + bias_dst[0]) = st.v[1];
      *reinterpret_cast<uint4*>(tb + bias_dst[1]) = st.v[2];
    }
    *reinterpret_cast<half_t*>(tb + code_dst) = st.code;
  };
  // Block j computes from LDS buffer j % 2 while the lane holds blocks j + 1
  // and j + 2 in registers (sets alternating, so the loop is unrolled by
  // two): after the compute it stores block j + 1, and after the barrier it
  // loads block j + 3 into the set just stored. A load has two blocks of
  // compute to land.
  Staged sa, sb;
  fetch(0, sa);
  stash(0, sa, 0);
  __syncthreads();
  fetch(32, sb);
  fetch(64, sa);
  if (active) step(tiles[0], 0, true);
  for (int k0 = 32, t = 1; k0 < Q;) {
    stash(t, sb, k0);
    __syncthreads();
    fetch(k0 + 64, sb);
    if (active) step(tiles[t], k0, false);
    k0 += 32;
    t ^= 1;
    if (k0 >= Q) break;
    stash(t, sa, k0);
    __syncthreads();
    fetch(k0 + 64, sa);
    if (active) step(tiles[t], k0, false);
    k0 += 32;
    t ^= 1;
  }
  run_sum += __shfl_xor(run_sum, 32);
  if (!active || myq >= Q) return;
  const float inv = 1.0f / run_sum;
  const half_t* gr = base + (row0 + myq) * ld4 + 3 * a.C + h * a.d;
  const int64_t src = a.transpose ? (int64_t)myq * a.B + b : row0 + myq;
  half_t* out = reinterpret_cast<half_t*>(a.weighted) + src * a.C + h * a.d;
  // The gate values are all read before the first store, which the
  // compiler could not move a read above (out and the gates may alias as
  // far as it knows): otherwise each read waits for a memory round trip.
  half4 gv[4];
#pragma unroll
  for (int g = 0; g < 4; g++) {
    const int c0 = 8 * g + 4 * hi;
    if (c0 < a.d) gv[g] = *reinterpret_cast<const half4*>(gr + c0);
  }
#pragma unroll
  for (int g = 0; g < 4; g++) {
    const int c0 = 8 * g + 4 * hi;
    if (c0 >= a.d) break;
    half4 r;
#pragma unroll
    for (int i = 0; i < 4; i++) r[i] = (half_t)(o[4 * g + i] * inv * (float)gv[g][i]);
    *reinterpret_cast<half4*>(out + c0) = r;
  }
}

// The same attention at head dimension 32 (every Evoformer attention), with
// more independent work a wave and no staging registers:
//  - a wave takes 64 queries of one (b, h), as two 32-query tiles against
//    each key block, so the K and V^T fragments it reads from LDS feed two
//    MFMAs each;
//  - a workgroup is two batch entries by two such waves (128 queries of one
//    head per entry), four waves meeting at one barrier a key block;
//  - K, V, the pair-bias tile and the mask codes of a key block arrive by
//    DMA (buffer_load ... lds) in two LDS buffers, one block ahead. That
//    leaves room for three workgroups a CU with a pair bias (four without):
//    the latency-bound block chain gains more from the third wave a SIMD
//    than it loses to the shorter lead. A resource per batch entry ends at
//    the entry's last row, so keys past the end load as zeros; their logits
//    are then -inf (their mask codes).
//  - a block's softmax first takes the probabilities at the current offset
//    m. When the tile's clamp bounds are far from m and every lane's 16
//    probabilities sum below 2^7 (so each is below 2^7), the exact path
//    would neither clamp (its clamped logits underflow to 0 either way) nor
//    move m, and would compute the same probabilities: they are kept. The
//    first block (and, with a pair bias, the last) and any block whose
//    check fails run the exact path of the kernel above.
// LDS buffer: K [entry][key][channel], the four 16-byte granules of key r
// stored at granule ^ ((r / 4) mod 4), so a fragment read's 16 keys fall on
// 16 different granules of the bank width, while each DMA instruction reads
// 16 keys' whole 64-byte pieces (32 keys' half pieces touched twice as many
// lines); V [entry][key][channel] (64-byte rows for the transposing reads);
// mask codes, 64 bytes an entry, both entries' brought by one DMA
// instruction of wave 0 (one resource over the pair's two code rows; a
// missing second entry reads zeros); pair bias [query][key] f32, the eight
// 16-byte granules of row q stored at granule ^ ((q / 2) mod 8): a fragment
// read's 16 consecutive rows then fall on 16 different granules of the LDS's
// 256-byte bank width (with ^ (q mod 8), rows q and q + 8 collided).
constexpr int kF2Entries = 2;
constexpr int kF2QueryWaves = 2;
constexpr int kF2Tiles = 2;
constexpr int kF2Threads = 64 * kF2Entries * kF2QueryWaves;
constexpr int kF2Queries = 32 * kF2Tiles * kF2QueryWaves;  // of each entry
constexpr int kF2Buffers = 2;
constexpr int kF2HeadGroup = 4;  // heads an XCD's workgroups share (grid order)
constexpr int kF2K = 0, kF2V = 4096, kF2Code = 8192, kF2Bias = 9216;
constexpr int kF2BufBias = kF2Bias + kF2Queries * 128;
constexpr int kF2BufNoBias = kF2Bias;
constexpr float kF2FastSum = 128.0f;

template <bool BIAS>
__global__ __launch_bounds__(kF2Threads, BIAS ? 3 : 4) void attention_flash2_kernel(FlashArgs a) {
  extern __shared__ __attribute__((aligned(1024))) unsigned char smem[];
  constexpr int BUF = BIAS ? kF2BufBias : kF2BufNoBias;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 31, hi = lane >> 5;
  const int bi = wave / kF2QueryWaves, qi = wave % kF2QueryWaves;
  const int Q = a.Q, C = a.C;
  const int qblocks = (Q + kF2Queries - 1) / kF2Queries;
  // Workgroups run on the XCDs in turn; renumbered so that each XCD takes a
  // contiguous range. Within it the order is (head group, batch pair, head,
  // query block), four heads a group: the workgroups of one batch pair and
  // head group run together and share that XCD's L2 (the group's heads read
  // every byte of the 128-byte lines of K and V they touch), and those an
  // XCD runs at once need the pair bias of four heads, not of all eight of
  // the MSA attentions. Groups of 2 and 8 heads measured slower. (With a
  // head count that 4 does not divide: (batch pair, head, query block).)
  const unsigned G = gridDim.x;
  const unsigned vid = (G % 8 == 0) ? (blockIdx.x % 8) * (G / 8) + blockIdx.x / 8 : blockIdx.x;
  const int hp = a.H % kF2HeadGroup == 0 ? kF2HeadGroup : a.H;
  const unsigned per_pair = (unsigned)(hp * qblocks);
  const unsigned pairs = (unsigned)((a.B + kF2Entries - 1) / kF2Entries);
  const unsigned hg = vid / (pairs * per_pair), rr = vid % (pairs * per_pair);
  const int qb = (int)(rr % qblocks);
  const int h = (int)(hg * hp + (rr % per_pair) / qblocks);
  const int64_t b0 = (int64_t)(rr / per_pair) * kF2Entries;
  const int qbase = qb * kF2Queries;
  const half_t* base = reinterpret_cast<const half_t*>(a.qkvg);
  const int64_t ld4 = 4 * (int64_t)C;
  const uint32_t row_bytes = (uint32_t)(2 * ld4);

  // This wave's batch entry; an entry past the last loads the last one's rows
  // (never used).
  const int64_t b = b0 + bi;
  const int64_t be = b < a.B ? b : a.B - 1;
  const int32x4_t kv_rsrc = make_rsrc(base + be * Q * ld4, (uint32_t)Q * row_bytes);
  const int32x4_t code_rsrc =
      make_rsrc(a.key_mask + b0 * a.code_stride, 2u * (uint32_t)a.code_stride * (uint32_t)min<int64_t>(2, a.B - b0));
  int32x4_t bias_rsrc{};
  if (BIAS) bias_rsrc = make_rsrc(a.bias + (int64_t)h * Q * a.stride, 4u * (uint32_t)Q * (uint32_t)a.stride);
  const uint32_t lds0 = (uint32_t)reinterpret_cast<uintptr_t>(smem);
  // Per-lane parts of the block's DMA offsets (block k0 adds k0 rows or keys).
  const int k_key = 16 * qi + (lane >> 2);
  const uint32_t k_off = (uint32_t)(2 * (C + 32 * h) + 16 * ((lane & 3) ^ ((k_key >> 2) & 3)));
  const uint32_t v_off = (uint32_t)(2 * (2 * C + 32 * h) + 16 * (lane & 3));
  const int v_key = 16 * qi + (lane >> 2);
  // Bias load n (rows 8 n + lane / 8) puts granule g of its row at slot
  // g ^ ((row / 2) mod 8) = g ^ (4 (n mod 2) + lane / 16): the lane at slot
  // lane % 8 fetches that granule.
  auto b_gran = [&](int n) { return (uint32_t)(16 * ((lane & 7) ^ (4 * (n & 1) + (lane >> 4)))); };
  auto issue = [&](int j) {
    const uint32_t buf = lds0 + (uint32_t)((j % kF2Buffers) * BUF);
    const int k0 = 32 * j;
    dma16(kv_rsrc, buf + kF2K + 2048 * bi + 1024 * qi, (uint32_t)(k0 + k_key) * row_bytes + k_off);
    dma16(kv_rsrc, buf + kF2V + 2048 * bi + 1024 * qi, (uint32_t)(k0 + v_key) * row_bytes + v_off);
    if (wave == 0)
      dma4(code_rsrc, buf + kF2Code,
           lane < 32 ? 2u * ((uint32_t)(lane >> 4) * (uint32_t)a.code_stride + (uint32_t)(k0 + 2 * (lane & 15)))
                     : kOutOfRange);
    if (BIAS) {
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int n = 4 * wave + i;  // bias rows 8 n .. 8 n + 7 of the workgroup's 128
        dma16(bias_rsrc, buf + kF2Bias + 1024 * n,
              4u * ((uint32_t)(qbase + 8 * n + (lane >> 3)) * (uint32_t)a.stride + (uint32_t)k0) + b_gran(n));
      }
    }
  };
  const int nblk = (Q + 31) >> 5;
  issue(0);

  // This wave's queries: tile t holds qbase + 32 (2 qi + t) + col.
  const bool active = b < a.B && qbase + 64 * qi < Q;  // idle waves still load and meet every barrier
  const int64_t row0 = be * Q;
  half8 qf[kF2Tiles][2];
#pragma unroll
  for (int t = 0; t < kF2Tiles; t++) {
    const int q = min(qbase + 32 * (2 * qi + t) + col, Q - 1);
    const half_t* qr = base + (row0 + q) * ld4 + 32 * h + 8 * hi;
    qf[t][0] = *reinterpret_cast<const half8*>(qr);
    qf[t][1] = *reinterpret_cast<const half8*>(qr + 16);
  }
  // Everything in flight, the query fragments included, lands here: the
  // compiler then knows no load of its own is outstanding in the loop, where
  // its wait for one would also wait for every DMA issued after it.
  wait_vmcnt<0>();

  floatx16 o[kF2Tiles];
  float run_sum[kF2Tiles], lo[kF2Tiles], up[kF2Tiles];
  // How far the clamp bounds are from m beyond what the fast softmax needs
  // (up >= kSlack + 1, lo <= -kClampReach); negative before the first block.
  float margin[kF2Tiles];
  half4 bm_frag[kF2Tiles];
  const half_t one = (half_t)1.0f;
#pragma unroll
  for (int t = 0; t < kF2Tiles; t++) {
    o[t] = floatx16{};
    run_sum[t] = 0.0f;
    lo[t] = -kLogitBound;
    up[t] = kLogitBound;
    margin[t] = -1.0f;
    // The mask step's B operand, (kMaskScale, -m) per query: every lane holds
    // it (the A operand is zero on lanes 32-63), so m reads back from it.
    bm_frag[t] = half4{(half_t)kMaskScale, (half_t)0.0f, (half_t)0.0f, (half_t)0.0f};
  }
  const int tr_key = 4 * hi + ((lane & 15) >> 2), tr_ch = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);

  // The exact softmax step of one tile (the kernel above): the clamp where it
  // can matter, m moved, then the probabilities. Keys past the end come with
  // -inf logits (their mask codes), which the clamp leaves alone. (The
  // variant without a pair bias sets them again in the last block, as the
  // kernel above does: its registers then fit four waves a SIMD. The
  // threshold passes through an empty asm so that the compares stay in the
  // last block instead of being computed ahead in every block.)
  auto exact = [&](int t, floatx16& x, bool first, bool last, int k0, half8 (&pf)[2]) {
    auto drop_past_end = [&]() {
      int rem = Q - k0 - 4 * hi;  // element 4 g + i is key k0 + 8 g + 4 hi + i
      asm volatile("" : "+v"(rem));
#pragma unroll
      for (int g = 0; g < 4; g++)
#pragma unroll
        for (int i = 0; i < 4; i++)
          if (8 * g + i >= rem) x[4 * g + i] = -INFINITY;
    };
    if (!BIAS && last) drop_past_end();
    float bm = x[0];
#pragma unroll
    for (int v = 1; v < 16; v++) bm = fmaxf(bm, x[v]);
    if (__builtin_amdgcn_ballot_w64(bm > up[t] || bm < lo[t] + kClampReach)) {
#pragma unroll
      for (int v = 0; v < 16; v++)
        x[v] = x[v] == -INFINITY ? x[v] : __builtin_amdgcn_fmed3f(x[v], lo[t], up[t]);
      if (!BIAS && last) drop_past_end();
      bm = __builtin_amdgcn_fmed3f(bm, lo[t], up[t]);
    }
    if (first || __builtin_amdgcn_ballot_w64(bm > kSlack)) {
      const float m = -(float)bm_frag[t][1];
      const float pm = fmaxf(bm, __shfl_xor(bm, 32));
      const float want = first ? pm : m + fmaxf(pm, 0.0f);
      const float mn = (float)(half_t)want;
      const float delta = mn - m;
#pragma unroll
      for (int v = 0; v < 16; v++) x[v] -= delta;
      lo[t] -= delta;
      up[t] -= delta;
      if (!first) {
        const float f = __builtin_amdgcn_exp2f(-delta);
        run_sum[t] *= f;
#pragma unroll
        for (int v = 0; v < 16; v++) o[t][v] *= f;
      }
      bm_frag[t][1] = (half_t)(-mn);
    }
#pragma unroll
    for (int v = 0; v < 16; v += 2) {
      const half2v pp = half2v{(half_t)__builtin_amdgcn_exp2f(x[v]), (half_t)__builtin_amdgcn_exp2f(x[v + 1])};
      run_sum[t] = __builtin_amdgcn_fdot2(pp, half2v{one, one}, run_sum[t], false);
      pf[v >> 3][v & 7] = pp[0];
      pf[v >> 3][(v & 7) + 1] = pp[1];
    }
    margin[t] = fminf(up[t] - (kSlack + 1.0f), -kClampReach - lo[t]);
  };

  for (int j = 0; j < nblk; j++) {
    // Block j is the only one in flight; once it has landed the barrier
    // publishes it and retires buffer (j + 1) % 2, whose block j - 1 every
    // wave has finished.
    wait_vmcnt<0>();
    block_barrier<false>();
    if (j + 1 < nblk) issue(j + 1);
    if (!active) continue;
    const unsigned char* bp = smem + (j % kF2Buffers) * BUF;
    const bool first = j == 0;
    const unsigned char* kp = bp + kF2K + 2048 * bi + 64 * col;
    const int ksw = (col >> 2) & 3;
    const half8 kf0 = *reinterpret_cast<const half8*>(kp + 16 * (hi ^ ksw));
    const half8 kf1 = *reinterpret_cast<const half8*>(kp + 16 * ((2 + hi) ^ ksw));
    const half_t code = *reinterpret_cast<const half_t*>(bp + kF2Code + 64 * bi + 2 * col);
    const half4 am = hi ? half4{} : half4{code, one, (half_t)0.0f, (half_t)0.0f};
    floatx16 sc[kF2Tiles];
#pragma unroll
    for (int t = 0; t < kF2Tiles; t++) {
      sc[t] = floatx16{};
      if constexpr (BIAS) {
        const unsigned char* brow = bp + kF2Bias + 128 * (32 * (2 * qi + t) + col);
#pragma unroll
        for (int g = 0; g < 4; g++) {
          const float4 v = *reinterpret_cast<const float4*>(brow + 16 * ((2 * g + hi) ^ ((col >> 1) & 7)));
          sc[t][4 * g] = v.x, sc[t][4 * g + 1] = v.y, sc[t][4 * g + 2] = v.z, sc[t][4 * g + 3] = v.w;
        }
      }
      sc[t] = mfma_f16(kf0, qf[t][0], sc[t]);
      sc[t] = mfma_f16(kf1, qf[t][1], sc[t]);
      sc[t] = __builtin_amdgcn_mfma_f32_32x32x8f16(am, bm_frag[t], sc[t], 0, 0, 0);
    }
    const unsigned char* vp = bp + kF2V + 2048 * bi + 64 * tr_key + 2 * tr_ch;
    auto read_v = [&](int s) {
      const short4v l4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4v*)(vp + 1024 * s));
      const short4v u4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4v*)(vp + 1024 * s + 512));
      return __builtin_bit_cast(half8, short8v{l4[0], l4[1], l4[2], l4[3], u4[0], u4[1], u4[2], u4[3]});
    };
    // A tile's probabilities at the current offset and their sum; whether
    // the exact step must redo them.
    half8 pf[kF2Tiles][2];
    float bs[kF2Tiles];
    auto fast = [&](int t) {
      bs[t] = 0.0f;
#pragma unroll
      for (int v = 0; v < 16; v += 2) {
        const half2v pp =
            half2v{(half_t)__builtin_amdgcn_exp2f(sc[t][v]), (half_t)__builtin_amdgcn_exp2f(sc[t][v + 1])};
        bs[t] = __builtin_amdgcn_fdot2(pp, half2v{one, one}, bs[t], false);
        pf[t][v >> 3][v & 7] = pp[0];
        pf[t][v >> 3][(v & 7) + 1] = pp[1];
      }
      return __builtin_amdgcn_ballot_w64(!(bs[t] < kF2FastSum) || margin[t] < 0.0f);
    };
    {
      // One tile at a time, V^T after: fewer live registers, for three waves a
      // SIMD with a pair bias, four without.
#pragma unroll
      for (int t = 0; t < kF2Tiles; t++) {
        // The fast check holds in the last block too (keys past the end
        // have -inf logits); the variant without a bias uses it there, the
        // one with a bias keeps the exact step, which its registers favour
        // (three waves a SIMD measured faster that way).
        const bool last = j + 1 == nblk;
        bool slow = first || (BIAS && last);
        if (!slow) {
          slow = fast(t) != 0;
          if (!slow) run_sum[t] += bs[t];
        }
        if (slow) exact(t, sc[t], first, last, 32 * j, pf[t]);
      }
#pragma unroll
      for (int s = 0; s < 2; s++) {
        const half8 vf = read_v(s);
#pragma unroll
        for (int t = 0; t < kF2Tiles; t++) o[t] = mfma_f16(vf, pf[t][s], o[t]);
      }
    }
  }
  if (!active) return;
#pragma unroll
  for (int t = 0; t < kF2Tiles; t++) {
    const float rs = run_sum[t] + __shfl_xor(run_sum[t], 32);
    const int myq = qbase + 32 * (2 * qi + t) + col;
    if (myq >= Q) continue;
    const float inv = 1.0f / rs;
    const half_t* gr = base + (row0 + myq) * ld4 + 3 * C + 32 * h;
    const int64_t src = a.transpose ? (int64_t)myq * a.B + b : row0 + myq;
    half_t* out = reinterpret_cast<half_t*>(a.weighted) + src * C + 32 * h;
    half4 gv[4];
#pragma unroll
    for (int g = 0; g < 4; g++) gv[g] = *reinterpret_cast<const half4*>(gr + 8 * g + 4 * hi);
#pragma unroll
    for (int g = 0; g < 4; g++) {
      half4 r;
#pragma unroll
      for (int i = 0; i < 4; i++) r[i] = (half_t)(o[t][4 * g + i] * inv * (float)gv[g][i]);
      *reinterpret_cast<half4*>(out + 8 * g + 4 * hi) = r;
    }
  }
}

// Whether a call can take the head-dimension-32 kernel: its 32-bit buffer
// offsets cover an entry's rows, a head's bias plane and the read-ahead.
bool flash2_eligible(const afhip_attention_desc& d, int stride) {
  const int64_t Q = d.queries;
  return fast_path(d) && d.channels / d.heads == 32 && (Q + 32) * 8 * (int64_t)d.channels < ((int64_t)1 << 31) &&
         (Q + kF2Queries) * (int64_t)stride * 4 < ((int64_t)1 << 31);
}

// out += y over f16 tensors (f32 sum, one rounding): the residual step of
// an output projection the streaming kernel computed without it.
__global__ __launch_bounds__(256) void attention_residual_kernel(half_t* __restrict__ out,
                                                                 const half_t* __restrict__ y, int64_t n) {
  const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 8;
  if (i + 8 <= n) {
    half8 a = *reinterpret_cast<const half8*>(out + i);
    const half8 b = *reinterpret_cast<const half8*>(y + i);
#pragma unroll
    for (int e = 0; e < 8; e++) a[e] = (half_t)((float)a[e] + (float)b[e]);
    *reinterpret_cast<half8*>(out + i) = a;
  } else {
    for (int64_t j = i; j < n; j++) out[j] = (half_t)((float)out[j] + (float)y[j]);
  }
}

template <typename IT, typename OT>
int launch_rows_typed(const RowsArgs& r, const char* label, hipStream_t st) {
  const bool vec = (reinterpret_cast<uintptr_t>(r.x) & 15) == 0 &&
                   (!r.out || (reinterpret_cast<uintptr_t>(r.out) & 15) == 0);
  const dim3 block(256);
  const bool fits = (!r.w || r.H <= 8) && r.rows < ((int64_t)1 << 24);
  const bool four = !r.w || r.H <= 4;
  auto grid = [&](int per_block) { return dim3((unsigned)std::min<int64_t>(ceil_div(r.rows, per_block), 4096)); };
  if (vec && fits && r.C == 64)
    return four ? launch(label, attention_rows_kernel<IT, OT, 8, 4>, grid(32), block, 0, st, r)
                : launch(label, attention_rows_kernel<IT, OT, 8, 8>, grid(32), block, 0, st, r);
  if (vec && fits && r.C == 128)
    return four ? launch(label, attention_rows_kernel<IT, OT, 16, 4>, grid(16), block, 0, st, r)
                : launch(label, attention_rows_kernel<IT, OT, 16, 8>, grid(16), block, 0, st, r);
  if (vec && fits && r.C == 256)
    return four ? launch(label, attention_rows_kernel<IT, OT, 32, 4>, grid(8), block, 0, st, r)
                : launch(label, attention_rows_kernel<IT, OT, 32, 8>, grid(8), block, 0, st, r);
  return launch(label, attention_rows_any_kernel<IT, OT>, dim3((unsigned)ceil_div(r.rows, 4)), block, 0, st, r);
}

int launch_rows(const RowsArgs& r, int in_dtype, int out_dtype, const char* label, hipStream_t st) {
  if (in_dtype == AFHIP_F16)
    return out_dtype == AFHIP_F16 ? launch_rows_typed<half_t, half_t>(r, label, st)
                                  : launch_rows_typed<half_t, float>(r, label, st);
  return out_dtype == AFHIP_F16 ? launch_rows_typed<float, half_t>(r, label, st)
                                : launch_rows_typed<float, float>(r, label, st);
}

}  // namespace

extern "C" {

int afhip_attention_weights_size(const afhip_attention_desc* desc, size_t* bytes) {
  if (int s = validate(desc)) return s;
  AFHIP_REQUIRE(bytes != nullptr, "output is NULL");
  *bytes = weights_layout(*desc).total;
  return AFHIP_OK;
}

int afhip_attention_workspace_size(const afhip_attention_desc* desc, size_t* bytes) {
  if (int s = validate(desc)) return s;
  AFHIP_REQUIRE(bytes != nullptr, "output is NULL");
  *bytes = workspace_layout(*desc).total;
  return AFHIP_OK;
}

int afhip_attention_prepare_weights(const afhip_attention_desc* desc, const float* packed, void* prepared,
                                    void* stream) {
  if (int s = require_open()) return s;
  if (int s = validate(desc)) return s;
  AFHIP_REQUIRE(packed && prepared, "NULL weights");
  const auto& d = *desc;
  const AttentionWeights w = weights_layout(d);
  char* p = (char*)prepared;
  const int sep = d.pair_bias == AFHIP_PAIR_BIAS_SEPARATE;
  const int pc = sep ? d.pair_channels : d.channels;
  hipStream_t st = (hipStream_t)stream;
  if (d.precision == AFHIP_PRECISION_F16)
    return launch("attention.prepare", attention_prepare_kernel<half_t>, dim3(1024), dim3(256), 0, st, packed,
                  d.channels, d.heads, pc, sep, d.pair_bias != 0, (float*)(p + w.ln_scale), (float*)(p + w.ln_offset),
                  (half_t*)(p + w.w_proj), (float*)(p + w.b_proj), (half_t*)(p + w.w_out), (float*)(p + w.b_out),
                  (float*)(p + w.pair_scale), (float*)(p + w.pair_offset), (float*)(p + w.w_bias));
  return launch("attention.prepare", attention_prepare_kernel<float>, dim3(1024), dim3(256), 0, st, packed,
                d.channels, d.heads, pc, sep, d.pair_bias != 0, (float*)(p + w.ln_scale), (float*)(p + w.ln_offset),
                (float*)(p + w.w_proj), (float*)(p + w.b_proj), (float*)(p + w.w_out), (float*)(p + w.b_out),
                (float*)(p + w.pair_scale), (float*)(p + w.pair_offset), (float*)(p + w.w_bias));
}

int afhip_attention_run(const afhip_attention_desc* desc, const void* activations, const float* mask,
                        const void* pair_activations, const void* prepared, void* out, void* workspace,
                        size_t workspace_bytes, void* stream) {
  if (int s = require_open()) return s;
  if (int s = validate(desc)) return s;
  AFHIP_REQUIRE(activations && mask && prepared && out, "NULL tensor");
  const auto& d = *desc;
  AFHIP_REQUIRE(d.pair_bias != AFHIP_PAIR_BIAS_SEPARATE || pair_activations != nullptr,
                "a separate pair bias needs its pair activations");
  const AttentionWeights w = weights_layout(d);
  const AttentionWorkspace ws = workspace_layout(d);
  AFHIP_REQUIRE(workspace && workspace_bytes >= ws.total, "workspace of %zu bytes is smaller than %zu",
                workspace_bytes, ws.total);
  hipStream_t st = (hipStream_t)stream;
  const bool f16 = d.precision == AFHIP_PRECISION_F16;
  const bool fast = fast_path(d);
  const float unit = fast ? kLog2e : 1.0f;  // logits in base-2 units on the fast path
  const int ct = f16 ? AFHIP_F16 : AFHIP_F32;
  const char* wp = (const char*)prepared;
  char* wsb = (char*)workspace;
  const int B = d.batch, Q = d.queries, C = d.channels, H = d.heads;
  const int64_t rows = (int64_t)B * Q;
  float* bias = d.pair_bias ? (float*)(wsb + ws.bias) : nullptr;
  int s;

  // 1. LayerNorm in attention order, the key bias, and a normalized-input pair bias.
  {
    RowsArgs r{};
    r.x = activations;
    r.rows = rows;
    r.C = C;
    r.B = B;
    r.Q = Q;
    r.transpose = d.transpose;
    r.scale = (const float*)(wp + w.ln_scale);
    r.offset = (const float*)(wp + w.ln_offset);
    r.eps = d.epsilon;
    r.out = wsb + ws.normalized;
    r.mask = mask;
    if (fast) {
      r.key_mask = (half_t*)(wsb + ws.key_mask);
    } else {
      r.key_bias = (float*)(wsb + ws.key_bias);
      r.key_scale = 1e9f;
    }
    if (d.pair_bias == AFHIP_PAIR_BIAS_NORMALIZED_INPUT) {
      r.w = (const float*)(wp + w.w_bias);
      r.H = H;
      r.bias_scale = unit;
      r.bias = bias;
    }
    r.stride = ws.stride;
    r.code_stride = ws.code_stride;
    if ((s = launch_rows(r, d.in_dtype, ct, "attention.norm", st))) return s;
  }
  // 2. A separate pair source: its own LayerNorm, projected to the heads.
  if (d.pair_bias == AFHIP_PAIR_BIAS_SEPARATE) {
    RowsArgs r{};
    r.x = pair_activations;
    r.rows = (int64_t)Q * Q;
    r.C = d.pair_channels;
    r.B = Q;
    r.Q = Q;
    r.scale = (const float*)(wp + w.pair_scale);
    r.offset = (const float*)(wp + w.pair_offset);
    r.eps = d.epsilon;
    r.w = (const float*)(wp + w.w_bias);
    r.H = H;
    r.bias_scale = unit;
    r.bias = bias;
    r.stride = ws.stride;
    if ((s = launch_rows(r, d.in_dtype, AFHIP_F32, "attention.pair_bias", st))) return s;
  }
  // 3. q, k, v, g in one GEMM with the ATTENTION epilogue.
  {
    GemmArgs g;
    g.a = wsb + ws.normalized;
    g.b = wp + w.w_proj;
    g.c = wsb + ws.qkvg;
    g.bias = (const float*)(wp + w.b_proj);
    g.M = (int)rows;
    g.N = 4 * C;
    g.K = C;
    g.lda = C;
    g.ldb = C;
    g.ldc = 4 * C;
    g.flags = AFHIP_EPILOGUE_BIAS | AFHIP_EPILOGUE_ATTENTION;
    g.head_cols = C;
    g.q_scale = unit / sqrtf((float)(C / H));
    GemmTypes t{d.precision, ct, ct, ct};
    if ((s = run_gemm(g, t, select_variant(t, g.M, g.N, g.K, 1), "attention.project", st))) return s;
  }
  // 4. Attention.
  {
    FlashArgs fa{};
    fa.qkvg = wsb + ws.qkvg;
    fa.key_bias = (const float*)(wsb + ws.key_bias);
    fa.key_mask = (const half_t*)(wsb + ws.key_mask);
    fa.bias = bias;
    fa.weighted = wsb + ws.weighted;
    fa.B = B;
    fa.Q = Q;
    fa.C = C;
    fa.H = H;
    fa.d = C / H;
    fa.transpose = d.transpose;
    fa.stride = ws.stride;
    fa.code_stride = ws.code_stride;
    fa.clamp = 1e8f;
    if (flash2_eligible(d, ws.stride)) {
      const int64_t groups = ceil_div(B, kF2Entries) * H * ceil_div(Q, kF2Queries);
      AFHIP_REQUIRE(groups < ((int64_t)1 << 31), "attention grid too large");
      if (bias) {
        auto k = attention_flash2_kernel<true>;
        if ((s = allow_lds((const void*)k, kF2Buffers * kF2BufBias))) return s;
        s = launch("attention.flash", k, dim3((unsigned)groups), dim3(kF2Threads), kF2Buffers * kF2BufBias, st, fa);
      } else {
        auto k = attention_flash2_kernel<false>;
        if ((s = allow_lds((const void*)k, kF2Buffers * kF2BufNoBias))) return s;
        s = launch("attention.flash", k, dim3((unsigned)groups), dim3(kF2Threads), kF2Buffers * kF2BufNoBias, st,
                   fa);
      }
    } else if (fast) {
      const int64_t groups = ceil_div(B, kFlashBatch) * H * ceil_div(Q, 32 * kFlashQueryWaves);
      AFHIP_REQUIRE(groups < ((int64_t)1 << 31), "attention grid too large");
      s = bias ? launch("attention.flash", attention_flash_f16_kernel<true>, dim3((unsigned)groups),
                        dim3(kFlashThreads), 0, st, fa)
               : launch("attention.flash", attention_flash_f16_kernel<false>, dim3((unsigned)groups),
                        dim3(kFlashThreads), 0, st, fa);
    } else {
      s = f16 ? launch_flash_generic<half_t>(fa, st, std::make_integer_sequence<int, 32>{})
              : launch_flash_generic<float>(fa, st, std::make_integer_sequence<int, 32>{});
    }
    if (s) return s;
  }
  // 5. The output projection, rows in source order.
  {
    GemmArgs g;
    g.a = wsb + ws.weighted;
    g.b = wp + w.w_out;
    g.c = out;
    g.residual = out;
    g.bias = (const float*)(wp + w.b_out);
    g.M = (int)rows;
    g.N = C;
    g.K = C;
    g.lda = C;
    g.ldb = C;
    g.ldc = C;
    g.flags = AFHIP_EPILOGUE_BIAS | (d.residual ? AFHIP_EPILOGUE_RESIDUAL : 0u);
    GemmTypes t{d.precision, ct, ct, d.out_dtype};
    // With the residual, the streaming kernel adds the f16 projection into
    // the output itself (f32 sum, one rounding) at C <= 128, reading the old
    // values a tile ahead of its stores. At C = 256 its registers are full:
    // it writes the projection to the (by now unused) normalised rows, and a
    // vectorised pass adds them in, to the same result.
    GemmArgs gs = g;
    gs.flags &= ~AFHIP_EPILOGUE_RESIDUAL;
    gs.residual = nullptr;
    const bool fused = C <= 128;
    if (d.residual && !fused) gs.c = wsb + ws.normalized;
    const bool aligned = (reinterpret_cast<uintptr_t>(out) & 15) == 0;
    if (stream_eligible(gs, t) && (!d.residual || aligned)) {
      if ((s = run_gemm_stream(gs, t, "attention.output", st, d.residual && fused))) return s;
      if (d.residual && !fused) {
        const int64_t n = rows * C;
        if ((s = launch("attention.residual", attention_residual_kernel, dim3((unsigned)ceil_div(n, 2048)),
                        dim3(256), 0, st, (half_t*)out, (const half_t*)(wsb + ws.normalized), n)))
          return s;
      }
    } else if ((s = run_gemm(g, t, select_variant(t, g.M, g.N, g.K, 1), "attention.output", st))) {
      return s;
    }
  }
  return AFHIP_OK;
}

}  // extern "C"

}  // namespace afhip
