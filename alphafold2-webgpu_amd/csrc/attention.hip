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
// The attention step itself is a flash kernel. At f16 precision with
// head_dim 32 it runs on the MFMA as S^T = K Q^T and O^T = V^T P^T: a lane
// then holds one query's scores for 16 keys and the same query's output for
// 16 channels, so the running maximum, sum and rescale stay inside the lane
// (one exchange with the lane 32 away), and the probabilities feed the second
// MFMA from the registers they were computed in. Any other head dimension or
// f32 precision runs a one-thread-per-query kernel in f32.
#include <algorithm>
#include <cmath>
#include <utility>

#include "gemm.h"

namespace afhip {

namespace {

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

struct AttentionWorkspace {
  size_t normalized, key_bias, qkvg, bias, weighted, total;
  int bias_stride;
};

AttentionWorkspace workspace_layout(const afhip_attention_desc& d) {
  AttentionWorkspace w{};
  const size_t es = d.precision == AFHIP_PRECISION_F16 ? 2 : 4;
  const size_t rows = (size_t)d.batch * d.queries, C = d.channels;
  size_t at = 0;
  auto take = [&](size_t bytes) {
    size_t here = at;
    at = round_up((int64_t)(at + bytes), 256);
    return here;
  };
  w.bias_stride = (int)round_up(d.queries, 4);
  w.normalized = take(es * rows * C);
  w.key_bias = take(4 * rows);
  w.qkvg = take(es * rows * 4 * C);
  w.bias = take(d.pair_bias ? 4 * (size_t)d.heads * d.queries * w.bias_stride : 0);
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

// LayerNorm of the rows in attention order, one wave a row: x_hat in the
// compute dtype, and the row's key bias 1e9 (mask - 1) (attention.ts:688-690).
template <typename IT, typename CT>
__global__ __launch_bounds__(256) void attention_norm_kernel(const IT* __restrict__ x, const float* __restrict__ mask,
                                                             int B, int Q, int C, int transpose,
                                                             const float* __restrict__ scale,
                                                             const float* __restrict__ offset, float eps,
                                                             CT* __restrict__ out, float* __restrict__ key_bias) {
  const int lane = threadIdx.x & 63;
  const int64_t rows = (int64_t)B * Q;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int64_t b = row / Q, q = row % Q;
  const int64_t src = transpose ? q * B + b : row;
  const IT* xr = x + src * C;
  float s = 0.0f;
  for (int c = lane; c < C; c += 64) s += ld(xr, c);
  for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
  const float mean = s / (float)C;
  float v = 0.0f;
  for (int c = lane; c < C; c += 64) {
    const float dlt = ld(xr, c) - mean;
    v += dlt * dlt;
  }
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  const float rstd = 1.0f / sqrtf(v / (float)C + eps);
  for (int c = lane; c < C; c += 64) out[row * C + c] = (CT)((ld(xr, c) - mean) * rstd * scale[c] + offset[c]);
  if (lane == 0) key_bias[row] = 1e9f * (mask[src] - 1.0f);
}

// The pair bias bias[h][q][k] (attention.ts:631-661) for q, k < Q: sixteen
// lanes a row (q, k), each taking every sixteenth channel, eight heads a pass.
// Normalized-input: the row is x_hat[q Q + k] as is. Separate: the row is the
// pair activation [q][k], LayerNormed with its own affine first.
template <typename PT>
__global__ __launch_bounds__(256) void attention_bias_kernel(const PT* __restrict__ src, int Q, int Cp, int H,
                                                             int normalize, const float* __restrict__ scale,
                                                             const float* __restrict__ offset, float eps,
                                                             const float* __restrict__ w, int stride,
                                                             float* __restrict__ bias) {
  const int lane16 = threadIdx.x & 15;
  const int64_t row = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4);
  const bool live = row < (int64_t)Q * Q;
  const int64_t r = live ? row : 0;  // a row past the end still reduces (over row 0), storing nothing
  const PT* pr = src + r * Cp;
  float mean = 0.0f, rstd = 1.0f;
  if (normalize) {
    float s = 0.0f;
    for (int c = lane16; c < Cp; c += 16) s += ld(pr, c);
    s = row_sum16(s);
    mean = s / (float)Cp;
    float v = 0.0f;
    for (int c = lane16; c < Cp; c += 16) {
      const float dlt = ld(pr, c) - mean;
      v += dlt * dlt;
    }
    rstd = 1.0f / sqrtf(row_sum16(v) / (float)Cp + eps);
  }
  const int64_t q = row / Q, k = row % Q;
  for (int h0 = 0; h0 < H; h0 += 8) {  // eight heads a pass
    float acc[8] = {};
    for (int c = lane16; c < Cp; c += 16) {
      float y = ld(pr, c);
      if (normalize) y = (y - mean) * rstd * scale[c] + offset[c];
#pragma unroll
      for (int h = 0; h < 8; h++)
        if (h0 + h < H) acc[h] += y * w[(int64_t)c * H + h0 + h];
    }
    float mine = 0.0f;
#pragma unroll
    for (int h = 0; h < 8; h++) {
      const float t = row_sum16(acc[h]);
      if (h == lane16) mine = t;
    }
    if (live && lane16 < 8 && h0 + lane16 < H) bias[((int64_t)(h0 + lane16) * Q + q) * stride + k] = mine;
  }
}

struct FlashArgs {
  const void* qkvg;         // [B Q][4C]: q (scaled), k, v, g (sigmoid)
  const float* key_bias;    // [B][Q] in attention order
  const float* bias;        // [H][Q][stride] or null
  void* weighted;           // [B Q][C] in source order
  int B, Q, C, H, d, transpose, stride;
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
    float logit = dot + a.key_bias[b * a.Q + k];
    if (a.bias) logit += a.bias[((int64_t)h * a.Q + q) * a.stride + k];
    logit = fminf(fmaxf(logit, -1e8f), 1e8f);
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
// O^T = V^T P^T; V^T's A fragment takes the same key order from an LDS copy
// of the block transposed to [d][key]. Both k-steps of the second MFMA sum
// over the block's 32 keys in a permuted order, the same on both operands.
constexpr int kFlashWaves = 4;

__global__ __launch_bounds__(64 * kFlashWaves) void attention_flash_f16_kernel(FlashArgs a) {
  __shared__ __attribute__((aligned(16))) half_t vt_all[kFlashWaves][32][32 + 8];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int col = lane & 31, hi = lane >> 5;
  const int qblocks = (a.Q + 32 * kFlashWaves - 1) / (32 * kFlashWaves);
  const int64_t bh = blockIdx.x / qblocks;
  const int h = (int)(bh % a.H);
  const int64_t b = bh / a.H;
  const int q0 = (int)(blockIdx.x % qblocks) * 32 * kFlashWaves + 32 * wave;
  if (q0 >= a.Q) return;  // the whole wave: no barrier below spans waves
  half_t(*vt)[32 + 8] = vt_all[wave];

  const half_t* base = reinterpret_cast<const half_t*>(a.qkvg);
  const int64_t ld4 = 4 * (int64_t)a.C;
  const int64_t row0 = b * a.Q;
  const int myq = q0 + col;
  const bool qlive = myq < a.Q;
  // Q^T fragments: Q[myq][16 s + 8 hi .. + 8].
  half8 qf[2];
  {
    const half_t* qr = base + (row0 + (qlive ? myq : 0)) * ld4 + h * 32;
#pragma unroll
    for (int s = 0; s < 2; s++) qf[s] = qlive ? *reinterpret_cast<const half8*>(qr + 16 * s + 8 * hi) : half8{};
  }
  const float* brow = a.bias ? a.bias + ((int64_t)h * a.Q + (qlive ? myq : 0)) * a.stride : nullptr;
  const float* kb = a.key_bias + row0;

  floatx16 o = {};  // O^T: lane holds query myq, channels 8 (v / 4) + 4 hi + v % 4
  float run_max = -1e30f, run_sum = 0.0f;
  constexpr float kLog2e = 1.4426950408889634f;
  for (int k0 = 0; k0 < a.Q; k0 += 32) {
    const int mykey = k0 + col;
    const bool klive = mykey < a.Q;
    const half_t* kr = base + (row0 + (klive ? mykey : 0)) * ld4 + a.C + h * 32;
    half8 kf[2], vraw[2];
#pragma unroll
    for (int s = 0; s < 2; s++) {
      kf[s] = klive ? *reinterpret_cast<const half8*>(kr + 16 * s + 8 * hi) : half8{};
      vraw[s] = klive ? *reinterpret_cast<const half8*>(kr + a.C + 16 * s + 8 * hi) : half8{};
    }
    // V^T for this block: vt[d][key], d = 16 s + 8 hi + e, key = col.
#pragma unroll
    for (int s = 0; s < 2; s++)
#pragma unroll
      for (int e = 0; e < 8; e++) vt[16 * s + 8 * hi + e][col] = vraw[s][e];

    floatx16 st = {};
#pragma unroll
    for (int s = 0; s < 2; s++) st = mfma_f16(kf[s], qf[s], st);

    // Logits of this lane's query for keys k0 + 8 g + 4 hi + i (g, i < 4).
    float lg[16];
    float bm = -1e30f;
#pragma unroll
    for (int g = 0; g < 4; g++) {
      const int key = k0 + 8 * g + 4 * hi;
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int kk = key + i;
        float x = -1e30f;  // keys past the end take no weight
        if (kk < a.Q) {
          x = st[4 * g + i] + kb[kk];
          if (brow) x += brow[kk];
          x = fminf(fmaxf(x, -1e8f), 1e8f);
        }
        lg[4 * g + i] = x;
        bm = fmaxf(bm, x);
      }
    }
    bm = fmaxf(bm, __shfl_xor(bm, 32));
    const float new_max = fmaxf(run_max, bm);
    const float scale = __builtin_amdgcn_exp2f((run_max - new_max) * kLog2e);
    float ps = 0.0f;
    half8 pf[2];
#pragma unroll
    for (int v = 0; v < 16; v++) {
      const float p = __builtin_amdgcn_exp2f((lg[v] - new_max) * kLog2e);
      ps += p;
      pf[v >> 3][v & 7] = (half_t)p;
    }
    ps += __shfl_xor(ps, 32);
    run_sum = run_sum * scale + ps;
    run_max = new_max;
#pragma unroll
    for (int v = 0; v < 16; v++) o[v] *= scale;

    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's V^T writes are done
    __builtin_amdgcn_wave_barrier();
    // V^T A fragments in the key order of P: keys 16 s + 4 hi + [0, 4) and
    // 16 s + 8 + 4 hi + [0, 4) for channel col.
#pragma unroll
    for (int s = 0; s < 2; s++) {
      const half4 lo = *reinterpret_cast<const half4*>(&vt[col][16 * s + 4 * hi]);
      const half4 up = *reinterpret_cast<const half4*>(&vt[col][16 * s + 8 + 4 * hi]);
      const half8 vf = half8{lo[0], lo[1], lo[2], lo[3], up[0], up[1], up[2], up[3]};
      o = mfma_f16(vf, pf[s], o);
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);  // the reads are done before the next block overwrites vt
    __builtin_amdgcn_wave_barrier();
  }
  if (!qlive) return;
  const float inv = 1.0f / run_sum;
  const half_t* gr = base + (row0 + myq) * ld4 + 3 * a.C + h * 32;
  const int64_t src = a.transpose ? (int64_t)myq * a.B + b : row0 + myq;
  half_t* out = reinterpret_cast<half_t*>(a.weighted) + src * a.C + h * 32;
#pragma unroll
  for (int g = 0; g < 4; g++) {
    const int c0 = 8 * g + 4 * hi;
    const half4 gv = *reinterpret_cast<const half4*>(gr + c0);
    half4 r;
#pragma unroll
    for (int i = 0; i < 4; i++) r[i] = (half_t)(o[4 * g + i] * inv * (float)gv[i]);
    *reinterpret_cast<half4*>(out + c0) = r;
  }
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
  const int ct = f16 ? AFHIP_F16 : AFHIP_F32;
  const char* wp = (const char*)prepared;
  char* wsb = (char*)workspace;
  const int B = d.batch, Q = d.queries, C = d.channels, H = d.heads;
  const int64_t rows = (int64_t)B * Q;
  int s;

  // 1. LayerNorm in attention order, and the key bias.
  {
    const dim3 grid((unsigned)ceil_div(rows, 4));
    const float* sc = (const float*)(wp + w.ln_scale);
    const float* of = (const float*)(wp + w.ln_offset);
    float* kb = (float*)(wsb + ws.key_bias);
    void* xn = wsb + ws.normalized;
    if (d.in_dtype == AFHIP_F32)
      s = f16 ? launch("attention.norm", attention_norm_kernel<float, half_t>, grid, dim3(256), 0, st,
                       (const float*)activations, mask, B, Q, C, d.transpose, sc, of, d.epsilon, (half_t*)xn, kb)
              : launch("attention.norm", attention_norm_kernel<float, float>, grid, dim3(256), 0, st,
                       (const float*)activations, mask, B, Q, C, d.transpose, sc, of, d.epsilon, (float*)xn, kb);
    else
      s = f16 ? launch("attention.norm", attention_norm_kernel<half_t, half_t>, grid, dim3(256), 0, st,
                       (const half_t*)activations, mask, B, Q, C, d.transpose, sc, of, d.epsilon, (half_t*)xn, kb)
              : launch("attention.norm", attention_norm_kernel<half_t, float>, grid, dim3(256), 0, st,
                       (const half_t*)activations, mask, B, Q, C, d.transpose, sc, of, d.epsilon, (float*)xn, kb);
    if (s) return s;
  }
  // 2. q, k, v, g in one GEMM with the ATTENTION epilogue.
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
    g.q_scale = 1.0f / sqrtf((float)(C / H));
    GemmTypes t{d.precision, ct, ct, ct};
    if ((s = run_gemm(g, t, select_variant(t, g.M, g.N, g.K, 1), "attention.project", st))) return s;
  }
  // 3. The pair bias.
  float* bias = nullptr;
  if (d.pair_bias) {
    bias = (float*)(wsb + ws.bias);
    const bool sep = d.pair_bias == AFHIP_PAIR_BIAS_SEPARATE;
    const int Cp = sep ? d.pair_channels : C;
    const dim3 grid((unsigned)ceil_div((int64_t)Q * Q, 16));
    const float* ps = (const float*)(wp + w.pair_scale);
    const float* po = (const float*)(wp + w.pair_offset);
    const float* wb = (const float*)(wp + w.w_bias);
    const bool src16 = sep ? d.in_dtype == AFHIP_F16 : f16;
    const void* src = sep ? pair_activations : (const void*)(wsb + ws.normalized);
    s = src16 ? launch("attention.pair_bias", attention_bias_kernel<half_t>, grid, dim3(256), 0, st,
                       (const half_t*)src, Q, Cp, H, (int)sep, ps, po, d.epsilon, wb, ws.bias_stride, bias)
              : launch("attention.pair_bias", attention_bias_kernel<float>, grid, dim3(256), 0, st,
                       (const float*)src, Q, Cp, H, (int)sep, ps, po, d.epsilon, wb, ws.bias_stride, bias);
    if (s) return s;
  }
  // 4. Attention.
  {
    FlashArgs fa{};
    fa.qkvg = wsb + ws.qkvg;
    fa.key_bias = (const float*)(wsb + ws.key_bias);
    fa.bias = bias;
    fa.weighted = wsb + ws.weighted;
    fa.B = B;
    fa.Q = Q;
    fa.C = C;
    fa.H = H;
    fa.d = C / H;
    fa.transpose = d.transpose;
    fa.stride = ws.bias_stride;
    if (f16 && fa.d == 32) {
      const int64_t qblocks = ceil_div(Q, 32 * kFlashWaves);
      AFHIP_REQUIRE((int64_t)B * H * qblocks < ((int64_t)1 << 31), "attention grid too large");
      s = launch("attention.flash", attention_flash_f16_kernel, dim3((unsigned)(B * H * qblocks)),
                 dim3(64 * kFlashWaves), 0, st, fa);
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
    if ((s = run_gemm(g, t, select_variant(t, g.M, g.N, g.K, 1), "attention.output", st))) return s;
  }
  return AFHIP_OK;
}

}  // extern "C"

}  // namespace afhip
