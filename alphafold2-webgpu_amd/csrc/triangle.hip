// Triangle multiplication (outgoing and incoming) for gfx950.
//
// Three launches per output block, replacing the reference's seven kernels
// (src/triangle/shaders.ts:151-589):
//
//  1. tri_project: LayerNorm of 64 pair rows in LDS, the four projections
//     (a, a-gate, b, b-gate) on MFMA, the gated product a = mask*(x+b)*sig(g+bg)
//     staged through LDS and stored channel-major as [c][row]. The direction
//     is folded into which pair a row reads: outgoing row r is pair r;
//     incoming row r = j*L + k reads pair (k, j). Both directions therefore
//     leave the contraction the same NT problem.
//  2. the contraction: one batched GEMM over the hidden channels through the
//     shared tiled GEMM, out[c][i][j] = sum_k R[c][i][k] C[c][j][k] with
//     (R, C) = (a, b) outgoing, (b, a) incoming. That is AlphaFold's
//     "ikc,jkc->ijc" and "kjc,kic->ijc" (src/triangle/shaders.ts:452-495).
//  3. tri_output: the contracted tile (channel-major, 64 pairs) is normalised
//     over the hidden channels in LDS and projected by linearZ; the same pairs
//     of z are normalised and projected by linearG; out = (p + bz)*sig(g + bg).
//     The gate is recomputed here from z rather than stored and re-read.
#include <algorithm>
#include <cmath>
#include <cstring>

#include "gemm.h"
#include "triangle_fast.h"

namespace afhip {

namespace {

constexpr int kRows = 64;  // pair rows per workgroup in the projection kernels
constexpr int kC = 128;    // the fast path's c_z = c_hidden

struct TriWeights {
  // Offsets in bytes into the prepared buffer.
  size_t ln_in_w, ln_in_b, w_proj, b_proj, ln_out_w, ln_out_b, w_z, b_z, w_g, b_g;
  size_t fold_w, fold_b;  // the f16 fast path's folded weights (0 when not eligible)
  size_t total;
  int czp, chp, czo;  // padded input width (multiple of 32), padded hidden, padded output rows
};

TriWeights tri_layout(const afhip_triangle_desc& d) {
  TriWeights w{};
  size_t es = d.precision == AFHIP_PRECISION_F16 ? 2 : 4;
  w.czp = (int)round_up(d.c_z, 32);
  w.chp = (int)round_up(d.c_hidden, 32);
  w.czo = (int)round_up(d.c_z, 32);
  size_t at = 0;
  auto take = [&](size_t bytes) {
    size_t here = at;
    at = round_up((int64_t)(at + bytes), 256);
    return here;
  };
  w.ln_in_w = take(4 * (size_t)d.c_z);
  w.ln_in_b = take(4 * (size_t)d.c_z);
  w.w_proj = take(es * 4 * (size_t)w.chp * w.czp);
  w.b_proj = take(4 * 4 * (size_t)w.chp);
  w.ln_out_w = take(4 * (size_t)d.c_hidden);
  w.ln_out_b = take(4 * (size_t)d.c_hidden);
  w.w_z = take(es * (size_t)w.czo * w.chp);
  w.b_z = take(4 * (size_t)w.czo);
  w.w_g = take(es * (size_t)w.czo * w.czp);
  w.b_g = take(4 * (size_t)w.czo);
  if (triangle_fast_eligible(d)) {
    w.fold_w = take(2 * (size_t)kFoldMatrices * d.c_z * d.c_z);
    w.fold_b = take(4 * (size_t)kFoldMatrices * d.c_z);
  }
  w.total = at;
  return w;
}

struct TriWorkspace {
  size_t op_a, op_b, contracted, total;
  int64_t cstride;  // elements between channels of an operand
  int64_t bstride;  // elements between channels of the contracted block
  int block_rows;
};

TriWorkspace tri_workspace(const afhip_triangle_desc& d) {
  TriWorkspace w{};
  size_t es = d.precision == AFHIP_PRECISION_F16 ? 2 : 4;
  int64_t L = d.length, P = L * L;
  w.block_rows = d.block_rows > 0 ? std::min(d.block_rows, d.length) : d.length;
  // The fast output kernels address a block's z, contracted values and
  // output with 32-bit buffer offsets: at long lengths the block shrinks to
  // what they reach (the result does not depend on the block).
  if (triangle_fast_eligible(d)) w.block_rows = std::min(w.block_rows, triangle_fast_block_rows(d));
  w.cstride = round_up(P, 64);
  w.bstride = round_up((int64_t)w.block_rows * L, 64);
  size_t at = 0;
  auto take = [&](size_t bytes) {
    size_t here = at;
    at = round_up((int64_t)(at + bytes), 256);
    return here;
  };
  w.op_a = take(es * (size_t)d.c_hidden * w.cstride);
  w.op_b = take(es * (size_t)d.c_hidden * w.cstride);
  w.contracted = take(es * (size_t)d.c_hidden * w.bstride);
  w.total = at;
  return w;
}

// ---------------------------------------------------------------------------
// Shared LDS helpers
// ---------------------------------------------------------------------------

// Mean and 1/sigma over `channels` of 64 columns of a channel-major f32 tile
// (xs[c * pitch + q]); four lanes per column, two-pass as the reference's
// statistics kernels compute them (shaders.ts:242-281, :501-522).
__device__ __forceinline__ void column_stats(const float* xs, int pitch, int channels, float eps, int tid,
                                             float& mean, float& rstd) {
  const int q = tid >> 2, part = tid & 3;
  float s = 0.0f;
  for (int c = part; c < channels; c += 4) s += xs[c * pitch + q];
  s += __shfl_xor(s, 1);
  s += __shfl_xor(s, 2);
  mean = s / (float)channels;
  float v = 0.0f;
  for (int c = part; c < channels; c += 4) {
    float d = xs[c * pitch + q] - mean;
    v += d * d;
  }
  v += __shfl_xor(v, 1);
  v += __shfl_xor(v, 2);
  rstd = fast_rsqrt(v / (float)channels + eps);
}

template <typename T> __device__ __forceinline__ float ldf(const T* p) { return (float)*p; }

// ---------------------------------------------------------------------------
// 1. Gated projections
// ---------------------------------------------------------------------------

struct ProjectArgs {
  const void* z;
  const float* mask;
  const float* ln_w;
  const float* ln_b;
  const void* w_proj;  // [4][chp][czp]: ap, ag, bp, bg
  const float* b_proj; // [4][chp]
  void* out_a;
  void* out_b;
  int64_t cstride;
  int L, P, cz, ch, czp, chp;
  int incoming;
  float eps;
};

template <typename ZT, bool F16MATH>
__global__ __launch_bounds__(256) void tri_project_kernel(ProjectArgs a) {
  using CT = typename std::conditional<F16MATH, half_t, float>::type;
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  // xs: f32 [czp][kRows + 1], channel-major raw z; an: CT [kRows][czp + 8] (f16 only);
  // stage: CT [64][kRows + 8] output transpose.
  const int xpitch = kRows + 1;
  float* xs = reinterpret_cast<float*>(smem);
  size_t off = round_up((int64_t)a.czp * xpitch * 4, 16);
  CT* an = reinterpret_cast<CT*>(smem + off);
  const int apitch = a.czp + 8;
  if (F16MATH) off += round_up((int64_t)kRows * apitch * 2, 16);
  CT* stage = reinterpret_cast<CT*>(smem + off);
  constexpr int spitch = kRows + 8;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r0 = blockIdx.x * kRows;
  const ZT* z = reinterpret_cast<const ZT*>(a.z);

  // Load 64 pair rows, transposed to channel-major in LDS.
  for (int idx = tid; idx < kRows * a.czp; idx += 256) {
    const int i = idx / a.czp, c = idx - i * a.czp;
    const int r = r0 + i;
    float v = 0.0f;
    if (r < a.P && c < a.cz) {
      const int p = a.incoming ? (r % a.L) * a.L + r / a.L : r;
      v = ldf(z + (int64_t)p * a.cz + c);
    }
    xs[c * xpitch + i] = v;
  }
  __syncthreads();
  float mean, rstd;
  column_stats(xs, xpitch, a.cz, a.eps, tid, mean, rstd);
  {
    const int q = tid >> 2, part = tid & 3;
    for (int c = part; c < a.czp; c += 4) {
      float v = c < a.cz ? (xs[c * xpitch + q] - mean) * rstd * a.ln_w[c] + a.ln_b[c] : 0.0f;
      if (F16MATH) an[q * apitch + c] = (CT)v;
      else xs[c * xpitch + q] = v;
    }
  }
  __syncthreads();

  const CT* W = reinterpret_cast<const CT*>(a.w_proj);
  const int rw = 32 * (wave & 1);
  for (int o = 0; o < 2; o++) {
    const CT* wp = W + (size_t)(2 * o) * a.chp * a.czp;
    const CT* wg = W + (size_t)(2 * o + 1) * a.chp * a.czp;
    const float* bp = a.b_proj + (2 * o) * a.chp;
    const float* bg = a.b_proj + (2 * o + 1) * a.chp;
    CT* out = reinterpret_cast<CT*>(o == 0 ? a.out_a : a.out_b);
    for (int h0 = 0; h0 < a.chp; h0 += 64) {
      const int hc = h0 + 32 * (wave >> 1);
      if (hc < a.chp) {
        floatx16 accp, accg;
#pragma unroll
        for (int v = 0; v < 16; v++) accp[v] = accg[v] = 0.0f;
        const int n = hc + (lane & 31);
        if constexpr (F16MATH) {
          for (int k = 0; k < a.czp; k += 16) {
            const int kk = k + 8 * (lane >> 5);
            half8 af = *reinterpret_cast<const half8*>(an + (rw + (lane & 31)) * apitch + kk);
            half8 bpf = *reinterpret_cast<const half8*>(wp + (size_t)n * a.czp + kk);
            half8 bgf = *reinterpret_cast<const half8*>(wg + (size_t)n * a.czp + kk);
            accp = mfma_f16(af, bpf, accp);
            accg = mfma_f16(af, bgf, accg);
          }
        } else {
          for (int k = 0; k < a.czp; k += 2) {
            const int kk = k + (lane >> 5);
            float af = xs[kk * xpitch + rw + (lane & 31)];
            accp = mfma_f32(af, wp[(size_t)n * a.czp + kk], accp);
            accg = mfma_f32(af, wg[(size_t)n * a.czp + kk], accg);
          }
        }
        const float bpv = bp[n], bgv = bg[n];
#pragma unroll
        for (int v = 0; v < 16; v++) {
          const int i = rw + mfma_row(v, lane);
          const int r = r0 + i;
          float val = 0.0f;
          if (r < a.P) {
            const int p = a.incoming ? (r % a.L) * a.L + r / a.L : r;
            val = a.mask[p] * (accp[v] + bpv) * sigmoidf_(accg[v] + bgv);
          }
          stage[(n - h0) * spitch + i] = (CT)val;
        }
      }
      __syncthreads();
      // 64 channels x 64 rows, written along the rows of each channel.
      for (int idx = tid; idx < 64 * kRows; idx += 256) {
        const int hl = idx / kRows, i = idx - hl * kRows;
        const int h = h0 + hl, r = r0 + i;
        if (h < a.ch && r < a.P) out[(int64_t)h * a.cstride + r] = stage[hl * spitch + i];
      }
      __syncthreads();
    }
  }
}

// ---------------------------------------------------------------------------
// 3. Hidden LayerNorm, output projection and gate
// ---------------------------------------------------------------------------

struct OutputArgs {
  const void* contracted;  // CT [ch][bstride], pairs of this block
  int64_t bstride;
  const void* z;
  const float* ln_in_w;
  const float* ln_in_b;
  const float* ln_out_w;
  const float* ln_out_b;
  const void* w_z;  // [czo][chp]
  const float* b_z;
  const void* w_g;  // [czo][czp]
  const float* b_g;
  void* out;
  int pair0;        // first pair of this block
  int pairs;        // pairs in this block
  int cz, ch, czp, chp;
  int residual;
  float eps;
};

// Loads 64 columns of a channel-major tile (xs[c][q]) and normalises them in
// place (f32) or into an[q][c] (f16). Returns after a barrier.
template <typename CT, bool F16MATH>
__device__ __forceinline__ void normalize_tile(float* xs, int xpitch, CT* an, int apitch, int channels, int padded,
                                               const float* w, const float* b, float eps, int tid) {
  float mean, rstd;
  column_stats(xs, xpitch, channels, eps, tid, mean, rstd);
  const int q = tid >> 2, part = tid & 3;
  __syncthreads();
  for (int c = part; c < padded; c += 4) {
    float v = c < channels ? (xs[c * xpitch + q] - mean) * rstd * w[c] + b[c] : 0.0f;
    if (F16MATH) an[q * apitch + c] = (CT)v;
    else xs[c * xpitch + q] = v;
  }
  __syncthreads();
}

// acc[t] += A (64 x K from LDS) * W^T for the wave's column tiles.
template <typename CT, bool F16MATH>
__device__ __forceinline__ void tile_gemm(floatx16 (&acc)[2], const float* xs, int xpitch, const CT* an, int apitch,
                                          const CT* W, int K, int czo, int lane, int wave) {
  const int rw = 32 * (wave & 1);
#pragma unroll
  for (int t = 0; t < 2; t++) {
    const int j = (wave >> 1) + 2 * t;
    if (32 * j >= czo) continue;
    const int n = 32 * j + (lane & 31);
    if constexpr (F16MATH) {
      for (int k = 0; k < K; k += 16) {
        const int kk = k + 8 * (lane >> 5);
        half8 af = *reinterpret_cast<const half8*>(an + (rw + (lane & 31)) * apitch + kk);
        half8 bf = *reinterpret_cast<const half8*>(W + (size_t)n * K + kk);
        acc[t] = mfma_f16(af, bf, acc[t]);
      }
    } else {
      for (int k = 0; k < K; k += 2) {
        const int kk = k + (lane >> 5);
        acc[t] = mfma_f32(xs[kk * xpitch + rw + (lane & 31)], W[(size_t)n * K + kk], acc[t]);
      }
    }
  }
}

template <typename ZT, typename OT, bool F16MATH>
__global__ __launch_bounds__(256) void tri_output_kernel(OutputArgs a) {
  using CT = typename std::conditional<F16MATH, half_t, float>::type;
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int xpitch = kRows + 1;
  const int kmax = a.chp > a.czp ? a.chp : a.czp;
  float* xs = reinterpret_cast<float*>(smem);
  CT* an = reinterpret_cast<CT*>(smem + round_up((int64_t)kmax * xpitch * 4, 16));
  const int apitch = kmax + 8;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int q0 = blockIdx.x * kRows;
  const CT* X = reinterpret_cast<const CT*>(a.contracted);
  const ZT* z = reinterpret_cast<const ZT*>(a.z);

  // Phase 1: contracted tile, channel-major as stored.
  for (int idx = tid; idx < a.chp * kRows; idx += 256) {
    const int c = idx / kRows, q = idx - c * kRows;
    float v = 0.0f;
    if (c < a.ch && q0 + q < a.pairs) v = (float)X[(int64_t)c * a.bstride + q0 + q];
    xs[c * xpitch + q] = v;
  }
  __syncthreads();
  normalize_tile<CT, F16MATH>(xs, xpitch, an, apitch, a.ch, a.chp, a.ln_out_w, a.ln_out_b, a.eps, tid);
  floatx16 accz[2], accg[2];
#pragma unroll
  for (int t = 0; t < 2; t++)
#pragma unroll
    for (int v = 0; v < 16; v++) accz[t][v] = accg[t][v] = 0.0f;
  tile_gemm<CT, F16MATH>(accz, xs, xpitch, an, apitch, reinterpret_cast<const CT*>(a.w_z), a.chp,
                         (int)round_up(a.cz, 32), lane, wave);
  __syncthreads();

  // Phase 2: the same pairs of z, transposed to channel-major.
  for (int idx = tid; idx < kRows * a.czp; idx += 256) {
    const int q = idx / a.czp, c = idx - q * a.czp;
    float v = 0.0f;
    if (c < a.cz && q0 + q < a.pairs) v = (float)z[(int64_t)(a.pair0 + q0 + q) * a.cz + c];
    xs[c * xpitch + q] = v;
  }
  __syncthreads();
  normalize_tile<CT, F16MATH>(xs, xpitch, an, apitch, a.cz, a.czp, a.ln_in_w, a.ln_in_b, a.eps, tid);
  tile_gemm<CT, F16MATH>(accg, xs, xpitch, an, apitch, reinterpret_cast<const CT*>(a.w_g), a.czp,
                         (int)round_up(a.cz, 32), lane, wave);

  OT* out = reinterpret_cast<OT*>(a.out);
  const int rw = 32 * (wave & 1);
#pragma unroll
  for (int t = 0; t < 2; t++) {
    const int j = (wave >> 1) + 2 * t;
    const int n = 32 * j + (lane & 31);
    if (n >= a.cz) continue;
    const float bz = a.b_z[n], bg = a.b_g[n];
#pragma unroll
    for (int v = 0; v < 16; v++) {
      const int q = q0 + rw + mfma_row(v, lane);
      if (q >= a.pairs) continue;
      float y = (accz[t][v] + bz) * sigmoidf_(accg[t][v] + bg);
      const int64_t at = (int64_t)(a.pair0 + q) * a.cz + n;
      if (a.residual) y += (float)out[at];
      out[at] = (OT)y;
    }
  }
}

// ---------------------------------------------------------------------------
// Weight preparation: f32 [out][in] tensors -> padded CT matrices
// ---------------------------------------------------------------------------

// The fast path's weights with the LayerNorm affines folded in, so its
// kernels normalise to x_hat = (x - mean) / sigma and nothing more:
//   W' = s W diag(gamma),  b' = s (b + W beta),
// gamma, beta the LayerNorm feeding the matrix and s = -log2(e) for the two
// gates (their sigmoid then reads 1 / (1 + 2^acc)). Matrices, in order:
// AP, AG, BP, BG (LayerNorm-in), Z (LayerNorm-out), G (LayerNorm-in), each
// 128 x 128 in MFMA fragment order (fold_index); every product and the bias
// sum are taken in double and rounded once (weights to f16, biases to f32).
struct FoldSources {
  const float* w[kFoldMatrices];
  const float* b[kFoldMatrices];
  const float* gamma[kFoldMatrices];
  const float* beta[kFoldMatrices];
  float scale[kFoldMatrices];
};

__global__ void fold_weights_kernel(FoldSources src, int n_out, int n_in, half_t* __restrict__ w_out,
                                    float* __restrict__ b_out) {
  const int id = blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= kFoldMatrices * n_out) return;
  const int m = id / n_out, n = id - m * n_out;
  const double s = src.scale[m];
  const float* w = src.w[m] + (size_t)n * n_in;
  double bias = src.b[m][n];
  for (int k = 0; k < n_in; k++) {
    bias += (double)w[k] * (double)src.beta[m][k];
    w_out[fold_index(m, n, k)] = (half_t)(s * (double)w[k] * (double)src.gamma[m][k]);
  }
  b_out[(size_t)m * n_out + n] = (float)(s * bias);
}

template <typename CT>
__global__ void pad_matrix_kernel(const float* __restrict__ src, int rows, int cols, CT* __restrict__ dst,
                                  int prow, int pcol) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)prow * pcol) return;
  int r = (int)(i / pcol), c = (int)(i % pcol);
  dst[i] = (r < rows && c < cols) ? (CT)src[(int64_t)r * cols + c] : (CT)0.0f;
}

__global__ void pad_vector_kernel(const float* __restrict__ src, int n, float* __restrict__ dst, int pn) {
  int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < pn) dst[i] = i < n ? src[i] : 0.0f;
}

template <typename CT>
int pad_matrix(const float* src, int rows, int cols, void* dst, int prow, int pcol, hipStream_t s) {
  int64_t n = (int64_t)prow * pcol;
  return launch("tri_prepare", pad_matrix_kernel<CT>, dim3((unsigned)ceil_div(n, 256)), dim3(256), 0, s, src, rows,
                cols, (CT*)dst, prow, pcol);
}

int pad_vector(const float* src, int n, void* dst, int pn, hipStream_t s) {
  return launch("tri_prepare", pad_vector_kernel, dim3((unsigned)ceil_div(pn, 256)), dim3(256), 0, s, src, n,
                (float*)dst, pn);
}

int validate(const afhip_triangle_desc* d) {
  AFHIP_REQUIRE(d != nullptr, "descriptor is NULL");
  AFHIP_REQUIRE(d->length > 0 && d->c_z > 0 && d->c_hidden > 0,
                "length, cZ and cHidden must be positive (received %d, %d, %d)", d->length, d->c_z, d->c_hidden);
  AFHIP_REQUIRE((int64_t)d->length * d->length <= (int64_t)1 << 30, "length %d is too large", d->length);
  AFHIP_REQUIRE(d->c_z <= 128, "cZ %d exceeds the 128 channels the output kernel tiles", d->c_z);
  AFHIP_REQUIRE(d->c_hidden <= 256, "cHidden %d exceeds 256", d->c_hidden);
  AFHIP_REQUIRE(d->direction == AFHIP_TRIANGLE_OUTGOING || d->direction == AFHIP_TRIANGLE_INCOMING,
                "unknown direction %d", d->direction);
  AFHIP_REQUIRE(valid_precision(d->precision), "unknown precision %d", d->precision);
  AFHIP_REQUIRE(valid_float_dtype(d->pair_dtype) && valid_float_dtype(d->out_dtype), "pair and output dtypes must be f32 or f16");
  AFHIP_REQUIRE(d->block_rows >= 0, "blockRows must be non-negative");
  AFHIP_REQUIRE(d->epsilon > 0.0f && std::isfinite(d->epsilon), "epsilon must be finite and positive; received %g",
                (double)d->epsilon);
  return AFHIP_OK;
}

template <typename ZT, bool F16MATH>
int launch_project(const ProjectArgs& pa, size_t shared, hipStream_t s) {
  if (int st = allow_lds((const void*)tri_project_kernel<ZT, F16MATH>, shared)) return st;
  return launch("triangle.project", tri_project_kernel<ZT, F16MATH>, dim3((unsigned)ceil_div(pa.P, kRows)),
                dim3(256), shared, s, pa);
}

template <typename ZT, typename OT, bool F16MATH>
int launch_output(const OutputArgs& oa, size_t shared, hipStream_t s) {
  if (int st = allow_lds((const void*)tri_output_kernel<ZT, OT, F16MATH>, shared)) return st;
  return launch("triangle.output", tri_output_kernel<ZT, OT, F16MATH>, dim3((unsigned)ceil_div(oa.pairs, kRows)),
                dim3(256), shared, s, oa);
}

template <bool F16MATH>
int dispatch_project(int zd, const ProjectArgs& pa, size_t shared, hipStream_t s) {
  if (zd == AFHIP_F32) return launch_project<float, F16MATH>(pa, shared, s);
  return launch_project<half_t, F16MATH>(pa, shared, s);
}

template <bool F16MATH>
int dispatch_output(int zd, int od, const OutputArgs& oa, size_t shared, hipStream_t s) {
  if (zd == AFHIP_F32) {
    if (od == AFHIP_F32) return launch_output<float, float, F16MATH>(oa, shared, s);
    return launch_output<float, half_t, F16MATH>(oa, shared, s);
  }
  if (od == AFHIP_F32) return launch_output<half_t, float, F16MATH>(oa, shared, s);
  return launch_output<half_t, half_t, F16MATH>(oa, shared, s);
}

}  // namespace

}  // namespace afhip

using namespace afhip;

extern "C" {

int afhip_triangle_weights_size(const afhip_triangle_desc* desc, size_t* bytes) {
  if (int s = validate(desc)) return s;
  AFHIP_REQUIRE(bytes != nullptr, "output is NULL");
  *bytes = tri_layout(*desc).total;
  return AFHIP_OK;
}

int afhip_triangle_fast_path(const afhip_triangle_desc* desc, int32_t* fast) {
  if (int s = validate(desc)) return s;
  AFHIP_REQUIRE(fast != nullptr, "output is NULL");
  *fast = triangle_fast_eligible(*desc) ? 1 : 0;
  return AFHIP_OK;
}

int afhip_triangle_workspace_size(const afhip_triangle_desc* desc, size_t* bytes) {
  if (int s = validate(desc)) return s;
  AFHIP_REQUIRE(bytes != nullptr, "output is NULL");
  *bytes = tri_workspace(*desc).total;
  return AFHIP_OK;
}

int afhip_triangle_prepare_weights(const afhip_triangle_desc* desc, const float* packed, void* prepared, void* stream) {
  if (int s = require_open()) return s;
  if (int s = validate(desc)) return s;
  AFHIP_REQUIRE(packed && prepared, "NULL weights");
  const auto& d = *desc;
  const TriWeights w = tri_layout(d);
  hipStream_t st = (hipStream_t)stream;
  const int cz = d.c_z, ch = d.c_hidden;
  // Offsets of the sixteen tensors in ORDER (src/triangle/weights.ts:4-10).
  size_t o[17];
  size_t sizes[16] = {(size_t)cz, (size_t)cz, (size_t)ch * cz, (size_t)ch, (size_t)ch * cz, (size_t)ch,
                      (size_t)ch * cz, (size_t)ch, (size_t)ch * cz, (size_t)ch, (size_t)ch, (size_t)ch,
                      (size_t)cz * ch, (size_t)cz, (size_t)cz * cz, (size_t)cz};
  o[0] = 0;
  for (int i = 0; i < 16; i++) o[i + 1] = o[i] + sizes[i];
  char* base = (char*)prepared;
  const bool f16 = d.precision == AFHIP_PRECISION_F16;
  size_t es = f16 ? 2 : 4;
  auto mat = [&](int index, int rows, int cols, size_t dst, int prow, int pcol) {
    return f16 ? pad_matrix<half_t>(packed + o[index], rows, cols, base + dst, prow, pcol, st)
               : pad_matrix<float>(packed + o[index], rows, cols, base + dst, prow, pcol, st);
  };
  int s;
  if ((s = pad_vector(packed + o[0], cz, base + w.ln_in_w, cz, st))) return s;
  if ((s = pad_vector(packed + o[1], cz, base + w.ln_in_b, cz, st))) return s;
  for (int k = 0; k < 4; k++) {  // ap, ag, bp, bg at ORDER 2, 4, 6, 8
    if ((s = mat(2 + 2 * k, ch, cz, w.w_proj + es * (size_t)k * w.chp * w.czp, w.chp, w.czp))) return s;
    if ((s = pad_vector(packed + o[3 + 2 * k], ch, base + w.b_proj + 4 * (size_t)k * w.chp, w.chp, st))) return s;
  }
  if ((s = pad_vector(packed + o[10], ch, base + w.ln_out_w, ch, st))) return s;
  if ((s = pad_vector(packed + o[11], ch, base + w.ln_out_b, ch, st))) return s;
  if ((s = mat(12, cz, ch, w.w_z, w.czo, w.chp))) return s;
  if ((s = pad_vector(packed + o[13], cz, base + w.b_z, w.czo, st))) return s;
  if ((s = mat(14, cz, cz, w.w_g, w.czo, w.czp))) return s;
  if ((s = pad_vector(packed + o[15], cz, base + w.b_g, w.czo, st))) return s;
  if (triangle_fast_eligible(d)) {
    // ORDER indices: LN-in 0/1, AP 2/3, AG 4/5, BP 6/7, BG 8/9, LN-out 10/11, Z 12/13, G 14/15.
    const int wi[kFoldMatrices] = {2, 4, 6, 8, 12, 14};
    const int gi[kFoldMatrices] = {0, 0, 0, 0, 10, 0};
    const float kNegLog2e = -1.4426950408889634f;
    const float sc[kFoldMatrices] = {1.0f, kNegLog2e, 1.0f, kNegLog2e, 1.0f, kNegLog2e};
    FoldSources fs{};
    for (int m = 0; m < kFoldMatrices; m++) {
      fs.w[m] = packed + o[wi[m]];
      fs.b[m] = packed + o[wi[m] + 1];
      fs.gamma[m] = packed + o[gi[m]];
      fs.beta[m] = packed + o[gi[m] + 1];
      fs.scale[m] = sc[m];
    }
    if ((s = launch("tri_prepare", fold_weights_kernel, dim3((unsigned)ceil_div(kFoldMatrices * cz, 128)), dim3(128),
                    0, st, fs, cz, cz, (half_t*)(base + w.fold_w), (float*)(base + w.fold_b))))
      return s;
  }
  return AFHIP_OK;
}

int afhip_triangle_run(const afhip_triangle_desc* desc, const void* z, const float* mask, const void* prepared,
                       void* out, void* workspace, size_t workspace_bytes, void* stream) {
  if (int s = require_open()) return s;
  if (int s = validate(desc)) return s;
  AFHIP_REQUIRE(z && mask && prepared && out, "NULL tensor");
  const auto& d = *desc;
  const TriWeights w = tri_layout(d);
  const TriWorkspace ws = tri_workspace(d);
  AFHIP_REQUIRE(workspace != nullptr && workspace_bytes >= ws.total, "workspace of %zu bytes is smaller than %zu",
                workspace_bytes, ws.total);
  hipStream_t st = (hipStream_t)stream;
  const bool f16 = d.precision == AFHIP_PRECISION_F16;
  const char* wb = (const char*)prepared;
  char* wsb = (char*)workspace;
  const int L = d.length;
  const int P = L * L;

  ProjectArgs pa{};
  pa.z = z;
  pa.mask = mask;
  pa.ln_w = (const float*)(wb + w.ln_in_w);
  pa.ln_b = (const float*)(wb + w.ln_in_b);
  pa.w_proj = wb + w.w_proj;
  pa.b_proj = (const float*)(wb + w.b_proj);
  pa.out_a = wsb + ws.op_a;
  pa.out_b = wsb + ws.op_b;
  pa.cstride = ws.cstride;
  pa.L = L;
  pa.P = P;
  pa.cz = d.c_z;
  pa.ch = d.c_hidden;
  pa.czp = w.czp;
  pa.chp = w.chp;
  pa.incoming = d.direction == AFHIP_TRIANGLE_INCOMING;
  pa.eps = d.epsilon;
  // AlphaFold's widths in f16 take the persistent kernels of
  // triangle_fast.hip; every other shape and the f32 path take the tiles below.
  const bool fast = triangle_fast_eligible(d) && (reinterpret_cast<uintptr_t>(z) & 15) == 0;
  int s;
  if (fast) {
    FastProjectArgs fa{};
    fa.z = z;
    fa.mask = mask;
    fa.w_proj = (const half_t*)(wb + w.fold_w);
    fa.b_proj = (const float*)(wb + w.fold_b);
    fa.out_a = (half_t*)pa.out_a;
    fa.out_b = (half_t*)pa.out_b;
    fa.cstride = ws.cstride;
    fa.L = L;
    fa.P = P;
    fa.incoming = pa.incoming;
    fa.eps = d.epsilon;
    s = launch_triangle_project_f16(fa, d.pair_dtype, st);
  } else {
    size_t psh = round_up((int64_t)w.czp * (kRows + 1) * 4, 16) +
                 (f16 ? round_up((int64_t)kRows * (w.czp + 8) * 2, 16) : 0) + (size_t)64 * (kRows + 8) * (f16 ? 2 : 4);
    s = f16 ? dispatch_project<true>(d.pair_dtype, pa, psh, st) : dispatch_project<false>(d.pair_dtype, pa, psh, st);
  }
  if (s) return s;

  // Row operand and column operand of the contraction (see the file comment).
  const void* row_op = pa.incoming ? pa.out_b : pa.out_a;
  const void* col_op = pa.incoming ? pa.out_a : pa.out_b;
  const size_t es = f16 ? 2 : 4;
  GemmTypes types{d.precision, f16 ? AFHIP_F16 : AFHIP_F32, f16 ? AFHIP_F16 : AFHIP_F32, f16 ? AFHIP_F16 : AFHIP_F32};
  const int kmax = std::max(w.chp, w.czp);
  size_t osh = round_up((int64_t)kmax * (kRows + 1) * 4, 16) + (f16 ? (size_t)kRows * (kmax + 8) * 2 : 0);
  for (int i0 = 0; i0 < L; i0 += ws.block_rows) {
    const int count = std::min(ws.block_rows, L - i0);
    GemmArgs g;
    g.a = (const char*)row_op + es * (size_t)i0 * L;
    g.b = col_op;
    g.c = wsb + ws.contracted;
    g.M = count;
    g.N = L;
    g.K = L;
    g.lda = L;
    g.ldb = L;
    g.ldc = L;
    g.sa = ws.cstride;
    g.sb = ws.cstride;
    g.sc = ws.bstride;
    g.batch = d.c_hidden;
    afhip_variant v = select_variant(types, count, L, L, d.c_hidden);
    if ((s = run_gemm(g, types, v, "triangle.contract", st))) return s;

    OutputArgs oa{};
    oa.contracted = wsb + ws.contracted;
    oa.bstride = ws.bstride;
    oa.z = z;
    oa.ln_in_w = pa.ln_w;
    oa.ln_in_b = pa.ln_b;
    oa.ln_out_w = (const float*)(wb + w.ln_out_w);
    oa.ln_out_b = (const float*)(wb + w.ln_out_b);
    oa.w_z = wb + w.w_z;
    oa.b_z = (const float*)(wb + w.b_z);
    oa.w_g = wb + w.w_g;
    oa.b_g = (const float*)(wb + w.b_g);
    oa.out = out;
    oa.pair0 = i0 * L;
    oa.pairs = count * L;
    oa.cz = d.c_z;
    oa.ch = d.c_hidden;
    oa.czp = w.czp;
    oa.chp = w.chp;
    oa.residual = d.residual;
    oa.eps = d.epsilon;
    if (fast) {
      FastOutputArgs fo{};
      fo.contracted = (const half_t*)oa.contracted;
      fo.bstride = oa.bstride;
      fo.z = z;
      fo.w_z = (const half_t*)(wb + w.fold_w) + (size_t)4 * kC * kC;
      fo.b_z = (const float*)(wb + w.fold_b) + 4 * kC;
      fo.w_g = (const half_t*)(wb + w.fold_w) + (size_t)5 * kC * kC;
      fo.b_g = (const float*)(wb + w.fold_b) + 5 * kC;
      fo.out = out;
      fo.pair0 = oa.pair0;
      fo.pairs = oa.pairs;
      fo.residual = oa.residual;
      fo.eps = d.epsilon;
      s = launch_triangle_output_f16(fo, d.pair_dtype, d.out_dtype, st);
    } else {
      s = f16 ? dispatch_output<true>(d.pair_dtype, d.out_dtype, oa, osh, st)
              : dispatch_output<false>(d.pair_dtype, d.out_dtype, oa, osh, st);
    }
    if (s) return s;
  }
  return AFHIP_OK;
}

}  // extern "C"
