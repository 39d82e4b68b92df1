// Outer-product mean for gfx950.
//
// The reference (src/evoformer/outer-product-mean.ts:549-646) runs normalize,
// project, pair-count, then per residue block a contraction and an output
// projection. Here:
//
//  1. opm_project: LayerNorm of 64 MSA rows in LDS and both projections on
//     MFMA, mask*(x + b). Rows are visited residue-major (row r = i*S + s
//     reads MSA row (s, i)), so each output channel (i, a) receives a run of
//     consecutive sequences: left and right are stored [L*c_o][S], the
//     contraction axis contiguous, which is the k-contiguous operand layout
//     the shared GEMM stages with 16-byte loads.
//     Under f16 arithmetic with c_outer = 32 and c_m of 64, 128 or 256 (the
//     MSA and extra-MSA stacks) a persistent kernel does the same per tile
//     of 64 sequences of one residue: 16-byte row loads one tile ahead,
//     LayerNorm statistics across the lanes holding a row, the projection
//     weights resident in VGPRs, and 128-byte channel-major stores.
//  2. pair count: count[i][j] = sum_s mask[s][i] mask[s][j] (:317-332), as an
//     f32 GEMM of the transposed mask with itself (exact for 0/1 masks, whose
//     partial sums are small integers). With the fast projection its tiles
//     are extra workgroups of the projection's launch.
//  3. per residue block, the contraction through the shared GEMM,
//     outer[i][j][a][b] = sum_s left[s][i][a] right[s][j][b] / (eps + count),
//     divided in its epilogue as the reference's contraction does
//     (:350-417), then the output projection through the shared GEMM with
//     the bias scaled by the same 1/(eps + count) (:433-481).
//     Under f16 arithmetic with c_outer = 32 and c_z in (96, 128] (the
//     model's shapes) both run in one launch instead (run_opm_fused): each
//     256 x 256 contraction tile is an 8 x 8 block of pairs whose outer
//     blocks go through LDS straight into the output projection, so outer
//     never reaches memory and the residue blocking has nothing left to
//     bound (the same arithmetic, the same f16 rounding of outer).
#include <algorithm>
#include <cmath>

#include "gemm.h"

namespace afhip {

namespace {

constexpr int kRows = 64;

// The single-launch contraction + output projection applies.
bool fused_ok(const afhip_opm_desc& d) {
  return d.precision == AFHIP_PRECISION_F16 && d.c_outer == 32 && d.c_z > 96 && d.c_z <= 128;
}

struct OpmWeights {
  size_t ln_scale, ln_offset, w_lr, b_lr, w_out, b_out, total;
  int cmp;  // c_m padded to 32
  int cop;  // 2 * c_outer padded to 64 (projection columns)
  int czp;  // c_z padded to 32 (output rows of W_out^T)
};

OpmWeights opm_layout(const afhip_opm_desc& d) {
  OpmWeights w{};
  size_t es = d.precision == AFHIP_PRECISION_F16 ? 2 : 4;
  w.cmp = (int)round_up(d.c_m, 32);
  w.cop = (int)round_up(2 * d.c_outer, 64);
  w.czp = (int)round_up(d.c_z, 32);
  size_t at = 0;
  auto take = [&](size_t bytes) {
    size_t here = at;
    at = round_up((int64_t)(at + bytes), 256);
    return here;
  };
  w.ln_scale = take(4 * (size_t)d.c_m);
  w.ln_offset = take(4 * (size_t)d.c_m);
  w.w_lr = take(es * (size_t)w.cop * w.cmp);
  w.b_lr = take(4 * (size_t)w.cop);
  w.w_out = take(es * (size_t)w.czp * d.c_outer * d.c_outer);
  w.b_out = take(4 * (size_t)w.czp);
  w.total = at;
  return w;
}

struct OpmWorkspace {
  size_t left, right, outer, count, total;
  int64_t sp;  // sequence stride of left/right rows
  int row_block;
};

OpmWorkspace opm_workspace(const afhip_opm_desc& d) {
  OpmWorkspace w{};
  size_t es = d.precision == AFHIP_PRECISION_F16 ? 2 : 4;
  w.sp = round_up(d.sequences, 8);
  w.row_block = d.row_block > 0 ? std::min(d.row_block, d.length) : d.length;
  size_t at = 0;
  auto take = [&](size_t bytes) {
    size_t here = at;
    at = round_up((int64_t)(at + bytes), 256);
    return here;
  };
  const size_t rows = (size_t)d.length * d.c_outer;
  w.left = take(es * rows * w.sp);
  w.right = take(es * rows * w.sp);
  w.outer = take(fused_ok(d) ? 0 : es * (size_t)w.row_block * d.length * d.c_outer * d.c_outer);
  w.count = take(4 * (size_t)d.length * d.length);
  w.total = at;
  return w;
}

struct ProjectArgs {
  const void* msa;
  const float* mask;
  const float* ln_scale;
  const float* ln_offset;
  const void* w_lr;  // [cop][cmp]: rows [0, co) left, [co, 2co) right
  const float* b_lr;
  void* left;
  void* right;
  int64_t sp;
  int S, L, cm, co, cmp, cop;
  float eps;
};

template <typename MT, bool F16MATH>
__global__ __launch_bounds__(256) void opm_project_kernel(ProjectArgs a) {
  using CT = typename std::conditional<F16MATH, half_t, float>::type;
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int xpitch = kRows + 1;
  float* xs = reinterpret_cast<float*>(smem);
  size_t off = round_up((int64_t)a.cmp * xpitch * 4, 16);
  CT* an = reinterpret_cast<CT*>(smem + off);
  const int apitch = a.cmp + 8;
  if (F16MATH) off += round_up((int64_t)kRows * apitch * 2, 16);
  CT* stage = reinterpret_cast<CT*>(smem + off);
  constexpr int spitch = kRows + 8;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int rows = a.S * a.L;
  const int r0 = blockIdx.x * kRows;
  const MT* msa = reinterpret_cast<const MT*>(a.msa);

  for (int idx = tid; idx < kRows * a.cmp; idx += 256) {
    const int i = idx / a.cmp, c = idx - i * a.cmp;
    const int r = r0 + i;
    float v = 0.0f;
    if (r < rows && c < a.cm) {
      const int res = r / a.S, s = r - res * a.S;
      v = (float)msa[((int64_t)s * a.L + res) * a.cm + c];
    }
    xs[c * xpitch + i] = v;
  }
  __syncthreads();
  {
    const int q = tid >> 2, part = tid & 3;
    float sum = 0.0f;
    for (int c = part; c < a.cm; c += 4) sum += xs[c * xpitch + q];
    sum += __shfl_xor(sum, 1);
    sum += __shfl_xor(sum, 2);
    const float mean = sum / (float)a.cm;
    float var = 0.0f;
    for (int c = part; c < a.cm; c += 4) {
      float d = xs[c * xpitch + q] - mean;
      var += d * d;
    }
    var += __shfl_xor(var, 1);
    var += __shfl_xor(var, 2);
    const float rstd = fast_rsqrt(var / (float)a.cm + a.eps);
    for (int c = part; c < a.cmp; c += 4) {
      float v = c < a.cm ? (xs[c * xpitch + q] - mean) * rstd * a.ln_scale[c] + a.ln_offset[c] : 0.0f;
      if (F16MATH) an[q * apitch + c] = (CT)v;
      else xs[c * xpitch + q] = v;
    }
  }
  __syncthreads();

  const CT* W = reinterpret_cast<const CT*>(a.w_lr);
  const int rw = 32 * (wave & 1);
  for (int n0 = 0; n0 < a.cop; n0 += 64) {
    const int nc = n0 + 32 * (wave >> 1);
    floatx16 acc;
#pragma unroll
    for (int v = 0; v < 16; v++) acc[v] = 0.0f;
    const int n = nc + (lane & 31);
    if constexpr (F16MATH) {
      for (int k = 0; k < a.cmp; k += 16) {
        const int kk = k + 8 * (lane >> 5);
        half8 af = *reinterpret_cast<const half8*>(an + (rw + (lane & 31)) * apitch + kk);
        half8 bf = *reinterpret_cast<const half8*>(W + (size_t)n * a.cmp + kk);
        acc = mfma_f16(af, bf, acc);
      }
    } else {
      for (int k = 0; k < a.cmp; k += 2) {
        const int kk = k + (lane >> 5);
        acc = mfma_f32(xs[kk * xpitch + rw + (lane & 31)], W[(size_t)n * a.cmp + kk], acc);
      }
    }
    const float bias = a.b_lr[n];
#pragma unroll
    for (int v = 0; v < 16; v++) {
      const int i = rw + mfma_row(v, lane);
      const int r = r0 + i;
      float val = 0.0f;
      if (r < rows) {
        const int res = r / a.S, s = r - res * a.S;
        val = a.mask[(int64_t)s * a.L + res] * (acc[v] + bias);
      }
      stage[(n - n0) * spitch + i] = (CT)val;
    }
    __syncthreads();
    // Channel (res, o) of left or right receives this tile's run of sequences.
    for (int idx = tid; idx < 64 * kRows; idx += 256) {
      const int nl = idx / kRows, i = idx - nl * kRows;
      const int col = n0 + nl, r = r0 + i;
      if (col >= 2 * a.co || r >= rows) continue;
      const int res = r / a.S, s = r - res * a.S;
      const bool is_left = col < a.co;
      const int o = is_left ? col : col - a.co;
      CT* dst = reinterpret_cast<CT*>(is_left ? a.left : a.right);
      dst[((int64_t)res * a.co + o) * a.sp + s] = stage[nl * spitch + i];
    }
    __syncthreads();
  }
}

// Pair counts count[i][j] = sum_s mask[s][i] mask[s][j] (the masked
// sequence count per pair, outer-product-mean.ts:317-332) of one 32 x 32
// tile, by the WAVES waves of the calling workgroup: they take interleaved
// two-sequence steps of the f32 MFMA, both operands read straight from the
// [S][L] mask (A = mask[s][i0 + m], B = mask[s][j0 + n]), then sum their
// partial tiles in LDS (`part`, WAVES x 4 KiB) in wave order, so the result
// does not depend on timing.
template <int WAVES>
__device__ __forceinline__ void pair_count_tile(const float* __restrict__ mask, int S, int L, float* __restrict__ count,
                                                int tile, float* part) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int tiles = (L + 31) / 32;
  const int i0 = (tile / tiles) * 32, j0 = (tile % tiles) * 32;
  const int col = lane & 31, hi = lane >> 5;
  const bool in_i = i0 + col < L, in_j = j0 + col < L;
  floatx16 acc = {};
  // Four steps' loads go out together before their MFMAs.
  for (int s0 = 2 * wave; s0 < S; s0 += 8 * WAVES) {
    float a[4], b[4];
#pragma unroll
    for (int u = 0; u < 4; u++) {
      const int s = s0 + 2 * WAVES * u + hi;
      a[u] = s < S && in_i ? mask[(int64_t)s * L + i0 + col] : 0.0f;
      b[u] = s < S && in_j ? mask[(int64_t)s * L + j0 + col] : 0.0f;
    }
#pragma unroll
    for (int u = 0; u < 4; u++) acc = mfma_f32(a[u], b[u], acc);
  }
#pragma unroll
  for (int v = 0; v < 16; v++) part[(wave * 16 + v) * 64 + lane] = acc[v];
  __syncthreads();
  // Element (m, n) of the tile sits at row v = 4 (m / 8) + m % 4 of lane
  // n + 32 ((m / 4) % 2).
  for (int e = threadIdx.x; e < 1024; e += 64 * WAVES) {
    const int m = e >> 5, n = e & 31;
    const int v = 4 * (m >> 3) + (m & 3), l = n + 32 * ((m >> 2) & 1);
    float sum = 0.0f;
#pragma unroll
    for (int w = 0; w < WAVES; w++) sum += part[(w * 16 + v) * 64 + l];
    if (i0 + m < L && j0 + n < L) count[(int64_t)(i0 + m) * L + j0 + n] = sum;
  }
}

// The pair counts on their own: one 32 x 32 tile per sixteen-wave workgroup.
constexpr int kCountWaves = 16;
__global__ __launch_bounds__(64 * kCountWaves) void opm_pair_count_kernel(const float* __restrict__ mask, int S, int L,
                                                                          float* __restrict__ count) {
  __shared__ float part[kCountWaves * 16 * 64];
  pair_count_tile<kCountWaves>(mask, S, L, count, blockIdx.x, part);
}

// ---------------------------------------------------------------------------
// Fast projection: f16 arithmetic, c_outer = 32, c_m = CM in {64, 128, 256}.
// ---------------------------------------------------------------------------
constexpr int kFastRows = 64;  // sequences per tile, all of one residue
constexpr int kFastThreads = 256;

template <int CM> struct FastLayout {
  static constexpr int APITCH = CM + 8;                 // x_hat row, halves (16-byte shifted rows)
  static constexpr int SPITCH = kFastRows + 8;          // staging row (one channel), halves
  static constexpr int XHAT = 0;
  static constexpr int STG = XHAT + kFastRows * APITCH * 2;
  static constexpr int MASK = STG + 64 * SPITCH * 2;
  static constexpr int BYTES = MASK + kFastRows * 4;
};

template <typename MT> struct RowChunk;  // 8 consecutive channels of one row
template <> struct RowChunk<half_t> {
  uint4 v;
  __device__ void load(const half_t* p) { v = *reinterpret_cast<const uint4*>(p); }
  __device__ void zero() { v = make_uint4(0, 0, 0, 0); }
  __device__ void get(float* x) const {
    const half8 h = __builtin_bit_cast(half8, v);
#pragma unroll
    for (int e = 0; e < 8; e++) x[e] = (float)h[e];
  }
};
template <> struct RowChunk<float> {
  float4 a, b;
  __device__ void load(const float* p) {
    a = *reinterpret_cast<const float4*>(p);
    b = *reinterpret_cast<const float4*>(p + 4);
  }
  __device__ void zero() { a = b = make_float4(0.f, 0.f, 0.f, 0.f); }
  __device__ void get(float* x) const {
    x[0] = a.x, x[1] = a.y, x[2] = a.z, x[3] = a.w, x[4] = b.x, x[5] = b.y, x[6] = b.z, x[7] = b.w;
  }
};

// Persistent: workgroup g walks tiles g, g + grid, ... (tile t = residue
// t / tiles_per_res, sequences [64 (t % tiles_per_res), +64)). Each wave
// holds 16 rows of the next tile in VGPRs while the current one computes:
// LPR = CM / 8 lanes per row, 8 channels per lane. The projection is
// x_hat [64 x CM] (A operand, from LDS) times W^T (B operand, VGPRs): wave w
// computes rows 32 (w & 1) and output columns 32 (w >> 1) (left, then right).
// The first count_blocks workgroups of the launch compute the pair counts
// instead (one 32 x 32 tile each, pair_count_tile), so they need no launch
// of their own; they come first so they are dispatched first.
template <int CM, typename MT>
__global__ __launch_bounds__(kFastThreads, 2) void opm_project_fast_kernel(ProjectArgs a, int ntiles,
                                                                          int tiles_per_res, int count_blocks,
                                                                          float* __restrict__ count) {
  using Lay = FastLayout<CM>;
  constexpr int LPR = CM / 8;             // lanes per row
  constexpr int RPL = 64 / LPR;           // rows per wave-level load
  constexpr int LOADS = 16 / RPL;         // loads per wave per tile
  constexpr int KS = CM / 16;             // MFMA k-steps
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  half_t* const xhat = reinterpret_cast<half_t*>(smem + Lay::XHAT);
  half_t* const stg = reinterpret_cast<half_t*>(smem + Lay::STG);
  float* const mbuf = reinterpret_cast<float*>(smem + Lay::MASK);

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c0 = 8 * (lane % LPR);  // this lane's channels in a row
  const MT* msa = reinterpret_cast<const MT*>(a.msa);

  float gam[8], bet[8];
#pragma unroll
  for (int e = 0; e < 8; e++) {
    gam[e] = a.ln_scale[c0 + e];
    bet[e] = a.ln_offset[c0 + e];
  }
  // W [cop][cmp] rows n = 32 (wave >> 1) + lane % 32: the B fragment of k-step kk.
  const int n = 32 * (wave >> 1) + (lane & 31);
  const half_t* W = reinterpret_cast<const half_t*>(a.w_lr) + (size_t)n * a.cmp + 8 * (lane >> 5);
  half8 wf[KS];
#pragma unroll
  for (int kk = 0; kk < KS; kk++) wf[kk] = *reinterpret_cast<const half8*>(W + 16 * kk);
  const float bias = a.b_lr[n];

  RowChunk<MT> raw[LOADS];
  float mval = 0.0f;
  auto fetch = [&](int t) {
    const int res = t / tiles_per_res, s0 = (t - res * tiles_per_res) * kFastRows;
#pragma unroll
    for (int j = 0; j < LOADS; j++) {
      const int s = s0 + 16 * wave + RPL * j + lane / LPR;
      if (s < a.S) raw[j].load(msa + ((int64_t)s * a.L + res) * CM + c0);
      else raw[j].zero();
    }
    if (tid < kFastRows) mval = s0 + tid < a.S ? a.mask[(int64_t)(s0 + tid) * a.L + res] : 0.0f;
  };

  if ((int)blockIdx.x < count_blocks) {
    pair_count_tile<kFastThreads / 64>(a.mask, a.S, a.L, count, blockIdx.x, reinterpret_cast<float*>(smem));
    return;
  }
  const int G = (int)gridDim.x - count_blocks;
  int t = (int)blockIdx.x - count_blocks;
  if (t >= ntiles) return;
  fetch(t);
  for (; t < ntiles; t += G) {
    const int res = t / tiles_per_res, s0 = (t - res * tiles_per_res) * kFastRows;
    // LayerNorm: two-pass mean and biased variance in f32, eps inside the
    // root (outer-product-mean.ts:221-261), the affine applied per channel.
#pragma unroll
    for (int j = 0; j < LOADS; j++) {
      float x[8];
      raw[j].get(x);
      float sum = 0.0f;
#pragma unroll
      for (int e = 0; e < 8; e++) sum += x[e];
      const float mean = lane_sum<LPR>(sum) / (float)CM;
      float var = 0.0f;
#pragma unroll
      for (int e = 0; e < 8; e++) {
        const float d = x[e] - mean;
        var += d * d;
      }
      const float rstd = fast_rsqrt(lane_sum<LPR>(var) / (float)CM + a.eps);
      half8 h;
#pragma unroll
      for (int e = 0; e < 8; e++) h[e] = (half_t)((x[e] - mean) * rstd * gam[e] + bet[e]);
      const int row = 16 * wave + RPL * j + lane / LPR;
      *reinterpret_cast<half8*>(xhat + row * Lay::APITCH + c0) = h;
    }
    if (tid < kFastRows) mbuf[tid] = mval;
    if (t + G < ntiles) fetch(t + G);  // lands while this tile computes
    __syncthreads();

    floatx16 acc;
#pragma unroll
    for (int v = 0; v < 16; v++) acc[v] = 0.0f;
    const half_t* arow = xhat + (32 * (wave & 1) + (lane & 31)) * Lay::APITCH + 8 * (lane >> 5);
#pragma unroll
    for (int kk = 0; kk < KS; kk++) acc = mfma_f16(*reinterpret_cast<const half8*>(arow + 16 * kk), wf[kk], acc);
    // Lane holds column n and rows 32 (w & 1) + 8 g4 + 4 (lane / 32) + e:
    // mask * (x W + b), four consecutive sequences per 8-byte staging write.
#pragma unroll
    for (int g4 = 0; g4 < 4; g4++) {
      const int r = 32 * (wave & 1) + 8 * g4 + 4 * (lane >> 5);
      const floatx4 m4 = *reinterpret_cast<const floatx4*>(mbuf + r);
      half4 h;
#pragma unroll
      for (int e = 0; e < 4; e++) h[e] = (half_t)(m4[e] * (acc[4 * g4 + e] + bias));
      *reinterpret_cast<half4*>(stg + n * Lay::SPITCH + r) = h;
    }
    __syncthreads();
    // 64 channel rows of 128 bytes: wave w writes rows 16 w .. 16 w + 15,
    // eight lanes per row; sequences past sp (the padded row length) are
    // skipped, those in [S, sp) are zeros.
    u32x4 v[2];
#pragma unroll
    for (int j = 0; j < 2; j++) {
      const int ch = 16 * wave + 8 * j + (lane >> 3), chunk = lane & 7;
      const int sq = s0 + 8 * chunk;
      v[j] = *reinterpret_cast<const u32x4*>(stg + ch * Lay::SPITCH + 8 * chunk);
      if (sq < a.sp) {
        half_t* dst = reinterpret_cast<half_t*>(ch < 32 ? a.left : a.right);
        *reinterpret_cast<u32x4*>(dst + ((int64_t)res * 32 + (ch & 31)) * a.sp + sq) = v[j];
      }
    }
    stores_read(v[0], v[1]);
  }
}

// Zeros sequences [S, sp) of every left and right row (the fast projection
// writes them itself): the fused contraction reads whole 8-sequence chunks.
__global__ void opm_zero_tail_kernel(half_t* __restrict__ left, half_t* __restrict__ right, int64_t rows, int64_t sp,
                                     int S) {
  const int pad = (int)(sp - S);
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < 2 * rows * pad;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / pad;
    half_t* dst = r < rows ? left : right;
    dst[(r < rows ? r : r - rows) * sp + S + (int)(i - r * pad)] = (half_t)0.0f;
  }
}

bool project_fast_ok(const afhip_opm_desc& d) {
  return d.precision == AFHIP_PRECISION_F16 && d.c_outer == 32 && (d.c_m == 64 || d.c_m == 128 || d.c_m == 256);
}

// Three workgroups a CU (their VGPRs allow it at every c_m): 21.6 us
// against 23.5 us for two at N_seq = 512, N_res = 256, c_m = 256.
template <int CM, typename MT> int launch_fast(const ProjectArgs& pa, float* count, hipStream_t s) {
  auto k = opm_project_fast_kernel<CM, MT>;
  constexpr size_t bytes = FastLayout<CM>::BYTES;
  static_assert(bytes >= (size_t)(kFastThreads / 64) * 16 * 64 * 4, "the pair-count partials fit");
  if (int st = allow_lds((const void*)k, bytes)) return st;
  const int tiles_per_res = (int)ceil_div(pa.S, kFastRows);
  const int ntiles = tiles_per_res * pa.L;
  const int cus = device_cu_count() > 0 ? device_cu_count() : 256;
  const int grid = std::min(ntiles, 3 * cus);
  const int64_t count_tiles = ceil_div(pa.L, 32) * ceil_div(pa.L, 32);
  AFHIP_REQUIRE(grid + count_tiles < ((int64_t)1 << 31), "too many residues");
  return launch("opm.project", k, dim3((unsigned)(grid + count_tiles)), dim3(kFastThreads), bytes, s, pa, ntiles,
                tiles_per_res, (int)count_tiles, count);
}

template <typename MT> int launch_fast_cm(const ProjectArgs& pa, float* count, hipStream_t s) {
  if (pa.cm == 64) return launch_fast<64, MT>(pa, count, s);
  if (pa.cm == 128) return launch_fast<128, MT>(pa, count, s);
  return launch_fast<256, MT>(pa, count, s);
}

template <typename CT>
__global__ void opm_prepare_kernel(const float* __restrict__ packed, int cm, int co, int cz, int cmp, int cop, int czp,
                                   CT* __restrict__ w_lr, float* __restrict__ b_lr, CT* __restrict__ w_out,
                                   float* __restrict__ b_out, float* __restrict__ ln_s, float* __restrict__ ln_o,
                                   bool fused) {
  const float* ln_scale = packed;
  const float* ln_offset = ln_scale + cm;
  const float* left_w = ln_offset + cm;
  const float* left_b = left_w + (size_t)cm * co;
  const float* right_w = left_b + co;
  const float* right_b = right_w + (size_t)cm * co;
  const float* out_w = right_b + co;
  const float* out_b = out_w + (size_t)co * co * cz;
  const int64_t n_lr = (int64_t)cop * cmp, n_out = (int64_t)czp * co * co;
  const int64_t total = n_lr + n_out + cop + czp + 2 * cm;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    if (i < n_lr) {  // [cop][cmp] <- left/right [cm][co] transposed
      const int n = (int)(i / cmp), k = (int)(i % cmp);
      float v = 0.0f;
      if (k < cm && n < co) v = left_w[(size_t)k * co + n];
      else if (k < cm && n < 2 * co) v = right_w[(size_t)k * co + (n - co)];
      w_lr[i] = (CT)v;
    } else if (i < n_lr + n_out) {  // [czp][co*co] <- out [co*co][cz] transposed
      const int64_t j = i - n_lr;
      const int n = (int)(j / (co * co)), k = (int)(j % (co * co));
      // The fused kernel reads them in its fragment order.
      const int64_t at = fused ? opm_fused_weight_index(k, n) : j;
      w_out[at] = (CT)(n < cz ? out_w[(size_t)k * cz + n] : 0.0f);
    } else if (i < n_lr + n_out + cop) {
      const int n = (int)(i - n_lr - n_out);
      b_lr[n] = n < co ? left_b[n] : (n < 2 * co ? right_b[n - co] : 0.0f);
    } else if (i < n_lr + n_out + cop + czp) {
      const int n = (int)(i - n_lr - n_out - cop);
      b_out[n] = n < cz ? out_b[n] : 0.0f;
    } else {
      const int c = (int)(i - n_lr - n_out - cop - czp);
      if (c < cm) ln_s[c] = ln_scale[c];
      else ln_o[c - cm] = ln_offset[c - cm];
    }
  }
}

int validate(const afhip_opm_desc* d) {
  AFHIP_REQUIRE(d != nullptr, "descriptor is NULL");
  AFHIP_REQUIRE(d->sequences > 0 && d->length > 0 && d->c_m > 0 && d->c_outer > 0 && d->c_z > 0,
                "outer product mean dimensions must be positive safe integers");
  AFHIP_REQUIRE((int64_t)d->sequences * d->length <= (int64_t)1 << 30, "alignment too large");
  AFHIP_REQUIRE(d->c_m <= 512, "c_m %d exceeds 512", d->c_m);
  AFHIP_REQUIRE(valid_precision(d->precision), "unknown precision %d", d->precision);
  AFHIP_REQUIRE(valid_float_dtype(d->msa_dtype) && valid_float_dtype(d->out_dtype), "dtypes must be f32 or f16");
  AFHIP_REQUIRE(d->row_block >= 0, "rowBlockResidues must be non-negative");
  AFHIP_REQUIRE(d->layer_norm_epsilon > 0 && d->normalization_epsilon >= 0, "epsilons must be positive");
  return AFHIP_OK;
}

template <typename MT, bool F16MATH>
int launch_project(const ProjectArgs& pa, size_t shared, hipStream_t s) {
  if (int st = allow_lds((const void*)opm_project_kernel<MT, F16MATH>, shared)) return st;
  return launch("opm.project", opm_project_kernel<MT, F16MATH>, dim3((unsigned)ceil_div((int64_t)pa.S * pa.L, kRows)),
                dim3(256), shared, s, pa);
}

}  // namespace

}  // namespace afhip

using namespace afhip;

extern "C" {

int afhip_opm_weights_size(const afhip_opm_desc* desc, size_t* bytes) {
  if (int s = validate(desc)) return s;
  AFHIP_REQUIRE(bytes != nullptr, "output is NULL");
  *bytes = opm_layout(*desc).total;
  return AFHIP_OK;
}

int afhip_opm_workspace_size(const afhip_opm_desc* desc, size_t* bytes) {
  if (int s = validate(desc)) return s;
  AFHIP_REQUIRE(bytes != nullptr, "output is NULL");
  *bytes = opm_workspace(*desc).total;
  return AFHIP_OK;
}

int afhip_opm_prepare_weights(const afhip_opm_desc* desc, const float* packed, void* prepared, void* stream) {
  if (int s = require_open()) return s;
  if (int s = validate(desc)) return s;
  AFHIP_REQUIRE(packed && prepared, "NULL weights");
  const auto& d = *desc;
  const OpmWeights w = opm_layout(d);
  char* base = (char*)prepared;
  hipStream_t st = (hipStream_t)stream;
  dim3 grid(1024), block(256);
  float* ln_s = (float*)(base + w.ln_scale);
  float* ln_o = (float*)(base + w.ln_offset);
  if (d.precision == AFHIP_PRECISION_F16) {
    if (int s = launch("opm.prepare", opm_prepare_kernel<half_t>, grid, block, 0, st, packed, d.c_m, d.c_outer, d.c_z,
                       w.cmp, w.cop, w.czp, (half_t*)(base + w.w_lr), (float*)(base + w.b_lr),
                       (half_t*)(base + w.w_out), (float*)(base + w.b_out), ln_s, ln_o, fused_ok(d)))
      return s;
  } else {
    if (int s = launch("opm.prepare", opm_prepare_kernel<float>, grid, block, 0, st, packed, d.c_m, d.c_outer, d.c_z,
                       w.cmp, w.cop, w.czp, (float*)(base + w.w_lr), (float*)(base + w.b_lr),
                       (float*)(base + w.w_out), (float*)(base + w.b_out), ln_s, ln_o, false))
      return s;
  }
  return AFHIP_OK;
}

int afhip_opm_run(const afhip_opm_desc* desc, const void* activations, const float* mask, const void* prepared,
                  void* out, void* workspace, size_t workspace_bytes, void* stream) {
  if (int s = require_open()) return s;
  if (int s = validate(desc)) return s;
  AFHIP_REQUIRE(activations && mask && prepared && out, "NULL tensor");
  const auto& d = *desc;
  const OpmWeights w = opm_layout(d);
  const OpmWorkspace ws = opm_workspace(d);
  AFHIP_REQUIRE(workspace != nullptr && workspace_bytes >= ws.total, "workspace of %zu bytes is smaller than %zu",
                workspace_bytes, ws.total);
  hipStream_t st = (hipStream_t)stream;
  const bool f16 = d.precision == AFHIP_PRECISION_F16;
  const char* wb = (const char*)prepared;
  char* wsb = (char*)workspace;
  const int S = d.sequences, L = d.length, co = d.c_outer;

  ProjectArgs pa{};
  pa.msa = activations;
  pa.mask = mask;
  pa.ln_scale = (const float*)(wb + w.ln_scale);
  pa.ln_offset = (const float*)(wb + w.ln_offset);
  pa.w_lr = wb + w.w_lr;
  pa.b_lr = (const float*)(wb + w.b_lr);
  pa.left = wsb + ws.left;
  pa.right = wsb + ws.right;
  pa.sp = ws.sp;
  pa.S = S;
  pa.L = L;
  pa.cm = d.c_m;
  pa.co = co;
  pa.cmp = w.cmp;
  pa.cop = w.cop;
  pa.eps = d.layer_norm_epsilon;
  size_t psh = round_up((int64_t)w.cmp * (kRows + 1) * 4, 16) +
               (f16 ? round_up((int64_t)kRows * (w.cmp + 8) * 2, 16) : 0) + (size_t)64 * (kRows + 8) * (f16 ? 2 : 4);
  int s;
  float* count = (float*)(wsb + ws.count);
  // The fast projection computes the pair counts in the same launch.
  const bool fast = project_fast_ok(d) && (reinterpret_cast<uintptr_t>(activations) & 15) == 0;
  if (fast)
    s = d.msa_dtype == AFHIP_F32 ? launch_fast_cm<float>(pa, count, st) : launch_fast_cm<half_t>(pa, count, st);
  else if (f16)
    s = d.msa_dtype == AFHIP_F32 ? launch_project<float, true>(pa, psh, st) : launch_project<half_t, true>(pa, psh, st);
  else
    s = d.msa_dtype == AFHIP_F32 ? launch_project<float, false>(pa, psh, st) : launch_project<half_t, false>(pa, psh, st);
  if (s) return s;

  if (!fast) {
    const int64_t tiles = ceil_div(L, 32);
    if ((s = launch("opm.pair_count", opm_pair_count_kernel, dim3((unsigned)(tiles * tiles)), dim3(64 * kCountWaves),
                    0, st, mask, S, L, count)))
      return s;
  }

  if (fused_ok(d)) {
    if (!fast && ws.sp > S) {
      const int64_t rows = (int64_t)L * co, n = 2 * rows * (ws.sp - S);
      if ((s = launch("opm.zero_tail", opm_zero_tail_kernel, dim3((unsigned)std::min<int64_t>(ceil_div(n, 256), 1024)),
                      dim3(256), 0, st, (half_t*)(wsb + ws.left), (half_t*)(wsb + ws.right), rows, ws.sp, S)))
        return s;
    }
    GemmArgs g;
    g.a = wsb + ws.left;
    g.b = wsb + ws.right;
    g.c = out;
    g.bias = (const float*)(wb + w.b_out);
    g.opm_w = wb + w.w_out;
    g.M = g.N = L * co;
    g.K = (int)ws.sp;  // sequences [S, sp) are zeros
    g.lda = g.ldb = ws.sp;
    g.ldc = d.c_z;
    g.flags = d.residual ? AFHIP_EPILOGUE_RESIDUAL : 0u;
    g.opm_count = count;
    g.opm_length = L;
    g.opm_eps = d.normalization_epsilon;
    return run_opm_fused(g, d.out_dtype, "opm.fused", st);
  }
  const int ct = f16 ? AFHIP_F16 : AFHIP_F32;
  const size_t es = f16 ? 2 : 4;
  for (int i0 = 0; i0 < L; i0 += ws.row_block) {
    const int cnt = std::min(ws.row_block, L - i0);
    GemmArgs g;
    g.a = wsb + ws.left + es * (size_t)i0 * co * ws.sp;
    g.b = wsb + ws.right;
    g.c = wsb + ws.outer;
    g.M = cnt * co;
    g.N = L * co;
    g.K = S;
    g.lda = ws.sp;
    g.ldb = ws.sp;
    g.ldc = L * co;
    g.flags = EPILOGUE_OPM_CONTRACT;
    g.opm_count = count;
    g.opm_outer = co;
    g.opm_length = L;
    g.opm_row0 = i0;
    g.opm_eps = d.normalization_epsilon;
    GemmTypes t1{d.precision, ct, ct, ct};
    if ((s = run_gemm(g, t1, select_variant(t1, g.M, g.N, g.K, 1), "opm.contract", st))) return s;

    GemmArgs h;
    h.a = wsb + ws.outer;
    h.b = wb + w.w_out;
    h.c = (char*)out + dtype_size(d.out_dtype) * (size_t)i0 * L * d.c_z;
    h.residual = h.c;
    h.bias = (const float*)(wb + w.b_out);
    h.M = cnt * L;
    h.N = d.c_z;
    h.K = co * co;
    h.lda = co * co;
    h.ldb = co * co;
    h.ldc = d.c_z;
    h.flags = EPILOGUE_OPM_OUTPUT | (d.residual ? AFHIP_EPILOGUE_RESIDUAL : 0u);
    h.opm_count = count;
    h.opm_row0 = i0 * L;
    h.opm_eps = d.normalization_epsilon;
    GemmTypes t2{d.precision, ct, ct, d.out_dtype};
    if ((s = run_gemm(h, t2, select_variant(t2, h.M, h.N, h.K, 1), "opm.output", st))) return s;
  }
  return AFHIP_OK;
}

}  // extern "C"
