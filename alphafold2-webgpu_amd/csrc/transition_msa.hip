// The MSA transition in one persistent kernel for f16 precision at the
// AlphaFold widths (channels 256, hidden 1024): LayerNorm, linear 256 -> 1024
// with bias and ReLU, linear 1024 -> 256 with bias (+ the residual)
// (src/evoformer/transition.ts:179-234, :264-361; src/evoformer/block.ts:
// 1713-1716). The hidden activation (268 MB at 512 x 256 rows) never leaves
// the registers.
//
// The weights (1 MiB) do not fit a CU's registers, so they stream: a tile of
// 256 rows walks the hidden units in 32 blocks of 32, and each block's
// weights (W1 rows and W2 columns of those 32 units, 32 KiB in MFMA fragment
// order, prepared once) arrive by DMA in a ring of three LDS buffers shared
// by the workgroup's eight waves, two blocks ahead of their use.
//
// Each wave owns 32 rows of the tile (one MFMA column tile) for the whole
// tile:
//  - their normalised values stay in VGPRs as the B fragments of the first
//    linear (x_hat^T, 16 k-steps of 16 channels);
//  - per hidden block, h = ReLU(W1_b x_hat^T + b1_b) is 32 units x 32 rows of
//    f32 accumulators, a lane holding units 8 j + 4 (lane / 32) + [0, 4) of
//    row lane % 32;
//  - that accumulator is, packed to f16, the B operand of the second linear
//    as it stands: k-step s takes the lane's elements 8 s .. 8 s + 7, which
//    is hidden unit 8 (2 s + e / 4) + 4 (lane / 32) + e % 4 for element e.
//    W2's fragments are prepared in that unit order, so no exchange between
//    lanes is needed;
//  - out^T = W2 h^T accumulates over the 32 blocks into 256 channels x 32
//    rows of f32 (128 registers a lane).
// The LayerNorm affine is folded into W1 and b1 at prepare time
// (W1' = W1 diag(gamma), b1' = b1 + W1 beta), so a row is normalised with one
// multiply-add per value. One workgroup a CU, two waves a SIMD. (64 rows a
// wave would read each weight fragment for two MFMAs, but its 256 output
// accumulators fill the SIMD's accumulator registers, leaving none for the
// hidden block's.)
#include <algorithm>

#include "dma.h"
#include "transition_fused.h"

namespace afhip {

namespace {

constexpr int kC = 256, kH = 1024;
constexpr int kThreads = 512;
constexpr int kWaves = 8;
constexpr int kWaveRows = 32;                 // rows a wave owns
constexpr int kTileRows = kWaves * kWaveRows;  // 256
constexpr int kUnits = 32;                    // hidden units a block
constexpr int kBlocks = kH / kUnits;          // 32
constexpr int kBlockBytes = 32 * 1024;        // W1 fragments (16 KiB), then W2 fragments (16 KiB)
constexpr int kBuffers = 3;
constexpr int kLoadsPerWave = kBlockBytes / 1024 / kWaves;  // 4
constexpr int kB1 = kBuffers * kBlockBytes;   // LDS: folded first bias [1024] f32
constexpr int kB2 = kB1 + kH * 4;             // LDS: second bias [256] f32
constexpr int kLds = kB2 + kC * 4;

template <typename OT>
__global__ __launch_bounds__(kThreads, 1) void transition_msa_kernel(MsaTransitionArgs a, int ntiles) {
  extern __shared__ __attribute__((aligned(1024))) unsigned char smem[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 31, hi = lane >> 5;
  const int G = gridDim.x;
  const int t0 = blockIdx.x;
  if (t0 >= ntiles) return;

  // The biases go to LDS once.
  float* const b1s = reinterpret_cast<float*>(smem + kB1);
  float* const b2s = reinterpret_cast<float*>(smem + kB2);
  for (int i = tid; i < kH; i += kThreads) b1s[i] = a.b1[i];
  for (int i = tid; i < kC; i += kThreads) b2s[i] = a.b2[i];

  // Weight blocks: block j of this workgroup's stream (tile j / 32, hidden
  // block j % 32) goes to buffer j % 3; a wave's load i brings 1 KiB piece
  // wave + 4 i of it.
  const int32x4_t rw = make_rsrc(a.blocks, (uint32_t)(kBlocks * kBlockBytes));
  const uint32_t lds0 = (uint32_t)reinterpret_cast<uintptr_t>(smem);
  auto issue = [&](int j) {
    const int hb = j % kBlocks, buf = j % kBuffers;
#pragma unroll
    for (int i = 0; i < kLoadsPerWave; i++) {
      const int q = wave + kWaves * i;
      dma16(rw, lds0 + buf * kBlockBytes + q * 1024, (uint32_t)(hb * kBlockBytes + q * 1024 + 16 * lane));
    }
  };
  const int my_tiles = (ntiles - t0 + G - 1) / G;
  const int nblocks = my_tiles * kBlocks;
  issue(0);
  if (nblocks > 1) issue(1);

  int it = 0;
  for (int tile = t0; tile < ntiles; tile += G, it++) {
    // This wave's row: r0 + col.
    const int64_t row = (int64_t)tile * kTileRows + kWaveRows * wave + col;
    const bool live = row < a.rows;
    // x_hat fragments: xf[s] holds channels 16 s + 8 hi + [0, 8) of the row.
    // Rows past the end read as zeros.
    half8 xf[16];
    {
      const half_t* xr = a.x + row * kC + 8 * hi;
#pragma unroll
      for (int s = 0; s < 16; s++) {
        if (live) xf[s] = *reinterpret_cast<const half8*>(xr + 16 * s);
        else xf[s] = half8{};
      }
    }
    wait_vmcnt<0>();  // the rows, and every weight block issued so far
    block_barrier();  // the biases are in LDS (first tile); blocks it * 32, + 1 have landed
    // LayerNorm: a row's 256 channels are split between lanes col and
    // col + 32; two-pass mean and biased variance in f32, eps inside the
    // root. The affine is in W1 and b1.
    {
      float s1 = 0.0f;
#pragma unroll
      for (int s = 0; s < 16; s++)
#pragma unroll
        for (int e = 0; e < 8; e++) s1 += (float)xf[s][e];
      s1 += __shfl_xor(s1, 32);
      const float mean = s1 * (1.0f / kC);
      float s2 = 0.0f;
#pragma unroll
      for (int s = 0; s < 16; s++)
#pragma unroll
        for (int e = 0; e < 8; e++) {
          const float d = (float)xf[s][e] - mean;
          s2 += d * d;
        }
      s2 += __shfl_xor(s2, 32);
      const float rstd = fast_rsqrt(s2 * (1.0f / kC) + a.eps);
      const float shift = -mean * rstd;
#pragma unroll
      for (int s = 0; s < 16; s++)
#pragma unroll
        for (int e = 0; e < 8; e++) xf[s][e] = (half_t)fmaf((float)xf[s][e], rstd, shift);
    }

    floatx16 acc2[8];
#pragma unroll
    for (int ob = 0; ob < 8; ob++)
#pragma unroll
      for (int v = 0; v < 16; v++) acc2[ob][v] = 0.0f;

    for (int hb = 0; hb < kBlocks; hb++) {
      const int j = it * kBlocks + hb;
      // Block j has landed once at most the loads issued after it (block
      // j + 1's) are outstanding; with no block after it, all of them. The
      // barrier publishes it and retires buffer (j + 2) % 3, whose block
      // j - 1 every wave has finished.
      if (hb > 0) {
        if (j + 1 < nblocks) wait_vmcnt<kLoadsPerWave>();
        else wait_vmcnt<0>();
        block_barrier<false>();
      }
      if (j + 2 < nblocks) issue(j + 2);
      const unsigned char* wb = smem + (j % kBuffers) * kBlockBytes + 16 * lane;
      // First linear: acc1 = b1' + W1_b x_hat^T.
      floatx16 acc1;
      {
        const float* bb = b1s + kUnits * hb + 4 * hi;
#pragma unroll
        for (int g4 = 0; g4 < 4; g4++) {
          const floatx4 b4 = *reinterpret_cast<const floatx4*>(bb + 8 * g4);
#pragma unroll
          for (int e = 0; e < 4; e++) acc1[4 * g4 + e] = b4[e];
        }
      }
#pragma unroll
      for (int s = 0; s < 16; s++) acc1 = mfma_f16(*reinterpret_cast<const half8*>(wb + 1024 * s), xf[s], acc1);
      // ReLU, f16, and on to the second linear as its B operand.
      half8 hf[2];
#pragma unroll
      for (int s = 0; s < 2; s++)
#pragma unroll
        for (int e = 0; e < 8; e++) hf[s][e] = (half_t)fmaxf(acc1[8 * s + e], 0.0f);
#pragma unroll
      for (int ob = 0; ob < 8; ob++)
#pragma unroll
        for (int s = 0; s < 2; s++)
          acc2[ob] = mfma_f16(*reinterpret_cast<const half8*>(wb + 16384 + 1024 * (2 * ob + s)), hf[s], acc2[ob]);
    }

    // out = acc2 + b2 (+ the old out): lane holds channels 32 ob + 8 g4 +
    // 4 hi + [0, 4) of the row. The old values of a group of channel blocks
    // (two with f16 outputs, one with f32, as registers allow) are read
    // before their stores (a lane reads only what it writes).
    if (live) {
#pragma clang fp contract(off)
      typedef OT ot4 __attribute__((ext_vector_type(4)));
      OT* orow = reinterpret_cast<OT*>(a.out) + row * kC + 4 * hi;
      constexpr int GR = sizeof(OT) == 2 ? 2 : 1;
#pragma unroll
      for (int o2 = 0; o2 < 8; o2 += GR) {
        ot4 old[GR][4];
        if (a.residual) {
#pragma unroll
          for (int d = 0; d < GR; d++)
#pragma unroll
            for (int g4 = 0; g4 < 4; g4++)
              old[d][g4] = *reinterpret_cast<const ot4*>(orow + 32 * (o2 + d) + 8 * g4);
        }
#pragma unroll
        for (int d = 0; d < GR; d++)
#pragma unroll
          for (int g4 = 0; g4 < 4; g4++) {
            const int ob = o2 + d;
            const floatx4 b4 = *reinterpret_cast<const floatx4*>(b2s + 32 * ob + 8 * g4 + 4 * hi);
            ot4 y;
#pragma unroll
            for (int e = 0; e < 4; e++) {
              float v = acc2[ob][4 * g4 + e] + b4[e];
              if (a.residual) v += (float)old[d][g4][e];
              y[e] = (OT)v;
            }
            *reinterpret_cast<ot4*>(orow + 32 * ob + 8 * g4) = y;
          }
      }
    }
  }
}

// Folded, fragment-ordered weights from the packed f32 transition weights
// (packTransitionWeights order, src/evoformer/transition.ts:157-177):
// gamma [C], beta [C], firstWeight [C][H], firstBias [H], secondWeight [H][C],
// secondBias [C]. Block hb (32 units):
//   bytes [0, 16 KiB): W1' fragments (s, lane): unit n = 32 hb + lane % 32,
//     channels 16 s + 8 (lane / 32) + e, value f16(W1[k][n] gamma[k]);
//   bytes [16 KiB, 32 KiB): W2 fragments (ob, s, lane): channel m = 32 ob +
//     lane % 32, element e is unit 32 hb + 8 (2 s + e / 4) + 4 (lane / 32) +
//     e % 4, value f16(W2[unit][m]).
__global__ void msa_prepare_blocks_kernel(const float* __restrict__ packed, half_t* __restrict__ blocks) {
  const float* gamma = packed;
  const float* w1 = packed + 2 * kC;
  const float* w2 = w1 + kC * kH + kH;
  const int64_t total = (int64_t)kBlocks * kBlockBytes / 2;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const int hb = (int)(i / (kBlockBytes / 2));
    const int r = (int)(i % (kBlockBytes / 2));
    const int e = r & 7, ln = (r >> 3) & 63;
    float v;
    if (r < 8192) {
      const int s = r >> 9;
      const int n = kUnits * hb + (ln & 31), k = 16 * s + 8 * (ln >> 5) + e;
      v = w1[(int64_t)k * kH + n] * gamma[k];
    } else {
      const int f = (r - 8192) >> 9;  // 2 ob + s
      const int ob = f >> 1, s = f & 1;
      const int m = 32 * ob + (ln & 31);
      const int unit = kUnits * hb + 8 * (2 * s + (e >> 2)) + 4 * (ln >> 5) + (e & 3);
      v = w2[(int64_t)unit * kC + m];
    }
    blocks[i] = (half_t)v;
  }
}

// b1' = b1 + W1 beta (the folded LayerNorm offset), in double; b2 copied.
__global__ void msa_prepare_bias_kernel(const float* __restrict__ packed, float* __restrict__ b1f,
                                        float* __restrict__ b2f) {
  const float* beta = packed + kC;
  const float* w1 = packed + 2 * kC;
  const float* b1 = w1 + kC * kH;
  const float* b2 = b1 + kH + kH * kC;
  const int n = blockIdx.x * blockDim.x + threadIdx.x;
  if (n < kH) {
    double t = b1[n];
    for (int k = 0; k < kC; k++) t += (double)w1[(int64_t)k * kH + n] * beta[k];
    b1f[n] = (float)t;
  }
  if (n < kC) b2f[n] = b2[n];
}

}  // namespace

bool transition_msa_shape(const afhip_transition_desc& d) {
  return d.precision == AFHIP_PRECISION_F16 && d.channels == kC && d.hidden == kH && d.in_dtype == AFHIP_F16 &&
         d.rows > 0 && ceil_div(d.rows, kTileRows) < ((int64_t)1 << 30);
}

bool transition_msa_eligible(const afhip_transition_desc& d, const void* x, const void* out) {
  return transition_msa_shape(d) && (reinterpret_cast<uintptr_t>(x) & 15) == 0 &&
         (reinterpret_cast<uintptr_t>(out) & 15) == 0;
}

size_t transition_msa_weight_bytes() { return (size_t)kBlocks * kBlockBytes + 4 * (kH + kC); }

int prepare_transition_msa(const float* packed, void* dst, hipStream_t s) {
  half_t* blocks = reinterpret_cast<half_t*>(dst);
  float* b1f = reinterpret_cast<float*>(reinterpret_cast<char*>(dst) + (size_t)kBlocks * kBlockBytes);
  if (int st = launch("transition.prepare", msa_prepare_blocks_kernel, dim3(1024), dim3(256), 0, s, packed, blocks))
    return st;
  return launch("transition.prepare", msa_prepare_bias_kernel, dim3(ceil_div(kH, 256)), dim3(256), 0, s, packed, b1f,
                b1f + kH);
}

int launch_transition_msa(const MsaTransitionArgs& a, int out_dtype, hipStream_t s) {
  const int ntiles = (int)ceil_div(a.rows, kTileRows);
  const int cus = device_cu_count() > 0 ? device_cu_count() : 256;
  const dim3 grid((unsigned)std::min(ntiles, cus));
  if (out_dtype == AFHIP_F16) {
    auto k = transition_msa_kernel<half_t>;
    if (int st = allow_lds((const void*)k, kLds)) return st;
    return launch("transition.msa", k, grid, dim3(kThreads), kLds, s, a, ntiles);
  }
  auto k = transition_msa_kernel<float>;
  if (int st = allow_lds((const void*)k, kLds)) return st;
  return launch("transition.msa", k, grid, dim3(kThreads), kLds, s, a, ntiles);
}

}  // namespace afhip
