// The pair transition in one persistent kernel for f16 precision at the
// AlphaFold widths (channels 128, hidden 512): LayerNorm, linear 128 -> 512
// with bias and ReLU, linear 512 -> 128 with bias (+ the residual), with the
// hidden activation kept in LDS instead of a 2 GB round trip through HBM
// (src/evoformer/transition.ts:179-234, :264-361).
//
// A workgroup of eight waves walks 32-row tiles. Every wave holds, for the
// whole kernel, a 16 KiB slice of each weight matrix in VGPRs:
//   first linear:  hidden units 64 w .. 64 w + 63 (two 32-row MFMA tiles),
//   second linear: outputs 32 (w % 4) .. + 31 over hidden half w / 4,
// so the tile's x_hat (LDS) and hidden (LDS) are the only operands read per
// tile. Both MFMAs are issued weights-first (W as the A operand, the tile
// transposed as B), so a lane's accumulator column is one row of the tile
// and its values come in runs of four consecutive channels: 8-byte hidden
// writes, 16-byte output writes. Each bias rides in one more k-step: the A
// fragment holds the bias split into two f16 halves (hi + lo), the B
// fragment ones, so the MFMA adds it in f32. The second linear's two hidden
// halves meet in LDS: waves 4-7 leave their partial sums, waves 0-3 add them.
//
// Loads: waves 0-3 bring x tiles into a ring of three LDS stages by DMA (and
// issue no other vector-memory instruction, so their vmcnt waits are exact);
// waves 4-7 write the finished tile of the previous iteration from one of two
// staging buffers, with the residual read-modify-write there. A tile's
// LayerNorm runs during the previous tile's second linear, three barriers a
// tile.
#include <algorithm>

#include "dma.h"
#include "transition_fused.h"

namespace afhip {

namespace {

constexpr int kC = 128, kH = 512;
constexpr int kRows = 32;  // rows per tile
constexpr int kThreads = 512;
constexpr int kLoaders = 4;
constexpr int kXPitch = kC + 8;  // halves: x_hat rows
constexpr int kHPitch = kH + 8;  // halves: hidden rows

template <typename IT, typename OT> struct FusedLayout {
  static constexpr int XROW = kC * (int)sizeof(IT);
  static constexpr int STAGE = kRows * XROW;
  static constexpr int STAGES = 3;
  static constexpr int LOADS = STAGE / 1024;
  static constexpr int LPW = LOADS / kLoaders;
  static constexpr int XHAT = STAGES * STAGE;
  static constexpr int HID = XHAT + kRows * kXPitch * 2;
  static constexpr int PART = HID + kRows * kHPitch * 2;  // four waves' 32 x 32 f32 partial tiles
  static constexpr int ORow = kC * (int)sizeof(OT);
  static constexpr int OPITCH = ORow + 16;
  static constexpr int OUTB = PART + 4 * 64 * 16 * 4;
  static constexpr int BYTES = OUTB + 2 * kRows * OPITCH;
};
static_assert(FusedLayout<float, float>::BYTES <= 160 * 1024, "LDS budget");

__device__ __forceinline__ uint32_t pack_hilo(float b) {
  const half_t hi = (half_t)b;
  const half_t lo = (half_t)(b - (float)hi);
  return (uint32_t)__builtin_bit_cast(uint16_t, hi) | ((uint32_t)__builtin_bit_cast(uint16_t, lo) << 16);
}

template <typename IT, typename OT>
__global__ __launch_bounds__(kThreads, 1) void transition_fused_kernel(FusedTransitionArgs a, int ntiles) {
  using Lay = FusedLayout<IT, OT>;
  constexpr int S = Lay::STAGES;
  constexpr int LPW = Lay::LPW;
  extern __shared__ __attribute__((aligned(1024))) unsigned char smem[];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int G = gridDim.x;
  const int t0 = blockIdx.x;
  const int col = lane & 31, hi = lane >> 5;

  // B fragment of the bias k-step: (1, 1) at k = 0, 1 of lanes 0-31.
  const half8 ones = __builtin_bit_cast(half8, u32x4{lane < 32 ? 0x3C003C00u : 0u, 0u, 0u, 0u});

  // First linear, A operand: W1[n][k], n = 64 wave + 32 cb + lane % 32,
  // k = 16 s + 8 (lane / 32); step 8 is the bias.
  half8 w1f[2][9];
#pragma unroll
  for (int cb = 0; cb < 2; cb++) {
    const int n = 64 * wave + 32 * cb + col;
    const half_t* wp = a.w1 + (size_t)n * kC + 8 * hi;
#pragma unroll
    for (int s = 0; s < 8; s++) w1f[cb][s] = *reinterpret_cast<const half8*>(wp + 16 * s);
    w1f[cb][8] = __builtin_bit_cast(half8, u32x4{lane < 32 ? pack_hilo(a.b1[n]) : 0u, 0u, 0u, 0u});
  }
  // Second linear, A operand: W2[n][k], n = 32 cb2 + lane % 32,
  // k = 256 kh + 16 s + 8 (lane / 32); step 16 is the bias (half 0 only).
  const int cb2 = wave & 3, kh = wave >> 2;
  half8 w2f[17];
  {
    const int n = 32 * cb2 + col;
    const half_t* wp = a.w2 + (size_t)n * kH + 256 * kh + 8 * hi;
#pragma unroll
    for (int s = 0; s < 16; s++) w2f[s] = *reinterpret_cast<const half8*>(wp + 16 * s);
    w2f[16] = __builtin_bit_cast(half8, u32x4{lane < 32 && kh == 0 ? pack_hilo(a.b2[n]) : 0u, 0u, 0u, 0u});
  }
  // LayerNorm: sixteen lanes a row, eight channels each.
  const int lrow = tid >> 4, lpart = tid & 15;
  float sc[8], of[8];
#pragma unroll
  for (int e = 0; e < 8; e++) {
    sc[e] = a.scale[8 * lpart + e];
    of[e] = a.offset[8 * lpart + e];
  }
  wait_vmcnt<0>();  // weights in hand before the tile loads queue up behind them

  // Loads: load i of a loader wave brings 1 KiB block q = wave + 4 i of the
  // tile (rows are contiguous in x); rows past the end read as zeros.
  const int32x4_t rx = make_rsrc(a.x, (uint32_t)((int64_t)a.rows * Lay::XROW));
  const uint32_t lds0 = (uint32_t)reinterpret_cast<uintptr_t>(smem);
  auto issue = [&](int tile, int stage) {  // loader waves only
    const int64_t lim = a.rows - (int64_t)tile * kRows;
#pragma unroll
    for (int i = 0; i < LPW; i++) {
      const int q = wave + kLoaders * i;
      const uint32_t voff = (uint32_t)(q * 1024 + 16 * lane);
      const bool in = (int64_t)(voff / Lay::XROW) < lim;
      dma16_so(rx, lds0 + stage * Lay::STAGE + q * 1024, in ? voff : kOutOfRange, (uint32_t)tile * Lay::STAGE);
    }
  };

  // Stores (waves 4-7) of the tile in staging buffer `buf`, 16-byte chunks,
  // the residual added when asked.
  constexpr int OCH = Lay::ORow / 16;           // chunks a row
  constexpr int OPER = kRows * OCH / 256;       // chunks a thread
  static_assert(OPER == 2 || OPER == 4, "stores go in groups of two or four");
  auto store_tile = [&](int buf, int tile) {
    const int t4 = tid - 4 * 64;
    const unsigned char* ob = smem + Lay::OUTB + buf * kRows * Lay::OPITCH;
    u32x4 v[OPER];
#pragma unroll
    for (int k = 0; k < OPER; k++) {
      const int idx = t4 + 256 * k;
      const int r = idx / OCH, c = idx % OCH;
      v[k] = *reinterpret_cast<const u32x4*>(ob + r * Lay::OPITCH + 16 * c);
      const int64_t row = (int64_t)tile * kRows + r;
      if (row >= a.rows) continue;
      unsigned char* dst = reinterpret_cast<unsigned char*>(a.out) + row * Lay::ORow + 16 * c;
      if (a.residual) {
        const u32x4 old = *reinterpret_cast<const u32x4*>(dst);
        constexpr int E = 16 / (int)sizeof(OT);
        OT* vv = reinterpret_cast<OT*>(&v[k]);
        const OT* rr = reinterpret_cast<const OT*>(&old);
#pragma unroll
        for (int e = 0; e < E; e++) vv[e] = (OT)((float)vv[e] + (float)rr[e]);
      }
      *reinterpret_cast<u32x4*>(dst) = v[k];
    }
    if constexpr (OPER == 2) stores_read(v[0], v[1]);
    else stores_read(v[0], v[1], v[2], v[3]);
  };

  half_t* const xhat = reinterpret_cast<half_t*>(smem + Lay::XHAT);
  half_t* const hid = reinterpret_cast<half_t*>(smem + Lay::HID);
  float* const part = reinterpret_cast<float*>(smem + Lay::PART);

  // LayerNorm of the tile in stage slot `slot` into x_hat: two-pass mean and
  // biased variance in f32, eps inside the root (transition.ts:179-234).
  auto layer_norm = [&](int slot) {
    const unsigned char* st = smem + slot * Lay::STAGE + lrow * Lay::XROW;
    float x[8];
    if constexpr (sizeof(IT) == 2) {
      const half8 h = *reinterpret_cast<const half8*>(st + 16 * lpart);
#pragma unroll
      for (int e = 0; e < 8; e++) x[e] = (float)h[e];
    } else {
      const floatx4 f0 = reinterpret_cast<const floatx4*>(st + 32 * lpart)[0];
      const floatx4 f1 = reinterpret_cast<const floatx4*>(st + 32 * lpart)[1];
#pragma unroll
      for (int e = 0; e < 4; e++) {
        x[e] = f0[e];
        x[e + 4] = f1[e];
      }
    }
    float s1 = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; e++) s1 += x[e];
    const float mean = row_sum16(s1) / (float)kC;
    float s2 = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; e++) {
      const float d = x[e] - mean;
      s2 += d * d;
    }
    const float rstd = fast_rsqrt(row_sum16(s2) / (float)kC + a.eps);
    half8 h;
#pragma unroll
    for (int e = 0; e < 8; e++) h[e] = (half_t)((x[e] - mean) * rstd * sc[e] + of[e]);
    *reinterpret_cast<half8*>(xhat + lrow * kXPitch + 8 * lpart) = h;
  };

  if (t0 >= ntiles) return;
  // Tile i of this workgroup (tile t0 + i G) goes to stage slot i % 3. Slots
  // for tiles 0, 1, 2 are issued here; tile i + 3 is issued once tile i has
  // been normalised.
  if (wave < kLoaders) {
#pragma unroll
    for (int s = 0; s < S; s++)
      if (t0 + s * G < ntiles) issue(t0 + s * G, s);
    // Tile 0 has landed once at most tiles 1 and 2 are outstanding.
    if (t0 + 2 * G < ntiles) wait_vmcnt<2 * LPW>();
    else if (t0 + G < ntiles) wait_vmcnt<LPW>();
    else wait_vmcnt<0>();
  }
  block_barrier();
  layer_norm(0);

  // Per tile i, three barriers:
  //   A: x_hat(i) is complete, tile i + 1 has landed, staging(i - 1) is complete
  //      -> loaders refill tile i's slot with tile i + 3, storers write tile
  //         i - 1, everyone runs the first linear
  //   B: hidden(i) is complete and x_hat is free
  //      -> the second linear, with tile i + 1's LayerNorm in the same
  //         straight-line block so its vector work issues under the MFMAs
  //   C: the partial sums are complete -> waves 0-3 finish the tile into staging
  int it = 0, tile = t0;
  for (; tile < ntiles; it++, tile += G) {
    if (wave < kLoaders) {
      // Tile it + 1 has landed once at most tile it + 2's loads are outstanding.
      if (tile + 2 * G < ntiles) wait_vmcnt<LPW>();
      else wait_vmcnt<0>();
    }
    block_barrier();  // A
    if (wave < kLoaders) {
      if (tile + 3 * G < ntiles) issue(tile + 3 * G, it % S);
    } else if (it > 0) {
      store_tile((it + 1) & 1, tile - G);
    }

    // First linear: hidden units 64 wave .. + 63 of the 32 rows.
    {
      floatx16 acc[2] = {};
#pragma unroll
      for (int s = 0; s < 8; s++) {
        const half8 xf = *reinterpret_cast<const half8*>(xhat + col * kXPitch + 16 * s + 8 * hi);
        acc[0] = mfma_f16(w1f[0][s], xf, acc[0]);
        acc[1] = mfma_f16(w1f[1][s], xf, acc[1]);
      }
      acc[0] = mfma_f16(w1f[0][8], ones, acc[0]);
      acc[1] = mfma_f16(w1f[1][8], ones, acc[1]);
#pragma unroll
      for (int cb = 0; cb < 2; cb++)
#pragma unroll
        for (int g4 = 0; g4 < 4; g4++) {
          half4 h;
#pragma unroll
          for (int e = 0; e < 4; e++) h[e] = (half_t)fmaxf(acc[cb][4 * g4 + e], 0.0f);
          *reinterpret_cast<half4*>(hid + col * kHPitch + 64 * wave + 32 * cb + 8 * g4 + 4 * hi) = h;
        }
    }
    block_barrier();  // B

    // Second linear: outputs 32 cb2 .. + 31 over hidden half kh; then the
    // next tile's LayerNorm (past the last tile it normalises a stale slot,
    // whose x_hat nothing reads).
    floatx16 acc2 = {};
#pragma unroll
    for (int s = 0; s < 16; s++) {
      const half8 hf = *reinterpret_cast<const half8*>(hid + col * kHPitch + 256 * kh + 16 * s + 8 * hi);
      acc2 = mfma_f16(w2f[s], hf, acc2);
    }
    acc2 = mfma_f16(w2f[16], ones, acc2);  // the bias; its fragment is zero on the waves of half 1
    layer_norm((it + 1) % S);
    if (kh != 0) {
      floatx4* pp = reinterpret_cast<floatx4*>(part + (cb2 * 64 + lane) * 16);
#pragma unroll
      for (int q = 0; q < 4; q++) pp[q] = floatx4{acc2[4 * q], acc2[4 * q + 1], acc2[4 * q + 2], acc2[4 * q + 3]};
    }
    block_barrier();  // C
    if (kh == 0) {
      const floatx4* pp = reinterpret_cast<const floatx4*>(part + (cb2 * 64 + lane) * 16);
      unsigned char* ob = smem + Lay::OUTB + (it & 1) * kRows * Lay::OPITCH + col * Lay::OPITCH;
#pragma unroll
      for (int g4 = 0; g4 < 4; g4++) {
        const floatx4 p = pp[g4];
        const int n0 = 32 * cb2 + 8 * g4 + 4 * hi;
        if constexpr (sizeof(OT) == 4) {
          *reinterpret_cast<floatx4*>(ob + 4 * n0) =
              floatx4{acc2[4 * g4] + p[0], acc2[4 * g4 + 1] + p[1], acc2[4 * g4 + 2] + p[2], acc2[4 * g4 + 3] + p[3]};
        } else {
          half4 h;
#pragma unroll
          for (int e = 0; e < 4; e++) h[e] = (half_t)(acc2[4 * g4 + e] + p[e]);
          *reinterpret_cast<half4*>(ob + 2 * n0) = h;
        }
      }
    }
  }
  block_barrier();  // the last tile's staging is complete
  if (wave >= kLoaders) store_tile((it + 1) & 1, tile - G);
}

template <typename IT, typename OT> int launch_fused(const FusedTransitionArgs& a, hipStream_t s) {
  const int ntiles = (int)ceil_div(a.rows, kRows);
  const int cus = device_cu_count() > 0 ? device_cu_count() : 256;
  auto k = transition_fused_kernel<IT, OT>;
  constexpr int bytes = FusedLayout<IT, OT>::BYTES;
  if (int st = allow_lds((const void*)k, bytes)) return st;
  return launch("transition.fused", k, dim3(std::min(ntiles, cus)), dim3(kThreads), bytes, s, a, ntiles);
}

}  // namespace

bool transition_fused_shape(const afhip_transition_desc& d) {
  return d.precision == AFHIP_PRECISION_F16 && d.channels == kC && d.hidden == kH &&
         d.rows * (int64_t)kC * 4 < (int64_t)kOutOfRange;
}

bool transition_fused_eligible(const afhip_transition_desc& d, const void* x, const void* out) {
  return transition_fused_shape(d) && (reinterpret_cast<uintptr_t>(x) & 15) == 0 &&
         (reinterpret_cast<uintptr_t>(out) & 15) == 0;
}

int launch_transition_fused(const FusedTransitionArgs& a, int in_dtype, int out_dtype, hipStream_t s) {
  if (in_dtype == AFHIP_F16)
    return out_dtype == AFHIP_F16 ? launch_fused<half_t, half_t>(a, s) : launch_fused<half_t, float>(a, s);
  return out_dtype == AFHIP_F16 ? launch_fused<float, half_t>(a, s) : launch_fused<float, float>(a, s);
}

}  // namespace afhip
