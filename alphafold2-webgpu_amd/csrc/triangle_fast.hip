// Triangle multiplication, f16 precision at c_z = c_hidden = 128 (AlphaFold's
// widths): the projection and output kernels, written for HBM throughput.
//
// Both are persistent (one 512-lane workgroup per CU walking 64-pair tiles)
// and split their eight waves by role:
//  - waves 0-3 issue the tile loads, straight into a ring of LDS stages
//    (buffer_load ... lds), STAGES - 1 tiles ahead of the tile being
//    computed. They issue no other vector-memory instruction, so the
//    s_waitcnt vmcnt that says "this tile has landed" is exact.
//  - waves 4-7 write the finished tile back from an LDS staging area with
//    16-byte stores that cover whole 128-byte lines.
//  - all eight compute: LayerNorm out of the stage into an f16 operand tile,
//    then MFMA with weights held in VGPRs for the whole kernel
//    (2 x 8 half8 fragments = 64 VGPRs per wave).
//
// tri_project: wave w projects operand (w >> 2) (a or b), channels
// [32 (w & 3), +32), projection and gate together. The MFMA is issued as
// W (A operand) x zn^T (B operand), so each accumulator is channel-major and
// a = mask (p + bp) sigmoid(g + bg) drops into the [channel][pair] staging
// that becomes the contraction's channel-major operand rows.
//
// tri_output: the contraction tile arrives channel-major; its LayerNorm over
// the 128 hidden channels is computed as per-wave partial statistics (each
// wave owns 16 channels of every pair) merged with Chan's formula, so no
// transpose is needed. z's LayerNorm, linearZ and linearG follow, and
// out = (p + bz) sigmoid(g + bg) (+ out when accumulating) is written along
// the pair's 128 channels.
#include <algorithm>

#include "dma.h"
#include "triangle_fast.h"

namespace afhip {

namespace {

constexpr int kTile = 64;            // pairs per tile
constexpr int kC = 128;              // c_z = c_hidden
constexpr int kThreads = 512;
constexpr int kLoaderWaves = 4;
constexpr int kPitch = kC + 8;       // halves: 272-byte operand rows, 16-byte aligned, conflict-free fragments
constexpr int kOutPitch = kTile + 8; // halves: projection staging rows

__device__ __forceinline__ int pair_of(int r, int L, bool incoming) {
  if (!incoming) return r;
  const int j = r / L;
  return (r - j * L) * L + j;
}

// Eight consecutive channels of one row of a stage, as f32.
template <typename T> __device__ __forceinline__ void read8(const unsigned char* p, float* x);
template <> __device__ __forceinline__ void read8<half_t>(const unsigned char* p, float* x) {
  const half8 h = *reinterpret_cast<const half8*>(p);
#pragma unroll
  for (int e = 0; e < 8; e++) x[e] = (float)h[e];
}
template <> __device__ __forceinline__ void read8<float>(const unsigned char* p, float* x) {
  const floatx4 a = reinterpret_cast<const floatx4*>(p)[0];
  const floatx4 b = reinterpret_cast<const floatx4*>(p)[1];
#pragma unroll
  for (int e = 0; e < 4; e++) {
    x[e] = a[e];
    x[e + 4] = b[e];
  }
}

// LayerNorm of a 128-channel row held by 16 consecutive lanes (8 channels
// each): two-pass mean and biased variance in f32, eps inside the root, as
// the reference's statistics kernels compute them (src/triangle/shaders.ts:
// 242-281); the normalised f16 values go to dst (8 halves).
__device__ __forceinline__ void layer_norm16(const float* x, const float* w, const float* b, float eps,
                                             half_t* dst) {
  float s = 0.0f;
#pragma unroll
  for (int e = 0; e < 8; e++) s += x[e];
  s += __shfl_xor(s, 1);
  s += __shfl_xor(s, 2);
  s += __shfl_xor(s, 4);
  s += __shfl_xor(s, 8);
  const float mean = s * (1.0f / kC);
  float v = 0.0f;
#pragma unroll
  for (int e = 0; e < 8; e++) {
    const float d = x[e] - mean;
    v += d * d;
  }
  v += __shfl_xor(v, 1);
  v += __shfl_xor(v, 2);
  v += __shfl_xor(v, 4);
  v += __shfl_xor(v, 8);
  const float rstd = fast_rsqrt(v * (1.0f / kC) + eps);
  half8 h;
#pragma unroll
  for (int e = 0; e < 8; e++) h[e] = (half_t)((x[e] - mean) * rstd * w[e] + b[e]);
  *reinterpret_cast<half8*>(dst) = h;
}

// Loader-wave wait: stage `it` has landed once at most the loads issued
// after it (`later` instructions) are outstanding.
template <int LATER> __device__ __forceinline__ void wait_stage(bool later_issued) {
  if (later_issued) wait_vmcnt<LATER>();
  else wait_vmcnt<0>();
}

// ---------------------------------------------------------------------------
// Projection
// ---------------------------------------------------------------------------

template <typename ZT> struct ProjectLayout {
  static constexpr int ZROW = kC * (int)sizeof(ZT);   // bytes of one pair row of z
  static constexpr int ZBYTES = kTile * ZROW;         // 16 KiB (f16) or 32 KiB (f32)
  static constexpr int STAGE = ZBYTES + kTile * 4;    // + the tile's mask
  static constexpr int STAGES = sizeof(ZT) == 2 ? 4 : 2;
  static constexpr int ZLOADS = ZBYTES / 1024;        // wave-level 16-byte loads per tile
  static constexpr int LPW = ZLOADS / kLoaderWaves;   // per loader wave (wave 0 adds the mask)
  static constexpr int ROWS_PER_LOAD = 1024 / ZROW;
  static constexpr int LANES_PER_ROW = 64 / ROWS_PER_LOAD;
  static constexpr int ZN = STAGES * STAGE;
  static constexpr int OUT = ZN + kTile * kPitch * 2;
  static constexpr int PARAMS = OUT + 2 * kC * kOutPitch * 2;
  static constexpr int BYTES = PARAMS + 6 * kC * 4;
};

template <typename ZT>
__global__ __launch_bounds__(kThreads, 1) void tri_project_f16_kernel(FastProjectArgs a, int ntiles) {
  using Lay = ProjectLayout<ZT>;
  extern __shared__ __attribute__((aligned(1024))) unsigned char smem[];
  half_t* zn = reinterpret_cast<half_t*>(smem + Lay::ZN);
  half_t* ost = reinterpret_cast<half_t*>(smem + Lay::OUT);
  float* ln = reinterpret_cast<float*>(smem + Lay::PARAMS);  // w [128], b [128]
  float* bias = ln + 2 * kC;                                  // ap, ag, bp, bg [128] each

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int o = wave >> 2;         // 0: a (left), 1: b (right)
  const int hb = 32 * (wave & 3);  // channel block
  const int G = gridDim.x;

  for (int i = tid; i < 2 * kC; i += kThreads) ln[i] = i < kC ? a.ln_w[i] : a.ln_b[i - kC];
  for (int i = tid; i < 4 * kC; i += kThreads) bias[i] = a.b_proj[i];

  // Weight fragments: W[n][k] with n = hb + lane % 32, k = 16 s + 8 (lane / 32).
  const half_t* wp = a.w_proj + (size_t)(2 * o) * kC * kC + (size_t)(hb + (lane & 31)) * kC + 8 * (lane >> 5);
  const half_t* wg = wp + (size_t)kC * kC;
  half8 fp[8], fg[8];
#pragma unroll
  for (int s = 0; s < 8; s++) {
    fp[s] = *reinterpret_cast<const half8*>(wp + 16 * s);
    fg[s] = *reinterpret_cast<const half8*>(wg + 16 * s);
  }
  wait_vmcnt<0>();  // weights in hand before the tile loads queue up behind them

  const int32x4_t rz = make_rsrc(a.z, (uint32_t)((int64_t)a.P * Lay::ZROW));
  const int32x4_t rm = make_rsrc(a.mask, (uint32_t)((int64_t)a.P * 4));
  const uint32_t lds0 = (uint32_t)reinterpret_cast<uintptr_t>(smem);
  auto issue = [&](int tile, int stage) {  // loader waves only
    const uint32_t base = lds0 + stage * Lay::STAGE;
#pragma unroll
    for (int i = 0; i < Lay::LPW; i++) {
      const int q = wave + kLoaderWaves * i;
      const int row = q * Lay::ROWS_PER_LOAD + lane / Lay::LANES_PER_ROW;
      const int chunk = lane % Lay::LANES_PER_ROW;
      const int r = tile * kTile + row;
      const uint32_t off =
          r < a.P ? (uint32_t)pair_of(r, a.L, a.incoming) * Lay::ZROW + 16u * chunk : kOutOfRange;
      dma16(rz, base + q * 1024, off);
    }
    if (wave == 0) {
      const int r = tile * kTile + lane;
      const uint32_t off = r < a.P ? (uint32_t)pair_of(r, a.L, a.incoming) * 4u : kOutOfRange;
      dma4(rm, base + Lay::ZBYTES, off);
    }
  };

  int tile = blockIdx.x;
  if (wave < kLoaderWaves) {
#pragma unroll
    for (int s = 0; s < Lay::STAGES - 1; s++)
      if (tile + s * G < ntiles) issue(tile + s * G, s);
  }
  const float* bp = bias + (2 * o) * kC;
  const float* bg = bias + (2 * o + 1) * kC;

  for (int it = 0; tile < ntiles; it++, tile += G) {
    const int stage = it % Lay::STAGES;
    if (wave < kLoaderWaves) {
      const bool later = tile + (Lay::STAGES - 2) * G < ntiles;
      if (wave == 0) wait_stage<(Lay::STAGES - 2) * (Lay::LPW + 1)>(later);
      else wait_stage<(Lay::STAGES - 2) * Lay::LPW>(later);
    }
    block_barrier();  // B1: stage `it` is complete; stage it - 1 and zn are free
    if (wave < kLoaderWaves && tile + (Lay::STAGES - 1) * G < ntiles)
      issue(tile + (Lay::STAGES - 1) * G, (it + Lay::STAGES - 1) % Lay::STAGES);

    const unsigned char* st = smem + stage * Lay::STAGE;
#pragma unroll
    for (int pass = 0; pass < 2; pass++) {
      const int row = pass * 32 + (tid >> 4);
      const int c0 = (tid & 15) * 8;
      float x[8];
      read8<ZT>(st + row * Lay::ZROW + c0 * (int)sizeof(ZT), x);
      layer_norm16(x, ln + c0, ln + kC + c0, a.eps, zn + row * kPitch + c0);
    }
    block_barrier();  // B2: zn is complete

    const float* mk = reinterpret_cast<const float*>(st + Lay::ZBYTES);
#pragma unroll
    for (int sub = 0; sub < 2; sub++) {
      floatx16 accp, accg;
#pragma unroll
      for (int v = 0; v < 16; v++) accp[v] = accg[v] = 0.0f;
      const half_t* zrow = zn + (sub * 32 + (lane & 31)) * kPitch + 8 * (lane >> 5);
#pragma unroll
      for (int s = 0; s < 8; s++) {
        const half8 zf = *reinterpret_cast<const half8*>(zrow + 16 * s);
        accp = mfma_f16(fp[s], zf, accp);
        accg = mfma_f16(fg[s], zf, accg);
      }
      const int p = sub * 32 + (lane & 31);
      const float m = mk[p];
#pragma unroll
      for (int v = 0; v < 16; v++) {
        const int c = hb + mfma_row(v, lane);
        const float val = m * (accp[v] + bp[c]) * sigmoidf_(accg[v] + bg[c]);
        ost[(o * kC + c) * kOutPitch + p] = (half_t)val;
      }
    }
    block_barrier();  // B3: the staged tile is complete

    if (wave >= kLoaderWaves) {
      // 256 channel rows x 64 pairs: eight 16-byte chunks per row. Pairs past
      // P land in the operand's padding (its rows are cstride >= 64 * ntiles
      // long), which the contraction never reads.
      const int t4 = tid - kLoaderWaves * 64;
#pragma unroll
      for (int k = 0; k < 8; k++) {
        const int idx = t4 + 256 * k;
        const int row = idx >> 3, chunk = idx & 7;
        const uint4 v = *reinterpret_cast<const uint4*>(ost + row * kOutPitch + chunk * 8);
        half_t* dst = (row < kC ? a.out_a : a.out_b) + (size_t)(row & (kC - 1)) * a.cstride +
                      (size_t)tile * kTile + chunk * 8;
        *reinterpret_cast<uint4*>(dst) = v;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Output
// ---------------------------------------------------------------------------

template <typename ZT, typename OT> struct OutputLayout {
  static constexpr int ZROW = kC * (int)sizeof(ZT);
  static constexpr int XBYTES = kC * kTile * 2;      // contraction tile, [128 channels][64 pairs] f16
  static constexpr int ZBYTES = kTile * ZROW;
  static constexpr int STAGE = XBYTES + ZBYTES;
  static constexpr int STAGES = sizeof(ZT) == 2 ? 3 : 2;
  static constexpr int XLOADS = XBYTES / 1024;       // 8 channel rows per load
  static constexpr int ZLOADS = ZBYTES / 1024;
  static constexpr int LPW = (XLOADS + ZLOADS) / kLoaderWaves;
  static constexpr int ZROWS_PER_LOAD = 1024 / ZROW;
  static constexpr int ZLANES_PER_ROW = 64 / ZROWS_PER_LOAD;
  static constexpr int OROW = kC * (int)sizeof(OT);  // staged output row (the stage it aliases is dead by then)
  static_assert(kTile * OROW <= STAGE, "output staging fits in a stage");
  static constexpr int HN = STAGES * STAGE;
  static constexpr int GN = HN + kTile * kPitch * 2;
  static constexpr int PART = GN + kTile * kPitch * 2;   // [8 waves][64 pairs] x (mean, m2)
  static constexpr int PARAMS = PART + 8 * kTile * 2 * 4;
  static constexpr int BYTES = PARAMS + 6 * kC * 4;
};

template <typename ZT, typename OT>
__global__ __launch_bounds__(kThreads, 1) void tri_output_f16_kernel(FastOutputArgs a, int ntiles) {
  using Lay = OutputLayout<ZT, OT>;
  extern __shared__ __attribute__((aligned(1024))) unsigned char smem[];
  half_t* hn = reinterpret_cast<half_t*>(smem + Lay::HN);
  half_t* gn = reinterpret_cast<half_t*>(smem + Lay::GN);
  float2* part = reinterpret_cast<float2*>(smem + Lay::PART);
  float* ln = reinterpret_cast<float*>(smem + Lay::PARAMS);  // out w, out b, in w, in b, bz, bg

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nt = 32 * (wave & 3), rh = 32 * (wave >> 2);
  const int G = gridDim.x;
  for (int i = tid; i < kC; i += kThreads) {
    ln[i] = a.ln_out_w[i];
    ln[kC + i] = a.ln_out_b[i];
    ln[2 * kC + i] = a.ln_in_w[i];
    ln[3 * kC + i] = a.ln_in_b[i];
    ln[4 * kC + i] = a.b_z[i];
    ln[5 * kC + i] = a.b_g[i];
  }

  const half_t* wz = a.w_z + (size_t)(nt + (lane & 31)) * kC + 8 * (lane >> 5);
  const half_t* wgp = a.w_g + (size_t)(nt + (lane & 31)) * kC + 8 * (lane >> 5);
  half8 fz[8], fg[8];
#pragma unroll
  for (int s = 0; s < 8; s++) {
    fz[s] = *reinterpret_cast<const half8*>(wz + 16 * s);
    fg[s] = *reinterpret_cast<const half8*>(wgp + 16 * s);
  }
  wait_vmcnt<0>();  // weights in hand before the tile loads queue up behind them

  const int32x4_t rx = make_rsrc(a.contracted, (uint32_t)((int64_t)kC * a.bstride * 2));
  const int32x4_t rz =
      make_rsrc(reinterpret_cast<const unsigned char*>(a.z) + (size_t)a.pair0 * Lay::ZROW,
                (uint32_t)((int64_t)a.pairs * Lay::ZROW));
  const uint32_t lds0 = (uint32_t)reinterpret_cast<uintptr_t>(smem);
  auto issue = [&](int tile, int stage) {  // loader waves only
    const uint32_t base = lds0 + stage * Lay::STAGE;
    const int q0 = tile * kTile;
#pragma unroll
    for (int i = 0; i < Lay::LPW; i++) {
      const int q = wave + kLoaderWaves * i;
      uint32_t off;
      if (q < Lay::XLOADS) {  // channel rows 8q + lane / 8, pairs q0 + 8 (lane % 8) ..
        const int c = 8 * q + (lane >> 3);
        const int p = q0 + 8 * (lane & 7);
        off = p < a.pairs ? (uint32_t)(((int64_t)c * a.bstride + p) * 2) : kOutOfRange;
        dma16(rx, base + q * 1024, off);
      } else {
        const int zq = q - Lay::XLOADS;
        const int row = zq * Lay::ZROWS_PER_LOAD + lane / Lay::ZLANES_PER_ROW;
        const int chunk = lane % Lay::ZLANES_PER_ROW;
        const int p = q0 + row;
        off = p < a.pairs ? (uint32_t)p * Lay::ZROW + 16u * chunk : kOutOfRange;
        dma16(rz, base + q * 1024, off);
      }
    }
  };

  int tile = blockIdx.x;
  if (wave < kLoaderWaves) {
#pragma unroll
    for (int s = 0; s < Lay::STAGES - 1; s++)
      if (tile + s * G < ntiles) issue(tile + s * G, s);
  }

  for (int it = 0; tile < ntiles; it++, tile += G) {
    const int stage = it % Lay::STAGES;
    if (wave < kLoaderWaves) wait_stage<(Lay::STAGES - 2) * Lay::LPW>(tile + (Lay::STAGES - 2) * G < ntiles);
    block_barrier();  // B1: stage `it` complete; the previous tile's staging is written out
    if (wave < kLoaderWaves && tile + (Lay::STAGES - 1) * G < ntiles)
      issue(tile + (Lay::STAGES - 1) * G, (it + Lay::STAGES - 1) % Lay::STAGES);

    unsigned char* st = smem + stage * Lay::STAGE;
    // Hidden statistics, partial: wave w holds channels [16 w, 16 w + 16) of pair `lane`.
    float xh[16];
    {
      const half_t* xs = reinterpret_cast<const half_t*>(st);
      float s = 0.0f;
#pragma unroll
      for (int e = 0; e < 16; e++) {
        xh[e] = (float)xs[(16 * wave + e) * kTile + lane];
        s += xh[e];
      }
      const float mean = s * (1.0f / 16);
      float m2 = 0.0f;
#pragma unroll
      for (int e = 0; e < 16; e++) {
        const float d = xh[e] - mean;
        m2 += d * d;
      }
      part[wave * kTile + lane] = make_float2(mean, m2);
    }
    // z's LayerNorm, rows of 16 lanes.
#pragma unroll
    for (int pass = 0; pass < 2; pass++) {
      const int row = pass * 32 + (tid >> 4);
      const int c0 = (tid & 15) * 8;
      float x[8];
      read8<ZT>(st + Lay::XBYTES + row * Lay::ZROW + c0 * (int)sizeof(ZT), x);
      layer_norm16(x, ln + 2 * kC + c0, ln + 3 * kC + c0, a.eps, gn + row * kPitch + c0);
    }
    block_barrier();  // B2: partial statistics and gn complete
    {
      // Chan et al.: merge eight (mean, M2) over 16 channels each.
      float mean = 0.0f;
#pragma unroll
      for (int w = 0; w < 8; w++) mean += part[w * kTile + lane].x;
      mean *= 1.0f / 8;
      float m2 = 0.0f;
#pragma unroll
      for (int w = 0; w < 8; w++) {
        const float2 pw = part[w * kTile + lane];
        const float d = pw.x - mean;
        m2 += pw.y + 16.0f * d * d;
      }
      const float rstd = fast_rsqrt(m2 * (1.0f / kC) + a.eps);
      half8 h0, h1;
#pragma unroll
      for (int e = 0; e < 8; e++) {
        const int c = 16 * wave + e;
        h0[e] = (half_t)((xh[e] - mean) * rstd * ln[c] + ln[kC + c]);
        h1[e] = (half_t)((xh[e + 8] - mean) * rstd * ln[c + 8] + ln[kC + c + 8]);
      }
      half_t* dst = hn + lane * kPitch + 16 * wave;
      reinterpret_cast<half8*>(dst)[0] = h0;
      reinterpret_cast<half8*>(dst)[1] = h1;
    }
    block_barrier();  // B3: hn complete; the stage is dead and becomes the output staging

    floatx16 accz, accg;
#pragma unroll
    for (int v = 0; v < 16; v++) accz[v] = accg[v] = 0.0f;
    const half_t* hrow = hn + (rh + (lane & 31)) * kPitch + 8 * (lane >> 5);
    const half_t* grow = gn + (rh + (lane & 31)) * kPitch + 8 * (lane >> 5);
#pragma unroll
    for (int s = 0; s < 8; s++) {
      accz = mfma_f16(*reinterpret_cast<const half8*>(hrow + 16 * s), fz[s], accz);
      accg = mfma_f16(*reinterpret_cast<const half8*>(grow + 16 * s), fg[s], accg);
    }
    {
      const int n = nt + (lane & 31);
      const float bzn = ln[4 * kC + n], bgn = ln[5 * kC + n];
      OT* ost = reinterpret_cast<OT*>(st);
#pragma unroll
      for (int v = 0; v < 16; v++) {
        const int q = rh + mfma_row(v, lane);
        ost[q * kC + n] = (OT)((accz[v] + bzn) * sigmoidf_(accg[v] + bgn));
      }
    }
    block_barrier();  // B4: the output tile is staged

    if (wave >= kLoaderWaves) {
      // 64 pair rows of OROW bytes in 16-byte chunks, straight to [pair][128].
      constexpr int CHUNKS = Lay::OROW / 16;
      constexpr int PER_LANE = kTile * CHUNKS / 256;
      const int t4 = tid - kLoaderWaves * 64;
      const int q0 = tile * kTile;
#pragma unroll
      for (int k = 0; k < PER_LANE; k++) {
        const int idx = t4 + 256 * k;
        const int q = idx / CHUNKS, chunk = idx % CHUNKS;
        if (q0 + q >= a.pairs) continue;
        uint4 v = *reinterpret_cast<const uint4*>(st + q * Lay::OROW + chunk * 16);
        unsigned char* dst =
            reinterpret_cast<unsigned char*>(a.out) + ((size_t)a.pair0 + q0 + q) * Lay::OROW + chunk * 16;
        if (a.residual) {
          const uint4 r = *reinterpret_cast<const uint4*>(dst);
          constexpr int E = 16 / (int)sizeof(OT);
          OT* vv = reinterpret_cast<OT*>(&v);
          const OT* rr = reinterpret_cast<const OT*>(&r);
#pragma unroll
          for (int e = 0; e < E; e++) vv[e] = (OT)((float)vv[e] + (float)rr[e]);
        }
        *reinterpret_cast<uint4*>(dst) = v;
      }
    }
  }
}

int grid_for(int tiles) {
  const int cus = device_cu_count() > 0 ? device_cu_count() : 256;
  return std::max(1, std::min(tiles, cus));
}

template <typename K> int prepare_lds(K kernel, int bytes) { return allow_lds((const void*)kernel, (size_t)bytes); }

}  // namespace

bool triangle_fast_eligible(const afhip_triangle_desc& d) {
  if (d.precision != AFHIP_PRECISION_F16 || d.c_z != kC || d.c_hidden != kC) return false;
  // Byte offsets into z (and the mask) must stay below the out-of-range marker.
  const int64_t P = (int64_t)d.length * d.length;
  return P * kC * (d.pair_dtype == AFHIP_F32 ? 4 : 2) < (int64_t)kOutOfRange;
}

int launch_triangle_project_f16(const FastProjectArgs& a, int pair_dtype, hipStream_t s) {
  const int tiles = (int)ceil_div(a.P, kTile);
  const dim3 g(grid_for(tiles)), b(kThreads);
  if (pair_dtype == AFHIP_F16) {
    auto k = tri_project_f16_kernel<half_t>;
    if (int st = prepare_lds(k, ProjectLayout<half_t>::BYTES)) return st;
    return launch("triangle.project", k, g, b, ProjectLayout<half_t>::BYTES, s, a, tiles);
  }
  auto k = tri_project_f16_kernel<float>;
  if (int st = prepare_lds(k, ProjectLayout<float>::BYTES)) return st;
  return launch("triangle.project", k, g, b, ProjectLayout<float>::BYTES, s, a, tiles);
}

template <typename ZT, typename OT> int launch_output(const FastOutputArgs& a, hipStream_t s) {
  const int tiles = (int)ceil_div(a.pairs, kTile);
  auto k = tri_output_f16_kernel<ZT, OT>;
  constexpr int bytes = OutputLayout<ZT, OT>::BYTES;
  if (int st = prepare_lds(k, bytes)) return st;
  return launch("triangle.output", k, dim3(grid_for(tiles)), dim3(kThreads), bytes, s, a, tiles);
}

int launch_triangle_output_f16(const FastOutputArgs& a, int pair_dtype, int out_dtype, hipStream_t s) {
  if (pair_dtype == AFHIP_F16) {
    if (out_dtype == AFHIP_F32) return launch_output<half_t, float>(a, s);
    return launch_output<half_t, half_t>(a, s);
  }
  if (out_dtype == AFHIP_F32) return launch_output<float, float>(a, s);
  return launch_output<float, half_t>(a, s);
}

}  // namespace afhip
