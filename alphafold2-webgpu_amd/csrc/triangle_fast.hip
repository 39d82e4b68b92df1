// Triangle multiplication, f16 precision at c_z = c_hidden = 128 (AlphaFold's
// widths): the projection and output kernels, written for HBM throughput.
//
// Both are persistent (one 512-lane workgroup per CU walking 64-pair tiles)
// and split their eight waves by role:
//  - waves 0-3 issue the tile loads, straight into a ring of LDS stages
//    (buffer_load ... lds) several tiles ahead. Besides those they issue
//    only a fixed number of stores a tile, so the s_waitcnt vmcnt that says
//    "this tile has landed" is exact.
//  - the finished tile goes back to HBM with 16-byte stores that cover
//    whole 128-byte lines: from an LDS staging area (the projection: each
//    wave stores the rows it wrote, right after writing them) or straight
//    from the accumulators (the pipelined output kernel).
//  - all eight compute, with the weights held in VGPRs for the whole kernel
//    (2 x 8 half8 fragments = 64 VGPRs per wave).
//
// The weights come folded (fold_weights_kernel, triangle.hip): the
// LayerNorm affines live inside W and b, so normalising is one FMA per
// element (x_hat = x rstd - mean rstd), the biases seed the accumulators,
// and the gates' rows carry -log2(e), so sigmoid(g) = 1 / (1 + 2^acc).
//
// tri_project: wave w projects operand (w >> 2) (a or b), channels
// [32 (w & 3), +32), projection and gate together. The MFMA is issued as
// zn (A operand) x W^T (B operand): a lane's accumulator column is one
// channel and its rows come in runs of four consecutive pairs, so
// a = mask p sigmoid(g) goes into the [channel][pair] staging (the
// contraction's channel-major operand rows) as 8-byte writes. The loop is
// software-pipelined: tile t's MFMAs and tile t+1's LayerNorm are one
// straight-line block (two zn buffers), so the matrix and vector pipes
// overlap, with one barrier per tile.
//
// tri_output: the contraction tile arrives channel-major; its LayerNorm over
// the 128 hidden channels is computed as per-wave partial statistics (each
// wave owns 16 channels of every pair) merged with Chan's formula, so no
// transpose is needed. z's LayerNorm, linearZ and linearG follow, and
// out = p sigmoid(g) (+ out when accumulating) is written along the pair's
// 128 channels.
#include <algorithm>
#include <type_traits>

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

// x_hat of a 128-channel row held by 16 consecutive lanes (8 channels each):
// two-pass mean and biased variance in f32, eps inside the root, as the
// reference's statistics kernels compute them (src/triangle/shaders.ts:
// 242-281); the affine is folded into the weights. 8 halves to dst.
__device__ __forceinline__ void normalize16(const float* x, float eps, half_t* dst) {
  float s = 0.0f;
#pragma unroll
  for (int e = 0; e < 8; e++) s += x[e];
  s = row_sum16(s);
  const float mean = s * (1.0f / kC);
  float v = 0.0f;
#pragma unroll
  for (int e = 0; e < 8; e++) {
    const float d = x[e] - mean;
    v += d * d;
  }
  v = row_sum16(v);
  const float rstd = fast_rsqrt(v * (1.0f / kC) + eps);
  const float shift = -mean * rstd;
  half8 h;
#pragma unroll
  for (int e = 0; e < 8; e++) h[e] = (half_t)fmaf(x[e], rstd, shift);
  *reinterpret_cast<half8*>(dst) = h;
}

// sigmoid of the gate whose accumulator holds -(g) log2(e).
__device__ __forceinline__ float gate_of(float acc) { return fast_rcp(1.0f + __builtin_amdgcn_exp2f(acc)); }

// Loader-wave wait: a tile has landed once at most the loads issued after
// it (LATER instructions, when all were issued) are outstanding.
template <int LATER> __device__ __forceinline__ void wait_stage(bool later_issued) {
  if (later_issued) wait_vmcnt<LATER>();
  else wait_vmcnt<0>();
}

// wait_vmcnt<BASE + STEP * min(k, KMAX)>() for a wave-uniform k.
template <int BASE, int STEP, int KMAX> __device__ __forceinline__ void wait_vmcnt_by(int k) {
  if constexpr (KMAX == 0) {
    wait_vmcnt<BASE>();
  } else {
    if (k >= KMAX) wait_vmcnt<BASE + STEP * KMAX>();
    else wait_vmcnt_by<BASE, STEP, KMAX - 1>(k);
  }
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
  static constexpr int ZN = STAGES * STAGE;                 // two x_hat tiles
  static constexpr int MASK = ZN + 2 * kTile * kPitch * 2;  // two tiles' masks
  static constexpr int OUT = MASK + 2 * kTile * 4;          // [256 channels][64 pairs] staging
  static constexpr int BYTES = OUT + 2 * kC * kOutPitch * 2;
};

template <typename ZT, bool INCOMING>
__global__ __launch_bounds__(kThreads, 1) void tri_project_f16_kernel(FastProjectArgs a, int ntiles) {
  using Lay = ProjectLayout<ZT>;
  constexpr int S = Lay::STAGES;
  extern __shared__ __attribute__((aligned(1024))) unsigned char smem[];
  half_t* const zn_base = reinterpret_cast<half_t*>(smem + Lay::ZN);
  float* const mask_base = reinterpret_cast<float*>(smem + Lay::MASK);
  half_t* const ost = reinterpret_cast<half_t*>(smem + Lay::OUT);

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int o = wave >> 2;         // 0: a (left), 1: b (right)
  const int hb = 32 * (wave & 3);  // channel block
  const int G = gridDim.x;
  const int t0 = blockIdx.x;

  // Weight fragments (the B operand): W[n][k] with n = hb + lane % 32,
  // k = 16 s + 8 (lane / 32); the biases of this lane's channel. They are
  // waited for together with the first two tiles, below.
  const int ch = hb + (lane & 31);
  const half_t* wp = a.w_proj + (size_t)(2 * o) * kC * kC;
  const half_t* wg = wp + (size_t)kC * kC;
  half8 fp[8], fg[8];
#pragma unroll
  for (int s = 0; s < 8; s++) {
    fp[s] = fold_fragment(wp, wave & 3, s, lane);
    fg[s] = fold_fragment(wg, wave & 3, s, lane);
  }
  const float bp = a.b_proj[(2 * o) * kC + ch];
  const float bg = a.b_proj[(2 * o + 1) * kC + ch];

  // Incoming lanes read z (and the mask) at their own offsets into the whole
  // tensor (triangle_fast_eligible keeps it within 32 bits); outgoing tiles
  // are consecutive pairs, addressed through a resource based at the tile.
  const int32x4_t rz = make_rsrc(a.z, (uint32_t)std::min<int64_t>((int64_t)a.P * Lay::ZROW, UINT32_MAX));
  const int32x4_t rm = make_rsrc(a.mask, (uint32_t)((int64_t)a.P * 4));
  const uint32_t lds0 = (uint32_t)reinterpret_cast<uintptr_t>(smem);
  // Load geometry: load i of a loader wave fills stage row
  // row_i = (wave + 4 i) * ROWS_PER_LOAD + lane / LANES_PER_ROW, 16-byte chunk
  // lane % LANES_PER_ROW; wave 0 also loads the tile's 64 mask values.
  // Outgoing pairs are consecutive rows of z: the lane's offset within the
  // tile is fixed and the tile's base is the base of the tile's resource;
  // rows past P read as zeros. Incoming pairs are z
  // transposed: row r of the tile stream is pair (r % L) * L + r / L, whose
  // coordinates (r / L, r % L) each lane advances by G * 64 rows per issued
  // tile instead of dividing.
  constexpr int NL = Lay::LPW + 1;  // the loads, then the mask (wave 0)
  uint32_t vofs[NL];
  int ci[NL], ck[NL];  // incoming: r / L and r % L of the lane's next row
  const int dq = (G * kTile) / a.L, dr = (G * kTile) % a.L;
#pragma unroll
  for (int i = 0; i < NL; i++) {
    const int row = i < Lay::LPW ? (wave + kLoaderWaves * i) * Lay::ROWS_PER_LOAD + lane / Lay::LANES_PER_ROW : lane;
    const int chunk = i < Lay::LPW ? lane % Lay::LANES_PER_ROW : 0;
    if constexpr (INCOMING) {
      const int r = t0 * kTile + row;
      ci[i] = r / a.L;
      ck[i] = r - ci[i] * a.L;
      vofs[i] = 16u * chunk;
    } else {
      vofs[i] = i < Lay::LPW ? (uint32_t)(row * Lay::ZROW + 16 * chunk) : (uint32_t)(4 * row);
    }
  }
  auto issue = [&](int tile, int stage) {  // loader waves only, tiles t0, t0 + G, ... in order
    const uint32_t base = lds0 + stage * Lay::STAGE;
#pragma unroll
    for (int i = 0; i < NL; i++) {
      if (i == Lay::LPW && wave != 0) break;
      const uint32_t lds = i < Lay::LPW ? base + (wave + kLoaderWaves * i) * 1024 : base + Lay::ZBYTES;
      const uint32_t esz = i < Lay::LPW ? (uint32_t)Lay::ZROW : 4u;
      if constexpr (INCOMING) {
        // Rows past P read pair 0: their results land in the operands'
        // padding, which the contraction never reads.
        const uint32_t off = ci[i] < a.L ? (uint32_t)(ck[i] * a.L + ci[i]) * esz + vofs[i] : vofs[i];
        if (i < Lay::LPW) dma16(rz, lds, off);
        else dma4(rm, lds, off);
        ck[i] += dr;
        ci[i] += dq;
        if (ck[i] >= a.L) {
          ck[i] -= a.L;
          ci[i] += 1;
        }
      } else {
        // A resource based at the tile's first pair and ending at P (or past
        // the tile): rows past P read as zeros.
        const int64_t first = (int64_t)tile * kTile;
        const int rows = min(kTile, a.P - tile * kTile);
        const int32x4_t rt = i < Lay::LPW
                                 ? make_rsrc(reinterpret_cast<const unsigned char*>(a.z) + first * Lay::ZROW,
                                             (uint32_t)(rows * Lay::ZROW))
                                 : make_rsrc(a.mask + first, (uint32_t)(rows * 4));
        if (i < Lay::LPW) dma16(rt, lds, vofs[i]);
        else dma4(rt, lds, vofs[i]);
      }
    }
  };
  // Loader waves. Before the loop the weights and the first two tiles are
  // waited for together (the compiler's own wait for the weights, which
  // follows the untracked tile loads, would drain them anyway). In pass `it`: tile it + 1
  // has landed once what was issued after its loads is all that may be
  // pending: the loads of tiles it + 2 .. it + S - 1 and, since every wave
  // stores its rows of each finished tile (kStores instructions a pass), the
  // stores of the min(it, S - 1) passes since. Vector-memory instructions
  // complete in issue order, loads and stores alike. When a later tile was
  // not issued (the end of the range), wait for everything.
  constexpr int kStores = 2 * kC * kTile * 2 / 1024 / (kThreads / 64);  // a wave's 32 rows of 64 pairs, 1 KiB a store
  auto wait_next = [&](int it, bool later_issued) {
    if (!later_issued) wait_vmcnt<0>();
    else if (wave == 0) wait_vmcnt_by<(S - 2) * (Lay::LPW + 1), kStores, S - 1>(it);
    else wait_vmcnt_by<(S - 2) * Lay::LPW, kStores, S - 1>(it);
  };
  // x_hat of the tile in `stage` into zn; the tile's mask into mdst (the
  // stage is refilled before the tile's epilogue runs).
  auto layer_norm_tile = [&](int stage, half_t* zn, float* mdst) {
    const unsigned char* st = smem + stage * Lay::STAGE;
#pragma unroll
    for (int pass = 0; pass < 2; pass++) {
      const int row = pass * 32 + (tid >> 4);
      const int c0 = (tid & 15) * 8;
      float x[8];
      read8<ZT>(st + row * Lay::ZROW + c0 * (int)sizeof(ZT), x);
      normalize16(x, a.eps, zn + row * kPitch + c0);
    }
    // Every wave copies the same 64 values (no branch, so this stays in the
    // straight-line block the MFMAs are scheduled with) and learns whether
    // they are all 1.
    const float mv = reinterpret_cast<const float*>(st + Lay::ZBYTES)[lane];
    mdst[lane] = mv;
    return __builtin_amdgcn_ballot_w64(mv == 1.0f) == ~0ull;
  };

  // A wave's stores: its 32 channel rows of the staged tile, store k
  // covering rows 8 k + lane / 8, 16-byte chunk lane % 8 (pairs 8 (lane % 8)
  // ..), so each instruction writes eight whole 128-byte row pieces. The
  // lane's offsets are fixed, the tile's base rides in the scalar offset.
  static_assert(kStores == 4, "32 rows, eight a store");
  const int srow = lane >> 3, schunk = lane & 7;
  const half_t* const sown = ost + (o * kC + hb + srow) * kOutPitch + schunk * 8;
  // The store resource covers the wave's own 32 channels.
  uint32_t svof[kStores];
#pragma unroll
  for (int k = 0; k < kStores; k++) svof[k] = (uint32_t)(((int64_t)(srow + 8 * k) * a.cstride + schunk * 8) * 2);
  const int obytes = (int)((int64_t)32 * a.cstride * 2);
  const __amdgpu_buffer_rsrc_t rso =
      __builtin_amdgcn_make_buffer_rsrc((o == 0 ? a.out_a : a.out_b) + (int64_t)hb * a.cstride, 0, obytes, 0x00020000);

  if (t0 >= ntiles) return;
  // The weights and the first two tiles load at once; the other stages are
  // filled once they have landed.
  static_assert(S >= 2, "two tiles in the first wait");
  if (wave < kLoaderWaves) {
    issue(t0, 0);
    if (t0 + G < ntiles) issue(t0 + G, 1);
  }
  wait_vmcnt<0>();
  if (wave < kLoaderWaves) {
#pragma unroll
    for (int s = 2; s < S; s++)
      if (t0 + s * G < ntiles) issue(t0 + s * G, s);
  }
  block_barrier();  // the first tile has landed
  bool ones = layer_norm_tile(0, zn_base, mask_base);

  // One pass; MASKED false (every mask value of the tile 1) leaves out the
  // multiplication by the mask, which would not change a bit.
  int it = 0, tile = t0;
  auto pass = [&](auto masked) -> bool {
    constexpr bool MASKED = decltype(masked)::value;
    bool ones_next;
    const half_t* zn = zn_base + (it & 1) * kTile * kPitch;
    const float* mk = mask_base + (it & 1) * kTile;
    half_t* orow = ost + (o * kC + ch) * kOutPitch;
    floatx16 accp[2], accg[2];
#pragma unroll
    for (int sub = 0; sub < 2; sub++)
#pragma unroll
      for (int v = 0; v < 16; v++) {
        accp[sub][v] = bp;
        accg[sub][v] = bg;
      }
    // Both sub-tiles' x_hat fragments are read first. The next tile's
    // LayerNorm writes the other x_hat buffer, and the compiler cannot tell
    // the buffers apart: reads issued after those writes waited for them,
    // which left sub-tile 1's MFMAs bunched behind their reads with no vector
    // work between them.
    half8 zf[2][8];
#pragma unroll
    for (int sub = 0; sub < 2; sub++) {
      const half_t* zrow = zn + (sub * 32 + (lane & 31)) * kPitch + 8 * (lane >> 5);
#pragma unroll
      for (int s = 0; s < 8; s++) zf[sub][s] = *reinterpret_cast<const half8*>(zrow + 16 * s);
    }
    auto mfma_sub = [&](int sub) {
#pragma unroll
      for (int s = 0; s < 8; s++) {
        accp[sub] = mfma_f16(zf[sub][s], fp[s], accp[sub]);
        accg[sub] = mfma_f16(zf[sub][s], fg[s], accg[sub]);
      }
    };
    auto epilogue_sub = [&](int sub) {
#pragma unroll
      for (int g4 = 0; g4 < 4; g4++) {
        // rows 4 g4 .. 4 g4 + 3 of the accumulator: pairs p0 .. p0 + 3
        const int p0 = sub * 32 + 8 * g4 + 4 * (lane >> 5);
        half4 h;
        if constexpr (MASKED) {
          const floatx4 m4 = *reinterpret_cast<const floatx4*>(mk + p0);
#pragma unroll
          for (int e = 0; e < 4; e++)
            h[e] = (half_t)(m4[e] * accp[sub][4 * g4 + e] * gate_of(accg[sub][4 * g4 + e]));
        } else {
#pragma unroll
          for (int e = 0; e < 4; e++) h[e] = (half_t)(accp[sub][4 * g4 + e] * gate_of(accg[sub][4 * g4 + e]));
        }
        *reinterpret_cast<half4*>(orow + p0) = h;
      }
    };
    // Sub-tile 0's MFMAs beside the next tile's LayerNorm (a tile past the
    // end normalises whatever the stage holds, into a buffer nobody reads),
    // sub-tile 1's beside sub-tile 0's gates; the scheduling groups below ask
    // the compiler to interleave each MFMA with vector work instead of
    // issuing them back to back.
    mfma_sub(0);
    ones_next =
        layer_norm_tile((it + 1) % S, zn_base + ((it + 1) & 1) * kTile * kPitch, mask_base + ((it + 1) & 1) * kTile);
    mfma_sub(1);
    epilogue_sub(0);
    epilogue_sub(1);
#pragma unroll
    for (int i = 0; i < 32; i++) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
      __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);  // then six VALU (four and nine measured 2-3% slower)
    }
    // The wave's own rows go out as soon as it has written them (LDS
    // accesses of one wave complete in order), so no barrier waits for the
    // whole staged tile; the next pass's barrier covers zn[(it + 1) % 2].
    // Pairs past P land in the operand's padding (its rows are cstride >=
    // 64 * ntiles long), which the contraction never reads.
    {
      u32x4 v[kStores];
#pragma unroll
      for (int k = 0; k < kStores; k++) v[k] = *reinterpret_cast<const u32x4*>(sown + 8 * k * kOutPitch);
#pragma unroll
      for (int k = 0; k < kStores; k++)
        __builtin_amdgcn_raw_buffer_store_b128(v[k], rso, svof[k], (uint32_t)tile * kTile * 2, 0);
      stores_read(v[0], v[1], v[2], v[3]);
    }
    return ones_next;
  };
  for (; tile < ntiles; it++, tile += G) {
    // Tiles it + 2 .. it + S - 1 may still be in flight; tile it + 1 must be in.
    if (wave < kLoaderWaves) wait_next(it, tile + (S - 1) * G < ntiles);
    block_barrier();  // zn[it % 2] complete, the next tile landed
    if (wave < kLoaderWaves && tile + S * G < ntiles) issue(tile + S * G, it % S);
    ones = ones ? pass(std::false_type{}) : pass(std::true_type{});
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
  static constexpr int OROW = kC * (int)sizeof(OT);  // bytes of one output row
  // The output tile is staged in a buffer of its own and written out while
  // the next tile is normalised; rows padded by 16 bytes so the 32 pair rows
  // one store instruction covers fall in different bank groups.
  static constexpr int OPITCH = OROW + 16;
  // The normalised hidden tile (hn) lives in the tile's own stage, dead once
  // its statistics and z's x_hat are taken.
  static_assert(kTile * kPitch * 2 <= STAGE, "hn fits its stage");
  static constexpr int GN = STAGES * STAGE;
  static constexpr int PART = GN + kTile * kPitch * 2;   // [8 waves][64 pairs] x (mean, m2)
  static constexpr int OUT = PART + 8 * kTile * 2 * 4;
  static constexpr int BYTES = OUT + kTile * OPITCH;
};
static_assert(OutputLayout<half_t, float>::BYTES <= 160 * 1024 && OutputLayout<float, float>::BYTES <= 160 * 1024,
              "LDS budget");

template <typename ZT, typename OT>
__global__ __launch_bounds__(kThreads, 1) void tri_output_f16_kernel(FastOutputArgs a, int ntiles) {
  using Lay = OutputLayout<ZT, OT>;
  extern __shared__ __attribute__((aligned(1024))) unsigned char smem[];
  half_t* gn = reinterpret_cast<half_t*>(smem + Lay::GN);
  float2* part = reinterpret_cast<float2*>(smem + Lay::PART);
  unsigned char* const ob = smem + Lay::OUT;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nt = 32 * (wave & 3), rh = 32 * (wave >> 2);
  const int G = gridDim.x;

  // Weight fragments (the A operand): W[n][k] with n = nt + lane % 32; the
  // biases of this lane's accumulator rows n = nt + mfma_row(v).
  half8 fz[8], fg[8];
#pragma unroll
  for (int s = 0; s < 8; s++) {
    fz[s] = fold_fragment(a.w_z, wave & 3, s, lane);
    fg[s] = fold_fragment(a.w_g, wave & 3, s, lane);
  }
  // Rows mfma_row(v, lane) come in runs of four: 8 (v / 4) + 4 (lane / 32) ..
  float bzv[16], bgv[16];
#pragma unroll
  for (int g4 = 0; g4 < 4; g4++) {
    const floatx4 z4 = *reinterpret_cast<const floatx4*>(a.b_z + nt + 8 * g4 + 4 * (lane >> 5));
    const floatx4 q4 = *reinterpret_cast<const floatx4*>(a.b_g + nt + 8 * g4 + 4 * (lane >> 5));
#pragma unroll
    for (int e = 0; e < 4; e++) {
      bzv[4 * g4 + e] = z4[e];
      bgv[4 * g4 + e] = q4[e];
    }
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

  // Waves 4-7 write a staged output tile: 64 pair rows of OROW bytes in
  // 16-byte chunks, straight to [pair][128], the residual added when asked.
  auto store_tile = [&](int t) {
    constexpr int CHUNKS = Lay::OROW / 16;
    constexpr int PER_LANE = kTile * CHUNKS / 256;
    const int t4 = tid - kLoaderWaves * 64;
    const int q0 = t * kTile;
    static_assert(PER_LANE % 4 == 0, "stores go in groups of four");
#pragma unroll
    for (int k0 = 0; k0 < PER_LANE; k0 += 4) {
      u32x4 v[4];
#pragma unroll
      for (int k = 0; k < 4; k++) {
        const int idx = t4 + 256 * (k0 + k);
        const int q = idx / CHUNKS, chunk = idx % CHUNKS;
        v[k] = *reinterpret_cast<const u32x4*>(ob + q * Lay::OPITCH + chunk * 16);
        unsigned char* dst =
            reinterpret_cast<unsigned char*>(a.out) + ((size_t)a.pair0 + q0 + q) * Lay::OROW + chunk * 16;
        if (q0 + q >= a.pairs) continue;
        if (a.residual) {
          const u32x4 r = *reinterpret_cast<const u32x4*>(dst);
          constexpr int E = 16 / (int)sizeof(OT);
          OT* vv = reinterpret_cast<OT*>(&v[k]);
          const OT* rr = reinterpret_cast<const OT*>(&r);
#pragma unroll
          for (int e = 0; e < E; e++) vv[e] = (OT)((float)vv[e] + (float)rr[e]);
        }
        *reinterpret_cast<u32x4*>(dst) = v[k];
      }
      stores_read(v[0], v[1], v[2], v[3]);
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
    block_barrier();  // B1: stage `it` complete; the previous tile is staged
    if (wave < kLoaderWaves) {
      if (tile + (Lay::STAGES - 1) * G < ntiles)
        issue(tile + (Lay::STAGES - 1) * G, (it + Lay::STAGES - 1) % Lay::STAGES);
    } else if (it > 0) {
      store_tile(tile - G);  // the staging is read out before B3 and rewritten after it
    }

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
    // z's x_hat, rows of 16 lanes.
#pragma unroll
    for (int pass = 0; pass < 2; pass++) {
      const int row = pass * 32 + (tid >> 4);
      const int c0 = (tid & 15) * 8;
      float x[8];
      read8<ZT>(st + Lay::XBYTES + row * Lay::ZROW + c0 * (int)sizeof(ZT), x);
      normalize16(x, a.eps, gn + row * kPitch + c0);
    }
    block_barrier();  // B2: partial statistics and gn complete; the stage is dead
    half_t* const hn = reinterpret_cast<half_t*>(st);
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
      const float shift = -mean * rstd;
      half8 h0, h1;
#pragma unroll
      for (int e = 0; e < 8; e++) {
        h0[e] = (half_t)fmaf(xh[e], rstd, shift);
        h1[e] = (half_t)fmaf(xh[e + 8], rstd, shift);
      }
      half_t* dst = hn + lane * kPitch + 16 * wave;
      reinterpret_cast<half8*>(dst)[0] = h0;
      reinterpret_cast<half8*>(dst)[1] = h1;
    }
    block_barrier();  // B3: hn complete; the staging has been read out

    // W (A operand) x x_hat^T (B operand): the accumulator's column is the
    // pair rh + lane % 32 and its rows come in runs of four consecutive
    // output channels, staged as one 4-element write each.
    floatx16 accz, accg;
#pragma unroll
    for (int v = 0; v < 16; v++) {
      accz[v] = bzv[v];
      accg[v] = bgv[v];
    }
    const half_t* hrow = hn + (rh + (lane & 31)) * kPitch + 8 * (lane >> 5);
    const half_t* grow = gn + (rh + (lane & 31)) * kPitch + 8 * (lane >> 5);
#pragma unroll
    for (int s = 0; s < 8; s++) {
      accz = mfma_f16(fz[s], *reinterpret_cast<const half8*>(hrow + 16 * s), accz);
      accg = mfma_f16(fg[s], *reinterpret_cast<const half8*>(grow + 16 * s), accg);
    }
    {
      unsigned char* orow = ob + (rh + (lane & 31)) * Lay::OPITCH;
#pragma unroll
      for (int g4 = 0; g4 < 4; g4++) {
        const int n0 = nt + 8 * g4 + 4 * (lane >> 5);
        OT y[4];
#pragma unroll
        for (int e = 0; e < 4; e++) y[e] = (OT)(accz[4 * g4 + e] * gate_of(accg[4 * g4 + e]));
        if constexpr (sizeof(OT) == 4) {
          *reinterpret_cast<floatx4*>(orow + n0 * 4) = floatx4{(float)y[0], (float)y[1], (float)y[2], (float)y[3]};
        } else {
          half4 h;
#pragma unroll
          for (int e = 0; e < 4; e++) h[e] = (half_t)y[e];
          *reinterpret_cast<half4*>(orow + n0 * 2) = h;
        }
      }
    }
  }
  block_barrier();  // the last tile is staged
  if (wave >= kLoaderWaves) store_tile(tile - G);
}

// ---------------------------------------------------------------------------
// Output, software-pipelined (f16 z)
// ---------------------------------------------------------------------------
//
// The same arithmetic as tri_output_f16_kernel in the same order, so the
// results are bit-identical, but tile t's hidden statistics and z LayerNorm
// run in one straight-line block with tile t-1's MFMAs and gate epilogue, so
// the matrix and vector pipes overlap (the sequential kernel spent ~6.4k
// cycles a tile, its phases one after another behind three barriers). The
// normalised tiles (hn, gn) are double-buffered, which the LDS budget allows
// only by giving up the output staging: each wave stores its accumulator
// rows itself (four consecutive channels a lane, 16 bytes in f32), through a
// buffer resource over [pair0, pair0 + pairs) so ragged pairs are dropped and
// every wave issues the same number of vector-memory instructions, which
// keeps the loader waves' vmcnt waits exact. Two barriers a tile:
//   B1: tile t's stage has landed; hn[t-1] (and gn[t-1]) complete.
//   B2: tile t's partial statistics and gn[t] complete; stage t is dead.
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));

struct PipeLayout {
  static constexpr int ZROW = kC * 2;
  static constexpr int XBYTES = kC * kTile * 2;  // contraction tile, [128 channels][64 pairs] f16
  static constexpr int ZBYTES = kTile * ZROW;
  static constexpr int STAGE = XBYTES + ZBYTES;
  static constexpr int STAGES = 2;
  static constexpr int XLOADS = XBYTES / 1024;
  static constexpr int ZLOADS = ZBYTES / 1024;
  static constexpr int LPW = (XLOADS + ZLOADS) / kLoaderWaves;
  static constexpr int ZROWS_PER_LOAD = 1024 / ZROW;
  static constexpr int ZLANES_PER_ROW = 64 / ZROWS_PER_LOAD;
  static constexpr int NBUF = kTile * kPitch * 2;  // one normalised tile
  static constexpr int GN = STAGES * STAGE;         // two z x_hat tiles
  static constexpr int HN = GN + 2 * NBUF;          // two hidden x_hat tiles
  static constexpr int PART = HN + 2 * NBUF;        // [8 waves][64 pairs] x (mean, m2)
  static constexpr int BYTES = PART + 8 * kTile * 2 * 4;
};
static_assert(PipeLayout::BYTES <= 160 * 1024, "LDS budget");

template <typename OT>
__global__ __launch_bounds__(kThreads, 1) void tri_output_pipe_kernel(FastOutputArgs a, int ntiles) {
  using Lay = PipeLayout;
  extern __shared__ __attribute__((aligned(1024))) unsigned char smem[];
  float2* part = reinterpret_cast<float2*>(smem + Lay::PART);

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nt = 32 * (wave & 3), rh = 32 * (wave >> 2);
  const int G = gridDim.x;

  half8 fz[8], fg[8];
#pragma unroll
  for (int s = 0; s < 8; s++) {
    fz[s] = fold_fragment(a.w_z, wave & 3, s, lane);
    fg[s] = fold_fragment(a.w_g, wave & 3, s, lane);
  }
  // Rows mfma_row(v, lane) come in runs of four: 8 (v / 4) + 4 (lane / 32) ..
  float bzv[16], bgv[16];
#pragma unroll
  for (int g4 = 0; g4 < 4; g4++) {
    const floatx4 z4 = *reinterpret_cast<const floatx4*>(a.b_z + nt + 8 * g4 + 4 * (lane >> 5));
    const floatx4 q4 = *reinterpret_cast<const floatx4*>(a.b_g + nt + 8 * g4 + 4 * (lane >> 5));
#pragma unroll
    for (int e = 0; e < 4; e++) {
      bzv[4 * g4 + e] = z4[e];
      bgv[4 * g4 + e] = q4[e];
    }
  }
  // The weights are waited for together with the first tile, below.

  const int32x4_t rx = make_rsrc(a.contracted, (uint32_t)((int64_t)kC * a.bstride * 2));
  const int32x4_t rz = make_rsrc(reinterpret_cast<const unsigned char*>(a.z) + (size_t)a.pair0 * Lay::ZROW,
                                 (uint32_t)((int64_t)a.pairs * Lay::ZROW));
  constexpr int OROW = kC * (int)sizeof(OT);
  const __amdgpu_buffer_rsrc_t ro = __builtin_amdgcn_make_buffer_rsrc(
      reinterpret_cast<unsigned char*>(a.out) + (size_t)a.pair0 * OROW, 0, (int)((int64_t)a.pairs * OROW), 0x00020000);
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

  // Tile t's partial hidden statistics (wave w holds channels [16 w, +16)
  // of pair `lane`) and z's x_hat into gn[buf].
  float xh[16];
  auto stats_and_zln = [&](int stage, int buf) {
    const unsigned char* st = smem + stage * Lay::STAGE;
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
    half_t* gn = reinterpret_cast<half_t*>(smem + Lay::GN + buf * Lay::NBUF);
#pragma unroll
    for (int pass = 0; pass < 2; pass++) {
      const int row = pass * 32 + (tid >> 4);
      const int c0 = (tid & 15) * 8;
      float x[8];
      read8<half_t>(st + Lay::XBYTES + row * Lay::ZROW + c0 * 2, x);
      normalize16(x, a.eps, gn + row * kPitch + c0);
    }
  };
  // Chan et al.: merge eight (mean, M2) over 16 channels each; x_hat of the
  // wave's 16 channels of pair `lane` into hn[buf].
  auto merge = [&](int buf) {
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
    const float shift = -mean * rstd;
    half8 h0, h1;
#pragma unroll
    for (int e = 0; e < 8; e++) {
      h0[e] = (half_t)fmaf(xh[e], rstd, shift);
      h1[e] = (half_t)fmaf(xh[e + 8], rstd, shift);
    }
    half_t* dst = reinterpret_cast<half_t*>(smem + Lay::HN + buf * Lay::NBUF) + lane * kPitch + 16 * wave;
    reinterpret_cast<half8*>(dst)[0] = h0;
    reinterpret_cast<half8*>(dst)[1] = h1;
  };
  // W (A operand) x x_hat^T (B operand) for tile `t` from buffers `buf`: the
  // accumulator's column is the pair rh + lane % 32, its rows four
  // consecutive output channels per group; out = p sigmoid(g) (+ the old
  // value, read first). Stores past the tile's valid pairs fall outside the
  // resource and are dropped.
  auto project_store = [&](int t, int buf, bool residual) {
    // The product, its rounding to OT and the residual add each round on
    // their own (no fused multiply-add, no mixed-precision fused forms): f32
    // outputs equal the staged kernel's bit for bit, and f16 outputs round
    // the f32 product (the staged kernel let the compiler fuse that
    // conversion, one ulp apart at most).
#pragma clang fp contract(off)
    const uint32_t orow = (uint32_t)(t * kTile + rh + (lane & 31)) * OROW;
    typedef OT ot4 __attribute__((ext_vector_type(4)));
    ot4 old[4];
    if (residual) {
#pragma unroll
      for (int g4 = 0; g4 < 4; g4++) {
        const uint32_t off = orow + (uint32_t)(nt + 8 * g4 + 4 * (lane >> 5)) * (uint32_t)sizeof(OT);
        if constexpr (sizeof(OT) == 4)
          old[g4] = __builtin_bit_cast(ot4, __builtin_amdgcn_raw_buffer_load_b128(ro, off, 0, 0));
        else
          old[g4] = __builtin_bit_cast(ot4, __builtin_amdgcn_raw_buffer_load_b64(ro, off, 0, 0));
      }
    }
    floatx16 accz, accg;
#pragma unroll
    for (int v = 0; v < 16; v++) {
      accz[v] = bzv[v];
      accg[v] = bgv[v];
    }
    const half_t* hrow =
        reinterpret_cast<const half_t*>(smem + Lay::HN + buf * Lay::NBUF) + (rh + (lane & 31)) * kPitch + 8 * (lane >> 5);
    const half_t* grow =
        reinterpret_cast<const half_t*>(smem + Lay::GN + buf * Lay::NBUF) + (rh + (lane & 31)) * kPitch + 8 * (lane >> 5);
#pragma unroll
    for (int s = 0; s < 8; s++) {
      accz = mfma_f16(fz[s], *reinterpret_cast<const half8*>(hrow + 16 * s), accz);
      accg = mfma_f16(fg[s], *reinterpret_cast<const half8*>(grow + 16 * s), accg);
    }
#pragma unroll
    for (int g4 = 0; g4 < 4; g4++) {
      const uint32_t off = orow + (uint32_t)(nt + 8 * g4 + 4 * (lane >> 5)) * (uint32_t)sizeof(OT);
      ot4 y;
#pragma unroll
      for (int e = 0; e < 4; e++) {
        y[e] = (OT)(accz[4 * g4 + e] * gate_of(accg[4 * g4 + e]));
        if (residual) y[e] = (OT)((float)y[e] + (float)old[g4][e]);
      }
      if constexpr (sizeof(OT) == 4)
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, y), ro, off, 0, 0);
      else
        __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, y), ro, off, 0, 0);
    }
  };
  const bool residual = a.residual != 0;
  // A loader's tile has landed once at most the vector-memory instructions
  // it issued after that tile's loads are outstanding: the previous tile's
  // residual reads and stores (four each), or none on the first pass.
  auto wait_tile = [&](bool after_stores) {
    if (!after_stores) wait_vmcnt<0>();
    else if (residual) wait_vmcnt<8>();
    else wait_vmcnt<4>();
  };

  const int t0 = blockIdx.x;
  if (t0 >= ntiles) return;
  if (wave < kLoaderWaves) issue(t0, 0);
  // First tile: statistics only. Every wave's weights have landed too.
  wait_vmcnt<0>();
  block_barrier();  // B1
  if (wave < kLoaderWaves && t0 + G < ntiles) issue(t0 + G, 1);
  stats_and_zln(0, 0);
  block_barrier();  // B2
  merge(0);
  int it = 1;
  for (int tile = t0 + G; tile < ntiles; it++, tile += G) {
    const int buf = it & 1;
    if (wave < kLoaderWaves) wait_tile(it > 1);
    block_barrier();  // B1: stage `buf` landed, hn[buf ^ 1] complete
    if (wave < kLoaderWaves && tile + G < ntiles) issue(tile + G, buf ^ 1);
    // Tile it-1's MFMAs and epilogue beside tile it's statistics: one block.
    project_store(tile - G, buf ^ 1, residual);
    stats_and_zln(buf, buf);
    // One MFMA, then fourteen VALU (the block's ~180 vector instructions
    // spread over its 16 MFMAs). Measured at L = 384: 33.4 us against 33.8
    // for twelve, 34.3 for eighteen, 34.6 for six and 34.8 with no hint.
#pragma unroll
    for (int i = 0; i < 16; i++) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, 14, 0);
    }
    block_barrier();  // B2: partial statistics and gn[buf] complete; stage buf is dead
    merge(buf);
  }
  block_barrier();  // hn of the last tile complete
  project_store(t0 + (it - 1) * G, (it - 1) & 1, residual);
}

int grid_for(int tiles) {
  const int cus = device_cu_count() > 0 ? device_cu_count() : 256;
  return std::max(1, std::min(tiles, cus));
}

template <typename K> int prepare_lds(K kernel, int bytes) { return allow_lds((const void*)kernel, (size_t)bytes); }

}  // namespace

bool triangle_fast_eligible(const afhip_triangle_desc& d) {
  if (d.precision != AFHIP_PRECISION_F16 || d.c_z != kC || d.c_hidden != kC) return false;
  const int64_t P = (int64_t)d.length * d.length;
  // The incoming projection reads z transposed, each lane at its own 32-bit
  // byte offset into all of z; every other access is rebased per tile, per
  // wave or per block of output rows. Operand channels of 32 stay below 2 GiB.
  const int64_t zrow = (int64_t)kC * (d.pair_dtype == AFHIP_F32 ? 4 : 2);
  if (d.direction == AFHIP_TRIANGLE_INCOMING && P * zrow > (int64_t)UINT32_MAX) return false;
  return P <= ((int64_t)1 << 26) && 32 * (P + 64) * 2 < ((int64_t)1 << 31);
}

int triangle_fast_block_rows(const afhip_triangle_desc& d) {
  // Per block of B rows (B L pairs): z and the output take B L rows of
  // 128 channels, the contracted values 128 channels of round_up(B L, 64).
  const int64_t widest = std::max<int64_t>(d.pair_dtype == AFHIP_F32 ? 4 : 2, d.out_dtype == AFHIP_F32 ? 4 : 2);
  const int64_t pairs = (((int64_t)1 << 31) - 1) / (kC * widest) - 64;
  const int64_t most = std::max<int64_t>(1, std::min<int64_t>(d.length, pairs / d.length));
  // As many blocks as that takes, of equal size (no short last block).
  const int64_t blocks = ceil_div(d.length, most);
  return (int)ceil_div(d.length, blocks);
}

template <typename ZT, bool INCOMING> int launch_project(const FastProjectArgs& a, hipStream_t s) {
  const int tiles = (int)ceil_div(a.P, kTile);
  auto k = tri_project_f16_kernel<ZT, INCOMING>;
  if (int st = prepare_lds(k, ProjectLayout<ZT>::BYTES)) return st;
  return launch("triangle.project", k, dim3(grid_for(tiles)), dim3(kThreads), ProjectLayout<ZT>::BYTES, s, a, tiles);
}

int launch_triangle_project_f16(const FastProjectArgs& a, int pair_dtype, hipStream_t s) {
  // Buffer offsets are 32-bit: the operands' 128 rows and z must stay below 2 GiB.
  const int64_t zrow = (int64_t)kC * (pair_dtype == AFHIP_F32 ? 4 : 2);
  AFHIP_REQUIRE((int64_t)32 * a.cstride * 2 < ((int64_t)1 << 31) && (!a.incoming || (int64_t)a.P * zrow <= UINT32_MAX),
                "triangle of %d pairs exceeds the projection kernel's buffer offsets", a.P);
  if (pair_dtype == AFHIP_F16)
    return a.incoming ? launch_project<half_t, true>(a, s) : launch_project<half_t, false>(a, s);
  return a.incoming ? launch_project<float, true>(a, s) : launch_project<float, false>(a, s);
}

template <typename ZT, typename OT> int launch_output(const FastOutputArgs& a, hipStream_t s) {
  const int tiles = (int)ceil_div(a.pairs, kTile);
  if constexpr (sizeof(ZT) == 2) {  // the pipelined kernel (its double buffers fit with f16 z)
    AFHIP_REQUIRE((int64_t)a.pairs * kC * (int64_t)sizeof(OT) < ((int64_t)1 << 31),
                  "triangle of %d pairs exceeds the output kernel's 2 GiB bound", a.pairs);
    auto k = tri_output_pipe_kernel<OT>;
    constexpr int bytes = PipeLayout::BYTES;
    if (int st = prepare_lds(k, bytes)) return st;
    return launch("triangle.output", k, dim3(grid_for(tiles)), dim3(kThreads), bytes, s, a, tiles);
  }
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
