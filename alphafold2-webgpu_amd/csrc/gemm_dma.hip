// The LDS_DMA GEMM kernel family for gfx950: C[b] = epilogue(A[b] B[b]^T)
// with A [M][K] and B [N][K] f16 (k-contiguous), f32 accumulation. Three
// template variants widen the operand forms: a row-contiguous A [K][M]
// (AK: k rows in LDS, transposing fragment reads), an f32 A under f16
// arithmetic (AF: f32 rows in LDS, rounded to f16 as fragments are read) and
// f32 arithmetic on f32 operands (FP32: f32 rows, the f32 MFMA).
//
// It carries the triangle multiplication's O(L^3) contraction (per hidden
// channel b, out[b][i][j] = sum_k R[b][i][k] C[b][j][k]; the reference
// dispatches it once per channel along z, src/triangle/shaders.ts:452-496),
// the outer-product-mean contraction and the f16 projections.
//
// Design:
//  - One workgroup of WM x WN wave64s owns a BM x BN output tile (each wave
//    (BM/WM) x (BN/WN) in 32 x 32 v_mfma_f32_32x32x16_f16 tiles) and walks
//    K in steps of 32 halves: 2 x 2 waves for the 128- and 192-row tiles, two
//    of which share a CU; 2 x 4 waves, one workgroup a CU, for 256 x 256.
//  - Operands travel global -> LDS without passing through VGPRs
//    (buffer_load_dwordx4 ... lds). A k-step stage is (BM + BN) rows of
//    64 bytes; each wave-level load instruction fills 16 rows (1 KiB of LDS,
//    lane l -> row l/4, 16-byte slot l%4). Rows that are only 4-byte aligned
//    (K or a leading dimension not a multiple of 8 halves) load with
//    buffer_load_dword ... lds instead: 4 rows an instruction, 16 lanes a row,
//    into the same stage layout. STAGES stages are in flight, so the
//    loads for step k + STAGES - 1 are issued while step k computes, and one
//    barrier per k-step both publishes a stage and retires the one to refill.
//  - Bank conflicts: a row's four 16-byte chunks are stored XOR-swizzled,
//    slot = chunk ^ ((row >> 2) & 3), so the 16 rows a 16-lane group of an
//    MFMA fragment read cover all 16 bank groups of a 256-byte line. The
//    swizzle is applied by choosing which global chunk each lane loads.
//  - Ragged edges cost nothing: every load goes through a buffer resource
//    bounded to the tile's valid rows, and chunks past K get an offset beyond
//    the resource, so the hardware returns zeros for both.
//  - Tiles are numbered so that consecutive tiles (one batch's tiles, which
//    share operand panels) run on one XCD: workgroup ids are dealt round-robin
//    over the eight XCDs, so tile t = (id % 8) * per_xcd + id / 8.
//  - The 256 x 256 tile runs a pipelined schedule: each k-step's two
//    16-deep halves are read into separate fragment registers, and the
//    barrier that publishes stage k + 1 sits between the MFMAs of the first
//    half and those of the second, so a wave waits at the barrier while its
//    MFMAs still run and starts the next step with operands already in
//    registers. Five stages keep the loads three steps ahead.
//  - The epilogue is the register-staged kernel's (gemm_kernel.h), so both
//    families give the same epilogue arithmetic.
#include <algorithm>
#include <type_traits>

#include "dma.h"
#include "gemm_kernel.h"

namespace afhip {

namespace {

constexpr int kBK = 32;        // halves per k-step
constexpr int kRowBytes = 64;  // one row of a k-step stage
// Tiles of one batch entry are visited in runs of kTileGroup tile rows,
// column by column within a run, so the tiles resident at once on an XCD
// (consecutive indices) form a block that shares few A and B panels: on the
// outer-product mean's 32 x 32 tiles of 256, an XCD's 32 concurrent tiles
// read 8 A and 4 B panels (3 MiB, within its 4 MiB L2) instead of 1 A and
// 32 B panels (8.25 MiB). Measured there: 109.5 us against 114.4 us.
constexpr int kTileGroup = 8;

__device__ __forceinline__ int swizzle(int row) { return (row >> 2) & 3; }
// The slot of a 128-byte f32 A row's 16-byte chunk: chunk ^ swizzle_f32(row)
// puts the rows of 8 (and of 16) consecutive lanes on distinct banks.
__device__ __forceinline__ int swizzle_f32(int row) { return ((row >> 1) & 7) ^ ((row & 1) << 2); }

// Bytes of one k-step stage: A's part (BM rows of 32 k, 4-byte elements for
// an f32 A) then B's (BN rows of 32 k, likewise).
constexpr int dma_stage_bytes(int bm, int bn, bool a_f32, bool b_f32 = false) {
  return bm * (a_f32 ? 2 * kRowBytes : kRowBytes) + bn * (b_f32 ? 2 * kRowBytes : kRowBytes);
}

typedef short short4v __attribute__((ext_vector_type(4)));
typedef short short8v __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) short4v lds_short4v;
typedef float f32x4v __attribute__((ext_vector_type(4)));
typedef float f32x8v __attribute__((ext_vector_type(8)));

// Epilogue families: GENERIC applies g.flags; OPM_FUSED is the outer-product
// mean's output projection run on the finished contraction tile.
constexpr int kEpiGeneric = 0;
constexpr int kEpiOpmFused = 1;

template <int BM, int BN, int STAGES, int WM, int WN, bool PIPE, typename TC, int EPI = kEpiGeneric, int LW = 16,
          bool AK = false, bool AF = false, bool FP32 = false>
__global__ __launch_bounds__(64 * WM * WN, WM * WN == 4 ? 2 : 1) void gemm_dma_kernel(gemm_detail::KernelArgs ka) {
  constexpr int WAVES = WM * WN;
  constexpr int kThreads = 64 * WAVES;
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int TM = WTM / 32, TN = WTN / 32;
  static_assert(LW == 16 || LW == 4, "16- or 4-byte loads");
  // An f32 A (f16 arithmetic) keeps 128-byte rows of 32 k in its part of a
  // stage and is rounded to f16 as the fragments are read.
  // f32 arithmetic (FP32): A and B both f32 in 128-byte rows, on the f32
  // MFMA (32 x 32 x 2), with the register-staged kernel's k pairing.
  static_assert(!AF || (LW == 16 && !AK && EPI == kEpiGeneric), "f32 A tiles");
  static_assert(!FP32 || (LW == 16 && !AK && !AF && EPI == kEpiGeneric), "f32 tiles");
  constexpr bool A4 = AF || FP32;  // A rows of 4-byte elements
  constexpr int AROW = A4 ? 2 * kRowBytes : kRowBytes;    // bytes of a k-contiguous A row
  constexpr int BROW = FP32 ? 2 * kRowBytes : kRowBytes;  // and of a B row
  constexpr int A_BYTES = BM * AROW;
  constexpr int STAGE_BYTES = dma_stage_bytes(BM, BN, A4, FP32);
  constexpr int RPL = LW;                     // stage rows of 64 bytes a wave-level load fills
  constexpr int LPR = 64 / LW;                // lanes a row
  constexpr int A_LOADS = A_BYTES / (64 * LW);  // wave-level load instructions per stage: A's
  constexpr int LOADS = (STAGE_BYTES) / (64 * LW);  // and all
  constexpr int LPW = LOADS / WAVES;          // per wave
  static_assert(WTM % 32 == 0 && WTN % 32 == 0 && LOADS % WAVES == 0, "tile shape");
  static_assert(BM % RPL == 0 && A_BYTES % (64 * LW) == 0, "a load instruction fills rows of one operand");
  static_assert((STAGES - 2) * LPW < 64, "vmcnt holds at most 63 outstanding loads");
  static_assert(!PIPE || STAGES >= 4, "the pipelined schedule keeps STAGES - 2 steps in flight");
  // A k-major A ([K][M], a row-contiguous source) keeps the stage's A part as
  // 32 k rows of BM halves: an A load instruction fills KRPL whole k rows.
  static_assert(!AK || (LW == 16 && (BM == 128 || BM == 256) && EPI == kEpiGeneric), "k-major A tiles");
  constexpr int AROWB = BM * 2;          // bytes of a k row of a k-major A stage
  constexpr int KRPL = 1024 / AROWB;     // k rows an A load instruction fills
  constexpr int CPK = BM / 8;            // 16-byte chunks of such a k row
  extern __shared__ __attribute__((aligned(1024))) unsigned char smem[];

  const GemmArgs& g = ka.g;
  const int id = blockIdx.x;
  const int t = (id & 7) * ka.per_xcd + (id >> 3);
  if (t >= ka.total_tiles) return;
  const int per_batch = ka.tiles_m * ka.tiles_n;
  const int bt = t / per_batch;
  const int rt = t - bt * per_batch;
  const int run = rt / (kTileGroup * ka.tiles_n);
  const int run_rows = min(ka.tiles_m - run * kTileGroup, kTileGroup);
  const int in_run = rt - run * kTileGroup * ka.tiles_n;
  const int m0 = (run * kTileGroup + in_run % run_rows) * BM;
  const int n0 = (in_run / run_rows) * BN;

  const int lane = threadIdx.x & 63;
  // Wave-uniform by construction; readfirstlane lets the compiler keep the
  // buffer resource choice below in scalar registers.
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = (wave / WN) * WTM;
  const int wn = (wave % WN) * WTN;

  using TA = typename std::conditional<A4, float, half_t>::type;
  using TB = typename std::conditional<FP32, float, half_t>::type;
  // A lane's MFMA operand for one 32-row block and half-step: 8 k.
  using Frag = typename std::conditional<FP32, f32x8v, half8>::type;
  const TA* A = reinterpret_cast<const TA*>(g.a) + (int64_t)bt * g.sa + (AK ? (int64_t)m0 : (int64_t)m0 * g.lda);
  const TB* B = reinterpret_cast<const TB*>(g.b) + (int64_t)bt * g.sb + (int64_t)n0 * g.ldb;
  const int rows_a = min(BM, g.M - m0);
  const int rows_b = min(BN, g.N - n0);
  // k-major: from column m0 of k row 0 to column M of k row K - 1. A k row's
  // columns past M (whole chunks: M % 8 == 0) read the next row's first
  // columns or zeros, which reach only output rows >= M.
  const int32x4_t ra = AK ? make_rsrc(A, (uint32_t)(((int64_t)(g.K - 1) * g.lda + g.M - m0) * 2))
                          : make_rsrc(A, (uint32_t)((int64_t)rows_a * g.lda * sizeof(TA)));
  const int32x4_t rb = make_rsrc(B, (uint32_t)((int64_t)rows_b * g.ldb * sizeof(TB)));

  // This lane's part of each of the wave's load instructions: instruction
  // q = wave + WAVES i fills stage bytes [64 LW q, 64 LW (q + 1)), A's rows
  // for q < A_LOADS, then B's. For 64-byte rows the lane fills bytes
  // [LW s, LW s + LW) of row RPL q + lane / LPR, s = lane % LPR, which lie in
  // 16-byte slot LW s / 16: it loads the same bytes of global chunk
  // slot ^ swizzle(row).
  uint32_t base_off[LPW];
  int chunk_k[LPW];  // the first k the lane's bytes hold
#pragma unroll
  for (int i = 0; i < LPW; i++) {
    const int q = wave + WAVES * i;
    if ((A4 && q < A_LOADS) || (FP32 && q >= A_LOADS)) {
      // 128-byte f32 rows: row 8 q' + lane / 8 of the operand (q' = q, or
      // q - A_LOADS for B), slot lane % 8, which holds the row's chunk (4 k)
      // slot ^ swizzle_f32(row).
      const bool is_a = q < A_LOADS;
      const int row = 8 * (is_a ? q : q - A_LOADS) + lane / 8;
      const int chunk = (lane % 8) ^ swizzle_f32(row);
      chunk_k[i] = 4 * chunk;
      base_off[i] = (uint32_t)((int64_t)row * (is_a ? g.lda : g.ldb) * 4 + 16 * chunk);
      continue;
    }
    if (AK && q < A_LOADS) {
      // k-major A: k row kr of the stage, 16-byte slot lane % CPK, which
      // holds chunk (columns m / 8) slot ^ 4 (kr mod 4), so that the four k
      // rows a transposing read spans sit in different banks.
      const int kr = KRPL * q + lane / CPK;
      chunk_k[i] = kr;
      base_off[i] = (uint32_t)((int64_t)kr * g.lda * 2 + 16 * ((lane % CPK) ^ (4 * (kr & 3))));
      continue;
    }
    const bool is_a = q < A_LOADS;
    const int row = RPL * (is_a ? q : q - A_LOADS) + lane / LPR;  // of the operand's tile
    const int byte = LW * (lane % LPR);
    const int chunk = (byte >> 4) ^ swizzle(row);
    const int inner = 16 * chunk + (byte & 15);
    chunk_k[i] = inner / 2;
    base_off[i] = (uint32_t)((int64_t)row * (is_a ? g.lda : g.ldb) * 2 + inner);
  }
  const uint32_t lds0 = (uint32_t)reinterpret_cast<uintptr_t>(smem);

  auto issue = [&](int ks, int stage) {
    const int k0 = ks * kBK;
#pragma unroll
    for (int i = 0; i < LPW; i++) {
      const int q = wave + WAVES * i;
      const bool is_a = q < A_LOADS;
      const uint32_t step = AK && is_a ? (uint32_t)k0 * (uint32_t)g.lda * 2u
                                       : ((A4 && is_a) || (FP32 && !is_a) ? 4u : 2u) * k0;
      const uint32_t off = k0 + chunk_k[i] < g.K ? base_off[i] + step : kOutOfRange;
      if constexpr (LW == 16) dma16(is_a ? ra : rb, lds0 + stage * STAGE_BYTES + q * 64 * LW, off);
      else dma4(is_a ? ra : rb, lds0 + stage * STAGE_BYTES + q * 64 * LW, off);
    }
  };

  floatx16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; i++)
#pragma unroll
    for (int j = 0; j < TN; j++)
#pragma unroll
      for (int v = 0; v < 16; v++) acc[i][j][v] = 0.0f;

  const int nk = (g.K + kBK - 1) / kBK;
#pragma unroll
  for (int s = 0; s < STAGES - 1; s++)
    if (s < nk) issue(s, s);

  // The fused outer-product-mean epilogue (EPI == kEpiOpmFused): the tile is
  // PI x PJ pairs (NPB blocks of 32); wave w computes output channels
  // 32 (w % 4) + [0, 32) over part w / 4 of the KP parts of the 1024 k, in
  // NG groups of 64. Its inputs that do not depend on the contraction load
  // while it runs: the reciprocal of (eps + count) for the wave's pairs, the
  // bias of its output channel and the first PRE groups of its weight
  // fragments. (Extra vector-memory loads only
  // make the waits on the stage loads stricter: loads complete in order.)
  constexpr int PI = BM / 32, PJ = BN / 32, NPAIR = PI * PJ, NPB = NPAIR / 32;
  constexpr int KP = WAVES / 4, NG = 16 / (KP > 0 ? KP : 1), PRE = 2, AHEAD = 6;
  float rcpv[TM][TN] = {};
  float bz = 0.0f;
  half8 wf[NG][4];
  const half_t* wrow = nullptr;
  if constexpr (EPI == kEpiOpmFused) {
    static_assert(NPAIR % 32 == 0 && WAVES % 4 == 0 && (KP == 1 || (KP == 2 && NPB == 2)),
                  "the fused epilogue's work split");
    const int L = g.opm_length, ib = m0 >> 5, jb = n0 >> 5;
    auto count_at = [&](int i, int j) { return i < L && j < L ? g.opm_count[(int64_t)i * L + j] : 0.0f; };
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
      for (int j = 0; j < TN; j++)
        rcpv[i][j] = 1.0f / (g.opm_eps + count_at(ib + (wm >> 5) + i, jb + (wn >> 5) + j));
    bz = g.bias[32 * (wave & 3) + (lane & 31)];
    // Fragment (Q, t) of output-channel block zb starts at half
    // ((zb * 16 + Q) * 4 + t) * 512; the wave's part starts at Q = (16 / KP) kh.
    wrow = reinterpret_cast<const half_t*>(g.opm_w) + ((wave & 3) * 16 + (16 / KP) * (wave >> 2)) * 2048 + 8 * lane;
#pragma unroll
    for (int q = 0; q < PRE; q++)
#pragma unroll
      for (int t = 0; t < 4; t++) wf[q][t] = *reinterpret_cast<const half8*>(wrow + 2048 * q + 512 * t);
  }

  const int frag_row = lane & 31;
  // Fragments of half kk (16 halves of k) of a stage: chunk 2 kk + lane / 32.
  auto read_frags = [&](const unsigned char* st, int kk, Frag* af, Frag* bf) {
    const int chunk = 2 * kk + (lane >> 5);
#pragma unroll
    for (int i = 0; i < TM; i++) {
      if constexpr (AK) {
        // Two transposing reads (ds_read_b64_tr_b16: in a 16-lane group, lane
        // x gets as element j element x % 4 of the 8 bytes lane 4 j + x / 4
        // addressed): lane 16 g + p addresses k row 16 kk + 8 hi + 4 r + p / 4
        // (hi = lane / 32)
        // at columns m = wm + 32 i + 16 (g % 2) + 4 (p % 4) .., so lane l ends
        // with k 16 kk + 8 hi + [0, 8) of row wm + 32 i + l % 32, the
        // fragment a k-contiguous A gives.
        const int p = lane & 15;
        const int m = wm + 32 * i + 16 * ((lane >> 4) & 1) + 4 * (p & 3);
        short4v part[2];
#pragma unroll
        for (int r = 0; r < 2; r++) {
          const int k = 16 * kk + 8 * (lane >> 5) + 4 * r + (p >> 2);
          part[r] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (lds_short4v*)(st + k * AROWB + 16 * ((m >> 3) ^ (4 * (k & 3))) + 2 * (m & 7)));
        }
        af[i] = __builtin_bit_cast(half8, short8v{part[0][0], part[0][1], part[0][2], part[0][3], part[1][0],
                                                  part[1][1], part[1][2], part[1][3]});
      } else if constexpr (A4) {
        // The lane's 8 k are f32 chunks 2 chunk and 2 chunk + 1 of its row;
        // under f16 arithmetic rounded to f16 (to nearest even, as the
        // register-staged kernels' loaders round).
        const int row = wm + 32 * i + frag_row;
        const unsigned char* rp = st + row * AROW;
        const int sw = swizzle_f32(row);
        const f32x4v lo = *reinterpret_cast<const f32x4v*>(rp + 16 * ((2 * chunk) ^ sw));
        const f32x4v hi = *reinterpret_cast<const f32x4v*>(rp + 16 * ((2 * chunk + 1) ^ sw));
        if constexpr (FP32) af[i] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
        else af[i] = __builtin_convertvector(__builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7), half8);
      } else {
        const int row = wm + 32 * i + frag_row;
        af[i] = *reinterpret_cast<const half8*>(st + row * kRowBytes + ((chunk ^ swizzle(row)) << 4));
      }
    }
#pragma unroll
    for (int j = 0; j < TN; j++) {
      const int row = wn + 32 * j + frag_row;
      if constexpr (FP32) {
        const unsigned char* rp = st + A_BYTES + row * BROW;
        const int sw = swizzle_f32(row);
        const f32x4v lo = *reinterpret_cast<const f32x4v*>(rp + 16 * ((2 * chunk) ^ sw));
        const f32x4v hi = *reinterpret_cast<const f32x4v*>(rp + 16 * ((2 * chunk + 1) ^ sw));
        bf[j] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
      } else {
        bf[j] = *reinterpret_cast<const half8*>(st + A_BYTES + row * kRowBytes + ((chunk ^ swizzle(row)) << 4));
      }
    }
  };
  // Issued as B x A^T: the accumulator's rows are output columns, so a lane
  // ends with four consecutive columns of one output row per group (the same
  // products summed in the same k order as A x B^T).
  auto mfmas = [&](const Frag* af, const Frag* bf) {
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
      for (int j = 0; j < TN; j++) {
        if constexpr (FP32) {
          // The f32 MFMA takes k = 16 kk + e from lanes 0-31 and + 8 from
          // lanes 32-63, e = 0 .. 7 in order: the register-staged kernel's
          // pairs and order.
#pragma unroll
          for (int e = 0; e < 8; e++) acc[i][j] = mfma_f32(bf[j][e], af[i][e], acc[i][j]);
        } else {
          acc[i][j] = mfma_f16(bf[j], af[i], acc[i][j]);
        }
      }
  };
  if constexpr (PIPE) {
    // The rest of the prologue: stages nk .. STAGES - 2 are issued too (their
    // offsets are all past K, so they load zeros without touching memory),
    // and every step issues one stage, so each wait below counts a fixed
    // number of loads and the loop body has no branches: a branch around a
    // wait or a barrier would join paths with different LDS reads pending,
    // and the compiler then waits for all of them before the next MFMA.
#pragma unroll
    for (int s = 0; s < STAGES - 1; s++)
      if (s >= nk) issue(s, s);
    // Stage 0 has landed once at most stages 1 .. STAGES - 2 are pending.
    wait_vmcnt<(STAGES - 2) * LPW>();
    block_barrier<false>();
    Frag a0[TM], b0[TN], a1[TM], b1[TN];
    read_frags(smem, 0, a0, b0);
    // sched_barrier(0) keeps the compiler from moving instructions across
    // the phase boundaries: left free, it reuses one set of fragment
    // registers for both halves (so a half's reads wait for the other half's
    // MFMAs) and hoists MFMAs above the barrier.
    for (int ks = 0; ks + 1 < nk; ks++) {
      read_frags(smem + (ks % STAGES) * STAGE_BYTES, 1, a1, b1);
      __builtin_amdgcn_sched_barrier(0);
      mfmas(a0, b0);
      __builtin_amdgcn_sched_barrier(0);
      // Stage ks + 1 has landed once at most stages ks + 2 .. ks + STAGES - 2
      // are pending; the barrier publishes it and retires stage ks - 1, whose
      // fragments every wave consumed before this point.
      wait_vmcnt<(STAGES - 3) * LPW>();
      block_barrier<false>();
      issue(ks + STAGES - 1, (ks + STAGES - 1) % STAGES);
      read_frags(smem + ((ks + 1) % STAGES) * STAGE_BYTES, 0, a0, b0);
      __builtin_amdgcn_sched_barrier(0);
      mfmas(a1, b1);
      __builtin_amdgcn_sched_barrier(0);
    }
    read_frags(smem + ((nk - 1) % STAGES) * STAGE_BYTES, 1, a1, b1);
    mfmas(a0, b0);
    mfmas(a1, b1);
    wait_vmcnt<0>();  // the zero loads past K land before the stages are reused
  } else
  for (int ks = 0; ks < nk; ks++) {
    // Stage ks is complete once at most the later stages' loads are pending;
    // the barrier then publishes it and retires stage ks - 1 for refilling.
    if (ks + STAGES - 2 < nk) wait_vmcnt<(STAGES - 2) * LPW>();
    else wait_vmcnt<0>();
    block_barrier<false>();  // this loop writes no LDS itself
    if (ks + STAGES - 1 < nk) issue(ks + STAGES - 1, (ks + STAGES - 1) % STAGES);
    const unsigned char* st = smem + (ks % STAGES) * STAGE_BYTES;
#pragma unroll
    for (int kk = 0; kk < 2; kk++) {
      Frag af[TM], bf[TN];
      read_frags(st, kk, af, bf);
      mfmas(af, bf);
    }
    asm volatile("" ::: "memory");
  }

  if constexpr (EPI == kEpiOpmFused) {
#pragma clang fp contract(off)
    // The tile is the pair block i in [ib, ib + PI) x j in [jb, jb + PJ):
    // acc[i][j] of wave (wm, wn) is pair p = PJ il + jl with il = wm / 32 + i,
    // jl = wn / 32 + j, its row a = lane % 32 and columns
    // b = 8 g4 + 4 (lane / 32) + [0, 4) in group g4.
    //  1. outer / (eps + count) goes to LDS as f16, pair p in a 2 KiB row
    //     of its own: (a, b) at half k' = 128 (b / 4) + 4 a + b % 4, whose
    //     16-byte chunk c = k' / 8 sits at slot c ^ (p % 16), so each
    //     wave-level write is 512 contiguous bytes and the 16 rows a 16-lane
    //     group of a fragment read covers fall on distinct banks.
    //  2. out[p][z] = sum_k outer[p][k] W[k][z] on MFMA, every 32-pair block
    //     against the wave's channels and k part: A fragments from the LDS
    //     rows, B fragments from the weights in the same k order (an
    //     L2-resident 256 KiB array stored in load order, so each
    //     wave-level load is 1 KiB contiguous), PRE groups loaded during the
    //     contraction, the rest AHEAD groups ahead of their MFMAs.
    //  3. With two k parts they meet in LDS past the pair rows: wave part kh
    //     keeps pair block kh and adds part 0 + part 1 in that order. Then
    //     bias / (eps + count) (and the residual) is added and each row of 32
    //     consecutive channels is stored.
    constexpr int ROW = 2048;
    constexpr int XFER = NPAIR * ROW;
    static_assert(XFER + (KP == 2 ? WAVES * 16 * 64 * 4 : 0) <= STAGES * STAGE_BYTES,
                  "the pair rows and the exchange fit the stage memory");
    const int L = g.opm_length;
    const int ib = m0 >> 5, jb = n0 >> 5;
    const int a = lane & 31, h = lane >> 5;
    block_barrier<false>();  // every wave is done reading the stages
#pragma unroll
    for (int i = 0; i < TM; i++) {
      const int il = (wm >> 5) + i;
#pragma unroll
      for (int j = 0; j < TN; j++) {
        const int jl = (wn >> 5) + j;
        const int p = PJ * il + jl;
        unsigned char* row = smem + p * ROW + 8 * (a & 1);
#pragma unroll
        for (int g4 = 0; g4 < 4; g4++) {
          half4 v;
#pragma unroll
          for (int e = 0; e < 4; e++) v[e] = (half_t)(acc[i][j][4 * g4 + e] * rcpv[i][j]);
          const int c = (2 * g4 + h) * 16 + (a >> 1);
          *reinterpret_cast<half4*>(row + 16 * (c ^ (p & 15))) = v;
        }
      }
    }
    // Group q of the wave's part: chunks (16 bytes) (128 / KP) kh + 8 q + 4 h
    // + t, t = 0..3, of the pair rows, against the same chunks of weight row
    // z, which the array holds in load order (opm_fused_weight_index).
    auto load_group = [&](int q) {
#pragma unroll
      for (int t = 0; t < 4; t++) wf[q][t] = *reinterpret_cast<const half8*>(wrow + 2048 * q + 512 * t);
    };
#pragma unroll
    for (int q = PRE; q < PRE + AHEAD; q++)
      if (q < NG) load_group(q);
    block_barrier();
    const int zb = wave & 3, kh = wave >> 2;
    const int z = 32 * zb + a;
    constexpr int FIN = KP == 2 ? 1 : NPB;  // pair blocks this wave stores
    // eps + count of the pairs this lane stores, p = 32 pb + 8 (r / 4) + 4 h
    // + r % 4, read while the MFMAs run.
    float dnv[FIN][16];
#pragma unroll
    for (int f = 0; f < FIN; f++) {
      const int pb = KP == 2 ? kh : f;
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int p = 32 * pb + 8 * (r >> 2) + 4 * h + (r & 3);
        const int i = ib + p / PJ, j = jb + p % PJ;
        dnv[f][r] = g.opm_eps + (i < L && j < L ? g.opm_count[(int64_t)i * L + j] : 0.0f);
      }
    }
    const unsigned char* arow = smem + a * ROW;
    const int aswz = a & 15;  // the rows 32 pb + a share their low four bits
    floatx16 part[NPB];
#pragma unroll
    for (int pb = 0; pb < NPB; pb++)
#pragma unroll
      for (int v = 0; v < 16; v++) part[pb][v] = 0.0f;
    float bterm[FIN][16];  // bias / (eps + count), computed among the MFMAs
#pragma unroll
    for (int q = 0; q < NG; q++) {
      if (q + PRE + AHEAD < NG) load_group(q + PRE + AHEAD);
      if (q == NG / 2) {
#pragma unroll
        for (int f = 0; f < FIN; f++)
#pragma unroll
          for (int r = 0; r < 16; r++) bterm[f][r] = bz / dnv[f][r];
      }
#pragma unroll
      for (int t = 0; t < 4; t++) {
        const int c = (128 / KP) * kh + 8 * q + 4 * h + t;
#pragma unroll
        for (int pb = 0; pb < NPB; pb++) {
          const half8 af = *reinterpret_cast<const half8*>(arow + 32 * pb * ROW + 16 * (c ^ aswz));
          part[pb] = mfma_f16(af, wf[q][t], part[pb]);
        }
      }
    }
    // part[pb][r] = this wave's part of out[p][z], p = 32 pb + 8 (r / 4) + 4 h + r % 4.
    float y[NPB][16];
    if constexpr (KP == 2) {
      // The exchange area lies past the pair rows, so no wave waits for the
      // others to finish reading them.
      // Slot (zb, pair block) holds each lane's 16 values as four 16-byte
      // chunks, chunk c of lane l at l * 64 + 16 (c ^ (l / 4 % 4)): the 16
      // lanes of an access fall on distinct banks.
      unsigned char* const xfer = smem + XFER;
      const int give = 1 - kh;
      const int xs = (lane >> 2) & 3;
#pragma unroll
      for (int c = 0; c < 4; c++) {
        floatx4 v;
#pragma unroll
        for (int e = 0; e < 4; e++) v[e] = kh ? part[0][4 * c + e] : part[1][4 * c + e];
        *reinterpret_cast<floatx4*>(xfer + (zb * 2 + give) * 4096 + lane * 64 + 16 * (c ^ xs)) = v;
      }
      block_barrier();
#pragma unroll
      for (int c = 0; c < 4; c++) {
        const floatx4 other = *reinterpret_cast<const floatx4*>(xfer + (zb * 2 + kh) * 4096 + lane * 64 + 16 * (c ^ xs));
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const float mine = kh ? part[1][4 * c + e] : part[0][4 * c + e];
          y[0][4 * c + e] = kh ? other[e] + mine : mine + other[e];
        }
      }
    } else {
#pragma unroll
      for (int pb = 0; pb < NPB; pb++)
#pragma unroll
        for (int r = 0; r < 16; r++) y[pb][r] = part[pb][r];
    }
    const bool residual = (g.flags & AFHIP_EPILOGUE_RESIDUAL) != 0;
    TC* C = reinterpret_cast<TC*>(g.c);
#pragma unroll
    for (int f = 0; f < FIN; f++) {
      const int pb = KP == 2 ? kh : f;
      int64_t at[16];
      bool on[16];
      float old[16];
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int p = 32 * pb + 8 * (r >> 2) + 4 * h + (r & 3);
        const int i = ib + p / PJ, j = jb + p % PJ;
        on[r] = i < L && j < L && z < g.ldc;
        at[r] = ((int64_t)i * L + j) * g.ldc + z;
        old[r] = 0.0f;
      }
      if (residual) {  // every old value in flight before the first store
#pragma unroll
        for (int r = 0; r < 16; r++)
          if (on[r]) old[r] = (float)C[at[r]];
      }
#pragma unroll
      for (int r = 0; r < 16; r++) {
        float v = y[f][r] + bterm[f][r];
        if (residual) v += old[r];
        if (on[r]) C[at[r]] = (TC)v;
      }
    }
    return;
  }
  if constexpr (sizeof(TC) == 2) {
    if (g.flags == 0 && !g.c_column_major && (g.ldc & 7) == 0 && (reinterpret_cast<uintptr_t>(g.c) & 15) == 0 &&
        (g.sc & 7) == 0) {
      // Plain f16 store (the contraction's case), staged through the stage
      // memory (BM x BN halves fit in it) so that every wave-level store
      // writes whole 128-byte lines. Row r keeps 16-byte chunk c at slot
      // c ^ (r & 7); a lane holds row wm + 32 i + lane % 32 and, per group g4,
      // columns wn + 32 j + 8 g4 + 4 (lane / 32) + [0, 4): one 8-byte write.
      static_assert(BM * BN * 2 <= STAGES * STAGE_BYTES, "the tile fits the stage memory");
      constexpr int ROWB = BN * 2;
      block_barrier<false>();  // every wave is done reading the stages
#pragma unroll
      for (int i = 0; i < TM; i++) {
        const int r = wm + 32 * i + (lane & 31);
#pragma unroll
        for (int j = 0; j < TN; j++)
#pragma unroll
          for (int g4 = 0; g4 < 4; g4++) {
            const int chunk = (wn + 32 * j + 8 * g4) >> 3;
            half4 h;
#pragma unroll
            for (int e = 0; e < 4; e++) h[e] = (half_t)acc[i][j][4 * g4 + e];
            *reinterpret_cast<half4*>(smem + r * ROWB + 16 * (chunk ^ (r & 7)) + 8 * (lane >> 5)) = h;
          }
      }
      block_barrier();
      half_t* C = reinterpret_cast<half_t*>(g.c) + (int64_t)bt * g.sc;
      constexpr int CPR = BN / 8;  // 16-byte chunks per row
      static_assert((BM * CPR) % (2 * kThreads) == 0, "stores go in pairs");
      for (int idx0 = threadIdx.x; idx0 < BM * CPR; idx0 += 2 * kThreads) {
        u32x4 v[2];
#pragma unroll
        for (int k = 0; k < 2; k++) {
          const int idx = idx0 + k * kThreads;
          const int r = idx / CPR, c = idx - r * CPR;
          const int row = m0 + r, col = n0 + 8 * c;
          v[k] = *reinterpret_cast<const u32x4*>(smem + r * ROWB + 16 * (c ^ (r & 7)));
          if (row < g.M) {
            half_t* dst = C + (int64_t)row * g.ldc + col;
            if (col + 8 <= g.N) {
              *reinterpret_cast<u32x4*>(dst) = v[k];
            } else {
              const half8 h = __builtin_bit_cast(half8, v[k]);
              for (int e = 0; e < 8 && col + e < g.N; e++) dst[e] = h[e];
            }
          }
        }
        stores_read(v[0], v[1]);
      }
      return;
    }
  }
  if constexpr (sizeof(TC) == 2) {
    if (g.flags == EPILOGUE_OPM_CONTRACT && !g.c_column_major && g.opm_outer == 32 &&
        (reinterpret_cast<uintptr_t>(g.c) & 15) == 0) {
      // Outer-product-mean contraction with c_outer = 32: row = i_local * 32
      // + a, col = j * 32 + b, so each 32 x 32 MFMA tile is one pair (i, j)
      // and lands as the contiguous 2 KiB block outer[i_local][j][a][b],
      // divided by (eps + count[i][j]) (one reciprocal per block). The tile
      // is staged through the stage memory as in the plain case, then every
      // wave-level store writes half a block (1 KiB of whole lines).
      static_assert(BM * BN * 2 <= STAGES * STAGE_BYTES, "the tile fits the stage memory");
      constexpr int ROWB = BN * 2;
      block_barrier<false>();  // every wave is done reading the stages
#pragma unroll
      for (int i = 0; i < TM; i++) {
        const int r = wm + 32 * i + (lane & 31);
        const int il = (m0 + wm + 32 * i) >> 5;
#pragma unroll
        for (int j = 0; j < TN; j++) {
          const int jj = (n0 + wn + 32 * j) >> 5;
          const float cnt = il < (g.M >> 5) && jj < g.opm_length
                                ? g.opm_count[(int64_t)(g.opm_row0 + il) * g.opm_length + jj]
                                : 0.0f;
          const float rcp = 1.0f / (g.opm_eps + cnt);
#pragma unroll
          for (int g4 = 0; g4 < 4; g4++) {
            const int chunk = (wn + 32 * j + 8 * g4) >> 3;
            half4 h;
#pragma unroll
            for (int e = 0; e < 4; e++) h[e] = (half_t)(acc[i][j][4 * g4 + e] * rcp);
            *reinterpret_cast<half4*>(smem + r * ROWB + 16 * (chunk ^ (r & 7)) + 8 * (lane >> 5)) = h;
          }
        }
      }
      block_barrier();
      half_t* C = reinterpret_cast<half_t*>(g.c);
      constexpr int BLOCKS = (BM / 32) * (BN / 32);
      // Half-block h of tile block q: rows a in [16 h, 16 h + 16), 4 lanes per
      // 64-byte row.
      static_assert((2 * BLOCKS) % (2 * WAVES) == 0, "stores go in pairs");
      for (int idx0 = threadIdx.x >> 6; idx0 < 2 * BLOCKS; idx0 += 2 * WAVES) {
        u32x4 v[2];
#pragma unroll
        for (int k = 0; k < 2; k++) {
          const int idx = idx0 + k * WAVES;
          const int q = idx >> 1, half = idx & 1;
          const int bi = q / (BN / 32), bj = q - bi * (BN / 32);
          const int a = 16 * half + (lane >> 2), c = lane & 3;  // 16-byte chunk c of the 64-byte row
          const int il = (m0 >> 5) + bi, jj = (n0 >> 5) + bj;
          const int r = 32 * bi + a, chunk = 4 * bj + c;
          v[k] = *reinterpret_cast<const u32x4*>(smem + r * ROWB + 16 * (chunk ^ (r & 7)));
          if (32 * il < g.M && jj < g.opm_length)
            *reinterpret_cast<u32x4*>(C + (((int64_t)il * g.opm_length + jj) * 32 + a) * 32 + 8 * c) = v[k];
        }
        stores_read(v[0], v[1]);
      }
      return;
    }
  }
  if ((g.flags & ~gemm_detail::kRowwiseEpilogue) == 0 && !g.c_column_major) {
    // Row-wise epilogues (plain, scale, bias, ReLU, residual, the
    // outer-product-mean output's bias / (eps + count)) straight from the
    // accumulators: lane holds row m0 + wm + 32 i + lane % 32 and, per group
    // g4, columns n0 + wn + 32 j + 8 g4 + 4 (lane / 32) + [0, 4).
    auto aligned4 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & (4 * sizeof(TC) - 1)) == 0; };
    const bool vec4 = (g.ldc & 3) == 0 && (g.sc & 3) == 0 && aligned4(g.c) &&
                      (!(g.flags & AFHIP_EPILOGUE_RESIDUAL) || aligned4(g.residual));
    if (!(g.flags & EPILOGUE_OPM_OUTPUT) && vec4 && m0 + BM <= g.M && n0 + BN <= g.N) {
      // A whole tile with scale, bias, ReLU and residual at most: no global
      // read waits behind a store. The output may alias the residual (and,
      // as far as the compiler knows, the scale and bias), so it keeps such a
      // read after any earlier store; interleaved, that was one memory round
      // trip per four outputs. Here the tile's scale and bias go to LDS once
      // (the stages are idle), and the residual values of each 32-row block
      // are read before its first store: a lane reads only the elements it
      // later writes. The arithmetic is epilogue_row4's, step for step.
#pragma clang fp contract(off)
      typedef TC tc4 __attribute__((ext_vector_type(4)));
      const uint32_t flags = g.flags;
      float* const bl = reinterpret_cast<float*>(smem);
      float* const sl = bl + BN;
      const TC* R = reinterpret_cast<const TC*>(g.residual) + (int64_t)bt * g.sc;
      TC* C = reinterpret_cast<TC*>(g.c) + (int64_t)bt * g.sc;
      auto load_res = [&](int i, tc4(&res)[TN][4]) {
        const int row = m0 + wm + 32 * i + (lane & 31);
#pragma unroll
        for (int j = 0; j < TN; j++)
#pragma unroll
          for (int g4 = 0; g4 < 4; g4++)
            res[j][g4] = *reinterpret_cast<const tc4*>(R + (int64_t)row * g.ldc + n0 + wn + 32 * j + 8 * g4 +
                                                       4 * (lane >> 5));
      };
      // With f16 outputs the residual reads run one row block ahead of the
      // stores (block 0's before the bias staging), so their round trips
      // overlap the stores instead of preceding them; f32 has no registers
      // to spare for the second block.
      constexpr bool kAhead = sizeof(TC) == 2;
      tc4 res_a[TN][4], res_b[TN][4];
      if (kAhead && (flags & AFHIP_EPILOGUE_RESIDUAL)) load_res(0, res_a);
      if (flags & (AFHIP_EPILOGUE_BIAS | AFHIP_EPILOGUE_SCALE)) {
        block_barrier<false>();  // every wave is done reading the stages
        for (int c = threadIdx.x; c < BN; c += kThreads) {
          if (flags & AFHIP_EPILOGUE_BIAS) bl[c] = g.bias[n0 + c];
          if (flags & AFHIP_EPILOGUE_SCALE) sl[c] = g.scale[n0 + c];
        }
        block_barrier();
      }
#pragma unroll
      for (int i = 0; i < TM; i++) {
        const int row = m0 + wm + 32 * i + (lane & 31);
        tc4(&res)[TN][4] = (!kAhead || i % 2 == 0) ? res_a : res_b;
        if (flags & AFHIP_EPILOGUE_RESIDUAL) {
          if (!kAhead) load_res(i, res);
          else if (i + 1 < TM) load_res(i + 1, i % 2 == 0 ? res_b : res_a);
        }
#pragma unroll
        for (int j = 0; j < TN; j++)
#pragma unroll
          for (int g4 = 0; g4 < 4; g4++) {
            const int col = n0 + wn + 32 * j + 8 * g4 + 4 * (lane >> 5);
            tc4 v;
#pragma unroll
            for (int e = 0; e < 4; e++) {
              float y = acc[i][j][4 * g4 + e];
              if (flags & AFHIP_EPILOGUE_SCALE) y *= sl[wn + 32 * j + 8 * g4 + 4 * (lane >> 5) + e];
              if (flags & AFHIP_EPILOGUE_BIAS) y += bl[wn + 32 * j + 8 * g4 + 4 * (lane >> 5) + e];
              if (flags & AFHIP_EPILOGUE_RELU) y = fmaxf(y, 0.0f);
              if (flags & AFHIP_EPILOGUE_RESIDUAL) y += (float)res[j][g4][e];
              v[e] = (TC)y;
            }
            *reinterpret_cast<tc4*>(C + (int64_t)row * g.ldc + col) = v;
          }
      }
      return;
    }
#pragma unroll
    for (int i = 0; i < TM; i++) {
      const int row = m0 + wm + 32 * i + (lane & 31);
      if (row >= g.M) continue;
#pragma unroll
      for (int j = 0; j < TN; j++)
#pragma unroll
        for (int g4 = 0; g4 < 4; g4++) {
          const int col = n0 + wn + 32 * j + 8 * g4 + 4 * (lane >> 5);
          if (col >= g.N) continue;
          float y[4] = {acc[i][j][4 * g4], acc[i][j][4 * g4 + 1], acc[i][j][4 * g4 + 2], acc[i][j][4 * g4 + 3]};
          gemm_detail::epilogue_row4<TC>(g, bt, row, col, y, min(4, g.N - col), vec4);
        }
    }
    return;
  }
  if (g.c_column_major && (g.flags & ~(AFHIP_EPILOGUE_SCALE | AFHIP_EPILOGUE_BIAS | AFHIP_EPILOGUE_RELU |
                                       AFHIP_EPILOGUE_RESIDUAL)) == 0) {
    // A column-major output with the row-wise epilogues, straight from the
    // accumulators: for element v a lane holds row m0 + wm + 32 i + lane % 32
    // of column n0 + wn + 32 j + mfma_row(v, lane), so each half-wave's 32
    // lanes write 32 consecutive elements of one output column. The steps
    // and roundings are epilogue_store's.
#pragma clang fp contract(off)
    const uint32_t flags = g.flags;
    TC* const C = reinterpret_cast<TC*>(g.c) + (int64_t)bt * g.sc;
    const TC* const R =
        (flags & AFHIP_EPILOGUE_RESIDUAL) ? reinterpret_cast<const TC*>(g.residual) + (int64_t)bt * g.sc : nullptr;
#pragma unroll
    for (int i = 0; i < TM; i++) {
      const int row = m0 + wm + 32 * i + (lane & 31);
#pragma unroll
      for (int j = 0; j < TN; j++) {
#pragma unroll 1
        for (int g4 = 0; g4 < 4; g4++) {
          float y[4];
#pragma unroll
          for (int e = 0; e < 4; e++) y[e] = acc[i][j][4 * g4 + e];
          const int col0 = n0 + wn + 32 * j + 8 * g4 + 4 * (lane >> 5);
#pragma unroll
          for (int e = 0; e < 4; e++) {
            const int col = col0 + e;
            if (row >= g.M || col >= g.N) continue;
            float t = y[e];
            if (flags & AFHIP_EPILOGUE_SCALE) t *= g.scale[col];
            if (flags & AFHIP_EPILOGUE_BIAS) t += g.bias[col];
            if (flags & AFHIP_EPILOGUE_RELU) t = fmaxf(t, 0.0f);
            const int64_t at = (int64_t)col * g.ldc + row;
            if (flags & AFHIP_EPILOGUE_RESIDUAL) t += (float)R[at];
            C[at] = (TC)t;
          }
        }
      }
    }
    return;
  }
  // Any other epilogue: each wave passes its 32 x 32 tiles through a private
  // LDS square and applies the epilogue in a rolled loop, so the code stays
  // small and the accumulators never need dynamic indexing.
  block_barrier<false>();  // every wave is done reading the stages
  float* sq = reinterpret_cast<float*>(smem) + wave * (32 * 33);
#pragma unroll
  for (int i = 0; i < TM; i++)
#pragma unroll
    for (int j = 0; j < TN; j++) {
#pragma unroll
      for (int v = 0; v < 16; v++) sq[(lane & 31) * 33 + mfma_row(v, lane)] = acc[i][j][v];
      __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the square is written
      __builtin_amdgcn_wave_barrier();
      const int col = n0 + wn + 32 * j + (lane & 31);
#pragma unroll 1
      for (int e = 0; e < 16; e++) {
        const int r = e + 16 * (lane >> 5);
        const int row = m0 + wm + 32 * i + r;
        const float y = sq[r * 33 + (lane & 31)];
        if (row < g.M && col < g.N) gemm_detail::epilogue_store<TC>(g, bt, row, col, y);
      }
      __builtin_amdgcn_s_waitcnt(0xc07f);  // reads done before the next tile overwrites
      __builtin_amdgcn_wave_barrier();
    }
}

template <int BM, int BN, int STAGES, int WM, int WN, bool PIPE, typename TC, int LW = 16, bool AK = false,
          bool AF = false, bool FP32 = false>
int launch_tile(const GemmArgs& g, const char* label, hipStream_t s) {
  gemm_detail::KernelArgs ka;
  ka.g = g;
  ka.tiles_m = (int)ceil_div(g.M, BM);
  ka.tiles_n = (int)ceil_div(g.N, BN);
  const int64_t total = (int64_t)ka.tiles_m * ka.tiles_n * g.batch;
  if (total > ((int64_t)1 << 30)) return set_error(AFHIP_ERR_INVALID_ARGUMENT, "GEMM has too many tiles");
  ka.total_tiles = (int)total;
  ka.per_xcd = (int)ceil_div(total, 8);
  const size_t shared = (size_t)STAGES * dma_stage_bytes(BM, BN, AF || FP32, FP32);
  auto kernel = gemm_dma_kernel<BM, BN, STAGES, WM, WN, PIPE, TC, kEpiGeneric, LW, AK, AF, FP32>;
  if (int st = allow_lds((const void*)kernel, shared)) return st;
  return launch(label, kernel, dim3((unsigned)(ka.per_xcd * 8)), dim3(64 * WM * WN), shared, s, ka);
}

template <int BM, int BN, int STAGES, int WM, int WN, bool PIPE, typename TC>
int launch_opm_fused(const GemmArgs& g, const char* label, hipStream_t s) {
  gemm_detail::KernelArgs ka;
  ka.g = g;
  ka.tiles_m = (int)ceil_div(g.M, BM);
  ka.tiles_n = (int)ceil_div(g.N, BN);
  ka.total_tiles = ka.tiles_m * ka.tiles_n;
  ka.per_xcd = (int)ceil_div(ka.total_tiles, 8);
  const size_t shared = (size_t)STAGES * dma_stage_bytes(BM, BN, false);
  auto kernel = gemm_dma_kernel<BM, BN, STAGES, WM, WN, PIPE, TC, kEpiOpmFused>;
  if (int st = allow_lds((const void*)kernel, shared)) return st;
  return launch(label, kernel, dim3((unsigned)(ka.per_xcd * 8)), dim3(64 * WM * WN), shared, s, ka);
}

// The 256 x 256 tile (64 pairs, one workgroup a CU). Measured at N_seq = 512,
// N_res = 256 (f32 out): 106 us against 109 us for 128 x 256 tiles (32 pairs,
// two workgroups a CU, twice the weight traffic).
template <typename TC> int launch_opm_fused_tile(const GemmArgs& g, const char* label, hipStream_t s) {
  return launch_opm_fused<256, 256, 5, 2, 4, true, TC>(g, label, s);
}

// Operand rows whose k-runs are 16-byte aligned load 16 bytes a lane;
// otherwise (4-byte aligned, dma_eligible) 4 bytes a lane.
bool dma_wide(const GemmArgs& g) {
  auto al16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  return al16(g.a) && al16(g.b) && g.K % 8 == 0 && g.lda % 8 == 0 && g.ldb % 8 == 0 && g.sa % 8 == 0 && g.sb % 8 == 0;
}

template <typename TC>
int launch_typed(const GemmArgs& g, const GemmTypes& t, int tm, int tn, const char* label, hipStream_t s) {
  // f32 arithmetic (dma_eligible: f32 operands in 16-byte rows) on 64 x 64
  // tiles whatever the selection: four 16 KiB stages, three in flight, two
  // workgroups a CU; the f32 MFMA's rate makes the small tile's operand
  // traffic no limit.
  if (t.precision == AFHIP_PRECISION_F32)
    return launch_tile<64, 64, 4, 2, 2, false, TC, 16, false, false, true>(g, label, s);
  const bool a_f32 = t.a_dtype == AFHIP_F32;
  // An f32 A (dma_eligible: 16-byte rows) on 128 x 128 tiles whatever the
  // selection: three stages of 24 KiB keep two workgroups a CU, where
  // 128 x 256 (32 KiB stages) keeps one. Measured on MI355X, f16 out
  // (128 x 128 / 128 x 256): 29972 x 1024 x 256 31.4 / 36.5 us,
  // 29972 x 256 x 1024 36.5 / 40.5, 4096 x 1024 x 4096 58.0 / 63.7.
  if (a_f32) return launch_tile<128, 128, 3, 2, 2, false, TC, 16, false, true>(g, label, s);
  // A k-major A (dma_eligible: 16-byte rows) on the tiles whose k rows fill
  // whole load instructions. 192 x 192 runs as 128 x 256 where that still
  // gives every CU two tiles, else as 128 x 128 (8192 x 512 x 8192 on
  // MI355X: 87.0 us against 96.2 us).
  if (g.a_row_contiguous) {
    const int64_t cus = device_cu_count() > 0 ? device_cu_count() : 256;
    if (tm == 192 && ceil_div(g.M, 128) * ceil_div(g.N, 256) * g.batch >= 2 * cus) tn = 256, tm = 128;
    if (tm == 128 && tn == 256) return launch_tile<128, 256, 3, 2, 2, false, TC, 16, true>(g, label, s);
    if (tm == 256 && tn == 256) return launch_tile<256, 256, 5, 2, 4, true, TC, 16, true>(g, label, s);
    return launch_tile<128, 128, 4, 2, 2, false, TC, 16, true>(g, label, s);
  }
  // 4-byte loads take four times the instructions; the 128 x 128 tile (five
  // stages of 16 loads a wave, three in flight) keeps them within vmcnt's
  // range.
  if (!dma_wide(g)) return launch_tile<128, 128, 5, 2, 2, false, TC, 4>(g, label, s);
  if (tm == 192 && tn == 192) return launch_tile<192, 192, 3, 2, 2, false, TC>(g, label, s);
  if (tm == 128 && tn == 128) return launch_tile<128, 128, 4, 2, 2, false, TC>(g, label, s);
  if (tm == 128 && tn == 256) return launch_tile<128, 256, 3, 2, 2, false, TC>(g, label, s);
  if (tm == 256 && tn == 256) return launch_tile<256, 256, 5, 2, 4, true, TC>(g, label, s);
  return set_error(AFHIP_ERR_INVALID_ARGUMENT, "unsupported LDS_DMA tile %dx%d", tm, tn);
}

}  // namespace

bool dma_tile_supported(int tm, int tn) {
  return (tm == 192 && tn == 192) || (tm == 128 && tn == 128) || (tm == 128 && tn == 256) || (tm == 256 && tn == 256);
}

bool dma_eligible(const GemmArgs& g, const GemmTypes& t) {
  auto al4 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 3) == 0; };
  auto al16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  if (g.M <= 0 || g.N <= 0 || g.K <= 0 || g.batch <= 0) return false;
  // f32 arithmetic: f32 operands, both k-contiguous, in 16-byte chunks of
  // 4 k (K a multiple of 4, so no chunk runs past K).
  if (t.precision == AFHIP_PRECISION_F32)
    return t.a_dtype == AFHIP_F32 && t.b_dtype == AFHIP_F32 && !g.a_row_contiguous && al16(g.a) && al16(g.b) &&
           g.K % 4 == 0 && g.lda % 4 == 0 && g.ldb % 4 == 0 && g.sa % 4 == 0 && g.sb % 4 == 0 && g.lda >= g.K &&
           g.ldb >= g.K && (int64_t)256 * std::max(g.lda, g.ldb) * 4 < (int64_t)kOutOfRange;
  if (t.precision != AFHIP_PRECISION_F16 || t.b_dtype != AFHIP_F16) return false;
  if (t.a_dtype != AFHIP_F16 && t.a_dtype != AFHIP_F32) return false;
  // An f32 A loads 16-byte chunks of 4 k (k-contiguous rows), B 16-byte
  // chunks of 8: K a multiple of 8, so no chunk runs past K.
  if (t.a_dtype == AFHIP_F32)
    return !g.a_row_contiguous && al16(g.a) && al16(g.b) && g.K % 8 == 0 && g.lda % 4 == 0 && g.sa % 4 == 0 &&
           g.ldb % 8 == 0 && g.sb % 8 == 0 && g.lda >= g.K && g.ldb >= g.K &&
           (int64_t)256 * g.lda * 4 < (int64_t)kOutOfRange && (int64_t)256 * g.ldb * 2 < (int64_t)kOutOfRange;
  // A k-major A loads whole 16-byte chunks of its k rows.
  if (g.a_row_contiguous)
    return dma_wide(g) && g.M % 8 == 0 && g.lda >= g.M && g.ldb >= g.K &&
           (int64_t)g.K * g.lda * 2 < (int64_t)kOutOfRange && (int64_t)256 * g.ldb * 2 < (int64_t)kOutOfRange;
  // 16-byte loads (dma_wide) or, for rows that are only 4-byte aligned,
  // 4-byte loads, which need K and the strides even.
  if (!al4(g.a) || !al4(g.b)) return false;
  if (g.K % 2 || g.lda % 2 || g.ldb % 2 || g.sa % 2 || g.sb % 2) return false;
  if (g.lda < g.K || g.ldb < g.K) return false;
  // Byte offsets within a 256-row panel stay below the out-of-range marker.
  return (int64_t)256 * std::max(g.lda, g.ldb) * 2 < (int64_t)kOutOfRange;
}

void dma_heuristic_tile(int64_t M, int64_t N, int64_t K, int64_t batch, int* tm, int* tn) {
  // Measured on MI355X (kernel time; triangle contractions 128 x L^3, the
  // outer-product-mean contraction and output):
  //            128x128  192x192  128x256  256x256
  //  L = 1024   394 us   373 us   340 us   335 us
  //  L = 768    186      155      160      164
  //  L = 512     52       55       48       49
  //  L = 384     28       25       30       36
  //  OPM 8192x8192x512       123 / 96 / 104 / 95;  OPM 65536x128x1024   28 / 37 / 36 / 34
  //  131072x256x1024 (MSA transition, second linear, + residual)  188 / 225 / 162 / 159
  //  131072x128x1024                                                98 / 127 / 128 / 128
  // so: 256 x 256 for long K on large outputs with 256-aligned columns; else 192 x 192 when its
  // ragged edges waste at most 1/20 of the work and there are at least two
  // tiles a CU; else 128 x 256 when K and the output are wide enough; else
  // 128 x 128, which keeps ragged-edge waste low and the tile count high.
  const int64_t cus = device_cu_count() > 0 ? device_cu_count() : 256;
  auto waste = [](int64_t x, int64_t t) { return (double)(ceil_div(x, t) * t - x) / (double)x; };
  if (K >= 1024 && M >= 1024 && N >= 256 && waste(M, 256) <= 0.05 && waste(N, 256) <= 0.05 &&
      ceil_div(M, 256) * ceil_div(N, 256) * batch >= cus) {
    *tm = *tn = 256;
    return;
  }
  if (waste(M, 192) <= 0.05 && waste(N, 192) <= 0.05 && ceil_div(M, 192) * ceil_div(N, 192) * batch >= 2 * cus) {
    *tm = *tn = 192;
    return;
  }
  if (K >= 512 && M >= 512 && N >= 512 && waste(M, 128) <= 0.05 && waste(N, 256) <= 0.05 &&
      ceil_div(M, 128) * ceil_div(N, 256) * batch >= 2 * cus) {
    *tm = 128;
    *tn = 256;
    return;
  }
  *tm = *tn = 128;
}

int run_opm_fused(const GemmArgs& g, int c_dtype, const char* label, hipStream_t s) {
  auto al16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  if (g.M != 32 * g.opm_length || g.N != g.M || g.K <= 0 || g.K % 8 || g.lda % 8 || g.ldb % 8 || g.lda < g.K ||
      g.ldb < g.K || !al16(g.a) || !al16(g.b) || !al16(g.opm_w) || g.ldc <= 96 || g.ldc > 128 ||
      (int64_t)256 * std::max(g.lda, g.ldb) * 2 >= (int64_t)kOutOfRange || (int64_t)g.opm_length * 32 > (1 << 24))
    return set_error(AFHIP_ERR_INVALID_ARGUMENT, "fused outer-product-mean launch outside its shape");
  if (c_dtype == AFHIP_F16) return launch_opm_fused_tile<half_t>(g, label, s);
  return launch_opm_fused_tile<float>(g, label, s);
}

int run_gemm_dma(const GemmArgs& g, const GemmTypes& t, int tm, int tn, const char* label, hipStream_t s) {
  if (t.c_dtype == AFHIP_F16) return launch_typed<half_t>(g, t, tm, tn, label, s);
  return launch_typed<float>(g, t, tm, tn, label, s);
}

}  // namespace afhip
