// The STREAM GEMM kernel for gfx950: weight-stationary, activation-streaming.
//
// It carries the HBM-bound projections: many rows, a short inner dimension
// (K = 64, 128 or 256) and a weight small enough to live in registers, as the
// MSA row-attention's fused q/k/v/gate projection with int8 weights
// (src/runtime/gemm.ts:150-206 mixed-q8 variant; per-output-channel scales,
// src/runtime/q8.ts). Every byte of the activations is read from HBM once
// and every output byte written once; the arithmetic hides under that
// traffic.
//
// Design:
//  - A workgroup of four wave64s owns 256 columns of the output (a slice:
//    four 64-column chunks, one from each quarter of the columns, so every
//    workgroup carries the same mix of epilogue work) and walks 32-row tiles
//    of A; two workgroups share a CU and, having no barrier in common, drift
//    apart so one's MFMAs overlap the other's epilogue and stores. Each wave keeps W for its 64 columns in VGPRs,
//    widened to f16 once at launch (int8 -> f16 is exact), as the A operand
//    of v_mfma_f32_32x32x16_f16; the activation tile is the B operand. The
//    accumulator's rows are therefore output columns, four consecutive ones
//    per lane, which the epilogue writes to LDS as 8-byte groups.
//  - The per-output-channel scale multiplies the f32 accumulator in the
//    epilogue: sum_k a[k] * (q[k][n] * s[n]) = s[n] * sum_k a[k] * q[k][n],
//    with the products a * q exact in f32.
//  - Activation tiles travel global -> LDS without passing through VGPRs
//    (buffer_load_dwordx4 ... lds), three stages: two tiles are in flight
//    while one computes. A row's 16-byte chunks are stored XOR-swizzled
//    (slot = chunk ^ (row & 7)) so the 32 rows an MFMA fragment reads spread
//    over all bank groups.
//  - Waves 0-1 issue the loads and waves 2-3 the stores, so a loader's
//    vmcnt counts its own loads only and its wait for a tile is exact. The
//    output tile is staged in LDS and leaves as two 512-byte rows per
//    wave-level buffer_store_dwordx4; buffer stores at offsets past the
//    resource are dropped, which covers ragged rows and columns.
//  - Workgroup b takes slice (b / 8) % slices of row-tile group
//    (b / 8 / slices) * 8 + b % 8, so every slice of a row tile runs on the
//    same XCD (ids are dealt round-robin over eight XCDs) and the re-reads
//    of an activation tile hit that XCD's L2.
//  - The epilogue applies the register-staged kernel's operations in its
//    order (scale, bias, attention q-scaling or gate, ReLU) with the same
//    roundings, so the two families give bit-identical outputs.
//  - Adding into the output (out += f16(result), for the attention output's
//    residual), the storer waves read the old values of a tile one pass
//    before they store it, so the read's latency hides under a pass of
//    MFMAs, and add them to the staged f16 result in f32 with one rounding:
//    the result of writing the product and adding it in a second pass, in
//    one. (The register-staged kernel's RESIDUAL epilogue rounds once, so
//    this is not that epilogue.)
#include <algorithm>
#include <type_traits>

#include "dma.h"
#include "gemm.h"

namespace afhip {

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = 4;
constexpr int kLoaders = 2;         // waves 0-1 load, waves 2-3 store
constexpr int kBM = 32;             // rows per tile
constexpr int kBN = 64 * kWaves;    // columns per slice
constexpr int kStages = 3;


template <int K> struct StreamLayout {
  static constexpr int RB = 2 * K;                     // bytes of one activation row
  static constexpr int SLOTS = RB / 16;                // its 16-byte chunks
  static constexpr int STAGE = kBM * RB;
  static constexpr int LPW = STAGE / 1024 / kLoaders;  // wave-level loads per tile, per loader
  static constexpr int ROWS_PER_LOAD = 1024 / RB;
  static constexpr int OROW = 2 * kBN;                 // staging row: 512 bytes, 16-byte chunks XOR-swizzled
  static constexpr int OBUF = kBM * OROW;              // one staging buffer (16 KiB)
  static constexpr int OUT = kStages * STAGE;
  static constexpr int BYTES = OUT + 2 * OBUF;         // 80 KiB at K = 256: two workgroups fill a CU
  static_assert(LPW >= 1 && STAGE % (1024 * kLoaders) == 0, "tile shape");
  static_assert(LPW * 2 == K / 16, "one load per two k-steps");
  static_assert((kBM / 2 / (kWaves - kLoaders)) % (K / 32) == 0, "stores spread evenly over the k-steps");
  static_assert((kStages - 2) * LPW < 64, "vmcnt holds at most 63 outstanding loads");
};

struct StreamArgs {
  const half_t* a;
  const void* w;
  half_t* c;
  const float* scale;
  const float* bias;
  int M, N;
  int64_t lda, ldw, ldc;
  uint32_t flags;
  int head_cols;
  float q_scale;
  int ntiles, slices, groups;
};

template <typename TW> __device__ __forceinline__ half8 load_w8(const TW* p);
template <> __device__ __forceinline__ half8 load_w8<half_t>(const half_t* p) {
  return *reinterpret_cast<const half8*>(p);
}
template <> __device__ __forceinline__ half8 load_w8<int8_t>(const int8_t* p) {
  const uint2 v = *reinterpret_cast<const uint2*>(p);
  half8 h;
#pragma unroll
  for (int e = 0; e < 4; e++) {
    h[e] = (half_t)(float)(int8_t)(v.x >> (8 * e));
    h[4 + e] = (half_t)(float)(int8_t)(v.y >> (8 * e));
  }
  return h;
}

constexpr int kPlain = 0, kQuery = 1, kGate = 2;  // a wave's attention block role

// x[i] = x[i] * s_i (+ b_i) for i = I..15, where s_i and b_i are lane i of
// this lane's 16-lane row in the registers s and b, read through DPP
// row_newbcast as the multiply's and add's first operand: one VGPR holds a
// lane's 16 per-column factors. Two roundings, as the register-staged
// epilogue (no fused multiply-add). x comes straight from MFMAs, whose results
// a VALU instruction may read only 18 wait states later, and the compiler's
// hazard padding does not see into inline assembly: the first statement pads
// them itself, and the SGPR token keeps the statements in order behind it.
// s and b are written once at launch, far ahead of their DPP reads.
template <int I, bool BIAS>
__device__ __forceinline__ void scale_row(floatx16& x, float s, float b, int& tok) {
  if constexpr (I < 16) {
    float y;
    if constexpr (I == 0)
      asm("s_nop 7\n\ts_nop 7\n\ts_nop 3\n\tv_mul_f32_dpp %0, %2, %3 row_newbcast:0 row_mask:0xf bank_mask:0xf"
          : "=v"(y), "+s"(tok)
          : "v"(s), "v"(x[I]));
    else
      asm("v_mul_f32_dpp %0, %2, %3 row_newbcast:%4 row_mask:0xf bank_mask:0xf"
          : "=v"(y), "+s"(tok)
          : "v"(s), "v"(x[I]), "n"(I));
    if constexpr (BIAS) {
      float z;
      asm("v_add_f32_dpp %0, %2, %3 row_newbcast:%4 row_mask:0xf bank_mask:0xf"
          : "=v"(z), "+s"(tok)
          : "v"(b), "v"(y), "n"(I));
      y = z;
    }
    x[I] = y;
    scale_row<I + 1, BIAS>(x, s, b, tok);
  }
}

template <int K, typename TW, bool BIAS, bool RELU, bool RESID>
__global__ __launch_bounds__(kThreads, 2) void gemm_stream_kernel(StreamArgs g) {
  using Lay = StreamLayout<K>;
  constexpr int KS = K / 16;  // MFMA k-steps
  extern __shared__ __attribute__((aligned(1024))) unsigned char smem[];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int y = blockIdx.x >> 3;
  const int slice = y % g.slices;
  const int group = (y / g.slices) * 8 + (blockIdx.x & 7);
  if (group >= g.ntiles) return;
  // Column chunks of 64 are dealt across slices: wave w of slice s takes
  // chunk (3 - w) * slices + s, so each workgroup holds one chunk from each
  // quarter of the columns and every workgroup carries the same mix of
  // epilogue work. For the attention projection the loader waves get the
  // gate and v chunks, the storer waves k and q.
  const int wn = 64 * ((3 - wave) * g.slices + slice);  // this wave's first column

  // Per-column scale and bias: accumulator element v of column block cb
  // belongs to column wn + 32 cb + 8 (v / 4) + 4 (lane / 32) + v % 4, so lane
  // l keeps the factor of element v = l % 16 for its half of the wave.
  // Without a scale the registers hold 1, an exact no-op.
  float ts[2], tb[2];
#pragma unroll
  for (int cb = 0; cb < 2; cb++) {
    const int n = wn + 32 * cb + 8 * ((lane & 15) >> 2) + 4 * (lane >> 5) + (lane & 3);
    ts[cb] = (g.flags & AFHIP_EPILOGUE_SCALE) && n < g.N ? g.scale[n] : 1.0f;
    tb[cb] = BIAS && n < g.N ? g.bias[n] : 0.0f;
  }

  // W[n][k] fragments: lane -> column wn + 32 cb + lane % 32, k = 16 s + 8 (lane / 32).
  half8 wf[2][KS];
  const TW* W = reinterpret_cast<const TW*>(g.w);
#pragma unroll
  for (int cb = 0; cb < 2; cb++) {
    const int n = wn + 32 * cb + (lane & 31);
#pragma unroll
    for (int s = 0; s < KS; s++) {
      if (n < g.N) {
        wf[cb][s] = load_w8<TW>(W + (int64_t)n * g.ldw + 16 * s + 8 * (lane >> 5));
      } else {
#pragma unroll
        for (int e = 0; e < 8; e++) wf[cb][s][e] = (half_t)0.0f;
      }
    }
  }
  wait_vmcnt<0>();  // weights in hand before the tile loads queue behind them

  const uint32_t lds0 = (uint32_t)reinterpret_cast<uintptr_t>(smem);
  // A tile's loads: loader wave w issues wave-level load q = w + 2 i for
  // i < LPW, filling stage rows [q * ROWS_PER_LOAD, +ROWS_PER_LOAD); the lane
  // fetches global chunk slot ^ (row & 7) into its slot. Rows past the tile's
  // valid ones fall past the resource and load zeros.
  auto tile_rsrc = [&](int tile) {
    const int row0 = tile * kBM;
    const int rows = min(kBM, g.M - row0);
    return make_rsrc(g.a + (int64_t)row0 * g.lda, (uint32_t)((int64_t)rows * g.lda * 2));
  };
  auto load_offset = [&](int i) {
    const int q = wave + kLoaders * i;
    const int row = q * Lay::ROWS_PER_LOAD + lane / Lay::SLOTS;
    const int chunk = (lane % Lay::SLOTS) ^ (row & 7);
    return (uint32_t)(row * g.lda * 2 + 16 * chunk);
  };
  auto issue = [&](int tile, int stage) {  // loader waves only
    const int32x4_t ra = tile_rsrc(tile);
#pragma unroll
    for (int i = 0; i < Lay::LPW; i++)
      dma16(ra, lds0 + stage * Lay::STAGE + (wave + kLoaders * i) * 1024, load_offset(i));
  };

  unsigned char* const ost = smem + Lay::OUT;
  const bool loader = wave < kLoaders;
  // k-step s reads chunk 2 s + h of row p (h = lane / 32) at slot
  // (2 s + h) ^ (p & 7) = 2 (s & ~3) + [2 ((s & 3) ^ (p >> 1 & 3)) + (h ^ (p & 1))]:
  // four lane addresses plus immediate offsets.
  const int xbase = (lane & 31) * Lay::RB + 16 * ((lane >> 5) ^ (lane & 1));
  const int xswz = 32 * ((lane >> 1) & 3);

  // Storer waves: a staged tile's 32 rows of 512 bytes, two rows per
  // wave-level store, kPer stores per storer wave. Row r keeps 16-byte chunk
  // c at slot c ^ (r & 7); staging chunk c belongs to wave c / 8. A store
  // that should not happen gets an offset past the resource and is dropped,
  // so the code has no branch.
  constexpr int kPer = kBM / 2 / (kWaves - kLoaders);
  auto store_rsrc = [&](int tile) {
    const int row0 = tile * kBM;
    const int rows = min(kBM, g.M - row0);
    return __builtin_amdgcn_make_buffer_rsrc(g.c + (int64_t)row0 * g.ldc, 0, (int)((int64_t)rows * g.ldc * 2),
                                             0x00020000);
  };
  const int scol = 64 * ((3 - ((lane & 31) >> 3)) * g.slices + slice) + 8 * (lane & 7);
  auto part_offset = [&](int i, bool on) {
    const int r = 2 * ((wave - kLoaders) * kPer + i) + (lane >> 5);
    return on && scol < g.N ? (uint32_t)(r * g.ldc * 2 + 2 * scol) : kOutOfRange;
  };
  auto store_part = [&](__amdgpu_buffer_rsrc_t rc, int buf, int i, bool on, const u32x4& old) {
    const int c = lane & 31;
    const int r = 2 * ((wave - kLoaders) * kPer + i) + (lane >> 5);
    u32x4 v = *reinterpret_cast<const u32x4*>(ost + buf * Lay::OBUF + r * Lay::OROW + 16 * (c ^ (r & 7)));
    if constexpr (RESID) {
      half8 h = __builtin_bit_cast(half8, v);
      const half8 o = __builtin_bit_cast(half8, old);
#pragma unroll
      for (int e = 0; e < 8; e++) h[e] = (half_t)((float)o[e] + (float)h[e]);
      v = __builtin_bit_cast(u32x4, h);
    }
    __builtin_amdgcn_raw_buffer_store_b128(v, rc, part_offset(i, on), 0, 0);
    stores_read(v);
  };
  // The old values under a storer's part of a tile (zeros past the resource).
  auto load_part = [&](__amdgpu_buffer_rsrc_t rc, int i, bool on) {
    return __builtin_amdgcn_raw_buffer_load_b128(rc, part_offset(i, on), 0, 0);
  };

  // The persistent loop, software-pipelined: tile t's MFMAs, tile t-1's
  // epilogue and the wave's memory duty (a loader issues tile t+2's loads, a
  // storer writes out tile t-2) are one straight-line block, so the matrix,
  // vector and memory pipes overlap. The wave's attention mode and its duty
  // are template arguments of the loop, which keeps that block free of
  // branches.
  auto run = [&](auto mode_tag, auto loader_tag) {
    constexpr int MODE = decltype(mode_tag)::value;
    constexpr bool LOADER = decltype(loader_tag)::value;
    int tok = 0;
    auto epilogue = [&](floatx16 (&acc)[2], int buf) {
      const int p = lane & 31;
      unsigned char* const ob = ost + buf * Lay::OBUF + p * Lay::OROW + 8 * (lane >> 5);
#pragma unroll
      for (int cb = 0; cb < 2; cb++) {
        floatx16& v = acc[cb];  // transformed in place: the tile's accumulators die here
        scale_row<0, BIAS>(v, ts[cb], tb[cb], tok);
#pragma unroll
        for (int i = 0; i < 16; i++) {
          if constexpr (MODE == kGate) v[i] = sigmoidf_(v[i]);
          if constexpr (MODE == kQuery) v[i] *= g.q_scale;
          if constexpr (RELU) v[i] = fmaxf(v[i], 0.0f);
        }
#pragma unroll
        for (int g4 = 0; g4 < 4; g4++) {
          // Columns wn + 32 cb + 8 g4 + 4 (lane / 32) + e: staging chunk
          // 8 wave + 4 cb + g4, half lane / 32.
          const int chunk = 8 * wave + 4 * cb + g4;
          half4 h;
#pragma unroll
          for (int e = 0; e < 4; e++) h[e] = (half_t)v[4 * g4 + e];
          *reinterpret_cast<half4*>(ob + 16 * (chunk ^ (p & 7))) = h;
        }
      }
    };

    floatx16 prev[2];
#pragma unroll
    for (int cb = 0; cb < 2; cb++)
#pragma unroll
      for (int v = 0; v < 16; v++) prev[cb][v] = 0.0f;
    // A storer's old values (adding into the output): part i holds the tile
    // it stores this pass until that store is formed, then is read again for
    // the tile whose epilogue runs this pass.
    u32x4 rcur[kPer];
#pragma unroll
    for (int i = 0; i < kPer; i++) rcur[i] = u32x4{0u, 0u, 0u, 0u};
    int tile = group;
    if constexpr (LOADER) {
      issue(tile, 0);
      if (tile + g.groups < g.ntiles) issue(tile + g.groups, 1);
    }
    // Pass `it` computes tile it's products and tile it-1's epilogue into
    // staging buffer it & 1, while the storers write out buffer (it-1) & 1
    // (tile it-2) from the pass before. One barrier per pass: it publishes the
    // landed tile and the finished buffer, and retires the oldest stage.
    int it = 0;
    for (; tile < g.ntiles; it++, tile += g.groups) {
      const int stage = it % kStages;
      // The tile has landed once only the next tile's loads are pending.
      if constexpr (LOADER) {
        if (tile + g.groups < g.ntiles) wait_vmcnt<Lay::LPW>();
        else wait_vmcnt<0>();
      }
      block_barrier();
      // A loader's loads for tile it+2 (LPW == KS / 2: one per two k-steps)
      // and a storer's stores of tile it-2 (kPer per pass) ride along the
      // MFMAs, so a stalled issue overlaps matrix work.
      const int fill = LOADER && tile + 2 * g.groups < g.ntiles;
      const int32x4_t rn = tile_rsrc(tile + 2 * g.groups);
      const uint32_t ln = lds0 + ((it + 2) % kStages) * Lay::STAGE + wave * 1024;
      const bool drain = it >= 2;
      const __amdgpu_buffer_rsrc_t rc = store_rsrc(drain ? tile - 2 * g.groups : tile);
      const bool ahead = it >= 1;
      const __amdgpu_buffer_rsrc_t rp = store_rsrc(ahead ? tile - g.groups : tile);
      const int sbuf = (it - 1) & 1;

      floatx16 cur[2];
#pragma unroll
      for (int cb = 0; cb < 2; cb++)
#pragma unroll
        for (int v = 0; v < 16; v++) cur[cb][v] = 0.0f;
      const unsigned char* st = smem + stage * Lay::STAGE + xbase;
#pragma unroll
      for (int s = 0; s < KS; s++) {
        if (s % 2 == 0) {
          if constexpr (LOADER) {
            dma16_if(rn, ln + kLoaders * (s / 2) * 1024, load_offset(s / 2), fill);
          } else {
#pragma unroll
            for (int j = 0; j < kPer / (KS / 2); j++) {
              const int i = (s / 2) * (kPer / (KS / 2)) + j;
              store_part(rc, sbuf, i, drain, rcur[i]);
              if constexpr (RESID) rcur[i] = load_part(rp, i, ahead);
            }
          }
        }
        const half8 xf = *reinterpret_cast<const half8*>(st + ((32 * (s & 3)) ^ xswz) + 128 * (s >> 2));
        cur[0] = mfma_f16(wf[0][s], xf, cur[0]);
        cur[1] = mfma_f16(wf[1][s], xf, cur[1]);
      }
      epilogue(prev, it & 1);  // tile it-1 (on the first pass, zeros nobody stores)
#pragma unroll
      for (int cb = 0; cb < 2; cb++) prev[cb] = cur[cb];
    }
    // Drain: tile it-2 waits in buffer (it-1) & 1, tile it-1 in the accumulators.
    block_barrier();
    if constexpr (!LOADER) {
      if (it >= 2) {
        const __amdgpu_buffer_rsrc_t rc = store_rsrc(tile - 2 * g.groups);
#pragma unroll
        for (int i = 0; i < kPer; i++) store_part(rc, (it - 1) & 1, i, true, rcur[i]);
      }
    }
    epilogue(prev, it & 1);
    block_barrier();
    if constexpr (!LOADER) {
      const __amdgpu_buffer_rsrc_t rc = store_rsrc(tile - g.groups);
      if constexpr (RESID) {
#pragma unroll
        for (int i = 0; i < kPer; i++) rcur[i] = load_part(rc, i, true);
      }
#pragma unroll
      for (int i = 0; i < kPer; i++) store_part(rc, it & 1, i, true, rcur[i]);
    }
  };

  const int mode = (g.flags & AFHIP_EPILOGUE_ATTENTION) ? wn / g.head_cols : -1;
  using Load = std::integral_constant<bool, true>;
  using Store = std::integral_constant<bool, false>;
  if (loader) {
    if (mode == 3) run(std::integral_constant<int, kGate>{}, Load{});
    else if (mode == 0) run(std::integral_constant<int, kQuery>{}, Load{});
    else run(std::integral_constant<int, kPlain>{}, Load{});
  } else {
    if (mode == 3) run(std::integral_constant<int, kGate>{}, Store{});
    else if (mode == 0) run(std::integral_constant<int, kQuery>{}, Store{});
    else run(std::integral_constant<int, kPlain>{}, Store{});
  }
}

template <int K, typename TW, bool BIAS, bool RELU, bool RESID>
int launch_k(const StreamArgs& a, const char* label, hipStream_t s) {
  auto kernel = gemm_stream_kernel<K, TW, BIAS, RELU, RESID>;
  constexpr size_t shared = StreamLayout<K>::BYTES;
  if (int st = allow_lds((const void*)kernel, shared)) return st;
  return launch(label, kernel, dim3((unsigned)(a.groups * a.slices)), dim3(kThreads), shared, s, a);
}

template <int K, typename TW>
int dispatch_epi(const StreamArgs& a, bool bias, bool relu, bool resid, const char* label, hipStream_t s) {
  // Adding into the output comes only with a bias and no ReLU (the attention
  // output), at K <= 128: at K = 256 the weights leave no registers for the
  // old values.
  if constexpr (K <= 128) {
    if (resid) return launch_k<K, TW, true, false, true>(a, label, s);
  }
  if (bias)
    return relu ? launch_k<K, TW, true, true, false>(a, label, s) : launch_k<K, TW, true, false, false>(a, label, s);
  return relu ? launch_k<K, TW, false, true, false>(a, label, s) : launch_k<K, TW, false, false, false>(a, label, s);
}

int dispatch_k(const StreamArgs& a, int K, bool q8, bool bias, bool relu, bool resid, const char* label,
               hipStream_t s) {
  switch (K) {
    case 64:
      return q8 ? dispatch_epi<64, int8_t>(a, bias, relu, resid, label, s)
                : dispatch_epi<64, half_t>(a, bias, relu, resid, label, s);
    case 128:
      return q8 ? dispatch_epi<128, int8_t>(a, bias, relu, resid, label, s)
                : dispatch_epi<128, half_t>(a, bias, relu, resid, label, s);
    default:
      return q8 ? dispatch_epi<256, int8_t>(a, bias, relu, resid, label, s)
                : dispatch_epi<256, half_t>(a, bias, relu, resid, label, s);
  }
}

}  // namespace

bool stream_shape_ok(const GemmTypes& t, int64_t M, int64_t N, int64_t K, int batch) {
  if (t.precision != AFHIP_PRECISION_F16 || t.a_dtype != AFHIP_F16 || t.c_dtype != AFHIP_F16) return false;
  if (t.b_dtype != AFHIP_F16 && t.b_dtype != AFHIP_I8) return false;
  return batch == 1 && M > 0 && N % 64 == 0 && N > 0 && (K == 64 || K == 128 || K == 256);
}

bool stream_eligible(const GemmArgs& g, const GemmTypes& t) {
  if (!stream_shape_ok(t, g.M, g.N, g.K, g.batch)) return false;
  if (g.a_row_contiguous || g.c_column_major) return false;
  const uint32_t allowed = AFHIP_EPILOGUE_SCALE | AFHIP_EPILOGUE_BIAS | AFHIP_EPILOGUE_ATTENTION | AFHIP_EPILOGUE_RELU;
  if (g.flags & ~allowed) return false;
  // Each wave's 64 columns must lie in one attention block (q, k, v or gate).
  if ((g.flags & AFHIP_EPILOGUE_ATTENTION) && (g.head_cols <= 0 || g.head_cols % 64)) return false;
  auto aligned = [](const void* p, uintptr_t n) { return (reinterpret_cast<uintptr_t>(p) & (n - 1)) == 0; };
  if (!aligned(g.a, 16) || !aligned(g.c, 16) || !aligned(g.b, t.b_dtype == AFHIP_I8 ? 8 : 16)) return false;
  if (g.lda % 8 || g.ldb % 8 || g.ldc % 8 || g.lda < g.K || g.ldb < g.K || g.ldc < g.N) return false;
  // Byte offsets within one 64-row tile fit the 32-bit buffer offsets.
  return (int64_t)kBM * std::max(g.lda, g.ldc) * 2 < (int64_t)kOutOfRange;
}

int run_gemm_stream(const GemmArgs& g, const GemmTypes& t, const char* label, hipStream_t s, bool add_f16) {
  AFHIP_REQUIRE(stream_eligible(g, t), "operands the STREAM kernel cannot take");
  AFHIP_REQUIRE(!add_f16 || ((g.flags & AFHIP_EPILOGUE_BIAS) && !(g.flags & (AFHIP_EPILOGUE_RELU | AFHIP_EPILOGUE_ATTENTION)) &&
                              g.K <= 128),
                "the STREAM kernel adds into its output only after a plain bias epilogue, at K <= 128");
  StreamArgs a;
  a.a = reinterpret_cast<const half_t*>(g.a);
  a.w = g.b;
  a.c = reinterpret_cast<half_t*>(g.c);
  a.scale = g.scale;
  a.bias = g.bias;
  a.M = g.M;
  a.N = g.N;
  a.lda = g.lda;
  a.ldw = g.ldb;
  a.ldc = g.ldc;
  a.flags = g.flags;
  a.head_cols = g.head_cols;
  a.q_scale = g.q_scale;
  a.ntiles = (int)ceil_div(g.M, kBM);
  a.slices = (int)ceil_div(g.N, kBN);
  const int cus = device_cu_count() > 0 ? device_cu_count() : 256;
  // Row-tile groups: a multiple of 8 (the XCD count) giving about two
  // workgroups per CU, and no more groups than tiles need.
  int groups = (int)round_up(std::max<int64_t>(1, 2 * cus / a.slices), 8);
  groups = std::min<int>(groups, (int)round_up(a.ntiles, 8));
  a.groups = groups;
  const bool q8 = t.b_dtype == AFHIP_I8;
  const bool bias = g.flags & AFHIP_EPILOGUE_BIAS, relu = g.flags & AFHIP_EPILOGUE_RELU;
  return dispatch_k(a, g.K, q8, bias, relu, add_f16, label, s);
}

}  // namespace afhip
