// Triangle multiplication, f16 precision at c_z = c_hidden = 128 (AlphaFold's
// widths): the projection and output kernels written for HBM throughput.
//
// Both are persistent: a grid of at most two workgroups per CU walks 64-row
// tiles. Each of the eight waves keeps its 32 output channels' weights in
// VGPRs for the whole kernel (2 x 8 half8 fragments = 64 VGPRs), so the MFMA
// loop reads only LDS; the next tile's global loads are issued before the
// current tile's MFMAs and consumed after them.
//
// tri_project_f16: wave w projects operand (w >> 2) (a or b), channels
// [32 * (w & 3), +32), both projection and gate. The MFMA is issued as
// W (A operand) x zn^T (B operand), so the accumulator comes out channel-major:
// lane l holds pair (l % 32) of 16 channels, and 32 lanes store 32 consecutive
// pairs of one channel of the [c][row] operand.
//
// tri_output_f16: wave w computes output channels [32 * (w & 3), +32) for
// pairs [32 * (w >> 2), +32) of the tile, both linearZ (from the normalised
// contraction) and linearG (from the normalised z), and stores
// (p + bz) * sigmoid(g + bg) along the pair's 128 output channels.
#include <algorithm>

#include "gemm.h"
#include "triangle_fast.h"

namespace afhip {

namespace {

constexpr int kTile = 64;        // rows (pairs) per tile
constexpr int kC = 128;          // c_z = c_hidden
constexpr int kPitch = kC + 8;   // halves; 272-byte rows keep 16-byte alignment
constexpr int kThreads = 512;

template <typename T> struct Raw16;  // 16 consecutive elements in registers
template <> struct Raw16<half_t> {
  uint4 v[2];
  __device__ void load(const half_t* p) {
    v[0] = reinterpret_cast<const uint4*>(p)[0];
    v[1] = reinterpret_cast<const uint4*>(p)[1];
  }
  __device__ void zero() { v[0] = v[1] = make_uint4(0, 0, 0, 0); }
  __device__ float get(int e) const { return (float)reinterpret_cast<const half_t*>(v)[e]; }
};
template <> struct Raw16<float> {
  uint4 v[4];
  __device__ void load(const float* p) {
#pragma unroll
    for (int i = 0; i < 4; i++) v[i] = reinterpret_cast<const uint4*>(p)[i];
  }
  __device__ void zero() {
#pragma unroll
    for (int i = 0; i < 4; i++) v[i] = make_uint4(0, 0, 0, 0);
  }
  __device__ float get(int e) const { return reinterpret_cast<const float*>(v)[e]; }
};

// LayerNorm of one row held by 8 consecutive lanes (16 channels each),
// written as f16 to dst (16 halves). Two-pass mean / variance in f32.
template <typename T>
__device__ __forceinline__ void normalize16(const Raw16<T>& raw, const float* w, const float* b, float eps,
                                            half_t* dst) {
  float x[16];
  float s = 0.0f;
#pragma unroll
  for (int e = 0; e < 16; e++) {
    x[e] = raw.get(e);
    s += x[e];
  }
  s += __shfl_xor(s, 1);
  s += __shfl_xor(s, 2);
  s += __shfl_xor(s, 4);
  const float mean = s * (1.0f / kC);
  float v = 0.0f;
#pragma unroll
  for (int e = 0; e < 16; e++) {
    const float d = x[e] - mean;
    v += d * d;
  }
  v += __shfl_xor(v, 1);
  v += __shfl_xor(v, 2);
  v += __shfl_xor(v, 4);
  const float rstd = 1.0f / sqrtf(v * (1.0f / kC) + eps);
  half8 h0, h1;
#pragma unroll
  for (int e = 0; e < 8; e++) {
    h0[e] = (half_t)((x[e] - mean) * rstd * w[e] + b[e]);
    h1[e] = (half_t)((x[e + 8] - mean) * rstd * w[e + 8] + b[e + 8]);
  }
  reinterpret_cast<half8*>(dst)[0] = h0;
  reinterpret_cast<half8*>(dst)[1] = h1;
}

__device__ __forceinline__ int pair_of(int r, int L, bool incoming) {
  if (!incoming) return r;
  const int j = r / L;
  return (r - j * L) * L + j;
}

template <typename ZT>
__global__ __launch_bounds__(kThreads, 1) void tri_project_f16_kernel(FastProjectArgs a) {
  __shared__ __attribute__((aligned(16))) half_t zn[2][kTile * kPitch];
  __shared__ float ln[2 * kC];
  __shared__ float bias[4 * kC];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int o = wave >> 2;                 // 0: a (left), 1: b (right)
  const int hb = 32 * (wave & 3);          // channel block
  const int ntiles = (a.P + kTile - 1) / kTile;

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

  // Normaliser role: row tid / 8, channels [16 (tid % 8), +16).
  const int nrow = tid >> 3, nchunk = (tid & 7) * 16;
  const ZT* z = reinterpret_cast<const ZT*>(a.z);
  Raw16<ZT> raw;
  auto load_tile = [&](int tile) {
    const int r = tile * kTile + nrow;
    if (r < a.P) raw.load(z + (size_t)pair_of(r, a.L, a.incoming) * kC + nchunk);
    else raw.zero();
  };

  int tile = blockIdx.x;
  if (tile < ntiles) load_tile(tile);
  __syncthreads();  // ln and bias staged
  int cur = 0;
  if (tile < ntiles) normalize16(raw, ln + nchunk, ln + kC + nchunk, a.eps, &zn[0][nrow * kPitch + nchunk]);
  __syncthreads();

  half_t* out = o == 0 ? a.out_a : a.out_b;
  const float* bp = bias + (2 * o) * kC;
  const float* bg = bias + (2 * o + 1) * kC;
  for (; tile < ntiles; tile += gridDim.x) {
    const int next = tile + gridDim.x;
    if (next < ntiles) load_tile(next);
    const half_t* zt = zn[cur];
#pragma unroll
    for (int sub = 0; sub < 2; sub++) {
      floatx16 accp, accg;
#pragma unroll
      for (int v = 0; v < 16; v++) accp[v] = accg[v] = 0.0f;
      const half_t* zrow = zt + (sub * 32 + (lane & 31)) * kPitch + 8 * (lane >> 5);
#pragma unroll
      for (int s = 0; s < 8; s++) {
        const half8 zf = *reinterpret_cast<const half8*>(zrow + 16 * s);
        accp = mfma_f16(fp[s], zf, accp);
        accg = mfma_f16(fg[s], zf, accg);
      }
      const int r = tile * kTile + sub * 32 + (lane & 31);
      if (r < a.P) {
        const float m = a.mask[pair_of(r, a.L, a.incoming)];
#pragma unroll
        for (int v = 0; v < 16; v++) {
          const int c = hb + mfma_row(v, lane);
          const float val = m * (accp[v] + bp[c]) * sigmoidf_(accg[v] + bg[c]);
          out[(size_t)c * a.cstride + r] = (half_t)val;
        }
      }
    }
    if (next < ntiles) normalize16(raw, ln + nchunk, ln + kC + nchunk, a.eps, &zn[cur ^ 1][nrow * kPitch + nchunk]);
    __syncthreads();
    cur ^= 1;
  }
}

template <typename ZT, typename OT>
__global__ __launch_bounds__(kThreads, 1) void tri_output_f16_kernel(FastOutputArgs a) {
  constexpr int xpitch = kTile + 2;  // halves; odd word stride spreads the column reads over banks
  __shared__ __attribute__((aligned(16))) half_t xt[kC * xpitch];
  __shared__ __attribute__((aligned(16))) half_t hn[kTile * kPitch];
  __shared__ __attribute__((aligned(16))) half_t gn[kTile * kPitch];
  __shared__ float ln[4 * kC];  // ln_out w, ln_out b, ln_in w, ln_in b

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nt = 32 * (wave & 3), rh = 32 * (wave >> 2);
  const int ntiles = (a.pairs + kTile - 1) / kTile;
  for (int i = tid; i < 4 * kC; i += kThreads) {
    const int k = i / kC, c = i % kC;
    ln[i] = k == 0 ? a.ln_out_w[c] : k == 1 ? a.ln_out_b[c] : k == 2 ? a.ln_in_w[c] : a.ln_in_b[c];
  }

  const half_t* wz = a.w_z + (size_t)(nt + (lane & 31)) * kC + 8 * (lane >> 5);
  const half_t* wgp = a.w_g + (size_t)(nt + (lane & 31)) * kC + 8 * (lane >> 5);
  half8 fz[8], fg[8];
#pragma unroll
  for (int s = 0; s < 8; s++) {
    fz[s] = *reinterpret_cast<const half8*>(wz + 16 * s);
    fg[s] = *reinterpret_cast<const half8*>(wgp + 16 * s);
  }
  const int n = nt + (lane & 31);
  const float bz = a.b_z[n], bgv = a.b_g[n];

  // Loader roles: contraction tile as [channel tid / 4][16 pairs], z tile as
  // [pair tid / 8][16 channels].
  const int xc = tid >> 2, xq = (tid & 3) * 16;
  const int zq = tid >> 3, zc = (tid & 7) * 16;
  const half_t* X = a.contracted;
  const ZT* z = reinterpret_cast<const ZT*>(a.z);
  Raw16<half_t> xraw;
  Raw16<ZT> zraw;
  auto load_tile = [&](int tile) {
    const int q0 = tile * kTile;
    if (q0 + xq + 16 <= a.pairs) {
      xraw.load(X + (size_t)xc * a.bstride + q0 + xq);
    } else {
      half_t tmp[16];
#pragma unroll
      for (int e = 0; e < 16; e++) tmp[e] = q0 + xq + e < a.pairs ? X[(size_t)xc * a.bstride + q0 + xq + e] : (half_t)0.0f;
      xraw.v[0] = reinterpret_cast<uint4*>(tmp)[0];
      xraw.v[1] = reinterpret_cast<uint4*>(tmp)[1];
    }
    if (q0 + zq < a.pairs) zraw.load(z + (size_t)(a.pair0 + q0 + zq) * kC + zc);
    else zraw.zero();
  };

  int tile = blockIdx.x;
  if (tile < ntiles) load_tile(tile);
  __syncthreads();  // ln staged
  OT* out = reinterpret_cast<OT*>(a.out);
  for (; tile < ntiles; tile += gridDim.x) {
    const int q0 = tile * kTile;
    // Raw contraction into LDS, channel-major; z normalised straight from registers.
    {  // 132-byte rows are 4-byte aligned only: eight dword stores
      uint32_t* dst = reinterpret_cast<uint32_t*>(&xt[xc * xpitch + xq]);
      const uint32_t* src = reinterpret_cast<const uint32_t*>(xraw.v);
#pragma unroll
      for (int i = 0; i < 8; i++) dst[i] = src[i];
    }
    normalize16(zraw, ln + 2 * kC + zc, ln + 3 * kC + zc, a.eps, &gn[zq * kPitch + zc]);
    __syncthreads();
    {  // hidden LayerNorm: pair zq, channels [zc, zc + 16) read down the columns of xt
      Raw16<half_t> col;
      half_t tmp[16];
#pragma unroll
      for (int e = 0; e < 16; e++) tmp[e] = xt[(zc + e) * xpitch + zq];
      col.v[0] = reinterpret_cast<uint4*>(tmp)[0];
      col.v[1] = reinterpret_cast<uint4*>(tmp)[1];
      normalize16(col, ln + zc, ln + kC + zc, a.eps, &hn[zq * kPitch + zc]);
    }
    const int next = tile + gridDim.x;
    if (next < ntiles) load_tile(next);
    __syncthreads();
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
#pragma unroll
    for (int v = 0; v < 16; v++) {
      const int q = q0 + rh + mfma_row(v, lane);
      if (q < a.pairs) {
        float y = (accz[v] + bz) * sigmoidf_(accg[v] + bgv);
        const size_t at = (size_t)(a.pair0 + q) * kC + n;
        if (a.residual) y += (float)out[at];
        out[at] = (OT)y;
      }
    }
    __syncthreads();
  }
}

int grid_for(int tiles) {
  const int cus = device_cu_count() > 0 ? device_cu_count() : 256;
  return std::max(1, std::min(tiles, cus));
}

}  // namespace

bool triangle_fast_eligible(const afhip_triangle_desc& d) {
  return d.precision == AFHIP_PRECISION_F16 && d.c_z == kC && d.c_hidden == kC;
}

int launch_triangle_project_f16(const FastProjectArgs& a, int pair_dtype, hipStream_t s) {
  const int tiles = (int)ceil_div(a.P, kTile);
  if (pair_dtype == AFHIP_F16)
    return launch("triangle.project", tri_project_f16_kernel<half_t>, dim3(grid_for(tiles)), dim3(kThreads), 0, s, a);
  return launch("triangle.project", tri_project_f16_kernel<float>, dim3(grid_for(tiles)), dim3(kThreads), 0, s, a);
}

int launch_triangle_output_f16(const FastOutputArgs& a, int pair_dtype, int out_dtype, hipStream_t s) {
  const int tiles = (int)ceil_div(a.pairs, kTile);
  dim3 g(grid_for(tiles)), b(kThreads);
  if (pair_dtype == AFHIP_F16) {
    if (out_dtype == AFHIP_F32) return launch("triangle.output", tri_output_f16_kernel<half_t, float>, g, b, 0, s, a);
    return launch("triangle.output", tri_output_f16_kernel<half_t, half_t>, g, b, 0, s, a);
  }
  if (out_dtype == AFHIP_F32) return launch("triangle.output", tri_output_f16_kernel<float, float>, g, b, 0, s, a);
  return launch("triangle.output", tri_output_f16_kernel<float, half_t>, g, b, 0, s, a);
}

}  // namespace afhip
