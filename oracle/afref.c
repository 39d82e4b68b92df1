/*
 * afref — CPU restatement of alphafold2-webgpu's reference arithmetic for the
 * GEMM / triangle-multiplication / outer-product-mean path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker the parity tests,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg compare the HIP
 * library against. Nothing in the product (libafhip, the afhip Python
 * package, the N-API addon) links, loads or calls it.
 *
 * The reference's CPU code is TypeScript evaluated in JavaScript doubles and
 * stored into Float32Array after every operation. Each function below keeps
 * that discipline: accumulate in double, round to float where the reference
 * stores into a Float32Array. Build with -ffp-contract=off so no product is
 * fused into an add the reference performs separately.
 *
 * Each function cites the reference file:line whose behaviour it restates
 * (paths relative to the alphafold2-webgpu checkout).
 */
#ifdef _OPENMP
#include <omp.h>
#endif
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define EXPORT __attribute__((visibility("default")))

/* ------------------------------------------------------------------------ */
/* f16 codec                                                                 */
/* ------------------------------------------------------------------------ */

/* src/runtime/float16.ts:5-29 (numberToFloat16). Round-to-nearest-even for
 * normal results. The subnormal branch shifts the mantissa right before it
 * rounds, dropping bits a sticky bit would keep; that is restated as written
 * (it differs from IEEE RNE only for subnormal halves on an exact-tie
 * remainder). */
EXPORT uint16_t afref_f32_to_f16(float value) {
  uint32_t bits;
  memcpy(&bits, &value, 4);
  uint32_t sign = (bits >> 16) & 0x8000u;
  int32_t exponent = (int32_t)((bits >> 23) & 0xffu) - 127 + 15;
  uint32_t mantissa = bits & 0x7fffffu;
  if (((bits >> 23) & 0xffu) == 0xffu) return (uint16_t)(sign | (mantissa == 0 ? 0x7c00u : 0x7e00u));
  if (exponent >= 0x1f) return (uint16_t)(sign | 0x7c00u);
  if (exponent <= 0) {
    if (exponent < -10) return (uint16_t)sign;
    mantissa = (mantissa | 0x800000u) >> (uint32_t)(1 - exponent);
    return (uint16_t)(sign | ((mantissa + 0x0fffu + ((mantissa >> 13) & 1u)) >> 13));
  }
  mantissa += 0x0fffu + ((mantissa >> 13) & 1u);
  if (mantissa & 0x800000u) {
    mantissa = 0;
    exponent += 1;
    if (exponent >= 0x1f) return (uint16_t)(sign | 0x7c00u);
  }
  return (uint16_t)(sign | ((uint32_t)exponent << 10) | (mantissa >> 13));
}

/* src/reference/dtype.ts:28-35 (float16ToNumber). */
EXPORT float afref_f16_to_f32(uint16_t bits) {
  double sign = (bits & 0x8000u) == 0 ? 1.0 : -1.0;
  int exponent = (bits >> 10) & 0x1f;
  int fraction = bits & 0x03ff;
  if (exponent == 0) return (float)(fraction == 0 ? sign * 0.0 : sign * ldexp(1.0, -14) * (fraction / 1024.0));
  if (exponent == 0x1f) return fraction == 0 ? (float)(sign * INFINITY) : NAN;
  return (float)(sign * ldexp(1.0, exponent - 15) * (1.0 + fraction / 1024.0));
}

/* src/runtime/float16.ts:31-35 (float32ToFloat16Array). */
EXPORT void afref_f32_to_f16_array(const float* values, uint16_t* out, size_t count) {
  for (size_t i = 0; i < count; i++) out[i] = afref_f32_to_f16(values[i]);
}

EXPORT void afref_f16_to_f32_array(const uint16_t* values, float* out, size_t count) {
  for (size_t i = 0; i < count; i++) out[i] = afref_f16_to_f32(values[i]);
}

/* ------------------------------------------------------------------------ */
/* int8 codecs                                                               */
/* ------------------------------------------------------------------------ */

/* tools/quantize-web-model.ts:98-119. Symmetric int8 over flat blocks of
 * `block` elements in storage order: scale = f16(max|w| / 127), a zero scale
 * decodes as 1, q = clamp(round(w / scale), -127, 127). Math.round rounds
 * halves toward +infinity, which floor(x + 0.5) restates. */
EXPORT void afref_q8_block_encode(const float* values, size_t count, int block,
                                  int8_t* codes, uint16_t* scales) {
  size_t blocks = (count + (size_t)block - 1) / (size_t)block;
  for (size_t b = 0; b < blocks; b++) {
    size_t start = b * (size_t)block;
    size_t end = start + (size_t)block < count ? start + (size_t)block : count;
    double maximum = 0.0;
    for (size_t i = start; i < end; i++) {
      double m = fabs((double)values[i]);
      if (m > maximum) maximum = m;
    }
    uint16_t scale_bits = afref_f32_to_f16((float)(maximum / 127.0));
    double scale = afref_f16_to_f32(scale_bits);
    if (scale == 0.0) scale = 1.0;
    scales[b] = scale_bits;
    for (size_t i = start; i < end; i++) {
      double q = floor((double)values[i] / scale + 0.5);
      if (q > 127.0) q = 127.0;
      if (q < -127.0) q = -127.0;
      codes[i] = (int8_t)q;
    }
  }
}

/* src/reference/dtype.ts:66-99 (readTensorRange, int8 branch): value number
 * start + i decodes as codes[start + i] * f32(scales[(start + i) / block]). */
EXPORT void afref_q8_block_decode(const int8_t* codes, const uint16_t* scales, int block,
                                  size_t start, size_t count, float* out) {
  for (size_t i = 0; i < count; i++) {
    size_t absolute = start + i;
    double scale = afref_f16_to_f32(scales[absolute / (size_t)block]);
    out[i] = (float)((double)codes[absolute] * scale);
  }
}

/* Per-output-channel dequantisation of a [K][N] int8 weight with an f32 scale
 * per column: w[k][n] = f32(q[k][n]) * scale[n], one correctly rounded f32
 * product. The reference has no such format (its bundle is block-64, see
 * above); this is the closed form the mixed-q8 GEMM path is held to. */
EXPORT void afref_q8_channel_decode(const int8_t* q, const float* scale, int K, int N, float* out) {
  for (int k = 0; k < K; k++)
    for (int n = 0; n < N; n++) {
      volatile float product = (float)q[(size_t)k * N + n] * scale[n];
      out[(size_t)k * N + n] = product;
    }
}

/* ------------------------------------------------------------------------ */
/* Seeded inputs                                                             */
/* ------------------------------------------------------------------------ */

/* splitmix64 (Steele, Lea, Flood 2014), the generator the benchmark inputs
 * are defined over. */
static uint64_t splitmix64_next(uint64_t* state) {
  uint64_t z = (*state += 0x9e3779b97f4a7c15ull);
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

/* Uniform double in [0, 1) from the top 53 bits. */
static double splitmix_uniform(uint64_t* state) {
  return (double)(splitmix64_next(state) >> 11) * (1.0 / 9007199254740992.0);
}

/* Normal(mean, variance) floats: splitmix64 then Box-Muller, both outputs of
 * a pair used in order. Variance, not standard deviation, as the benchmark
 * configurations state N(mu, v). */
EXPORT void afref_normal_f32(uint64_t seed, double mean, double variance, size_t count, float* out) {
  uint64_t state = seed;
  double sd = sqrt(variance);
  size_t i = 0;
  while (i < count) {
    double u1 = splitmix_uniform(&state);
    double u2 = splitmix_uniform(&state);
    if (u1 <= 0.0) u1 = 1.0 / 9007199254740992.0;
    double r = sqrt(-2.0 * log(u1));
    double t = 6.283185307179586 * u2;
    out[i++] = (float)(mean + sd * r * cos(t));
    if (i < count) out[i++] = (float)(mean + sd * r * sin(t));
  }
}

/* Uniform floats in [low, high). */
EXPORT void afref_uniform_f32(uint64_t seed, double low, double high, size_t count, float* out) {
  uint64_t state = seed;
  for (size_t i = 0; i < count; i++) out[i] = (float)(low + (high - low) * splitmix_uniform(&state));
}

/* Uniform integers in [low, high] inclusive, as int8 (weights of the q8 path). */
EXPORT void afref_uniform_i8(uint64_t seed, int low, int high, size_t count, int8_t* out) {
  uint64_t state = seed;
  uint64_t span = (uint64_t)(high - low + 1);
  for (size_t i = 0; i < count; i++) out[i] = (int8_t)(low + (int)(splitmix64_next(&state) % span));
}

/* src/testing/deterministic-input.ts:7-16 (generator): a mulberry32-style
 * 32-bit generator returning values in [0, 1). */
EXPORT void afref_mulberry_uniform(uint32_t seed, size_t count, double* out) {
  uint32_t state = seed;
  for (size_t i = 0; i < count; i++) {
    state += 0x6d2b79f5u;
    uint32_t value = state;
    value = (value ^ (value >> 15)) * (value | 1u);
    value ^= value + (value ^ (value >> 7)) * (value | 61u);
    out[i] = (double)(value ^ (value >> 14)) / 4294967296.0;
  }
}

/* test/gemm-half-precision.gpu.test.ts:44-50 and
 * src/runtime/gemm-selection.ts:307-313: an LCG stepped by 1664525 and
 * 1013904223 (mod 2^32), mapped to state / 2^32 - 0.5. */
EXPORT void afref_lcg_values(uint32_t seed, size_t count, float* out) {
  uint32_t state = seed;
  for (size_t i = 0; i < count; i++) {
    state = state * 1664525u + 1013904223u;
    out[i] = (float)((double)state / 4294967296.0 - 0.5);
  }
}

/* ------------------------------------------------------------------------ */
/* GEMM                                                                      */
/* ------------------------------------------------------------------------ */

/* test/gemm-half-precision.gpu.test.ts:52-68: A x W + bias summed in double,
 * A row-major [M][K], W [K][N]. bias may be NULL. */
EXPORT void afref_gemm_f64(const float* a, const float* w, const float* bias,
                           int M, int K, int N, double* out) {
  for (int m = 0; m < M; m++)
    for (int n = 0; n < N; n++) {
      double total = 0.0;
      for (int k = 0; k < K; k++) total += (double)a[(size_t)m * K + k] * (double)w[(size_t)k * N + n];
      out[(size_t)m * N + n] = total + (bias ? (double)bias[n] : 0.0);
    }
}

/* src/evoformer/transition.ts:91-138 (createLinearShader): output =
 * A[M][K] . W[K][N] + bias, max(., 0) when relu, added into out when residual.
 * The sum is kept in double and stored once. */
EXPORT void afref_linear(const float* a, const float* w, const float* bias, int M, int K, int N,
                         int relu, int residual, float* out) {
  for (int m = 0; m < M; m++)
    for (int n = 0; n < N; n++) {
      double total = 0.0;
      for (int k = 0; k < K; k++) total += (double)a[(size_t)m * K + k] * (double)w[(size_t)k * N + n];
      double stored = total + (bias ? (double)bias[n] : 0.0);
      if (relu && stored < 0.0) stored = 0.0;
      if (residual) stored += (double)out[(size_t)m * N + n];
      out[(size_t)m * N + n] = (float)stored;
    }
}

/* src/evoformer/attention.ts:497-589 (attentionProjectShader store): four
 * projections of X[M][K] by W_{q,k,v,g}[K][H*D]; q scaled by 1/sqrt(D),
 * g = sigmoid(x + gate_bias). w is [K][4*H*D], the four matrices side by side
 * as columns [q | k | v | g], which is the column order the fused dispatch
 * covers. Outputs are [M][H*D] each. */
EXPORT void afref_attention_project(const float* x, const float* w, const float* gate_bias,
                                    int M, int K, int HD, int D,
                                    float* q, float* kout, float* v, float* g) {
  int N = 4 * HD;
  double inv_sqrt = 1.0 / sqrt((double)D);
  for (int m = 0; m < M; m++)
    for (int n = 0; n < N; n++) {
      double total = 0.0;
      for (int k = 0; k < K; k++) total += (double)x[(size_t)m * K + k] * (double)w[(size_t)k * N + n];
      int matrix = n / HD;
      size_t index = (size_t)m * HD + (size_t)(n % HD);
      if (matrix == 0) q[index] = (float)(total * inv_sqrt);
      else if (matrix == 1) kout[index] = (float)total;
      else if (matrix == 2) v[index] = (float)total;
      else {
        double biased = total + (gate_bias ? (double)gate_bias[n % HD] : 0.0);
        g[index] = (float)(1.0 / (1.0 + exp(-biased)));
      }
    }
}

/* ------------------------------------------------------------------------ */
/* Threads                                                                   */
/* ------------------------------------------------------------------------ */

/* The triangle loops below split their outer (row or pair) loop over OpenMP
 * threads. Every stored value is still computed by one thread in the
 * reference's order, so any thread count gives the same bits; the count only
 * matters to bench.py's CPU baseline (one thread, then all cores). */
EXPORT void afref_set_threads(int threads) {
#ifdef _OPENMP
  omp_set_num_threads(threads > 0 ? threads : 1);
#else
  (void)threads;
#endif
}

EXPORT int afref_max_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

/* ------------------------------------------------------------------------ */
/* Triangle multiplication                                                   */
/* ------------------------------------------------------------------------ */

static double sigmoid(double value) { return 1.0 / (1.0 + exp(-value)); }

/* src/triangle/cpu-reference.ts:6-31 (normalizeRows). */
static void normalize_rows(const float* input, size_t rows, int channels, const float* weight,
                           const float* bias, double epsilon, float* output) {
#pragma omp parallel for schedule(static)
  for (size_t row = 0; row < rows; row++) {
    const float* x = input + row * (size_t)channels;
    double mean = 0.0;
    for (int c = 0; c < channels; c++) mean += (double)x[c];
    mean /= channels;
    double variance = 0.0;
    for (int c = 0; c < channels; c++) {
      double centered = (double)x[c] - mean;
      variance += centered * centered;
    }
    double inverse_std = 1.0 / sqrt(variance / channels + epsilon);
    for (int c = 0; c < channels; c++)
      output[row * (size_t)channels + c] =
          (float)(((double)x[c] - mean) * inverse_std * (double)weight[c] + (double)bias[c]);
  }
}

/* src/triangle/cpu-reference.ts:33-54 (project): weight is [out][in]. */
static void project(const float* input, size_t rows, int in_channels, int out_channels,
                    const float* weight, const float* bias, float* output) {
#pragma omp parallel for schedule(static)
  for (size_t row = 0; row < rows; row++)
    for (int o = 0; o < out_channels; o++) {
      double value = (double)bias[o];
      const float* wrow = weight + (size_t)o * in_channels;
      const float* x = input + row * (size_t)in_channels;
      for (int c = 0; c < in_channels; c++) value += (double)x[c] * (double)wrow[c];
      output[row * (size_t)out_channels + o] = (float)value;
    }
}

/* Offsets of the sixteen tensors in the packed weight array, in the order of
 * src/triangle/weights.ts:4-10 (ORDER). */
EXPORT void afref_triangle_weight_offsets(int cz, int ch, size_t offsets[17]) {
  size_t sizes[16] = {
      (size_t)cz, (size_t)cz,
      (size_t)ch * cz, (size_t)ch, (size_t)ch * cz, (size_t)ch,
      (size_t)ch * cz, (size_t)ch, (size_t)ch * cz, (size_t)ch,
      (size_t)ch, (size_t)ch,
      (size_t)cz * ch, (size_t)cz, (size_t)cz * cz, (size_t)cz};
  size_t at = 0;
  for (int i = 0; i < 16; i++) { offsets[i] = at; at += sizes[i]; }
  offsets[16] = at;
}

/* Triangle multiplication, both directions.
 *
 * direction 0 (outgoing): src/triangle/cpu-reference.ts:56-100,
 *   contracted[i][j][h] = sum_k a[i][k][h] * b[j][k][h].
 * direction 1 (incoming): the contraction of src/triangle/shaders.ts:452-495
 *   (AlphaFold's einsum "kjc,kic->ijc"), contracted[i][j][h] =
 *   sum_k a[k][j][h] * b[k][i][h], with everything around the contraction
 *   exactly as in the outgoing reference.
 * a = left projection (linearAP/AG), b = right (linearBP/BG); weights packed
 * in ORDER. Every intermediate is stored to f32 as the reference stores it
 * into a Float32Array; every sum is accumulated in double. */
EXPORT void afref_triangle(int direction, int length, int cz, int ch, const float* z,
                           const float* mask, const float* weights, double epsilon, float* out) {
  size_t off[17];
  afref_triangle_weight_offsets(cz, ch, off);
  const float *ln_in_w = weights + off[0], *ln_in_b = weights + off[1];
  const float *ap_w = weights + off[2], *ap_b = weights + off[3];
  const float *ag_w = weights + off[4], *ag_b = weights + off[5];
  const float *bp_w = weights + off[6], *bp_b = weights + off[7];
  const float *bg_w = weights + off[8], *bg_b = weights + off[9];
  const float *ln_out_w = weights + off[10], *ln_out_b = weights + off[11];
  const float *z_w = weights + off[12], *z_b = weights + off[13];
  const float *g_w = weights + off[14], *g_b = weights + off[15];
  size_t L = (size_t)length, pairs = L * L;

  float* zn = (float*)malloc(pairs * cz * sizeof(float));
  float* ap = (float*)malloc(pairs * ch * sizeof(float));
  float* ag = (float*)malloc(pairs * ch * sizeof(float));
  float* bp = (float*)malloc(pairs * ch * sizeof(float));
  float* bg = (float*)malloc(pairs * ch * sizeof(float));
  normalize_rows(z, pairs, cz, ln_in_w, ln_in_b, epsilon, zn);
  project(zn, pairs, cz, ch, ap_w, ap_b, ap);
  project(zn, pairs, cz, ch, ag_w, ag_b, ag);
  project(zn, pairs, cz, ch, bp_w, bp_b, bp);
  project(zn, pairs, cz, ch, bg_w, bg_b, bg);
#pragma omp parallel for schedule(static)
  for (size_t pair = 0; pair < pairs; pair++) {
    double m = (double)mask[pair];
    for (int h = 0; h < ch; h++) {
      size_t index = pair * ch + h;
      ap[index] = (float)((double)ap[index] * sigmoid((double)ag[index]) * m);
      bp[index] = (float)((double)bp[index] * sigmoid((double)bg[index]) * m);
    }
  }
  free(ag);
  free(bg);

  /* Channel-major copies so the k loop walks memory; the values and the
   * order of the sum are unchanged. */
  float* at = (float*)malloc(pairs * ch * sizeof(float));
  float* bt = (float*)malloc(pairs * ch * sizeof(float));
#pragma omp parallel for schedule(static)
  for (size_t pair = 0; pair < pairs; pair++)
    for (int h = 0; h < ch; h++) {
      at[(size_t)h * pairs + pair] = ap[pair * ch + h];
      bt[(size_t)h * pairs + pair] = bp[pair * ch + h];
    }
  float* contracted = ap; /* reuse: ap is no longer read */
  for (int h = 0; h < ch; h++) {
    const float* ah = at + (size_t)h * pairs;
    const float* bh = bt + (size_t)h * pairs;
#pragma omp parallel for schedule(static)
    for (size_t i = 0; i < L; i++)
      for (size_t j = 0; j < L; j++) {
        double value = 0.0;
        if (direction == 0) {
          const float* ar = ah + i * L;
          const float* br = bh + j * L;
          for (size_t k = 0; k < L; k++) value += (double)ar[k] * (double)br[k];
        } else {
          for (size_t k = 0; k < L; k++) value += (double)ah[k * L + j] * (double)bh[k * L + i];
        }
        contracted[(i * L + j) * ch + h] = (float)value;
      }
  }
  free(at);
  free(bt);

  float* normalized = bp; /* reuse */
  normalize_rows(contracted, pairs, ch, ln_out_w, ln_out_b, epsilon, normalized);
  project(normalized, pairs, ch, cz, z_w, z_b, out);
  float* gate = (float*)malloc(pairs * cz * sizeof(float));
  project(zn, pairs, cz, cz, g_w, g_b, gate);
#pragma omp parallel for schedule(static)
  for (size_t index = 0; index < pairs * cz; index++)
    out[index] = (float)((double)out[index] * sigmoid((double)gate[index]));
  free(gate);
  free(zn);
  free(ap);
  free(bp);
}

/* ------------------------------------------------------------------------ */
/* Outer-product mean                                                        */
/* ------------------------------------------------------------------------ */

/* test/outer-product-mean-reference.gpu.test.ts:22-78 (reference), with the
 * epsilons of src/evoformer/outer-product-mean.ts:82-90 passed in.
 * activations [S][L][cM]; mask [S][L]; weights in the order of
 * packOuterProductMeanWeights (outer-product-mean.ts:64-79): layerNormScale
 * [cM], layerNormOffset [cM], leftWeight [cM][cO], leftBias [cO], rightWeight
 * [cM][cO], rightBias [cO], outputWeight [cO*cO][cZ], outputBias [cZ].
 * The per-pair outer product accumulates into a Float32Array there, so each
 * += is rounded to f32 here too. */
EXPORT void afref_opm(int sequences, int length, int cm, int co, int cz, const float* activations,
                      const float* mask, const float* weights, double ln_epsilon,
                      double norm_epsilon, float* out) {
  size_t S = (size_t)sequences, L = (size_t)length, rows = S * L;
  const float* ln_scale = weights;
  const float* ln_offset = ln_scale + cm;
  const float* left_w = ln_offset + cm;
  const float* left_b = left_w + (size_t)cm * co;
  const float* right_w = left_b + co;
  const float* right_b = right_w + (size_t)cm * co;
  const float* out_w = right_b + co;
  const float* out_b = out_w + (size_t)co * co * cz;

  float* normalized = (float*)malloc(rows * cm * sizeof(float));
  for (size_t row = 0; row < rows; row++) {
    const float* x = activations + row * cm;
    double sum = 0.0;
    for (int c = 0; c < cm; c++) sum += (double)x[c];
    double mean = sum / cm;
    double squared = 0.0;
    for (int c = 0; c < cm; c++) squared += ((double)x[c] - mean) * ((double)x[c] - mean);
    double inverse_std = 1.0 / sqrt(squared / cm + ln_epsilon);
    for (int c = 0; c < cm; c++)
      normalized[row * cm + c] =
          (float)(((double)x[c] - mean) * inverse_std * (double)ln_scale[c] + (double)ln_offset[c]);
  }
  float* left = (float*)malloc(rows * co * sizeof(float));
  float* right = (float*)malloc(rows * co * sizeof(float));
  for (int side = 0; side < 2; side++) {
    const float* w = side == 0 ? left_w : right_w;
    const float* b = side == 0 ? left_b : right_b;
    float* dst = side == 0 ? left : right;
    for (size_t row = 0; row < rows; row++)
      for (int o = 0; o < co; o++) {
        double total = (double)b[o];
        for (int c = 0; c < cm; c++) total += (double)normalized[row * cm + c] * (double)w[(size_t)c * co + o];
        dst[row * co + o] = (float)((double)mask[row] * total);
      }
  }
  free(normalized);
  float* pair = (float*)malloc((size_t)co * co * sizeof(float));
  for (size_t i = 0; i < L; i++)
    for (size_t j = 0; j < L; j++) {
      memset(pair, 0, (size_t)co * co * sizeof(float));
      double count = 0.0;
      for (size_t s = 0; s < S; s++) {
        count += (double)mask[s * L + i] * (double)mask[s * L + j];
        const float* lrow = left + (s * L + i) * co;
        const float* rrow = right + (s * L + j) * co;
        for (int a = 0; a < co; a++) {
          double lv = (double)lrow[a];
          for (int b = 0; b < co; b++)
            pair[a * co + b] = (float)((double)pair[a * co + b] + lv * (double)rrow[b]);
        }
      }
      double scale = 1.0 / (norm_epsilon + count);
      for (int zc = 0; zc < cz; zc++) {
        double total = (double)out_b[zc];
        for (int k = 0; k < co * co; k++) total += (double)pair[k] * (double)out_w[(size_t)k * cz + zc];
        out[(i * L + j) * cz + zc] = (float)(total * scale);
      }
    }
  free(pair);
  free(left);
  free(right);
}

/* ------------------------------------------------------------------------ */
/* Transition                                                                */
/* ------------------------------------------------------------------------ */

/* src/evoformer/transition.ts:179-234 and :264-361 (TransitionGpu.run):
 * LayerNorm over channels, linear channels->hidden + bias + ReLU, linear
 * hidden->channels + bias. Weights packed as packTransitionWeights
 * (transition.ts:157-177): scale [C], offset [C], first [C][H], firstBias
 * [H], second [H][C], secondBias [C]. Each stage is stored to f32. */
EXPORT void afref_transition(size_t rows, int channels, int hidden, const float* activations,
                             const float* weights, double epsilon, float* out) {
  const float* scale = weights;
  const float* offset = scale + channels;
  const float* w1 = offset + channels;
  const float* b1 = w1 + (size_t)channels * hidden;
  const float* w2 = b1 + hidden;
  const float* b2 = w2 + (size_t)hidden * channels;
  float* normalized = (float*)malloc((size_t)channels * sizeof(float));
  float* h = (float*)malloc((size_t)hidden * sizeof(float));
  for (size_t row = 0; row < rows; row++) {
    normalize_rows(activations + row * channels, 1, channels, scale, offset, epsilon, normalized);
    for (int o = 0; o < hidden; o++) {
      double total = 0.0;
      for (int c = 0; c < channels; c++) total += (double)normalized[c] * (double)w1[(size_t)c * hidden + o];
      double stored = total + (double)b1[o];
      h[o] = (float)(stored < 0.0 ? 0.0 : stored);
    }
    for (int o = 0; o < channels; o++) {
      double total = 0.0;
      for (int c = 0; c < hidden; c++) total += (double)h[c] * (double)w2[(size_t)c * channels + o];
      out[row * channels + o] = (float)(total + (double)b2[o]);
    }
  }
  free(normalized);
  free(h);
}
