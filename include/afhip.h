/*
 * afhip — MI355X (gfx950) kernels for alphafold2-webgpu's matrix-multiplication
 * hot path, behind a C ABI.
 *
 * Conventions
 *  - Every entry point returns an int status (AFHIP_OK or a negative code) and
 *    never lets a C++ exception cross the boundary. The message of the last
 *    failure on the calling thread is afhip_last_error().
 *  - Tensor arguments are device pointers (HBM). A caller without its own
 *    allocator uses afhip_buffer_*; a caller with one (PyTorch, a HIP
 *    execution layer) passes its own pointers.
 *  - `stream` is a hipStream_t passed as void*; NULL is the null stream.
 *    Launches are asynchronous on that stream.
 *  - Weights are prepared once by the *_prepare_weights entry points into the
 *    layout and precision the kernels read (the counterpart of the reference's
 *    packWeights), then passed to every run.
 *  - Workspaces are caller-owned; *_workspace_size says how many bytes.
 *
 * Reference interfaces replaced are cited as file:line of the
 * alphafold2-webgpu checkout.
 */
#ifndef AFHIP_H
#define AFHIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define AFHIP_ABI_VERSION 3

#if defined(__GNUC__)
#define AFHIP_API __attribute__((visibility("default")))
#else
#define AFHIP_API
#endif

/* Status codes. The error vocabulary of the reference: RangeError for shapes
 * and limits (src/triangle/types.ts:42-52, src/runtime/gemm.ts:372-374) maps
 * to AFHIP_ERR_INVALID_ARGUMENT; "WebGPU validation failed"
 * (src/triangle/webgpu.ts:191-192) maps to AFHIP_ERR_HIP. */
#define AFHIP_OK 0
#define AFHIP_ERR_INVALID_ARGUMENT (-1)
#define AFHIP_ERR_OUT_OF_MEMORY (-2)
#define AFHIP_ERR_HIP (-3)
#define AFHIP_ERR_UNSUPPORTED (-4)
#define AFHIP_ERR_NOT_OPEN (-5)

/* Element types. */
#define AFHIP_F32 0
#define AFHIP_F16 1
#define AFHIP_I8 2

/* Arithmetic of a kernel's products and accumulator.
 * F32: f32 operands, f32 products and sums (MFMA f32).
 * F16: operands rounded to f16, f32 accumulation (MFMA f16); the reference's
 *      "matrix" precision with an f16 unit (src/runtime/gemm.ts:150-206).
 * Pure f16 accumulation is never offered, as SHIPPABLE_GEMM_PRECISIONS
 * (src/runtime/gemm-selection.ts:160-162) excludes it. */
#define AFHIP_PRECISION_F32 0
#define AFHIP_PRECISION_F16 1

/* ---------------------------------------------------------------------- */
/* Context, errors, device report                                          */
/* ---------------------------------------------------------------------- */

/* Thread-local message of the last failure; never NULL. */
AFHIP_API const char* afhip_last_error(void);
AFHIP_API int afhip_abi_version(void);

/* Selects the device for this process. Replaces request_device
 * (native/wgpu-backend/src/device.rs:205-255) / requestAlphaFoldDevice
 * (src/runtime/device.ts:375-467); one context per process, as the wgpu
 * backend keeps one (device.rs:130-131). */
AFHIP_API int afhip_open(int device_ordinal);
AFHIP_API int afhip_close(void);

/* JSON: name, gfx arch, CU count, clocks, LDS, HBM bytes. Replaces the
 * adapter report of native/wgpu-backend/src/report.rs:61. */
AFHIP_API int afhip_device_report(char* json, size_t capacity);

/* ---------------------------------------------------------------------- */
/* Buffers (native/wgpu-backend/src/lib.rs create_buffer, write_buffer,   */
/* map_buffer, destroy_buffer)                                            */
/* ---------------------------------------------------------------------- */

AFHIP_API int afhip_buffer_create(size_t bytes, void** out);
AFHIP_API int afhip_buffer_destroy(void* buffer);
AFHIP_API int afhip_buffer_write(void* buffer, size_t offset, const void* source, size_t bytes);
AFHIP_API int afhip_buffer_read(const void* buffer, size_t offset, void* destination, size_t bytes);
AFHIP_API int afhip_synchronize(void* stream);

/* ---------------------------------------------------------------------- */
/* GEMM plan and dispatch                                                 */
/* ---------------------------------------------------------------------- */

/* Epilogue flags, applied in this order to the f32 accumulator:
 *   SCALE      y *= scale[column]            (mixed-q8 per-channel scale)
 *   BIAS       y += bias[column]
 *   ATTENTION  columns [0,heads*head_dim) are q: y *= 1/sqrt(head_dim);
 *              columns [3*heads*head_dim, 4*heads*head_dim) are the gate:
 *              y = sigmoid(y); src/evoformer/attention.ts:555-563
 *   RELU       y = max(y, 0)                  src/evoformer/transition.ts:126
 *   RESIDUAL   y += residual[row][column]     (may alias the output) */
#define AFHIP_EPILOGUE_SCALE 1u
#define AFHIP_EPILOGUE_BIAS 2u
#define AFHIP_EPILOGUE_ATTENTION 4u
#define AFHIP_EPILOGUE_RELU 8u
#define AFHIP_EPILOGUE_RESIDUAL 16u

/* Weight layouts. The reference's weightContiguous (gemm.ts:292-314):
 * COLUMN is W[k][n] (weights[k*N+n], the linear's layout); K is W[n][k]
 * (the triangle's [out][in]). */
#define AFHIP_WEIGHT_COLUMN_CONTIGUOUS 0
#define AFHIP_WEIGHT_K_CONTIGUOUS 1

/* Source (A) layouts: the reference's sourceContiguous (gemm.ts:308-321)
 * and GemmOperandArray.columnMajor (:341-360). K_CONTIGUOUS is A[m][k]
 * (element at m*lda + k, the default); ROW_CONTIGUOUS is A stored [k][m]
 * (element at k*lda + m), as the outer-product mean's sequence-accumulated
 * operands (outer-product-mean.ts:376-389) and the incoming triangle
 * contraction (src/triangle/shaders.ts:488) have it. */
#define AFHIP_SOURCE_K_CONTIGUOUS 0
#define AFHIP_SOURCE_ROW_CONTIGUOUS 1

/* Output layouts. ROW_MAJOR is C[m][n] (element at m*ldc + n, the default);
 * COLUMN_MAJOR is C stored [n][m] (element at n*ldc + m), the
 * column-major result a matrixEpilogue writes (gemm.ts:268-285), as the
 * triangle projections store their channel-major operands. */
#define AFHIP_OUTPUT_ROW_MAJOR 0
#define AFHIP_OUTPUT_COLUMN_MAJOR 1

/* The plan a caller describes; the counterpart of TiledGemmShader
 * (src/runtime/gemm.ts:230-339) with its WGSL fragments replaced by an
 * enumerated description. C[b][m][n] = epilogue(sum_k A[b][m][k] W[b][k][n]).
 * lda, ldw and ldc are the strides between the operands' outer index
 * (rows of A[m][k], or k of A[k][m]; and so on). A row-contiguous source and
 * a column-major output run on REGISTER_STAGED or LDS_DMA (not STREAM). */
typedef struct afhip_gemm_desc {
  int32_t rows;          /* M */
  int32_t inner;         /* K */
  int32_t columns;       /* N */
  int32_t batch;         /* >= 1 */
  int32_t precision;     /* AFHIP_PRECISION_* */
  int32_t a_dtype;       /* AFHIP_F32 | AFHIP_F16 */
  int32_t w_dtype;       /* AFHIP_F32 | AFHIP_F16 | AFHIP_I8 */
  int32_t w_layout;      /* AFHIP_WEIGHT_* */
  int32_t out_dtype;     /* AFHIP_F32 | AFHIP_F16 */
  uint32_t epilogue;     /* AFHIP_EPILOGUE_* */
  int32_t heads;         /* ATTENTION only */
  int32_t head_dim;      /* ATTENTION only */
  int64_t lda, ldw, ldc; /* leading dimensions in elements; 0 = packed */
  int64_t batch_stride_a, batch_stride_w, batch_stride_c; /* elements */
  int32_t a_layout;      /* AFHIP_SOURCE_* (0: A[m][k]) */
  int32_t c_layout;      /* AFHIP_OUTPUT_* (0: C[m][n]) */
} afhip_gemm_desc;

typedef struct afhip_gemm_plan afhip_gemm_plan;

/* Validates the description and chooses a kernel (afhip_gemm_select). */
AFHIP_API int afhip_gemm_plan_create(const afhip_gemm_desc* desc, afhip_gemm_plan** out);
AFHIP_API int afhip_gemm_plan_destroy(afhip_gemm_plan* plan);
/* Bytes of device workspace a run needs (a W transpose for the
 * column-contiguous layout; 0 otherwise). */
AFHIP_API int afhip_gemm_workspace_size(const afhip_gemm_plan* plan, size_t* bytes);
/* scale: f32 [N] (SCALE); bias: f32 [N] (BIAS); residual: laid out as the
 * output, of the output dtype (RESIDUAL). Unused pointers may be NULL. */
AFHIP_API int afhip_gemm_run(const afhip_gemm_plan* plan, const void* a, const void* w, const float* scale,
                   const float* bias, const void* residual, void* c, void* workspace,
                   size_t workspace_bytes, void* stream);

/* afhip_gemm_run without a workspace argument and without allocating: the
 * workspace the plan needs (afhip_gemm_workspace_size) lives in a device
 * array of afhip_gemm_static_scratch_bytes (8 MiB) that the library holds on
 * each GPU it runs on until the process ends. No counterpart in the
 * reference: it is for callers that cannot allocate device memory (HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). A plan
 * whose workspace exceeds the array is refused (AFHIP_ERR_INVALID_ARGUMENT).
 * Calls that overlap on one GPU share the array and race; no timing events
 * are recorded for its launches. Same results as afhip_gemm_run. */
AFHIP_API int afhip_gemm_run_static(const afhip_gemm_plan* plan, const void* a, const void* w, const float* scale,
                                    const float* bias, const void* residual, void* c, void* stream);
AFHIP_API int afhip_gemm_static_scratch_bytes(size_t* bytes);

/* gemmGrid (src/runtime/gemm.ts:368-379): the reference's workgroup grid
 * for an M x N output, row tiles past 65,535 folded into x. Host logic kept
 * for callers that still size WebGPU-style grids. */
AFHIP_API int afhip_gemm_grid(int64_t rows, int64_t columns, int32_t tile_columns, int32_t tile_rows,
                    uint32_t out_xy[2]);

/* The variant the library runs a description with: the counterpart of
 * GemmVariant (src/runtime/gemm.ts:150-206). */
typedef struct afhip_variant {
  int32_t precision;   /* AFHIP_PRECISION_* */
  int32_t tile_rows;   /* REGISTER_STAGED: 64 | 128; LDS_DMA: 128 | 192; STREAM: 64 */
  int32_t tile_columns;/* REGISTER_STAGED: 64 | 128; LDS_DMA: 128 | 192 | 256; STREAM: 512 */
  int32_t tile_inner;  /* 32 */
  int32_t vectorized;  /* 16-byte operand loads */
  int32_t source;      /* 0 heuristic, 1 calibrated, 2 pinned */
  int32_t kernel;      /* AFHIP_KERNEL_* */
} afhip_variant;

/* Kernel families a variant can name.
 * REGISTER_STAGED: operands pass through VGPRs into double-buffered LDS; any
 *   operand dtype (f32, f16, int8 weights), tiles 64 or 128 on each side.
 * LDS_DMA: operands go global -> LDS directly (buffer loads into LDS), several
 *   k-steps in flight; f16 operands (an int8 weight is widened to f16 by the
 *   plan first, exactly) with an even K: 16-byte loads when K and the leading
 *   dimensions are multiples of 8, 4-byte loads (128x128 tiles) otherwise;
 *   tiles 128x128, 192x192, 128x256 or 256x256. An f32 source under f16
 *   precision (K a multiple of 8, 16-byte aligned rows) is staged as f32 and
 *   rounded to f16 as the MFMA fragments are read, on 128x128 tiles; a
 *   row-contiguous source (M a multiple of 8, 16-byte aligned k rows) is
 *   staged as k rows and read through transposing LDS loads. f32 precision
 *   (f32 operands, K a multiple of 4, 16-byte aligned rows) runs the f32
 *   MFMA on 64x64 tiles whatever the variant's tile, with the
 *   REGISTER_STAGED kernel's bits. The counterpart of the reference's
 *   matrix kernel with deeper k-staging (src/runtime/gemm.ts:470-479).
 * STREAM: weight-stationary: the weight stays in registers and 64-row tiles of
 *   the activations stream past it, each byte read and written once; f16
 *   activations and output, f16 or int8 weights, K of 64, 128 or 256, columns
 *   a multiple of 64, no batch, SCALE/BIAS/ATTENTION/RELU epilogues (BIAS up
 *   to K = 128); other operands run on a tiled family instead. The
 *   counterpart of the reference's mixed-q8 projection kernels
 *   (src/runtime/gemm.ts:150-206) for the bandwidth-bound projections. */
#define AFHIP_KERNEL_REGISTER_STAGED 0
#define AFHIP_KERNEL_LDS_DMA 1
#define AFHIP_KERNEL_STREAM 2

/* Shape-driven selection: the calibrated answer for this description's
 * shape class if one is held, else the heuristic. Replaces gemmVariant()
 * and gemmVariantCandidates (gemm-selection.ts:234-272). */
AFHIP_API int afhip_gemm_select(const afhip_gemm_desc* desc, afhip_variant* out);
/* Measures every candidate tile for the description's shape class on the
 * open device (correctness check first, on rows sampled from every batch,
 * then interleaved timing, as measureGemmVariants does,
 * gemm-selection.ts:471-531), installs and returns the winner. Replaces
 * calibrateGemmVariant (:560-660). A candidate that fails to run is dropped
 * and one whose error exceeds 0.02 of the largest reference value refused;
 * when none is left, nothing is installed and the heuristic's variant is
 * returned (source 0), as the reference keeps its f32 kernel. */
AFHIP_API int afhip_gemm_calibrate(const afhip_gemm_desc* desc, afhip_variant* out);
/* Pins a variant for every plan created afterwards (NULL unpins); the
 * counterpart of forceGemmVariant (gemm-selection.ts:122-125). */
AFHIP_API int afhip_gemm_force_variant(const afhip_variant* variant);
/* Calibration document (JSON, keyed by device, driver and shape class);
 * the counterpart of readCalibration/writeCalibration
 * (src/runtime/calibration-store.ts:119-131). A document that fails
 * validation is ignored, as isGemmVariant rejects one (gemm-selection.ts:543-558). */
AFHIP_API int afhip_calibration_load(const char* path);
AFHIP_API int afhip_calibration_save(const char* path);
/* Forgets every calibrated answer held in this process (the selection falls
 * back to the heuristic until a calibration or a document installs one). */
AFHIP_API int afhip_calibration_clear(void);

/* Faults a test forces on one calibration candidate from the host, so the
 * calibration's failure handling can be exercised without a failing kernel:
 * RUN makes the candidate count as one that failed to run (dropped, as
 * measureGemmVariants drops it, gemm-selection.ts:482-495); RESULT offsets
 * the candidate's result by 5% of the reference's largest value as the check
 * reads it (refused, :584-586); LAST_BATCH does the same to the rows of
 * the shape's last batch entry only, so a check that sampled fewer batches
 * would let the candidate through. NONE clears the candidate's fault; NONE
 * with kernel < 0 clears them all. No counterpart in the reference beyond
 * those rules; for tests. */
#define AFHIP_CALIBRATION_FAULT_NONE 0
#define AFHIP_CALIBRATION_FAULT_RUN 1
#define AFHIP_CALIBRATION_FAULT_RESULT 2
#define AFHIP_CALIBRATION_FAULT_LAST_BATCH 3
AFHIP_API int afhip_calibration_inject(int32_t kernel, int32_t tile_rows, int32_t tile_columns, int32_t fault);

/* Weight preparation for GEMM plans: W[k][n] -> W[n][k] (and f32 -> f16 when
 * dst_dtype is F16). Element types of src and dst given explicitly. */
AFHIP_API int afhip_pack_weight(const void* src, int32_t src_dtype, int32_t rows_k, int32_t columns_n,
                      void* dst, int32_t dst_dtype, void* stream);

/* ---------------------------------------------------------------------- */
/* Quantised weights                                                       */
/* ---------------------------------------------------------------------- */

/* Per-output-channel int8: w[k][n] = f32(q[k][n]) * scale[n] (one rounded
 * product, bit-exact against the closed form). */
AFHIP_API int afhip_dequant_q8_channel(const int8_t* q, const float* scale, int32_t rows_k, int32_t columns_n,
                             float* out, void* stream);
/* The reference bundle's mixed-q8 format: flat blocks of `block` codes, one
 * f16 scale each; decodes values [start, start+count). Replaces the int8
 * branch of readTensorRange (src/reference/dtype.ts:66-99). */
AFHIP_API int afhip_dequant_q8_block(const int8_t* codes, const uint16_t* scales_f16, int32_t block, int64_t start,
                           int64_t count, float* out, void* stream);
/* The same bundle format straight into a GEMM operand, with no f32 copy of
 * the weight: the tensor [rows_k][columns_n] ([in][out], as the bundle stores
 * it) starting at element `start` is decoded as above (bit-exact) and
 * written packed k-contiguous, W[n][k], in F32 or F16 (round to nearest
 * even), ready for a plan with w_layout AFHIP_WEIGHT_K_CONTIGUOUS and w_dtype
 * dst_dtype.
 * Block scales vary with k as well as n (scale index (start + k N + n) /
 * block), so they are applied here, not in the GEMM epilogue. Replaces
 * readTensorRange's int8 branch (src/reference/dtype.ts:66-99) followed by
 * the host upload and packing of the decoded f32 weight. */
AFHIP_API int afhip_pack_weight_q8_block(const int8_t* codes, const uint16_t* scales_f16, int32_t block,
                                         int64_t start, int32_t rows_k, int32_t columns_n, void* dst,
                                         int32_t dst_dtype, void* stream);

/* ---------------------------------------------------------------------- */
/* Triangle multiplication                                                 */
/* ---------------------------------------------------------------------- */

#define AFHIP_TRIANGLE_OUTGOING 0
#define AFHIP_TRIANGLE_INCOMING 1

/* Replaces TriangleMultiplication{Outgoing,Incoming}Gpu.run
 * (src/triangle/webgpu.ts:56-214) and encodeTriangleMultiplication
 * (src/evoformer/block.ts:1497-1671). */
typedef struct afhip_triangle_desc {
  int32_t length;     /* L */
  int32_t c_z;
  int32_t c_hidden;
  int32_t direction;  /* AFHIP_TRIANGLE_* */
  int32_t precision;  /* AFHIP_PRECISION_* */
  int32_t pair_dtype; /* z: AFHIP_F32 | AFHIP_F16 */
  int32_t out_dtype;  /* AFHIP_F32 | AFHIP_F16 */
  int32_t block_rows; /* output residue rows per block; 0 = all (TriangleGpuOptions.blockRows) */
  int32_t residual;   /* out += result (the block encoder's residualOutput) */
  float epsilon;      /* LayerNorm epsilon, 1e-5 by default */
} afhip_triangle_desc;

/* Bytes of the prepared weight buffer and of the workspace. */
AFHIP_API int afhip_triangle_weights_size(const afhip_triangle_desc* desc, size_t* bytes);
AFHIP_API int afhip_triangle_workspace_size(const afhip_triangle_desc* desc, size_t* bytes);
/* packed: the sixteen f32 tensors in the order of src/triangle/weights.ts:4-10
 * (ORDER), weights [out][in], as packWeights lays them out (weights.ts:20-34). */
AFHIP_API int afhip_triangle_prepare_weights(const afhip_triangle_desc* desc, const float* packed, void* prepared,
                                   void* stream);
/* Which kernels a run of this descriptor takes: *fast = 1 for the persistent
 * f16 kernels (c_z = c_hidden = 128, f16 precision, z 16-byte aligned, and an
 * incoming z of at most 4 GiB), 0 for the general ones; results agree within
 * the precision's tolerance either way. The counterpart of afhip_gemm_select
 * for this operator (the reference has one kernel set, src/triangle/shaders.ts). */
AFHIP_API int afhip_triangle_fast_path(const afhip_triangle_desc* desc, int32_t* fast);
/* z [L][L][c_z]; mask [L][L] f32; out [L][L][c_z]. */
AFHIP_API int afhip_triangle_run(const afhip_triangle_desc* desc, const void* z, const float* mask,
                       const void* prepared, void* out, void* workspace, size_t workspace_bytes,
                       void* stream);

/* ---------------------------------------------------------------------- */
/* Outer-product mean                                                      */
/* ---------------------------------------------------------------------- */

/* Replaces OuterProductMeanGpu.run (src/evoformer/outer-product-mean.ts:549-646)
 * and encodeOuterProductMean (src/evoformer/block.ts:1115-1246). */
typedef struct afhip_opm_desc {
  int32_t sequences;  /* S */
  int32_t length;     /* L */
  int32_t c_m;
  int32_t c_outer;
  int32_t c_z;
  int32_t precision;  /* AFHIP_PRECISION_* */
  int32_t msa_dtype;  /* activations: AFHIP_F32 | AFHIP_F16 */
  int32_t out_dtype;  /* AFHIP_F32 | AFHIP_F16 */
  int32_t row_block;  /* residues per contraction block; 0 = all (rowBlockResidues). It
                       * bounds the f16/f32 `outer` block in the workspace; at f16
                       * precision with c_outer 32 and c_z in (96, 128] the contraction
                       * and output projection run fused with no `outer` at all, and
                       * row_block changes nothing. Results never depend on it. */
  int32_t residual;   /* out += result */
  float layer_norm_epsilon;    /* 1e-5 */
  float normalization_epsilon; /* 1e-3 */
} afhip_opm_desc;

AFHIP_API int afhip_opm_weights_size(const afhip_opm_desc* desc, size_t* bytes);
AFHIP_API int afhip_opm_workspace_size(const afhip_opm_desc* desc, size_t* bytes);
/* packed: f32 tensors in the order of packOuterProductMeanWeights
 * (outer-product-mean.ts:64-79): layerNormScale [c_m], layerNormOffset [c_m],
 * leftWeight [c_m][c_outer], leftBias, rightWeight [c_m][c_outer],
 * rightBias, outputWeight [c_outer*c_outer][c_z], outputBias [c_z]. */
AFHIP_API int afhip_opm_prepare_weights(const afhip_opm_desc* desc, const float* packed, void* prepared, void* stream);
/* activations [S][L][c_m]; mask [S][L] f32; out [L][L][c_z]. */
AFHIP_API int afhip_opm_run(const afhip_opm_desc* desc, const void* activations, const float* mask, const void* prepared,
                  void* out, void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------- */
/* Transition                                                              */
/* ---------------------------------------------------------------------- */

/* Replaces TransitionGpu.run (src/evoformer/transition.ts:264-361):
 * LayerNorm, linear channels->hidden + bias + ReLU, linear hidden->channels + bias. */
typedef struct afhip_transition_desc {
  int64_t rows;
  int32_t channels;
  int32_t hidden;
  int32_t precision;  /* AFHIP_PRECISION_* */
  int32_t in_dtype;   /* AFHIP_F32 | AFHIP_F16 */
  int32_t out_dtype;  /* AFHIP_F32 | AFHIP_F16 */
  int32_t residual;   /* out += result */
  float epsilon;
} afhip_transition_desc;

AFHIP_API int afhip_transition_weights_size(const afhip_transition_desc* desc, size_t* bytes);
AFHIP_API int afhip_transition_workspace_size(const afhip_transition_desc* desc, size_t* bytes);
/* packed: f32 in the order of packTransitionWeights (transition.ts:157-177):
 * layerNormScale [C], layerNormOffset [C], firstWeight [C][H], firstBias [H],
 * secondWeight [H][C], secondBias [C]. */
AFHIP_API int afhip_transition_prepare_weights(const afhip_transition_desc* desc, const float* packed, void* prepared,
                                     void* stream);
/* At f16 precision, channels 128 with hidden 512 (the pair transition) and
 * channels 256 with hidden 1024 and f16 activations (the MSA transition) run
 * as one fused kernel: the workspace size is 0, and activations and out must
 * be 16-byte aligned. activations == out is allowed (in place). */
AFHIP_API int afhip_transition_run(const afhip_transition_desc* desc, const void* activations, const void* prepared,
                         void* out, void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------- */
/* Gated attention with pair bias                                          */
/* ---------------------------------------------------------------------- */

/* Pair bias sources (AttentionPairBias, src/evoformer/attention.ts:31-45). */
#define AFHIP_PAIR_BIAS_NONE 0
#define AFHIP_PAIR_BIAS_NORMALIZED_INPUT 1 /* the normalised input itself; batch == queries */
#define AFHIP_PAIR_BIAS_SEPARATE 2         /* pair activations [queries][queries][pair_channels] */

/* Replaces AttentionGpu.run (src/evoformer/attention.ts:1321-1452) and the
 * block encoder's encodeAttention (src/evoformer/block.ts): MSA row attention
 * with pair bias (separate), MSA column attention (transposed, no bias),
 * triangle attention starting and ending node (normalized-input, the ending
 * node transposed). Limits as validate (attention.ts:102-141): head
 * dimension channels / heads integral and at most 32. */
typedef struct afhip_attention_desc {
  int32_t batch;         /* B */
  int32_t queries;       /* Q (AttentionInput.queryLength) */
  int32_t channels;      /* C */
  int32_t heads;         /* H, at most 8 */
  int32_t transpose;     /* entry (b, q) is source row q*B + b instead of b*Q + q */
  int32_t pair_bias;     /* AFHIP_PAIR_BIAS_* */
  int32_t pair_channels; /* SEPARATE only */
  int32_t precision;     /* AFHIP_PRECISION_* */
  int32_t in_dtype;      /* activations and pair activations: AFHIP_F32 | AFHIP_F16 */
  int32_t out_dtype;     /* AFHIP_F32 | AFHIP_F16 */
  int32_t residual;      /* out += result */
  float epsilon;         /* LayerNorm epsilon, 1e-5 by default */
} afhip_attention_desc;

AFHIP_API int afhip_attention_weights_size(const afhip_attention_desc* desc, size_t* bytes);
AFHIP_API int afhip_attention_workspace_size(const afhip_attention_desc* desc, size_t* bytes);
/* packed: f32 in the order of packAttentionWeights (attention.ts:179-201):
 * queryNormScale [C], queryNormOffset [C], query/key/value/gatingWeight
 * [C][C] each ([in][out]), gatingBias [C], outputWeight [C][C], outputBias
 * [C]; then for SEPARATE the pair layerNormScale and layerNormOffset
 * [pair_channels] and projectionWeight [pair_channels][H], for
 * NORMALIZED_INPUT projectionWeight [C][H]. */
AFHIP_API int afhip_attention_prepare_weights(const afhip_attention_desc* desc, const float* packed, void* prepared,
                                    void* stream);
/* activations [B*Q][C] in source order; mask [B*Q] f32 in source order;
 * pair_activations [Q][Q][pair_channels] (SEPARATE, else NULL); out [B*Q][C]
 * in source order. */
AFHIP_API int afhip_attention_run(const afhip_attention_desc* desc, const void* activations, const float* mask,
                        const void* pair_activations, const void* prepared, void* out, void* workspace,
                        size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------- */
/* Execution layer                                                         */
/* ---------------------------------------------------------------------- */

/* Device-resident tensors across operator calls, so a block's steps chain on
 * the device without host round trips. Replaces WebGpuExecution
 * (src/runtime/execution.ts:153-555) and its GpuBufferAllocator
 * (src/runtime/allocator.ts:168-388): requests of 1 MiB or more take whole
 * mebibytes; a released tensor's buffer goes to an idle pool, and a request
 * takes the smallest idle buffer that covers it and is at most twice its
 * size; idle buffers untouched for four submitted boundaries are freed and
 * the pool is trimmed to its cap. One execution is used from one thread. */
typedef struct afhip_execution afhip_execution;

/* Caps the resident bytes of every execution on the open device together;
 * 0 removes the cap. Replaces setGpuMemoryBudget (allocator.ts:66-71). */
AFHIP_API int afhip_set_memory_budget(uint64_t bytes);
/* Replaces gpuMemoryResident (allocator.ts:74). */
AFHIP_API int afhip_memory_resident(uint64_t* bytes);
/* max_pooled_bytes: the idle pool's cap, 0 for 864 MiB (COMPACT_GPU_POOL_BYTES,
 * allocator.ts:30); stream: where uploads and chained steps run. Replaces
 * the WebGpuExecution constructor (execution.ts:183-199). */
AFHIP_API int afhip_execution_create(uint64_t max_pooled_bytes, void* stream, afhip_execution** out);
/* Releases every tensor and frees the pool (WebGpuExecution.release,
 * execution.ts:549-554). */
AFHIP_API int afhip_execution_destroy(afhip_execution* ex);
/* allocate and upload (execution.ts:201-221; allocator.ts:197-285). Past the
 * budget: AFHIP_ERR_OUT_OF_MEMORY with a message naming the label
 * (GpuMemoryBudgetError, allocator.ts:76-90). Labels differing only in a
 * trailing index share a group in the snapshot (allocator.ts:110). */
AFHIP_API int afhip_execution_allocate(afhip_execution* ex, const char* label, uint64_t bytes, void** out);
AFHIP_API int afhip_execution_upload(afhip_execution* ex, const char* label, const void* host, uint64_t bytes,
                                     void** out);
/* One tensor back to the idle pool (AllocatedGpuBuffer.release,
 * allocator.ts:159-165). */
AFHIP_API int afhip_execution_release(afhip_execution* ex, void* tensor);
/* checkpoint and releaseSince (execution.ts:531-547): every tensor allocated
 * after the checkpoint goes back to the pool. */
AFHIP_API int afhip_execution_checkpoint(const afhip_execution* ex, uint64_t* out);
AFHIP_API int afhip_execution_release_since(afhip_execution* ex, uint64_t checkpoint);
/* A submitted boundary (noteSubmitted, execution.ts:533; allocator.ts:332-341). */
AFHIP_API int afhip_execution_note_submitted(afhip_execution* ex);
/* JSON AllocationSnapshot (allocator.ts:8-25, :376-387): currentBytes,
 * peakBytes, peakComposition, residentBytes, peakResidentBytes, pooledBytes,
 * allocationCount, bufferCount. */
AFHIP_API int afhip_execution_snapshot(const afhip_execution* ex, char* json, size_t capacity);
/* base += update over `elements` values, each f32 or f16 (addInPlace,
 * execution.ts:415-450). */
AFHIP_API int afhip_execution_add_in_place(afhip_execution* ex, void* base, int32_t base_dtype, const void* update,
                                           int32_t update_dtype, int64_t elements);

typedef struct afhip_pair_stack_desc {
  afhip_opm_desc opm;               /* out_dtype = the pair's dtype */
  afhip_triangle_desc outgoing;     /* pair_dtype = out_dtype = the pair's dtype */
  afhip_triangle_desc incoming;
  afhip_attention_desc attention_start; /* batch = queries = L, channels = c_z, dtypes the pair's */
  afhip_attention_desc attention_end;
  afhip_transition_desc transition; /* rows = L * L, channels = c_z, in/out dtype = the pair's */
} afhip_pair_stack_desc;

/* Prepared weight buffers (afhip_*_prepare_weights); NULL skips a step. */
typedef struct afhip_pair_stack_weights {
  const void* opm;
  const void* outgoing;
  const void* incoming;
  const void* attention_start;
  const void* attention_end;
  const void* transition;
} afhip_pair_stack_weights;

/* The pair-representation steps of encodeEvoformerBlock
 * (src/evoformer/block.ts:1673-1759), in the block's order, each adding into
 * `pair` in place: outer-product mean (:1683-1689, :1718), triangle
 * multiplication outgoing then incoming (:1720-1725), triangle attention
 * around the starting node then the ending node (:1727-1745, normalized-input
 * pair bias, the ending node transposed), pair transition (:1747-1750). Each
 * step's workspace comes from the execution's pool and returns to it once the
 * step is queued; the descriptors' residual flags, directions, transposes and
 * pair bias sources are set here. */
AFHIP_API int afhip_execution_pair_stack(afhip_execution* ex, const afhip_pair_stack_desc* desc,
                                         const afhip_pair_stack_weights* weights, const void* msa,
                                         const float* msa_mask, void* pair, const float* pair_mask);

/* A whole Evoformer block: encodeEvoformerBlock (src/evoformer/block.ts:
 * 1673-1759). MSA row attention with the pair bias (separate source: the
 * pair, :1690-1702), MSA column attention (transposed, :1704-1711), MSA
 * transition (:1713-1716), then the pair stack above; the outer-product mean
 * runs first instead when opm_first is set (outerProductMeanFirst,
 * :1689). Everything updates `msa` and `pair` in place. The MSA and the pair
 * share one dtype. */
typedef struct afhip_evoformer_block_desc {
  afhip_attention_desc msa_row;        /* batch = S, queries = L, channels = c_m, pair_channels = c_z */
  afhip_attention_desc msa_column;     /* batch = L, queries = S, channels = c_m */
  afhip_transition_desc msa_transition; /* rows = S * L, channels = c_m */
  afhip_pair_stack_desc pair;
  int32_t opm_first;
} afhip_evoformer_block_desc;

typedef struct afhip_evoformer_block_weights {
  const void* msa_row;        /* afhip_attention_prepare_weights, SEPARATE pair bias */
  const void* msa_column;     /* afhip_attention_prepare_weights, no pair bias */
  const void* msa_transition; /* afhip_transition_prepare_weights */
  afhip_pair_stack_weights pair;
} afhip_evoformer_block_weights;

AFHIP_API int afhip_execution_evoformer_block(afhip_execution* ex, const afhip_evoformer_block_desc* desc,
                                              const afhip_evoformer_block_weights* weights, void* msa,
                                              const float* msa_mask, void* pair, const float* pair_mask);

/* ---------------------------------------------------------------------- */
/* Kernel timing                                                           */
/* ---------------------------------------------------------------------- */

/* When enabled, every kernel the library launches is bracketed by hipEvents
 * on its own stream and its duration accumulated under its label; the
 * counterpart of WebGpuExecution's timestamp profile
 * (src/runtime/execution.ts:329-345, :482-513). Reading synchronises the
 * recorded events. JSON: {"label": {"count": n, "total_ms": t}, ...}. */
AFHIP_API int afhip_timing_enable(int enable);
AFHIP_API int afhip_timing_reset(void);
AFHIP_API int afhip_timing_report(char* json, size_t capacity);

#ifdef __cplusplus
}
#endif

#endif /* AFHIP_H */
