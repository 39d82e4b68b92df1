// Types of the afhip Node-API shim (index.js), matching the reference's
// operator signatures so TypeScript callers swap the class and nothing else:
// src/triangle/webgpu.ts:9-23, :42-214, src/triangle/types.ts:1-40,
// src/evoformer/outer-product-mean.ts:21-40, src/evoformer/transition.ts:18-31,
// src/runtime/allocator.ts:8-29.

/** One label's share of the live working set (allocator.ts:8-12). */
export interface AllocationShare {
  readonly label: string;
  readonly bytes: number;
  readonly count: number;
}

/** AllocationSnapshot (src/runtime/allocator.ts:14-29). */
export interface AllocationSnapshot {
  readonly currentBytes: number;
  readonly peakBytes: number;
  readonly peakComposition: readonly AllocationShare[];
  readonly residentBytes: number;
  readonly peakResidentBytes: number;
  readonly pooledBytes: number;
  readonly allocationCount: number;
  readonly bufferCount: number;
}

/** TriangleGpuResult, OuterProductMeanResult, TransitionResult, AttentionResult. */
export interface OperatorResult {
  readonly output: Float32Array;
  readonly elapsedMilliseconds: number;
  readonly memory: AllocationSnapshot;
}

export type Precision = "f32" | "f16";

/** TriangleShape (src/triangle/types.ts:3-7). */
export interface TriangleShape {
  readonly length: number;
  readonly cZ: number;
  readonly cHidden: number;
}

export interface TriangleMultiplicationWeights {
  readonly layerNormInWeight: Float32Array;
  readonly layerNormInBias: Float32Array;
  readonly linearAPWeight: Float32Array;
  readonly linearAPBias: Float32Array;
  readonly linearAGWeight: Float32Array;
  readonly linearAGBias: Float32Array;
  readonly linearBPWeight: Float32Array;
  readonly linearBPBias: Float32Array;
  readonly linearBGWeight: Float32Array;
  readonly linearBGBias: Float32Array;
  readonly layerNormOutWeight: Float32Array;
  readonly layerNormOutBias: Float32Array;
  readonly linearZWeight: Float32Array;
  readonly linearZBias: Float32Array;
  readonly linearGWeight: Float32Array;
  readonly linearGBias: Float32Array;
}

/** TriangleMultiplicationInput (src/triangle/types.ts:28-34); z may also be
 * f16 bit patterns in a Uint16Array (an addition). */
export interface TriangleMultiplicationInput {
  readonly shape: TriangleShape;
  readonly z: Float32Array | Uint16Array;
  readonly mask: Float32Array;
  readonly weights: TriangleMultiplicationWeights;
  readonly epsilon?: number;
}

/** TriangleGpuOptions (src/triangle/webgpu.ts:9-16). */
export interface TriangleGpuOptions {
  readonly precision?: Precision;
  readonly blockRows?: number;
  /** Accepted for compatibility; the operands are stored in the precision's
   * dtype, and a value that differs is reported once as a Node warning
   * (code AFHIP_OPTION). Values other than "f32" / "f16" throw RangeError. */
  readonly wholeStorage?: "f32" | "f16";
}

/** Every operator owns its allocator; release() frees its pooled buffers
 * (after any run still pending on it has finished). */
declare class HipOperator {
  release(): void;
}

export declare class TriangleMultiplicationOutgoingGpu extends HipOperator {
  constructor(device?: unknown);
  run(input: TriangleMultiplicationInput, options?: TriangleGpuOptions): Promise<OperatorResult>;
}

export declare class TriangleMultiplicationIncomingGpu extends HipOperator {
  constructor(device?: unknown);
  run(input: TriangleMultiplicationInput, options?: TriangleGpuOptions): Promise<OperatorResult>;
}

export interface OuterProductMeanWeights {
  layerNormScale: Float32Array;
  layerNormOffset: Float32Array;
  leftWeight: Float32Array;
  leftBias: Float32Array;
  rightWeight: Float32Array;
  rightBias: Float32Array;
  outputWeight: Float32Array;
  outputBias: Float32Array;
}

/** OuterProductMeanInput (src/evoformer/outer-product-mean.ts:21-34). */
export interface OuterProductMeanInput {
  readonly activations: Float32Array;
  readonly mask: Float32Array;
  readonly sequences: number;
  readonly length: number;
  readonly cM: number;
  readonly cOuter: number;
  readonly cZ: number;
  readonly weights: OuterProductMeanWeights;
  readonly layerNormEpsilon?: number;
  readonly normalizationEpsilon?: number;
  readonly rowBlockResidues?: number;
}

/** Additions: the arithmetic precision, from the constructor or a run. */
export interface HipOperatorOptions {
  readonly precision?: Precision;
}

export declare class OuterProductMeanGpu extends HipOperator {
  constructor(device?: unknown, options?: HipOperatorOptions);
  run(input: OuterProductMeanInput, options?: HipOperatorOptions): Promise<OperatorResult>;
}

export interface TransitionWeights {
  layerNormScale: Float32Array;
  layerNormOffset: Float32Array;
  firstWeight: Float32Array;
  firstBias: Float32Array;
  secondWeight: Float32Array;
  secondBias: Float32Array;
}

/** TransitionInput (src/evoformer/transition.ts:18-25). */
export interface TransitionInput {
  readonly activations: Float32Array;
  readonly rows: number;
  readonly channels: number;
  readonly hiddenChannels: number;
  readonly weights: TransitionWeights;
  readonly epsilon?: number;
}

export declare class TransitionGpu extends HipOperator {
  constructor(device?: unknown, options?: HipOperatorOptions);
  run(input: TransitionInput, options?: HipOperatorOptions): Promise<OperatorResult>;
}

/** Shape of the chained pair steps (include/afhip.h afhip_pair_stack_desc). */
export interface PairStackShape {
  length: number;
  sequences?: number;
  cM?: number;
  cZ?: number;
  cOuter?: number;
  cHidden?: number;
  transitionFactor?: number;
  precision?: 0 | 1;
  pairDtype?: 0 | 1;
  msaDtype?: 0 | 1;
  opmRowBlock?: number;
  triangleBlockRows?: number;
  attentionHeads?: number;
}

export interface EvoformerBlockShape extends PairStackShape {
  msaHeads?: number;
  msaTransitionFactor?: number;
  opmFirst?: boolean;
}

/** The block's MSA weights (src/evoformer/block.ts:86-88) with the pair stack's. */
export interface EvoformerBlockWeights extends PairStackWeights {
  msaRowAttention?: { attention: AttentionWeights; pairLayerNormScale: Float32Array;
    pairLayerNormOffset: Float32Array; pairProjectionWeight: Float32Array };
  msaColumnAttention?: { attention: AttentionWeights };
  msaTransition?: TransitionWeights;
}

export interface PreparedEvoformerBlock extends PreparedPairStack {
  msaRowAttention?: number;
  msaColumnAttention?: number;
  msaTransition?: number;
}

/** AttentionWeights (src/evoformer/attention.ts:19-29). */
export interface AttentionWeights {
  queryNormScale: Float32Array;
  queryNormOffset: Float32Array;
  queryWeight: Float32Array;
  keyWeight: Float32Array;
  valueWeight: Float32Array;
  gatingWeight: Float32Array;
  gatingBias: Float32Array;
  outputWeight: Float32Array;
  outputBias: Float32Array;
}

/** AttentionPairBias (src/evoformer/attention.ts:31-45). */
export type AttentionPairBias =
  | { source: "separate"; activations: Float32Array; channels: number; layerNormScale: Float32Array;
      layerNormOffset: Float32Array; projectionWeight: Float32Array }
  | { source: "normalized-input"; projectionWeight: Float32Array };

/** AttentionInput (src/evoformer/attention.ts:47-58). */
export interface AttentionInput {
  activations: Float32Array;
  mask: Float32Array;
  batch: number;
  queryLength: number;
  channels: number;
  heads: number;
  transpose?: boolean;
  weights: AttentionWeights;
  pairBias?: AttentionPairBias;
  epsilon?: number;
}

/** AttentionGpu (src/evoformer/attention.ts:1321-1452). */
export declare class AttentionGpu extends HipOperator {
  constructor(device?: unknown, options?: HipOperatorOptions);
  run(input: AttentionInput, options?: HipOperatorOptions): Promise<OperatorResult>;
}

export declare function packAttentionWeights(weights: AttentionWeights, pairBias?: AttentionPairBias): Float32Array;

/** The block's triangle attention weights (src/evoformer/block.ts:1727-1745). */
export interface TriangleAttentionWeights {
  heads?: number;
  attention: AttentionWeights;
  pairProjectionWeight: Float32Array;
}

export interface PairStackWeights {
  outerProductMean?: OuterProductMeanWeights;
  triangleMultiplicationOutgoing?: TriangleMultiplicationWeights;
  triangleMultiplicationIncoming?: TriangleMultiplicationWeights;
  triangleAttentionStarting?: TriangleAttentionWeights;
  triangleAttentionEnding?: TriangleAttentionWeights;
  pairTransition?: TransitionWeights;
}

/** Prepared weight buffers, as preparePairStack returns them. */
export interface PreparedPairStack {
  outerProductMean?: number;
  triangleOutgoing?: number;
  triangleIncoming?: number;
  triangleAttentionStarting?: number;
  triangleAttentionEnding?: number;
  pairTransition?: number;
}

/** AllocationSnapshot (src/runtime/allocator.ts:8-25). */
export interface AllocationSnapshot {
  currentBytes: number;
  peakBytes: number;
  peakComposition: { label: string; bytes: number; count: number }[];
  residentBytes: number;
  peakResidentBytes: number;
  pooledBytes: number;
  allocationCount: number;
  bufferCount: number;
}

/** WebGpuExecution's counterpart (src/runtime/execution.ts:153-555): device
 * tensors as buffer handles from a pool, and the pair steps of an Evoformer
 * block chained on the device (src/evoformer/block.ts:1683-1750). */
export declare class HipExecution {
  constructor(options?: { maxPooledBytes?: number });
  upload(label: string, data: ArrayBufferView): number;
  allocate(label: string, bytes: number): number;
  read<T extends ArrayBufferView>(buffer: number, target: T): T;
  releaseTensor(buffer: number): void;
  checkpoint(): number;
  releaseSince(checkpoint: number): void;
  noteSubmitted(): void;
  snapshot(): AllocationSnapshot;
  addInPlace(base: number, update: number, elements: number, baseDtype?: 0 | 1, updateDtype?: 0 | 1): void;
  preparePairStack(shape: PairStackShape, weights: PairStackWeights): PreparedPairStack;
  /** encodeEvoformerBlock (src/evoformer/block.ts:1673-1759): MSA steps, then the pair steps. */
  prepareEvoformerBlock(shape: EvoformerBlockShape, weights: EvoformerBlockWeights): PreparedEvoformerBlock;
  evoformerBlock(shape: EvoformerBlockShape, prepared: PreparedEvoformerBlock, msa: number, msaMask: number,
    pair: number, pairMask: number): void;
  pairStack(shape: PairStackShape, prepared: PreparedPairStack, pair: number, pairMask: number, msa?: number,
            msaMask?: number): void;
  release(): void;
}
export declare function setGpuMemoryBudget(bytes?: number | null): void;
export declare function gpuMemoryResident(): number;

/** The GEMM plan description (include/afhip.h afhip_gemm_desc). */
export interface GemmDesc {
  rows: number;
  inner: number;
  columns: number;
  batch?: number;
  precision?: number;
  aDtype?: number;
  wDtype?: number;
  wLayout?: number;
  outDtype?: number;
  epilogue?: number;
  heads?: number;
  headDim?: number;
  lda?: number;
  ldw?: number;
  ldc?: number;
  batchStrideA?: number;
  batchStrideW?: number;
  batchStrideC?: number;
  /** 0: A[m][k] (sourceContiguous "k"); 1: A stored [k][m] (sourceContiguous "row", gemm.ts:308-360). */
  aLayout?: 0 | 1;
  /** 0: C[m][n]; 1: C stored [n][m] (a column-major matrixEpilogue, gemm.ts:268-285). */
  cLayout?: 0 | 1;
}

/** GemmVariant (src/runtime/gemm.ts:150-206) as the library reports it. */
export interface GemmVariant {
  precision: number;
  tileRows: number;
  tileColumns: number;
  tileInner: number;
  source: number;
  kernel: number;
}

export declare function requestHipDevice(ordinal?: number): { report: Record<string, unknown> };
export declare function gemmGrid(rows: number, columns: number, tileColumns?: number, tileRows?: number): [number, number];
export declare function gemmSelect(desc: GemmDesc): GemmVariant;
export declare function calibrateGemmVariant(desc: GemmDesc): GemmVariant;
export declare function forceGemmVariant(variant?: Partial<GemmVariant> | null): void;
export declare function calibrationLoad(file: string): void;
export declare function calibrationSave(file: string): void;
/** Decodes the bundle's mixed-q8 weight [rowsK][columnsN] (int8 codes and f16
 * scale bits in device buffers, flat blocks of `block`, from element `start`)
 * into the packed GEMM operand W[n][k] of `dtype` in buffer `dst`
 * (readTensorRange's int8 branch, src/reference/dtype.ts:66-99, on the device). */
export declare function packWeightQ8Block(codes: number, scales: number, block: number, start: number, rowsK: number,
                                          columnsN: number, dst: number, dtype: 0 | 1): void;
export declare function validateTriangleInput(input: TriangleMultiplicationInput): void;
export declare function packTriangleWeights(weights: TriangleMultiplicationWeights): Float32Array;
export declare function errorMetrics(
  actual: ArrayLike<number>,
  expected: ArrayLike<number>,
): { meanAbsoluteError: number; maxAbsoluteError: number; rootMeanSquareError: number };
export declare const TRIANGLE_ORDER: readonly string[];
export declare const DTYPE: { f32: 0; f16: 1; i8: 2 };
export declare const PRECISION: { f32: 0; f16: 1 };
export declare const KERNEL: { register: 0; lds_dma: 1; stream: 2 };
export declare const SOURCE: { k: 0; row: 1 };
export declare const OUTPUT: { row: 0; column: 1 };
export declare function validateOuterProductMeanInput(input: OuterProductMeanInput): void;
export declare function validateTransitionInput(input: TransitionInput): void;
export declare const EPILOGUE: { scale: 1; bias: 2; attention: 4; relu: 8; residual: 16 };
