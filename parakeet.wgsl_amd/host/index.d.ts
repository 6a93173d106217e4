// Type declarations of parakeet.wgsl_amd/host (index.js): the reference's
// GEMM op interface (src/webgpu/kernels/gemm.ts:358-470, encoder.ts:308-432,
// arena.ts:5-15, package.ts:45-50) over HIP device memory.

export interface TensorRecord {
  readonly dtype: "float16" | "float32" | "uint32";
  readonly logicalShape: readonly number[];
  readonly storageShape: readonly number[];
  readonly byteLength: number;
  readonly layout: string;
}

export interface HipBuffer {
  readonly label: string;
  readonly size: number;
  /** Device address. */
  readonly address: bigint;
  destroy(): void;
}

export interface BufferBinding {
  readonly buffer: HipBuffer;
  readonly offset: number;
  readonly size: number;
}

/** package.ts:45-50 */
export interface GpuTensor {
  readonly sourceRecord: TensorRecord;
  readonly runtimeRecord: TensorRecord;
  readonly buffer: HipBuffer;
  readonly binding: BufferBinding;
}

/** arena.ts:5-15 */
export interface ArenaSlice {
  readonly label: string;
  readonly bufferIndex?: number;
  readonly byteOffset: number;
  readonly byteLength: number;
}

/** execution-shape.ts:1-4 */
export interface EncoderDispatchShape {
  readonly batchSize: number;
  readonly rows: number;
}

export type GemmActivation = "none" | "silu" | "relu";

export interface HipTimestampQuerySet {
  write(index: number): void;
  elapsedMs(begin: number, end: number): number;
  destroy(): void;
}

export interface TimestampWrites {
  readonly querySet: HipTimestampQuerySet;
  readonly beginningOfPassWriteIndex?: number;
  readonly endOfPassWriteIndex?: number;
}

export interface HipCommandBuffer {
  readonly label: string;
}

export interface HipCommandEncoder {
  finish(): HipCommandBuffer;
}

export interface HipQueue {
  writeBuffer(buffer: HipBuffer, bufferOffset: number, data: ArrayBuffer | ArrayBufferView): void;
  submit(commandBuffers: readonly HipCommandBuffer[]): void;
  onSubmittedWorkDone(): Promise<void>;
  readBuffer(buffer: HipBuffer, offset: number, size: number): Promise<ArrayBuffer>;
}

export interface DeviceInfo {
  readonly name: string;
  readonly arch: string;
  readonly computeUnits: number;
  readonly wavefrontSize: number;
  readonly globalMemoryBytes: number;
  readonly ldsBytesPerBlock: number;
  readonly clockKhz: number;
}

export declare class HipGpuDevice {
  static create(options?: { index?: number }): HipGpuDevice;
  readonly info: DeviceInfo;
  readonly queue: HipQueue;
  readonly limits: { readonly minStorageBufferOffsetAlignment: number };
  createBuffer(descriptor: { label?: string; size: number }): HipBuffer;
  createCommandEncoder(descriptor?: { label?: string }): HipCommandEncoder;
  createQuerySet(descriptor: { type: "timestamp"; count: number }): HipTimestampQuerySet;
  destroy(): void;
}

export declare class GpuActivationArena {
  constructor(device: HipGpuDevice, byteLength: number, label?: string);
  readonly byteLength: number;
  slice(label: string, byteOffset: number, byteLength: number): ArenaSlice;
  binding(slice: ArenaSlice): BufferBinding;
  upload(device: HipGpuDevice, destination: ArenaSlice, data: ArrayBuffer | ArrayBufferView): void;
  destroy(): void;
}

/** gemm.ts:375-385 */
export interface PreparedPaletteWeight {
  readonly source: GpuTensor;
  readonly palette: GpuTensor;
  readonly paletteGroupColumns: number;
  readonly inner: number;
  readonly columns: number;
  readonly runtimeLayout: string;
  readonly binding: BufferBinding;
  readonly preparation: { destroy(): void };
}

/** gemm.ts:358-373 */
export interface GemmDescriptor {
  readonly label: string;
  readonly a: ArenaSlice;
  readonly b: GpuTensor;
  readonly bPalette?: GpuTensor;
  readonly paletteGroupColumns?: number;
  readonly output: ArenaSlice;
  readonly rows: number;
  readonly inner: number;
  readonly columns: number;
  readonly bias?: GpuTensor;
  readonly residual?: ArenaSlice;
  readonly residualScale?: number;
  readonly activation?: GemmActivation;
  readonly preparedPaletteWeight?: PreparedPaletteWeight;
  /**
   * This library only: GLU epilogue (PK_GEMM_GLU). Columns [0, N/2) are GLU
   * values, [N/2, N) gates; the output is [rows, N/2] value * sigmoid(gate).
   */
  readonly glu?: boolean;
  /**
   * This library only: keep the output stores ordinary
   * (PK_GEMM_CACHED_OUTPUT); the f16 pair-code kernels otherwise store the
   * output non-temporally.
   */
  readonly cachedOutput?: boolean;
}

export interface GemmPlan {
  readonly workgroups: readonly [number, number, number];
  readonly blockThreads: number;
  readonly tileRows: number;
  readonly tileColumns: number;
  readonly splitInner: number;
  readonly ldsBytes: number;
  readonly workspaceBytes: number;
  readonly flops: number;
  readonly algorithmicBytes: number;
  readonly kernel: string;
  /** The launch stores its output non-temporally (see cachedOutput). */
  readonly streamStores: boolean;
}

/** gemm.ts:400-470, encoder.ts:308-316 (ManagedDispatch) */
export declare class GemmDispatch {
  readonly label: string;
  readonly output: ArenaSlice;
  encode(encoder: HipCommandEncoder, timestampWrites?: TimestampWrites, shape?: EncoderDispatchShape): void;
  destroy(): void;
  plan(activeRows?: number): GemmPlan;
}

export interface GemmKernelOptions {
  /** Accept shapes outside the reference's 15 production signatures. */
  readonly allowSyntheticShapes?: boolean;
}

declare class PaletteGemmKernel {
  readonly portableLoadEncoding: null;
  readonly transientPaletteParameterBytes: number;
  readonly transientPaletteParameterUsedSlots: number;
  readonly transientPaletteDispatchCount: number;
  readonly transientPaletteExpandedBytes: number;
  createDispatch(descriptor: GemmDescriptor): GemmDispatch;
  createPreparedPaletteWeight(descriptor: GemmDescriptor, scratchOffset: number): PreparedPaletteWeight;
  validateDescriptor(descriptor: GemmDescriptor): void;
  destroy(): void;
}

/** gemm.ts:483-855 */
export declare class F16GemmKernel extends PaletteGemmKernel {
  static create(device: HipGpuDevice, arena: GpuActivationArena,
                executionProfile?: { precision: "fp16" }, options?: GemmKernelOptions): Promise<F16GemmKernel>;
}

/** gemm.ts:2974-3340 */
export declare class F32GemmKernel extends PaletteGemmKernel {
  static create(device: HipGpuDevice, arena: GpuActivationArena,
                executionProfile?: { precision: "fp32" }, options?: GemmKernelOptions): Promise<F32GemmKernel>;
}

/** encoder.ts:356-368 */
export interface EncoderGemmBackend {
  readonly portableF16LoadEncoding: null;
  readonly transientPaletteParameterBytes: number;
  readonly transientPaletteParameterUsedSlots: number;
  readonly transientPaletteDispatchCount: number;
  readonly transientPaletteExpandedBytes: number;
  createDispatch(descriptor: GemmDescriptor): GemmDispatch;
  createPreparedPaletteWeight(descriptor: GemmDescriptor, scratchOffset: number): PreparedPaletteWeight;
}

export declare function createEncoderGemmBackend(kernel: F16GemmKernel | F32GemmKernel): EncoderGemmBackend;
export declare function paletteBitsForLayout(layout: string): 5 | 6 | undefined;
export declare function createGpuTensor(device: HipGpuDevice,
                                        records: { sourceRecord: TensorRecord; runtimeRecord: TensorRecord; label?: string },
                                        data: ArrayBuffer | ArrayBufferView): GpuTensor;
export declare function paletteTensorRecords(options: {
  paletteBits: 5 | 6; inner: number; columns: number; paletteGroups?: number; paletteDtype?: "float16" | "float32";
}): {
  weight: { sourceRecord: TensorRecord; runtimeRecord: TensorRecord };
  palette: { sourceRecord: TensorRecord; runtimeRecord: TensorRecord };
};

/* ---- Conformer convolution tail (src/webgpu/kernels/conformer-conv.ts) ---- */

export declare const CONFORMER_CONV_CHANNELS: 1024;
export declare const CONFORMER_CONV_POINTWISE_CHANNELS: 2048;
export declare const CONFORMER_CONV_KERNEL_SIZE: 9;
export declare const CONFORMER_DEPTHWISE_WEIGHT_LAYOUT: "kernel-channel-vec4";
export declare const CONFORMER_FOLDED_BATCH_NORM_LAYOUT: "channel";

/** conformer-conv.ts:31-45 */
export interface ConformerConvShape {
  readonly batchSize: number;
  readonly frames: number;
}
export interface ConformerConvPlan extends ConformerConvShape {
  readonly rows: number;
  readonly inputByteLength: number;
  readonly outputByteLength: number;
  readonly validLengthsByteLength: number;
  readonly depthwiseWeightByteLength: number;
  readonly affineByteLength: number;
  /** This library's launch grid (one dimension used). */
  readonly workgroups: readonly [number, number, number];
  /** 0: the GLU window lives in registers. */
  readonly workgroupStorageBytes: number;
  readonly blockThreads: number;
  readonly algorithmicBytes: number;
  readonly kernel: string;
}

/** conformer-conv.ts:47-64 */
export interface FusedConformerConvDescriptor extends ConformerConvShape {
  readonly label: string;
  /** Profile-scalar [rows, 2048]: GLU values [0, 1024), gates [1024, 2048). */
  readonly pointwiseInput: ArenaSlice;
  /** Profile-scalar [9, 1024], kernel-channel-vec4. */
  readonly depthwiseWeights: GpuTensor;
  /** f32 [1024] gamma / sqrt(var + eps). */
  readonly batchNormScale: GpuTensor;
  /** f32 [1024] beta - mean * scale. */
  readonly batchNormShift: GpuTensor;
  /** u32 valid frames per window. */
  readonly validLengths: ArenaSlice;
  /** Profile-scalar [rows, 1024]; must not overlap the pointwise input. */
  readonly output: ArenaSlice;
  /**
   * This library only: the pointwise input is the [rows, 1024] GLU written by
   * a GEMM with the GLU epilogue (PK_CONV_INPUT_GLU).
   */
  readonly pointwiseInputIsGlu?: boolean;
}

export declare function planFusedConformerConv(shape: ConformerConvShape,
                                               executionProfile?: { precision: "fp16" | "fp32" }): ConformerConvPlan;
export declare function conformerConvTensorRecords(options?: { dtype?: "float16" | "float32" }): {
  depthwiseWeights: { sourceRecord: TensorRecord; runtimeRecord: TensorRecord };
  batchNormScale: { sourceRecord: TensorRecord; runtimeRecord: TensorRecord };
  batchNormShift: { sourceRecord: TensorRecord; runtimeRecord: TensorRecord };
};

/** conformer-conv.ts:117-162 */
export declare class FusedConformerConvDispatch {
  readonly label: string;
  readonly result: { readonly output: ArenaSlice; readonly rows: number; readonly channels: 1024 };
  encode(encoder: HipCommandEncoder, timestampWrites?: TimestampWrites, shape?: EncoderDispatchShape): void;
  destroy(): void;
  plan(activeBatch?: number): ConformerConvPlan;
}

/** conformer-conv.ts:174-350 */
export declare class FusedConformerConvKernel {
  static create(device: HipGpuDevice, arena: GpuActivationArena, uniformParameterCapacity: number,
                executionProfile?: { precision: "fp16" | "fp32" }): Promise<FusedConformerConvKernel>;
  readonly uniformParameterPoolBytes: number;
  readonly uniformParameterPoolUsedSlots: number;
  validateDescriptor(descriptor: FusedConformerConvDescriptor): void;
  createDispatch(descriptor: FusedConformerConvDescriptor): FusedConformerConvDispatch;
  destroy(): void;
}

/* ---- Relative-position attention (src/webgpu/kernels/attention.ts) ---- */

/** attention.ts:39-49 */
export interface RelativeAttentionDescriptor {
  readonly label: string;
  /** Profile-scalar [rows, 3072]: Q, K, V blocks of 1024, head h at 128h. */
  readonly qkv: ArenaSlice;
  /** "head-vector-position-vec4" [8, 32, 2T-1, 4] package tensor (or, with
   *  projectedPositionsRowMajor, a [2T-1, 1024] arena slice). */
  readonly projectedPositions: GpuTensor | ArenaSlice;
  readonly biasU: GpuTensor;
  readonly biasV: GpuTensor;
  readonly validLengths: ArenaSlice;
  /** Profile-scalar [rows, 1024]; must not overlap qkv. */
  readonly output: ArenaSlice;
  readonly batchSize: number;
  /** 1..4096 here (the reference: 1..192). */
  readonly frames: number;
  /** This library only: positions are a row-major [2T-1, 1024] arena slice. */
  readonly projectedPositionsRowMajor?: boolean;
}

export interface RelativeAttentionPlan {
  readonly workgroups: readonly [number, number, number];
  readonly blockThreads: number;
  readonly workgroupStorageBytes: number;
  readonly queryTiles: number;
  readonly algorithmicBytes: number;
  readonly kernel: string;
}

/** attention.ts:51-97 */
export declare class RelativeAttentionDispatch {
  readonly label: string;
  readonly output: ArenaSlice;
  encode(encoder: HipCommandEncoder, timestampWrites?: TimestampWrites, shape?: EncoderDispatchShape): void;
  destroy(): void;
  plan(activeBatch?: number): RelativeAttentionPlan;
}

/** attention.ts:105-321 */
export declare class RelativeAttentionKernel {
  static create(device: HipGpuDevice, arena: GpuActivationArena, uniformParameterCapacity: number,
                executionProfile?: { precision: "fp16" | "fp32" }): Promise<RelativeAttentionKernel>;
  readonly uniformParameterPoolBytes: number;
  readonly uniformParameterPoolUsedSlots: number;
  validateDescriptor(descriptor: RelativeAttentionDescriptor): void;
  createDispatch(descriptor: RelativeAttentionDescriptor): RelativeAttentionDispatch;
  destroy(): void;
}

export declare function relativeAttentionTensorRecords(frames: number, options?: { dtype?: "float16" | "float32" }): {
  projectedPositions: { sourceRecord: TensorRecord; runtimeRecord: TensorRecord };
  biasU: { sourceRecord: TensorRecord; runtimeRecord: TensorRecord };
  biasV: { sourceRecord: TensorRecord; runtimeRecord: TensorRecord };
};

/* ---- Row LayerNorm (src/webgpu/kernels/layernorm.ts) ---- */

/** layernorm.ts LayerNormDescriptor */
export interface LayerNormDescriptor {
  readonly label: string;
  readonly input: ArenaSlice;
  /** May be the input slice (in place). */
  readonly output: ArenaSlice;
  /** float32 "channel" [channels] package tensors. */
  readonly gamma: GpuTensor;
  readonly beta: GpuTensor;
  readonly rows: number;
  /** Multiple of 4. */
  readonly channels: number;
  /** Default 1e-5. */
  readonly epsilon?: number;
}

/** layernorm.ts:29-72 */
export declare class LayerNormDispatch {
  readonly label: string;
  readonly output: ArenaSlice;
  encode(encoder: HipCommandEncoder, timestampWrites?: TimestampWrites, shape?: EncoderDispatchShape): void;
  destroy(): void;
}

/** layernorm.ts:74-247 */
export declare class LayerNormKernel {
  static create(device: HipGpuDevice, arena: GpuActivationArena, uniformParameterCapacity: number,
                executionProfile?: { precision: "fp16" | "fp32" }): Promise<LayerNormKernel>;
  readonly uniformParameterPoolBytes: number;
  validateDescriptor(descriptor: LayerNormDescriptor): void;
  createDispatch(descriptor: LayerNormDescriptor): LayerNormDispatch;
  destroy(): void;
}

export declare function channelTensorRecords(channels: number): { sourceRecord: TensorRecord; runtimeRecord: TensorRecord };

/* ---- Subsampling front end (src/webgpu/kernels/subsampling.ts) ---- */

/** subsampling.ts:119-122 */
export declare function subsamplingOutputDimension(input: number): number;
/** subsampling.ts:124-135 */
export declare function subsamplingValidLength(featureLength: number, steps: number): number;

/** subsampling.ts FusedSubsamplingConv0Depthwise2Descriptor (:98-111) */
export interface FusedSubsamplingConv0Depthwise2Descriptor {
  readonly label: string;
  /** f32 feature-major [batch, 128, inputHeight]. */
  readonly input: ArenaSlice;
  readonly conv0Weights: GpuTensor;
  readonly conv0Bias: GpuTensor;
  readonly depthwiseWeights: GpuTensor;
  readonly depthwiseBias: GpuTensor;
  /** Channel-last [batch, Ho, Wo, 256]. */
  readonly output: ArenaSlice;
  readonly validLengths: ArenaSlice;
  readonly validLengthBatchOffset?: number;
  readonly batchSize: number;
  /** Feature frames (the reference fixes 1501; any count here). */
  readonly inputHeight: number;
  /** 128 */
  readonly inputWidth: number;
  /** 256 */
  readonly channels: number;
}

/** subsampling.ts DepthwiseSubsamplingDescriptor (:84-96) */
export interface DepthwiseSubsamplingDescriptor {
  readonly label: string;
  readonly input: ArenaSlice;
  readonly weights: GpuTensor;
  readonly bias: GpuTensor;
  readonly output: ArenaSlice;
  readonly validLengths: ArenaSlice;
  readonly validLengthBatchOffset?: number;
  readonly validLengthSubsamplingSteps: number;
  readonly batchSize: number;
  readonly inputHeight: number;
  readonly inputWidth: number;
  readonly channels: number;
}

/** subsampling.ts SubsamplingTimeMaskDescriptor (:573-585) */
export interface SubsamplingTimeMaskDescriptor {
  readonly label: string;
  readonly values: ArenaSlice;
  readonly validLengths: ArenaSlice;
  readonly batchSize: number;
  readonly height: number;
  readonly width: number;
  readonly channels: number;
  readonly validLengthBatchOffset?: number;
  readonly validLengthSubsamplingSteps: number;
}

export interface SubsamplingPlan {
  readonly workgroups: readonly [number, number, number];
  readonly outputHeight: number;
  readonly outputWidth: number;
  readonly blockThreads: number;
  readonly workgroupStorageBytes: number;
  readonly algorithmicBytes: number;
  readonly flops: number;
  readonly kernel: string;
}

/** subsampling.ts:208-248 and :587-618; shape.batchSize (this library only) selects a prefix. */
export declare class SubsamplingDispatch {
  readonly label: string;
  readonly output: ArenaSlice;
  readonly outputHeight: number;
  readonly outputWidth: number;
  encode(encoder: HipCommandEncoder, timestampWrites?: TimestampWrites, shape?: { batchSize?: number }): void;
  destroy(): void;
  plan(activeBatch?: number): SubsamplingPlan;
}

export declare class FusedSubsamplingConv0Depthwise2Kernel {
  static create(device: HipGpuDevice, arena: GpuActivationArena, uniformParameterCapacity: number,
                executionProfile?: { precision: "fp16" | "fp32" }): Promise<FusedSubsamplingConv0Depthwise2Kernel>;
  validateDescriptor(descriptor: FusedSubsamplingConv0Depthwise2Descriptor): void;
  createDispatch(descriptor: FusedSubsamplingConv0Depthwise2Descriptor): SubsamplingDispatch;
  destroy(): void;
}

export declare class DepthwiseSubsamplingKernel {
  static create(device: HipGpuDevice, arena: GpuActivationArena, uniformParameterCapacity: number,
                executionProfile?: { precision: "fp16" | "fp32" }): Promise<DepthwiseSubsamplingKernel>;
  validateDescriptor(descriptor: DepthwiseSubsamplingDescriptor): void;
  createDispatch(descriptor: DepthwiseSubsamplingDescriptor): SubsamplingDispatch;
  destroy(): void;
}

export declare class SubsamplingTimeMaskKernel {
  static create(device: HipGpuDevice, arena: GpuActivationArena, uniformParameterCapacity: number,
                executionProfile?: { precision: "fp16" | "fp32" }): Promise<SubsamplingTimeMaskKernel>;
  validateDescriptor(descriptor: SubsamplingTimeMaskDescriptor): void;
  createDispatch(descriptor: SubsamplingTimeMaskDescriptor): SubsamplingDispatch;
  destroy(): void;
}

export declare function subsamplingTensorRecords(options?: { dtype?: "float16" | "float32"; channels?: number }): {
  conv0Weights: { sourceRecord: TensorRecord; runtimeRecord: TensorRecord };
  depthwiseWeights: { sourceRecord: TensorRecord; runtimeRecord: TensorRecord };
  bias: { sourceRecord: TensorRecord; runtimeRecord: TensorRecord };
};

/* ---- Encoder graph (src/webgpu/encoder.ts) ---- */

/** encoder.ts:441-479 */
export declare function deriveEncoderValidLength(featureLength: number): number;
export declare function deriveEncoderValidLengths(featureLengths: readonly number[], batchSize?: number): Uint32Array;

/** The ParakeetGpuPackage surface the graph reads (package.ts:52-): tensors by name. */
export interface EncoderModel {
  tensor(name: string): GpuTensor;
}

export interface ParakeetEncoderGraphOptions {
  /** Windows (default 16). */
  readonly batchSize?: number;
  /** Conformer layers (default 24). */
  readonly layers?: number;
  /** fbank frames per window (default 1501). */
  readonly featureFrames?: number;
  /** PW1's GLU epilogue (this library only). */
  readonly fusedGlu?: boolean;
  /** Active prefixes keep the capacity's kernels (this library only; default: a dedicated graph's plans). */
  readonly prefixSamePlan?: boolean;
  readonly label?: string;
  /** encoder.ts:1299-1305: fp16 (default) or fp32 (an fp32 package; f32 outputs). */
  readonly executionProfile?: { precision: "fp16" | "fp32" };
}

/** encoder.ts:1200-1862 */
export declare class ParakeetEncoderGraph {
  static create(device: HipGpuDevice, model: EncoderModel & { readonly precision?: string },
                options?: ParakeetEncoderGraphOptions): Promise<ParakeetEncoderGraph>;
  readonly batchSize: number;
  readonly frames: number;
  /** "f16" or "f32": the element of the output buffers. */
  readonly precision: "f16" | "f32";
  /** 6 front-end launches + 15 per layer + the projector. */
  readonly dispatchCount: number;
  readonly outputBuffer: HipBuffer;
  readonly projectedOutputBuffer: HipBuffer;
  uploadFeatures(features: Float32Array): void;
  uploadValidFeatureLengths(featureLengths: readonly number[]): Uint32Array;
  encode(encoder: HipCommandEncoder, validFeatureLengths: readonly number[],
         options?: { useGraph?: boolean; timestamps?: { querySet: HipTimestampQuerySet; first?: number } }): Uint32Array;
  destroy(): void;
}

export declare const PARAKEET_FEATURE_BINS: 128;
export declare const PARAKEET_FEATURE_FRAMES: 1501;
export declare const PARAKEET_ENCODER_FRAMES: 188;
export declare const PARAKEET_PROJECTED_CHANNELS: 640;
export declare const ENCODER_LAYER_DISPATCHES: 15;

/* ------------------------------------------------------------ TDT decoder */

export declare const TDT_DECODER_OVERFLOW: 1;
/** A team barrier gave up waiting (this library only). */
export declare const TDT_DECODER_SYNC_TIMEOUT: 2;
/** The causes in one window's status word. */
export declare function decodeTdtStatus(word: number): { overflow: boolean; syncTimeout: boolean; unknown: number };
export declare const TDT_BLANK_TOKEN: 1024;

/** tdt-decoder.ts:39-52 (one workgroup per window here). */
export interface TdtDecoderExecutionPlan {
  readonly workgroupCount: number;
  readonly blockThreads: number;
  readonly predictorScratchByteLength: number;
}
export declare function planTdtDecoderExecution(batchSize: number): TdtDecoderExecutionPlan;

/** tdt-decoder.ts:54-82: every slice comes from the kernel's arena. */
export interface TdtDecoderDescriptor {
  readonly label?: string;
  readonly encoderProjected: ArenaSlice;
  readonly encodedLengths: ArenaSlice;
  readonly decodeStarts: ArenaSlice;
  readonly decodeEnds: ArenaSlice;
  readonly flushFinals: ArenaSlice;
  readonly state: ArenaSlice;
  readonly predictorScratch: ArenaSlice;
  readonly tokens: ArenaSlice;
  readonly tokenFrames: ArenaSlice;
  readonly tokenDurations: ArenaSlice;
  readonly metadata: ArenaSlice;
  readonly batchSize: number;
  readonly frames: number;
  readonly maxTokens: number;
}

/** tdt-decoder.ts:84-137 */
export declare class TdtDecoderDispatch {
  readonly label: string;
  /** Workgroups per window of the next launch (this library only). */
  readonly teamSize: number;
  /** 0 chooses, 1 one workgroup per window, 8 or 16 a team (this library only). */
  setTeamSize(members: number): void;
  encode(encoder: HipCommandEncoder, timestampWrites?: TimestampWrites, activeBatchSize?: number): void;
  destroy(): void;
}

/** tdt-decoder.ts:139-366 (fp16 and fp32 profiles; teams are fp16 only). */
export declare class PersistentTdtDecoderKernel {
  static create(device: HipGpuDevice, arena: GpuActivationArena, model: EncoderModel & { readonly precision?: string },
                executionProfile?: { precision: "fp16" | "fp32" }): Promise<PersistentTdtDecoderKernel>;
  validateDescriptor(descriptor: TdtDecoderDescriptor): void;
  createDispatch(descriptor: TdtDecoderDescriptor): TdtDecoderDispatch;
}

/* --------------------------------------------------------- package format */

export interface ParakeetTensorRecord {
  readonly shard: string;
  readonly byteOffset: number;
  readonly byteLength: number;
  readonly dtype: "float16" | "float32" | "uint32";
  readonly logicalShape: readonly number[];
  readonly storageShape: readonly number[];
  readonly layout: string;
}
export interface ParakeetFileRecord {
  readonly name: string;
  readonly byteLength: number;
  readonly sha256: string;
}
export interface ParakeetManifest {
  readonly format: "parakeet-webgpu-v1" | "parakeet-webgpu-fp32-v1";
  readonly source: unknown;
  readonly config: Readonly<Record<string, unknown>>;
  readonly files: readonly ParakeetFileRecord[];
  readonly tensors: Readonly<Record<string, ParakeetTensorRecord>>;
}
export interface RuntimePackageMemoryPlan {
  readonly packedDownloadBytes: number;
  readonly retainedRuntimeBytes: number;
  readonly expandedRuntimeBytes: number;
  readonly runtimeGpuBytes: number;
  readonly largestRuntimeShardBytes: number;
  readonly loaderPeakGpuBytes: number;
  readonly runtimeBufferCount: number;
}
export interface RuntimePackagePlan {
  readonly buffers: readonly { id: string; label: string; byteLength: number; tensorCount: number }[];
  readonly tensors: ReadonlyMap<string, { name: string; sourceRecord: ParakeetTensorRecord; runtimeRecord: TensorRecord }>;
  readonly shards: readonly ({ file: ParakeetFileRecord; hashOnly: true } |
                             { file: ParakeetFileRecord; hashOnly: false; runtimeBufferId: string })[];
  readonly memory: RuntimePackageMemoryPlan;
}
export declare const PARAKEET_FP16_PACKAGE_FORMAT: "parakeet-webgpu-v1";
export declare const PARAKEET_FP32_PACKAGE_FORMAT: "parakeet-webgpu-fp32-v1";
export declare const PARAKEET_FP16_MANIFEST_SHA256: string;
export declare const PARAKEET_FP32_MANIFEST_SHA256: string;
export declare function parseParakeetManifest(value: unknown): ParakeetManifest;
export declare function parakeetManifestPrecision(manifest: ParakeetManifest): "fp16" | "fp32";
export declare function parakeetManifestSha256(precision: "fp16" | "fp32"): string;
export declare function planRuntimePackage(manifest: ParakeetManifest): RuntimePackagePlan;
export declare function alignRuntimeOffset(value: number): number;

export interface ParakeetPackageLoadOptions {
  readonly expectedPrecision: "fp16" | "fp32";
  /** A manifest other than the two published ones (this library only). */
  readonly manifestSha256?: string;
  readonly onProgress?: (progress: { phase: string; file?: string; loadedBytes: number; totalBytes: number }) => void;
}

/** package.ts:52-232 over HIP: one HBM allocation per resident shard. */
export declare class ParakeetGpuPackage implements EncoderModel {
  static load(device: HipGpuDevice, manifestPath: string, options: ParakeetPackageLoadOptions): Promise<ParakeetGpuPackage>;
  readonly memory: RuntimePackageMemoryPlan;
  readonly precision: "fp16" | "fp32";
  readonly manifestUrl: string;
  readonly manifestSha256: string;
  readonly manifestListedBytes: number;
  readonly manifest: ParakeetManifest;
  readonly tokenizer: unknown;
  tensor(name: string): GpuTensor;
  releaseInitializationMetadata(): void;
  destroy(): void;
}
