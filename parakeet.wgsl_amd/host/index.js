// @ts-check
/*
 * parakeet.wgsl_amd/host - the palette GEMM op interface of parakeet.wgsl
 * over HIP, for Node.
 *
 * It mirrors the reference's TypeScript GEMM owners so the encoder graph can
 * bind to it unchanged:
 *   F16GemmKernel / F32GemmKernel      src/webgpu/kernels/gemm.ts:483-855, :2974-3340
 *     .create(device, arena, profile)  gemm.ts:519-619
 *     .createDispatch(descriptor)      gemm.ts:621-704, :3097-3182
 *     .createPreparedPaletteWeight     gemm.ts:706-748, :3186-3232
 *     transientPalette* counters       gemm.ts:502-516 (always 0 here: the
 *                                      fused kernels never expand weights)
 *   GemmDispatch.encode / destroy      gemm.ts:400-470
 *   createEncoderGemmBackend(kernel)   the EncoderGemmBackend adapter of
 *                                      src/webgpu/encoder.ts:356-432
 *   GpuActivationArena                 src/webgpu/arena.ts (slice, binding,
 *                                      upload, destroy)
 *   paletteBitsForLayout               src/model/runtime-plan.ts:352-368
 *   FusedConformerConvKernel           src/webgpu/kernels/conformer-conv.ts:174-350
 *     .create(device, arena, capacity, profile)  :194-253
 *     .createDispatch(descriptor)      :255-344 (record checks :403-432 here,
 *                                      the numeric contract in pk_conv_validate)
 *   FusedConformerConvDispatch.encode / destroy  :117-162
 *   planFusedConformerConv             :72-115 (rows and byte lengths are the
 *                                      reference's; workgroups is this
 *                                      library's own launch)
 *   RelativeAttentionKernel            src/webgpu/kernels/attention.ts:105-321
 *     .create / .createDispatch        :130-314 (record checks :323-370 here,
 *                                      the numeric contract in pk_attention_validate)
 *   RelativeAttentionDispatch.encode / destroy   :51-97
 *   LayerNormKernel / LayerNormDispatch  src/webgpu/kernels/layernorm.ts:29-281
 *   FusedSubsamplingConv0Depthwise2Kernel, DepthwiseSubsamplingKernel,
 *   SubsamplingTimeMaskKernel, SubsamplingDispatch,
 *   subsamplingOutputDimension / subsamplingValidLength
 *                                      src/webgpu/kernels/subsampling.ts:119-790
 *   ParakeetEncoderGraph               src/webgpu/encoder.ts:1200-1862 (create
 *     from a model's tensors, uploadFeatures, uploadValidFeatureLengths,
 *     encode: front end, 24 layers, projector, as one native graph)
 *   deriveEncoderValidLength(s)        encoder.ts:441-479
 * The WebGPU device, queue, buffers and command encoder are replaced by HIP
 * equivalents with the same shapes (HipGpuDevice, queue.writeBuffer /
 * submit / onSubmittedWorkDone, createCommandEncoder().finish()).
 *
 * Record-level checks (tensor layouts, dtypes, shapes of the package
 * records) run here with the reference's messages; the numeric contract
 * (shape, registry, palette geometry, binding sizes) is checked by the C ABI
 * (pk_gemm_validate), which throws the same messages. Written as plain
 * ES2019 CommonJS with JSDoc types (index.d.ts declares the API) so it runs
 * on the Node 12 of this image without a TypeScript compiler.
 */
"use strict";

const path = require("path");

/** @type {any} */
let nativeModule = null;
function native() {
  if (nativeModule === null) {
    // The addon is built in-tree next to libpk_palette.so; there is no
    // fallback: without it the host fails loudly. PK_NAPI_ADDON names another
    // build of it (the host-side sanitizer build of the CPU tests).
    nativeModule = require(process.env.PK_NAPI_ADDON || path.join(__dirname, "..", "lib", "pk_napi.node"));
  }
  return nativeModule;
}

const STORAGE_ALIGNMENT = 256;
const PALETTE_LAYOUT = "output-group-by-palette-lut";
const F16_TILE_INNER = 32;
const F32_TILE_INNER = 32;
const FP32_PACKED_K = 4;
const TRANSIENT_PALETTE_WEIGHT_SCRATCH_BYTES = 8650752;
const FP32_TRANSIENT_PALETTE_WEIGHT_SCRATCH_BYTES = 17301504;
const REQUIRE_PRODUCTION_SIGNATURE = 1;
const GEMM_GLU = 2;
const GEMM_ROW_NORM = 4;
const GEMM_CACHED_OUTPUT = 8;
const CONV_INPUT_GLU = 1;

/** runtime-plan.ts:352-368 */
function paletteBitsForLayout(layout) {
  if (layout === "k-by-output-row-major-palette5-lsb-u32") return 5;
  if (layout === "k-by-output-row-major-palette6-lsb-u32") return 6;
  return undefined;
}

function shapeKey(shape) {
  return Array.prototype.join.call(shape, ",");
}

function isSafe(n) {
  return Number.isSafeInteger(n);
}

/* ---------------------------------------------------------------- device */

class HipBuffer {
  constructor(device, label, size, address) {
    this.device = device;
    this.label = label;
    this.size = size;
    /** device address (BigInt) */
    this.address = address;
    this.destroyed = false;
  }

  destroy() {
    if (this.destroyed) return;
    this.destroyed = true;
    native().free(this.device.context, this.address);
  }
}

class HipQueue {
  constructor(device) {
    this.device = device;
  }

  /** GPUQueue.writeBuffer: the copy is complete on return. */
  writeBuffer(buffer, bufferOffset, data) {
    if (buffer.destroyed) throw new Error(`${buffer.label} was destroyed`);
    const bytes = data.byteLength;
    if (!isSafe(bufferOffset) || bufferOffset < 0 || bufferOffset + bytes > buffer.size)
      throw new RangeError(`Write does not fit ${buffer.label}`);
    native().upload(this.device.context, buffer.address, bufferOffset, data);
  }

  /** Reads `size` bytes at `offset` back to the host (mapAsync readback). */
  readBuffer(buffer, offset, size) {
    if (!isSafe(offset) || !isSafe(size) || offset < 0 || size < 0 || offset + size > buffer.size)
      return Promise.reject(new RangeError(`Read does not fit ${buffer.label}`));
    return this.onSubmittedWorkDone().then(() => {
      const out = new ArrayBuffer(size);
      native().download(this.device.context, buffer.address, offset, out);
      return out;
    });
  }

  /** Runs the recorded commands in order on the device's stream. */
  submit(commandBuffers) {
    for (const commandBuffer of commandBuffers) {
      if (commandBuffer.submitted) throw new Error(`${commandBuffer.label} was already submitted`);
      commandBuffer.submitted = true;
      for (const command of commandBuffer.commands) command();
    }
  }

  /** Resolves once every submitted command has finished (a worker-thread wait). */
  onSubmittedWorkDone() {
    return native().synchronizeAsync(this.device.context);
  }
}

class HipCommandEncoder {
  constructor(device, label) {
    this.device = device;
    this.label = label;
    /** @type {Array<() => void>} */
    this.commands = [];
    this.finished = false;
  }

  /** Appends one command (used by GemmDispatch.encode). */
  record(command) {
    if (this.finished) throw new Error(`${this.label} is already finished`);
    this.commands.push(command);
  }

  finish() {
    this.finished = true;
    return { label: this.label, commands: this.commands.slice(), submitted: false };
  }
}

/** Timestamp queries as HIP events (GpuTimestampRecorder, timestamp.ts:44-80). */
class HipTimestampQuerySet {
  constructor(device, count) {
    this.device = device;
    this.events = [];
    for (let i = 0; i < count; ++i) this.events.push(native().eventCreate(device.context));
  }

  write(index) {
    native().eventRecord(this.device.context, this.events[index], null);
  }

  /** Milliseconds between two written queries (after the work is done). */
  elapsedMs(begin, end) {
    return native().eventElapsedMs(this.device.context, this.events[begin], this.events[end]);
  }

  destroy() {
    for (const e of this.events) native().eventDestroy(this.device.context, e);
    this.events = [];
  }
}

class HipGpuDevice {
  constructor(context, index) {
    this.context = context;
    this.index = index;
    this.info = native().deviceInfo(context);
    this.queue = new HipQueue(this);
    this.limits = { minStorageBufferOffsetAlignment: STORAGE_ALIGNMENT };
    this.destroyed = false;
  }

  /** A HIP device; `index` selects the GPU (default 0). */
  static create(options) {
    const index = options && options.index !== undefined ? options.index : 0;
    return new HipGpuDevice(native().contextCreate(index), index);
  }

  createBuffer(descriptor) {
    const size = descriptor.size;
    if (!isSafe(size) || size <= 0) throw new RangeError(`Invalid buffer size for ${descriptor.label}`);
    return new HipBuffer(this, descriptor.label || "buffer", size, native().alloc(this.context, size));
  }

  createCommandEncoder(descriptor) {
    return new HipCommandEncoder(this, (descriptor && descriptor.label) || "command-encoder");
  }

  createQuerySet(descriptor) {
    if (descriptor.type !== "timestamp") throw new Error("only timestamp query sets exist");
    return new HipTimestampQuerySet(this, descriptor.count);
  }

  destroy() {
    if (this.destroyed) return;
    this.destroyed = true;
    native().contextDestroy(this.context);
  }
}

/* ----------------------------------------------------------------- arena */

/** arena.ts: one device allocation handed out as 256-byte aligned slices. */
class GpuActivationArena {
  constructor(device, byteLength, label) {
    if (!isSafe(byteLength) || byteLength <= 0)
      throw new RangeError("Activation arena must contain at least one buffer");
    this.device = device;
    this.label = label || "parakeet-activation-arena";
    this.buffer = device.createBuffer({ label: this.label, size: byteLength });
    this.buffers = [this.buffer];
    this.bufferByteLengths = [byteLength];
    this.byteLength = byteLength;
    this.destroyed = false;
  }

  slice(label, byteOffset, byteLength) {
    this.assertAlive();
    if (
      !isSafe(byteOffset) ||
      !isSafe(byteLength) ||
      byteOffset < 0 ||
      byteLength <= 0 ||
      byteOffset % STORAGE_ALIGNMENT !== 0 ||
      byteLength % 4 !== 0 ||
      byteOffset + byteLength > this.byteLength
    ) {
      throw new RangeError(`Invalid activation slice ${label}`);
    }
    return { label, byteOffset, byteLength };
  }

  binding(slice) {
    this.assertAlive();
    if (slice.byteOffset < 0 || slice.byteLength <= 0 || slice.byteOffset + slice.byteLength > this.byteLength)
      throw new RangeError(`Invalid activation slice ${slice.label}`);
    return { buffer: this.buffer, offset: slice.byteOffset, size: slice.byteLength };
  }

  upload(device, destination, data) {
    const binding = this.binding(destination);
    if (data.byteLength > destination.byteLength || data.byteLength % 4 !== 0)
      throw new RangeError(`Upload does not fit ${destination.label}`);
    device.queue.writeBuffer(binding.buffer, binding.offset, data);
  }

  destroy() {
    if (this.destroyed) return;
    this.destroyed = true;
    this.buffer.destroy();
  }

  assertAlive() {
    if (this.destroyed) throw new Error("Activation arena was destroyed");
  }
}

/**
 * A GpuTensor (package.ts:45-50) over a fresh device buffer holding `data`.
 * `records` = {sourceRecord, runtimeRecord} in the package's record shape
 * (manifest.ts:27-35, runtime-plan.ts:41-49).
 */
function createGpuTensor(device, records, data) {
  const byteLength = records.runtimeRecord.byteLength;
  if (data.byteLength !== byteLength) throw new RangeError("tensor data does not match its runtime record");
  const buffer = device.createBuffer({ label: records.label || "tensor", size: byteLength });
  device.queue.writeBuffer(buffer, 0, data);
  return {
    sourceRecord: records.sourceRecord,
    runtimeRecord: records.runtimeRecord,
    buffer,
    binding: { buffer, offset: 0, size: byteLength },
  };
}

/** Package records of a palettized weight and its palette (convert.py:2159-2203). */
function paletteTensorRecords(options) {
  const bits = options.paletteBits;
  const dtype = options.paletteDtype || "float16";
  const codesPerGroup = bits === 5 ? 32 : 16;
  const wordsPerGroup = bits === 5 ? 5 : 3;
  const groups = (options.inner * options.columns) / codesPerGroup;
  const layout = `k-by-output-row-major-palette${bits}-lsb-u32`;
  const weight = {
    dtype: "uint32",
    logicalShape: [options.inner, options.columns],
    storageShape: [groups, wordsPerGroup],
    byteLength: groups * wordsPerGroup * 4,
    layout,
  };
  const entries = 1 << bits;
  const paletteGroups = options.paletteGroups || 1;
  const palette = {
    dtype,
    logicalShape: [paletteGroups, entries],
    storageShape: [paletteGroups, entries],
    byteLength: paletteGroups * entries * (dtype === "float16" ? 2 : 4),
    layout: PALETTE_LAYOUT,
  };
  return {
    weight: { sourceRecord: weight, runtimeRecord: weight },
    palette: { sourceRecord: palette, runtimeRecord: palette },
  };
}

/* ------------------------------------------------------ record checks */

/** requireGemmShape (gemm.ts:971-1010; FP32 :3342-3400), numeric part first. */
function requireWeightRecords(descriptor, fp32) {
  if (
    !isSafe(descriptor.rows) ||
    descriptor.rows <= 0 ||
    !isSafe(descriptor.inner) ||
    descriptor.inner <= 0 ||
    descriptor.inner % (fp32 ? F32_TILE_INNER : F16_TILE_INNER) !== 0 ||
    !isSafe(descriptor.columns) ||
    descriptor.columns <= 0 ||
    descriptor.columns % (fp32 ? FP32_PACKED_K : 8) !== 0
  ) {
    throw new RangeError(`Unsupported${fp32 ? " FP32" : ""} GEMM shape for ${descriptor.label}`);
  }
  const source = descriptor.b.sourceRecord;
  const paletteBits = paletteBitsForLayout(source.layout);
  const what = fp32 ? " FP32" : "";
  if (shapeKey(source.logicalShape) !== `${descriptor.inner},${descriptor.columns}`) {
    throw new Error(
      `${descriptor.label}${what} weight package does not match K=${descriptor.inner}, N=${descriptor.columns}`,
    );
  }
  if (paletteBits === undefined || source.dtype !== "uint32") {
    throw new Error(`${descriptor.label} has an unsupported${what} weight format`);
  }
  const codesPerGroup = paletteBits === 5 ? 32 : 16;
  const wordsPerGroup = paletteBits === 5 ? 5 : 3;
  const elements = descriptor.inner * descriptor.columns;
  if (elements % codesPerGroup !== 0) {
    throw new Error(`${descriptor.label}${what} palette codes are not group aligned`);
  }
  const groups = elements / codesPerGroup;
  if (source.byteLength !== groups * wordsPerGroup * 4 || shapeKey(source.storageShape) !== `${groups},${wordsPerGroup}`) {
    throw new Error(`${descriptor.label} has invalid packed${what} palette indices`);
  }
  return paletteBits;
}

/** requireRuntimeWeight's record part (gemm.ts:1069-1161; FP32 :3422-3470). */
function requirePaletteRecords(descriptor, paletteBits, fp32) {
  const runtime = descriptor.b.runtimeRecord;
  const source = descriptor.b.sourceRecord;
  const palette = descriptor.bPalette;
  const entries = 1 << paletteBits;
  const paletteDtype = fp32 ? "float32" : "float16";
  const elem = fp32 ? 4 : 2;
  const groups = palette === undefined ? undefined : palette.runtimeRecord.storageShape[0];
  if (
    paletteBitsForLayout(runtime.layout) !== paletteBits ||
    runtime.dtype !== "uint32" ||
    runtime.layout !== source.layout ||
    shapeKey(runtime.logicalShape) !== `${descriptor.inner},${descriptor.columns}` ||
    shapeKey(runtime.storageShape) !== shapeKey(source.storageShape) ||
    runtime.byteLength !== source.byteLength ||
    palette === undefined ||
    palette.sourceRecord.dtype !== paletteDtype ||
    palette.sourceRecord.layout !== PALETTE_LAYOUT ||
    palette.runtimeRecord.dtype !== paletteDtype ||
    palette.runtimeRecord.layout !== PALETTE_LAYOUT ||
    shapeKey(palette.runtimeRecord.logicalShape) !== shapeKey(palette.sourceRecord.logicalShape) ||
    shapeKey(palette.runtimeRecord.storageShape) !== `${groups},${entries}` ||
    palette.runtimeRecord.byteLength !== groups * entries * elem ||
    !isSafe(descriptor.paletteGroupColumns) ||
    descriptor.paletteGroupColumns <= 0 ||
    descriptor.paletteGroupColumns * groups !== descriptor.columns
  ) {
    throw new Error(`${descriptor.label} has invalid transient${fp32 ? " FP32" : ""} palette weights`);
  }
  return groups;
}

/* ------------------------------------------------- conformer convolution */

const CONFORMER_CONV_CHANNELS = 1024;
const CONFORMER_CONV_POINTWISE_CHANNELS = 2048;
const CONFORMER_CONV_KERNEL_SIZE = 9;
const CONFORMER_DEPTHWISE_WEIGHT_LAYOUT = "kernel-channel-vec4";
const CONFORMER_FOLDED_BATCH_NORM_LAYOUT = "channel";

function precisionOf(executionProfile) {
  return executionProfile === undefined || executionProfile.precision === "fp16" ? "f16" : "f32";
}

/** planFusedConformerConv (conformer-conv.ts:72-115). */
function planFusedConformerConv(shape, executionProfile) {
  for (const [value, name] of [[shape.batchSize, "batchSize"], [shape.frames, "frames"]]) {
    if (!isSafe(value) || value <= 0) throw new RangeError(`${name} must be a positive integer`);
  }
  const plan = native().convPlanShape(precisionOf(executionProfile), shape.batchSize, shape.frames, 0);
  return Object.assign({ batchSize: shape.batchSize, frames: shape.frames }, plan);
}

/** requirePackedTensor (conformer-conv.ts:403-432), on the tensor's runtime record. */
function requirePackedTensor(tensor, dtype, shape, layout, byteLength, label) {
  const record = tensor.runtimeRecord;
  const storageShape = shape.length === 2 ? [shape[0], shape[1] / 4, 4] : shape;
  if (
    record.dtype !== dtype ||
    record.layout !== layout ||
    record.byteLength !== byteLength ||
    shapeKey(record.logicalShape) !== shapeKey(shape) ||
    shapeKey(record.storageShape) !== shapeKey(storageShape)
  ) {
    throw new Error(
      `${label} must be ${dtype} ${layout} logical [${shape.join(",")}], ` +
        `storage [${storageShape.join(",")}], ${byteLength} bytes`,
    );
  }
}

/** Package records of the depthwise weights and folded batch norm. */
function conformerConvTensorRecords(options) {
  const dtype = (options && options.dtype) || "float16";
  const scalar = dtype === "float16" ? 2 : 4;
  const weights = {
    dtype,
    logicalShape: [CONFORMER_CONV_KERNEL_SIZE, CONFORMER_CONV_CHANNELS],
    storageShape: [CONFORMER_CONV_KERNEL_SIZE, CONFORMER_CONV_CHANNELS / 4, 4],
    byteLength: CONFORMER_CONV_KERNEL_SIZE * CONFORMER_CONV_CHANNELS * scalar,
    layout: CONFORMER_DEPTHWISE_WEIGHT_LAYOUT,
  };
  const affine = {
    dtype: "float32",
    logicalShape: [CONFORMER_CONV_CHANNELS],
    storageShape: [CONFORMER_CONV_CHANNELS],
    byteLength: CONFORMER_CONV_CHANNELS * 4,
    layout: CONFORMER_FOLDED_BATCH_NORM_LAYOUT,
  };
  return {
    depthwiseWeights: { sourceRecord: weights, runtimeRecord: weights },
    batchNormScale: { sourceRecord: affine, runtimeRecord: affine },
    batchNormShift: { sourceRecord: affine, runtimeRecord: affine },
  };
}

function addressOf(binding) {
  return binding.buffer.address + BigInt(binding.offset);
}

class FusedConformerConvDispatch {
  constructor(label, result, op, batchSize) {
    this.label = label;
    this.result = result;
    this.op = op;
    this.batchSize = batchSize;
    this.destroyed = false;
  }

  /** encode (conformer-conv.ts:128-157): shape.batchSize selects the active windows. */
  encode(encoder, timestampWrites, shape) {
    if (this.destroyed) throw new Error(`${this.label} was destroyed`);
    const active = shape === undefined || shape.batchSize === undefined ? this.batchSize : shape.batchSize;
    if (!isSafe(active) || active <= 0 || active > this.batchSize)
      throw new RangeError(`${this.label} active batch must be in [1, ${this.batchSize}]`);
    const op = this.op;
    encoder.record(() => {
      const qs = timestampWrites ? timestampWrites.querySet : null;
      const begin = qs && timestampWrites.beginningOfPassWriteIndex !== undefined
        ? qs.events[timestampWrites.beginningOfPassWriteIndex] : null;
      const end = qs && timestampWrites.endOfPassWriteIndex !== undefined
        ? qs.events[timestampWrites.endOfPassWriteIndex] : null;
      native().convEnqueue(op, active, null, begin, end);
    });
  }

  destroy() {
    if (this.destroyed) return;
    this.destroyed = true;
    native().convDestroy(this.op);
  }

  plan(activeBatch) {
    return native().convPlan(this.op, activeBatch || 0);
  }
}

class FusedConformerConvKernel {
  constructor(device, arena, executionProfile) {
    this.device = device;
    this.arena = arena;
    this.precision = precisionOf(executionProfile);
    this.executionProfile = executionProfile;
    this.destroyed = false;
  }

  /** The kernels are compiled into the library: no pipeline or uniform pool to build. */
  static create(device, arena, uniformParameterCapacity, executionProfile) {
    return Promise.resolve(new FusedConformerConvKernel(device, arena, executionProfile));
  }

  get uniformParameterPoolBytes() {
    return 0;
  }

  get uniformParameterPoolUsedSlots() {
    return 0;
  }

  nativeDescriptor(descriptor) {
    const plan = planFusedConformerConv(descriptor, this.executionProfile);
    const dtype = this.precision === "f16" ? "float16" : "float32";
    requirePackedTensor(descriptor.depthwiseWeights, dtype,
                        [CONFORMER_CONV_KERNEL_SIZE, CONFORMER_CONV_CHANNELS], CONFORMER_DEPTHWISE_WEIGHT_LAYOUT,
                        plan.depthwiseWeightByteLength, `${descriptor.label} depthwise weights`);
    requirePackedTensor(descriptor.batchNormScale, "float32", [CONFORMER_CONV_CHANNELS],
                        CONFORMER_FOLDED_BATCH_NORM_LAYOUT, plan.affineByteLength,
                        `${descriptor.label} folded batch norm scale`);
    requirePackedTensor(descriptor.batchNormShift, "float32", [CONFORMER_CONV_CHANNELS],
                        CONFORMER_FOLDED_BATCH_NORM_LAYOUT, plan.affineByteLength,
                        `${descriptor.label} folded batch norm shift`);
    const input = this.arena.binding(descriptor.pointwiseInput);
    const output = this.arena.binding(descriptor.output);
    const valid = this.arena.binding(descriptor.validLengths);
    const w = descriptor.depthwiseWeights.binding;
    const scale = descriptor.batchNormScale.binding;
    const shift = descriptor.batchNormShift.binding;
    return {
      label: descriptor.label,
      flags: descriptor.pointwiseInputIsGlu ? CONV_INPUT_GLU : 0,
      precision: this.precision,
      batchSize: descriptor.batchSize,
      frames: descriptor.frames,
      pointwiseInput: addressOf(input),
      pointwiseInputBytes: input.size,
      depthwiseWeights: addressOf(w),
      depthwiseWeightsBytes: w.size,
      batchNormScale: addressOf(scale),
      batchNormScaleBytes: scale.size,
      batchNormShift: addressOf(shift),
      batchNormShiftBytes: shift.size,
      validLengths: addressOf(valid),
      validLengthsBytes: valid.size,
      output: addressOf(output),
      outputBytes: output.size,
    };
  }

  validateDescriptor(descriptor) {
    native().convValidate(this.nativeDescriptor(descriptor));
  }

  /** createDispatch (conformer-conv.ts:255-344). */
  createDispatch(descriptor) {
    if (this.destroyed) throw new Error("Parakeet Conformer convolution kernel was destroyed");
    const op = native().convCreate(this.device.context, this.nativeDescriptor(descriptor));
    const rows = descriptor.batchSize * descriptor.frames;
    return new FusedConformerConvDispatch(
      descriptor.label, { output: descriptor.output, rows, channels: CONFORMER_CONV_CHANNELS }, op,
      descriptor.batchSize);
  }

  destroy() {
    this.destroyed = true;
  }
}

/* ------------------------------------------------ relative attention */

const ATTENTION_POSITIONS_ROW_MAJOR = 1;

/** requireProjectedPositions (attention.ts:323-353). */
function requireProjectedPositions(tensor, positionRows, fp32) {
  const dtype = fp32 ? "float32" : "float16";
  const logical = [positionRows, 1024];
  const storage = [8, 32, positionRows, 4];
  const record = tensor.runtimeRecord;
  if (
    record.dtype !== dtype ||
    record.layout !== "head-vector-position-vec4" ||
    record.byteLength !== positionRows * 1024 * (fp32 ? 4 : 2) ||
    shapeKey(record.logicalShape) !== shapeKey(logical) ||
    shapeKey(record.storageShape) !== shapeKey(storage)
  ) {
    throw new Error(
      `Projected positions must be ${dtype} head-vector-position-vec4, ` +
        `logical [${logical.join(",")}], storage [${storage.join(",")}]`,
    );
  }
}

/** requireAttentionBias (attention.ts:355-370). */
function requireAttentionBias(tensor, label) {
  const record = tensor.runtimeRecord;
  if (
    record.dtype !== "float32" ||
    record.layout !== "head-by-channel" ||
    record.byteLength !== 4096 ||
    shapeKey(record.logicalShape) !== "8,128" ||
    shapeKey(record.storageShape) !== "8,128"
  ) {
    throw new Error(`${label} must be float32 head-by-channel logical/storage [8,128]`);
  }
}

/** Package records of the projected positions and the u / v biases. */
function relativeAttentionTensorRecords(frames, options) {
  const dtype = (options && options.dtype) || "float16";
  const rows = 2 * frames - 1;
  const positions = {
    dtype,
    logicalShape: [rows, 1024],
    storageShape: [8, 32, rows, 4],
    byteLength: rows * 1024 * (dtype === "float16" ? 2 : 4),
    layout: "head-vector-position-vec4",
  };
  const bias = { dtype: "float32", logicalShape: [8, 128], storageShape: [8, 128], byteLength: 4096,
                 layout: "head-by-channel" };
  return {
    projectedPositions: { sourceRecord: positions, runtimeRecord: positions },
    biasU: { sourceRecord: bias, runtimeRecord: bias },
    biasV: { sourceRecord: bias, runtimeRecord: bias },
  };
}

class RelativeAttentionDispatch {
  constructor(label, output, op, batchSize) {
    this.label = label;
    this.output = output;
    this.op = op;
    this.batchSize = batchSize;
    this.destroyed = false;
  }

  /** encode (attention.ts:62-91): shape.batchSize selects the active windows. */
  encode(encoder, timestampWrites, shape) {
    if (this.destroyed) throw new Error(`${this.label} was destroyed`);
    const active = shape === undefined || shape.batchSize === undefined ? this.batchSize : shape.batchSize;
    if (!isSafe(active) || active <= 0 || active > this.batchSize)
      throw new RangeError(`${this.label} active batch must be in [1, ${this.batchSize}]`);
    const op = this.op;
    encoder.record(() => {
      const qs = timestampWrites ? timestampWrites.querySet : null;
      const begin = qs && timestampWrites.beginningOfPassWriteIndex !== undefined
        ? qs.events[timestampWrites.beginningOfPassWriteIndex] : null;
      const end = qs && timestampWrites.endOfPassWriteIndex !== undefined
        ? qs.events[timestampWrites.endOfPassWriteIndex] : null;
      native().attentionEnqueue(op, active, null, begin, end);
    });
  }

  destroy() {
    if (this.destroyed) return;
    this.destroyed = true;
    native().attentionDestroy(this.op);
  }

  plan(activeBatch) {
    return native().attentionPlan(this.op, activeBatch || 0);
  }
}

class RelativeAttentionKernel {
  constructor(device, arena, executionProfile) {
    this.device = device;
    this.arena = arena;
    this.fp32 = executionProfile !== undefined && executionProfile.precision === "fp32";
    this.destroyed = false;
  }

  /** create (attention.ts:130-217): the kernels are compiled into the library. */
  static create(device, arena, uniformParameterCapacity, executionProfile) {
    return Promise.resolve(new RelativeAttentionKernel(device, arena, executionProfile));
  }

  get uniformParameterPoolBytes() {
    return 0;
  }

  get uniformParameterPoolUsedSlots() {
    return 0;
  }

  nativeDescriptor(descriptor) {
    if (!isSafe(descriptor.batchSize) || descriptor.batchSize <= 0 || !isSafe(descriptor.frames) ||
        descriptor.frames <= 0)
      throw new RangeError(`Unsupported attention shape for ${descriptor.label}`);
    const rowMajor = descriptor.projectedPositionsRowMajor === true;
    if (!rowMajor) requireProjectedPositions(descriptor.projectedPositions, descriptor.frames * 2 - 1, this.fp32);
    requireAttentionBias(descriptor.biasU, `${descriptor.label} bias U`);
    requireAttentionBias(descriptor.biasV, `${descriptor.label} bias V`);
    const qkv = this.arena.binding(descriptor.qkv);
    const output = this.arena.binding(descriptor.output);
    const valid = this.arena.binding(descriptor.validLengths);
    const positions = rowMajor ? this.arena.binding(descriptor.projectedPositions) : descriptor.projectedPositions.binding;
    const u = descriptor.biasU.binding;
    const v = descriptor.biasV.binding;
    return {
      label: descriptor.label,
      flags: rowMajor ? ATTENTION_POSITIONS_ROW_MAJOR : 0,
      precision: this.fp32 ? "f32" : "f16",
      batchSize: descriptor.batchSize,
      frames: descriptor.frames,
      qkv: addressOf(qkv),
      qkvBytes: qkv.size,
      projectedPositions: addressOf(positions),
      projectedPositionsBytes: positions.size,
      biasU: addressOf(u),
      biasUBytes: u.size,
      biasV: addressOf(v),
      biasVBytes: v.size,
      validLengths: addressOf(valid),
      validLengthsBytes: valid.size,
      output: addressOf(output),
      outputBytes: output.size,
    };
  }

  validateDescriptor(descriptor) {
    native().attentionValidate(this.nativeDescriptor(descriptor));
  }

  /** createDispatch (attention.ts:219-314). */
  createDispatch(descriptor) {
    if (this.destroyed) throw new Error("Parakeet relative attention kernel was destroyed");
    const op = native().attentionCreate(this.device.context, this.nativeDescriptor(descriptor));
    return new RelativeAttentionDispatch(descriptor.label, descriptor.output, op, descriptor.batchSize);
  }

  destroy() {
    this.destroyed = true;
  }
}

/* ------------------------------------------------------------ kernels */

class GemmDispatch {
  constructor(label, output, op, rows) {
    this.label = label;
    this.output = output;
    this.op = op;
    this.rows = rows;
    this.destroyed = false;
  }

  /**
   * GemmDispatch.encode (gemm.ts:419-463): records the launch; `shape`
   * re-plans for an active row prefix; `timestampWrites` = {querySet,
   * beginningOfPassWriteIndex?, endOfPassWriteIndex?}.
   */
  encode(encoder, timestampWrites, shape) {
    if (this.destroyed) throw new Error(`${this.label} was destroyed`);
    let rows = 0;
    if (shape !== undefined) {
      const activeRows = shape.rows;
      if (!isSafe(activeRows) || activeRows <= 0 || activeRows > this.rows)
        throw new RangeError(`${this.label} active rows must be in [1, ${this.rows}]`);
      rows = activeRows;
    }
    const op = this.op;
    encoder.record(() => {
      // The kernel's own dispatch stamps the pass's timestamp queries.
      const qs = timestampWrites ? timestampWrites.querySet : null;
      const begin = qs && timestampWrites.beginningOfPassWriteIndex !== undefined
        ? qs.events[timestampWrites.beginningOfPassWriteIndex] : null;
      const end = qs && timestampWrites.endOfPassWriteIndex !== undefined
        ? qs.events[timestampWrites.endOfPassWriteIndex] : null;
      native().gemmEnqueue(op, rows, null, begin, end);
    });
  }

  /** Idempotent (gemm.ts:465-469). */
  destroy() {
    if (this.destroyed) return;
    this.destroyed = true;
    native().gemmDestroy(this.op);
  }

  /** The launch a given active row count gets (planF16SubgroupGemm). */
  plan(activeRows) {
    return native().gemmPlan(this.op, activeRows || 0);
  }
}

class PaletteGemmKernel {
  constructor(device, arena, fp32, options) {
    this.device = device;
    this.arena = arena;
    this.fp32 = fp32;
    this.productionOnly = !(options && options.allowSyntheticShapes);
    this.destroyed = false;
    this.portableLoadEncoding = null;
  }

  get transientPaletteParameterBytes() {
    return 0;
  }

  get transientPaletteParameterUsedSlots() {
    return 0;
  }

  /** No palette expansion ever runs: the kernels decode in registers. */
  get transientPaletteDispatchCount() {
    return 0;
  }

  get transientPaletteExpandedBytes() {
    return 0;
  }

  kernelName() {
    return this.fp32 ? "Parakeet FP32 GEMM kernel" : "Parakeet GEMM kernel";
  }

  /** The native descriptor of a reference GemmDescriptor. */
  nativeDescriptor(descriptor, prepared) {
    const fp32 = this.fp32;
    const paletteBits = requireWeightRecords(descriptor, fp32);
    const groups = requirePaletteRecords(descriptor, paletteBits, fp32);
    if (this.productionOnly) {
      const expanded = descriptor.inner * descriptor.columns * (fp32 ? 4 : 2);
      const limit = fp32 ? FP32_TRANSIENT_PALETTE_WEIGHT_SCRATCH_BYTES : TRANSIENT_PALETTE_WEIGHT_SCRATCH_BYTES;
      if (expanded > limit) {
        throw new Error(`${descriptor.label} exceeds transient${fp32 ? " FP32" : ""} palette scratch`);
      }
    }
    const a = this.arena.binding(descriptor.a);
    const out = this.arena.binding(descriptor.output);
    const b = descriptor.b.binding;
    const palette = descriptor.bPalette.binding;
    /** @type {any} */
    const d = {
      label: descriptor.label,
      flags: (this.productionOnly ? REQUIRE_PRODUCTION_SIGNATURE : 0) | (descriptor.glu ? GEMM_GLU : 0) |
        (descriptor.rowNorm ? GEMM_ROW_NORM : 0) | (descriptor.cachedOutput ? GEMM_CACHED_OUTPUT : 0),
      precision: fp32 ? "f32" : "f16",
      paletteBits,
      rows: descriptor.rows,
      inner: descriptor.inner,
      columns: descriptor.columns,
      paletteGroups: groups,
      paletteGroupColumns: descriptor.paletteGroupColumns,
      a: a.buffer.address + BigInt(a.offset),
      aBytes: a.size,
      palette: palette.buffer.address + BigInt(palette.offset),
      paletteBytes: palette.size,
      output: out.buffer.address + BigInt(out.offset),
      outputBytes: out.size,
      activation: descriptor.activation || "none",
    };
    if (prepared === undefined) {
      d.packed = b.buffer.address + BigInt(b.offset);
      d.packedBytes = b.size;
    } else {
      d.prepared = prepared.native;
    }
    if (descriptor.bias !== undefined) {
      d.bias = descriptor.bias.binding.buffer.address + BigInt(descriptor.bias.binding.offset);
      d.biasBytes = descriptor.bias.binding.size;
    }
    if (descriptor.residual !== undefined) {
      const r = this.arena.binding(descriptor.residual);
      d.residual = r.buffer.address + BigInt(r.offset);
      d.residualBytes = r.size;
    }
    if (descriptor.residualScale !== undefined) d.residualScale = descriptor.residualScale;
    if (descriptor.rowNorm) {
      // {gamma, beta, epsilon?}: the op multiplies LayerNorm(a) (no reference counterpart)
      const { gamma, beta, epsilon } = descriptor.rowNorm;
      d.normGamma = gamma.binding.buffer.address + BigInt(gamma.binding.offset);
      d.normGammaBytes = gamma.binding.size;
      d.normBeta = beta.binding.buffer.address + BigInt(beta.binding.offset);
      d.normBetaBytes = beta.binding.size;
      if (epsilon !== undefined) d.normEpsilon = epsilon;
    }
    return d;
  }

  /** The descriptor contract alone (no device work). */
  validateDescriptor(descriptor) {
    native().gemmValidate(this.nativeDescriptor(descriptor, undefined));
  }

  createDispatch(descriptor) {
    if (this.destroyed) throw new Error(`${this.kernelName()} was destroyed`);
    const prepared = descriptor.preparedPaletteWeight;
    if (prepared !== undefined) {
      if (
        prepared.source !== descriptor.b ||
        prepared.palette !== descriptor.bPalette ||
        prepared.paletteGroupColumns !== descriptor.paletteGroupColumns ||
        prepared.inner !== descriptor.inner ||
        prepared.columns !== descriptor.columns
      ) {
        throw new Error(`${descriptor.label} has a mismatched prepared palette weight`);
      }
    }
    const d = this.nativeDescriptor(descriptor, prepared);
    const op = native().gemmCreate(this.device.context, d);
    return new GemmDispatch(descriptor.label, descriptor.output, op, descriptor.rows);
  }

  /**
   * createPreparedPaletteWeight (gemm.ts:706-748): the weight is re-ordered
   * once into the kernels' operand order; several dispatches may share it.
   * `scratchOffset` is checked as the reference checks its scratch slice.
   */
  createPreparedPaletteWeight(descriptor, scratchOffset) {
    if (this.destroyed) throw new Error(`${this.kernelName()} was destroyed`);
    if (descriptor.preparedPaletteWeight !== undefined)
      throw new Error(`${descriptor.label} cannot prepare an already prepared weight`);
    const d = this.nativeDescriptor(descriptor, undefined);
    native().gemmValidate(d);
    const size = descriptor.inner * descriptor.columns * (this.fp32 ? 4 : 2);
    const limit = this.fp32 ? FP32_TRANSIENT_PALETTE_WEIGHT_SCRATCH_BYTES : TRANSIENT_PALETTE_WEIGHT_SCRATCH_BYTES;
    if (
      !isSafe(scratchOffset) ||
      scratchOffset < 0 ||
      scratchOffset % STORAGE_ALIGNMENT !== 0 ||
      (this.productionOnly && scratchOffset + size > limit)
    ) {
      throw new RangeError(
        `${descriptor.label} has an invalid${this.fp32 ? " FP32" : ""} transient palette scratch slice`,
      );
    }
    const weight = native().preparedWeightCreate(this.device.context, {
      label: descriptor.label,
      paletteBits: d.paletteBits,
      inner: descriptor.inner,
      columns: descriptor.columns,
      packed: d.packed,
      packedBytes: d.packedBytes,
    });
    return {
      source: descriptor.b,
      palette: descriptor.bPalette,
      paletteGroupColumns: descriptor.paletteGroupColumns,
      inner: descriptor.inner,
      columns: descriptor.columns,
      runtimeLayout: "operand-order",
      binding: descriptor.b.binding,
      preparation: { destroy: () => native().preparedWeightDestroy(weight) },
      native: weight,
    };
  }

  destroy() {
    this.destroyed = true;
  }
}

class F16GemmKernel extends PaletteGemmKernel {
  /**
   * create(device, arena, executionProfile?, options?) - the reference's
   * fixed production signatures are enforced unless
   * options.allowSyntheticShapes is set.
   */
  static create(device, arena, executionProfile, options) {
    if (executionProfile !== undefined && executionProfile.precision !== "fp16")
      return Promise.reject(new Error("Parakeet FP16 GEMM requires an FP16 execution profile"));
    return Promise.resolve(new F16GemmKernel(device, arena, false, options));
  }
}

class F32GemmKernel extends PaletteGemmKernel {
  static create(device, arena, executionProfile, options) {
    if (executionProfile !== undefined && executionProfile.precision !== "fp32")
      return Promise.reject(new Error("Parakeet FP32 GEMM requires an FP32 execution profile"));
    return Promise.resolve(new F32GemmKernel(device, arena, true, options));
  }
}

/** The EncoderGemmBackend adapter of encoder.ts:356-432. */
function createEncoderGemmBackend(kernel) {
  return {
    get portableF16LoadEncoding() {
      return kernel.portableLoadEncoding;
    },
    get transientPaletteParameterBytes() {
      return kernel.transientPaletteParameterBytes;
    },
    get transientPaletteParameterUsedSlots() {
      return kernel.transientPaletteParameterUsedSlots;
    },
    get transientPaletteDispatchCount() {
      return kernel.transientPaletteDispatchCount;
    },
    get transientPaletteExpandedBytes() {
      return kernel.transientPaletteExpandedBytes;
    },
    createDispatch(descriptor) {
      return kernel.createDispatch(descriptor);
    },
    createPreparedPaletteWeight(descriptor, scratchOffset) {
      return kernel.createPreparedPaletteWeight(descriptor, scratchOffset);
    },
  };
}

/* ------------------------------------------------------------ LayerNorm */

/** layernorm.ts requirePackedTensor: a float32 "channel" record of [C]. */
function requireChannelTensor(tensor, channels, byteLength, label) {
  const record = tensor.runtimeRecord;
  if (
    record.dtype !== "float32" ||
    record.layout !== "channel" ||
    record.byteLength !== byteLength ||
    shapeKey(record.logicalShape) !== String(channels) ||
    shapeKey(record.storageShape) !== String(channels)
  ) {
    throw new Error(`${label} must be float32 channel logical/storage [${channels}], ${byteLength} bytes`);
  }
}

class LayerNormDispatch {
  constructor(label, output, op, rows) {
    this.label = label;
    this.output = output;
    this.op = op;
    this.rows = rows;
    this.destroyed = false;
  }

  /** encode (layernorm.ts:45-66): shape.rows selects the active rows. */
  encode(encoder, timestampWrites, shape) {
    if (this.destroyed) throw new Error(`${this.label} was destroyed`);
    const rows = shape === undefined || shape.rows === undefined ? this.rows : shape.rows;
    if (!isSafe(rows) || rows <= 0 || rows > this.rows)
      throw new RangeError(`${this.label} active rows must be in [1, ${this.rows}]`);
    const op = this.op;
    encoder.record(() => {
      const [begin, end] = timestampEvents(timestampWrites);
      native().layernormEnqueue(op, rows, null, begin, end);
    });
  }

  destroy() {
    if (this.destroyed) return;
    this.destroyed = true;
    native().layernormDestroy(this.op);
  }
}

class LayerNormKernel {
  constructor(device, arena, executionProfile) {
    this.device = device;
    this.arena = arena;
    this.precision = precisionOf(executionProfile);
    this.destroyed = false;
  }

  /** create (layernorm.ts:120-162): the kernel is compiled into the library. */
  static create(device, arena, uniformParameterCapacity, executionProfile) {
    return Promise.resolve(new LayerNormKernel(device, arena, executionProfile));
  }

  get uniformParameterPoolBytes() {
    return 0;
  }

  nativeDescriptor(descriptor) {
    if (!isSafe(descriptor.rows) || !isSafe(descriptor.channels) || descriptor.rows <= 0 ||
        descriptor.channels <= 0 || descriptor.channels % 4 !== 0)
      throw new RangeError(`Invalid LayerNorm shape for ${descriptor.label}`);
    const input = this.arena.binding(descriptor.input);
    const output = this.arena.binding(descriptor.output);
    const affineBytes = descriptor.channels * 4;
    requireChannelTensor(descriptor.gamma, descriptor.channels, affineBytes, `${descriptor.label} gamma`);
    requireChannelTensor(descriptor.beta, descriptor.channels, affineBytes, `${descriptor.label} beta`);
    const d = {
      label: descriptor.label,
      precision: this.precision,
      rows: descriptor.rows,
      channels: descriptor.channels,
      input: addressOf(input),
      inputBytes: input.size,
      gamma: addressOf(descriptor.gamma.binding),
      gammaBytes: descriptor.gamma.binding.size,
      beta: addressOf(descriptor.beta.binding),
      betaBytes: descriptor.beta.binding.size,
      output: addressOf(output),
      outputBytes: output.size,
      epsilon: descriptor.epsilon === undefined ? 1e-5 : descriptor.epsilon,
    };
    if (descriptor.next) {
      // {gamma, beta, output}: the same dispatch also writes LayerNorm(output)
      // with these parameters (a chained LayerNorm, no reference counterpart)
      const { gamma, beta } = descriptor.next;
      requireChannelTensor(gamma, descriptor.channels, affineBytes, `${descriptor.label} next gamma`);
      requireChannelTensor(beta, descriptor.channels, affineBytes, `${descriptor.label} next beta`);
      const next = this.arena.binding(descriptor.next.output);
      Object.assign(d, {
        nextGamma: addressOf(gamma.binding), nextGammaBytes: gamma.binding.size,
        nextBeta: addressOf(beta.binding), nextBetaBytes: beta.binding.size,
        nextOutput: addressOf(next), nextOutputBytes: next.size,
      });
    }
    return d;
  }

  validateDescriptor(descriptor) {
    native().layernormValidate(this.nativeDescriptor(descriptor));
  }

  /** createDispatch (layernorm.ts:165-240). */
  createDispatch(descriptor) {
    if (this.destroyed) throw new Error("Parakeet LayerNorm kernel was destroyed");
    const op = native().layernormCreate(this.device.context, this.nativeDescriptor(descriptor));
    return new LayerNormDispatch(descriptor.label, descriptor.output, op, descriptor.rows);
  }

  destroy() {
    this.destroyed = true;
  }
}

/** Package records of a LayerNorm gamma or beta (a float32 [C] "channel" tensor). */
function channelTensorRecords(channels) {
  const record = {
    dtype: "float32", logicalShape: [channels], storageShape: [channels], byteLength: channels * 4,
    layout: "channel",
  };
  return { sourceRecord: record, runtimeRecord: record };
}

/** The begin / end events of a timestampWrites descriptor (or nulls). */
function timestampEvents(timestampWrites) {
  const qs = timestampWrites ? timestampWrites.querySet : null;
  const begin = qs && timestampWrites.beginningOfPassWriteIndex !== undefined
    ? qs.events[timestampWrites.beginningOfPassWriteIndex] : null;
  const end = qs && timestampWrites.endOfPassWriteIndex !== undefined
    ? qs.events[timestampWrites.endOfPassWriteIndex] : null;
  return [begin, end];
}

/* ------------------------------------------------------------ subsampling */

const SUBSAMPLING_CONV0_WEIGHT_LAYOUT = "kh-kw-output-channel-vec4";
const SUBSAMPLING_DEPTHWISE_WEIGHT_LAYOUT = "kh-kw-channel-vec4";
const SUBSAMPLING_BIAS_LAYOUT = "output-channel";

/** subsamplingOutputDimension (subsampling.ts:119-122). */
function subsamplingOutputDimension(input) {
  if (!isSafe(input) || input <= 0) throw new RangeError("subsampling input dimension must be a positive integer");
  return native().subsamplingOutputDimension(input);
}

/** subsamplingValidLength (subsampling.ts:124-135). */
function subsamplingValidLength(featureLength, steps) {
  if (!isSafe(featureLength) || featureLength <= 0) throw new RangeError("featureLength must be a positive integer");
  if (!isSafe(steps) || steps <= 0) throw new RangeError("subsampling steps must be a positive integer");
  return native().subsamplingValidLength(featureLength, steps);
}

/** subsampling.ts requirePackedTensor (:1009-1034), [3,3,C] kernels and [C] biases. */
function requireSubsamplingTensor(tensor, dtype, shape, layout, byteLength, label) {
  const record = tensor.runtimeRecord;
  const storageShape = shape.length === 3 ? [shape[0], shape[1], shape[2] / 4, 4] : shape;
  if (
    record.dtype !== dtype ||
    record.layout !== layout ||
    record.byteLength !== byteLength ||
    shapeKey(record.logicalShape) !== shapeKey(shape) ||
    shapeKey(record.storageShape) !== shapeKey(storageShape)
  ) {
    throw new Error(
      `${label} must be ${dtype} ${layout} logical [${shape.join(",")}], ` +
        `storage [${storageShape.join(",")}], ${byteLength} bytes`,
    );
  }
}

/** Package records of the subsampling kernels and biases (convert.py:1264-1340). */
function subsamplingTensorRecords(options) {
  const dtype = (options && options.dtype) || "float16";
  const channels = (options && options.channels) || 256;
  const scalar = dtype === "float16" ? 2 : 4;
  const kernel = (layout) => {
    const r = { dtype, logicalShape: [3, 3, channels], storageShape: [3, 3, channels / 4, 4],
                byteLength: 9 * channels * scalar, layout };
    return { sourceRecord: r, runtimeRecord: r };
  };
  const bias = { dtype: "float32", logicalShape: [channels], storageShape: [channels], byteLength: channels * 4,
                 layout: SUBSAMPLING_BIAS_LAYOUT };
  return {
    conv0Weights: kernel(SUBSAMPLING_CONV0_WEIGHT_LAYOUT),
    depthwiseWeights: kernel(SUBSAMPLING_DEPTHWISE_WEIGHT_LAYOUT),
    bias: { sourceRecord: bias, runtimeRecord: bias },
  };
}

/** SubsamplingDispatch / SubsamplingTimeMaskDispatch (subsampling.ts:208-248, :587-618). */
class SubsamplingDispatch {
  constructor(label, output, op, batchSize, plan) {
    this.label = label;
    this.output = output;
    this.op = op;
    this.batchSize = batchSize;
    this.outputHeight = plan.outputHeight;
    this.outputWidth = plan.outputWidth;
    this.destroyed = false;
  }

  /** encode(encoder, timestampWrites?, shape?): shape.batchSize (this
      library's addition) selects an active prefix of the windows. */
  encode(encoder, timestampWrites, shape) {
    if (this.destroyed) throw new Error(`${this.label} was destroyed`);
    const active = shape === undefined || shape.batchSize === undefined ? this.batchSize : shape.batchSize;
    if (!isSafe(active) || active <= 0 || active > this.batchSize)
      throw new RangeError(`${this.label} active batch must be in [1, ${this.batchSize}]`);
    const op = this.op;
    encoder.record(() => {
      const [begin, end] = timestampEvents(timestampWrites);
      native().subsamplingEnqueue(op, active, null, begin, end);
    });
  }

  destroy() {
    if (this.destroyed) return;
    this.destroyed = true;
    native().subsamplingDestroy(this.op);
  }

  plan(activeBatch) {
    return native().subsamplingPlan(this.op, activeBatch || 0);
  }
}

class SubsamplingKernelBase {
  constructor(device, arena, executionProfile) {
    this.device = device;
    this.arena = arena;
    this.precision = precisionOf(executionProfile);
    this.dtype = this.precision === "f16" ? "float16" : "float32";
    this.destroyed = false;
  }

  get uniformParameterPoolBytes() {
    return 0;
  }

  slice(binding) {
    const b = this.arena.binding(binding);
    return [addressOf(b), b.size];
  }

  create(kind, native_desc, descriptor, batchSize) {
    if (this.destroyed) throw new Error(`${this.constructor.name} was destroyed`);
    const op = native().subsamplingCreate(this.device.context, kind, native_desc);
    const plan = native().subsamplingPlan(op, 0);
    return new SubsamplingDispatch(descriptor.label, descriptor.output || descriptor.values, op, batchSize, plan);
  }

  destroy() {
    this.destroyed = true;
  }
}

/** FusedSubsamplingConv0Depthwise2Kernel (subsampling.ts:250-436). */
class FusedSubsamplingConv0Depthwise2Kernel extends SubsamplingKernelBase {
  static create(device, arena, uniformParameterCapacity, executionProfile) {
    return Promise.resolve(new FusedSubsamplingConv0Depthwise2Kernel(device, arena, executionProfile));
  }

  nativeDescriptor(descriptor) {
    const scalar = this.precision === "f16" ? 2 : 4;
    const channels = descriptor.channels;
    requireSubsamplingTensor(descriptor.conv0Weights, this.dtype, [3, 3, channels], SUBSAMPLING_CONV0_WEIGHT_LAYOUT,
                             9 * channels * scalar, `${descriptor.label} conv0 weights`);
    requireSubsamplingTensor(descriptor.conv0Bias, "float32", [channels], SUBSAMPLING_BIAS_LAYOUT, channels * 4,
                             `${descriptor.label} conv0 bias`);
    requireSubsamplingTensor(descriptor.depthwiseWeights, this.dtype, [3, 3, channels],
                             SUBSAMPLING_DEPTHWISE_WEIGHT_LAYOUT, 9 * channels * scalar,
                             `${descriptor.label} depthwise2 weights`);
    requireSubsamplingTensor(descriptor.depthwiseBias, "float32", [channels], SUBSAMPLING_BIAS_LAYOUT, channels * 4,
                             `${descriptor.label} depthwise2 bias`);
    const [input, inputBytes] = this.slice(descriptor.input);
    const [output, outputBytes] = this.slice(descriptor.output);
    const [valid, validBytes] = this.slice(descriptor.validLengths);
    const t = (x) => [addressOf(x.binding), x.binding.size];
    const [w0, w0b] = t(descriptor.conv0Weights), [b0, b0b] = t(descriptor.conv0Bias);
    const [wd, wdb] = t(descriptor.depthwiseWeights), [bd, bdb] = t(descriptor.depthwiseBias);
    return {
      label: descriptor.label, precision: this.precision, batchSize: descriptor.batchSize,
      inputHeight: descriptor.inputHeight, inputWidth: descriptor.inputWidth, channels,
      input, inputBytes, conv0Weights: w0, conv0WeightsBytes: w0b, conv0Bias: b0, conv0BiasBytes: b0b,
      depthwiseWeights: wd, depthwiseWeightsBytes: wdb, depthwiseBias: bd, depthwiseBiasBytes: bdb,
      output, outputBytes, validLengths: valid, validLengthsBytes: validBytes,
      validLengthBatchOffset: descriptor.validLengthBatchOffset || 0,
    };
  }

  validateDescriptor(descriptor) {
    native().subsamplingValidate("fused", this.nativeDescriptor(descriptor));
  }

  /** createDispatch (subsampling.ts:334-425). */
  createDispatch(descriptor) {
    return this.create("fused", this.nativeDescriptor(descriptor), descriptor, descriptor.batchSize);
  }
}

/** DepthwiseSubsamplingKernel (subsampling.ts:438-571). */
class DepthwiseSubsamplingKernel extends SubsamplingKernelBase {
  static create(device, arena, uniformParameterCapacity, executionProfile) {
    return Promise.resolve(new DepthwiseSubsamplingKernel(device, arena, executionProfile));
  }

  nativeDescriptor(descriptor) {
    const scalar = this.precision === "f16" ? 2 : 4;
    const channels = descriptor.channels;
    if (isSafe(channels) && channels > 0 && channels % 4 === 0) {
      requireSubsamplingTensor(descriptor.weights, this.dtype, [3, 3, channels], SUBSAMPLING_DEPTHWISE_WEIGHT_LAYOUT,
                               9 * channels * scalar, `${descriptor.label} weights`);
      requireSubsamplingTensor(descriptor.bias, "float32", [channels], SUBSAMPLING_BIAS_LAYOUT, channels * 4,
                               `${descriptor.label} bias`);
    }
    const [input, inputBytes] = this.slice(descriptor.input);
    const [output, outputBytes] = this.slice(descriptor.output);
    const [valid, validBytes] = this.slice(descriptor.validLengths);
    return {
      label: descriptor.label, precision: this.precision, batchSize: descriptor.batchSize,
      inputHeight: descriptor.inputHeight, inputWidth: descriptor.inputWidth, channels,
      input, inputBytes, weights: addressOf(descriptor.weights.binding), weightsBytes: descriptor.weights.binding.size,
      bias: addressOf(descriptor.bias.binding), biasBytes: descriptor.bias.binding.size, output, outputBytes,
      validLengths: valid, validLengthsBytes: validBytes,
      validLengthBatchOffset: descriptor.validLengthBatchOffset || 0,
      validLengthSubsamplingSteps: descriptor.validLengthSubsamplingSteps,
    };
  }

  validateDescriptor(descriptor) {
    native().subsamplingValidate("depthwise", this.nativeDescriptor(descriptor));
  }

  /** createDispatch (subsampling.ts:495-560). */
  createDispatch(descriptor) {
    return this.create("depthwise", this.nativeDescriptor(descriptor), descriptor, descriptor.batchSize);
  }
}

/** SubsamplingTimeMaskKernel (subsampling.ts:620-793). */
class SubsamplingTimeMaskKernel extends SubsamplingKernelBase {
  static create(device, arena, uniformParameterCapacity, executionProfile) {
    return Promise.resolve(new SubsamplingTimeMaskKernel(device, arena, executionProfile));
  }

  nativeDescriptor(descriptor) {
    const [values, valuesBytes] = this.slice(descriptor.values);
    const [valid, validBytes] = this.slice(descriptor.validLengths);
    return {
      label: descriptor.label, precision: this.precision, batchSize: descriptor.batchSize,
      height: descriptor.height, width: descriptor.width, channels: descriptor.channels,
      values, valuesBytes, validLengths: valid, validLengthsBytes: validBytes,
      validLengthBatchOffset: descriptor.validLengthBatchOffset || 0,
      validLengthSubsamplingSteps: descriptor.validLengthSubsamplingSteps,
    };
  }

  validateDescriptor(descriptor) {
    native().subsamplingValidate("mask", this.nativeDescriptor(descriptor));
  }

  /** createDispatch (subsampling.ts:698-790). */
  createDispatch(descriptor) {
    return this.create("mask", this.nativeDescriptor(descriptor), descriptor, descriptor.batchSize);
  }
}

/* ---------------------------------------------------------- encoder graph */

const PARAKEET_FEATURE_BINS = 128;
const PARAKEET_FEATURE_FRAMES = 1501;
const PARAKEET_ENCODER_FRAMES = 188;
const PARAKEET_ENCODER_CHANNELS = 1024;
const PARAKEET_INTERMEDIATE_CHANNELS = 4096;
const PARAKEET_SUBSAMPLING_CHANNELS = 256;
const PARAKEET_PROJECTED_CHANNELS = 640;
const PARAKEET_ENCODER_LAYERS = 24;
const ENCODER_LAYER_DISPATCHES = 15;

/** deriveSubsamplingLengths / deriveEncoderValidLength (encoder.ts:441-458). */
function deriveEncoderValidLength(featureLength) {
  if (!isSafe(featureLength) || featureLength <= 0) throw new RangeError("featureLength must be a positive integer");
  if (featureLength > PARAKEET_FEATURE_FRAMES)
    throw new RangeError(`featureLength must not exceed ${PARAKEET_FEATURE_FRAMES}`);
  return native().subsamplingValidLength(featureLength, 3);
}

/** deriveEncoderValidLengths (encoder.ts:460-479). */
function deriveEncoderValidLengths(featureLengths, batchSize) {
  const n = batchSize === undefined ? featureLengths.length : batchSize;
  if (!isSafe(n) || n <= 0) throw new RangeError("batchSize must be a positive integer");
  if (featureLengths.length !== n) throw new RangeError(`Expected ${n} feature lengths, got ${featureLengths.length}`);
  const out = new Uint32Array(n);
  for (let i = 0; i < n; ++i) {
    if (featureLengths[i] === undefined) throw new RangeError(`Missing feature length ${i}`);
    out[i] = deriveEncoderValidLength(featureLengths[i]);
  }
  return out;
}

/** requireTensorRecord (encoder.ts:2550-2581) on both records of a tensor. */
function requireEncoderTensor(model, name, spec) {
  const tensor = model.tensor(name);
  const scalar = spec.dtype === "float16" ? 2 : 4;
  const expected = spec.storageShape.reduce((a, b) => a * b, 1) * scalar;
  for (const kind of ["source", "runtime"]) {
    const record = kind === "source" ? tensor.sourceRecord : tensor.runtimeRecord;
    if (
      record.dtype !== spec.dtype ||
      record.layout !== spec.layout ||
      record.byteLength !== expected ||
      shapeKey(record.logicalShape) !== shapeKey(spec.logicalShape) ||
      shapeKey(record.storageShape) !== shapeKey(spec.storageShape)
    ) {
      throw new Error(
        `${name} ${kind} must be ${spec.dtype} ${spec.layout}, logical ` +
          `[${spec.logicalShape.join(",")}], storage [${spec.storageShape.join(",")}]`,
      );
    }
  }
  return addressOf(tensor.binding);
}

/** executionDtype (encoder.ts:2625-2631): the profile's activation and palette dtype. */
function executionDtype(precision) {
  return precision === "f32" ? "float32" : "float16";
}

/** matrixTensor (encoder.ts:2458-2512): packed codes and palette addresses. */
function encoderMatrix(model, name, inner, columns, bits, groups, precision) {
  const codesPerGroup = bits === 5 ? 32 : 16;
  const wordsPerGroup = bits === 5 ? 5 : 3;
  const packedGroups = (inner * columns) / codesPerGroup;
  if (!isSafe(packedGroups)) throw new Error(`${name} is not palette packing aligned`);
  const packed = requireEncoderTensor(model, name, {
    dtype: "uint32", logicalShape: [inner, columns], storageShape: [packedGroups, wordsPerGroup],
    layout: `k-by-output-row-major-palette${bits}-lsb-u32`,
  });
  const palette = requireEncoderTensor(model, `${name}.palette`, {
    dtype: executionDtype(precision), logicalShape: [groups, 1 << bits], storageShape: [groups, 1 << bits],
    layout: "output-group-by-palette-lut",
  });
  return { packed, palette };
}

function channelAddress(model, name, channels, layout) {
  return requireEncoderTensor(model, name, {
    dtype: "float32", logicalShape: [channels], storageShape: [channels], layout,
  });
}

function kernelAddress(model, name, layout, precision) {
  return requireEncoderTensor(model, name, {
    dtype: executionDtype(precision), logicalShape: [3, 3, PARAKEET_SUBSAMPLING_CHANNELS],
    storageShape: [3, 3, PARAKEET_SUBSAMPLING_CHANNELS / 4, 4], layout,
  });
}

/** The native descriptor of one layer from the model's tensors (encoder.ts:1868-2135). */
function encoderLayerDescriptor(model, index, frames, precision) {
  const prefix = `encoder.layers.${index}`;
  const norms = ["norm_feed_forward1", "norm_self_att", "norm_conv", "norm_feed_forward2", "norm_out"];
  const m = (name, inner, columns, bits, groups) =>
    encoderMatrix(model, `${prefix}.${name}`, inner, columns, bits || 5, groups || 1, precision);
  const dtype = executionDtype(precision);
  const C = PARAKEET_ENCODER_CHANNELS, H = PARAKEET_INTERMEDIATE_CHANNELS;
  const bias = (name) => requireEncoderTensor(model, `${prefix}.self_attn.${name}`, {
    dtype: "float32", logicalShape: [8, 128], storageShape: [8, 128], layout: "head-by-channel",
  });
  return {
    normGamma: norms.map((n) => channelAddress(model, `${prefix}.${n}.weight`, C, "channel")),
    normBeta: norms.map((n) => channelAddress(model, `${prefix}.${n}.bias`, C, "channel")),
    ff1Linear1: m("feed_forward1.linear1.weight", C, H),
    ff1Linear2: m("feed_forward1.linear2.weight", H, C),
    qkv: m("self_attn.qkv.weight", C, 3 * C, 5, 3),
    projectedPositions: requireEncoderTensor(model, `${prefix}.self_attn.projected_positions`, {
      dtype, logicalShape: [2 * frames - 1, C], storageShape: [8, 32, 2 * frames - 1, 4],
      layout: "head-vector-position-vec4",
    }),
    biasU: bias("bias_u"),
    biasV: bias("bias_v"),
    oProj: m("self_attn.o_proj.weight", C, C, 6),
    pointwise1: m("conv.pointwise_conv1.weight", C, 2 * C),
    depthwise: requireEncoderTensor(model, `${prefix}.conv.depthwise_conv.weight`, {
      dtype, logicalShape: [9, C], storageShape: [9, C / 4, 4], layout: "kernel-channel-vec4",
    }),
    bnScale: channelAddress(model, `${prefix}.conv.norm.scale`, C, "channel"),
    bnShift: channelAddress(model, `${prefix}.conv.norm.shift`, C, "channel"),
    pointwise2: m("conv.pointwise_conv2.weight", C, C),
    ff2Linear1: m("feed_forward2.linear1.weight", C, H),
    ff2Linear2: m("feed_forward2.linear2.weight", H, C),
  };
}

/** The front end's native descriptor (encoder.ts:2140-2300). */
function encoderSubsamplingDescriptor(model, precision) {
  const p = "encoder.subsampling";
  const S = PARAKEET_SUBSAMPLING_CHANNELS;
  return {
    conv0Weights: kernelAddress(model, `${p}.layers.0.weight`, SUBSAMPLING_CONV0_WEIGHT_LAYOUT, precision),
    conv0Bias: channelAddress(model, `${p}.layers.0.bias`, S, SUBSAMPLING_BIAS_LAYOUT),
    depthwise2Weights: kernelAddress(model, `${p}.layers.2.weight`, SUBSAMPLING_DEPTHWISE_WEIGHT_LAYOUT, precision),
    depthwise2Bias: channelAddress(model, `${p}.layers.2.bias`, S, SUBSAMPLING_BIAS_LAYOUT),
    pointwise3: encoderMatrix(model, `${p}.layers.3.weight`, S, S, 5, 1, precision),
    pointwise3Bias: channelAddress(model, `${p}.layers.3.bias`, S, SUBSAMPLING_BIAS_LAYOUT),
    depthwise5Weights: kernelAddress(model, `${p}.layers.5.weight`, SUBSAMPLING_DEPTHWISE_WEIGHT_LAYOUT, precision),
    depthwise5Bias: channelAddress(model, `${p}.layers.5.bias`, S, SUBSAMPLING_BIAS_LAYOUT),
    pointwise6: encoderMatrix(model, `${p}.layers.6.weight`, S, S, 5, 1, precision),
    pointwise6Bias: channelAddress(model, `${p}.layers.6.bias`, S, SUBSAMPLING_BIAS_LAYOUT),
    linear: encoderMatrix(model, `${p}.linear.weight`, 16 * S, PARAKEET_ENCODER_CHANNELS, 5, 1, precision),
    linearBias: channelAddress(model, `${p}.linear.bias`, PARAKEET_ENCODER_CHANNELS, SUBSAMPLING_BIAS_LAYOUT),
  };
}

/**
 * ParakeetEncoderGraph (encoder.ts:1200-1862) over this library's encoder
 * runtime: `model.tensor(name)` returns the package's GpuTensors
 * (package.ts:45-50) under the reference's names; the graph owns the
 * feature input, the lengths, the encoder output and the projector output.
 */
class ParakeetEncoderGraph {
  constructor(device, handle, buffers, options) {
    this.device = device;
    this.handle = handle;
    this.buffers = buffers;
    this.batchSize = options.batchSize;
    this.frames = options.frames;
    this.featureFrames = options.featureFrames;
    this.layers = options.layers;
    this.precision = options.precision;
    this.info = native().encoderInfo(handle);
    this.destroyed = false;
  }

  /**
   * create(device, model, options?): options.batchSize (windows, default
   * 16), options.layers (default 24), options.fusedGlu (PW1's GLU
   * epilogue; default true, false keeps the GLU in the convolution),
   * options.fusedNorms (the four LayerNorms that feed a GEMM
   * run inside it), options.unchainedNorms (one launch per LayerNorm;
   * by default a layer's last LayerNorm also writes the next layer's
   * first) and options.prefixSamePlan (active windows below the capacity
   * keep the capacity's kernels, bit-identical to the full pass's windows;
   * by default they run the plans of a graph built for that many windows),
   * none with a reference counterpart, options.featureFrames (default
   * 1501), and options.executionProfile (encoder.ts:1299-1305: {precision:
   * "fp16"} by default, or {precision: "fp32"} for an fp32 package: f32
   * activations, palettes, positions and convolution weights, and f32
   * encoder and projector outputs).
   */
  static create(device, model, options) {
    try {
      return Promise.resolve(ParakeetEncoderGraph.build(device, model, options || {}));
    } catch (error) {
      return Promise.reject(error);
    }
  }

  static build(device, model, o) {
    const precision = precisionOf(o.executionProfile);
    const profile = precision === "f32" ? "fp32" : "fp16";
    // requireEncoderConfig (encoder.ts:2584-2593)
    if (model.precision !== undefined && model.precision !== profile)
      throw new Error(`Parakeet ${profile} encoder cannot use ${model.precision} model weights`);
    const elem = precision === "f32" ? 4 : 2;
    const batchSize = o.batchSize === undefined ? 16 : o.batchSize;
    const layers = o.layers === undefined ? PARAKEET_ENCODER_LAYERS : o.layers;
    const featureFrames = o.featureFrames === undefined ? PARAKEET_FEATURE_FRAMES : o.featureFrames;
    if (!isSafe(batchSize) || batchSize <= 0) throw new RangeError("Encoder batch capacity must be a positive integer");
    let frames = featureFrames;
    for (let i = 0; i < 3; ++i) frames = subsamplingOutputDimension(frames);
    const layerDescriptors = [];
    for (let i = 0; i < layers; ++i) layerDescriptors.push(encoderLayerDescriptor(model, i, frames, precision));
    const subsampling = encoderSubsamplingDescriptor(model, precision);
    const projector = encoderMatrix(model, "encoder_projector.weight", PARAKEET_ENCODER_CHANNELS,
                                    PARAKEET_PROJECTED_CHANNELS, 5, 1, precision);
    const projectorBias = channelAddress(model, "encoder_projector.bias", PARAKEET_PROJECTED_CHANNELS,
                                         "output-channel");
    const rows = batchSize * frames;
    const make = (label, size) => device.createBuffer({ label, size });
    const buffers = {
      features: make("fbank-feature-major", batchSize * PARAKEET_FEATURE_BINS * featureFrames * 4),
      featureLengths: make("feature-lengths", batchSize * 4),
      encoderLengths: make("encoder-lengths", batchSize * 4),
      output: make("encoder-output", rows * PARAKEET_ENCODER_CHANNELS * elem),
      projectedOutput: make("encoder-projector-output", rows * PARAKEET_PROJECTED_CHANNELS * elem),
    };
    let handle;
    try {
      handle = native().encoderCreate(device.context, {
        label: o.label || "encoder", precision, fusedGlu: o.fusedGlu !== false, fusedNorms: o.fusedNorms === true,
        unchainedNorms: o.unchainedNorms === true, prefixSamePlan: o.prefixSamePlan === true, batchSize, frames,
        layers: layerDescriptors, validLengths: buffers.encoderLengths.address,
        input: buffers.features.address, output: buffers.output.address, subsampling, featureFrames,
        featureLengths: buffers.featureLengths.address, projector, projectorBias,
        projectedChannels: PARAKEET_PROJECTED_CHANNELS, projectedOutput: buffers.projectedOutput.address,
      });
    } catch (error) {
      for (const b of Object.values(buffers)) b.destroy();
      throw error;
    }
    return new ParakeetEncoderGraph(device, handle, buffers, { batchSize, frames, featureFrames, layers, precision });
  }

  /** Launches in one pass (6 front end + 15 per layer + the projector). */
  get dispatchCount() {
    return this.info.launches;
  }

  /** uploadFeatures (encoder.ts:1536-1553): f32 [windows, 128, F] feature-major. */
  uploadFeatures(features) {
    this.assertAlive();
    const perItem = PARAKEET_FEATURE_BINS * this.featureFrames * 4;
    if (features.byteLength <= 0 || features.byteLength > this.buffers.features.size ||
        features.byteLength % perItem !== 0)
      throw new RangeError(`Expected 1-${this.batchSize} complete feature items, got ${features.byteLength} bytes`);
    this.device.queue.writeBuffer(this.buffers.features, 0, features);
  }

  /** uploadValidFeatureLengths (encoder.ts:1555-1582): raw and derived lengths. */
  uploadValidFeatureLengths(featureLengths) {
    this.assertAlive();
    const n = featureLengths.length;
    if (!isSafe(n) || n <= 0 || n > this.batchSize)
      throw new RangeError(`Encoder active batch must be in [1, ${this.batchSize}]`);
    const raw = new Uint32Array(n);
    for (let i = 0; i < n; ++i) {
      const value = featureLengths[i];
      if (value === undefined || !isSafe(value) || value <= 0 || value > this.featureFrames)
        throw new RangeError(`Feature length ${i} must be in [1, ${this.featureFrames}]`);
      raw[i] = value;
    }
    const derived = deriveEncoderValidLengths(Array.from(raw), n);
    this.device.queue.writeBuffer(this.buffers.featureLengths, 0, raw);
    this.device.queue.writeBuffer(this.buffers.encoderLengths, 0, derived);
    return derived;
  }

  /**
   * encode(encoder, validFeatureLengths, options?) (encoder.ts:1690-1706):
   * uploads the lengths and records one pass over the active windows;
   * options.useGraph replays the pass from a HIP graph, options.timestamps
   * = {querySet, first} stamps every launch (start 2i, end 2i+1 from
   * `first`).
   */
  encode(encoder, validFeatureLengths, options) {
    this.assertAlive();
    const derived = this.uploadValidFeatureLengths(validFeatureLengths);
    const active = derived.length;
    const handle = this.handle;
    const o = options || {};
    if (o.timestamps) {
      const qs = o.timestamps.querySet, first = o.timestamps.first || 0;
      const n = this.info.launches;
      if (qs.events.length < first + 2 * n) throw new RangeError(`the query set needs ${first + 2 * n} entries`);
      const starts = [], ends = [];
      for (let i = 0; i < n; ++i) {
        starts.push(qs.events[first + 2 * i]);
        ends.push(qs.events[first + 2 * i + 1]);
      }
      encoder.record(() => native().encoderEnqueueProfiled(handle, active, null, starts, ends));
    } else {
      const graph = o.useGraph === true;
      encoder.record(() => native().encoderEnqueue(handle, active, null, graph));
    }
    return derived;
  }

  /** Device buffers of the encoder output [windows*188, 1024] and the projector output [.., 640],
   * f16 in the fp16 profile and f32 in the fp32 profile. */
  get outputBuffer() {
    return this.buffers.output;
  }

  get projectedOutputBuffer() {
    return this.buffers.projectedOutput;
  }

  destroy() {
    if (this.destroyed) return;
    this.destroyed = true;
    native().encoderDestroy(this.handle);
    for (const b of Object.values(this.buffers)) b.destroy();
  }

  assertAlive() {
    if (this.destroyed) throw new Error("Parakeet encoder graph was destroyed");
  }
}

/* ------------------------------------------------------------ TDT decoder */

const TDT_HIDDEN_SIZE = 640;
const TDT_GATE_SIZE = 4 * TDT_HIDDEN_SIZE;
const TDT_LSTM_INPUT_SIZE = 2 * TDT_HIDDEN_SIZE;
const TDT_TOKEN_OUTPUTS = 1025;
const TDT_BLANK_TOKEN = 1024;
const TDT_HEAD_STORAGE_OUTPUTS = 1032;
const TDT_DECODER_OVERFLOW = 1;
/** Status bit of a team barrier that gave up waiting (no reference counterpart). */
const TDT_DECODER_SYNC_TIMEOUT = 2;

/**
 * The causes in one window's status word (the metadata's second half):
 * overflow (more tokens than maxTokens, tdt-decoder.ts:1756-1775),
 * syncTimeout (a team barrier gave up: the window's outputs are incomplete
 * and it must be decoded again) and any bits this library does not define.
 */
function decodeTdtStatus(word) {
  if (!isSafe(word) || word < 0 || word > 0xffffffff) throw new RangeError("TDT status must be a u32 word");
  const known = TDT_DECODER_OVERFLOW | TDT_DECODER_SYNC_TIMEOUT;
  return {
    overflow: (word & TDT_DECODER_OVERFLOW) !== 0,
    syncTimeout: (word & TDT_DECODER_SYNC_TIMEOUT) !== 0,
    unknown: ((word >>> 0) & ~known) >>> 0,
  };
}

/**
 * planTdtDecoderExecution (tdt-decoder.ts:39-52). This library runs one
 * workgroup of 640 threads per window (the reference pairs windows in a
 * workgroup), so workgroupCount = batchSize; the scratch size is the
 * reference's.
 */
function planTdtDecoderExecution(batchSize) {
  if (!isSafe(batchSize) || batchSize <= 0) throw new RangeError("TDT decoder batchSize must be a positive integer");
  return native().tdtPlanExecution(batchSize);
}

/** requireTensor (tdt-decoder.ts:458-478). */
function requireDecoderTensor(tensor, dtype, storageShape, layout) {
  const source = tensor.sourceRecord;
  const runtime = tensor.runtimeRecord;
  const shape = shapeKey(storageShape);
  if (source.dtype !== dtype || shapeKey(source.storageShape) !== shape || source.layout !== layout ||
      runtime.dtype !== dtype || shapeKey(runtime.storageShape) !== shape || runtime.layout !== layout ||
      runtime.byteLength !== source.byteLength || runtime.byteOffset % 4 !== 0)
    throw new Error(`Unexpected decoder tensor ${source.layout} [${source.storageShape.join(",")}]`);
  return tensor;
}

/**
 * requireDecoderWeights (tdt-decoder.ts:378-456): the nine decoder tensors,
 * all in the resident decoder.bin shard buffer; returns the native weight
 * descriptor (addresses and byte sizes).
 */
function requireDecoderWeights(model, precision) {
  const t = (name, dtype, shape, layout) => requireDecoderTensor(model.tensor(name), dtype, shape, layout);
  const lstmLayout = "input-hidden-k-by-ifgo-row-major-vec4";
  const weightDtype = executionDtype(precision);
  const tensors = {
    embedding: t("decoder.embedding.weight", weightDtype, [TDT_TOKEN_OUTPUTS, TDT_HIDDEN_SIZE],
                 "token-by-channel-row-major"),
    lstmWeight0: t("decoder.lstm.weight_l0", weightDtype, [TDT_LSTM_INPUT_SIZE, TDT_GATE_SIZE], lstmLayout),
    lstmWeight1: t("decoder.lstm.weight_l1", weightDtype, [TDT_LSTM_INPUT_SIZE, TDT_GATE_SIZE], lstmLayout),
    projectorWeight: t("decoder.decoder_projector.weight", weightDtype, [TDT_HIDDEN_SIZE, TDT_HIDDEN_SIZE],
                       "k-by-output-row-major-vec4"),
    headWeight: t("joint.head.weight", weightDtype, [TDT_HIDDEN_SIZE, TDT_HEAD_STORAGE_OUTPUTS],
                  "k-by-output-row-major-vec4"),
    lstmBias0: t("decoder.lstm.bias_l0", "float32", [TDT_GATE_SIZE], "ifgo-gates"),
    lstmBias1: t("decoder.lstm.bias_l1", "float32", [TDT_GATE_SIZE], "ifgo-gates"),
    projectorBias: t("decoder.decoder_projector.bias", "float32", [TDT_HIDDEN_SIZE], "output-channel"),
    headBias: t("joint.head.bias", "float32", [TDT_HEAD_STORAGE_OUTPUTS], "output-channel-padded-vec4"),
  };
  const buffer = tensors.embedding.buffer;
  const weights = {};
  for (const name of Object.keys(tensors)) {
    const tensor = tensors[name];
    if (tensor.sourceRecord.shard !== "decoder.bin" || tensor.runtimeRecord.bufferId !== "source-shard-decoder.bin" ||
        tensor.buffer !== buffer)
      throw new Error("Persistent TDT decoder requires one resident decoder source shard");
    weights[name] = addressOf(tensor.binding);
    weights[`${name}Bytes`] = tensor.binding.size;
  }
  return weights;
}

class TdtDecoderDispatch {
  constructor(label, op, batchCapacity) {
    this.label = label;
    this.op = op;
    this.batchCapacity = batchCapacity;
    this.destroyed = false;
  }

  /** encode (tdt-decoder.ts:84-130): activeBatchSize selects a prefix of the windows. */
  encode(encoder, timestampWrites, activeBatchSize) {
    if (this.destroyed) throw new Error(`${this.label} was destroyed`);
    const active = activeBatchSize === undefined ? this.batchCapacity : activeBatchSize;
    if (!isSafe(active) || active <= 0 || active > this.batchCapacity)
      throw new RangeError(`${this.label} active batch must be in [1, ${this.batchCapacity}]`);
    const op = this.op;
    encoder.record(() => {
      const [begin, end] = timestampEvents(timestampWrites);
      native().tdtEnqueue(op, active, null, begin, end);
    });
  }

  destroy() {
    if (this.destroyed) return;
    this.destroyed = true;
    native().tdtDestroy(this.op);
  }

  /** Workgroups per window of the next launch (no reference counterpart). */
  get teamSize() {
    return native().tdtTeamSize(this.op);
  }

  /** 0 chooses, 1 one workgroup per window, 8 or 16 a team (no reference counterpart). */
  setTeamSize(members) {
    native().tdtSetTeamSize(this.op, members);
  }
}

/**
 * PersistentTdtDecoderKernel (tdt-decoder.ts:139-366): greedy TDT decoding
 * with the whole autoregressive loop inside one launch, over the package's
 * resident decoder shard; the fp16 profile (f16 weights and encoder rows)
 * or the fp32 profile (f32 weights and encoder rows, one workgroup per
 * window).
 */
class PersistentTdtDecoderKernel {
  constructor(device, arena, weights, precision) {
    this.device = device;
    this.arena = arena;
    this.weights = weights;
    this.precision = precision;
  }

  /** create(device, arena, model, executionProfile?) (:164-292). */
  static create(device, arena, model, executionProfile) {
    try {
      const precision = precisionOf(executionProfile);
      const profile = precision === "f32" ? "fp32" : "fp16";
      if (model.precision !== undefined && model.precision !== profile)
        throw new Error(`TDT decoder ${profile} profile cannot use ${model.precision} decoder weights`);
      return Promise.resolve(new PersistentTdtDecoderKernel(device, arena, requireDecoderWeights(model, precision),
                                                            precision));
    } catch (error) {
      return Promise.reject(error);
    }
  }

  nativeDescriptor(descriptor) {
    for (const name of ["batchSize", "frames", "maxTokens"]) {
      const value = descriptor[name];
      if (!isSafe(value) || value <= 0) throw new RangeError(`Invalid TDT decoder ${name}`);
    }
    const out = {
      label: descriptor.label === undefined ? "parakeet-persistent-tdt-decode" : descriptor.label,
      precision: this.precision,
      batchSize: descriptor.batchSize,
      frames: descriptor.frames,
      maxTokens: descriptor.maxTokens,
      weights: this.weights,
    };
    for (const name of ["encoderProjected", "encodedLengths", "decodeStarts", "decodeEnds", "flushFinals", "state",
                        "predictorScratch", "tokens", "tokenFrames", "tokenDurations", "metadata"]) {
      const binding = this.arena.binding(descriptor[name]);
      out[name] = addressOf(binding);
      out[`${name}Bytes`] = binding.size;
    }
    return out;
  }

  validateDescriptor(descriptor) {
    native().tdtValidate(this.nativeDescriptor(descriptor));
  }

  /** createDispatch (:294-366) with validateDescriptor (:507-547). */
  createDispatch(descriptor) {
    const nativeDescriptor = this.nativeDescriptor(descriptor);
    const op = native().tdtCreate(this.device.context, nativeDescriptor);
    return new TdtDecoderDispatch(nativeDescriptor.label, op, descriptor.batchSize);
  }
}

module.exports = {
  native,
  paletteBitsForLayout,
  HipGpuDevice,
  HipBuffer,
  HipCommandEncoder,
  GpuActivationArena,
  createGpuTensor,
  paletteTensorRecords,
  F16GemmKernel,
  F32GemmKernel,
  GemmDispatch,
  createEncoderGemmBackend,
  TRANSIENT_PALETTE_WEIGHT_SCRATCH_BYTES,
  FP32_TRANSIENT_PALETTE_WEIGHT_SCRATCH_BYTES,
  F16_TILE_INNER,
  F32_TILE_INNER,
  FP32_PACKED_K,
  FusedConformerConvKernel,
  FusedConformerConvDispatch,
  planFusedConformerConv,
  conformerConvTensorRecords,
  CONFORMER_CONV_CHANNELS,
  CONFORMER_CONV_POINTWISE_CHANNELS,
  CONFORMER_CONV_KERNEL_SIZE,
  CONFORMER_DEPTHWISE_WEIGHT_LAYOUT,
  CONFORMER_FOLDED_BATCH_NORM_LAYOUT,
  RelativeAttentionKernel,
  RelativeAttentionDispatch,
  relativeAttentionTensorRecords,
  LayerNormKernel,
  LayerNormDispatch,
  channelTensorRecords,
  subsamplingOutputDimension,
  subsamplingValidLength,
  subsamplingTensorRecords,
  FusedSubsamplingConv0Depthwise2Kernel,
  DepthwiseSubsamplingKernel,
  SubsamplingTimeMaskKernel,
  SubsamplingDispatch,
  deriveEncoderValidLength,
  deriveEncoderValidLengths,
  ParakeetEncoderGraph,
  PARAKEET_FEATURE_BINS,
  PARAKEET_FEATURE_FRAMES,
  PARAKEET_ENCODER_FRAMES,
  PARAKEET_PROJECTED_CHANNELS,
  ENCODER_LAYER_DISPATCHES,
  planTdtDecoderExecution,
  PersistentTdtDecoderKernel,
  TdtDecoderDispatch,
  TDT_DECODER_OVERFLOW,
  TDT_DECODER_SYNC_TIMEOUT,
  decodeTdtStatus,
  TDT_BLANK_TOKEN,
  ...require("./package.js"),
};
