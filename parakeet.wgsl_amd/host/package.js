// @ts-check
/*
 * parakeet.wgsl_amd/host/package - the parakeet-webgpu-v1 package format:
 * manifest validation, the fixed runtime plan and the loader that makes
 * every weight shard resident in HBM, for Node over HIP.
 *
 * Mirrors, with the reference's names, checks and messages:
 *   parseParakeetManifest, parakeetManifestPrecision,
 *   parakeetManifestSha256              src/model/manifest.ts:118-283
 *   planRuntimePackage, paletteBitsForLayout, alignRuntimeOffset and the
 *   package contract constants          src/model/runtime-plan.ts:1-352, :490-863
 *   ParakeetGpuPackage.load / tensor /
 *   releaseInitializationMetadata /
 *   destroy                             src/model/package.ts:52-232
 *   the shard loader (stream, SHA-256,
 *   word-aligned upload, cleanup)        src/model/package.ts:233-500
 *
 * Shards come from the local file system next to the manifest instead of
 * HTTP. Each resident shard becomes one device allocation (hipMalloc through
 * HipGpuDevice.createBuffer) holding the shard's bytes exactly as packed, so
 * a tensor is its shard's buffer plus the record's byteOffset; the palette
 * GEMMs prepare their own operand layouts from these bytes at create time.
 * `options.manifestSha256` (no reference counterpart) admits a package
 * other than the two published manifests, e.g. a synthetic one of the same
 * inventory.
 */
"use strict";

const crypto = require("crypto");
const fs = require("fs");
const path = require("path");

const PARAKEET_FP16_PACKAGE_FORMAT = "parakeet-webgpu-v1";
const PARAKEET_FP32_PACKAGE_FORMAT = "parakeet-webgpu-fp32-v1";
const PARAKEET_FP16_ENCODER_WEIGHT_FORMAT = "mixed-palette5-o-proj-palette6-fp16-lut";
const PARAKEET_FP32_ENCODER_WEIGHT_FORMAT = "mixed-palette5-o-proj-palette6-fp32-lut";
const PARAKEET_FP16_MANIFEST_SHA256 = "11a359db3d050fd82b002c745b24a5280f3ff13a76834b548df671c95c786c65";
const PARAKEET_FP32_MANIFEST_SHA256 = "28dee836aefc2bfb01236fda6d10e1df7447724d2489040168549999ea267b1b";
const PARAKEET_FFN_SOURCE_WIDTH = 4096;
const PARAKEET_SOURCE = Object.freeze({
  repository: "nvidia/parakeet-tdt-0.6b-v2",
  revision: "ae9ad07059c7c739ffaf932226a8fe64ae2620b0",
  archive: Object.freeze({
    name: "parakeet-tdt-0.6b-v2.nemo",
    byteLength: 2472222720,
    sha256: "d99e39955c9d3d0350d8fb7c75e40c64a2b2eaeb003883d7c941fd2e8747b28c",
  }),
  weights: Object.freeze({
    name: "model_weights.ckpt",
    byteLength: 2471920514,
    sha256: "fb1cbe2765fb80c02c0f874b6ea2c2bd24048c3618c092584fd086c6366e48a9",
  }),
  license: "CC-BY-4.0",
});

/* The fixed model configuration every package declares (manifest.ts:218-243). */
const PARAKEET_FIXED_CONFIG = Object.freeze({
  sampleRate: 16000,
  windowSamples: 240000,
  windowSeconds: 15,
  windowOverlapSeconds: 2,
  featureBins: 128,
  fftSize: 512,
  windowSize: 400,
  hopSize: 160,
  preemphasis: 0.97,
  logZeroGuard: 2 ** -24,
  normalizationEpsilon: 1e-5,
  subsamplingFactor: 8,
  encoderLayers: 24,
  encoderHiddenSize: 1024,
  attentionHeads: 8,
  attentionHeadSize: 128,
  convolutionKernelSize: 9,
  decoderHiddenSize: 640,
  decoderLayers: 2,
  vocabularySize: 1025,
  blankTokenId: 1024,
  jointOutputSize: 1030,
  jointStorageOutputSize: 1032,
  maxSymbolsPerStep: 10,
});

const RUNTIME_STORAGE_ALIGNMENT = 256;
const RUNTIME_BUFFER_LIMIT_BYTES = 128 * 1024 * 1024;
const ENCODER_LAYER_COUNT = 24;
const COMMON_TRANSIENT_PALETTE_MATRIX_COUNT = 4;
const RETAINED_RUNTIME_TENSOR_COUNT = 795;
const RESIDENT_SHARD_COUNT = 26;
const FP16_PACKED_DOWNLOAD_BYTES = 405063936;
const FP16_RETAINED_RUNTIME_BYTES = 404930560;
const FP16_LARGEST_RUNTIME_SHARD_BYTES = 16999168;
const FP32_PACKED_DOWNLOAD_BYTES = 440517632;
const FP32_RETAINED_RUNTIME_BYTES = 440384256;
const FP32_LARGEST_RUNTIME_SHARD_BYTES = 33558528;
const PALETTE_LAYOUT = "output-group-by-palette-lut";

/* Byte totals of the two published packages (runtime-plan.ts:124-142). */
const PACKAGE_CONTRACTS = Object.freeze({
  fp16: Object.freeze({
    precision: "fp16",
    paletteDtype: "float16",
    paletteElementBytes: 2,
    packedDownloadBytes: FP16_PACKED_DOWNLOAD_BYTES,
    retainedRuntimeBytes: FP16_RETAINED_RUNTIME_BYTES,
    decoderShardBytes: FP16_LARGEST_RUNTIME_SHARD_BYTES,
    encoderLayerShardBytes: 16050176,
    subsamplingShardBytes: 2727168,
  }),
  fp32: Object.freeze({
    precision: "fp32",
    paletteDtype: "float32",
    paletteElementBytes: 4,
    packedDownloadBytes: FP32_PACKED_DOWNLOAD_BYTES,
    retainedRuntimeBytes: FP32_RETAINED_RUNTIME_BYTES,
    decoderShardBytes: FP32_LARGEST_RUNTIME_SHARD_BYTES,
    encoderLayerShardBytes: 16836864,
    subsamplingShardBytes: 2740992,
  }),
});

const PREPROCESSOR_SHARD = "preprocessor.bin";
const PREPROCESSOR_TENSORS = new Set(["preprocessor.window", "preprocessor.mel_filters"]);
const COMMON_TRANSIENT_PALETTE_TENSORS = new Set([
  "encoder.subsampling.layers.3.weight",
  "encoder.subsampling.layers.6.weight",
  "encoder.subsampling.linear.weight",
  "encoder_projector.weight",
]);

const isObject = (v) => typeof v === "object" && v !== null;
const isPositiveInteger = (v) => Number.isSafeInteger(v) && v > 0;
const isNonnegativeInteger = (v) => Number.isSafeInteger(v) && v >= 0;
const isShape = (v) => Array.isArray(v) && v.every(isPositiveInteger);
const sum = (values) => values.reduce((a, b) => a + b, 0);

/* ------------------------------------------------------------- manifest */

function parakeetManifestPrecision(manifest) {
  return manifest.format === PARAKEET_FP16_PACKAGE_FORMAT ? "fp16" : "fp32";
}

function parakeetManifestSha256(precision) {
  return precision === "fp16" ? PARAKEET_FP16_MANIFEST_SHA256 : PARAKEET_FP32_MANIFEST_SHA256;
}

function sameSource(source) {
  const s = PARAKEET_SOURCE;
  return isObject(source) && source.repository === s.repository && source.revision === s.revision &&
    isObject(source.archive) && source.archive.name === s.archive.name &&
    source.archive.byteLength === s.archive.byteLength && source.archive.sha256 === s.archive.sha256 &&
    isObject(source.weights) && source.weights.name === s.weights.name &&
    source.weights.byteLength === s.weights.byteLength && source.weights.sha256 === s.weights.sha256 &&
    source.license === s.license;
}

/** requireFixedConfig (manifest.ts:213-267). */
function requireFixedConfig(config, encoderWeightFormat) {
  for (const name of Object.keys(PARAKEET_FIXED_CONFIG)) {
    if (config[name] !== PARAKEET_FIXED_CONFIG[name])
      throw new Error(`Unsupported Parakeet config ${name}=${String(config[name])}`);
  }
  if (!Array.isArray(config.durations) || config.durations.join(",") !== "0,1,2,3,4")
    throw new Error("Unsupported TDT duration table");
  if (config.encoderWeightFormat !== encoderWeightFormat || config.intermediateSize !== PARAKEET_FFN_SOURCE_WIDTH)
    throw new Error("Unsupported Parakeet fixed encoder package contract");
}

/** parseParakeetManifest (manifest.ts:135-211): the same checks in the same order. */
function parseParakeetManifest(value) {
  if (!isObject(value) || (value.format !== PARAKEET_FP16_PACKAGE_FORMAT && value.format !== PARAKEET_FP32_PACKAGE_FORMAT))
    throw new Error(`Expected ${PARAKEET_FP16_PACKAGE_FORMAT} or ${PARAKEET_FP32_PACKAGE_FORMAT} model manifest`);
  const fp32 = value.format === PARAKEET_FP32_PACKAGE_FORMAT;
  if (!sameSource(value.source)) throw new Error("Invalid Parakeet source metadata");
  if (!isObject(value.config)) throw new Error("Invalid Parakeet model config");
  requireFixedConfig(value.config, fp32 ? PARAKEET_FP32_ENCODER_WEIGHT_FORMAT : PARAKEET_FP16_ENCODER_WEIGHT_FORMAT);
  if (!Array.isArray(value.files) || !isObject(value.tensors)) throw new Error("Invalid Parakeet package tables");
  for (const file of value.files) {
    if (!isObject(file) || typeof file.name !== "string" || !isPositiveInteger(file.byteLength) ||
        typeof file.sha256 !== "string" || !/^[0-9a-f]{64}$/.test(file.sha256))
      throw new Error("Invalid Parakeet file record");
  }
  const knownFiles = new Set(value.files.map((file) => file.name));
  for (const name of Object.keys(value.tensors)) {
    const t = value.tensors[name];
    if (!isObject(t) || typeof t.shard !== "string" || !knownFiles.has(t.shard) ||
        !isNonnegativeInteger(t.byteOffset) || t.byteOffset % 256 !== 0 || !isPositiveInteger(t.byteLength) ||
        (t.dtype !== "float16" && t.dtype !== "float32" && t.dtype !== "uint32") ||
        (fp32 && t.dtype === "float16") || !isShape(t.logicalShape) || !isShape(t.storageShape) ||
        typeof t.layout !== "string")
      throw new Error(`Invalid packed tensor ${name}`);
  }
  return value;
}

/* ---------------------------------------------------------- runtime plan */

function paletteBitsForLayout(layout) {
  if (layout === "k-by-output-row-major-palette5-lsb-u32") return 5;
  if (layout === "k-by-output-row-major-palette6-lsb-u32") return 6;
  return undefined;
}

function alignRuntimeOffset(value) {
  if (!Number.isSafeInteger(value) || value < 0) throw new RangeError("Runtime tensor offset must be nonnegative");
  return Math.ceil(value / RUNTIME_STORAGE_ALIGNMENT) * RUNTIME_STORAGE_ALIGNMENT;
}

const sourceBufferId = (fileName) => `source-shard-${fileName}`;

/** requireSourceRange (runtime-plan.ts:624-640). */
function requireSourceRange(name, record, files) {
  const file = files.get(record.shard);
  if (file === undefined) throw new Error(`${name} is not stored in a binary shard`);
  if (record.byteOffset % RUNTIME_STORAGE_ALIGNMENT !== 0 || record.byteLength % 4 !== 0 ||
      record.byteOffset + record.byteLength > file.byteLength)
    throw new Error(`${name} exceeds its aligned source shard`);
}

/** validatePalettePair (runtime-plan.ts:527-598). */
function validatePalettePair(name, source, paletteName, palette, bits, contract) {
  if (source.dtype !== "uint32" || source.logicalShape.length !== 2)
    throw new Error(`${name} has invalid palette indices`);
  const [inner, columns] = source.logicalShape;
  const codesPerGroup = bits === 5 ? 32 : 16;
  const wordsPerGroup = bits === 5 ? 5 : 3;
  const scalars = inner * columns;
  if (!Number.isSafeInteger(scalars) || columns % codesPerGroup !== 0 || scalars % codesPerGroup !== 0)
    throw new Error(`${name} has unaligned palette codes`);
  const groups = scalars / codesPerGroup;
  if (source.storageShape.join(",") !== `${groups},${wordsPerGroup}` ||
      source.byteLength !== groups * wordsPerGroup * 4)
    throw new Error(`${name} has invalid packed palette storage`);
  const entries = 1 << bits;
  if (palette.shard !== source.shard || palette.dtype !== contract.paletteDtype || palette.layout !== PALETTE_LAYOUT ||
      palette.logicalShape.length !== 2 || palette.logicalShape[1] !== entries ||
      palette.storageShape.join(",") !== palette.logicalShape.join(","))
    throw new Error(`${paletteName} has invalid palette storage`);
  const paletteGroups = palette.logicalShape[0];
  const groupColumns = columns / paletteGroups;
  if (columns % paletteGroups !== 0 || groupColumns % codesPerGroup !== 0 ||
      palette.byteLength !== paletteGroups * entries * contract.paletteElementBytes)
    throw new Error(`${paletteName} does not partition output columns`);
  return groupColumns;
}

function residentTensor(name, source, target) {
  if (source.byteOffset % 4 !== 0 || source.byteLength % 4 !== 0)
    throw new Error(`${name} cannot be copied as GPU words`);
  target.tensorCount += 1;
  return {
    name,
    sourceRecord: source,
    runtimeRecord: {
      bufferId: target.id,
      byteOffset: source.byteOffset,
      byteLength: source.byteLength,
      dtype: source.dtype,
      logicalShape: source.logicalShape,
      storageShape: source.storageShape,
      layout: source.layout,
    },
  };
}

/** requireFixedInventory (runtime-plan.ts:654-770). */
function requireFixedInventory(sourceBuffers, packed, contract) {
  if (sourceBuffers.size !== RESIDENT_SHARD_COUNT)
    throw new Error(`Resident source shard count changed: ${sourceBuffers.size}`);
  const decoder = sourceBuffers.get("decoder.bin");
  const subsampling = sourceBuffers.get("encoder-subsampling.bin");
  if (decoder === undefined || alignRuntimeOffset(decoder.cursor) !== contract.decoderShardBytes ||
      subsampling === undefined || alignRuntimeOffset(subsampling.cursor) !== contract.subsamplingShardBytes)
    throw new Error(`Resident ${contract.precision} common-source shard inventory changed`);
  for (let layer = 0; layer < ENCODER_LAYER_COUNT; ++layer) {
    const name = `encoder-layer-${String(layer).padStart(2, "0")}.bin`;
    const buffer = sourceBuffers.get(name);
    if (buffer === undefined || alignRuntimeOffset(buffer.cursor) !== contract.encoderLayerShardBytes)
      throw new Error(`Resident ${contract.precision} encoder-layer shard inventory changed: ${name}`);
  }
  const misplaced = (item) => paletteBitsForLayout(item.runtimeRecord.layout) === undefined ||
    item.runtimeRecord.dtype !== "uint32" ||
    (item.name.startsWith("encoder.layers.")
      ? !item.runtimeRecord.bufferId.startsWith("source-shard-encoder-layer-")
      : !COMMON_TRANSIENT_PALETTE_TENSORS.has(item.name));
  if (packed.length !== ENCODER_LAYER_COUNT * 8 + COMMON_TRANSIENT_PALETTE_MATRIX_COUNT || packed.some(misplaced))
    throw new Error(`Packed encoder-layer matrix inventory changed: ${packed.length}`);
  const palette5 = packed.filter((item) => paletteBitsForLayout(item.runtimeRecord.layout) === 5).length;
  const palette6 = packed.length - palette5;
  if (palette5 !== 172 || palette6 !== 24)
    throw new Error(`Packed palette topology changed: ${palette5} palette5, ${palette6} palette6`);
  const layerCounts = new Array(ENCODER_LAYER_COUNT).fill(0);
  for (const item of packed) {
    if (COMMON_TRANSIENT_PALETTE_TENSORS.has(item.name)) continue;
    const match = item.name.match(/^encoder\.layers\.(\d+)\./);
    if (match === null) throw new Error(`Packed matrix ${item.name} has no encoder layer`);
    const layer = Number(match[1]);
    if (layerCounts[layer] === undefined) throw new Error(`Packed matrix ${item.name} has invalid encoder layer`);
    layerCounts[layer] += 1;
  }
  if (layerCounts.some((count) => count !== 8))
    throw new Error(`Packed encoder layer inventories changed: ${layerCounts.join(",")}`);
  const common = packed.filter((item) => COMMON_TRANSIENT_PALETTE_TENSORS.has(item.name)).length;
  if (common !== COMMON_TRANSIENT_PALETTE_MATRIX_COUNT)
    throw new Error(`Common packed matrix inventory changed: ${common}`);
}

function shardLoadRank(name) {
  if (name === "decoder.bin") return 0;
  if (name === "encoder-subsampling.bin") return 1;
  if (/^encoder-layer-\d{2}\.bin$/.test(name)) return 2;
  return 3;
}

/* String order of the reference's localeCompare on these ASCII names. */
const compareNames = (a, b) => (a < b ? -1 : a > b ? 1 : 0);

/**
 * planRuntimePackage (runtime-plan.ts:144-340): every non-preprocessor shard
 * stays resident as one buffer, all 196 palette matrices stay packed, and the
 * inventory and byte totals must be those of the published package.
 */
function planRuntimePackage(manifest) {
  const contract = PACKAGE_CONTRACTS[parakeetManifestPrecision(manifest)];
  const binaryFiles = manifest.files.filter((file) => file.name.endsWith(".bin"));
  const fileMap = new Map(binaryFiles.map((file) => [file.name, file]));
  const sourceBuffers = new Map(
    binaryFiles.filter((file) => file.name !== PREPROCESSOR_SHARD).map((file) => [
      file.name,
      { id: sourceBufferId(file.name), label: `parakeet-source-${file.name}`, cursor: file.byteLength, tensorCount: 0 },
    ]),
  );
  const tensors = new Map();
  const packed = [];
  const consumedPalettes = new Set();
  let skippedPreprocessor = 0;
  const add = (plan) => {
    if (tensors.has(plan.name)) throw new Error(`Duplicate runtime tensor ${plan.name}`);
    tensors.set(plan.name, plan);
  };
  const names = Object.keys(manifest.tensors).sort(compareNames);
  for (const name of names) {
    const source = manifest.tensors[name];
    requireSourceRange(name, source, fileMap);
    if (contract.precision === "fp32" && source.dtype === "float16")
      throw new Error(`${name} cannot retain float16 storage in the FP32 package`);
    if (PREPROCESSOR_TENSORS.has(name)) {
      if (source.shard !== PREPROCESSOR_SHARD) throw new Error(`${name} must remain sourced from preprocessor.bin`);
      skippedPreprocessor += 1;
      continue;
    }
    const target = sourceBuffers.get(source.shard);
    if (target === undefined) throw new Error(`${name} cannot use GPU-unresident ${source.shard}`);
    const bits = paletteBitsForLayout(source.layout);
    if (bits !== undefined) {
      const paletteName = `${name}.palette`;
      const palette = manifest.tensors[paletteName];
      if (palette === undefined) throw new Error(`${name} is missing ${paletteName}`);
      requireSourceRange(paletteName, palette, fileMap);
      validatePalettePair(name, source, paletteName, palette, bits, contract);
      const plan = residentTensor(name, source, target);
      add(plan);
      packed.push(plan);
      consumedPalettes.add(paletteName);
      continue;
    }
    add(residentTensor(name, source, target));
  }
  const unowned = Object.keys(manifest.tensors)
    .filter((name) => manifest.tensors[name].layout === PALETTE_LAYOUT && !consumedPalettes.has(name));
  if (unowned.length > 0) throw new Error(`Unowned palette LUT tensors: ${unowned.join(",")}`);
  if (skippedPreprocessor !== PREPROCESSOR_TENSORS.size)
    throw new Error("The package must contain exactly two Wasm-owned preprocessor tensors");
  requireFixedInventory(sourceBuffers, packed, contract);
  const retainedRuntimeBytes = sum([...sourceBuffers.values()].map((b) => alignRuntimeOffset(b.cursor)));
  if (retainedRuntimeBytes !== contract.retainedRuntimeBytes)
    throw new Error(`Retained ${contract.precision} runtime package changed: ${retainedRuntimeBytes} bytes`);
  if (tensors.size !== RETAINED_RUNTIME_TENSOR_COUNT)
    throw new Error(`Retained runtime tensor count changed: ${tensors.size}`);
  const buffers = [...sourceBuffers.values()].map((b) => ({
    id: b.id, label: b.label, byteLength: alignRuntimeOffset(b.cursor), tensorCount: b.tensorCount,
  }));
  for (const buffer of buffers) {
    if (buffer.byteLength <= 0 || buffer.byteLength > RUNTIME_BUFFER_LIMIT_BYTES)
      throw new Error(`${buffer.id} exceeds the fixed 128 MiB runtime-buffer boundary`);
  }
  const shards = [...binaryFiles]
    .sort((a, b) => shardLoadRank(a.name) - shardLoadRank(b.name) || compareNames(a.name, b.name))
    .map((file) => {
      if (file.name === PREPROCESSOR_SHARD) return { file, hashOnly: true };
      const target = sourceBuffers.get(file.name);
      if (target === undefined) throw new Error(`${file.name} has no resident source buffer`);
      return { file, runtimeBufferId: target.id, hashOnly: false };
    });
  requireWholeShardInventory(shards, buffers);
  const memory = {
    packedDownloadBytes: sum(binaryFiles.map((file) => file.byteLength)),
    retainedRuntimeBytes,
    expandedRuntimeBytes: 0,
    runtimeGpuBytes: retainedRuntimeBytes,
    largestRuntimeShardBytes: Math.max(...shards.filter((s) => !s.hashOnly).map((s) => s.file.byteLength)),
    loaderPeakGpuBytes: retainedRuntimeBytes,
    runtimeBufferCount: buffers.length,
  };
  requireFixedMemory(memory, contract);
  return { buffers, tensors, shards, memory };
}

/** requireWholeRuntimeShardInventory (runtime-plan.ts:819-858). */
function requireWholeShardInventory(shards, buffers) {
  const plans = new Map(buffers.map((b) => [b.id, b]));
  const seen = new Set();
  let hashOnly = 0;
  for (const shard of shards) {
    if (shard.hashOnly) {
      hashOnly += 1;
      if (shard.file.name !== PREPROCESSOR_SHARD)
        throw new Error(`${shard.file.name} cannot be a hash-only runtime shard`);
      continue;
    }
    const target = plans.get(shard.runtimeBufferId);
    if (target === undefined || target.byteLength !== shard.file.byteLength || seen.has(shard.runtimeBufferId))
      throw new Error(`${shard.file.name} is not a unique whole runtime shard`);
    seen.add(shard.runtimeBufferId);
  }
  if (hashOnly !== 1 || seen.size !== ENCODER_LAYER_COUNT + 2 || seen.size !== buffers.length)
    throw new Error("The fixed package must contain one hash-only preprocessor shard and 26 whole runtime shards");
}

/** requireFixedMemory (runtime-plan.ts:783-808). */
function requireFixedMemory(memory, contract) {
  const expected = {
    packedDownloadBytes: contract.packedDownloadBytes,
    retainedRuntimeBytes: contract.retainedRuntimeBytes,
    expandedRuntimeBytes: 0,
    runtimeGpuBytes: contract.retainedRuntimeBytes,
    largestRuntimeShardBytes: contract.decoderShardBytes,
    loaderPeakGpuBytes: contract.retainedRuntimeBytes,
    runtimeBufferCount: RESIDENT_SHARD_COUNT,
  };
  for (const name of Object.keys(expected)) {
    if (memory[name] !== expected[name])
      throw new Error(`Runtime ${contract.precision} package memory ${name} changed: ${String(memory[name])}`);
  }
}

/* ---------------------------------------------------------------- loader */

const SHARD_CHUNK_BYTES = 8 * 1024 * 1024;

function sha256Hex(bytes) {
  return crypto.createHash("sha256").update(bytes).digest("hex");
}

/**
 * streamAndValidateShard (package.ts:382-496): reads the file in chunks,
 * hashes every byte and, for a resident shard, writes the words to the
 * shard's device buffer as they arrive.
 */
function streamAndValidateShard(device, directory, file, target, onProgress) {
  const filePath = path.join(directory, file.name);
  let fd;
  try {
    fd = fs.openSync(filePath, "r");
  } catch (error) {
    throw new Error(`Model shard ${file.name} failed (${error.code || error.message})`);
  }
  try {
    const size = fs.fstatSync(fd).size;
    if (size > file.byteLength) throw new Error(`${file.name} exceeds declared size`);
    const hash = crypto.createHash("sha256");
    const chunk = Buffer.allocUnsafe(Math.min(SHARD_CHUNK_BYTES, Math.max(file.byteLength, 4)));
    let readBytes = 0;
    for (;;) {
      const n = fs.readSync(fd, chunk, 0, chunk.length, readBytes);
      if (n === 0) break;
      if (readBytes + n > file.byteLength) throw new Error(`${file.name} exceeds declared size`);
      const view = chunk.subarray(0, n);
      hash.update(view);
      if (target !== undefined) {
        if (n % 4 !== 0) throw new Error(`${file.name} ended before its aligned declared length`);
        device.queue.writeBuffer(target, readBytes, view);
      }
      readBytes += n;
      if (onProgress) onProgress(readBytes);
    }
    if (readBytes !== file.byteLength) throw new Error(`${file.name} ended before its aligned declared length`);
    if (hash.digest("hex") !== file.sha256) throw new Error(`${file.name} SHA-256 validation failed`);
  } finally {
    fs.closeSync(fd);
  }
}

function requiredFile(manifest, name) {
  const record = manifest.files.find((candidate) => candidate.name === name);
  if (record === undefined) throw new Error(`Model package is missing ${name}`);
  return record;
}

/**
 * ParakeetGpuPackage (package.ts:52-232): the validated manifest, the
 * runtime plan and one resident device buffer per weight shard.
 */
class ParakeetGpuPackage {
  constructor(manifest, tensorPlans, buffers, tokenizer, memory, provenance) {
    this._manifest = manifest;
    this._tokenizer = tokenizer;
    this._tensorPlans = tensorPlans;
    this.buffers = buffers;
    this.memory = memory;
    this.precision = parakeetManifestPrecision(manifest);
    this.manifestUrl = provenance.manifestUrl;
    this.manifestSha256 = provenance.manifestSha256;
    this.manifestListedBytes = sum(manifest.files.map((file) => file.byteLength));
    this.destroyed = false;
  }

  get manifest() {
    if (this._manifest === undefined) throw new Error("Parakeet model initialization metadata was released");
    return this._manifest;
  }

  get tokenizer() {
    if (this._tokenizer === undefined) throw new Error("Parakeet tokenizer metadata was released");
    return this._tokenizer;
  }

  /**
   * load(device, manifestPath, options): options.expectedPrecision ("fp16"
   * or "fp32", required), options.manifestSha256 (overrides the published
   * digest), options.onProgress({phase, file?, loadedBytes, totalBytes}).
   */
  static load(device, manifestPath, options) {
    return new Promise((resolve) => resolve(ParakeetGpuPackage.loadNow(device, manifestPath, options)));
  }

  static loadNow(device, manifestPath, options) {
    const o = options || {};
    const onProgress = o.onProgress;
    if (onProgress) onProgress({ phase: "manifest", loadedBytes: 0, totalBytes: 0 });
    let manifestBytes;
    try {
      manifestBytes = fs.readFileSync(manifestPath);
    } catch (error) {
      throw new Error(`Model manifest request failed (${error.code || error.message})`);
    }
    const manifestSha256 = sha256Hex(manifestBytes);
    const expected = o.manifestSha256 !== undefined ? o.manifestSha256 : parakeetManifestSha256(o.expectedPrecision);
    if (manifestSha256 !== expected)
      throw new Error(`Selected ${o.expectedPrecision} model manifest SHA-256 changed: ${manifestSha256}`);
    const manifest = parseParakeetManifest(JSON.parse(manifestBytes.toString("utf8")));
    const precision = parakeetManifestPrecision(manifest);
    if (precision !== o.expectedPrecision)
      throw new Error(`Selected ${o.expectedPrecision} execution but received a ${precision} model package`);
    const plan = planRuntimePackage(manifest);
    const directory = path.dirname(manifestPath);
    const buffers = new Map();
    try {
      let completed = 0;
      for (const shard of plan.shards) {
        const report = onProgress && ((loaded) => onProgress({
          phase: "weights", file: shard.file.name, loadedBytes: completed + loaded,
          totalBytes: plan.memory.packedDownloadBytes,
        }));
        if (shard.hashOnly) {
          streamAndValidateShard(device, directory, shard.file, undefined, report);
        } else {
          const buffer = device.createBuffer({ label: `parakeet-source-${shard.file.name}`, size: shard.file.byteLength });
          try {
            streamAndValidateShard(device, directory, shard.file, buffer, report);
          } catch (error) {
            buffer.destroy();
            throw error;
          }
          if (buffers.has(shard.runtimeBufferId)) {
            buffer.destroy();
            throw new Error(`Runtime buffer ${shard.runtimeBufferId} was already allocated`);
          }
          buffers.set(shard.runtimeBufferId, buffer);
        }
        completed += shard.file.byteLength;
      }
      if (buffers.size !== plan.buffers.length)
        throw new Error(`Runtime loader materialized ${buffers.size} of ${plan.buffers.length} buffers`);
      const tokenizerRecord = requiredFile(manifest, "tokenizer.json");
      if (onProgress) onProgress({ phase: "tokenizer", loadedBytes: 0, totalBytes: tokenizerRecord.byteLength });
      let tokenizerBytes;
      try {
        tokenizerBytes = fs.readFileSync(path.join(directory, tokenizerRecord.name));
      } catch (error) {
        throw new Error(`Tokenizer request failed (${error.code || error.message})`);
      }
      if (tokenizerBytes.length !== tokenizerRecord.byteLength || sha256Hex(tokenizerBytes) !== tokenizerRecord.sha256)
        throw new Error("Tokenizer integrity validation failed");
      const tokenizer = JSON.parse(tokenizerBytes.toString("utf8"));
      if (onProgress)
        onProgress({ phase: "ready", loadedBytes: plan.memory.packedDownloadBytes,
                     totalBytes: plan.memory.packedDownloadBytes });
      return new ParakeetGpuPackage(manifest, plan.tensors, buffers, tokenizer, plan.memory,
                                    { manifestUrl: manifestPath, manifestSha256 });
    } catch (error) {
      for (const buffer of buffers.values()) buffer.destroy();
      throw error;
    }
  }

  /** tensor(name) (package.ts:178-206): {sourceRecord, runtimeRecord, buffer, binding}. */
  tensor(name) {
    if (this.destroyed) throw new Error("Parakeet model package was destroyed");
    const plans = this._tensorPlans;
    const plan = plans === undefined ? undefined : plans.get(name);
    if (plan === undefined) {
      if (plans === undefined) throw new Error("Parakeet tensor metadata was released");
      throw new Error(`Unknown runtime tensor ${name}`);
    }
    const runtime = plan.runtimeRecord;
    const buffer = this.buffers.get(runtime.bufferId);
    if (buffer === undefined) throw new Error(`Runtime buffer ${runtime.bufferId} is not resident`);
    return {
      sourceRecord: plan.sourceRecord,
      runtimeRecord: runtime,
      buffer,
      binding: { buffer, offset: runtime.byteOffset, size: runtime.byteLength },
    };
  }

  releaseInitializationMetadata() {
    if (this.destroyed) throw new Error("Parakeet model package was destroyed");
    this._manifest = undefined;
    this._tokenizer = undefined;
    this._tensorPlans = undefined;
  }

  destroy() {
    if (this.destroyed) return;
    this.destroyed = true;
    this._manifest = undefined;
    this._tokenizer = undefined;
    this._tensorPlans = undefined;
    for (const buffer of new Set(this.buffers.values())) buffer.destroy();
    this.buffers.clear();
  }
}

module.exports = {
  PARAKEET_FP16_PACKAGE_FORMAT,
  PARAKEET_FP32_PACKAGE_FORMAT,
  PARAKEET_FP16_ENCODER_WEIGHT_FORMAT,
  PARAKEET_FP32_ENCODER_WEIGHT_FORMAT,
  PARAKEET_FP16_MANIFEST_SHA256,
  PARAKEET_FP32_MANIFEST_SHA256,
  PARAKEET_FFN_SOURCE_WIDTH,
  PARAKEET_SOURCE,
  PARAKEET_FIXED_CONFIG,
  RUNTIME_STORAGE_ALIGNMENT,
  RUNTIME_BUFFER_LIMIT_BYTES,
  FP16_PACKED_DOWNLOAD_BYTES,
  FP16_RETAINED_RUNTIME_BYTES,
  FP16_LARGEST_RUNTIME_SHARD_BYTES,
  FP32_PACKED_DOWNLOAD_BYTES,
  FP32_RETAINED_RUNTIME_BYTES,
  FP32_LARGEST_RUNTIME_SHARD_BYTES,
  parakeetManifestPrecision,
  parakeetManifestSha256,
  parseParakeetManifest,
  paletteBitsForLayout,
  alignRuntimeOffset,
  planRuntimePackage,
  ParakeetGpuPackage,
};
