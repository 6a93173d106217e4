// CPU checks of the Node host (no GPU): exports, record checks and the
// C ABI descriptor contract reached through the N-API addon. Run by
// tests/test_node_host.py; exits non-zero on the first failure.
"use strict";
const assert = require("assert");
const path = require("path");
const host = require(path.join(__dirname, "..", "..", "parakeet.wgsl_amd", "host"));

const native = host.native();
assert.strictEqual(native.abiVersion(), 1);
for (const name of ["contextCreate", "gemmCreate", "gemmValidate", "gemmEnqueue", "gemmDestroy", "gemmPlan",
                    "tdtCreate", "tdtEnqueue", "tdtSetTeamSize", "tdtTeamSize",
                    "preparedWeightCreate", "synchronizeAsync", "alloc", "upload", "download"]) {
  assert.strictEqual(typeof native[name], "function", name);
}
assert.strictEqual(host.paletteBitsForLayout("k-by-output-row-major-palette5-lsb-u32"), 5);
assert.strictEqual(host.paletteBitsForLayout("k-by-output-row-major-palette6-lsb-u32"), 6);
assert.strictEqual(host.paletteBitsForLayout("n256-k32-tile-major-f16"), undefined);

// A kernel over a stand-in device and arena: descriptor checks need no GPU.
const fakeBuffer = { address: 1n << 20n, label: "fake" };
const arena = Object.create(host.GpuActivationArena.prototype);
Object.assign(arena, { buffer: fakeBuffer, byteLength: 1 << 30, destroyed: false, label: "arena" });
function tensor(records) {
  return { sourceRecord: records.sourceRecord, runtimeRecord: records.runtimeRecord,
           binding: { buffer: fakeBuffer, offset: 0, size: records.runtimeRecord.byteLength } };
}
function descriptor(over) {
  const rows = over.rows || 7520, inner = over.inner || 1024, columns = over.columns || 4096;
  const bits = over.bits || 5;
  const rec = host.paletteTensorRecords({ paletteBits: bits, inner, columns, paletteGroups: over.groups || 1 });
  const d = {
    label: over.label || "encoder-layer-ff-expand",
    a: arena.slice("a", 0, rows * inner * 2),
    b: tensor(rec.weight),
    bPalette: tensor(rec.palette),
    paletteGroupColumns: columns / (over.groups || 1),
    output: arena.slice("c", 256 * 1024 * 1024, rows * columns * 2),
    rows, inner, columns,
  };
  if (over.activation !== undefined) d.activation = over.activation;
  if (over.residual) d.residual = arena.slice("r", 512 * 1024 * 1024, rows * columns * 2);
  if (over.residualScale !== undefined) d.residualScale = over.residualScale;
  if (over.mutate) over.mutate(d, rec);
  return d;
}

function throwsLike(fn, Kind, text) {
  let caught = null;
  try { fn(); } catch (e) { caught = e; }
  assert.ok(caught, `expected ${Kind.name}: ${text}`);
  assert.ok(caught instanceof Kind, `${caught.constructor.name} is not ${Kind.name}: ${caught.message}`);
  assert.ok(caught.message.includes(text), `"${caught.message}" lacks "${text}"`);
}

host.F16GemmKernel.create({}, arena).then((kernel) => {
  // A production signature passes (gemm.ts:204-356).
  kernel.validateDescriptor(descriptor({ activation: "silu" }));
  kernel.validateDescriptor(descriptor({ label: "encoder-layer-ff-contract", inner: 4096, columns: 1024,
                                         residual: true, residualScale: 0.5 }));
  kernel.validateDescriptor(descriptor({ label: "encoder-layer-attention-qkv", columns: 3072, groups: 3 }));
  // requireGemmShape (gemm.ts:971-1010)
  throwsLike(() => kernel.validateDescriptor(descriptor({ inner: 1000, activation: "silu" })), RangeError,
             "Unsupported GEMM shape for encoder-layer-ff-expand");
  throwsLike(() => kernel.validateDescriptor(descriptor({ columns: 4100, activation: "silu" })), RangeError,
             "Unsupported GEMM shape for encoder-layer-ff-expand");
  throwsLike(() => kernel.validateDescriptor(descriptor({ activation: "silu",
      mutate: (d) => { d.b.sourceRecord = Object.assign({}, d.b.sourceRecord, { logicalShape: [2048, 4096] }); } })),
      Error, "weight package does not match K=1024, N=4096");
  throwsLike(() => kernel.validateDescriptor(descriptor({ activation: "silu",
      mutate: (d) => { d.b.sourceRecord = Object.assign({}, d.b.sourceRecord, { layout: "n256-k32-tile-major-f16" }); } })),
      Error, "has an unsupported weight format");
  throwsLike(() => kernel.validateDescriptor(descriptor({ activation: "silu",
      mutate: (d) => { d.b.sourceRecord = Object.assign({}, d.b.sourceRecord, { byteLength: 4 }); } })),
      Error, "has invalid packed palette indices");
  // requireProductionSpecialization (gemm.ts:1031-1067)
  throwsLike(() => kernel.validateDescriptor(descriptor({})), Error,
             "encoder-layer-ff-expand is not a fixed production GEMM signature: M=7520, K=1024, N=4096, " +
             "activation=none, bias=false, residualScale=none");
  throwsLike(() => kernel.validateDescriptor(descriptor({ activation: "silu", residualScale: 0.5 })), Error,
             "supplies a residual scale without a residual");
  // requireRuntimeWeight (gemm.ts:1069-1161)
  throwsLike(() => kernel.validateDescriptor(descriptor({ activation: "silu",
      mutate: (d) => { d.bPalette.sourceRecord = Object.assign({}, d.bPalette.sourceRecord, { dtype: "float32" }); } })),
      Error, "has invalid transient palette weights");
  throwsLike(() => kernel.validateDescriptor(descriptor({ activation: "silu", mutate: (d) => { d.paletteGroupColumns = 1024; } })),
      Error, "has invalid transient palette weights");
  // rowNorm (PK_GEMM_ROW_NORM, no reference counterpart): f32 gamma and beta of K channels
  const normTensor = (size) => ({ binding: { buffer: fakeBuffer, offset: 0, size } });
  kernel.validateDescriptor(descriptor({ activation: "silu",
    mutate: (d) => { d.rowNorm = { gamma: normTensor(4096), beta: normTensor(4096), epsilon: 1e-5 }; } }));
  throwsLike(() => kernel.validateDescriptor(descriptor({ activation: "silu",
    mutate: (d) => { d.rowNorm = { gamma: normTensor(4096), beta: normTensor(4092) }; } })),
      Error, "row norm needs gamma and beta of 4096 bytes");
  throwsLike(() => kernel.validateDescriptor(descriptor({ activation: "silu",
    mutate: (d) => { d.rowNorm = { gamma: normTensor(4096), beta: normTensor(4096), epsilon: -1 }; } })),
      Error, "epsilon >= 0");
  // cachedOutput (PK_GEMM_CACHED_OUTPUT, no reference counterpart): a store hint the contract accepts
  kernel.validateDescriptor(descriptor({ activation: "silu", mutate: (d) => { d.cachedOutput = true; } }));
  // arena.ts slice rules
  throwsLike(() => arena.slice("x", 100, 64), RangeError, "Invalid activation slice x");
  // the counters of a fused kernel: nothing is ever expanded
  const backend = host.createEncoderGemmBackend(kernel);
  assert.strictEqual(backend.transientPaletteDispatchCount, 0);
  assert.strictEqual(backend.transientPaletteExpandedBytes, 0);
  // synthetic shapes are accepted when asked for
  return host.F16GemmKernel.create({}, arena, undefined, { allowSyntheticShapes: true }).then((synthetic) => {
    synthetic.validateDescriptor(descriptor({ rows: 300, inner: 1024, columns: 512, bits: 6 }));
    return host.FusedConformerConvKernel.create({}, arena, 64);
  }).then((conv) => {
    // planFusedConformerConv known answers (conformer-conv-kernel-shapes.test.ts:18-58)
    const plan = host.planFusedConformerConv({ batchSize: 2, frames: 188 });
    assert.strictEqual(plan.rows, 376);
    assert.strictEqual(plan.inputByteLength, 376 * host.CONFORMER_CONV_POINTWISE_CHANNELS * 2);
    assert.strictEqual(plan.outputByteLength, 376 * host.CONFORMER_CONV_CHANNELS * 2);
    assert.strictEqual(plan.validLengthsByteLength, 8);
    assert.strictEqual(plan.depthwiseWeightByteLength, host.CONFORMER_CONV_KERNEL_SIZE * 1024 * 2);
    assert.strictEqual(plan.affineByteLength, 4096);
    const plan32 = host.planFusedConformerConv({ batchSize: 2, frames: 188 }, { precision: "fp32" });
    assert.strictEqual(plan32.inputByteLength, 376 * 2048 * 4);
    assert.strictEqual(plan32.depthwiseWeightByteLength, 9 * 1024 * 4);
    assert.strictEqual(host.CONFORMER_DEPTHWISE_WEIGHT_LAYOUT, "kernel-channel-vec4");
    assert.strictEqual(host.CONFORMER_FOLDED_BATCH_NORM_LAYOUT, "channel");
    throwsLike(() => host.planFusedConformerConv({ batchSize: 0, frames: 188 }), RangeError,
               "batchSize must be a positive integer");
    throwsLike(() => host.planFusedConformerConv({ batchSize: 1, frames: 1.5 }), RangeError,
               "frames must be a positive integer");
    const rec = host.conformerConvTensorRecords();
    function convDescriptor(mutate) {
      const d = {
        label: "layer0-convolution-glu-depthwise-bn-silu", batchSize: 2, frames: 188,
        pointwiseInput: arena.slice("p", 0, 376 * 2048 * 2),
        depthwiseWeights: tensor(rec.depthwiseWeights),
        batchNormScale: tensor(rec.batchNormScale),
        batchNormShift: tensor(rec.batchNormShift),
        validLengths: arena.slice("v", 128 * 1024 * 1024, 8),
        output: arena.slice("z", 256 * 1024 * 1024, 376 * 1024 * 2),
      };
      if (mutate) mutate(d);
      return d;
    }
    conv.validateDescriptor(convDescriptor());
    throwsLike(() => conv.validateDescriptor(convDescriptor((d) => {
      d.output = arena.slice("z", 256 * 1024 * 1024, 376 * 1024 * 2 - 4);
    })), RangeError, "layer0-convolution-glu-depthwise-bn-silu output needs 770048 bytes; arena slice has 770044");
    throwsLike(() => conv.validateDescriptor(convDescriptor((d) => {
      d.depthwiseWeights = Object.assign({}, d.depthwiseWeights, {
        runtimeRecord: Object.assign({}, rec.depthwiseWeights.runtimeRecord, { layout: "channel" }) });
    })), Error, "depthwise weights must be float16 kernel-channel-vec4 logical [9,1024], storage [9,256,4], 18432 bytes");
    throwsLike(() => conv.validateDescriptor(convDescriptor((d) => {
      d.batchNormShift = Object.assign({}, d.batchNormShift, {
        runtimeRecord: Object.assign({}, rec.batchNormShift.runtimeRecord, { dtype: "float16" }) });
    })), Error, "folded batch norm shift must be float32 channel logical [1024], storage [1024], 4096 bytes");
    throwsLike(() => conv.validateDescriptor(convDescriptor((d) => {
      d.output = arena.slice("z", 4096, 376 * 1024 * 2);
    })), Error, "must not overlap the pointwise input");
    return host.RelativeAttentionKernel.create({}, arena, 64);
  }).then((attention) => {
    const rec = host.relativeAttentionTensorRecords(188);
    function attDescriptor(mutate) {
      const d = {
        label: "layer0-relative-attention", batchSize: 2, frames: 188,
        qkv: arena.slice("qkv", 0, 376 * 3072 * 2),
        projectedPositions: tensor(rec.projectedPositions),
        biasU: tensor(rec.biasU), biasV: tensor(rec.biasV),
        validLengths: arena.slice("v", 128 * 1024 * 1024, 8),
        output: arena.slice("ctx", 256 * 1024 * 1024, 376 * 1024 * 2),
      };
      if (mutate) mutate(d);
      return d;
    }
    attention.validateDescriptor(attDescriptor());
    throwsLike(() => attention.validateDescriptor(attDescriptor((d) => { d.frames = 0; })), RangeError,
               "Unsupported attention shape for layer0-relative-attention");
    throwsLike(() => attention.validateDescriptor(attDescriptor((d) => {
      d.qkv = arena.slice("qkv", 0, 376 * 3072 * 2 - 4);
    })), RangeError, "layer0-relative-attention QKV needs 2310144 bytes; arena slice has 2310140");
    throwsLike(() => attention.validateDescriptor(attDescriptor((d) => {
      d.projectedPositions = tensor(host.relativeAttentionTensorRecords(187).projectedPositions);
    })), Error, "Projected positions must be float16 head-vector-position-vec4, logical [375,1024], storage [8,32,375,4]");
    throwsLike(() => attention.validateDescriptor(attDescriptor((d) => {
      d.biasV = Object.assign({}, d.biasV, { runtimeRecord: Object.assign({}, rec.biasV.runtimeRecord, { dtype: "float16" }) });
    })), Error, "layer0-relative-attention bias V must be float32 head-by-channel logical/storage [8,128]");
    return host.LayerNormKernel.create({}, arena, 64);
  }).then((norm) => {
    // createDispatch checks of layernorm.ts:165-240
    const affine = host.channelTensorRecords(1024);
    function lnDescriptor(mutate) {
      const d = {
        label: "encoder.layers.0.norm_feed_forward1", rows: 3008, channels: 1024,
        input: arena.slice("x", 0, 3008 * 1024 * 2), output: arena.slice("y", 64 * 1024 * 1024, 3008 * 1024 * 2),
        gamma: tensor(affine), beta: tensor(affine),
      };
      if (mutate) mutate(d);
      return d;
    }
    norm.validateDescriptor(lnDescriptor());
    throwsLike(() => norm.validateDescriptor(lnDescriptor((d) => { d.channels = 1022; })), RangeError,
               "Invalid LayerNorm shape for encoder.layers.0.norm_feed_forward1");
    throwsLike(() => norm.validateDescriptor(lnDescriptor((d) => { d.output = arena.slice("y", 0, 1024); })),
               RangeError, "encoder.layers.0.norm_feed_forward1 output needs 6160384 bytes; arena slice has 1024");
    throwsLike(() => norm.validateDescriptor(lnDescriptor((d) => { d.beta = tensor(host.channelTensorRecords(512)); })),
               Error, "encoder.layers.0.norm_feed_forward1 beta must be float32 channel logical/storage [1024], 4096 bytes");
    // a chained LayerNorm (no reference counterpart): its output may be the input, never the output
    norm.validateDescriptor(lnDescriptor((d) => {
      d.next = { gamma: tensor(affine), beta: tensor(affine), output: d.input };
    }));
    throwsLike(() => norm.validateDescriptor(lnDescriptor((d) => {
      d.next = { gamma: tensor(affine), beta: tensor(affine), output: arena.slice("z", 64 * 1024 * 1024 + 2048, 3008 * 1024 * 2) };
    })), Error, "next output must not overlap the output");
    const wide = host.channelTensorRecords(4096);
    throwsLike(() => norm.validateDescriptor(lnDescriptor((d) => {
      d.channels = 4096;
      d.input = arena.slice("x", 0, 3008 * 4096 * 2);
      d.output = arena.slice("y", 64 * 1024 * 1024, 3008 * 4096 * 2);
      d.gamma = tensor(wide);
      d.beta = tensor(wide);
      d.next = { gamma: tensor(wide), beta: tensor(wide), output: d.input };
    })), RangeError, "chained LayerNorm needs rows of at most 4096 bytes");
    return host.FusedSubsamplingConv0Depthwise2Kernel.create({}, arena, 64);
  }).then((fused) => {
    // subsampling-kernel-shapes.test.ts:27-50 and createDispatch (subsampling.ts:334-387)
    assert.deepStrictEqual([1501, 751, 376].map((n) => host.subsamplingOutputDimension(n)), [751, 376, 188]);
    assert.deepStrictEqual([1, 2, 3].map((s) => host.subsamplingValidLength(799, s)), [400, 200, 100]);
    assert.deepStrictEqual(Array.from(host.deriveEncoderValidLengths([1500, 799, 1])), [188, 100, 1]);
    throwsLike(() => host.deriveEncoderValidLength(1502), RangeError, "featureLength must not exceed 1501");
    const rec = host.subsamplingTensorRecords();
    function fusedDescriptor(mutate) {
      const d = {
        label: "subsampling-fused-conv0-depthwise2-batch-0-size-3", batchSize: 3, inputHeight: 1501,
        inputWidth: 128, channels: 256, input: arena.slice("fbank", 0, 3 * 1501 * 128 * 4),
        conv0Weights: tensor(rec.conv0Weights), conv0Bias: tensor(rec.bias),
        depthwiseWeights: tensor(rec.depthwiseWeights), depthwiseBias: tensor(rec.bias),
        output: arena.slice("stage376", 64 * 1024 * 1024, 3 * 376 * 32 * 256 * 2),
        validLengths: arena.slice("lengths", 128 * 1024 * 1024, 12),
      };
      if (mutate) mutate(d);
      return d;
    }
    fused.validateDescriptor(fusedDescriptor());
    throwsLike(() => fused.validateDescriptor(fusedDescriptor((d) => { d.inputWidth = 80; })), RangeError,
               "Fused conv0+depthwise2 requires fixed");
    throwsLike(() => fused.validateDescriptor(fusedDescriptor((d) => {
      d.output = arena.slice("stage376", 64 * 1024 * 1024, 3 * 376 * 32 * 256 * 2 - 4);
    })), RangeError, "output needs 18481152 bytes; arena slice has 18481148");
    throwsLike(() => fused.validateDescriptor(fusedDescriptor((d) => { d.conv0Weights = tensor(rec.depthwiseWeights); })),
               Error, "conv0 weights must be float16 kh-kw-output-channel-vec4 logical [3,3,256], storage [3,3,64,4], 4608 bytes");
    return host.DepthwiseSubsamplingKernel.create({}, arena, 64).then((dw) => {
      const d = {
        label: "subsampling-depthwise5", batchSize: 3, inputHeight: 376, inputWidth: 32, channels: 256,
        input: arena.slice("p376", 0, 3 * 376 * 32 * 256 * 2), weights: tensor(rec.depthwiseWeights),
        bias: tensor(rec.bias), output: arena.slice("s188", 64 * 1024 * 1024, 3 * 188 * 16 * 256 * 2),
        validLengths: arena.slice("lengths", 128 * 1024 * 1024, 12), validLengthSubsamplingSteps: 3,
      };
      dw.validateDescriptor(d);
      throwsLike(() => dw.validateDescriptor(Object.assign({}, d, { validLengthSubsamplingSteps: 0 })), RangeError,
                 "subsampling-depthwise5 valid-length subsampling steps must be a positive integer");
      return host.SubsamplingTimeMaskKernel.create({}, arena, 64);
    }).then((mask) => {
      const d = {
        label: "subsampling-pointwise6-mask", batchSize: 3, height: 188, width: 16, channels: 256,
        values: arena.slice("p188", 0, 3 * 188 * 16 * 256 * 2), validLengths: arena.slice("lengths", 128 * 1024 * 1024, 12),
        validLengthSubsamplingSteps: 3,
      };
      mask.validateDescriptor(d);
      throwsLike(() => mask.validateDescriptor(Object.assign({}, d, { channels: 6 })), RangeError,
                 "Subsampling mask channels must be divisible by four");
    });
  }).then(() => {
    // ParakeetEncoderGraph.create resolves every tensor with requireTensorRecord (encoder.ts:2550-2581).
    const model = { tensor(name) { throw new Error(`Missing tensor ${name}`); } };
    return host.ParakeetEncoderGraph.create({}, model).then(() => assert.fail("created"), (e) => {
      assert.ok(/Missing tensor encoder\.layers\.0\.norm_feed_forward1\.weight/.test(e.message), String(e));
      const bad = { tensor(name) {
        const r = { dtype: "float16", layout: "channel", byteLength: 2048, logicalShape: [1024], storageShape: [1024] };
        return { sourceRecord: r, runtimeRecord: r, binding: { buffer: fakeBuffer, offset: 0, size: 2048 } };
      } };
      return host.ParakeetEncoderGraph.create({}, bad);
    }).then(() => assert.fail("created"), (e) => {
      assert.strictEqual(e.message, "encoder.layers.0.norm_feed_forward1.weight source must be float32 channel, " +
                         "logical [1024], storage [1024]");
      // requireEncoderConfig (encoder.ts:2588-2593): the profile must match the package
      const fp16Model = { precision: "fp16", tensor() { throw new Error("no tensor expected"); } };
      return host.ParakeetEncoderGraph.create({}, fp16Model, { executionProfile: { precision: "fp32" } });
    }).then(() => assert.fail("created"), (e) => {
      assert.strictEqual(e.message, "Parakeet fp32 encoder cannot use fp16 model weights");
      const fp32Model = { precision: "fp32", tensor() { throw new Error("no tensor expected"); } };
      return host.PersistentTdtDecoderKernel.create({}, arena, fp32Model, { precision: "fp16" });
    }).then(() => assert.fail("created"), (e) => {
      assert.strictEqual(e.message, "TDT decoder fp16 profile cannot use fp32 decoder weights");
      // status words: overflow and team sync timeout are separate causes
      assert.strictEqual(host.TDT_DECODER_SYNC_TIMEOUT, 2);
      assert.deepStrictEqual(host.decodeTdtStatus(0), { overflow: false, syncTimeout: false, unknown: 0 });
      assert.deepStrictEqual(host.decodeTdtStatus(1), { overflow: true, syncTimeout: false, unknown: 0 });
      assert.deepStrictEqual(host.decodeTdtStatus(2), { overflow: false, syncTimeout: true, unknown: 0 });
      assert.deepStrictEqual(host.decodeTdtStatus(0x80000003), { overflow: true, syncTimeout: true, unknown: 0x80000000 });
      assert.throws(() => host.decodeTdtStatus(-1), RangeError);
      console.log("host_cpu ok");
    });
  });
}).catch((e) => { console.error(e); process.exit(1); });
