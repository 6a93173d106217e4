// CPU checks of the package format in the Node host: manifest validation,
// the fixed runtime plan over the converter-shaped synthetic inventory, and
// the shard loader (streaming, SHA-256, errors) over a stand-in device.
// The expectations restate the reference's own tests
// (test/model/manifest.test.ts, test/model/runtime-plan.test.ts).
// argv: <fp16 manifest.json> <fp32 manifest.json> <written package manifest.json>
"use strict";
const assert = require("assert");
const fs = require("fs");
const path = require("path");
const host = require(path.join(__dirname, "..", "..", "parakeet.wgsl_amd", "host"));

const [fp16Path, fp32Path, packagePath] = process.argv.slice(2);
const load = (p) => JSON.parse(fs.readFileSync(p, "utf8"));
const clone = (v) => JSON.parse(JSON.stringify(v));

/* ---- manifest (manifest.test.ts) ---- */
assert.notStrictEqual(host.parakeetManifestSha256("fp16"), host.parakeetManifestSha256("fp32"));
assert.strictEqual(host.parakeetManifestSha256("fp16"), host.PARAKEET_FP16_MANIFEST_SHA256);
const base16 = load(fp16Path);
const base32 = load(fp32Path);
assert.strictEqual(host.parakeetManifestPrecision(host.parseParakeetManifest(clone(base16))), "fp16");
assert.strictEqual(host.parakeetManifestPrecision(host.parseParakeetManifest(clone(base32))), "fp32");
function rejects(manifest, pattern) {
  assert.throws(() => host.parseParakeetManifest(manifest), pattern);
}
{
  const m = clone(base16);
  m.config.encoderWeightFormat = host.PARAKEET_FP32_ENCODER_WEIGHT_FORMAT;
  rejects(m, /fixed encoder package contract/);
  const w = clone(base16);
  w.config.intermediateSize = 2560;
  rejects(w, /fixed encoder package contract/);
  const f = clone(base16);
  f.format = "parakeet-webgpu-fp64-v1";
  rejects(f, /Expected parakeet-webgpu-v1 or parakeet-webgpu-fp32-v1/);
  for (const [field, value] of [["vocabularySize", 8193], ["blankTokenId", 8192], ["jointOutputSize", 8198],
                                ["jointStorageOutputSize", 8200]]) {
    const v = clone(base16);
    v.config[field] = value;
    rejects(v, new RegExp(`Unsupported Parakeet config ${field}=`));
  }
  const d = clone(base16);
  d.config.durations = [0, 1, 2, 4];
  rejects(d, /Unsupported TDT duration table/);
  for (const change of [{ repository: "nvidia/parakeet-tdt-0.6b-v3" }, { revision: "other" }, { license: "MIT" },
                        { archive: Object.assign({}, base16.source.archive, { byteLength: 1 }) },
                        { weights: Object.assign({}, base16.source.weights, { sha256: "0".repeat(64) }) }]) {
    const s = clone(base16);
    Object.assign(s.source, change);
    rejects(s, /Invalid Parakeet source metadata/);
  }
  const h = clone(base32);
  h.tensors["decoder.lstm.bias_l0"].dtype = "float16";
  rejects(h, /Invalid packed tensor decoder\.lstm\.bias_l0/);
  const r = clone(base16);
  r.files[0].sha256 = "XYZ";
  rejects(r, /Invalid Parakeet file record/);
  const a = clone(base16);
  a.tensors["joint.head.bias"].byteOffset = 100;
  rejects(a, /Invalid packed tensor joint\.head\.bias/);
}

/* ---- plan (runtime-plan.test.ts) ---- */
for (const [manifest, precision] of [[base16, "fp16"], [base32, "fp32"]]) {
  const plan = host.planRuntimePackage(host.parseParakeetManifest(clone(manifest)));
  const fp32 = precision === "fp32";
  assert.strictEqual(plan.tensors.size, 795);
  assert.strictEqual(plan.buffers.length, 26);
  assert.deepStrictEqual(plan.memory, {
    packedDownloadBytes: fp32 ? host.FP32_PACKED_DOWNLOAD_BYTES : host.FP16_PACKED_DOWNLOAD_BYTES,
    retainedRuntimeBytes: fp32 ? host.FP32_RETAINED_RUNTIME_BYTES : host.FP16_RETAINED_RUNTIME_BYTES,
    expandedRuntimeBytes: 0,
    runtimeGpuBytes: fp32 ? host.FP32_RETAINED_RUNTIME_BYTES : host.FP16_RETAINED_RUNTIME_BYTES,
    largestRuntimeShardBytes: fp32 ? host.FP32_LARGEST_RUNTIME_SHARD_BYTES : host.FP16_LARGEST_RUNTIME_SHARD_BYTES,
    loaderPeakGpuBytes: fp32 ? host.FP32_RETAINED_RUNTIME_BYTES : host.FP16_RETAINED_RUNTIME_BYTES,
    runtimeBufferCount: 26,
  });
  const byId = new Map(plan.buffers.map((b) => [b.id, b]));
  assert.strictEqual(byId.get("source-shard-decoder.bin").byteLength,
                     fp32 ? host.FP32_LARGEST_RUNTIME_SHARD_BYTES : host.FP16_LARGEST_RUNTIME_SHARD_BYTES);
  assert.strictEqual(byId.get("source-shard-encoder-subsampling.bin").byteLength, fp32 ? 2740992 : 2727168);
  for (let layer = 0; layer < 24; ++layer) {
    const id = `source-shard-encoder-layer-${String(layer).padStart(2, "0")}.bin`;
    assert.strictEqual(byId.get(id).byteLength, fp32 ? 16836864 : 16050176, id);
  }
  assert.deepStrictEqual(plan.shards.map((s) => s.file.name), [
    "decoder.bin", "encoder-subsampling.bin",
    ...Array.from({ length: 24 }, (_, i) => `encoder-layer-${String(i).padStart(2, "0")}.bin`),
    "preprocessor.bin",
  ]);
  assert.strictEqual(plan.shards[26].hashOnly, true);
  assert(plan.shards.slice(0, 26).every((s) => s.hashOnly === false && s.runtimeBufferId === `source-shard-${s.file.name}`));
  const qkv = plan.tensors.get("encoder.layers.7.self_attn.qkv.weight");
  assert.deepStrictEqual(qkv.runtimeRecord, {
    bufferId: "source-shard-encoder-layer-07.bin", byteOffset: qkv.sourceRecord.byteOffset,
    byteLength: 1024 * 3072 / 32 * 5 * 4, dtype: "uint32", logicalShape: [1024, 3072],
    storageShape: [1024 * 3072 / 32, 5], layout: "k-by-output-row-major-palette5-lsb-u32",
  });
  const projector = plan.tensors.get("encoder_projector.weight").runtimeRecord;
  assert.strictEqual(projector.bufferId, "source-shard-decoder.bin");
  assert.deepStrictEqual(projector.storageShape, [20480, 5]);
  assert(!plan.tensors.has("preprocessor.window"));
  for (const tensor of plan.tensors.values()) {
    assert.strictEqual(tensor.runtimeRecord.byteOffset % 256, 0);
    assert.strictEqual(tensor.runtimeRecord.byteOffset, tensor.sourceRecord.byteOffset);
    assert.strictEqual(tensor.runtimeRecord.bufferId, `source-shard-${tensor.sourceRecord.shard}`);
  }
  // The converter's offsets that the reference test pins.
  assert.strictEqual(plan.tensors.get("encoder_projector.bias").runtimeRecord.byteOffset, fp32 ? 30909696 : 15671296);
  // fp32 stores the three 3x3 kernels in f32 (3 x 4608 more bytes before it).
  assert.strictEqual(plan.tensors.get("encoder.subsampling.layers.3.bias").runtimeRecord.byteOffset,
                     fp32 ? 58112 + 3 * 4608 : 58112);
  if (fp32) {
    assert.deepStrictEqual(plan.tensors.get("encoder.layers.7.self_attn.qkv.weight.palette").runtimeRecord.logicalShape,
                           [3, 32]);
    assert(![...plan.tensors.values()].some((t) => t.runtimeRecord.dtype === "float16"));
  }
}
assert.strictEqual(host.alignRuntimeOffset(0), 0);
assert.strictEqual(host.alignRuntimeOffset(1), 256);
assert.strictEqual(host.alignRuntimeOffset(257), 512);
assert.throws(() => host.alignRuntimeOffset(-1), /nonnegative/);

function planRejects(mutate, pattern, base) {
  const m = clone(base || base16);
  mutate(m);
  assert.throws(() => host.planRuntimePackage(m), pattern);
}
planRejects((m) => delete m.tensors["encoder.layers.0.self_attn.qkv.weight.palette"],
            /missing encoder\.layers\.0\.self_attn\.qkv\.weight\.palette/);
planRejects((m) => { m.tensors["encoder.layers.0.norm_out.bias"].byteOffset = 16050176; },
            /exceeds its aligned source shard/);
planRejects((m) => {
  Object.assign(m.tensors["encoder.layers.0.self_attn.o_proj.weight.palette"],
                { logicalShape: [1, 32], storageShape: [1, 32], byteLength: 64 });
}, /invalid palette storage/);
planRejects((m) => {
  const p = m.tensors["encoder.layers.0.self_attn.o_proj.weight.palette"];
  Object.assign(p, { dtype: "float16", byteLength: p.byteLength / 2 });
}, /invalid palette storage/, base32);
planRejects((m) => { m.tensors["encoder.layers.0.norm_out.bias"].dtype = "float16"; },
            /cannot retain float16 storage in the FP32 package/, base32);
planRejects((m) => {
  const name = "encoder.layers.0.self_attn.qkv.weight";
  const groups = 1024 * 3072 / 16;
  Object.assign(m.tensors[name], { byteLength: groups * 3 * 4, storageShape: [groups, 3],
                                   layout: "k-by-output-row-major-palette6-lsb-u32" });
  Object.assign(m.tensors[`${name}.palette`], { byteLength: 3 * 64 * 2, logicalShape: [3, 64], storageShape: [3, 64] });
}, /Packed palette topology changed/);
planRejects((m) => delete m.tensors["encoder.layers.0.norm_out.bias"], /Retained runtime tensor count changed: 794/);
planRejects((m) => {
  const f = m.files.find((file) => file.name === "decoder.bin");
  f.byteLength += 256;
}, /fp32 common-source shard inventory changed/, base32);
planRejects((m) => {
  const f = m.files.find((file) => file.name === "encoder-layer-03.bin");
  f.byteLength += 256;
}, /encoder-layer shard inventory changed: encoder-layer-03\.bin/);
planRejects((m) => { m.tensors["preprocessor.window"].shard = "decoder.bin"; },
            /preprocessor\.window must remain sourced from preprocessor\.bin/);
planRejects((m) => { m.tensors["stray.palette"] = Object.assign({}, m.tensors["encoder_projector.weight.palette"]); },
            /Unowned palette LUT tensors: stray\.palette/);

/* ---- loader over a stand-in device (package.ts:233-500) ---- */
class FakeBuffer {
  constructor(device, label, size) {
    Object.assign(this, { device, label, size, bytes: Buffer.alloc(size), destroyed: false,
                          address: BigInt(device.created.length + 1) << 32n });
  }
  destroy() {
    this.destroyed = true;
    this.device.live -= 1;
  }
}
const device = {
  live: 0,
  created: [],
  createBuffer(d) {
    const b = new FakeBuffer(this, d.label, d.size);
    this.live += 1;
    this.created.push(b);
    return b;
  },
  queue: { writeBuffer(buffer, offset, data) { Buffer.from(data.buffer, data.byteOffset, data.byteLength).copy(buffer.bytes, offset); } },
};
const written = load(packagePath);
const digest = require("crypto").createHash("sha256").update(fs.readFileSync(packagePath)).digest("hex");

async function main() {
  await assert.rejects(host.ParakeetGpuPackage.load(device, packagePath, { expectedPrecision: "fp16" }),
                       /Selected fp16 model manifest SHA-256 changed/);
  await assert.rejects(host.ParakeetGpuPackage.load(device, packagePath, { expectedPrecision: "fp32", manifestSha256: digest }),
                       /Selected fp32 execution but received a fp16 model package/);
  const phases = [];
  const pkg = await host.ParakeetGpuPackage.load(device, packagePath, {
    expectedPrecision: "fp16", manifestSha256: digest, onProgress: (p) => phases.push(p.phase),
  });
  assert.strictEqual(device.live, 26);
  assert.strictEqual(pkg.precision, "fp16");
  assert.strictEqual(pkg.manifestListedBytes, written.files.reduce((a, f) => a + f.byteLength, 0));
  assert.deepStrictEqual([phases[0], phases[phases.length - 2], phases[phases.length - 1]], ["manifest", "tokenizer", "ready"]);
  assert.strictEqual(pkg.tokenizer.type, "synthetic");
  const head = pkg.tensor("joint.head.bias");
  assert.strictEqual(head.buffer.label, "parakeet-source-decoder.bin");
  assert.deepStrictEqual(head.binding, { buffer: head.buffer, offset: 16994816, size: 4128 });
  // The resident buffer holds the shard's bytes as written.
  const shard = fs.readFileSync(path.join(path.dirname(packagePath), "decoder.bin"));
  assert(head.buffer.bytes.equals(shard));
  assert.throws(() => pkg.tensor("decoder.nope"), /Unknown runtime tensor decoder\.nope/);
  pkg.releaseInitializationMetadata();
  assert.throws(() => pkg.manifest, /initialization metadata was released/);
  assert.throws(() => pkg.tensor("joint.head.bias"), /tensor metadata was released/);
  pkg.destroy();
  pkg.destroy();
  assert.strictEqual(device.live, 0);
  assert.throws(() => pkg.tensor("joint.head.bias"), /package was destroyed/);

  // A corrupted shard fails its digest and frees every buffer made so far.
  const dir = path.dirname(packagePath);
  const layer = path.join(dir, "encoder-layer-05.bin");
  const original = fs.readFileSync(layer);
  const corrupted = Buffer.from(original);
  corrupted[1000] ^= 1;
  fs.writeFileSync(layer, corrupted);
  await assert.rejects(host.ParakeetGpuPackage.load(device, packagePath, { expectedPrecision: "fp16", manifestSha256: digest }),
                       /encoder-layer-05\.bin SHA-256 validation failed/);
  assert.strictEqual(device.live, 0);
  fs.writeFileSync(layer, original.subarray(0, original.length - 256));
  await assert.rejects(host.ParakeetGpuPackage.load(device, packagePath, { expectedPrecision: "fp16", manifestSha256: digest }),
                       /encoder-layer-05\.bin ended before its aligned declared length/);
  fs.writeFileSync(layer, original);
  const tokenizer = path.join(dir, "tokenizer.json");
  const tokenizerBytes = fs.readFileSync(tokenizer);
  fs.writeFileSync(tokenizer, Buffer.concat([tokenizerBytes, Buffer.from(" ")]));
  await assert.rejects(host.ParakeetGpuPackage.load(device, packagePath, { expectedPrecision: "fp16", manifestSha256: digest }),
                       /Tokenizer integrity validation failed/);
  fs.writeFileSync(tokenizer, tokenizerBytes);
  assert.strictEqual(device.live, 0);

  // Decoder weights: every tensor must come from the one decoder shard buffer.
  const again = await host.ParakeetGpuPackage.load(device, packagePath, { expectedPrecision: "fp16", manifestSha256: digest });
  const arena = Object.create(host.GpuActivationArena.prototype);
  await host.PersistentTdtDecoderKernel.create(device, arena, again);
  const split = { precision: "fp16", tensor: (name) => {
    const t = again.tensor(name);
    return name === "joint.head.weight" ? Object.assign({}, t, { buffer: { other: true } }) : t;
  } };
  await assert.rejects(host.PersistentTdtDecoderKernel.create(device, arena, split),
                       /Persistent TDT decoder requires one resident decoder source shard/);
  const wrong = { precision: "fp16", tensor: (name) => {
    const t = again.tensor(name);
    if (name !== "decoder.lstm.weight_l1") return t;
    return Object.assign({}, t, { sourceRecord: Object.assign({}, t.sourceRecord, { storageShape: [1280, 640, 4] }) });
  } };
  await assert.rejects(host.PersistentTdtDecoderKernel.create(device, arena, wrong),
                       /Unexpected decoder tensor input-hidden-k-by-ifgo-row-major-vec4 \[1280,640,4\]/);
  await assert.rejects(host.PersistentTdtDecoderKernel.create(device, arena, { precision: "fp32", tensor: again.tensor.bind(again) }),
                       /TDT decoder fp16 profile cannot use fp32 decoder weights/);
  again.destroy();
  assert.throws(() => host.planTdtDecoderExecution(0), /batchSize must be a positive integer/);
  console.log("package checks passed");
}

main().catch((error) => {
  console.error(error);
  process.exit(1);
});
